"""Synthetic GGUF images (``rie bench --synthetic``, crates/rie-core/src/testing.rs)
built by the native generator in librie_hip.so."""
from __future__ import annotations

import ctypes as C
import weakref

import numpy as np

from . import _lib

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 30
TYPES = {"F32": F32, "F16": F16, "BF16": BF16, "Q4_0": Q4_0, "Q4_1": Q4_1, "Q5_0": Q5_0, "Q5_1": Q5_1, "Q8_0": Q8_0,
         "Q2_K": Q2_K, "Q3_K": Q3_K, "Q4_K": Q4_K, "Q5_K": Q5_K, "Q6_K": Q6_K}

SynthSpec = _lib.SynthSpec


def tiny(arch: str, wtype: int) -> SynthSpec:
    """SyntheticSpec::tiny (testing.rs:127-154)"""
    s = SynthSpec()
    if _lib.lib().rie_hip_synth_tiny(arch.encode(), wtype, C.byref(s)):
        raise ValueError(arch)
    return s


def preset(name: str, wtype: int) -> SynthSpec:
    """SyntheticSpec::preset (testing.rs:157-212), plus the llama-3.1-8b shape"""
    s = SynthSpec()
    if _lib.lib().rie_hip_synth_preset(name.encode(), wtype, C.byref(s)):
        raise ValueError(f"unknown preset {name}")
    return s


def baseline_llama31_8b_q4_0(seed: int = 1, ctx: int = 8192) -> SynthSpec:
    """The Llama-3.1-8B-shaped Q4_0 workload: 32 layers, hidden 4096, 32/8 heads,
    head dim 128, FFN 14336, vocab 128256, untied Q4_0 output head, weights
    N(0, 0.02) quantized with quantize::q4_0, unit norms, RoPE base 5e5."""
    s = preset("llama-3.1-8b", Q4_0)
    s.embd_type = Q4_0
    s.output_type = Q4_0
    s.mode = 1
    s.rope_base = 500000.0
    s.ctx = ctx
    s.seed = seed
    return s


def build_array(spec: SynthSpec, n_threads: int = 0) -> np.ndarray:
    """SyntheticSpec::build (testing.rs:229-383) → the GGUF image as a uint8 array
    owning the library's buffer (no copy; freed with the array)."""
    p = C.POINTER(C.c_uint8)()
    n = _lib.lib().rie_hip_synth_build(C.byref(spec), C.byref(p), n_threads)
    if n == 0:
        raise RuntimeError("synthetic model build failed (unsupported type for this mode?)")
    arr = np.ctypeslib.as_array(p, (n,))
    weakref.finalize(arr, _lib.lib().rie_hip_free, C.cast(p, C.c_void_p))
    return arr


def build(spec: SynthSpec, n_threads: int = 0) -> bytes:
    """SyntheticSpec::build → GGUF image bytes"""
    return build_array(spec, n_threads).tobytes()
