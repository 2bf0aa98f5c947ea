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


def baseline_qwen3_1_7b_q4_0(seed: int = 1, ctx: int = 4096) -> SynthSpec:
    """The Qwen3-1.7B-shaped Q4_0 workload (`rie bench --synthetic qwen3-1.7b
    --wtype Q4_0` shape): 28 layers, hidden 2048, 16/8 heads of 128, FFN 6144,
    vocab 151936, QK-norm, tied Q6_K embeddings/head (testing.rs:188-201), weights
    N(0, 0.02), unit norms, RoPE base 1e6."""
    s = preset("qwen3-1.7b", Q4_0)
    s.mode, s.rope_base, s.ctx, s.seed = 1, 1e6, ctx, seed
    return s


def baseline_llama32_3b_q4_k_m(seed: int = 1, ctx: int = 4096) -> SynthSpec:
    """The Llama-3.2-3B-shaped Q4_K_M workload: 28 layers, hidden 3072, 24/8 heads
    of 128, FFN 8192, vocab 128256, tied embeddings; Q4_K matrices with Q6_K for
    attn_v, for ffn_down in the 14 layers llama.cpp's Q4_K_M widens, and for the
    embeddings/head; weights N(0, 0.02), unit norms, RoPE base 5e5."""
    s = preset("llama-3.2-3b", Q4_K)
    s.embd_type, s.output_type = Q6_K, Q6_K
    s.mode, s.mix, s.rope_base, s.ctx, s.seed = 1, 1, 5e5, ctx, seed
    return s


def baseline_qwen3_30b_a3b_q4_k(seed: int = 1, ctx: int = 4096) -> SynthSpec:
    """The Qwen3-30B-A3B-shaped MoE workload: 48 layers, hidden 2048, 32/4 heads of
    128, 128 experts of FFN 768 with top-8 softmax routing, vocab 151936, untied;
    Q4_K matrices, Q6_K embeddings and head, F32 router weights N(0, 1), other
    weights N(0, 0.02), unit norms, RoPE base 1e6."""
    s = preset("qwen3-30b-a3b", Q4_K)
    s.embd_type, s.output_type = Q6_K, Q6_K
    s.mode, s.rope_base, s.ctx, s.seed = 1, 1e6, ctx, seed
    return s


def quantize(ty: int, x: np.ndarray) -> np.ndarray:
    """The generator's weight quantizers (quantize::q4_0 / q8_0, quant/mod.rs:
    262-298, and this library's Q4_K / Q6_K) on a flat f32 array."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    bs, bb = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}[ty]
    out = np.zeros(x.size // bs * bb, np.uint8)
    if _lib.lib().rie_hip_quantize(ty, x.ctypes.data, x.size, out.ctypes.data) != 0:
        raise ValueError(f"no quantizer for type {ty} at {x.size} values")
    return out


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
