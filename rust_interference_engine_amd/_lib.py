"""Loads librie_hip.so (built in-tree from csrc/) and declares its C ABI
(include/rie_hip.h).  There is no fallback: without the library every entry
point raises."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "_build", "librie_hip.so")
HEADER = os.path.join(ROOT, "include", "rie_hip.h")


class SynthSpec(C.Structure):
    """rie_hip_synth_spec: SyntheticSpec (crates/rie-core/src/testing.rs:95-124) + workload mode"""
    _fields_ = [("arch", C.c_char * 32)] + [(n, C.c_uint32) for n in (
        "n_vocab", "n_embd", "n_layer", "n_head", "n_head_kv", "head_dim", "n_ff", "rope_dim", "ctx")] + [
        ("wtype", C.c_int32), ("embd_type", C.c_int32), ("tied_output", C.c_int32), ("qkv_bias", C.c_int32),
        ("qk_norm", C.c_int32), ("post_norms", C.c_int32), ("fused", C.c_int32),
        ("swa_window", C.c_uint32), ("n_expert", C.c_uint32), ("n_expert_used", C.c_uint32),
        ("n_ff_exp", C.c_uint32), ("n_ff_shexp", C.c_uint32), ("chat_template", C.c_int32), ("seed", C.c_uint64),
        ("mode", C.c_int32), ("rope_base", C.c_float), ("output_type", C.c_int32), ("mix", C.c_int32)]


class Config(C.Structure):
    _fields_ = [("n_ctx", C.c_int32), ("max_batch", C.c_int32), ("kv_type", C.c_int32), ("device", C.c_int32),
                ("use_graph", C.c_int32)]


def build(jobs: int = 8) -> None:
    """Compile librie_hip.so for gfx950 (hipcc cross-compiles without a GPU)."""
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", os.path.join(PKG, "csrc")], check=True)


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"librie_hip.so is not built ({LIB_PATH}); run __graft_entry__.build()")
    L = C.CDLL(LIB_PATH)
    P, S, I, F, D = C.c_void_p, C.c_size_t, C.c_int32, C.c_float, C.c_double
    CP, U8P = C.c_char_p, C.POINTER(C.POINTER(C.c_uint8))
    sig = {
        "rie_hip_default_config": (Config, []),
        "rie_hip_create": (P, [P, S, C.POINTER(Config), C.POINTER(I), CP, S]),
        "rie_hip_destroy": (None, [P]),
        "rie_hip_name": (S, [P, CP, S]),
        "rie_hip_max_batch": (S, [P]), "rie_hip_n_ctx": (S, [P]), "rie_hip_n_vocab": (S, [P]), "rie_hip_n_embd": (S, [P]),
        "rie_hip_kv_type": (I, [P]), "rie_hip_kv_bytes": (S, [P]), "rie_hip_weight_bytes": (S, [P]),
        "rie_hip_kv_row_bytes": (S, [P]),
        "rie_hip_forward": (I, [P, P, S, S, I, P, S, CP, S]),
        "rie_hip_hidden": (P, [P, C.POINTER(S)]),
        "rie_hip_forward_argmax": (I, [P, P, S, S, C.POINTER(C.c_uint32), CP, S]),
        "rie_hip_generate_greedy": (I, [P, S, S, P, CP, S]),
        "rie_hip_bench": (I, [P, S, S, C.POINTER(D), C.POINTER(D), CP, S]),
        "rie_hip_synth_tiny": (I, [CP, I, C.POINTER(SynthSpec)]),
        "rie_hip_synth_preset": (I, [CP, I, C.POINTER(SynthSpec)]),
        "rie_hip_synth_build": (S, [C.POINTER(SynthSpec), U8P, I]),
        "rie_hip_free": (None, [P]),
        "rie_hip_quantize": (I, [I, P, S, P]),
        "rie_hip_set_capture": (I, [P, I]),
        "rie_hip_set_attention_ranges": (I, [P, I]),
        "rie_hip_capture": (I, [P, S, I, P, S]),
        "rie_hip_kv_layer": (I, [P, S, I, P, S, P, S]),
        "rie_hip_profile_decode": (I, [P, S, I, CP, S, P, P, S, C.POINTER(S)]),
        "rie_hip_time_ffn_glu": (I, [P, I, C.POINTER(D), C.POINTER(S)]),
        "rie_hip_k_rmsnorm_quant": (I, [P, P, F, I, I, I, P, P, P, P, P, P]),
        "rie_hip_k_gemv": (I, [I, P, I, I, P, P, P, P, P, P, I, P]),
        "rie_hip_k_gemm": (I, [I, P, I, I, P, P, P, P, P, I, P]),
        "rie_hip_k_moe_route": (I, [P, I, I, I, I, I, P, P]),
        "rie_hip_k_argmax": (I, [P, I, P]),
        "rie_hip_k_argmax_noalloc": (I, [P, I, P, P, CP, S]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def declared_functions() -> list[str]:
    """Function names declared in include/rie_hip.h."""
    import re
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(rie_hip_\w+)\s*\(", txt)))
