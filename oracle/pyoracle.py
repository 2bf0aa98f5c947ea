"""ctypes binding of the oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the CPU-baseline leg of bench.py, where it is the checker or the timed CPU
reference.  The product package never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 30
TYPE_NAMES = {F32: "F32", F16: "F16", BF16: "BF16", Q4_0: "Q4_0", Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1",
              Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}
KV_F16, KV_Q8_0, KV_TURBO4 = 0, 1, 2
KV_SEED = 0x75426F5175616E74

BLOCK_Q8_0 = np.dtype([("qs", np.int8, 32), ("d", np.float32), ("s", np.float32), ("pad", np.uint8, 8)])
BLOCK_Q8K = np.dtype([("qs", np.int8, 256), ("bsums", np.int16, 16), ("d", np.float32), ("pad", np.uint8, 12)])
assert BLOCK_Q8_0.itemsize == 48 and BLOCK_Q8K.itemsize == 304


class SynthSpec(C.Structure):
    _fields_ = [("arch", C.c_char * 32)] + [(n, C.c_uint32) for n in (
        "n_vocab", "n_embd", "n_layer", "n_head", "n_head_kv", "head_dim", "n_ff", "rope_dim", "ctx")] + [
        ("wtype", C.c_int32), ("embd_type", C.c_int32), ("tied_output", C.c_int32), ("qkv_bias", C.c_int32),
        ("qk_norm", C.c_int32), ("post_norms", C.c_int32), ("fused", C.c_int32),
        ("swa_window", C.c_uint32), ("n_expert", C.c_uint32), ("n_expert_used", C.c_uint32),
        ("n_ff_exp", C.c_uint32), ("n_ff_shexp", C.c_uint32), ("chat_template", C.c_int32), ("seed", C.c_uint64)]


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P, S, I, F, U8P = C.c_void_p, C.c_size_t, C.c_int, C.c_float, C.POINTER(C.c_uint8)
        sig = {
            "or_f32_to_f16": (C.c_uint16, [F]), "or_f16_to_f32": (F, [C.c_uint16]),
            "or_f32_to_bf16": (C.c_uint16, [F]),
            "or_rng_init": (None, [P, C.c_uint64]), "or_rng_next": (C.c_uint64, [P]),
            "or_random_weight": (None, [P, I, S, S, F, P]),
            "or_dequantize_row": (None, [I, P, P, S]),
            "or_quantize_q8_0": (None, [P, P, S]), "or_quantize_q8_0_scalar": (None, [P, P, S]),
            "or_quantize_q8_k": (None, [P, P, S]),
            "or_quantize_weights_q4_0": (None, [P, S, P]), "or_quantize_weights_q8_0": (None, [P, S, P]),
            "or_vec_dot": (F, [I, P, P, S]), "or_block_idots": (None, [I, P, P, S, P]),
            "or_dot_f32": (F, [P, P, S]), "or_dot_f16_f32": (F, [P, P, S]), "or_axpy_f16": (None, [P, F, P, S]),
            "or_rmsnorm": (None, [P, P, P, S, F]), "or_rmsnorm_inplace": (None, [P, P, S, F]),
            "or_silu": (F, [F]), "or_softmax": (None, [P, S]),
            "or_rope_inv_freq": (None, [S, F, F, P, S, P]), "or_rope_table": (None, [P, S, S, P, P]),
            "or_rope_apply": (None, [P, S, I, P, P]),
            "or_turbo_block_size": (S, [S]), "or_turbo_row_bytes": (S, [S]),
            "or_turbo_signs": (None, [S, C.c_uint64, P]), "or_fwht": (None, [P, S]),
            "or_turbo_rotate": (None, [P, S, C.c_uint64]), "or_turbo_rotate_inverse": (None, [P, S, C.c_uint64]),
            "or_turbo_quantize_rotated": (None, [P, S, P]), "or_turbo_quantize": (None, [P, S, C.c_uint64, P]),
            "or_turbo_dot": (F, [P, S, P]), "or_turbo_axpy": (None, [P, S, F, P]),
            "or_turbo_dequantize": (None, [P, S, C.c_uint64, P]),
            "or_synth_tiny": (I, [C.c_char_p, I, C.POINTER(SynthSpec)]),
            "or_synth_preset": (I, [C.c_char_p, I, C.POINTER(SynthSpec)]),
            "or_synth_build": (S, [C.POINTER(SynthSpec), C.POINTER(U8P)]),
            "or_free": (None, [P]),
            "or_model_load": (P, [P, S, C.c_char_p, S]), "or_model_free": (None, [P]),
            "or_model_config": (None, [P, P, S]),
            "or_backend_new": (P, [P, S, S, I, I]), "or_backend_free": (None, [P]),
            "or_backend_kv_type": (I, [P]), "or_backend_kv_bytes": (S, [P]),
            "or_forward": (I, [P, P, S, S, I, P, S, C.c_char_p, S]),
            "or_hidden": (P, [P, C.POINTER(S)]), "or_kv_layer": (P, [P, S, I, C.POINTER(S)]),
            "or_set_capture": (None, [P, I]), "or_capture": (P, [P, S, I, C.POINTER(S)]),
            "or_argmax": (C.c_uint32, [P, S]),
            "or_moe_route": (None, [P, S, S, S, I, I, P, P]),
            "or_greedy": (I, [P, P, S, S, S, P, P, P, C.c_char_p, S]),
            "or_bench": (I, [P, S, S, C.POINTER(C.c_double), C.POINTER(C.c_double), C.c_char_p, S]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---- scalar / row helpers ------------------------------------------------------
def f32_to_f16(x: float) -> int:
    return lib().or_f32_to_f16(x)


class Rng:
    """testing.rs:10-30 via the oracle"""

    def __init__(self, seed: int):
        self.state = (C.c_uint64 * 1)()
        lib().or_rng_init(self.state, seed)

    def next_u64(self) -> int:
        return lib().or_rng_next(self.state)

    def random_weight(self, ty: int, rows: int, cols: int, gain: float = 1.0) -> np.ndarray:
        bs, bb = (1, {F32: 4, F16: 2, BF16: 2}[ty]) if ty in (F32, F16, BF16) else (
            (32 if ty in (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0) else 256),
            {Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}[ty])
        out = np.zeros(rows * cols // bs * bb, np.uint8)
        lib().or_random_weight(self.state, ty, rows, cols, gain, ptr(out))
        return out


def dequantize_row(ty: int, data: np.ndarray, n: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    data = np.ascontiguousarray(data, dtype=np.uint8)
    lib().or_dequantize_row(ty, ptr(data), ptr(out), n)
    return out


def quantize_q8_0(x: np.ndarray, scalar: bool = False) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32, BLOCK_Q8_0)
    (lib().or_quantize_q8_0_scalar if scalar else lib().or_quantize_q8_0)(ptr(x), ptr(out), x.size // 32)
    return out


def quantize_q8_k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 256, BLOCK_Q8K)
    lib().or_quantize_q8_k(ptr(x), ptr(out), x.size // 256)
    return out


def quantize_weights(ty: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    bb = {Q4_0: 18, Q8_0: 34}[ty]
    out = np.zeros(x.size // 32 * bb, np.uint8)
    (lib().or_quantize_weights_q4_0 if ty == Q4_0 else lib().or_quantize_weights_q8_0)(ptr(x), x.size, ptr(out))
    return out


def act_format(ty: int) -> str:
    if ty in (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0):
        return "q8_0"
    if ty in (Q4_K, Q5_K, Q6_K, Q2_K, Q3_K):
        return "q8k"
    return "f32"


def quantize_act(ty: int, x: np.ndarray) -> np.ndarray:
    f = act_format(ty)
    if f == "q8_0":
        return quantize_q8_0(x)
    if f == "q8k":
        return quantize_q8_k(x)
    return np.ascontiguousarray(x, dtype=np.float32)


def vec_dot(ty: int, w: np.ndarray, act: np.ndarray, n: int) -> float:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    return lib().or_vec_dot(ty, ptr(w), ptr(act), n)


def block_idots(ty: int, w: np.ndarray, act: np.ndarray, n: int) -> np.ndarray:
    bs = 32 if ty in (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0) else 256
    out = np.zeros(n // bs * (1 if bs == 32 else 2), np.int32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    lib().or_block_idots(ty, ptr(w), ptr(act), n, ptr(out))
    return out


def turbo_row_bytes(d: int) -> int:
    return lib().or_turbo_row_bytes(d)


def turbo_quantize(x: np.ndarray, seed: int = KV_SEED) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(turbo_row_bytes(x.size), np.uint8)
    lib().or_turbo_quantize(ptr(x), x.size, seed, ptr(out))
    return out


def turbo_dequantize(row: np.ndarray, d: int, seed: int = KV_SEED) -> np.ndarray:
    out = np.zeros(d, np.float32)
    row = np.ascontiguousarray(row, dtype=np.uint8)
    lib().or_turbo_dequantize(ptr(row), d, seed, ptr(out))
    return out


def turbo_rotate(x: np.ndarray, seed: int = KV_SEED, inverse: bool = False) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True)
    (lib().or_turbo_rotate_inverse if inverse else lib().or_turbo_rotate)(ptr(y), y.size, seed)
    return y


# ---- synthetic GGUF ----------------------------------------------------------------
def synth_spec(name: str, wtype: int) -> SynthSpec:
    s = SynthSpec()
    if name.startswith("tiny-"):
        rc = lib().or_synth_tiny(name[5:].encode(), wtype, C.byref(s))
    else:
        rc = lib().or_synth_preset(name.encode(), wtype, C.byref(s))
    if rc:
        raise ValueError(f"unknown preset {name}")
    return s


def synth_build(spec: SynthSpec) -> bytes:
    p = C.POINTER(C.c_uint8)()
    n = lib().or_synth_build(C.byref(spec), C.byref(p))
    try:
        return np.ctypeslib.as_array(p, (n,)).tobytes()  # string_at takes a 32-bit size
    finally:
        lib().or_free(p)


# ---- model / backend -------------------------------------------------------------------
class OracleError(RuntimeError):
    pass


CONFIG_KEYS = ("n_vocab", "n_embd", "n_layer", "n_head", "n_head_kv", "head_dim", "n_ff", "rope_dim",
               "rope_neox", "n_expert", "n_expert_used", "n_ff_exp", "ctx_train", "arch", "output_type",
               "embd_type", "swa_window", "swa_pattern", "gelu")


class Model:
    def __init__(self, gguf: bytes):
        self._buf = np.frombuffer(gguf, dtype=np.uint8)  # kept alive: weights are views into it
        err = C.create_string_buffer(512)
        self.h = lib().or_model_load(ptr(self._buf), self._buf.size, err, 512)
        if not self.h:
            raise OracleError(err.value.decode())
        cfg = np.zeros(20, np.int64)
        lib().or_model_config(self.h, ptr(cfg), 20)
        self.cfg = dict(zip(CONFIG_KEYS, (int(v) for v in cfg)))

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_model_free(self.h)
            self.h = None


class Backend:
    """CpuBackend (model/cpu.rs) restated; same forward contract as the Backend trait."""

    def __init__(self, model: Model, n_ctx: int, max_batch: int, kv: int = KV_F16, n_threads: int = 8):
        self.model = model
        self.h = lib().or_backend_new(model.h, n_ctx, max_batch, kv, n_threads)
        self.n_vocab = model.cfg["n_vocab"]
        self._n_ctx, self._max_batch = n_ctx, max_batch

    def n_ctx(self) -> int:
        return self._n_ctx

    def max_batch(self) -> int:
        return self._max_batch

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_backend_free(self.h)
            self.h = None

    @property
    def kv_type(self) -> int:
        return lib().or_backend_kv_type(self.h)

    def kv_bytes(self) -> int:
        return lib().or_backend_kv_bytes(self.h)

    def forward(self, tokens, pos: int, all_logits: bool = False, logits: np.ndarray | None = None) -> np.ndarray:
        toks = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        n = toks.size
        if logits is None:
            logits = np.zeros((n if all_logits else 1) * self.n_vocab, np.float32)
        err = C.create_string_buffer(512)
        rc = lib().or_forward(self.h, ptr(toks) if n else None, n, pos, int(all_logits), ptr(logits), logits.size, err, 512)
        if rc:
            raise OracleError(err.value.decode())
        return logits

    def hidden(self):
        rows = C.c_size_t()
        p = lib().or_hidden(self.h, C.byref(rows))
        if not p:
            return None
        e = self.model.cfg["n_embd"]
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (rows.value * e,)).copy()

    def kv_layer(self, layer: int, which: int) -> np.ndarray:
        nbytes = C.c_size_t()
        p = lib().or_kv_layer(self.h, layer, which, C.byref(nbytes))
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), (nbytes.value,)).copy()

    def set_capture(self, on: bool):
        lib().or_set_capture(self.h, int(on))

    def capture(self, layer: int, what: int):
        n = C.c_size_t()
        p = lib().or_capture(self.h, layer, what, C.byref(n))
        if not p:
            return None
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (n.value,)).copy()

    def greedy(self, prompt, n_gen: int, n_batch: int = 0):
        prompt = np.ascontiguousarray(np.asarray(prompt, dtype=np.uint32))
        toks = np.zeros(max(n_gen, 1), np.uint32)
        margins = np.zeros(max(n_gen, 1), np.float32)
        first = np.zeros(self.n_vocab, np.float32)
        err = C.create_string_buffer(512)
        rc = lib().or_greedy(self.h, ptr(prompt), prompt.size, n_batch, n_gen, ptr(toks), ptr(margins), ptr(first), err, 512)
        if rc:
            raise OracleError(err.value.decode())
        return toks[:n_gen], margins[:n_gen], first

    def bench(self, n_prompt: int, n_gen: int):
        pp, tg = C.c_double(), C.c_double()
        err = C.create_string_buffer(512)
        rc = lib().or_bench(self.h, n_prompt, n_gen, C.byref(pp), C.byref(tg), err, 512)
        if rc:
            raise OracleError(err.value.decode())
        return pp.value, tg.value


def argmax(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().or_argmax(ptr(x), x.size)


def moe_route(logits: np.ndarray, k: int, norm_topk: bool = True, unit_weights: bool = False):
    """moe_ffn's routing (model/cpu.rs:492-500) of logits [n_tok][n_exp]: the k
    chosen experts per token in ascending expert order, and their weights."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    n_tok, n_exp = logits.shape
    sel = np.zeros((n_tok, k), np.int32)
    wgt = np.zeros((n_tok, k), np.float32)
    lib().or_moe_route(ptr(logits), n_tok, n_exp, k, int(norm_topk), int(unit_weights), ptr(sel), ptr(wgt))
    return sel, wgt
