"""Python mirror of RIE's Backend contract over the HIP library.

The methods and their error behaviour follow ``trait Backend``
(crates/rie-core/src/model/mod.rs:303-320) and CpuBackend
(crates/rie-core/src/model/cpu.rs:93-429); errors carry the kind of the
reference's ``Error`` enum (crates/rie-core/src/error.rs:5-15).
"""
from __future__ import annotations

import ctypes as C
import enum

import numpy as np

from . import _lib


class KvType(enum.IntEnum):
    """KvType, model/cpu.rs:12-36"""
    F16 = 0
    Q8_0 = 1
    TURBO4 = 2

    @staticmethod
    def parse(s: str) -> "KvType | None":
        return {"f16": KvType.F16, "q8": KvType.Q8_0, "q8_0": KvType.Q8_0, "turbo4": KvType.TURBO4,
                "tq4": KvType.TURBO4, "turbo": KvType.TURBO4}.get(s.lower())


class RieError(Exception):
    KINDS = {-1: "Io", -2: "Format", -3: "Unsupported", -4: "Missing", -5: "Runtime"}

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code
        self.kind = self.KINDS.get(code, "Runtime")


def _check(rc: int, err) -> None:
    if rc != 0:
        raise RieError(rc, err.value.decode(errors="replace") if err is not None else "error")


def _u32(tokens) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))


class HipBackend:
    """The HIP backend: ``name``, ``max_batch``, ``n_ctx``, ``forward``, ``hidden``."""

    def __init__(self, gguf: bytes, n_ctx: int = 4096, max_batch: int = 64, kv_type: int = KvType.F16,
                 device: int = 0, use_graph: bool = True):
        L = _lib.lib()
        cfg = L.rie_hip_default_config()
        cfg.n_ctx, cfg.max_batch, cfg.kv_type, cfg.device, cfg.use_graph = n_ctx, max_batch, int(kv_type), device, int(use_graph)
        img = np.frombuffer(gguf, dtype=np.uint8)
        err = C.create_string_buffer(1024)
        code = C.c_int32(0)
        self._destroy = L.rie_hip_destroy  # held here: module globals may be gone when __del__ runs at exit
        self._h = L.rie_hip_create(img.ctypes.data, img.size, C.byref(cfg), C.byref(code), err, 1024)
        if not self._h:
            raise RieError(code.value, err.value.decode(errors="replace"))
        self.n_vocab = L.rie_hip_n_vocab(self._h)
        self.n_embd = L.rie_hip_n_embd(self._h)

    def close(self):
        if getattr(self, "_h", None):
            self._destroy(self._h)
            self._h = None

    __del__ = close

    # ---- Backend ----
    def name(self) -> str:
        buf = C.create_string_buffer(256)
        _lib.lib().rie_hip_name(self._h, buf, 256)
        return buf.value.decode()

    def max_batch(self) -> int:
        return _lib.lib().rie_hip_max_batch(self._h)

    def n_ctx(self) -> int:
        return _lib.lib().rie_hip_n_ctx(self._h)

    def forward(self, tokens, pos: int, all_logits: bool = False, logits: np.ndarray | None = None) -> np.ndarray:
        toks = _u32(tokens)
        if logits is None:
            logits = np.empty((toks.size if all_logits else 1) * self.n_vocab, np.float32)
        assert logits.dtype == np.float32 and logits.flags["C_CONTIGUOUS"]
        err = C.create_string_buffer(1024)
        rc = _lib.lib().rie_hip_forward(self._h, toks.ctypes.data if toks.size else None, toks.size, pos, int(all_logits),
                                        logits.ctypes.data, logits.size, err, 1024)
        _check(rc, err)
        return logits

    def hidden(self) -> np.ndarray | None:
        rows = C.c_size_t(0)
        p = _lib.lib().rie_hip_hidden(self._h, C.byref(rows))
        if not p:
            return None
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (rows.value * self.n_embd,)).copy()

    # ---- facts ----
    @property
    def kv_type(self) -> int:
        return _lib.lib().rie_hip_kv_type(self._h)

    def kv_bytes(self) -> int:
        return _lib.lib().rie_hip_kv_bytes(self._h)

    def weight_bytes(self) -> int:
        return _lib.lib().rie_hip_weight_bytes(self._h)

    # ---- device greedy ----
    def forward_argmax(self, tokens, pos: int) -> int:
        toks = _u32(tokens)
        nxt = C.c_uint32(0)
        err = C.create_string_buffer(1024)
        rc = _lib.lib().rie_hip_forward_argmax(self._h, toks.ctypes.data if toks.size else None, toks.size, pos,
                                               C.byref(nxt), err, 1024)
        _check(rc, err)
        return nxt.value

    def generate_greedy(self, pos: int, n_gen: int) -> np.ndarray:
        out = np.zeros(max(n_gen, 1), np.uint32)
        err = C.create_string_buffer(1024)
        _check(_lib.lib().rie_hip_generate_greedy(self._h, pos, n_gen, out.ctypes.data, err, 1024), err)
        return out[:n_gen]

    def bench(self, n_prompt: int, n_gen: int) -> tuple[float, float]:
        pp, tg = C.c_double(), C.c_double()
        err = C.create_string_buffer(1024)
        _check(_lib.lib().rie_hip_bench(self._h, n_prompt, n_gen, C.byref(pp), C.byref(tg), err, 1024), err)
        return pp.value, tg.value

    def profile_decode(self, pos: int, reps: int = 3) -> dict:
        """{kernel family: (total ms, launches)} of `reps` eager decode steps at pos"""
        names = C.create_string_buffer(4096)
        ms = np.zeros(64, np.float64)
        cnt = np.zeros(64, np.int32)
        n = C.c_size_t(0)
        rc = _lib.lib().rie_hip_profile_decode(self._h, pos, reps, names, 4096, ms.ctypes.data, cnt.ctypes.data, 64, C.byref(n))
        if rc:
            raise RieError(rc, "profile_decode failed")
        keys = names.value.decode().split("\n")[: n.value]
        return {k: (float(ms[i]), int(cnt[i])) for i, k in enumerate(keys)}

    def time_ffn_glu(self, reps: int = 3) -> tuple[float, int]:
        """(average µs, algorithmic bytes) of one single-token gate/up/SwiGLU launch"""
        us, nb = C.c_double(), C.c_size_t()
        rc = _lib.lib().rie_hip_time_ffn_glu(self._h, reps, C.byref(us), C.byref(nb))
        if rc:
            raise RieError(rc, "time_ffn_glu failed")
        return us.value, nb.value

    # ---- parity hooks ----
    def set_capture(self, on: bool) -> None:
        _lib.lib().rie_hip_set_capture(self._h, int(on))

    def set_attention_ranges(self, on: bool) -> None:
        """Single-token attention over context ranges at every length (the kernel
        used past the short-context limit); off: automatic."""
        _lib.lib().rie_hip_set_attention_ranges(self._h, int(on))

    def capture(self, layer: int, what: int, n: int) -> np.ndarray | None:
        out = np.zeros(n, np.float32)
        rc = _lib.lib().rie_hip_capture(self._h, layer, what, out.ctypes.data, n)
        return out if rc == 0 else None

    def kv_layer(self, layer: int, which: int, n_kv: int, slots: int):
        rb = _lib.lib().rie_hip_kv_row_bytes(self._h)
        out = np.zeros(n_kv * slots * rb, np.uint8)
        sc = np.zeros(n_kv * slots * 2, np.uint8)
        rc = _lib.lib().rie_hip_kv_layer(self._h, layer, which, out.ctypes.data, out.size, sc.ctypes.data, sc.size)
        if rc:
            raise RieError(rc, "kv_layer failed")
        return out.reshape(n_kv, slots, rb), sc.view(np.uint16).reshape(n_kv, slots)
