"""Minimal pure-Python GGUF v2/v3 reader (the file layout of gguf.rs:212-269),
independent of both the C oracle and the product's C++ reader."""
from __future__ import annotations

import struct

import numpy as np

import ggml_np as G

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


class GGUF:
    def __init__(self, data: bytes):
        self.data = data
        self.pos = 0
        magic, self.version = struct.unpack_from("<II", data, 0)
        assert magic == 0x46554747, "bad magic"
        self.pos = 8
        n_t, n_kv = struct.unpack_from("<QQ", data, self.pos)
        self.pos += 16
        self.kv = {}
        self.kv_order = []
        for _ in range(n_kv):
            k = self._str()
            ty = self._u32()
            self.kv[k] = self._val(ty)
            self.kv_order.append(k)
        infos = []
        for _ in range(n_t):
            name = self._str()
            nd = self._u32()
            dims = list(struct.unpack_from(f"<{nd}Q", data, self.pos))
            self.pos += 8 * nd
            ty = self._u32()
            off = struct.unpack_from("<Q", data, self.pos)[0]
            self.pos += 8
            infos.append((name, dims, ty, off))
        align = int(self.kv.get("general.alignment", 32))
        self.data_start = (self.pos + align - 1) // align * align
        self.tensors = {}
        self.tensor_order = []
        buf = np.frombuffer(data, np.uint8)
        for name, dims, ty, off in infos:
            n = int(np.prod(dims))
            size = G.row_bytes(ty, n)
            start = self.data_start + off
            self.tensors[name] = (ty, dims, buf[start:start + size])
            self.tensor_order.append((name, start, size))

    def _u32(self):
        v = struct.unpack_from("<I", self.data, self.pos)[0]
        self.pos += 4
        return v

    def _str(self):
        n = struct.unpack_from("<Q", self.data, self.pos)[0]
        self.pos += 8
        s = self.data[self.pos:self.pos + n].decode("utf-8", "replace")
        self.pos += n
        return s

    def _val(self, ty):
        if ty in _SCALAR:
            fmt = _SCALAR[ty]
            v = struct.unpack_from(fmt, self.data, self.pos)[0]
            self.pos += struct.calcsize(fmt)
            return v
        if ty == 8:
            return self._str()
        if ty == 9:
            et = self._u32()
            n = struct.unpack_from("<Q", self.data, self.pos)[0]
            self.pos += 8
            return [self._val(et) for _ in range(n)]
        raise ValueError(ty)

    def get(self, key, default=None):
        return self.kv.get(key, default)
