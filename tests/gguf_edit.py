"""Inserts one F32 tensor into a GGUF image (test helper, pure Python).

The image's key/value section and tensor infos are copied byte for byte, the
tensor count grows by one, the new info (one dimension, type F32) is appended
after the existing ones, and the new tensor's data goes after the existing data
at the file's alignment (general.alignment, default 32; the layout of
crates/rie-core/src/gguf.rs:212-269 and GgufWriter::to_bytes, 407-436).  Offsets
of the existing tensors are relative to the data section, so they do not change.
"""
from __future__ import annotations

import struct

import numpy as np

from gguf_np import GGUF


def _align(n: int, a: int) -> int:
    return (n + a - 1) // a * a


def add_f32_tensor(img: bytes, name: str, values: np.ndarray) -> bytes:
    g = GGUF(bytes(img))
    align = int(g.get("general.alignment", 32))
    data = bytes(img)
    # header: magic, version, tensor count, kv count; then the kv section and the infos
    magic, version, n_t, n_kv = struct.unpack_from("<IIQQ", data, 0)
    infos_end = g.pos  # the reader stops right after the last tensor info
    data_start = g.data_start
    old_data = data[data_start:]
    end = 0
    for tname, start, size in g.tensor_order:
        end = max(end, start - data_start + size)
    new_off = _align(end, align)
    vals = np.ascontiguousarray(values, dtype=np.float32)
    nb = name.encode("utf-8")
    info = struct.pack("<Q", len(nb)) + nb + struct.pack("<I", 1) + struct.pack("<Q", vals.size) + struct.pack("<I", 0) + \
        struct.pack("<Q", new_off)
    head = struct.pack("<IIQQ", magic, version, n_t + 1, n_kv) + data[24:infos_end] + info
    head += b"\0" * (_align(len(head), align) - len(head))
    body = old_data[:end] + b"\0" * (new_off - end) + vals.tobytes()
    return head + body
