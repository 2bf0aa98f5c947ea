"""GGUF tensor table (names, ggml types, dimensions, stored bytes) of an image,
for the benchmark's algorithmic byte and operation counts.  The layout is
GGUF v2/v3 (crates/rie-core/src/gguf.rs:195-269); metadata values are skipped,
not decoded."""
from __future__ import annotations

import struct

# (values per block, bytes per block) of the ggml types (quant/mod.rs:17-125)
BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
         10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210)}
_SCALAR_SIZE = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}


def _parse(img):
    """(metadata alignment, [(name, ggml type, dims, offset in the data region)],
    end of the tensor infos)"""
    b = memoryview(img).cast("B")
    magic, _version, n_t, n_kv = struct.unpack_from("<IIQQ", b, 0)
    if magic != 0x46554747:
        raise ValueError("not a GGUF image")
    pos = 24
    align = 32

    def skip(ty, pos):
        if ty in _SCALAR_SIZE:
            return pos + _SCALAR_SIZE[ty]
        if ty == 8:
            return pos + 8 + struct.unpack_from("<Q", b, pos)[0]
        if ty == 9:
            et, n = struct.unpack_from("<IQ", b, pos)
            pos += 12
            if et in _SCALAR_SIZE:
                return pos + n * _SCALAR_SIZE[et]
            for _ in range(n):
                pos = skip(et, pos)
            return pos
        raise ValueError(f"metadata value type {ty}")

    for _ in range(n_kv):
        klen = struct.unpack_from("<Q", b, pos)[0]
        key = bytes(b[pos + 8:pos + 8 + klen])
        pos += 8 + klen
        ty = struct.unpack_from("<I", b, pos)[0]
        if key == b"general.alignment" and ty == 4:  # u32 (gguf.rs:256-258)
            align = struct.unpack_from("<I", b, pos + 4)[0]
        pos = skip(ty, pos + 4)
    infos = []
    for _ in range(n_t):
        nlen = struct.unpack_from("<Q", b, pos)[0]
        name = bytes(b[pos + 8:pos + 8 + nlen]).decode()
        pos += 8 + nlen
        nd = struct.unpack_from("<I", b, pos)[0]
        dims = list(struct.unpack_from(f"<{nd}Q", b, pos + 4))
        pos += 4 + 8 * nd
        ty, off = struct.unpack_from("<IQ", b, pos)
        pos += 12
        infos.append((name, ty, dims, off))
    return align, infos, pos


def tensor_table(img) -> dict:
    """name -> (ggml type, dims (cols first), stored bytes)"""
    out = {}
    for name, ty, dims, _off in _parse(img)[1]:
        n = 1
        for d in dims:
            n *= d
        bs, bb = BLOCK[ty]
        out[name] = (ty, dims, n // bs * bb)
    return out


def tensor_offset(img, name: str) -> int:
    """byte offset of a tensor's data in the image: the data region starts at the
    end of the tensor infos rounded up to general.alignment (32 by default,
    gguf.rs:256-262)"""
    align, infos, end = _parse(img)
    start = (end + align - 1) // align * align
    for n, _ty, _dims, off in infos:
        if n == name:
            return start + off
    raise KeyError(name)


def per_token_costs(img, n_expert_used: int = 0) -> dict:
    """Algorithmic costs of one token through the layers and the head: the
    weight bytes a decode step reads (every matrix once at its stored size, the
    routed share of stacked expert tensors, one embedding row) and the int8
    multiply-accumulate count of the layer matrices (2·params per token,
    routed experts only)."""
    t = tensor_table(img)
    head = t.get("output.weight", t["token_embd.weight"])
    emb_ty, emb_dims, emb_bytes = t["token_embd.weight"]
    layer_bytes = layer_params = 0
    n_expert = 0
    for name, (ty, dims, nbytes) in t.items():
        if not name.startswith("blk.") or len(dims) < 2:
            continue  # norms and biases: negligible
        params = 1
        for d in dims:
            params *= d
        if len(dims) == 3:  # stacked experts [cols, rows, experts]
            n_expert = dims[2]
            share = n_expert_used / dims[2]
            layer_bytes += nbytes * share
            layer_params += params * share
        else:
            layer_bytes += nbytes
            layer_params += params
    head_params = head[1][0] * head[1][1]
    return {"layer_weight_bytes": int(layer_bytes), "head_bytes": head[2], "embd_row_bytes": emb_bytes // emb_dims[1],
            "layer_params": int(layer_params), "head_params": head_params, "n_expert": n_expert}
