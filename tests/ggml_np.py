"""Vectorised numpy restatement of the ggml block formats and RIE's activation
quantizers, written from the format definitions (quant/reference.rs:53-215,
quant/mod.rs:175-218, kernels/avx2.rs:153-184) independently of the C oracle,
so that the two implementations check each other.
"""
from __future__ import annotations

import numpy as np

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 30
BLOCK = {Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24), Q8_0: (32, 34), Q2_K: (256, 84),
         Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), F32: (1, 4), F16: (1, 2), BF16: (1, 2)}


def row_bytes(ty, n):
    bs, bb = BLOCK[ty]
    return n // bs * bb


def _f16(b2):
    """two little-endian bytes per row → float32"""
    return np.ascontiguousarray(b2).view(np.float16).reshape(-1).astype(np.float32)


def _k4_scales(q):
    """12-byte scale/min field → (sc, m) of shape (nb, 8)"""
    q = q.astype(np.uint8)
    sc = np.zeros((q.shape[0], 8), np.uint8)
    m = np.zeros((q.shape[0], 8), np.uint8)
    sc[:, :4] = q[:, 0:4] & 63
    m[:, :4] = q[:, 4:8] & 63
    sc[:, 4:] = (q[:, 8:12] & 0xF) | ((q[:, 0:4] >> 6) << 4)
    m[:, 4:] = (q[:, 8:12] >> 4) | ((q[:, 4:8] >> 6) << 4)
    return sc, m


def dequantize(ty: int, raw: np.ndarray, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    if ty == F32:
        return raw[: 4 * n].view(np.float32).copy()
    if ty == F16:
        return raw[: 2 * n].view(np.float16).astype(np.float32)
    if ty == BF16:
        return (raw[: 2 * n].view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    bs, bb = BLOCK[ty]
    nb = n // bs
    b = raw[: nb * bb].reshape(nb, bb)
    if ty == Q4_0:
        d = _f16(b[:, 0:2])[:, None]
        qs = b[:, 2:18]
        q = np.concatenate([(qs & 15).astype(np.int32) - 8, (qs >> 4).astype(np.int32) - 8], axis=1)
        return (q.astype(np.float32) * d).reshape(-1)
    if ty == Q4_1:
        d, m = _f16(b[:, 0:2])[:, None], _f16(b[:, 2:4])[:, None]
        qs = b[:, 4:20]
        q = np.concatenate([qs & 15, qs >> 4], axis=1).astype(np.float32)
        return (q * d + m).reshape(-1)
    if ty in (Q5_0, Q5_1):
        if ty == Q5_0:
            d, m, qh, qs = _f16(b[:, 0:2])[:, None], None, b[:, 2:6], b[:, 6:22]
        else:
            d, m, qh, qs = _f16(b[:, 0:2])[:, None], _f16(b[:, 2:4])[:, None], b[:, 4:8], b[:, 8:24]
        h = np.ascontiguousarray(qh).view(np.uint32).reshape(-1, 1)
        j = np.arange(16, dtype=np.uint32)[None, :]
        lo = (qs & 15).astype(np.uint32) | (((h >> j) & 1) << 4)
        hi = (qs >> 4).astype(np.uint32) | (((h >> (j + 16)) & 1) << 4)
        q = np.concatenate([lo, hi], axis=1).astype(np.int32)
        if ty == Q5_0:
            return ((q - 16).astype(np.float32) * d).reshape(-1)
        return (q.astype(np.float32) * d + m).reshape(-1)
    if ty == Q8_0:
        d = _f16(b[:, 0:2])[:, None]
        return (b[:, 2:34].view(np.int8).astype(np.float32) * d).reshape(-1)
    if ty == Q4_K:
        d, dmin = _f16(b[:, 0:2])[:, None], _f16(b[:, 2:4])[:, None]
        sc, mn = _k4_scales(b[:, 4:16])
        q = b[:, 16:144].reshape(nb, 4, 32)
        out = np.zeros((nb, 4, 2, 32), np.float32)
        for j in range(4):
            d1, m1 = d * sc[:, 2 * j:2 * j + 1].astype(np.float32), dmin * mn[:, 2 * j:2 * j + 1].astype(np.float32)
            d2, m2 = d * sc[:, 2 * j + 1:2 * j + 2].astype(np.float32), dmin * mn[:, 2 * j + 1:2 * j + 2].astype(np.float32)
            out[:, j, 0] = d1 * (q[:, j] & 15).astype(np.float32) - m1
            out[:, j, 1] = d2 * (q[:, j] >> 4).astype(np.float32) - m2
        return out.reshape(-1)
    if ty == Q5_K:
        d, dmin = _f16(b[:, 0:2])[:, None], _f16(b[:, 2:4])[:, None]
        sc, mn = _k4_scales(b[:, 4:16])
        qh = b[:, 16:48]
        ql = b[:, 48:176].reshape(nb, 4, 32)
        out = np.zeros((nb, 4, 2, 32), np.float32)
        for j in range(4):
            h1 = ((qh >> (2 * j)) & 1).astype(np.int32) * 16
            h2 = ((qh >> (2 * j + 1)) & 1).astype(np.int32) * 16
            d1, m1 = d * sc[:, 2 * j:2 * j + 1].astype(np.float32), dmin * mn[:, 2 * j:2 * j + 1].astype(np.float32)
            d2, m2 = d * sc[:, 2 * j + 1:2 * j + 2].astype(np.float32), dmin * mn[:, 2 * j + 1:2 * j + 2].astype(np.float32)
            out[:, j, 0] = d1 * ((ql[:, j] & 15).astype(np.int32) + h1).astype(np.float32) - m1
            out[:, j, 1] = d2 * ((ql[:, j] >> 4).astype(np.int32) + h2).astype(np.float32) - m2
        return out.reshape(-1)
    if ty == Q6_K:
        d = _f16(b[:, 208:210])[:, None]
        out = np.zeros((nb, 2, 4, 32), np.float32)
        for nn in range(2):
            ql = b[:, 64 * nn: 64 * nn + 64].astype(np.int32)
            qh = b[:, 128 + 32 * nn: 160 + 32 * nn].astype(np.int32)
            sc = b[:, 192 + 8 * nn: 200 + 8 * nn].view(np.int8).astype(np.float32)
            q1 = ((ql[:, :32] & 15) | ((qh & 3) << 4)) - 32
            q2 = ((ql[:, 32:] & 15) | (((qh >> 2) & 3) << 4)) - 32
            q3 = ((ql[:, :32] >> 4) | (((qh >> 4) & 3) << 4)) - 32
            q4 = ((ql[:, 32:] >> 4) | (((qh >> 6) & 3) << 4)) - 32
            isx = np.arange(32) // 16
            for k, qq in enumerate((q1, q2, q3, q4)):
                s = sc[:, isx + 2 * k]
                out[:, nn, k] = (d * s) * qq.astype(np.float32)
        return out.reshape(-1)
    if ty == Q2_K:
        scales = b[:, 0:16]
        q = b[:, 16:80]
        d, mn = _f16(b[:, 80:82])[:, None], _f16(b[:, 82:84])[:, None]
        out = np.zeros((nb, 256), np.float32)
        yi, is_ = 0, 0
        for nn in range(2):
            qq = q[:, 32 * nn:32 * nn + 32]
            for shift in (0, 2, 4, 6):
                for half in range(2):
                    sc = scales[:, is_:is_ + 1]
                    is_ += 1
                    dl, ml = d * (sc & 15).astype(np.float32), mn * (sc >> 4).astype(np.float32)
                    out[:, yi:yi + 16] = dl * ((qq[:, 16 * half:16 * half + 16] >> shift) & 3).astype(np.float32) - ml
                    yi += 16
        return out.reshape(-1)
    if ty == Q3_K:
        hm = b[:, 0:32]
        q = b[:, 32:96]
        s = b[:, 96:108]
        d_all = _f16(b[:, 108:110])[:, None]
        # 6-bit scales: low 4 bits from s[0:8] nibbles, high 2 bits from s[8:12]
        sc = np.zeros((nb, 16), np.int32)
        for i in range(16):
            low = (s[:, i] & 15) if i < 8 else (s[:, i - 8] >> 4)
            high = (s[:, 8 + (i % 4)] >> (2 * (i // 4))) & 3
            sc[:, i] = (low.astype(np.int32) | (high.astype(np.int32) << 4)) - 32
        out = np.zeros((nb, 256), np.float32)
        yi, is_, m = 0, 0, 1
        for nn in range(2):
            qq = q[:, 32 * nn:32 * nn + 32]
            for shift in (0, 2, 4, 6):
                for half in range(2):
                    dl = d_all * sc[:, is_:is_ + 1].astype(np.float32)
                    is_ += 1
                    idx = slice(16 * half, 16 * half + 16)
                    v = ((qq[:, idx] >> shift) & 3).astype(np.int32) - np.where(hm[:, idx] & m, 0, 4)
                    out[:, yi:yi + 16] = dl * v.astype(np.float32)
                    yi += 16
                m <<= 1
        return out.reshape(-1)
    raise ValueError(ty)


# ---- activation quantizers --------------------------------------------------------
def round_half_away(v: np.ndarray) -> np.ndarray:
    """Rust f32::round / C roundf, evaluated exactly in float64."""
    v64 = v.astype(np.float64)
    return np.sign(v64) * np.floor(np.abs(v64) + 0.5)


def quantize_q8_0_avx2(x: np.ndarray):
    """avx2.rs:153-184 → (qs int8 [nb,32], d f32 [nb], s f32 [nb])"""
    xb = np.asarray(x, np.float32).reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = np.rint(xb * idv[:, None]).astype(np.int64)  # RNE like _mm256_cvtps_epi32
    s = (d * q.sum(axis=1).astype(np.float32)).astype(np.float32)
    return np.clip(q, -127, 127).astype(np.int8), d, s


def quantize_q8_0_scalar(x: np.ndarray):
    """quant/mod.rs:175-189 (round half away from zero, s from the clamped codes)"""
    xb = np.asarray(x, np.float32).reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = np.clip(round_half_away(xb * idv[:, None]), -127, 127).astype(np.int64)
    s = (d * q.sum(axis=1).astype(np.float32)).astype(np.float32)
    return q.astype(np.int8), d, s


def quantize_q8_k(x: np.ndarray):
    """quant/mod.rs:191-218 → (qs int8 [nb,256], bsums int16 [nb,16], d f32 [nb])"""
    xb = np.asarray(x, np.float32).reshape(-1, 256)
    nb = xb.shape[0]
    idx = np.abs(xb).argmax(axis=1)  # first index of the largest |x|
    mx = xb[np.arange(nb), idx]
    qs = np.zeros((nb, 256), np.int8)
    d = np.zeros(nb, np.float32)
    nz = np.abs(mx) > 0
    iscale = np.zeros(nb, np.float32)
    iscale[nz] = (np.float32(-127.0) / mx[nz]).astype(np.float32)
    q = np.clip(round_half_away((iscale[:, None] * xb).astype(np.float32)), -127, 127)
    qs[nz] = q[nz].astype(np.int8)
    d[nz] = (np.float32(1.0) / iscale[nz]).astype(np.float32)
    bsums = qs.reshape(nb, 16, 16).astype(np.int32).sum(axis=2).astype(np.int16)
    return qs, bsums, d


def dequant_act(ty, x):
    """the activation values a kernel of weight type ty actually sees"""
    if ty in (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0):
        qs, d, _ = quantize_q8_0_avx2(x)
        return (qs.astype(np.float32) * d[:, None]).reshape(-1)
    if ty in (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K):
        qs, _, d = quantize_q8_k(x)
        return (qs.astype(np.float32) * d[:, None]).reshape(-1)
    return np.asarray(x, np.float32)
