"""Pins the oracle's unit functions against what the mathematics or an
independent implementation fixes: IEEE f16 rounding (numpy), hand-built known
answers for the quantizers, exact integer identities for the block dots, the
reference's own kernel tests (crates/rie-core/tests/kernels.rs) and the
TurboQuant invariants of turbo.rs:478-573.
"""
import math

import numpy as np
import pytest

import ggml_np as G

ALL_TYPES = [0, 1, 30, 2, 3, 6, 7, 8, 10, 11, 12, 13, 14]
BLOCK_TYPES = [2, 3, 6, 7, 8, 10, 11, 12, 13, 14]


# ---- f16 ------------------------------------------------------------------------
def test_f32_to_f16_is_ieee_round_to_nearest_even(oracle):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 4000).astype(np.float32),
        np.array([0.0, -0.0, 1.0, 65504.0, 65520.0, 65519.99, 1e-8, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                  2.0 ** -14, 2.0 ** -15 * 1.5, np.inf, -np.inf, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11], np.float32),
    ]).astype(np.float32)
    # exact ties in the normal range: mantissa ending in 1 followed by 12 zero bits
    ties = (np.arange(1, 200, dtype=np.uint32) << 13 | 0x1000 | 0x3F800000).view(np.float32)
    vals = np.concatenate([vals, ties, -ties])
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], np.uint16)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f16_to_f32_exact_for_every_half(oracle):
    L = oracle.lib()
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([L.or_f16_to_f32(int(v)) for v in h], np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))


# ---- Rng and random_weight (testing.rs:10-91) ------------------------------------
def _xorshift_py(seed, n):
    M = (1 << 64) - 1
    s = ((seed * 0x9E3779B97F4A7C15) & M) | 1
    out = []
    for _ in range(n):
        s ^= (s << 13) & M
        s ^= s >> 7
        s ^= (s << 17) & M
        out.append(s)
    return out


def test_rng_is_xorshift64_13_7_17(oracle):
    for seed in (0, 1, 7, 42, 0xDEADBEEF):
        r = oracle.Rng(seed)
        assert [r.next_u64() for _ in range(64)] == _xorshift_py(seed, 64)


def test_random_weight_layout_and_scales(oracle):
    """Block bytes are the little-endian Rng stream; scale fields are f16 in
    [k/2, k] with ~30% negative for signed formats (testing.rs:46-91)."""
    for ty, k, off in [(2, 0.01, [0]), (8, 0.001, [0]), (12, 0.001, [0, 2]), (14, 0.0001, [208])]:
        r = oracle.Rng(5)
        rows, cols = 64, 512
        w = r.random_weight(ty, rows, cols)
        bs, bb = G.BLOCK[ty]
        blocks = w.reshape(-1, bb)
        stream = np.array(_xorshift_py(5, (blocks.size + 7) // 8), np.uint64).view(np.uint8)[: blocks.size].reshape(-1, bb)
        mask = np.ones(bb, bool)
        for o in off:
            mask[o:o + 2] = False
        assert np.array_equal(blocks[:, mask], stream[:, mask])
        for i, o in enumerate(off):
            s = blocks[:, o:o + 2].copy().view(np.float16).astype(np.float32).reshape(-1)
            a = np.abs(s)
            assert a.min() >= np.float32(k * 0.5) * 0.999 and a.max() <= np.float32(k) * 1.001
            if i == 0 and ty in (2, 8, 14):
                frac = float((s < 0).mean())
                assert 0.2 < frac < 0.4
            else:
                assert (s > 0).all()


# ---- dequantization ---------------------------------------------------------------
@pytest.mark.parametrize("ty", ALL_TYPES)
def test_dequantize_matches_independent_numpy(oracle, ty):
    r = oracle.Rng(3)
    n = 1024
    w = r.random_weight(ty, 4, n)
    got = oracle.dequantize_row(ty, w, 4 * n)
    want = G.dequantize(ty, w, 4 * n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), ty


def test_q4_0_known_block(oracle):
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)  # d = 1.0
    blk[2:18] = np.arange(16, dtype=np.uint8) | (np.arange(15, -1, -1, dtype=np.uint8) << 4)
    y = oracle.dequantize_row(2, blk, 32)
    assert list(y[:16]) == [float(i - 8) for i in range(16)]
    assert list(y[16:]) == [float(15 - i - 8) for i in range(16)]


# Hand-built blocks for every other block layout.  Each block's fields are
# literal bytes chosen so that every scale, min, code and high bit differs from
# its neighbours; the expected values are read off the layouts of
# quant/reference.rs:8-215 by hand (scale/min unpacking: get_scale_min_k4 8-14,
# unpack_q3k_scales 30-51) and written either as literals or as the closed form
# "element i = scale(i)·code(i) − min(i)" of this particular block, so an index,
# nibble or shift slip in the oracle (or in the ggml_np transcription it is
# compared with) fails here.  d and min are powers of two: every expected value
# is exact in f32.
def _f16b(v):
    return list(np.array([v], np.float16).view(np.uint8))


def test_q4_1_known_block(oracle):
    # d = 0.5, m = -3.0, qs[j]: low nibble j, high nibble 15 - j
    blk = np.array(_f16b(0.5) + _f16b(-3.0) + [j | (15 - j) << 4 for j in range(16)], np.uint8)
    y = oracle.dequantize_row(3, blk, 32)
    assert np.array_equal(G.dequantize(3, blk, 32), y)  # the numpy transcription too
    assert list(y[:16]) == [j * 0.5 - 3 for j in range(16)]
    assert list(y[16:]) == [(15 - j) * 0.5 - 3 for j in range(16)]
    assert y[0] == -3.0 and y[15] == 4.5 and y[16] == 4.5 and y[31] == -3.0


def test_q5_0_known_block(oracle):
    # d = 1, qh = 0xFF005555 (bit j set for even j < 16, bits 24..31 set), qs[j] = j | (15-j) << 4
    blk = np.array(_f16b(1.0) + [0x55, 0x55, 0x00, 0xFF] + [j | (15 - j) << 4 for j in range(16)], np.uint8)
    y = oracle.dequantize_row(6, blk, 32)
    assert np.array_equal(G.dequantize(6, blk, 32), y)  # the numpy transcription too
    assert list(y[:16]) == [float(j if j % 2 == 0 else j - 16) for j in range(16)]
    assert list(y[16:]) == [float(-1 - j if j < 8 else 15 - j) for j in range(16)]
    assert list(y[:4]) == [0.0, -15.0, 2.0, -13.0] and list(y[22:26]) == [-7.0, -8.0, 7.0, 6.0]


def test_q5_1_known_block(oracle):
    # d = 0.25, m = 1, qh = 0x0F0F0F0F (bits 0-3, 8-11, 16-19, 24-27), qs[j] = (15-j) | j << 4
    blk = np.array(_f16b(0.25) + _f16b(1.0) + [0x0F] * 4 + [(15 - j) | j << 4 for j in range(16)], np.uint8)
    y = oracle.dequantize_row(7, blk, 32)
    assert np.array_equal(G.dequantize(7, blk, 32), y)  # the numpy transcription too
    hi = [16 if j % 8 < 4 else 0 for j in range(16)]
    assert list(y[:16]) == [((15 - j) + hi[j]) * 0.25 + 1 for j in range(16)]
    assert list(y[16:]) == [(j + hi[j]) * 0.25 + 1 for j in range(16)]
    assert y[0] == 8.75 and y[4] == 3.75 and y[16] == 5.0 and y[31] == 4.75


def test_q2_k_known_block(oracle):
    # scales[i] = i | (15 - i) << 4 (scale i, min 15 - i); code bytes 0xE4 (2-bit codes
    # 0,1,2,3 at shifts 0,2,4,6) at even and 0x1B (3,2,1,0) at odd positions; d = 1, min = 0.5
    blk = np.array([i | (15 - i) << 4 for i in range(16)] + [0xE4, 0x1B] * 32 + _f16b(1.0) + _f16b(0.5), np.uint8)
    assert blk.size == 84
    y = oracle.dequantize_row(10, blk, 256)
    assert np.array_equal(G.dequantize(10, blk, 256), y)  # the numpy transcription too
    for n in range(2):
        for it in range(4):
            for half in range(2):
                for l in range(16):
                    i = n * 8 + it * 2 + half
                    code = it if l % 2 == 0 else 3 - it
                    assert y[n * 128 + it * 32 + half * 16 + l] == i * code - 0.5 * (15 - i), (n, it, half, l)
    assert y[0] == -7.5 and y[1] == 0 * 3 - 7.5 and y[32 + 1] == 2 * 2 - 6.5 and y[254] == 15 * 3 - 0.0 and y[255] == 0.0


def test_q3_k_known_block(oracle):
    # 16 six-bit scales (before the -32 offset) 33 30 40 20 50 10 60 5 34 29 47 16 63 0 36 28,
    # packed as unpack_q3k_scales reads them: low nibbles of scales 0-7 / high nibbles of 8-15
    # in bytes 0-7, the top two bits of scales i, 4+i, 8+i, 12+i in byte 8+i
    sc_bytes = [0x21, 0xDE, 0xF8, 0x04, 0xF2, 0x0A, 0x4C, 0xC5, 0xEE, 0x11, 0xAE, 0x51]
    scales = [1, -2, 8, -12, 18, -22, 28, -27, 2, -3, 15, -16, 31, -32, 4, -4]
    hm = [0xA5 if i % 2 == 0 else 0x5A for i in range(32)]
    # 2-bit codes: 0xE4 (code = shift step) in the first 16 bytes of each 32-byte half, 0x1B
    # (3 - step) in the second; swapped for the second half
    q = [0xE4] * 16 + [0x1B] * 16 + [0x1B] * 16 + [0xE4] * 16
    blk = np.array(hm + q + sc_bytes + _f16b(1.0), np.uint8)
    assert blk.size == 110
    y = oracle.dequantize_row(11, blk, 256)
    assert np.array_equal(G.dequantize(11, blk, 256), y)  # the numpy transcription too
    for n in range(2):
        for it in range(4):
            for half in range(2):
                for l in range(16):
                    code = it if (half == 0) != (n == 1) else 3 - it
                    bit = (hm[l + 16 * half] >> (n * 4 + it)) & 1
                    want = scales[n * 8 + it * 2 + half] * (code - (0 if bit else 4))
                    assert y[n * 128 + it * 32 + half * 16 + l] == want, (n, it, half, l)
    # element 0: scale 1, code 0, hm bit 0 of 0xA5 set -> 0; element 1: hm 0x5A bit 0 clear -> 1·(0-4);
    # element 255: scale -4, code 3, bit 7 of 0x5A clear -> -4·(3-4)
    assert y[0] == 0.0 and y[1] == -4.0 and y[16] == -2 * 3 and y[255] == 4.0


# sc = 1 2 3 4 37 54 7 63, m = 9 10 11 12 45 22 19 50, packed as get_scale_min_k4 reads them
K4_SCALES = [0x81, 0xC2, 0x03, 0xC4, 0x89, 0x4A, 0x4B, 0xCC, 0xD5, 0x66, 0x37, 0x2F]
K4_SC, K4_M = [1, 2, 3, 4, 37, 54, 7, 63], [9, 10, 11, 12, 45, 22, 19, 50]


def test_q4_k_known_block(oracle):
    # d = 1, dmin = 0.5; code byte 32j+l: low nibble l % 16, high nibble (l + 5j) % 16
    qs = [(l % 16) | ((l + 5 * j) % 16) << 4 for j in range(4) for l in range(32)]
    blk = np.array(_f16b(1.0) + _f16b(0.5) + K4_SCALES + qs, np.uint8)
    assert blk.size == 144
    y = oracle.dequantize_row(12, blk, 256)
    assert np.array_equal(G.dequantize(12, blk, 256), y)  # the numpy transcription too
    for j in range(4):
        for l in range(32):
            assert y[64 * j + l] == K4_SC[2 * j] * (l % 16) - 0.5 * K4_M[2 * j], (j, l)
            assert y[64 * j + 32 + l] == K4_SC[2 * j + 1] * ((l + 5 * j) % 16) - 0.5 * K4_M[2 * j + 1], (j, l)
    assert y[0] == -4.5 and y[128 + 32 + 1] == 54 * 11 - 11.0 and y[255] == 63 * 14 - 25.0


def test_q5_k_known_block(oracle):
    # as the Q4_K block, plus high bits qh[l] = 0x93 (bits 0,1,4,7) for even l, 0x6C (2,3,5,6) for odd l
    qh = [0x93 if l % 2 == 0 else 0x6C for l in range(32)]
    ql = [(l % 16) | ((l + 5 * j) % 16) << 4 for j in range(4) for l in range(32)]
    blk = np.array(_f16b(1.0) + _f16b(0.5) + K4_SCALES + qh + ql, np.uint8)
    assert blk.size == 176
    y = oracle.dequantize_row(13, blk, 256)
    assert np.array_equal(G.dequantize(13, blk, 256), y)  # the numpy transcription too
    for j in range(4):
        for l in range(32):
            h1 = 16 * ((qh[l] >> (2 * j)) & 1)
            h2 = 16 * ((qh[l] >> (2 * j + 1)) & 1)
            assert y[64 * j + l] == K4_SC[2 * j] * ((l % 16) + h1) - 0.5 * K4_M[2 * j], (j, l)
            assert y[64 * j + 32 + l] == K4_SC[2 * j + 1] * (((l + 5 * j) % 16) + h2) - 0.5 * K4_M[2 * j + 1], (j, l)
    # element 0: qh[0] bit 0 set -> 1·(0+16) - 4.5; element 1: qh[1] = 0x6C bit 0 clear -> 1·1 - 4.5
    assert y[0] == 11.5 and y[1] == -3.5 and y[255] == 63 * (14 + 0) - 25.0


def test_q6_k_known_block(oracle):
    # ql[k]: low nibble k % 16, high nibble k // 16; qh[k] = 0xE4 for k < 32 (2-bit fields
    # 0,1,2,3), 0x1B for k >= 32 (3,2,1,0); signed scales 1 -2 3 -4 ... 15 -16; d = 1
    ql = [(k % 16) | (k // 16) << 4 for k in range(128)]
    qh = [0xE4] * 32 + [0x1B] * 32
    sc = [(i + 1) * (1 if i % 2 == 0 else -1) for i in range(16)]
    blk = np.array(ql + qh + [v & 0xFF for v in sc] + _f16b(1.0), np.uint8)
    assert blk.size == 210
    y = oracle.dequantize_row(14, blk, 256)
    assert np.array_equal(G.dequantize(14, blk, 256), y)  # the numpy transcription too
    for n in range(2):
        p = (0, 1, 2, 3) if n == 0 else (3, 2, 1, 0)
        for l in range(32):
            i = l // 16
            q1 = (l % 16) | p[0] << 4
            q2 = (l % 16) | p[1] << 4
            q3 = (4 * n + l // 16) | p[2] << 4
            q4 = (4 * n + 2 + l // 16) | p[3] << 4
            assert y[128 * n + l] == sc[8 * n + i] * (q1 - 32), (n, l)
            assert y[128 * n + l + 32] == sc[8 * n + i + 2] * (q2 - 32), (n, l)
            assert y[128 * n + l + 64] == sc[8 * n + i + 4] * (q3 - 32), (n, l)
            assert y[128 * n + l + 96] == sc[8 * n + i + 6] * (q4 - 32), (n, l)
    assert y[0] == -32.0 and y[255] == -16 * (7 - 32) and y[64] == 5 * (0 | 2 << 4) - 5 * 32


def test_turbo4_known_row(oracle):
    """quantize_rotated_4 (turbo.rs:140-164) on a hand-built rotated row of 128
    values: chunk c holds P[(g + 3c) % 8] in its first 16 values and -P[...] in
    its last 16, P = (2, -2, 1, -1, 0.5, -0.5, 0, 0).  rms = sqrt(1.3125); y/rms
    lands on levels 74, -74, 43, -43, 18, -18 and, for 0 (not above the zero
    midpoint), -6: codes 13, 2, 11, 4, 9, 6, 7.  The least-squares scale is
    (Σ y·c)/(Σ c²) = 46·400/15370 = 1.19714 -> f16 0x3CCA.  Codes go in Q4_0
    nibble order: byte 16c + j holds value 32c + j (low) and 32c + 16 + j (high)."""
    P = [2.0, -2.0, 1.0, -1.0, 0.5, -0.5, 0.0, 0.0]
    y = np.array([P[(g + 3 * (g // 32)) % 8] * (1 if g % 32 < 16 else -1) for g in range(128)], np.float32)
    out = np.zeros(66, np.uint8)
    oracle.lib().or_turbo_quantize_rotated(oracle.ptr(y), 128, oracle.ptr(out))
    T = [0x2D, 0xD2, 0x4B, 0xB4, 0x69, 0x96, 0x77, 0x77]
    assert list(out[:2]) == [0xCA, 0x3C]
    assert list(out[2:]) == [T[(j + 3 * c) % 8] for c in range(4) for j in range(16)]
    assert oracle.turbo_row_bytes(128) == 66 and oracle.turbo_row_bytes(96) == 54  # turbo.rs:571-572


# ---- activation quantizers ---------------------------------------------------------------
def test_q8_0_known_answers(oracle):
    x = np.zeros(64, np.float32)
    x[32:] = [127.0, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, -127.0] + [0.0] * 24  # d = 1, id = 1: exact ties
    q = oracle.quantize_q8_0(x)
    assert q[0]["d"] == 0 and q[0]["s"] == 0 and not q[0]["qs"].any()
    assert list(q[1]["qs"][:8]) == [127, 2, 4, -2, 0, 0, 2, -127]  # round half to even (AVX2)
    assert q[1]["d"] == np.float32(1.0) and q[1]["s"] == np.float32(6.0)
    qs = oracle.quantize_q8_0(x, scalar=True)  # RIE_DISABLE=simd: round half away from zero
    assert list(qs[1]["qs"][:8]) == [127, 3, 4, -3, 1, -1, 2, -127]


def test_q8_0_matches_numpy_restatement(oracle):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(32 * 500) * rng.uniform(0.01, 50, 32 * 500)).astype(np.float32)
    x[:32] = 0
    q = oracle.quantize_q8_0(x)
    qs, d, s = G.quantize_q8_0_avx2(x)
    assert np.array_equal(q["qs"], qs) and np.array_equal(q["d"], d) and np.array_equal(q["s"], s)
    q = oracle.quantize_q8_0(x, scalar=True)
    qs, d, s = G.quantize_q8_0_scalar(x)
    assert np.array_equal(q["qs"], qs) and np.array_equal(q["d"], d) and np.array_equal(q["s"], s)


def test_q8_k_known_answers(oracle):
    x = np.zeros(768, np.float32)
    x[256 + 3], x[256 + 10] = -2.0, 2.0  # first strictly-largest |x| is negative → d > 0
    x[512 + 1], x[512 + 9] = 2.0, -2.0   # first is positive → d < 0
    x[512 + 20] = 0.5
    q = oracle.quantize_q8_k(x)
    assert q[0]["d"] == 0 and not q[0]["qs"].any() and not q[0]["bsums"].any()
    assert q[1]["d"] == np.float32(1.0) / np.float32(63.5)
    assert q[1]["qs"][3] == -127 and q[1]["qs"][10] == 127
    assert q[2]["d"] == np.float32(1.0) / np.float32(-63.5)
    assert q[2]["qs"][1] == -127 and q[2]["qs"][9] == 127
    assert q[2]["qs"][20] == -32  # -63.5*0.5 = -31.75 → -32
    assert q[2]["bsums"][0] == -127 + 127 and q[2]["bsums"][1] == -32


def test_q8_k_matches_numpy_restatement(oracle):
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(256 * 100) * 3).astype(np.float32)
    q = oracle.quantize_q8_k(x)
    qs, bsums, d = G.quantize_q8_k(x)
    assert np.array_equal(q["qs"], qs) and np.array_equal(q["bsums"], bsums) and np.array_equal(q["d"], d)


# ---- int8 block dots ------------------------------------------------------------------------
def _reference_dot(oracle, ty, w, x):
    """tests/kernels.rs:10-29: dequantized weights · the quantized activation, in f64"""
    n = x.size
    wf = G.dequantize(ty, w, n).astype(np.float64)
    xa = G.dequant_act(ty, x).astype(np.float64)
    return float(wf @ xa), float(np.abs(wf * x.astype(np.float64)).sum())


@pytest.mark.parametrize("ty", ALL_TYPES)
def test_vec_dot_matches_dequantized_reference(oracle, ty):
    """tests/kernels.rs:36-64 with the reference's tolerance 1e-4·Σ|w·x| + 1e-5"""
    r = oracle.Rng(7)
    for n in (256, 512, 768, 2048):
        for _ in range(4):
            w = r.random_weight(ty, 1, n)
            x = (np.random.default_rng(n).uniform(-1, 1, n) * 2).astype(np.float32)
            act = oracle.quantize_act(ty, x)
            got = oracle.vec_dot(ty, w, act, n)
            want, mag = _reference_dot(oracle, ty, w, x)
            assert abs(got - want) <= 1e-4 * mag + 1e-5, (ty, n, got, want)


@pytest.mark.parametrize("ty", [2, 8, 6])
def test_block_idots_are_exact_integer_dots(oracle, ty):
    """For symmetric formats w_j = d_w·c_j exactly, so Σ_j w_j·q_j = d_w·idot in f64."""
    r = oracle.Rng(11)
    n = 2048
    w = r.random_weight(ty, 1, n)
    x = np.random.default_rng(3).standard_normal(n).astype(np.float32)
    act = oracle.quantize_q8_0(x)
    idots = oracle.block_idots(ty, w, act, n)
    wf = G.dequantize(ty, w, n).astype(np.float64).reshape(-1, 32)
    bs, bb = G.BLOCK[ty]
    d = w.reshape(-1, bb)[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1)
    lhs = (wf * act["qs"].astype(np.float64)).sum(axis=1)
    assert np.array_equal(lhs, d * idots.astype(np.float64))


@pytest.mark.parametrize("ty", [12, 13, 14])
def test_kquant_block_idots_decomposition(oracle, ty):
    """d·sumi − dmin·summ reproduces Σ dequant(w)·q to float precision; a wrong
    sub-block index or scale would miss by O(1)."""
    r = oracle.Rng(13)
    n = 2048
    w = r.random_weight(ty, 1, n)
    x = np.random.default_rng(4).standard_normal(n).astype(np.float32)
    act = oracle.quantize_q8_k(x)
    ints = oracle.block_idots(ty, w, act, n).reshape(-1, 2).astype(np.float64)
    bb = G.BLOCK[ty][1]
    blk = w.reshape(-1, bb)
    if ty == 14:
        d = blk[:, 208:210].copy().view(np.float16).astype(np.float64).reshape(-1)
        approx = d * ints[:, 0]
    else:
        d = blk[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1)
        dm = blk[:, 2:4].copy().view(np.float16).astype(np.float64).reshape(-1)
        approx = d * ints[:, 0] - dm * ints[:, 1]
    wf = G.dequantize(ty, w, n).astype(np.float64).reshape(-1, 256)
    exact = (wf * act["qs"].astype(np.float64)).sum(axis=1)
    assert np.allclose(approx, exact, rtol=1e-5, atol=1e-6 * np.abs(wf).sum(axis=1).max())


def test_float_kernels(oracle):
    """tests/kernels.rs:120-142"""
    L = oracle.lib()
    rng = np.random.default_rng(5)
    for n in (1, 7, 8, 15, 16, 33, 128, 1000):
        a = rng.uniform(-1, 1, n).astype(np.float32)
        b = rng.uniform(-1, 1, n).astype(np.float32)
        assert abs(L.or_dot_f32(oracle.ptr(a), oracle.ptr(b), n) - float(a.astype(np.float64) @ b)) < 1e-4 * n
        h = a.astype(np.float16)
        hb = np.ascontiguousarray(h.view(np.uint16))
        ah = h.astype(np.float64)
        assert abs(L.or_dot_f16_f32(oracle.ptr(hb), oracle.ptr(b), n) - float(ah @ b)) < 1e-4 * n
        y = b.copy()
        L.or_axpy_f16(oracle.ptr(y), 0.5, oracle.ptr(hb), n)
        assert np.abs(y - (b + 0.5 * ah)).max() < 1e-5


# ---- ops -------------------------------------------------------------------------------------
def test_rope_matches_complex_rotation(oracle):
    """ops.rs:115-130"""
    import ctypes as C
    L = oracle.lib()
    inv = np.zeros(4, np.float32)
    L.or_rope_inv_freq(8, 10000.0, 1.0, None, 0, oracle.ptr(inv))
    want = np.float32(10000.0) ** (np.float32(-2.0) * np.arange(4, dtype=np.float32) / np.float32(8))
    assert np.allclose(inv, want, rtol=2e-7)
    c, s = np.zeros(4, np.float32), np.zeros(4, np.float32)
    L.or_rope_table(oracle.ptr(inv), 4, 5, oracle.ptr(c), oracle.ptr(s))
    x0 = (np.arange(8, dtype=np.float32) * np.float32(0.3) - 1).astype(np.float32)
    x = x0.copy()
    L.or_rope_apply(oracle.ptr(x), 8, 0, oracle.ptr(c), oracle.ptr(s))
    assert abs((x0 ** 2).sum() - (x ** 2).sum()) < 1e-4
    assert abs(x[0] - (x0[0] * math.cos(5) - x0[1] * math.sin(5))) < 1e-5
    # NEOX pairs (i, i+d/2)
    y = x0.copy()
    L.or_rope_apply(oracle.ptr(y), 8, 1, oracle.ptr(c), oracle.ptr(s))
    z = (x0[:4] + 1j * x0[4:]) * np.exp(1j * 5.0 * inv.astype(np.float64))
    assert np.allclose(y[:4], z.real, atol=1e-5) and np.allclose(y[4:], z.imag, atol=1e-5)


def test_softmax_sums_to_one(oracle):
    v = np.array([1.0, 2.0, 3.0, -1000.0], np.float32)
    oracle.lib().or_softmax(oracle.ptr(v), 4)
    assert abs(v.sum() - 1) < 1e-6 and v[3] == 0


# ---- TurboQuant (turbo.rs) ---------------------------------------------------------------------
LM4 = [0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6180, 2.0690, 2.7326]
KV_LEVELS_I8 = [-126, -95, -74, -58, -43, -30, -18, -6, 6, 18, 30, 43, 58, 74, 95, 126]


def test_lloyd_max_levels_and_int8_table():
    """turbo.rs:493-512: each level is the conditional mean of N(0,1) over its
    cell; the int8 table is round(46·level) (turbo.rs:126-127)."""
    c = [-v for v in reversed(LM4)] + LM4
    phi = lambda t: math.exp(-0.5 * t * t) / math.sqrt(2 * math.pi)
    for i in range(16):
        lo = -12.0 if i == 0 else 0.5 * (c[i - 1] + c[i])
        hi = 12.0 if i == 15 else 0.5 * (c[i] + c[i + 1])
        xs = np.linspace(lo, hi, 20001)
        w = np.exp(-0.5 * xs * xs)
        assert abs((xs * w).sum() / w.sum() - c[i]) < 2e-3
    assert [int(round(46 * v)) for v in c] == KV_LEVELS_I8


def _splitmix_sign(seed, i):
    M = (1 << 64) - 1
    z = (seed + i * 0x9E3779B97F4A7C15) & M
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
    return 1.0 if ((z ^ (z >> 31)) & 1) == 0 else -1.0


def _hadamard(n):
    H = np.array([[1.0]])
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H


@pytest.mark.parametrize("d", [64, 96, 128, 80])
def test_rotation_is_block_hadamard_times_signs(oracle, d):
    """R = H·D per power-of-two block (turbo.rs:91-118), orthogonal and undone by Rᵀ."""
    b = oracle.lib().or_turbo_block_size(d)
    assert b == max(p for p in (1, 2, 4, 8, 16, 32, 64, 128, 256) if d % p == 0)
    signs = np.array([_splitmix_sign(7, i) for i in range(d)])
    R = np.zeros((d, d))
    for o in range(0, d, b):
        R[o:o + b, o:o + b] = _hadamard(b) / math.sqrt(b)
    R = R @ np.diag(signs)
    x = np.random.default_rng(d).uniform(-0.5, 0.5, d).astype(np.float32)
    y = oracle.turbo_rotate(x, seed=7)
    assert np.allclose(y, R @ x, atol=1e-6)
    assert np.allclose(oracle.turbo_rotate(y, seed=7, inverse=True), x, atol=1e-5)


def _turbo_quantize_rotated_np(y):
    """turbo.rs:140-164 for one 128-block, with sequential float32 sums"""
    c = (np.array(KV_LEVELS_I8, np.float32) / np.float32(46.0)).astype(np.float32)
    mids = (np.float32(0.5) * (c[:-1] + c[1:])).astype(np.float32)
    sq = np.cumsum((y * y).astype(np.float32), dtype=np.float32)[-1]
    rms = np.sqrt(np.float32(sq / np.float32(y.size)), dtype=np.float32)
    inv = np.float32(1.0) / rms if rms > 0 else np.float32(0.0)
    q = (((y * inv).astype(np.float32))[:, None] > mids[None, :]).sum(axis=1)
    num = np.cumsum((y * c[q]).astype(np.float32), dtype=np.float32)[-1]
    den = np.cumsum((c[q] * c[q]).astype(np.float32), dtype=np.float32)[-1]
    s = np.float32(num / den) if den > 0 else np.float32(0)
    codes = np.zeros(y.size // 2, np.uint8)
    for g in range(y.size):
        codes[(g // 32) * 16 + g % 16] |= np.uint8(q[g] << ((g % 32) // 16 * 4))
    return np.concatenate([np.array([s], np.float16).view(np.uint8), codes])


def test_turbo_codes_match_numpy_restatement(oracle):
    rng = np.random.default_rng(9)
    for _ in range(50):
        x = rng.standard_normal(128).astype(np.float32) * np.float32(rng.uniform(0.01, 10))
        y = oracle.turbo_rotate(x)
        row = oracle.turbo_quantize(x)
        assert np.array_equal(row, _turbo_quantize_rotated_np(y))


def test_four_bit_rows_accurate_with_outliers_and_dot_identities(oracle):
    """turbo.rs:532-573"""
    d = 128
    assert oracle.turbo_row_bytes(128) == 66 and oracle.turbo_row_bytes(96) == 54
    rng = np.random.default_rng(3)
    rel = 0.0
    L = oracle.lib()
    for _ in range(50):
        x = (rng.uniform(0, 1, d) - 0.5).astype(np.float32)
        x[5], x[77] = 20.0, -9.0
        row = oracle.turbo_quantize(x)
        y = oracle.turbo_dequantize(row, d)
        rel += math.sqrt(float(((x - y) ** 2).sum() / (x ** 2).sum()))
        q = (rng.uniform(0, 1, d) - 0.5).astype(np.float32)
        direct = float(q.astype(np.float64) @ y)
        qr = oracle.turbo_rotate(q)
        qq = oracle.quantize_q8_0(qr)
        deq = (qq["qs"].astype(np.float32) * qq["d"][:, None]).reshape(-1)
        yr = np.zeros(d, np.float32)
        L.or_turbo_axpy(oracle.ptr(yr), d, 1.0, oracle.ptr(row))
        exact = float(deq.astype(np.float64) @ yr)
        got = L.or_turbo_dot(oracle.ptr(qq), d, oracle.ptr(row))
        assert abs(got - exact) < 1e-3 * (1 + abs(exact))
        assert abs(exact - direct) < 0.01 * np.linalg.norm(q) * np.linalg.norm(y)
    assert rel / 50 < 0.12


def test_quantize_weights_roundtrip(oracle):
    """tests/kernels.rs:107-118"""
    x = np.random.default_rng(3).uniform(-1, 1, 1024).astype(np.float32)
    for ty, tol in ((8, 0.01), (2, 0.15)):
        y = G.dequantize(ty, oracle.quantize_weights(ty, x), 1024)
        assert np.abs(y - x).max() <= tol * np.abs(x).max()


# ---- MoE routing (model/cpu.rs:492-500) ---------------------------------------------------------
def _route_numpy(logits, k, norm_topk=True, unit_weights=False):
    """Independent restatement: f64 softmax, then a stable sort on (-p, index)."""
    sel, wgt = [], []
    for row in logits.astype(np.float64):
        p = np.exp(row - row.max())
        p /= p.sum()
        order = np.lexsort((np.arange(p.size), -p))[:k]
        w = np.ones(k) if unit_weights else (p[order] / p[order].sum() if norm_topk else p[order])
        asc = np.argsort(order)
        sel.append(order[asc])
        wgt.append(w[asc])
    return np.array(sel, np.int32), np.array(wgt)


def test_moe_route_known_answers(oracle):
    nan, inf = np.nan, np.inf
    # equal top pair: index order, weights exactly 1/2
    s, w = oracle.moe_route(np.array([[0, 2, 2, 1]], np.float32), 2)
    assert s.tolist() == [[1, 2]] and w.tolist() == [[0.5, 0.5]]
    # a three-way tie keeps the two lowest indices
    s, _ = oracle.moe_route(np.array([[1, 1, 1, 0]], np.float32), 2)
    assert s.tolist() == [[0, 1]]
    # -Inf logits get probability 0; the zero tie is broken by index
    s, w = oracle.moe_route(np.array([[-inf, 0, -inf, 0]], np.float32), 3)
    assert s.tolist() == [[0, 1, 3]] and w.tolist() == [[0.0, 0.5, 0.5]]
    # NaN, +Inf, or every logit -Inf: the softmax is NaN everywhere, every pair
    # compares Equal, so the first k experts are taken, with NaN weights
    for row in ([0, nan, 3, 1], [0, inf, 3, 1], [-inf] * 4):
        s, w = oracle.moe_route(np.array([row], np.float32), 2)
        assert s.tolist() == [[0, 1]] and np.isnan(w).all()
        s, w = oracle.moe_route(np.array([row], np.float32), 2, unit_weights=True)
        assert s.tolist() == [[0, 1]] and w.tolist() == [[1.0, 1.0]]
    # without renormalization the weights are the probabilities: e/(e+1+...) closed form
    s, w = oracle.moe_route(np.array([[1, 0]], np.float32), 1, norm_topk=False)
    assert s.tolist() == [[0]] and abs(w[0, 0] - np.e / (np.e + 1)) < 1e-6


def test_moe_route_matches_numpy_restatement(oracle):
    rng = np.random.default_rng(11)
    for n_exp, k in ((8, 2), (64, 6), (128, 8), (60, 4)):
        logits = (rng.integers(-6, 7, size=(40, n_exp)) * 0.5).astype(np.float32)  # many exact ties
        logits[::3] = rng.standard_normal((len(logits[::3]), n_exp)).astype(np.float32)
        for norm_topk, unit in ((True, False), (False, False), (True, True)):
            s, w = oracle.moe_route(logits, k, norm_topk, unit)
            s2, w2 = _route_numpy(logits, k, norm_topk, unit)
            assert np.array_equal(s, s2)
            np.testing.assert_allclose(w, w2, rtol=2e-6, atol=1e-7)
