"""Parity of the HIP path (through the C ABI) with the oracle on MI355X.

Bit-exact on identical inputs: Q8_0 / Q8_K activation codes and scales, the
per-block integer dot products, f16 / Q8_0 / Turbo4 KV codes, argmax.
Float results: GEMV rows within the reference's kernel tolerance
(tests/kernels.rs:60: 1e-4·Σ|w·x| + 1e-5), whole-model logits within the
reference's whole-model tolerances (tests/model.rs:340-375: 3e-3 f16, 0.03
quantized; 0.05 Q8_0 KV), greedy sequences identical.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

import rust_interference_engine_amd as R  # noqa: E402
from rust_interference_engine_amd import synth  # noqa: E402

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K, BF16 = 3, 6, 7, 10, 11, 13, 30
ALL_TYPES = [Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, F32, F16, BF16]


def act_fmt(ty):
    """activation format a weight type consumes (quant/mod.rs:118-124): 0 f32, 1 Q8_0, 2 Q8_K"""
    return 0 if ty in (F32, F16, BF16) else (2 if ty in (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K) else 1)


@pytest.fixture(scope="module")
def cuda():
    assert torch.cuda.is_available(), "these tests need the MI355X"
    return torch.device("cuda:0")


def dev(a: np.ndarray, cuda):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def host(t):
    return t.cpu().numpy()


def _quant_on_gpu(x, fmt, cuda, w=None, eps=1e-6):
    n, k = x.shape
    L = R.lib()
    xd = dev(x.astype(np.float32), cuda)
    wd = dev(w.astype(np.float32), cuda) if w is not None else None
    qs = torch.zeros(n * k, dtype=torch.int8, device=cuda)
    xn = torch.zeros(n * k, dtype=torch.float32, device=cuda)
    if fmt == 1:
        d = torch.zeros(n * k // 32, dtype=torch.float32, device=cuda)
        s = torch.zeros_like(d)
        isum = torch.zeros(n * k // 32, dtype=torch.int32, device=cuda)
        rc = L.rie_hip_k_rmsnorm_quant(xd.data_ptr(), wd.data_ptr() if wd is not None else None, eps, n, k, 1, xn.data_ptr(),
                                       qs.data_ptr(), d.data_ptr(), s.data_ptr(), isum.data_ptr(), None)
        assert rc == 0
        return dict(qs=host(qs).reshape(n, k), d=host(d), s=host(s), isum=host(isum), xn=host(xn).reshape(n, k),
                    dev=(qs, d, s, isum, None))
    d = torch.zeros(n * k // 256, dtype=torch.float32, device=cuda)
    bs = torch.zeros(n * k // 16, dtype=torch.int16, device=cuda)
    rc = L.rie_hip_k_rmsnorm_quant(xd.data_ptr(), wd.data_ptr() if wd is not None else None, eps, n, k, 2, xn.data_ptr(),
                                   qs.data_ptr(), d.data_ptr(), None, None, bs.data_ptr())
    assert rc == 0
    return dict(qs=host(qs).reshape(n, k), d=host(d), bsums=host(bs), xn=host(xn).reshape(n, k), dev=(qs, d, None, None, bs))


def _act_inputs(rng, n, k):
    x = (rng.standard_normal((n, k)) * rng.uniform(0.01, 20, (n, 1))).astype(np.float32)
    x[0, :32] = 0.0                                   # zero block
    x[0, 32:64] = np.arange(32, dtype=np.float32) - 15.5
    x[0, 64] = 127.0                                  # exact ties at id = 1
    x[0, 65:72] = [2.5, 3.5, -2.5, 0.5, -0.5, 1.5, -126.5]
    return x


def test_q8_0_activation_codes_bit_exact(oracle, cuda):
    rng = np.random.default_rng(0)
    for n, k in ((1, 256), (3, 4096), (5, 14336)):
        x = _act_inputs(rng, n, k)
        g = _quant_on_gpu(x, 1, cuda)
        for t in range(n):
            ref = oracle.quantize_q8_0(x[t])
            assert np.array_equal(g["qs"][t], ref["qs"].reshape(-1))
            nb = k // 32
            assert np.array_equal(g["d"][t * nb:(t + 1) * nb].view(np.uint32), ref["d"].view(np.uint32))
            assert np.array_equal(g["s"][t * nb:(t + 1) * nb].view(np.uint32), ref["s"].view(np.uint32))
            assert np.array_equal(g["isum"][t * nb:(t + 1) * nb], ref["qs"].astype(np.int32).sum(axis=1))


def test_q8_k_activation_codes_bit_exact(oracle, cuda):
    rng = np.random.default_rng(1)
    for n, k in ((1, 256), (4, 4096)):
        x = _act_inputs(rng, n, k)
        if k >= 1024:
            x[n - 1, 256:512] = 0.0
            x[n - 1, 512 + 3], x[n - 1, 512 + 10] = -7.0, 7.0  # first-max tie
        g = _quant_on_gpu(x, 2, cuda)
        for t in range(n):
            ref = oracle.quantize_q8_k(x[t])
            nb = k // 256
            assert np.array_equal(g["qs"][t], ref["qs"].reshape(-1))
            assert np.array_equal(g["d"][t * nb:(t + 1) * nb].view(np.uint32), ref["d"].view(np.uint32))
            assert np.array_equal(g["bsums"][t * k // 16:(t + 1) * k // 16], ref["bsums"].reshape(-1))


@pytest.mark.parametrize("k", [256, 2048, 4096, 14336, 4128])
def test_rmsnorm_then_quant_bitwise(oracle, cuda, k):
    """RMSNorm with the reference's summation order (ops.rs:7-14 over kernels/
    avx2.rs:186-203; 4128 leaves a partial 8-step group) then Q8_0 / Q8_K: the
    normalized rows, codes and scales equal the oracle's bit for bit on the
    same input rows.  Rows of dequantized Q4_0 weights (the first layer's input
    in a Q4_0 model) put many values on exact quantizer ties, where a
    reduction-order difference of one ulp in the norm would flip codes."""
    rng = np.random.default_rng(2 + k)
    n = 4
    x = rng.standard_normal((n, k)).astype(np.float32)
    blk = (np.round(rng.standard_normal((n, k)) * 3).clip(-8, 7) * 0.0123).astype(np.float32)  # Q4_0-like rows
    x[n // 2:] = blk[n // 2:]
    for w in ((1 + 0.1 * rng.uniform(-1, 1, k)).astype(np.float32), np.ones(k, np.float32)):
        L = oracle.lib()
        for fmt in (1, 2):
            if fmt == 2 and k % 256:
                continue
            g = _quant_on_gpu(x, fmt, cuda, w=w)
            for t in range(n):
                ref = np.zeros(k, np.float32)
                L.or_rmsnorm(oracle.ptr(ref), oracle.ptr(np.ascontiguousarray(x[t])), oracle.ptr(w), k, 1e-6)
                assert np.array_equal(g["xn"][t].view(np.uint32), ref.view(np.uint32)), (k, fmt, t)
                q = oracle.quantize_q8_0(ref) if fmt == 1 else oracle.quantize_q8_k(ref)
                assert np.array_equal(g["qs"][t], q["qs"].reshape(-1)), (k, fmt, t)
                nb = k // 32 if fmt == 1 else k // 256
                assert np.array_equal(g["d"][t * nb:(t + 1) * nb].view(np.uint32), q["d"].view(np.uint32)), (k, fmt, t)


def _gemv(ty, w, rows, k, act, act_f32, n_tok, cuda, gemm=False):
    L = R.lib()
    # an exact-size buffer: the entry points pad a copy for the kernels' word reads
    wd = dev(np.ascontiguousarray(w, dtype=np.uint8), cuda)
    out = torch.zeros(n_tok * rows, dtype=torch.float32, device=cuda)
    qs, d, s, isum, bs = act if act is not None else (None,) * 5
    p = lambda t: t.data_ptr() if t is not None else None
    fd = dev(act_f32, cuda) if act_f32 is not None else None
    if gemm:
        rc = L.rie_hip_k_gemm(ty, wd.data_ptr(), rows, k, p(qs), p(d), p(s), p(isum), p(bs), n_tok, out.data_ptr())
    else:
        rc = L.rie_hip_k_gemv(ty, wd.data_ptr(), rows, k, p(qs), p(d), p(s), p(isum), p(bs), p(fd), n_tok, out.data_ptr())
    assert rc == 0
    return host(out).reshape(n_tok, rows)


@pytest.mark.parametrize("ty", ALL_TYPES)
def test_gemv_matches_oracle_rows(oracle, cuda, ty):
    import ggml_np as G
    r = oracle.Rng(21 + ty)
    for k in (256, 2048, 4096):
        rows = 96
        w = r.random_weight(ty, rows, k)
        for n_tok in (1, 3, 6, 37):  # 37: the batched GEMV splits the tokens into groups of 16 (the last partial)
            x = (np.random.default_rng(k + n_tok).uniform(-1, 1, (n_tok, k)) * 2).astype(np.float32)
            fmt = act_fmt(ty)
            act = _quant_on_gpu(x, fmt, cuda)["dev"] if fmt else None
            got = _gemv(ty, w, rows, k, act, x if fmt == 0 else None, n_tok, cuda)
            wf = G.dequantize(ty, w, rows * k).reshape(rows, k).astype(np.float64)
            for t in range(n_tok):
                a = oracle.quantize_act(ty, x[t])
                rb = G.row_bytes(ty, k)
                want = np.array([oracle.vec_dot(ty, w[i * rb:(i + 1) * rb], a, k) for i in range(rows)])
                mag = np.abs(wf * x[t].astype(np.float64)).sum(axis=1)
                assert np.all(np.abs(got[t] - want) <= 1e-5 * mag + 1e-6), (ty, k, n_tok)


@pytest.mark.parametrize("ty", [Q4_0, Q8_0, Q4_K, Q6_K])
def test_gemm_matches_oracle_rows(oracle, cuda, ty):
    """The int8-MFMA prompt GEMM against the oracle's block dots, for row and
    token counts that are not multiples of the 32×32 tiles (Q4_K: Q8_K
    activations, superblock sums with the 6-bit scales and mins; Q6_K: signed
    16-value sub-block scales on K=16 MFMAs)."""
    import ggml_np as G
    r = oracle.Rng(31 + ty)
    shapes = ((128, 40, 9), (256, 200, 33), (4096, 96, 70), (1024, 300, 130))
    if ty in (Q4_0, Q8_0):
        # long K over few tiles: K split in four (65 stages of 128: splits of 16,
        # 16, 16 and 17 stages; 112 stages with a partial 128-token tile), and in
        # two (48 stages, the shortest K that splits)
        shapes += ((8320, 96, 200), (14336, 64, 130), (6144, 96, 130))
    if ty in (Q4_K, Q6_K):
        shapes = ((256, 40, 9), (512, 200, 33), (4096, 96, 70), (1024, 300, 130), (8192, 64, 512))
    if ty in (Q4_K, Q6_K):  # K split: 13 superblocks in two uneven splits (6 and 7)
        shapes += ((3328, 96, 70),)
    for k, rows, n_tok in shapes:
        w = r.random_weight(ty, rows, k)
        x = (np.random.default_rng(k + n_tok).uniform(-1, 1, (n_tok, k)) * 2).astype(np.float32)
        act = _quant_on_gpu(x, act_fmt(ty), cuda)["dev"]
        got = _gemv(ty, w, rows, k, act, None, n_tok, cuda, gemm=True)
        wf = G.dequantize(ty, w, rows * k).reshape(rows, k).astype(np.float64)
        rb = G.row_bytes(ty, k)
        for t in range(n_tok):
            a = oracle.quantize_act(ty, x[t])
            want = np.array([oracle.vec_dot(ty, w[i * rb:(i + 1) * rb], a, k) for i in range(rows)])
            mag = np.abs(wf * x[t].astype(np.float64)).sum(axis=1)
            assert np.all(np.abs(got[t] - want) <= 1e-5 * mag + 1e-6), (ty, k, rows, n_tok, t)


@pytest.mark.parametrize("ty", [Q4_0, Q8_0])
def test_gemm_per_block_integer_dots_exact(oracle, cuda, ty):
    """One non-zero activation block per token: every GEMM output is one rounding
    of (d_w·d_a)·idot, the reference's per-block term, for 40 tokens at once."""
    r = oracle.Rng(6)
    k, rows, n_tok = 1024, 64, 40
    w = r.random_weight(ty, rows, k)
    rng = np.random.default_rng(8)
    x = np.zeros((n_tok, k), np.float32)
    blocks = rng.integers(0, k // 32, n_tok)
    for t in range(n_tok):
        x[t, blocks[t] * 32:(blocks[t] + 1) * 32] = rng.standard_normal(32) * 3
    act = _quant_on_gpu(x, 1, cuda)
    got = _gemv(ty, w, rows, k, act["dev"], None, n_tok, cuda, gemm=True)
    rb = (18 if ty == Q4_0 else 34) * k // 32
    for t in range(n_tok):
        b = blocks[t]
        a = oracle.quantize_q8_0(x[t])
        for i in range(rows):
            idots = oracle.block_idots(ty, w[i * rb:(i + 1) * rb], a, k)
            blk = w[i * rb + b * (rb * 32 // k): i * rb + b * (rb * 32 // k) + 2]
            dw = np.frombuffer(blk.tobytes(), np.float16)[0].astype(np.float32)
            want = np.float32(np.float32(dw * a["d"][b]) * np.float32(idots[b]))
            assert got[t, i] == want, (t, b, i)


@pytest.mark.parametrize("ty", [Q4_0, Q8_0])
def test_gemv_per_block_integer_dots_exact(oracle, cuda, ty):
    """With one non-zero activation block the row result is one rounding of
    (d_w·d_a)·idot, so it pins every per-block int32 dot exactly."""
    r = oracle.Rng(5)
    k, rows = 2048, 64
    w = r.random_weight(ty, rows, k)
    rng = np.random.default_rng(7)
    for b in (0, 1, 17, k // 32 - 1):
        x = np.zeros((1, k), np.float32)
        x[0, b * 32:(b + 1) * 32] = rng.standard_normal(32) * 3
        act = _quant_on_gpu(x, 1, cuda)
        got = _gemv(ty, w, rows, k, act["dev"], None, 1, cuda)[0]
        a = oracle.quantize_q8_0(x[0])
        rb = (18 if ty == Q4_0 else 34) * k // 32
        for i in range(rows):
            idots = oracle.block_idots(ty, w[i * rb:(i + 1) * rb], a, k)
            blk = w[i * rb + b * (rb * 32 // k): i * rb + b * (rb * 32 // k) + 2]
            dw = np.frombuffer(blk.tobytes(), np.float16)[0].astype(np.float32)
            want = np.float32(np.float32(dw * a["d"][b]) * np.float32(idots[b]))
            assert got[i] == want, (b, i)


def test_argmax_first_index(oracle, cuda):
    L = R.lib()
    rng = np.random.default_rng(3)
    for n in (10, 128256, 151936):
        x = rng.standard_normal(n).astype(np.float32)
        x[n // 3] = x[2 * n // 3] = x.max() + 1  # tie: the first wins
        xd = dev(x, cuda)
        out = torch.zeros(1, dtype=torch.int32, device=cuda)
        assert L.rie_hip_k_argmax(xd.data_ptr(), n, out.data_ptr()) == 0
        assert int(host(out)[0]) == oracle.argmax(x) == n // 3


def test_moe_routing_matches_oracle_with_nonfinite_logits(oracle, cuda):
    """The routing wave (softmax, top-k with the index tie-break, weights) against
    the oracle's routing (model/cpu.rs:492-500), including rows whose softmax is NaN
    (a NaN or +Inf logit, or every logit -Inf): the reference's comparator calls
    NaN pairs Equal and takes experts 0..k-1.  Every selection must name a real
    expert, since the expert GEMVs address their weights with it."""
    L = R.lib()
    rng = np.random.default_rng(5)
    for n_exp, k in ((8, 2), (60, 4), (64, 6), (128, 8), (256, 8), (512, 16)):
        n_tok = 48
        logits = (rng.integers(-6, 7, size=(n_tok, n_exp)) * 0.5).astype(np.float32)  # exact ties
        logits[1::4] = rng.standard_normal((len(logits[1::4]), n_exp)).astype(np.float32)
        logits[2, 5 % n_exp] = np.nan
        logits[3, n_exp - 1] = np.inf
        logits[5, :] = -np.inf
        logits[6, : n_exp // 2] = -np.inf
        logits[7, 0] = -np.inf
        logits[9, :] = np.nan
        for norm_topk, unit in ((1, 0), (0, 0), (1, 1)):
            want_s, want_w = oracle.moe_route(logits, k, bool(norm_topk), bool(unit))
            ld = dev(logits, cuda)
            sel = torch.full((n_tok * k,), -7, dtype=torch.int32, device=cuda)
            wgt = torch.zeros(n_tok * k, dtype=torch.float32, device=cuda)
            assert L.rie_hip_k_moe_route(ld.data_ptr(), n_tok, n_exp, k, norm_topk, unit, sel.data_ptr(), wgt.data_ptr()) == 0
            got_s = host(sel).reshape(n_tok, k)
            got_w = host(wgt).reshape(n_tok, k)
            assert ((got_s >= 0) & (got_s < n_exp)).all()
            assert np.array_equal(got_s, want_s), (n_exp, k, np.argwhere(got_s != want_s)[:4])
            assert np.array_equal(np.isnan(got_w), np.isnan(want_w))
            fin = ~np.isnan(want_w)
            np.testing.assert_allclose(got_w[fin], want_w[fin], rtol=4e-6, atol=1e-8)
            for t in (2, 3, 5, 9):  # NaN softmax: the first k experts
                assert got_s[t].tolist() == list(range(k))


# ---- whole model ------------------------------------------------------------------------------
CASES = [
    ("llama", Q4_0, 0, 0.03), ("llama", Q8_0, 0, 0.03), ("llama", Q4_K, 0, 0.03), ("llama", Q6_K, 0, 0.03),
    ("llama", F16, 0, 3e-3), ("llama", F32, 0, 3e-3), ("qwen3", Q4_0, 0, 0.03), ("qwen2", Q4_0, 0, 0.03),
    ("gemma3", Q4_0, 0, 0.03), ("granite", F16, 0, 3e-3), ("phi3", Q4_0, 0, 0.03), ("gemma2", F16, 0, 3e-3),
    ("llama", Q4_0, 1, 0.05), ("llama", Q4_0, 2, 0.05), ("qwen3", Q4_K, 2, 0.05),
    ("llama", Q4_1, 0, 0.03), ("llama", Q5_0, 0, 0.03), ("llama", Q5_1, 0, 0.03), ("llama", Q2_K, 0, 0.03),
    ("llama", Q3_K, 0, 0.03), ("llama", Q5_K, 0, 0.03), ("llama", BF16, 0, 3e-3),
]


def _pair(oracle, arch, ty, kv, n_ctx=64, max_batch=4, mutate=None):
    spec = synth.tiny(arch, ty)
    if mutate:
        mutate(spec)
    gguf = synth.build(spec)
    g = R.HipBackend(gguf, n_ctx=n_ctx, max_batch=max_batch, kv_type=kv)
    o = oracle.Backend(oracle.Model(gguf), n_ctx, max_batch, kv, n_threads=4)
    return spec, g, o


@pytest.mark.parametrize("arch,ty,kv,tol", CASES)
def test_model_logits_match_oracle(oracle, cuda, arch, ty, kv, tol):
    from naive_model import max_rel_err
    mut = (lambda s: setattr(s, "rope_dim", 32)) if arch == "phi3" else None
    spec, g, o = _pair(oracle, arch, ty, kv, mutate=mut)
    nv = spec.n_vocab
    toks = [(i * 37 + 5) % nv for i in range(13)]
    pos = 0
    while pos < len(toks):  # batched prefill, all logits (tests/model.rs:314-329)
        end = min(pos + 4, len(toks))
        lg = g.forward(toks[pos:end], pos, True)
        lo = o.forward(toks[pos:end], pos, True)
        for t in range(end - pos):
            err = max_rel_err(lg[t * nv:(t + 1) * nv], lo[t * nv:(t + 1) * nv])
            assert err < tol, f"{arch} {ty} kv{kv}: batched token {pos + t}: {err}"
        pos = end
    spec, g, o = _pair(oracle, arch, ty, kv, max_batch=1, mutate=mut)
    for t, tok in enumerate(toks):  # token-by-token decode (graph replay)
        err = max_rel_err(g.forward([tok], t), o.forward([tok], t))
        assert err < tol, f"{arch} {ty} kv{kv}: decode token {t}: {err}"


@pytest.mark.parametrize("arch,ty", [("llama", Q4_0), ("llama", Q8_0), ("qwen3", Q4_0), ("gemma2", Q8_0), ("llama", Q4_K),
                                     ("qwen3", Q4_K), ("llama", Q6_K), ("qwen3", Q6_K)])
def test_prompt_batches_through_gemm_match_oracle(oracle, cuda, arch, ty):
    """Prompt batches of 24 and 40 tokens run the int8-MFMA GEMM (fused Q/K/V,
    wo, gate/up with SwiGLU/GELU, down) and must match the oracle like decode."""
    from naive_model import max_rel_err
    spec, g, o = _pair(oracle, arch, ty, 0, n_ctx=96, max_batch=40)
    nv = spec.n_vocab
    toks = [(i * 29 + 3) % nv for i in range(64)]
    for pos, end in ((0, 24), (24, 64)):
        lg = g.forward(toks[pos:end], pos, True)
        lo = o.forward(toks[pos:end], pos, True)
        for t in range(end - pos):
            err = max_rel_err(lg[t * nv:(t + 1) * nv], lo[t * nv:(t + 1) * nv])
            assert err < 0.03, f"{arch} {ty}: token {pos + t}: {err}"


MOE_CASES = [  # (arch, weight type, tolerance, mutate): routed experts, shared expert + sigmoid gate, Q8_0 and Q8_K experts
    ("qwen3moe", F16, 3e-3, None), ("qwen2moe", F16, 3e-3, None), ("qwen3moe", Q4_K, 0.03, None),
    ("qwen3moe", Q4_0, 0.03, None), ("llama", Q8_0, 0.03, "mixtral"),
    # a shared expert wider than the hidden size and the routed experts (scratch sized over it)
    ("qwen2moe", F16, 3e-3, "wide_shared"), ("qwen2moe", Q4_K, 0.03, "wide_shared"),
    # expert_used_count 0: the layers route to one expert (model/mod.rs:176)
    ("qwen3moe", Q4_K, 0.03, "zero_used"),
    # 128 experts, top-8, expert FFN 768 at hidden 1024 (the Qwen3-30B-A3B routing and widths)
    ("qwen3moe", Q4_K, 0.03, "a3b"),
]
MOE_MUTATIONS = {
    None: None,
    "mixtral": lambda s: [setattr(s, k, v) for k, v in (("n_expert", 4), ("n_expert_used", 2), ("n_ff_exp", 512))],
    "wide_shared": lambda s: setattr(s, "n_ff_shexp", 1024),
    "zero_used": lambda s: setattr(s, "n_expert_used", 0),
    "a3b": lambda s: [setattr(s, k, v) for k, v in (("n_expert", 128), ("n_expert_used", 8), ("n_ff_exp", 768),
                                                     ("n_embd", 1024))],
}


@pytest.mark.parametrize("arch,ty,tol,mut", MOE_CASES)
def test_mixture_of_experts_matches_oracle(oracle, cuda, arch, ty, tol, mut):
    """moe_ffn (cpu.rs:469-524): prompt batches (experts over gathered tokens)
    and single-token decode (routing and expert choice on the device, graph
    replay) against the oracle."""
    from naive_model import max_rel_err

    spec, g, o = _pair(oracle, arch, ty, 0, n_ctx=64, max_batch=16, mutate=MOE_MUTATIONS[mut])
    nv = spec.n_vocab
    toks = [(i * 41 + 7) % nv for i in range(20)]
    lg = g.forward(toks[:16], 0, True)
    lo = o.forward(toks[:16], 0, True)
    for t in range(16):
        err = max_rel_err(lg[t * nv:(t + 1) * nv], lo[t * nv:(t + 1) * nv])
        assert err < tol, f"{arch} {ty}: batched token {t}: {err}"
    for t in range(16, 20):
        err = max_rel_err(g.forward([toks[t]], t), o.forward([toks[t]], t))
        assert err < tol, f"{arch} {ty}: decode token {t}: {err}"


@pytest.mark.parametrize("n_prompt", [70, 33])
def test_moe_prompt_with_several_tiles_per_expert(oracle, cuda, n_prompt):
    """A prompt whose experts each receive more than one 32-token tile of routed
    tokens, the last one ragged (4 Q4_K experts, top-2: about n_prompt / 2 tokens
    per expert), in one batch: every logits row against the oracle (cpu.rs:469-524)."""
    from naive_model import max_rel_err

    spec, g, o = _pair(oracle, "qwen3moe", Q4_K, 0, n_ctx=128, max_batch=80, mutate=MOE_MUTATIONS["mixtral"])
    nv = spec.n_vocab
    toks = [(i * 53 + 11) % nv for i in range(n_prompt)]
    lg = g.forward(toks, 0, True)
    lo = o.forward(toks, 0, True)
    for t in range(n_prompt):
        err = max_rel_err(lg[t * nv:(t + 1) * nv], lo[t * nv:(t + 1) * nv])
        assert err < 0.03, f"prompt of {n_prompt}: token {t}: {err}"


PROLOGUE_WIDTHS = {  # hidden sizes past one superblock / one 4096-value pass, and the 768-wide expert FFN
    None: None,
    "e2048_ff768": lambda s: [setattr(s, k, v) for k, v in (("n_embd", 2048), ("n_ff_exp", 768), ("n_ff", 1536))],
    "e4096": lambda s: [setattr(s, k, v) for k, v in (("n_embd", 4096), ("n_ff", 1024), ("n_ff_exp", 768))],
    # the benchmark workloads' attention shapes: head dim 128, 4 / 8 / 2 query heads per KV head
    "heads_32_8": lambda s: [setattr(s, k, v) for k, v in (("n_embd", 4096), ("n_ff", 1024), ("n_head", 32),
                                                           ("n_head_kv", 8), ("head_dim", 128), ("rope_dim", 128))],
    "heads_32_4": lambda s: [setattr(s, k, v) for k, v in (("n_embd", 4096), ("n_ff", 1024), ("n_head", 32),
                                                           ("n_head_kv", 4), ("head_dim", 128), ("rope_dim", 128))],
    "heads_16_8": lambda s: [setattr(s, k, v) for k, v in (("n_embd", 2048), ("n_ff", 1024), ("n_head", 16),
                                                           ("n_head_kv", 8), ("head_dim", 128), ("rope_dim", 128))],
}


@pytest.mark.parametrize("arch,ty,width", [("qwen3moe", Q4_K, None), ("qwen3moe", Q4_0, None), ("llama", Q4_0, None),
                                           ("llama", Q4_K, None), ("qwen3moe", Q4_K, "e2048_ff768"),
                                           ("qwen3moe", Q4_0, "e2048_ff768"), ("llama", Q4_0, "e4096"),
                                           ("llama", Q4_K, "e4096"), ("llama", Q4_K, "e2048_ff768"),
                                           ("llama", Q4_0, "heads_32_8"), ("llama", Q4_0, "heads_32_4"),
                                           ("llama", Q4_0, "heads_16_8")])
def test_decode_prologues_equal_standalone_norm(oracle, cuda, arch, ty, width):
    """One-token decode normalizes x inside the GEMVs that read it: Q/K/V and
    gate/up (activation codes), and for MoE layers the router (f32 rows) and the
    experts' gate/up and down (the hidden's Q8_K); capture mode runs the
    standalone RMSNorm and quantizer launches instead.  Decoding the same tokens
    at the same positions both ways gives bitwise equal logits, at hidden sizes
    from one superblock to 4096 (several superblocks and 4096-value passes per
    workgroup), at the 768-wide expert FFN and at the benchmark workloads'
    attention shapes (head dim 128)."""
    spec, g, _ = _pair(oracle, arch, ty, 0, n_ctx=64, max_batch=16, mutate=PROLOGUE_WIDTHS[width])
    toks = [(i * 41 + 7) % spec.n_vocab for i in range(20)]
    g.forward(toks[:16], 0)
    fused = [np.array(g.forward([toks[t]], t)) for t in range(16, 20)]
    g.set_capture(True)
    for i, t in enumerate(range(16, 20)):
        plain = np.array(g.forward([toks[t]], t))
        assert np.array_equal(fused[i].view(np.uint32), plain.view(np.uint32)), \
            f"{arch} {ty}: token {t}: max diff {np.max(np.abs(fused[i] - plain))}"


ATTN_SHAPES = [  # (head_dim, n_head, n_head_kv): lanes per cache row 4/8/16/32, query groups 1..8
    (32, 4, 4), (128, 8, 2), (256, 8, 1), (64, 8, 1), (128, 6, 2), (64, 14, 2), (128, 12, 2),
]


@pytest.mark.parametrize("kv", [0, 2])
@pytest.mark.parametrize("n,forced", [(200, True), (1100, False)])
def test_decode_attention_range_counts(oracle, cuda, n, forced, kv):
    """The single-token range merge is compiled per range count: 4 ranges (200
    cached positions, split on request) and 32 (1100 positions), besides the 8, 16
    and 64 the other tests reach; 4 query heads of 128 per KV head.  Decode logits
    against the oracle after a prefill in 64-token batches."""
    from naive_model import max_rel_err

    def mut(s):
        s.head_dim, s.n_head, s.n_head_kv, s.rope_dim = 128, 8, 2, 128
    spec, g, o = _pair(oracle, "llama", Q8_0, kv, n_ctx=n + 8, max_batch=64, mutate=mut)
    nv = spec.n_vocab
    toks = [(i * 53 + 11) % nv for i in range(n)]
    pos = 0
    while pos < n - 3:
        end = min(pos + 64, n - 3)
        g.forward(toks[pos:end], pos)
        o.forward(toks[pos:end], pos)
        pos = end
    g.set_attention_ranges(forced)
    tol = 0.03 if kv == 0 else 0.06
    for t in range(n - 3, n):
        err = max_rel_err(g.forward([toks[t]], t), o.forward([toks[t]], t))
        assert err < tol, f"kv{kv}: {n} positions: decode token {t}: {err}"


@pytest.mark.parametrize("kv", [0, 1, 2])
@pytest.mark.parametrize("hd,nh,nkv", ATTN_SHAPES)
def test_attention_shapes_match_oracle(oracle, cuda, hd, nh, nkv, kv):
    """Attention over 300 cached positions (several tiles and context ranges)
    for head sizes 32..256 and 1..8 query heads per KV head, every cache type.
    The decode tokens run twice: with the automatic choice (one workgroup per
    query head at this length where the one-launch path applies) and with the
    context split into ranges merged across workgroups."""
    from naive_model import max_rel_err

    def mut(s):
        s.head_dim, s.n_head, s.n_head_kv, s.rope_dim = hd, nh, nkv, hd
    n_ctx = 320
    spec, g, o = _pair(oracle, "llama", Q8_0, kv, n_ctx=n_ctx, max_batch=64, mutate=mut)
    nv = spec.n_vocab
    toks = [(i * 53 + 11) % nv for i in range(300)]
    tol = 0.03 if kv == 0 else 0.06
    pos = 0
    while pos < 296:  # prefill in batches of 64 (several ranges per query)
        end = min(pos + 64, 296)
        lg = g.forward(toks[pos:end], pos, True)
        lo = o.forward(toks[pos:end], pos, True)
        for t in (0, end - pos - 1):
            err = max_rel_err(lg[t * nv:(t + 1) * nv], lo[t * nv:(t + 1) * nv])
            assert err < tol, f"hd {hd} G {nh // nkv} kv{kv}: batched token {pos + t}: {err}"
        pos = end
    want = {}
    for t in range(296, 300):  # single-token decode at 296..299 positions of context
        want[t] = o.forward([toks[t]], t)
        err = max_rel_err(g.forward([toks[t]], t), want[t])
        assert err < tol, f"hd {hd} G {nh // nkv} kv{kv}: decode token {t}: {err}"
    g.set_attention_ranges(True)  # the same positions again, rewriting their cache rows
    for t in range(296, 300):
        err = max_rel_err(g.forward([toks[t]], t), want[t])
        assert err < tol, f"hd {hd} G {nh // nkv} kv{kv}: decode token {t} over ranges: {err}"


PROMPT_ATTN_SHAPES = ATTN_SHAPES + [(64, 4, 2), (96, 6, 6)]


@pytest.mark.parametrize("hd,nh,nkv", PROMPT_ATTN_SHAPES)
def test_prompt_attention_matches_f64_on_captured_rows(oracle, cuda, hd, nh, nkv):
    """The attention output of prompt batches (f16 cache) against a float64
    evaluation of cpu.rs:550-634 on the same operands: the prepared queries the
    GPU used and the f16 cache rows it holds.  Batches start at positions 0, 64
    and 128 and end inside a 32-position tile, so the causal mask, the tile
    edges and every query-head grouping are pinned to f32 rounding: an f32
    score of magnitude |s| carries an error of a few 2^-24·|s|, which moves each
    softmax weight by that relative amount (a dropped or extra position moves
    the output by about max|V| / positions, orders of magnitude more)."""
    def mut(s):
        s.head_dim, s.n_head, s.n_head_kv, s.rope_dim = hd, nh, nkv, hd
    n_ctx = 160
    spec, g, _ = _pair(oracle, "llama", Q8_0, 0, n_ctx=n_ctx, max_batch=64, mutate=mut)
    g.set_capture(True)
    G, qd = nh // nkv, nh * hd
    toks = [(i * 53 + 11) % spec.n_vocab for i in range(150)]
    for pos0, end in ((0, 64), (64, 128), (128, 150)):
        n = end - pos0
        g.forward(toks[pos0:end], pos0)
        for layer in range(spec.n_layer):
            q = g.capture(layer, 3, n * qd).reshape(n, nh, hd).astype(np.float64)
            att = g.capture(layer, 2, n * qd).reshape(n, nh, hd)
            kr, _ = g.kv_layer(layer, 0, nkv, n_ctx)
            vr, _ = g.kv_layer(layer, 1, nkv, n_ctx)
            K = kr.view(np.float16).reshape(nkv, n_ctx, hd).astype(np.float64)
            V = vr.view(np.float16).reshape(nkv, n_ctx, hd).astype(np.float64)
            for t in range(n):
                p = pos0 + t
                for hq in range(nh):
                    kv = hq // G
                    s = K[kv, :p + 1] @ q[t, hq]
                    w = np.exp(s - s.max())
                    ref = (w / w.sum()) @ V[kv, :p + 1]
                    err = np.max(np.abs(att[t, hq] - ref))
                    vmax = np.max(np.abs(V[kv, :p + 1]))
                    assert err <= (8 * 2.0 ** -24 * np.max(np.abs(s)) + 5e-6) * vmax + 1e-6, \
                        f"hd {hd} G {G} layer {layer} token {p} head {hq}: {err}"


def _turbo_attention_f64(oracle, q, krows, kscales, vrows, vscales, hd):
    """cpu.rs:584-632 over a Turbo4 cache in float64: the query rotated and
    quantized to Q8_0 (the oracle's), integer level dots per 32-value chunk
    (dot_rotated_4, turbo.rs:178-193), softmax, the weighted levels
    (axpy_rotated_4) and the inverse rotation (turbo.rs:113-117)."""
    lv = np.array([-126, -95, -74, -58, -43, -30, -18, -6, 6, 18, 30, 43, 58, 74, 95, 126], np.float64)
    n = krows.shape[0]

    def codes(rows):
        c = np.empty((n, hd), np.int64)
        for ch in range(hd // 32):
            c[:, 32 * ch:32 * ch + 16] = rows[:, 16 * ch:16 * ch + 16] & 0xF
            c[:, 32 * ch + 16:32 * ch + 32] = rows[:, 16 * ch:16 * ch + 16] >> 4
        return c
    qa = oracle.quantize_q8_0(oracle.turbo_rotate(q.astype(np.float32)))
    qs, dq = qa["qs"].reshape(-1).astype(np.float64), qa["d"].astype(np.float64)
    ks = kscales.view(np.float16).astype(np.float64)
    vs = vscales.view(np.float16).astype(np.float64)
    s = ((lv[codes(krows)] * qs).reshape(n, hd // 32, 32).sum(axis=2) * dq).sum(axis=1) * ks / 46.0
    w = np.exp(s - s.max())
    vv = vs[:, None] * lv[codes(vrows)] / 46.0
    orot = ((w / w.sum())[:, None] * vv).sum(axis=0)
    return oracle.turbo_rotate(orot.astype(np.float32), inverse=True).astype(np.float64), s, vv


@pytest.mark.parametrize("nh,nkv", [(8, 2), (6, 2), (12, 2), (8, 8), (16, 2)])
def test_turbo_prompt_attention_matches_f64_on_captured_rows(oracle, cuda, nh, nkv):
    """Prompt attention over a Turbo4 cache (head dim 128: rotated, Q8_0-quantized
    queries against the level tiles on f16 matrix cores, inverse rotation in the
    epilogue) against float64 on the GPU's own captured queries and cache rows,
    for prompt batches starting at positions 0, 64 and 128 (causal tile edges,
    1 to 8 query heads per KV head)."""
    hd = 128

    def mut(s):
        s.head_dim, s.n_head, s.n_head_kv, s.rope_dim = hd, nh, nkv, hd
    n_ctx = 160
    spec, g, _ = _pair(oracle, "llama", Q8_0, 2, n_ctx=n_ctx, max_batch=64, mutate=mut)
    g.set_capture(True)
    G, qd = nh // nkv, nh * hd
    toks = [(i * 53 + 11) % spec.n_vocab for i in range(150)]
    for pos0, end in ((0, 64), (64, 128), (128, 150)):
        n = end - pos0
        g.forward(toks[pos0:end], pos0)
        for layer in range(spec.n_layer):
            q = g.capture(layer, 3, n * qd).reshape(n, nh, hd)
            att = g.capture(layer, 2, n * qd).reshape(n, nh, hd)
            kr, ksc = g.kv_layer(layer, 0, nkv, n_ctx)
            vr, vsc = g.kv_layer(layer, 1, nkv, n_ctx)
            # largest decoded V value up to each position, in the rotated and the original
            # domain: a relative error δ_j of probability j moves the output by δ_j·p_j·R⁻¹vv_j
            vrun = []
            for kv in range(nkv):
                _, _, vv = _turbo_attention_f64(oracle, q[0, 0], kr[kv, :end], ksc[kv, :end], vr[kv, :end], vsc[kv, :end], hd)
                m = [max(np.abs(r).max(), np.abs(oracle.turbo_rotate(r.astype(np.float32), inverse=True)).max()) for r in vv]
                vrun.append(np.maximum.accumulate(m))
            for t in range(n):
                p = pos0 + t
                for hq in range(nh):
                    kv = hq // G
                    ref, sc, _ = _turbo_attention_f64(oracle, q[t, hq], kr[kv, :p + 1], ksc[kv, :p + 1], vr[kv, :p + 1],
                                                      vsc[kv, :p + 1], hd)
                    vmax = vrun[kv][p]
                    err = np.max(np.abs(att[t, hq] - ref))
                    assert err <= (8 * 2.0 ** -24 * np.max(np.abs(sc)) + 5e-6) * vmax + 2e-6 * vmax + 1e-6, \
                        f"G {G} layer {layer} token {p} head {hq}: {err}"


@pytest.mark.parametrize("kv", [0, 2])
def test_prompt_attention_kv_splits_match_f64(oracle, cuda, kv):
    """Prompt batches far into the context split each query block's positions over
    several workgroups (2 at positions 1024.., 8 at 4032..), whose partials the range
    merge combines (and, for Turbo4, rotates back); a batch at 256.. stays in one
    pass.  Outputs against float64 on the captured queries and cache rows, to the
    bounds of the single-pass tests."""
    hd, nh, nkv = 128, 8, 2

    def mut(s):
        s.head_dim, s.n_head, s.n_head_kv, s.rope_dim = hd, nh, nkv, hd
    n_ctx = 4096
    spec, g, _ = _pair(oracle, "llama", Q8_0, kv, n_ctx=n_ctx, max_batch=64, mutate=mut)
    G, qd = nh // nkv, nh * hd
    toks = [(i * 53 + 11) % spec.n_vocab for i in range(n_ctx)]
    checked = 0
    for pos0 in range(0, n_ctx, 64):
        n = 64
        check = pos0 in (256, 1024, 4032)
        g.set_capture(check)
        g.forward(toks[pos0:pos0 + n], pos0)
        if not check:
            continue
        for layer in range(spec.n_layer):
            q = g.capture(layer, 3, n * qd).reshape(n, nh, hd)
            att = g.capture(layer, 2, n * qd).reshape(n, nh, hd)
            kr, ksc = g.kv_layer(layer, 0, nkv, n_ctx)
            vr, vsc = g.kv_layer(layer, 1, nkv, n_ctx)
            if kv == 0:
                K = kr.view(np.float16).reshape(nkv, n_ctx, hd).astype(np.float64)
                V = vr.view(np.float16).reshape(nkv, n_ctx, hd).astype(np.float64)
            else:
                # largest decoded V value up to each position in either domain; the
                # rotation is orthogonal, so a row's 2-norm bounds its unrotated values
                vrun = []
                for h in range(nkv):
                    _, _, vv = _turbo_attention_f64(oracle, q[0, 0], kr[h, :pos0 + n], ksc[h, :pos0 + n], vr[h, :pos0 + n],
                                                    vsc[h, :pos0 + n], hd)
                    m = np.maximum(np.abs(vv).max(axis=1), np.sqrt((vv * vv).sum(axis=1)))
                    vrun.append(np.maximum.accumulate(m))
            for t in range(0, n, 3 if kv == 0 else 7):
                p = pos0 + t
                for hq in range(nh):
                    h = hq // G
                    if kv == 0:
                        sc = K[h, :p + 1] @ q[t, hq].astype(np.float64)
                        w = np.exp(sc - sc.max())
                        ref = (w / w.sum()) @ V[h, :p + 1]
                        vmax = np.max(np.abs(V[h, :p + 1]))
                        bound = (8 * 2.0 ** -24 * np.max(np.abs(sc)) + 5e-6) * vmax + 1e-6
                    else:
                        ref, sc, _ = _turbo_attention_f64(oracle, q[t, hq], kr[h, :p + 1], ksc[h, :p + 1], vr[h, :p + 1],
                                                          vsc[h, :p + 1], hd)
                        vmax = vrun[h][p]
                        bound = (8 * 2.0 ** -24 * np.max(np.abs(sc)) + 5e-6) * vmax + 2e-6 * vmax + 1e-6
                    err = np.max(np.abs(att[t, hq] - ref))
                    assert err <= bound, f"kv{kv} layer {layer} token {p} head {hq}: {err} > {bound}"
                    checked += 1
    assert checked > 0


@pytest.mark.parametrize("hd,nh,nkv", ATTN_SHAPES)
def test_decode_attention_matches_f64_on_captured_rows(oracle, cuda, hd, nh, nkv):
    """Single-token attention (the fused launch: prep, append and attention, one
    workgroup per query head at this length, and again with context ranges and
    the range merge; groups of 6 and 8 query heads split in two workgroups) at
    positions 296..299 against a float64 evaluation of cpu.rs:550-634 on the
    prepared queries and the f16 cache rows, to the f32 bound of the prompt
    test above."""
    def mut(s):
        s.head_dim, s.n_head, s.n_head_kv, s.rope_dim = hd, nh, nkv, hd
    n_ctx = 320
    spec, g, _ = _pair(oracle, "llama", Q8_0, 0, n_ctx=n_ctx, max_batch=64, mutate=mut)
    G, qd = nh // nkv, nh * hd
    toks = [(i * 53 + 11) % spec.n_vocab for i in range(300)]
    for pos in range(0, 296, 64):
        g.forward(toks[pos:min(pos + 64, 296)], pos)
    g.set_capture(True)
    for ranges, p in [(r, p) for r in (False, True) for p in range(296, 300)]:
        g.set_attention_ranges(ranges)
        g.forward([toks[p]], p)
        for layer in range(spec.n_layer):
            q = g.capture(layer, 3, qd).reshape(nh, hd).astype(np.float64)
            att = g.capture(layer, 2, qd).reshape(nh, hd)
            kr, _ = g.kv_layer(layer, 0, nkv, n_ctx)
            vr, _ = g.kv_layer(layer, 1, nkv, n_ctx)
            K = kr.view(np.float16).reshape(nkv, n_ctx, hd).astype(np.float64)
            V = vr.view(np.float16).reshape(nkv, n_ctx, hd).astype(np.float64)
            for hq in range(nh):
                kv = hq // G
                s = K[kv, :p + 1] @ q[hq]
                w = np.exp(s - s.max())
                ref = (w / w.sum()) @ V[kv, :p + 1]
                err = np.max(np.abs(att[hq] - ref))
                vmax = np.max(np.abs(V[kv, :p + 1]))
                assert err <= (8 * 2.0 ** -24 * np.max(np.abs(s)) + 5e-6) * vmax + 1e-6, \
                    f"hd {hd} G {G} layer {layer} token {p} head {hq} ranges {ranges}: {err}"


@pytest.mark.parametrize("kv", [0, 1, 2])
def test_kv_codes_bit_exact_on_identical_inputs(oracle, cuda, kv):
    """The cache rows the GPU writes equal the reference encoders applied to the
    GPU's own post-RoPE K and V (f16 RNE; store_q8_0 cpu.rs:637-647; quantize_4
    turbo.rs:166-171)."""
    spec, g, _ = _pair(oracle, "qwen3", Q4_0, kv, n_ctx=32, max_batch=4)
    g.set_capture(True)
    hd, nkv = spec.head_dim, spec.n_head_kv

    def check(t0, n):  # cache slots t0..t0+n-1 against the captured rows of the last forward
        for layer in range(spec.n_layer):
            kpost = g.capture(layer, 4, n * nkv * hd).reshape(n, nkv, hd)
            vpost = g.capture(layer, 5, n * nkv * hd).reshape(n, nkv, hd)
            for which, src in ((0, kpost), (1, vpost)):
                rows, scales = g.kv_layer(layer, which, nkv, 32)
                for t in range(n):
                    for h in range(nkv):
                        x = src[t, h]
                        if kv == 0:
                            want = x.astype(np.float16).view(np.uint8)
                            assert np.array_equal(rows[h, t0 + t], want)
                        elif kv == 1:
                            assert np.array_equal(rows[h, t0 + t], oracle.quantize_weights(Q8_0, x))
                        else:
                            ref = oracle.turbo_quantize(x)
                            assert np.array_equal(rows[h, t0 + t], ref[2:]) and scales[h, t0 + t] == ref[:2].view(np.uint16)[0]

    g.forward([3, 77, 150, 9], 0)   # prompt: separate prep / append launch
    check(0, 4)
    for pos, tok in ((4, 41), (5, 6)):  # single tokens: prep and append inside the attention launch
        g.forward([tok], pos)
        check(pos, 1)


@pytest.mark.parametrize("kv", [0, 1, 2])
@pytest.mark.parametrize("arch", ["llama", "qwen3"])
def test_long_decode_matches_oracle(oracle, cuda, arch, kv):
    """132 single-token steps (query/key prep, cache append and attention in one
    launch) from position 8 to 139: every context length across tile and range
    boundaries, against the oracle.  Odd positions run the context-range kernel
    with its range merge, even ones one workgroup per query head, so each reads
    cache rows the other appended."""
    from naive_model import max_rel_err
    spec, g, o = _pair(oracle, arch, Q8_0, kv, n_ctx=160, max_batch=8)
    nv = spec.n_vocab
    toks = [(i * 31 + 7) % nv for i in range(140)]
    g.forward(toks[:8], 0)
    o.forward(toks[:8], 0)
    tol = 0.03 if kv == 0 else 0.05
    for pos in range(8, 140):
        g.set_attention_ranges(pos % 2 == 1)
        err = max_rel_err(g.forward([toks[pos]], pos), o.forward([toks[pos]], pos))
        assert err < tol, f"{arch} kv{kv}: decode position {pos}: {err}"


def _top2_margin(x):
    a = np.partition(x, -2)[-2:]
    return float(a[1] - a[0])


def greedy_agreement(g, o, prompt, n_steps, nv):
    """Teacher-forced greedy comparison: both backends are fed the CPU's choice
    each step.  Returns per-step (gpu argmax, cpu argmax, cpu top-2 margin,
    max |Δlogit|)."""
    lg, lo = g.forward(prompt, 0), o.forward(prompt, 0)
    rows = []
    for step in range(n_steps):
        ag, ac = R.argmax(lg), int(oracle_argmax(lo))
        rows.append((ag, ac, _top2_margin(lo), float(np.abs(lg - lo).max())))
        pos = len(prompt) + step
        lg, lo = g.forward([ac], pos), o.forward([ac], pos)
    return rows


def oracle_argmax(x):
    import pyoracle
    return pyoracle.argmax(x)


def check_greedy(oracle, arch, ty, n_steps=128, n_prompt=16, n_ctx=256):
    spec, g, o = _pair(oracle, arch, ty, 0, n_ctx=n_ctx, max_batch=16)
    nv = spec.n_vocab
    prompt = [(i * 7919 + 13) % nv for i in range(n_prompt)]
    rows = greedy_agreement(g, o, prompt, n_steps, nv)
    bad = [(i, r) for i, r in enumerate(rows) if r[0] != r[1]]
    noise = max(r[3] for r in rows)
    print(f"{arch} {ty}: {n_steps - len(bad)}/{n_steps} teacher-forced greedy steps agree; max |dlogit| {noise:.3g}; "
          f"disagreements (step, cpu margin, |dlogit|): {[(i, round(r[2], 5), round(r[3], 5)) for i, r in bad]}")
    for i, r in bad:  # a disagreement is allowed only inside the numerical noise band
        assert r[2] <= 2 * r[3], f"step {i}: cpu margin {r[2]} exceeds 2x logit difference {r[3]}"
    # free-running device greedy follows the CPU sequence up to the first near-tie
    first = bad[0][0] if bad else n_steps
    want, _, _ = oracle.Backend(oracle.Model(synth.build(spec)), n_ctx, 16, 0, n_threads=4).greedy(prompt, n_steps)
    got = R.Engine(R.HipBackend(synth.build(spec), n_ctx=n_ctx, max_batch=16)).greedy(prompt, n_steps)
    assert np.array_equal(got[:first], want[:first])
    return len(bad)


def test_greedy_128_steps_match_oracle_outside_near_ties(oracle, cuda):
    check_greedy(oracle, "llama", Q4_0)
    check_greedy(oracle, "qwen3", Q4_K)


def test_graph_replay_equals_eager(oracle, cuda):
    spec = synth.tiny("qwen3", Q4_0)
    gguf = synth.build(spec)
    a = R.HipBackend(gguf, n_ctx=64, max_batch=4, use_graph=True)
    b = R.HipBackend(gguf, n_ctx=64, max_batch=4, use_graph=False)
    toks = [5, 9, 200, 7, 31, 64]
    for i, t in enumerate(toks):
        assert np.array_equal(a.forward([t], i), b.forward([t], i))


def test_hidden_and_error_contract(oracle, cuda):
    spec, g, o = _pair(oracle, "llama", Q4_0, 0, n_ctx=16, max_batch=4)
    assert g.hidden() is None
    g.forward([1, 2, 3], 0, True)
    o.forward([1, 2, 3], 0, True)
    h, ho = g.hidden(), o.hidden()
    assert h.shape == ho.shape == (3 * spec.n_embd,)
    assert np.abs(h - ho).max() < 1e-3 * np.abs(ho).max()
    for toks, pos, msg in (([], 0, "empty batch"), ([1] * 5, 0, "exceeds max batch"), ([1, 2], 15, "context window full"),
                           ([999], 0, "out of range")):
        with pytest.raises(R.RieError, match=msg) as ei:
            g.forward(toks, pos)
        assert ei.value.kind == "Runtime"
    with pytest.raises(R.RieError, match="logits buffer too small"):
        g.forward([1, 2], 0, logits=np.zeros(10, np.float32))


@pytest.mark.parametrize("ty,tol", [(F16, 3e-3), (Q4_0, 0.03)])
def test_rope_frequency_factors_match_oracle(oracle, cuda, ty, tol):
    """A tiny llama carrying rope_freqs.weight (Llama-3.1's per-dimension RoPE
    factors, Rope::new ops.rs:65-78): an 11-token prompt as one batch (prompt
    head prep and attention), then 24 teacher-forced single-token steps (the
    fused decode attention, graph replay), logits against the oracle at the
    reference's whole-model tolerances (tests/model.rs:340-375)."""
    from naive_model import max_rel_err
    from test_oracle_model import rope_factor_image
    spec, _, img = rope_factor_image(oracle, ty)
    g = R.HipBackend(img, n_ctx=64, max_batch=16)
    o = oracle.Backend(oracle.Model(img), 64, 16, 0, n_threads=4)
    nv = spec.n_vocab
    prompt = [(i * 37 + 5) % nv for i in range(11)]
    lg, lo = g.forward(prompt, 0), o.forward(prompt, 0)
    assert max_rel_err(lg, lo) < tol
    for step in range(24):
        tok = oracle.argmax(lo)
        pos = len(prompt) + step
        lg, lo = g.forward([tok], pos), o.forward([tok], pos)
        err = max_rel_err(lg, lo)
        assert err < tol, (step, err)
    g.close()


@pytest.mark.parametrize("ty", [Q4_0, Q4_K])
def test_hidden_after_graph_replayed_decode_steps(cuda, ty):
    """Backend::hidden (model/mod.rs:314-319; read every decode step by the
    adapter path, engine.rs:304-320, 442) after single-token forwards that replay
    a captured graph: each call must return that step's normalized row, bitwise
    the row an eager backend (no graph) forms for the same tokens."""
    spec = synth.tiny("llama", ty)
    img = synth.build(spec)
    g = R.HipBackend(img, n_ctx=64, max_batch=4)
    e = R.HipBackend(img, n_ctx=64, max_batch=4, use_graph=False)
    prompt = [3, 14, 15, 92]
    g.forward(prompt, 0)
    e.forward(prompt, 0)
    assert np.array_equal(g.hidden(), e.hidden())
    tok, rows = 7, []
    for step in range(6):  # step 0 captures the graph, the rest replay it
        lg = g.forward([tok], 4 + step)
        le = e.forward([tok], 4 + step)
        assert np.array_equal(lg, le)
        hg, he = g.hidden(), e.hidden()
        assert np.array_equal(hg, he), step
        assert np.array_equal(g.hidden(), hg)  # asking twice gives the same row
        rows.append(hg)
        tok = int(np.argmax(lg))
    assert not any(np.array_equal(rows[i], rows[i + 1]) for i in range(len(rows) - 1))
    # the on-device greedy loop (one graph per step) leaves its last step's row
    nxt = g.forward_argmax([tok], 10)
    assert nxt == e.forward_argmax([tok], 10)
    g.generate_greedy(11, 3)
    e.generate_greedy(11, 3)
    assert np.array_equal(g.hidden(), e.hidden())


def test_engine_prefix_reuse(oracle, cuda):
    """engine_generation_prefix_reuse_and_determinism (crates/rie-core/tests/
    model.rs:384-410): the second request reuses the cached prefix and greedy
    decoding gives the same tokens; a fresh engine agrees too.  The re-evaluated
    last token runs through the single-token kernels instead of the batched
    ones, so its logits agree to float rounding (1e-5 of the largest), not bitwise."""
    spec = synth.tiny("llama", Q4_0)
    img = synth.build(spec)
    toks = [1, 5, 9, 33, 2, 8]

    def run(e):
        reused = e.eval_tokens(toks)
        first = e.logits().copy()
        out = []
        for _ in range(20):
            t = R.argmax(e.logits())
            out.append(t)
            e.eval_next(t)
        return reused, first, out

    e1 = R.Engine(R.HipBackend(img, n_ctx=64, max_batch=8))
    r1, l1, out1 = run(e1)
    r2, l2, out2 = run(e1)
    assert r1 == 0 and r2 == len(toks) - 1  # everything but the last token is reused
    assert np.abs(l2 - l1).max() <= 1e-5 * np.abs(l1).max()
    assert out1 == out2
    r3, l3, out3 = run(R.Engine(R.HipBackend(img, n_ctx=64, max_batch=8)))
    assert r3 == 0 and np.array_equal(l3, l1) and out3 == out1
