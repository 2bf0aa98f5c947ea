"""Pins the oracle's whole forward pass against the independent naive model
(tests/naive_model.py, the numpy form of crates/rie-core/tests/model.rs:17-301)
with the reference's own tolerances (tests/model.rs:340-534), and checks the KV
variants and engine semantics the reference tests (tests/model.rs:426-490)."""
import numpy as np
import pytest

from naive_model import NaiveModel, max_rel_err

F32, F16, Q4_0, Q4_1, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 0, 1, 2, 3, 6, 8, 10, 11, 12, 13, 14


def check_arch(oracle, name, wtype, tol, threads=3, mutate=None):
    """tests/model.rs:303-338: batched prefill (batch 4, all logits) and decode."""
    spec = oracle.synth_spec(name, wtype)
    if mutate:
        mutate(spec)
    gguf = oracle.synth_build(spec)
    ref = NaiveModel(gguf, emulate_act_quant=True)
    model = oracle.Model(gguf)
    nv = spec.n_vocab
    tokens = [(i * 37 + 5) % nv for i in range(13)]
    expect = ref.logits(tokens)
    be = oracle.Backend(model, 64, 4, n_threads=threads)
    pos = 0
    while pos < len(tokens):
        end = min(pos + 4, len(tokens))
        logits = be.forward(tokens[pos:end], pos, all_logits=True)
        for t in range(pos, end):
            err = max_rel_err(logits[(t - pos) * nv:(t - pos + 1) * nv], expect[t])
            assert err < tol, f"{name} {wtype}: batched token {t}: rel err {err}"
        pos = end
    be = oracle.Backend(model, 64, 1, n_threads=threads)
    for t, tok in enumerate(tokens):
        l1 = be.forward([tok], t)
        err = max_rel_err(l1, expect[t])
        assert err < tol, f"{name} {wtype}: decode token {t}: rel err {err}"


def test_llama_f32_exact(oracle):
    check_arch(oracle, "tiny-llama", F32, 2e-3)


@pytest.mark.parametrize("arch", ["llama", "qwen2", "qwen3", "phi3", "gemma", "gemma2", "gemma3", "granite"])
def test_all_architectures_f16(oracle, arch):
    mut = (lambda s: setattr(s, "rope_dim", 32)) if arch == "phi3" else None
    check_arch(oracle, f"tiny-{arch}", F16, 3e-3, threads=4, mutate=mut)


@pytest.mark.parametrize("ty", [Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q5_0, Q4_1, Q3_K, Q2_K])
def test_quantized_weights(oracle, ty):
    check_arch(oracle, "tiny-llama", ty, 0.03, threads=2)


def test_quantized_qwen3_and_gemma3(oracle):
    check_arch(oracle, "tiny-qwen3", Q4_K, 0.03, threads=4)
    check_arch(oracle, "tiny-gemma3", Q4_0, 0.03, threads=3)


def test_tied_embeddings_single_thread(oracle):
    check_arch(oracle, "tiny-qwen2", F16, 3e-3, threads=1, mutate=lambda s: setattr(s, "tied_output", 1))


def test_mixture_of_experts(oracle):
    check_arch(oracle, "tiny-qwen3moe", F16, 3e-3)
    check_arch(oracle, "tiny-qwen2moe", F16, 3e-3, threads=2)

    def mixtral(s):
        s.n_expert, s.n_expert_used, s.n_ff_exp = 4, 2, 512
    check_arch(oracle, "tiny-llama", F16, 3e-3, threads=4, mutate=mixtral)
    check_arch(oracle, "tiny-qwen3moe", Q4_K, 0.03, threads=4)


@pytest.mark.parametrize("arch,ty", [("llama", F16), ("qwen3", F16), ("gemma3", F16), ("phi3", Q4_0), ("llama", Q4_K)])
def test_q8_0_kv_cache_matches_f16(oracle, arch, ty):
    """tests/model.rs:426-454"""
    model = oracle.Model(oracle.synth_build(oracle.synth_spec(f"tiny-{arch}", ty)))
    a = oracle.Backend(model, 64, 4, oracle.KV_F16, 3)
    b = oracle.Backend(model, 64, 4, oracle.KV_Q8_0, 3)
    assert b.kv_type == oracle.KV_Q8_0
    assert b.kv_bytes() * 100 < a.kv_bytes() * 54
    nv = model.cfg["n_vocab"]
    toks = [(i * 29 + 3) % nv for i in range(14)]
    worst = 0.0
    for pos in range(0, 14, 4):
        la = a.forward(toks[pos:pos + 4], pos)
        lb = b.forward(toks[pos:pos + 4], pos)
        worst = max(worst, max_rel_err(lb, la))
    assert worst < 0.05


@pytest.mark.parametrize("arch,ty", [("llama", F16), ("qwen3", F16), ("gemma3", F16), ("phi3", Q4_0)])
def test_turbo4_kv_cache_tracks_f16(oracle, arch, ty):
    """tests/model.rs:456-490"""
    model = oracle.Model(oracle.synth_build(oracle.synth_spec(f"tiny-{arch}", ty)))
    a = oracle.Backend(model, 64, 4, oracle.KV_F16, 3)
    b = oracle.Backend(model, 64, 4, oracle.KV_TURBO4, 3)
    assert b.kv_type == oracle.KV_TURBO4
    assert b.kv_bytes() * 100 < a.kv_bytes() * 36
    nv = model.cfg["n_vocab"]
    toks = [(i * 29 + 3) % nv for i in range(20)]
    worst = 0.0
    for pos in range(0, 20, 4):
        la = a.forward(toks[pos:pos + 4], pos)
        lb = b.forward(toks[pos:pos + 4], pos)
        worst = max(worst, max_rel_err(lb, la))
    assert worst < 0.4


def test_turbo_attention_equals_attention_over_reconstruction(oracle):
    """cpu.rs:667-718 at model level: a Turbo4 cache and an f16 cache holding the
    reconstructed K/V give the same attention (same Q8_0 query quantization)."""
    model = oracle.Model(oracle.synth_build(oracle.synth_spec("tiny-llama", F16)))
    t = oracle.Backend(model, 64, 4, oracle.KV_TURBO4, 2)
    t.set_capture(True)
    toks = [(i * 29 + 3) % 384 for i in range(8)]
    t.forward(toks[:4], 0)
    t.forward(toks[4:], 4)
    hd, nkv, nh = 64, 2, 4
    rb = oracle.turbo_row_bytes(hd)
    kc, vc = t.kv_layer(0, 0).reshape(nkv, 64, rb), t.kv_layer(0, 1).reshape(nkv, 64, rb)
    q = t.capture(0, 3).reshape(4, nh, hd)
    att = t.capture(0, 2).reshape(4, nh, hd)
    L = oracle.lib()

    def rot_rows(rows):  # R·reconstruction = the rotated-domain row values
        out = []
        for r in rows:
            y = np.zeros(hd, np.float32)
            L.or_turbo_axpy(oracle.ptr(y), hd, 1.0, oracle.ptr(np.ascontiguousarray(r)))
            out.append(y)
        return np.stack(out).astype(np.float64)

    for tt in range(4):
        p = 4 + tt
        for h in range(nh):
            g = h // 2
            K = np.stack([oracle.turbo_dequantize(kc[g, j], hd) for j in range(p + 1)])
            V = np.stack([oracle.turbo_dequantize(vc[g, j], hd) for j in range(p + 1)])
            # exact rotated-domain math: scores use the Q8_0-quantized rotated query
            qq = oracle.quantize_q8_0(oracle.turbo_rotate(q[tt, h]))
            qdeq = (qq["qs"].astype(np.float64) * qq["d"][:, None]).reshape(-1)
            s = rot_rows(kc[g, :p + 1]) @ qdeq
            pr = np.exp(s - s.max())
            pr /= pr.sum()
            o = oracle.turbo_rotate((pr @ rot_rows(vc[g, :p + 1])).astype(np.float32), inverse=True)
            assert np.abs(o - att[tt, h]).max() < 1e-4
            # and ≈ ordinary attention over the reconstructed cache (int8 query noise only)
            s2 = K.astype(np.float64) @ q[tt, h]
            pr2 = np.exp(s2 - s2.max())
            pr2 /= pr2.sum()
            assert np.abs(pr2 @ V - att[tt, h]).max() < 2e-2


def test_greedy_is_deterministic_and_batch_independent(oracle):
    model = oracle.Model(oracle.synth_build(oracle.synth_spec("tiny-llama", Q4_0)))
    prompt = [(i * 7919 + 13) % 384 for i in range(20)]
    a, ma, _ = oracle.Backend(model, 128, 8, n_threads=2).greedy(prompt, 24)
    b, mb, _ = oracle.Backend(model, 128, 8, n_threads=5).greedy(prompt, 24)
    assert np.array_equal(a, b) and np.array_equal(ma, mb)


def test_forward_error_contract(oracle):
    """cpu.rs:215-231, 395-397: empty batch, batch > max, full context, bad token id, short logits."""
    model = oracle.Model(oracle.synth_build(oracle.synth_spec("tiny-llama", Q4_0)))
    be = oracle.Backend(model, 16, 4)
    for toks, pos, msg in (([], 0, "empty batch"), ([1] * 5, 0, "exceeds max batch"), ([1, 2], 15, "context window full"),
                           ([999], 0, "out of range")):
        with pytest.raises(oracle.OracleError, match=msg):
            be.forward(toks, pos)
    with pytest.raises(oracle.OracleError, match="logits buffer too small"):
        be.forward([1, 2], 0, logits=np.zeros(10, np.float32))


def rope_factor_image(oracle, wtype):
    """A tiny llama image carrying rope_freqs.weight (Llama-3.1's per-dimension
    RoPE factors): every other dimension pair slowed by 1.5-8x, one zero factor
    (left out by Rope::new, ops.rs:69-73)."""
    from gguf_edit import add_f32_tensor
    spec = oracle.synth_spec("tiny-llama", wtype)
    base = oracle.synth_build(spec)
    half = spec.rope_dim // 2
    fac = np.ones(half, np.float32)
    fac[::2] = np.array([1.5, 2.0, 3.0, 4.0, 8.0], np.float32)[np.arange(len(fac[::2])) % 5]
    fac[1] = 0.0
    return spec, base, add_f32_tensor(base, "rope_freqs.weight", fac)


def test_rope_frequency_factors(oracle):
    """rope_freqs.weight (Model::load, model/mod.rs:130-133; Rope::new,
    ops.rs:65-78): the oracle on an image carrying the factors agrees with the
    naive model that applies them, within the F32 whole-model tolerance, and the
    factors move the logits well past it (so the path is exercised)."""
    spec, base, img = rope_factor_image(oracle, F32)
    nv = spec.n_vocab
    tokens = [(i * 37 + 5) % nv for i in range(13)]
    expect = NaiveModel(img, emulate_act_quant=True).logits(tokens)
    be = oracle.Backend(oracle.Model(img), 64, 4, n_threads=3)
    plain = oracle.Backend(oracle.Model(base), 64, 4, n_threads=3)
    moved = 0.0
    for pos in range(0, len(tokens), 4):
        chunk = tokens[pos:pos + 4]
        lg = be.forward(chunk, pos, all_logits=True)
        lp = plain.forward(chunk, pos, all_logits=True)
        for t in range(len(chunk)):
            err = max_rel_err(lg[t * nv:(t + 1) * nv], expect[pos + t])
            assert err < 2e-3, f"token {pos + t}: rel err {err}"
            moved = max(moved, max_rel_err(lp[t * nv:(t + 1) * nv], lg[t * nv:(t + 1) * nv]))
    assert moved > 0.05, f"the factors moved the logits by only {moved}"
