"""Independent naive transformer: numpy restatement of the reference's whole-model
test oracle (crates/rie-core/tests/model.rs:17-301).  Everything is recomputed
for the whole sequence from dequantized weights, with float64 matrix-vector
products; like the reference test it optionally emulates the engine's 8-bit
activation quantization and the f16 KV cache so that the remaining differences
are summation order and rare rounding-tie flips.

It shares no code with the C oracle: GGUF parsing and dequantization come from
tests/ggml_np.py and tests/gguf_np.py.
"""
from __future__ import annotations

import numpy as np

import ggml_np as G
from gguf_np import GGUF


def _rms(x, w, eps):
    ss = np.float32(np.dot(x.astype(np.float64), x.astype(np.float64)) / x.size)
    s = np.float32(1.0) / np.sqrt(ss + np.float32(eps), dtype=np.float32)
    return (x * s * w).astype(np.float32)


class NaiveModel:
    def __init__(self, gguf: bytes, emulate_act_quant: bool = True):
        self.g = GGUF(gguf)
        self.arch = self.g.get("general.architecture")
        self.emulate = emulate_act_quant
        self._cache = {}

    def t(self, name):
        if name in self._cache:
            return self._cache[name]
        ti = self.g.tensors.get(name)
        if ti is None:
            return None
        ty, dims, raw = ti
        n = int(np.prod(dims))
        w = G.dequantize(ty, raw, n)
        cols = dims[0]
        val = (w.reshape(-1, cols) if len(dims) > 1 else w, ty)
        self._cache[name] = val
        return val

    def u(self, k):
        return int(self.g.get(f"{self.arch}.{k}"))

    def logits(self, tokens):
        a = self.arch
        e, nl, nh, nkv = self.u("embedding_length"), self.u("block_count"), self.u("attention.head_count"), self.u(
            "attention.head_count_kv")
        hd, ff, rd = self.u("attention.key_length"), self.u("feed_forward_length"), self.u("rope.dimension_count")
        eps = np.float32(1e-6)
        gemma = a.startswith("gemma")
        neox = a not in ("llama", "granite")
        swa_win = int(self.g.get(f"{a}.attention.sliding_window", 0))
        pattern = {"gemma2": 2, "gemma3": 6}.get(a, 0)
        granite = a == "granite"
        gf = lambda k, d: np.float32(self.g.get(f"{a}.{k}", d))
        embd_scale = np.sqrt(np.float32(e)) if gemma else (gf("embedding_scale", 1.0) if granite else np.float32(1))
        res_scale = gf("residual_scale", 1.0) if granite else np.float32(1)
        attn_scale = gf("attention.scale", 1.0) if granite else np.float32(1.0) / np.sqrt(np.float32(hd))
        cap_attn = 50.0 if a == "gemma2" else None
        cap_final = 30.0 if a == "gemma2" else None
        logit_scale = gf("logit_scale", 1.0) if granite else np.float32(1)
        base_global = gf("rope.freq_base", 10000.0)
        wtype = None

        def matvec(w, ty, x):
            xq = G.dequant_act(ty, x) if self.emulate else x
            return (w.astype(np.float64) @ xq.astype(np.float64)).astype(np.float32)

        # per-dimension frequency factors (Llama-3.1 rope_freqs.weight, else Phi-3's
        # rope_factors_short.weight): inv_freq[i] /= factor[i] where the factor is
        # nonzero (Rope::new, ops.rs:65-78; Model::load, model/mod.rs:130-133)
        fac_t = self.t("rope_freqs.weight")
        if fac_t is None:
            fac_t = self.t("rope_factors_short.weight")
        factors = None if fac_t is None else fac_t[0].reshape(-1).astype(np.float32)

        def rope(x, pos, base):
            i = np.arange(rd // 2)
            inv = np.power(np.float32(base), (np.float32(-2.0) * i.astype(np.float32) / np.float32(rd)), dtype=np.float32)
            if factors is not None:
                f = np.ones(rd // 2, np.float32)
                m = min(len(f), len(factors))
                f[:m] = np.where(factors[:m] != 0, factors[:m], np.float32(1))
                inv = (inv / f).astype(np.float32)
            th = (np.float32(pos) * inv).astype(np.float32)
            s, c = np.sin(th).astype(np.float32), np.cos(th).astype(np.float32)
            if neox:
                i0, i1 = i, i + rd // 2
            else:
                i0, i1 = 2 * i, 2 * i + 1
            x0, x1 = x[i0].copy(), x[i1].copy()
            x[i0] = x0 * c - x1 * s
            x[i1] = x0 * s + x1 * c

        embd, embd_ty = self.t("token_embd.weight")
        onorm, _ = self.t("output_norm.weight")
        out = self.t("output.weight")
        out_w, out_ty = out if out is not None else (embd, embd_ty)
        xs = [embd[tok] * embd_scale for tok in tokens]
        xs = [x.astype(np.float32) for x in xs]
        n = len(tokens)
        qd, kvd = nh * hd, nkv * hd
        for il in range(nl):
            get = lambda s: self.t(f"blk.{il}.{s}")
            qkv = get("attn_qkv.weight")
            if qkv is not None:
                f, wty = qkv
                wq, wk, wv = f[:qd], f[qd:qd + kvd], f[qd + kvd:]
            else:
                (wq, wty), (wk, _), (wv, _) = get("attn_q.weight"), get("attn_k.weight"), get("attn_v.weight")
            router = get("ffn_gate_inp.weight")
            wo, _ = get("attn_output.weight")
            if router is None:
                g_ = get("ffn_gate.weight")
                if g_ is not None:
                    (wg, fty), (wu, _) = g_, get("ffn_up.weight")
                else:
                    fu, fty = get("ffn_up.weight")
                    wg, wu = fu[:ff], fu[ff:]
                wd, _ = get("ffn_down.weight")

            def glu(wg, wu, wd, ty, h):
                gt = matvec(wg, ty, h)
                up = matvec(wu, ty, h)
                if gemma:
                    act = (np.float32(0.5) * gt * (1 + np.tanh(np.float32(0.7978846) * (gt + np.float32(0.044715) * gt * gt * gt)))).astype(np.float32)
                else:
                    act = (gt / (1 + np.exp(-gt))).astype(np.float32)
                return matvec(wd, ty, (act * up).astype(np.float32))

            is_swa = pattern > 0 and swa_win > 0 and il % pattern < pattern - 1
            base = np.float32(10000.0) if (a == "gemma3" and is_swa) else base_global
            an = get("attn_norm.weight")[0]
            qn, kn = get("attn_q_norm.weight"), get("attn_k_norm.weight")
            bq = get("attn_q.bias")
            qs, ks, vs = [], [], []
            for pos, x in enumerate(xs):
                h = _rms(x, an, eps)
                q, k, v = matvec(wq, wty, h), matvec(wk, wty, h), matvec(wv, wty, h)
                if bq is not None:
                    q = q + bq[0]
                    k = k + get("attn_k.bias")[0]
                    v = v + get("attn_v.bias")[0]
                q, k, v = q.astype(np.float32), k.astype(np.float32), v.astype(np.float32)
                for hh in range(nh):
                    s = q[hh * hd:(hh + 1) * hd]
                    if qn is not None:
                        s[:] = _rms(s, qn[0], eps)
                    rope(s, pos, base)
                for hh in range(nkv):
                    s = k[hh * hd:(hh + 1) * hd]
                    if kn is not None:
                        s[:] = _rms(s, kn[0], eps)
                    rope(s, pos, base)
                if self.emulate:
                    k = k.astype(np.float16).astype(np.float32)
                    v = v.astype(np.float16).astype(np.float32)
                qs.append(q)
                ks.append(k)
                vs.append(v)
            pan, pfn = get("post_attention_norm.weight"), get("post_ffw_norm.weight")
            fnorm = get("ffn_norm.weight")[0]
            for i in range(n):
                att = np.zeros(qd, np.float32)
                for hh in range(nh):
                    g = hh // (nh // nkv)
                    lo = max(0, i + 1 - swa_win) if is_swa else 0
                    sc = np.array([np.dot(qs[i][hh * hd:(hh + 1) * hd].astype(np.float64), ks[j][g * hd:(g + 1) * hd]) for j in
                                   range(lo, i + 1)], np.float32) * np.float32(attn_scale)
                    if cap_attn:
                        sc = cap_attn * np.tanh(sc / cap_attn)
                    p = np.exp(sc - sc.max())
                    p = p / p.sum()
                    vv = np.stack([vs[j][g * hd:(g + 1) * hd] for j in range(lo, i + 1)])
                    att[hh * hd:(hh + 1) * hd] = (p.astype(np.float64) @ vv.astype(np.float64)).astype(np.float32)
                o = matvec(wo, wty, att)
                if pan is not None:
                    o = _rms(o, pan[0], eps)
                xs[i] = (xs[i] + o * res_scale).astype(np.float32)
                h = _rms(xs[i], fnorm, eps)
                if router is None:
                    d = glu(wg, wu, wd, fty, h)
                else:
                    ne, kk, fx = self.u("expert_count"), self.u("expert_used_count"), self.u("expert_feed_forward_length")
                    (ga, ety), (ua, _), (da, _) = get("ffn_gate_exps.weight"), get("ffn_up_exps.weight"), get(
                        "ffn_down_exps.weight")
                    pr = (router[0].astype(np.float64) @ h.astype(np.float64))
                    pr = np.exp(pr - pr.max())
                    pr = pr / pr.sum()
                    order = sorted(range(ne), key=lambda j: (-pr[j], j))
                    top = order[:kk]
                    norm = 1.0 if a == "qwen2moe" else sum(pr[j] for j in top)
                    d = np.zeros(e, np.float64)
                    for x_ in top:
                        y = glu(ga[x_ * fx:(x_ + 1) * fx], ua[x_ * fx:(x_ + 1) * fx], da[x_ * e:(x_ + 1) * e], ety, h)
                        d += pr[x_] / norm * y
                    sg = get("ffn_gate_shexp.weight")
                    if sg is not None:
                        y = glu(sg[0], get("ffn_up_shexp.weight")[0], get("ffn_down_shexp.weight")[0], sg[1], h)
                        gw = get("ffn_gate_inp_shexp.weight")[0]
                        scs = 1.0 / (1.0 + np.exp(-np.dot(gw.astype(np.float64), h)))
                        d += scs * y
                    d = d.astype(np.float32)
                if pfn is not None:
                    d = _rms(d, pfn[0], eps)
                xs[i] = (xs[i] + d * res_scale).astype(np.float32)
        outs = []
        for x in xs:
            h = _rms(x, onorm, eps)
            hq = G.dequant_act(out_ty, h) if self.emulate else h
            l = (out_w.astype(np.float64) @ hq.astype(np.float64)).astype(np.float32)
            l = l / logit_scale
            if cap_final:
                l = cap_final * np.tanh(l / cap_final)
            outs.append(l.astype(np.float32))
        return outs


def max_rel_err(a, b):
    """tests/common/mod.rs:33-36"""
    scale = max(float(np.abs(b).max()), 1e-6)
    return float(np.abs(np.asarray(a) - np.asarray(b)).max()) / scale
