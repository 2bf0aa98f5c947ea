#!/usr/bin/env python3
"""Throughput of RIE's per-token forward loop on one MI355X.

Workload (Llama-3.1-8B-shaped synthetic model, Q4_0): 32 layers, hidden 4096,
32 query / 8 KV heads of 128, SwiGLU FFN 14336, vocab 128256, untied Q4_0 output
head, weights N(0, 0.02) quantized with quantize::q4_0, unit norms, RoPE base
5e5, f16 KV cache.  One step = Engine::bench (crates/rie-core/src/engine.rs:
540-564): a 512-token prompt evaluated as one batch (pp512), then 128 greedy
decode steps (tg128) with on-device argmax.  The GGUF image is uploaded once and
is resident in HBM before timing starts.

value = tg128 tokens/s; pp512 tokens/s is reported beside it, with its int8
MFMA roofline (2·tokens·layer parameters, the head for the last token, over 5
POPS).  The roofline entry is the dominant decode kernel (the fused
gate/up/SwiGLU GEMV), timed with HIP events on the backend's stream.
cpu_baseline is RIE's CPU path restated in C (the oracle) on the same image, on a
bounded sample, at 8 threads and at every physical core.  --workload selects the
other benchmark shapes (Qwen3-1.7B Q4_0, Llama-3.2-3B Q4_K_M, Qwen3-30B-A3B Q4_K).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E


WORKLOADS = {
    # name: (spec builder, description, attention heads (query, kv))
    "llama3.1-8b-q4_0": ("baseline_llama31_8b_q4_0", "llama-3.1-8b-shaped q4_0, pp512 then greedy tg128, f16 KV"),
    "qwen3-1.7b-q4_0": ("baseline_qwen3_1_7b_q4_0", "qwen3-1.7b-shaped q4_0 (tied q6_k head), pp512 then greedy tg128, f16 KV"),
    "llama3.2-3b-q4_k_m": ("baseline_llama32_3b_q4_k_m", "llama-3.2-3b-shaped q4_k_m mix (tied q6_k head), pp512 then greedy tg128, f16 KV"),
    "qwen3-30b-a3b-q4_k": ("baseline_qwen3_30b_a3b_q4_k", "qwen3-30b-a3b-shaped moe q4_k (128 experts, top-8), pp512 then greedy tg128, f16 KV"),
}
DEFAULT_WORKLOAD = "llama3.1-8b-q4_0"
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--gen", type=int, default=128)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default=DEFAULT_WORKLOAD,
                    help="the benchmark workload (default: the Llama-3.1-8B Q4_0 headline)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-only", action="store_true", help="short run of the roofline kernel (for counters)")
    ap.add_argument("--prefill-only", action="store_true", help="short run of pp512 prompts only (for counters)")
    ap.add_argument("--long-context", action="store_true",
                    help="the 32K-context workload instead: pp32768 then tg128 on the same 8B Q4_0 model, Turbo4 and f16 KV")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the forward loop on one GPU; runs on more than one GPU are not part of this build",
              file=sys.stderr)
        sys.exit(2)

    if args.kernel_only:
        return kernel_only(args)
    if args.long_context:
        return long_context(args)
    import torch

    import rust_interference_engine_amd as R
    from rust_interference_engine_amd import gguf, synth

    assert torch.cuda.is_available(), "needs the MI355X"
    builder, wl_desc = WORKLOADS[args.workload]
    t0 = time.time()
    spec = getattr(synth, builder)(seed=1, ctx=8192)
    img = synth.build_array(spec)
    t_gen = time.time() - t0
    E, V, L = spec.n_embd, spec.n_vocab, spec.n_layer
    kvd = spec.n_head_kv * spec.head_dim
    costs = gguf.per_token_costs(img, spec.n_expert_used if spec.n_expert else 0)
    n_ctx = args.prompt + args.gen + 64
    t0 = time.time()
    be = R.HipBackend(img, n_ctx=n_ctx, max_batch=args.prompt, kv_type=R.KvType.F16)
    t_load = time.time() - t0
    prompt = [(i * 7919 + 13) % V for i in range(args.prompt)]

    if args.prefill_only:  # counter runs: prompts only
        be.forward_argmax(prompt[:8], 0)
        for _ in range(max(args.steps, 1)):
            be.forward_argmax(prompt, 0)
        torch.cuda.synchronize()
        print(json.dumps({"prefill_only": args.workload, "steps": args.steps}), flush=True)
        return

    def step():
        torch.cuda.synchronize()
        a = time.perf_counter()
        be.forward_argmax(prompt, 0)
        torch.cuda.synchronize()
        b = time.perf_counter()
        toks = be.generate_greedy(args.prompt, args.gen)
        torch.cuda.synchronize()
        c = time.perf_counter()
        return b - a, c - b, toks

    be.forward_argmax(prompt[:8], 0)  # Engine::bench warm-up on the first 8 tokens
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    pp_t = tg_t = 0.0
    toks = None
    for _ in range(args.steps):
        a, b, toks = step()
        pp_t += a
        tg_t += b
    torch.cuda.synchronize()
    total = time.perf_counter() - t_start
    tg_tps = args.gen * args.steps / tg_t
    pp_tps = args.prompt * args.steps / pp_t

    # ---- the same 512-token prefill fed in micro-batches of 1, 128 and 512 tokens ----
    def prefill_batched(b):
        torch.cuda.synchronize()
        t = time.perf_counter()
        for p0 in range(0, args.prompt, b):
            be.forward_argmax(prompt[p0:p0 + b], p0)
        torch.cuda.synchronize()
        return args.prompt / (time.perf_counter() - t)
    by_batch = {str(b): round(prefill_batched(b), 1) for b in (1, 128)}
    by_batch[str(args.prompt)] = round(pp_tps, 1)

    # ---- algorithmic costs: decode bytes per token at mid context, prefill int8 ops ----
    ctx_mid = args.prompt + args.gen // 2
    kv_bytes = L * 2 * kvd * 2 * (ctx_mid + 1)  # K and V rows read, f16
    tok_bytes = costs["layer_weight_bytes"] + costs["head_bytes"] + costs["embd_row_bytes"] + kv_bytes
    pp_ops = 2 * args.prompt * costs["layer_params"] + 2 * costs["head_params"]  # head for the last token only
    pp_tops = pp_ops / (pp_t / args.steps) / 1e12

    # ---- roofline of the dominant decode kernel, timed live with HIP events ----
    # (the single-token gate/up/SwiGLU launch over every layer's weights in turn,
    # on the backend's stream, so each launch streams its weights from HBM)
    roofline = None
    if not spec.n_expert:
        glu_us, glu_bytes = be.time_ffn_glu(reps=3)
        achieved = glu_bytes / (glu_us / 1e6) / 1e9
        roofline = {"bound": "hbm", "kernel": "gemv_dec_kernel gate+up+SwiGLU (RMSNorm+quantization of x in the prologue, "
                                              "quantized hidden out)",
                    "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": measured_traffic() if args.workload == DEFAULT_WORKLOAD else None,
                    "traffic_source": ("rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this kernel, scaled by a 256 MiB copy: "
                                       "profiles/gemv_dec_gate_up_glu_llama8b_q4_0_pmc.md (not measured in this run)")
                    if args.workload == DEFAULT_WORKLOAD else None,
                    "bytes_per_launch": glu_bytes, "avg_launch_us": round(glu_us, 2)}
    prof = be.profile_decode(ctx_mid, reps=5)
    step_ms = sum(v[0] for v in prof.values()) / 5

    headline = args.workload == DEFAULT_WORKLOAD
    out = {
        "metric": "tg128 tok/s (Llama-3.1-8B Q4_0, after pp512)" if headline else f"tg128 tok/s ({args.workload}, after pp512)",
        "value": round(tg_tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x ggml blocks (int32 block dots, f32 accumulate)",
        "data": "synthetic: N(0,0.02) weights quantized to the workload's ggml types, prompt ids (i*7919+13) mod V",
        "config": {"workload": wl_desc, "prompt": args.prompt, "gen": args.gen, "layers": L, "hidden": E,
                   "ffn": spec.n_ff_exp if spec.n_expert else spec.n_ff, "vocab": V, "heads": [spec.n_head, spec.n_head_kv],
                   "experts": [spec.n_expert, spec.n_expert_used] if spec.n_expert else None},
        "pp512_tok_s": round(pp_tps, 1),
        "prefill_tok_s_by_batch": by_batch,
        "prefill_roofline": {"bound": "mfma", "achieved": round(pp_tops, 2), "peak": INT8_PEAK_TOPS, "unit": "TOP/s (int8)",
                             "frac": round(pp_tops / INT8_PEAK_TOPS, 4), "ops_per_prompt": int(pp_ops)},
        "decode_ms_per_token": round(tg_t / (args.gen * args.steps) * 1e3, 4),
        "decode_bytes_per_token": int(tok_bytes),
        "decode_effective_gbs": round(tok_bytes / (tg_t / (args.gen * args.steps)) / 1e9, 1),
        "decode_frac_hbm_roofline": round(tok_bytes / (tg_t / (args.gen * args.steps)) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": roofline,
        "eager_decode_kernel_ms": {k: round(v[0] / 5, 4) for k, v in prof.items()},
        "eager_decode_step_ms": round(step_ms, 3),
        "setup_s": {"synthesize": round(t_gen, 1), "upload": round(t_load, 1)},
        "greedy_head": [int(t) for t in toks[:8]],
    }
    if not args.no_cpu_baseline and headline:
        out["cpu_baseline"] = cpu_baseline(img, V, args)
    print(json.dumps(out), flush=True)


def measured_traffic():
    """HBM bytes per gate/up/SwiGLU launch from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, scaled by a copy of known size)."""
    path = os.path.join(ROOT, "profiles", "gemv_dec_gate_up_glu_llama8b_q4_0_pmc.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def long_context(args):
    """The 32K-context workload: the 8B Q4_0 model, a 32768-token prompt fed in
    512-token batches (Engine::eval_tokens chunking), then 128 greedy steps, with
    Turbo4 and with f16 KV caches.  One JSON line; not the bench line."""
    import torch

    import rust_interference_engine_amd as R
    from rust_interference_engine_amd import synth

    assert torch.cuda.is_available(), "needs the MI355X"
    n_prompt, n_gen, mb = 32768, 128, 512
    spec = synth.baseline_llama31_8b_q4_0(seed=1, ctx=n_prompt + n_gen + 128)
    img = synth.build_array(spec)
    V = spec.n_vocab
    prompt = [(i * 7919 + 13) % V for i in range(n_prompt)]
    res = {}
    for name, kv in (("turbo4", R.KvType.TURBO4), ("f16", R.KvType.F16)):
        be = R.HipBackend(img, n_ctx=n_prompt + n_gen + 64, max_batch=mb, kv_type=kv)
        be.forward_argmax(prompt[:8], 0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for p0 in range(0, n_prompt, mb):
            be.forward_argmax(prompt[p0:p0 + mb], p0)
            if p0 % (8 * mb) == 0:
                print(f"{name}: prefilled {p0 + mb} tokens", file=sys.stderr, flush=True)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        toks = be.generate_greedy(n_prompt, n_gen)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        res[name] = {"pp32768_tok_s": round(n_prompt / (t1 - t0), 1), "tg128_tok_s": round(n_gen / (t2 - t1), 2),
                     "kv_bytes": be.kv_bytes(), "greedy_head": [int(t) for t in toks[:8]]}
        print(f"{name}: {res[name]}", file=sys.stderr, flush=True)
        be.close()
    print(json.dumps({"metric": "pp32768 and tg128 tok/s at 32K context (Llama-3.1-8B Q4_0; Turbo4 vs f16 KV)", "n_gpus": 1,
                      "data": "synthetic: N(0,0.02) weights quantized to Q4_0, prompt ids (i*7919+13) mod V", **res}), flush=True)


def kernel_only(args):
    """Short run for counter collection: the gate/up/SwiGLU launch over all
    layers, then a device copy of known size that calibrates the counters."""
    import torch

    import rust_interference_engine_amd as R
    from rust_interference_engine_amd import synth

    spec = synth.baseline_llama31_8b_q4_0(seed=1, ctx=8192)
    img = synth.build_array(spec)
    be = R.HipBackend(img, n_ctx=64, max_batch=8, kv_type=R.KvType.F16)
    be.forward_argmax([13, 7932, 15851], 0)
    us, nb = be.time_ffn_glu(reps=1)
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"ffn_glu_avg_us": round(us, 2), "bytes_per_launch": nb, "copy_bytes": n}), flush=True)


def _cpu_model_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _physical_cores():
    """cores this process may run on, counted once per physical core"""
    allowed = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    seen = set()
    for c in allowed:
        try:
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/core_id") as f:
                core = f.read().strip()
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id") as f:
                pkg = f.read().strip()
            seen.add((pkg, core))
        except OSError:
            seen.add(("?", c))
    return max(1, len(seen)), len(allowed)


def cpu_baseline(img, V, args):
    """RIE's CPU path (the oracle: a C restatement of RIE's x86 backend, AVX2
    semantics, RIE's row chunking and fork/join pool) on the same GGUF image, at
    RIE's default of 8 threads (crates/rie-core/src/cpu.rs:100-102) and at every
    physical core.  Bounded sample: Engine::bench's warm-up on 8 tokens, one
    32-token prompt batch (whole 4-token tiles, as the 64-token chunks of RIE's
    default -b 64: pp512 is extrapolated from its rate), then 6 greedy decode
    steps at context 32-38 (the GPU's decode runs at 512-640; the KV share of the
    bytes per token is under 2% at either length)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as O

    phys, allowed = _physical_cores()
    m = O.Model(img)
    n_pp, n_gen = 32, 6
    prompt = [(i * 7919 + 13) % V for i in range(n_pp)]
    runs = {}
    for threads in sorted({min(8, allowed), phys}):
        b = O.Backend(m, 128, 64, O.KV_F16, n_threads=threads)
        b.forward(prompt[:8], 0)  # warm-up (engine.rs:544-546)
        t0 = time.perf_counter()
        logits = b.forward(prompt, 0)
        t1 = time.perf_counter()
        tok = O.argmax(logits)
        for i in range(n_gen):
            logits = b.forward([tok], n_pp + i)
            tok = O.argmax(logits)
        t2 = time.perf_counter()
        runs[threads] = {"threads": threads, "pp32_tok_s": round(n_pp / (t1 - t0), 2),
                         "pp512_tok_s_extrapolated": round(n_pp / (t1 - t0), 2), "tg_tok_s": round(n_gen / (t2 - t1), 3)}
        del b
    base = runs[min(8, allowed)]
    return {"value": base["tg_tok_s"], "unit": "tok/s", "cores": base["threads"], "kind": "port",
            "label": "RIE CPU path (C++ restatement)", "cpu_model": _cpu_model_name(), "nproc": os.cpu_count(),
            "physical_cores_allowed": phys, "runs": list(runs.values()),
            "sample": "same image; warm-up on 8 tokens, one 32-token prompt batch (pp512 extrapolated from its rate), "
                      "then 6 greedy decode steps at context 32-38; value = decode tok/s at 8 threads"}


if __name__ == "__main__":
    main()
