#!/usr/bin/env python3
"""Benchmark of the INT4 expert path on one MI355X.

Default run (no --mode): BASELINE config 1 is the headline `value`; config 2
(20B-shaped greedy decode) and config 4 (120B-shaped decode at batch 1 and
32) are timed in the same process and reported under `config`.

Config 1: one GPT-OSS-20B-shaped MoE layer at
batch-1 decode -- RMSNorm'd fp32 x [2880], fp32 router [32x2880] + bias,
top-4 of 32 INT4 gs64 experts (gate_up 5760x2880, down 2880x2880, biases),
clamped SwiGLU, softmax-weighted combine -- over fresh seeded tokens. A
"step" is one token through that layer, three launches (router, gate_up
with the in-launch top-4, down with the combine) replayed from a HIP graph.
Token t uses layer copy t % L (L = 24, the 20B model's MoE layers, 10.8 GB of
experts) so the expert bytes come from HBM, not from the 256 MB MALL.

value = algorithmic HBM bytes per token (experts + router + x/out) x tokens/s.
roofline = the dominant kernel (gate_up + SwiGLU, four routed experts per
launch): its algorithmic bytes per launch / its mean duration, from HIP
events on the engine stream around each of its launches in eager layers.
cpu_baseline = picchio's MoE layer on the host cores (oracle/_ref build of
the reference when present, else the C restatement).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
METRIC = "INT4 expert GEMV GB/s (% HBM peak); decode tok/s GPT-OSS-20B/120B shape"

D, INTER, HALF, E, K = 2880, 5760, 2880, 32, 4
EXPERT_BYTES = 12441600 + 1555200 + 34560          # packed + scales + biases
ROUTER_BYTES = E * D * 4 + E * 4
TOKEN_BYTES = K * EXPERT_BYTES + ROUTER_BYTES + 2 * D * 4      # 56,517,248

# HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE, then
# WRITE_SIZE, in passes of their own), scaled by what the two counters read
# for a 1 GiB device copy in the same call (x 2.000 and x 1.000):
#  * k_moe_ffn (the default, profiles/k_moe_ffn_moe_config1.txt), measured on
#    commit d70a076: FETCH_SIZE 27792.77 KiB x 2 + WRITE_SIZE 168.84 KiB;
#  * k_i4_gemv<SWIGLU> gate_up of the two-launch experts
#    (pk_set_moe_fused(e, 0)), measured on commit 0a0ca63: FETCH_SIZE
#    18425.54 KiB x 2 + WRITE_SIZE 45.04 KiB.
MOE_FFN_TRAFFIC = 57092529
GATE_UP_TRAFFIC = 37780589


def host_info():
    """CPU model, threads available to this process, NUMA nodes of the host."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        nodes = sorted(d for d in os.listdir("/sys/devices/system/node") if d.startswith("node"))
    except OSError:
        nodes = []
    return {"cpu_model": model, "threads_available": len(os.sched_getaffinity(0)),
            "numa_nodes": len(nodes), "nproc": os.cpu_count()}


def gate_up_bytes(n):
    """Algorithmic bytes of one gate_up launch over n experts: packed nibbles,
    scales, bias of each, x in, SwiGLU activations out."""
    return n * (INTER * D // 2 + INTER * (D // 64) * 4 + INTER * 4) + D * 4 + n * HALF * 4


def down_bytes(n):
    """One down launch over n experts: weights + scales + bias, activations in, outputs out."""
    return n * (D * HALF // 2 + D * (HALF // 64) * 4 + D * 4) + n * HALF * 4 + n * D * 4


def replay_ms(eng, ev0, ev1, n, enqueue, reps=3):
    """Mean duration of one of n launches captured in a graph and replayed
    back to back (events on the engine stream around each replay)."""
    eng.capture_begin()
    for t in range(n):
        enqueue(t)
    g = eng.capture_end()
    eng.graph_launch(g)
    eng.sync()
    tot = 0.0
    for _ in range(reps):
        ev0.record(eng.stream)
        eng.graph_launch(g)
        ev1.record(eng.stream)
        ev1.synchronize()
        tot += ev0.elapsed_time(ev1)
    eng.graph_destroy(g)
    return tot / (reps * n)


def token_inputs(n, seed):
    """x_t = rmsnorm(N(0,1)) with unit norm weights, fp32."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, D)).astype(np.float32)
    ms = (x.astype(np.float64) ** 2).sum(axis=1) / D
    r = (np.float32(1.0) / np.sqrt((ms.astype(np.float32) + np.float32(1e-5)))).astype(np.float32)
    return (x * r[:, None]).astype(np.float32)


def cpu_baseline(x, seed, budget_s):
    """picchio's moe_forward on the host (time-bounded sample of the same tokens)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_ffi import Oracle, Reference, reference_available, make_cfg
    o = Oracle()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    cfg = make_cfg(n_layers=1, n_experts=E, ctx_len=16, vocab=64)
    model = o.model_build(cfg, seed, threads)
    kind = "port"
    if reference_available():
        ref = Reference()
        ref.attach(model, cfg)
        run = lambda xt, out: ref.moe_forward(0, xt, out)
        kind = "reference"
    else:
        sel = np.empty(K, np.int32)
        w = np.empty(K, np.float32)
        run = lambda xt, out: o.moe_forward(model, 0, xt, out, sel, w, None)
    out = np.empty(D, np.float32)
    run(x[0], out)                                   # warm-up (page in)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        run(x[n % len(x)], out)
        n += 1
    dt = time.perf_counter() - t0
    o.model_free(model)
    return {"value": round(n * TOKEN_BYTES / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": kind, "tokens_per_s": round(n / dt, 2),
            "sample": f"{n} tokens of the same MoE layer (1 layer, 32 experts resident in RAM), "
                      f"{dt:.1f} s, OpenMP {threads} threads"}


def decode_bytes_per_token(cfg, pos):
    """Algorithmic HBM bytes of one forward_token at position pos: top-k
    experts, router, attention weights and biases, the KV rows each layer's
    window reads, the embedding row and the fp32 lm_head (+ logits out)."""
    D, H, KVH, hd = cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    E, K, V = cfg.n_experts, cfg.topk, cfg.vocab
    half = cfg.moe_inter // 2
    ng_d, ng_h = D // 64, half // 64
    expert = (cfg.moe_inter * D // 2 + cfg.moe_inter * ng_d * 4 + cfg.moe_inter * 4
              + D * half // 2 + D * ng_h * 4 + D * 4)
    qkv = (H + 2 * KVH) * hd
    attn = 4 * (qkv * D + D * H * hd + qkv + D + H) + 4 * 2 * D          # + two norms
    kv_dim = KVH * hd
    total = 0
    for l in range(cfg.n_layers):
        n_pos = min(pos + 1, cfg.sliding_window) if cfg.layer_type[l] == 0 else pos + 1
        total += K * expert + 4 * (E * D + E) + attn + 2 * 4 * n_pos * kv_dim + 4 * kv_dim * 2
    lm = V * D * (4 if cfg.lm_head_fmt == 0 else 1) + (0 if cfg.lm_head_fmt == 0 else 4 * V)
    return total + 4 * D + lm + 4 * D


def cpu_decode_baseline(cfg, seed, budget_s, prompt):
    """picchio's forward_token on the host cores for the same model shape
    (time-bounded sample)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_ffi import Oracle, Reference, reference_available
    o = Oracle()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    t0 = time.perf_counter()
    model = o.model_build(cfg, seed, threads)
    build_s = time.perf_counter() - t0
    if reference_available():
        ref = Reference()
        ref.attach(model, cfg)
        ref.reset_kv()
        step = lambda tok, pos: ref.forward_token(tok, pos)
        kind = "reference"
    else:
        step = lambda tok, pos: o.forward_token(model, tok, pos, None)
        kind = "port"
    tok = int(prompt[0])
    tok = step(tok, 0)                                  # warm-up (page in)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        tok = step(int(prompt[(n + 1) % len(prompt)]), n + 1)
        n += 1
    dt = time.perf_counter() - t0
    o.model_free(model)
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": threads, "kind": kind,
            "sample": f"{n} forward_token steps at positions 1..{n} of the same 20B-shaped model "
                      f"(all experts resident in RAM, fp32 lm_head), {dt:.1f} s, OpenMP {threads} "
                      f"threads; model build {build_s:.0f} s"}


def parse_sampling(spec):
    """--sample T,top_p,top_k,rep (picchio's defaults: 1.0,0.95,50,1.1) or None."""
    if not spec:
        return None
    t, p, k, r = spec.split(",")
    return float(t), float(p), int(k), float(r)


def measure_decode20b(args, steps, warmup, cpu_on):
    """GPT-OSS-20B-shaped model, 512-token prompt through
    prefill_tokens, then `steps` greedy decode steps replayed from the
    captured step graph. value = decode tokens/s."""
    import torch
    import picchio_amd as pa
    n_prompt = 512
    cfg = pa.gptoss_cfg(ctx_len=n_prompt + steps + 1)
    eng = pa.Engine(cfg)
    t0 = time.perf_counter()
    eng.build_synthetic(args.seed, what=7)
    eng.sync()
    print(f"[bench] 20B model built on the GPU: {eng.device_bytes() / 1e9:.2f} GB in "
          f"{time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    prompt = np.random.default_rng(args.seed + 100).integers(0, cfg.vocab, n_prompt).astype(np.int32)
    sampling = parse_sampling(args.sample)
    if sampling:
        eng.set_sampling(*sampling, args.seed)
    t0 = time.perf_counter()
    nxt = eng.prefill_tokens(prompt)
    prefill_s = time.perf_counter() - t0
    # warm-up: captures the step graph and runs `warmup` steps from the same state
    # (the sampler restarts from the same seed before each run)
    if sampling:
        eng.set_sampling(*sampling, args.seed)
    warm = eng.decode_replay(nxt, n_prompt, max(warmup, 1))
    if sampling:
        eng.set_sampling(*sampling, args.seed)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(eng.stream)
    toks = eng.decode_replay(nxt, n_prompt, steps)
    ev1.record(eng.stream)
    ev1.synchronize()
    ms = ev0.elapsed_time(ev1)
    assert list(toks[:len(warm)]) == list(warm), "decode is not deterministic"
    # per-kernel event brackets on one eager step (lm_head, attention)
    eng.profile(True)
    eng.forward_token(int(toks[-1]), n_prompt + steps, None)     # ctx_len leaves this position free
    lm_ms, _ = eng.profile_read(pa.PROF_LM_HEAD)
    att_ms, att_n = eng.profile_read(pa.PROF_ATTENTION)
    eng.profile(False)
    eng.close()
    tok_s = steps / (ms * 1e-3)
    bpt = sum(decode_bytes_per_token(cfg, n_prompt + i) for i in range(steps)) / steps
    lm_bytes = cfg.vocab * cfg.hidden * 4 + cfg.hidden * 4 + cfg.vocab * 4
    cpu = None
    if cpu_on:
        cpu = cpu_decode_baseline(cfg, args.seed, args.cpu_seconds, prompt)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)
    print(f"[bench] config 2: {tok_s:.1f} tok/s ({ms / steps * 1e3:.1f} us/token), prefill "
          f"{prefill_s:.3f} s", file=sys.stderr, flush=True)
    line = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms / steps, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "config2: GPT-OSS-20B-shaped " + ("sampled" if sampling else "greedy") +
                               " decode, batch 1, 512-token random-id prompt then 256 steps, all "
                               "experts HBM-resident",
                   "sampling": ({"temperature": sampling[0], "top_p": sampling[1], "top_k": sampling[2],
                                 "rep_penalty": sampling[3], "seed": args.seed} if sampling else "greedy"),
                   "layers": cfg.n_layers, "experts": cfg.n_experts, "vocab": cfg.vocab,
                   "lm_head": "fp32", "bytes_per_token": int(bpt),
                   "hbm_gbps": round(bpt * tok_s / 1e9, 1),
                   "hbm_frac": round(bpt * tok_s / 1e9 / HBM_PEAK_GBPS, 4),
                   "prefill_s": round(prefill_s, 3), "prefill_tok_s": round(n_prompt / prefill_s, 1),
                   "attention_us_per_layer": round(att_ms / max(att_n, 1) * 1e3, 2),
                   "first_tokens": [int(nxt)] + [int(t) for t in toks[:8]]},
        "roofline": {"bound": "hbm", "achieved": round(lm_bytes / (lm_ms * 1e-3) / 1e9, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(lm_bytes / (lm_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                     "traffic": None, "kernel": "k_lm_head<fp32> (201088 x 2880 GEMV, per-block maxima)",
                     "bytes_per_launch": lm_bytes, "mean_us": round(lm_ms * 1e3, 3)},
        "cpu_baseline": cpu,
    }
    return line


def measure_decode120b(args, steps, warmup, cpu_on):
    """GPT-OSS-120B-shaped model (36 layers, 128 INT4 experts
    per layer, ~65 GB of experts resident in HBM), a 4096-position KV context
    filled with synthetic rows, then `steps` greedy decode steps at batch 1
    (captured step graph) and at batch 32 (32 independent sequences in
    lockstep). value = batch-1 tokens/s."""
    import torch
    import picchio_amd as pa
    ctx, B = 4096, 32
    cfg = pa.gptoss_cfg(n_layers=36, n_experts=128, ctx_len=ctx + steps + 1)
    eng = pa.Engine(cfg)
    t0 = time.perf_counter()
    eng.build_synthetic(args.seed, what=7)
    eng.sync()
    print(f"[bench] 120B model built on the GPU: {eng.device_bytes() / 1e9:.2f} GB in "
          f"{time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    rng = np.random.default_rng(args.seed + 200)
    # batch 1
    eng.kv_fill_synthetic(0, ctx, args.seed)
    tok = int(rng.integers(0, cfg.vocab))
    warm = eng.decode_replay(tok, ctx, max(warmup, 1))
    ev0.record(eng.stream)
    toks1 = eng.decode_replay(tok, ctx, steps)
    ev1.record(eng.stream)
    ev1.synchronize()
    ms1 = ev0.elapsed_time(ev1)
    assert list(toks1[:len(warm)]) == list(warm), "decode is not deterministic"
    eng.profile(True)
    eng.forward_token(int(toks1[-1]), ctx + steps, None)
    lm_ms, _ = eng.profile_read(pa.PROF_LM_HEAD)
    eng.profile(False)
    # batch 32
    eng.batch_reserve(B)
    for sq in range(B):
        eng.kv_fill_synthetic(sq, ctx, args.seed + sq)
    first = rng.integers(0, cfg.vocab, B).astype(np.int32)
    eng.decode_batch(first, ctx, max(warmup, 1))
    ev0.record(eng.stream)
    out32 = eng.decode_batch(first, ctx, steps)
    ev1.record(eng.stream)
    ev1.synchronize()
    ms32 = ev0.elapsed_time(ev1)
    eng.close()
    tok1 = steps / (ms1 * 1e-3)
    tok32 = B * steps / (ms32 * 1e-3)
    bpt1 = sum(decode_bytes_per_token(cfg, ctx + i) for i in range(steps)) / steps
    # batch 32: expected distinct experts per layer under uniform routing
    E, Kk = cfg.n_experts, cfg.topk
    uniq = E * (1.0 - (1.0 - Kk / E) ** B)
    expert = (cfg.moe_inter * D // 2 + cfg.moe_inter * (D // 64) * 4 + cfg.moe_inter * 4
                           + D * HALF // 2 + D * (HALF // 64) * 4 + D * 4)
    kv_bytes = lambda pos: sum(2 * 4 * (min(pos + 1, 128) if cfg.layer_type[l] == 0 else pos + 1) * 512
                               for l in range(cfg.n_layers))
    dense = bpt1 - cfg.n_layers * Kk * expert - kv_bytes(ctx + steps // 2)
    bstep32 = dense + cfg.n_layers * uniq * expert + B * kv_bytes(ctx + steps // 2)
    lm_bytes = cfg.vocab * cfg.hidden * 4 + cfg.hidden * 4 + cfg.vocab * 4
    cpu = None
    if cpu_on:
        cpu = cpu_decode_baseline(cfg, args.seed, args.cpu_seconds, first)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)
    print(f"[bench] config 4: batch 1 {tok1:.1f} tok/s, batch 32 {tok32:.1f} tok/s", file=sys.stderr,
          flush=True)
    line = {
        "metric": METRIC, "value": round(tok1, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms1 / steps, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "config4: GPT-OSS-120B-shaped greedy decode (36 layers, 128 INT4 experts, "
                               "fp32 attention and lm_head), 4096-position synthetic KV context, "
                               f"{steps} steps at batch 1 and at batch 32",
                   "layers": cfg.n_layers, "experts": E, "vocab": cfg.vocab,
                   "batch1_tok_s": round(tok1, 2), "batch1_bytes_per_token": int(bpt1),
                   "batch1_hbm_gbps": round(bpt1 * tok1 / 1e9, 1),
                   "batch32_tok_s": round(tok32, 2), "batch32_ms_per_step": round(ms32 / steps, 4),
                   "batch32_bytes_per_step": int(bstep32),
                   "batch32_hbm_gbps": round(bstep32 * steps / (ms32 * 1e-3) / 1e9, 1),
                   "batch32_distinct_experts_per_layer": round(uniq, 1),
                   "kv_context": "synthetic N(0,1) rows for positions 0..4095 of every sequence",
                   "first_tokens_batch1": [int(t) for t in toks1[:6]],
                   "first_tokens_batch32_seq0": [int(t) for t in out32[:6, 0]]},
        "roofline": {"bound": "hbm", "achieved": round(lm_bytes / (lm_ms * 1e-3) / 1e9, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(lm_bytes / (lm_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "k_lm_head<fp32> (201088 x 2880 GEMV, per-block maxima)",
                     "bytes_per_launch": lm_bytes, "mean_us": round(lm_ms * 1e3, 3)},
        "cpu_baseline": cpu,
    }
    return line


def zipf_routing(T, E, K, seed, s=1.1, lo=16, hi=512):
    """BASELINE config 3 routing: per-expert pair counts proportional to
    (e+1)^-s, clipped to [lo, hi] and summing to T*K; slot i of the
    expert-sorted list goes to token i % T (an expert's run is shorter than T,
    so every token gets K distinct experts); tokens shuffled; combine weights
    = softmax of K random logits."""
    P = T * K
    x = (np.arange(E) + 1.0) ** -s
    a, b = 0.0, 1e9
    for _ in range(200):
        c = (a + b) / 2
        a, b = (c, b) if np.clip(c * x, lo, hi).sum() < P else (a, c)
    f = np.clip(c * x, lo, hi)
    counts = np.floor(f).astype(np.int64)
    for e in np.argsort(-(f - counts)):
        if counts.sum() >= P:
            break
        if counts[e] < hi:
            counts[e] += 1
    slots = np.repeat(np.arange(E), counts)[:P]
    sel = slots.reshape(K, T).T.copy()
    rng = np.random.default_rng(seed)
    sel = sel[rng.permutation(T)].astype(np.int32)
    lg = rng.standard_normal((T, K))
    w = np.exp(lg - lg.max(axis=1, keepdims=True))
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return sel, w, counts


def cpu_pairs_baseline(seed, budget_s, x, sel, w):
    """picchio's expert_apply (the per-pair work of forward_prefill's MoE,
    picchio.c:1885-1905) on the host cores, time-bounded sample of the pairs."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_ffi import Oracle, Reference, reference_available, make_cfg
    o = Oracle()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    cfg = make_cfg(n_layers=1, n_experts=E, ctx_len=16, vocab=64)
    model = o.model_build(cfg, seed, threads)
    if reference_available():
        ref = Reference()
        ref.attach(model, cfg)
        run = lambda e, xt, dst, wt: ref.expert_apply(0, e, xt, dst, wt)
        kind = "reference"
    else:
        run = lambda e, xt, dst, wt: o.expert_apply(model, 0, e, xt, dst, wt)
        kind = "port"
    dst = np.zeros(D, np.float32)
    T = x.shape[0]
    run(int(sel[0, 0]), x[0], dst, 1.0)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        t, k = divmod(n % (T * K), K)
        run(int(sel[t, k]), x[t], dst, float(w[t, k]))
        n += 1
    dt = time.perf_counter() - t0
    o.model_free(model)
    flops = 2.0 * (INTER * D + D * HALF)
    return {"value": round(n * flops / dt / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": kind,
            "pairs_per_s": round(n / dt, 1),
            "sample": f"{n} (token, expert) pairs of the config-3 routing through expert_apply, "
                      f"{dt:.1f} s, OpenMP {threads} threads"}


def run_prefill(args):
    """T=2048 tokens through one GPT-OSS-20B MoE layer as
    expert-grouped INT4 GEMMs on the matrix cores (8192 pairs, Zipf 1.1
    routing): f16 activation pairs on v_mfma_f32_32x32x16_f16 (default) or
    int8 limbs (--grouped int8). value = algorithmic TFLOP/s
    (2 x pairs x (5760x2880 + 2880x2880))."""
    import torch
    import picchio_amd as pa
    T = 2048
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=E, ctx_len=16, vocab=64)
    eng = pa.Engine(cfg)
    eng.build_synthetic(args.seed, what=1)
    f16 = args.grouped == "f16"
    eng.set_grouped_f16(f16)
    sel, w, counts = zipf_routing(T, E, K, args.seed)
    x = np.random.default_rng(args.seed + 7).standard_normal((T, D)).astype(np.float32)
    xd, sd, wd = eng.to_dev(x), eng.to_dev(sel), eng.to_dev(w)
    out = eng.empty((T, D), torch.float32)
    for _ in range(max(args.warmup, 1)):
        eng.moe_forward_grouped(0, xd, out, sd, wd)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(eng.stream)
    for _ in range(args.steps):
        eng.moe_forward_grouped(0, xd, out, sd, wd)
    ev1.record(eng.stream)
    ev1.synchronize()
    ms = ev0.elapsed_time(ev1) / args.steps
    eng.profile(True)
    for _ in range(5):
        eng.moe_forward_grouped(0, xd, out, sd, wd)
    gu_ms, gu_n = eng.profile_read(pa.PROF_EXPERT_GATE_UP)
    dn_ms, dn_n = eng.profile_read(pa.PROF_EXPERT_DOWN)
    eng.profile(False)
    gu_ms, dn_ms = gu_ms / gu_n, dn_ms / dn_n
    eng.close()
    P = T * K
    flops = 2.0 * P * (INTER * D + D * HALF)
    gu_flops = 2.0 * P * INTER * D
    tiles = int(sum((c + 31) // 32 for c in counts))
    cpu = None
    if not args.no_cpu:
        cpu = cpu_pairs_baseline(args.seed, args.cpu_seconds, x, sel, w)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)
    tfs = flops / (ms * 1e-3) / 1e12
    # MFMA work issued: every 32-pair half tile runs whole (f16: 2 halves per
    # activation, 64-pair tiles whose empty second half is skipped; int8: 3
    # limbs, 32-pair tiles)
    limbs, peak = (2, 2500.0) if f16 else (3, 5000.0)
    kern = "k_moe_f16<SWIGLU>" if f16 else "k_moe_mfma<SWIGLU>"
    line = {
        "metric": METRIC, "value": round(tfs, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16x2 (int4 weights, fp32 sums)" if f16 else "int8x3 (int4 weights)",
        "data": "synthetic",
        "config": {"workload": "config3: prefill MoE layer, T=2048 tokens, 8192 (token, expert) pairs "
                               "over 32 INT4 gs64 experts (Zipf 1.1, 16..512 per expert), expert-grouped "
                               + ("f16 MFMA GEMMs (2 activation halves)" if f16 else
                                  "int8 MFMA GEMMs (3 activation limbs)"),
                   "tokens": T, "pairs": P, "half_tiles_of_32": tiles,
                   "pairs_per_expert": [int(c) for c in counts],
                   "flops": flops, "gate_up_ms": round(gu_ms, 4), "down_ms": round(dn_ms, 4),
                   ("f16" if f16 else "int8") + "_mfma_flops_issued": limbs * 2 * tiles * 32 * (INTER * D + D * HALF)},
        "roofline": {"bound": "mfma", "achieved": round(gu_flops / (gu_ms * 1e-3) / 1e12, 1),
                     "peak": peak, "unit": "TFLOP/s",
                     "frac": round(gu_flops / (gu_ms * 1e-3) / 1e12 / peak, 4), "traffic": None,
                     "kernel": kern + " (gate_up, algorithmic flops vs the dense " +
                               ("fp16" if f16 else "int8") + " peak)",
                     "flops_per_launch": gu_flops, "mean_us": round(gu_ms * 1e3, 2)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


def measure_moe_layer(args):
    """the batch-1 MoE layer over fresh seeded tokens."""
    import torch
    import picchio_amd as pa

    L = args.layers
    cfg = pa.gptoss_cfg(n_layers=L, n_experts=E, ctx_len=16, vocab=64)
    eng = pa.Engine(cfg)
    if args.dot >= 0:
        eng.set_i4_dot(args.dot == 1)
    t0 = time.perf_counter()
    eng.build_synthetic(args.seed, what=1)
    build_s = time.perf_counter() - t0
    print(f"[bench] store built: {L} layers x {E} experts, {eng.device_bytes() / 1e9:.2f} GB in "
          f"{build_s:.1f} s", file=sys.stderr, flush=True)

    W, S = args.warmup, args.steps
    n_tok = W + S
    x = token_inputs(n_tok, 1000 + args.seed)
    xd = eng.to_dev(x)
    od = eng.empty((n_tok, D), torch.float32)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)

    # timed region: S tokens, three launches each, replayed from one graph
    def enqueue(t):
        eng.moe_forward(t % L, xd[t], od[t])
    eng.capture_begin()
    for t in range(W):
        enqueue(t)
    g_warm = eng.capture_end()
    eng.capture_begin()
    for t in range(W, n_tok):
        enqueue(t)
    g_run = eng.capture_end()
    eng.graph_launch(g_warm)
    eng.sync()
    torch.cuda.synchronize()
    ev0.record(eng.stream)
    eng.graph_launch(g_run)
    ev1.record(eng.stream)
    ev1.synchronize()
    ms = ev0.elapsed_time(ev1)
    eng.graph_destroy(g_warm)
    eng.graph_destroy(g_run)

    # the router launch alone over the same tokens, replayed the same way:
    # the expert launch's duration is the difference of the two graphs
    lg = eng.empty(E, torch.float32)
    eng.capture_begin()
    for t in range(W, n_tok):
        eng.router_logits(t % L, xd[t], lg)
    g_router = eng.capture_end()
    eng.graph_launch(g_router)
    eng.sync()
    ev0.record(eng.stream)
    eng.graph_launch(g_router)
    ev1.record(eng.stream)
    ev1.synchronize()
    ms_router = ev0.elapsed_time(ev1)
    eng.graph_destroy(g_router)

    # the launches of an eager pass with HIP events on the engine stream around
    # each (tells the one-launch experts from the two-launch ones; the eager
    # events add the dispatch to each launch, so the graph difference above is
    # the expert launch's duration)
    n_prof = max(min(args.profile_tokens, S), 1)
    eng.profile(True)
    for t in range(W, W + n_prof):
        enqueue(t)
    kern, eager = {}, {}
    for name, kind in (("router", pa.PROF_ROUTER), ("moe_ffn", pa.PROF_MOE_FFN),
                       ("gate_up", pa.PROF_EXPERT_GATE_UP), ("down_combine", pa.PROF_EXPERT_DOWN)):
        tot, cnt = eng.profile_read(kind)
        if cnt:
            eager[name] = tot / cnt
    eng.profile(False)
    fused = "moe_ffn" in eager
    if fused:
        kern = {"router": ms_router / S, "moe_ffn": (ms - ms_router) / S}
    else:
        kern = dict(eager)
    # streaming shape: all 32 experts of a layer copy in one gate_up launch
    act = eng.empty((E, HALF), torch.float32)
    all_e = eng.to_dev(np.arange(E, dtype=np.int32))
    st_ms = replay_ms(eng, ev0, ev1, L, lambda t: eng.expert_gate_up(t, all_e, xd[t], act))
    dot_on = args.dot == 1 or (args.dot < 0 and os.environ.get("PK_I4_DOT", "0") not in ("", "0"))
    arith = "integer-dot" if dot_on else "fp32 chains (bit-exact with quant.h)"
    eng.close()

    ms_tok = ms / S
    gbps = TOKEN_BYTES / (ms_tok * 1e-3) / 1e9
    if fused:
        # the dominant kernel: all routed experts of the token in one launch
        dom, dom_bytes = "moe_ffn", gate_up_bytes(K) + down_bytes(K)
        dom_name = ("k_moe_ffn (gate_up + bias + SwiGLU, then down + bias + routing-weighted combine, "
                    "the token's 4 routed experts selected in the launch)")
        traffic = MOE_FFN_TRAFFIC
    else:
        dom, dom_bytes = "gate_up", gate_up_bytes(K)
        dom_name = ("k_i4_gemv<SWIGLU> (gate_up + bias + SwiGLU, the layer's 4 routed experts "
                    "per launch, top-4 selected in the launch)")
        traffic = GATE_UP_TRAFFIC
    achieved = dom_bytes / (kern[dom] * 1e-3) / 1e9
    print(f"[bench] config 1: {S} tokens in {ms:.2f} ms: {ms_tok * 1e3:.2f} us/token, {gbps:.1f} GB/s; "
          f"kernels (us) " + ", ".join(f"{k} {v * 1e3:.2f}" for k, v in kern.items()) +
          f"; {dom} {achieved:.1f} GB/s ({arith})", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(x[:4000], args.seed, args.cpu_seconds)
        cpu.update(host_info())
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)
    return {
        "metric": METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": S,
        "warmup": W,
        "ms_per_step": round(ms_tok, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "config1: GPT-OSS-20B MoE layer, batch-1 decode, top-4 of 32 "
                               "INT4 gs64 experts, fresh seeded tokens",
                   "layer_copies": L, "experts": E, "topk": K, "hidden": D, "weights": "int4-gs64",
                   "expert_arithmetic": arith, "experts_one_launch": fused,
                   "bytes_per_token": TOKEN_BYTES, "tokens_per_s": round(1e3 / ms_tok, 1),
                   "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4), "chained": True,
                   "kernel_us": {k: round(v * 1e3, 3) for k, v in kern.items()},
                   "kernel_us_method": ("graph replays: router launches alone, and router + expert "
                                        "launches; the expert launch = the difference" if fused else
                                        "HIP events around each launch of an eager pass"),
                   "gate_up_32_experts_gbps": round(gate_up_bytes(E) / (st_ms * 1e-3) / 1e9, 1),
                   "gate_up_32_experts_hbm_frac": round(gate_up_bytes(E) / (st_ms * 1e-3) / 1e9
                                                        / HBM_PEAK_GBPS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": dom_name, "bytes_per_launch": dom_bytes, "mean_us": round(kern[dom] * 1e3, 3)},
        "cpu_baseline": cpu,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000, help="timed tokens (config 1) or decode steps")
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--layers", type=int, default=24, help="distinct MoE layer copies (config 1)")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile-tokens", type=int, default=400)
    ap.add_argument("--dot", type=int, default=-1,
                    help="config 1 expert arithmetic: 1 integer dot, 0 fp32 chains, -1 the engine's default")
    ap.add_argument("--grouped", choices=["f16", "int8"], default="f16",
                    help="config 3 arithmetic: f16 hi/lo activation pairs (default) or exact int8 limbs")
    ap.add_argument("--decode-steps", type=int, default=128,
                    help="default run: decode steps of configs 2 and 4")
    ap.add_argument("--sample", default="",
                    help="decode mode: draw tokens on the device with T,top_p,top_k,rep "
                         "(e.g. 1.0,0.95,50,1.1, picchio's defaults) instead of greedy")
    ap.add_argument("--mode", choices=["all", "kernels", "decode", "prefill", "decode120b"], default="all",
                    help="all (default): config 1 headline with configs 2 and 4 under config; "
                         "kernels: config 1 only; decode: config 2 (use --steps 256); prefill: "
                         "config 3, grouped MFMA MoE (--steps 20); decode120b: config 4 (--steps 128)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the expert path is built and timed on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured configuration).", file=sys.stderr)
        sys.exit(2)
    if args.mode == "decode":
        print(json.dumps(measure_decode20b(args, args.steps, args.warmup, not args.no_cpu)))
        return
    if args.mode == "prefill":
        run_prefill(args)
        return
    if args.mode == "decode120b":
        print(json.dumps(measure_decode120b(args, args.steps, args.warmup, not args.no_cpu)))
        return
    line = measure_moe_layer(args)
    if args.mode == "all":
        # configs 2 and 4 in the same run: decode tok/s of both model shapes
        # (the 120B CPU baseline is left out: its model build on the host
        # takes minutes; --mode decode120b measures it)
        ds = args.decode_steps
        d20 = measure_decode20b(args, ds, 8, not args.no_cpu)
        d120 = measure_decode120b(args, ds, 4, False)
        line["config"]["decode_20b"] = {"tok_s": d20["value"], "ms_per_token": d20["ms_per_step"],
                                        "steps": ds, **{k: d20["config"][k] for k in
                                                        ("workload", "bytes_per_token", "hbm_gbps", "hbm_frac",
                                                         "prefill_tok_s", "attention_us_per_layer")},
                                        "lm_head_roofline": d20["roofline"], "cpu_baseline": d20["cpu_baseline"]}
        line["config"]["decode_120b"] = {"batch1_tok_s": d120["config"]["batch1_tok_s"],
                                         "steps": ds, **{k: d120["config"][k] for k in
                                                         ("workload", "batch1_bytes_per_token", "batch1_hbm_gbps",
                                                          "batch32_tok_s", "batch32_ms_per_step",
                                                          "batch32_hbm_gbps")},
                                         "lm_head_roofline": d120["roofline"],
                                         "cpu_baseline": "not run by default (host model build takes minutes): "
                                                         "bench.py --mode decode120b"}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
