#!/usr/bin/env python3
"""Benchmark of the INT4 expert path on one MI355X.

Default run (no --mode): every BASELINE config in one process. Config 1 is
the headline `value`; configs 0, 2, 3 and 4 are reported under `config`,
each with its own roofline and same-run CPU baseline.

Config 1: one GPT-OSS-20B-shaped MoE layer at
batch-1 decode -- RMSNorm'd fp32 x [2880], fp32 router [32x2880] + bias,
top-4 of 32 INT4 gs64 experts (gate_up 5760x2880, down 2880x2880, biases),
clamped SwiGLU, softmax-weighted combine. A "step" is the config's 1000
fresh seeded tokens through that layer one after another (each token: the
router launch, then the experts launch), replayed from a HIP graph. Token t
uses layer copy t % L (L = 24, the 20B model's MoE layers, 10.8 GB of
experts) so the expert bytes come from HBM, not from the 256 MB MALL.

Expert arithmetic (configs 1, 2 and 4 at batch 1): by default the integer
dot -- the input as exact base-16 digit records, exact int32 group sums, the
fp32 scale fold; per layer within 2e-5 of picchio's fp32 chains and the same
256-step greedy stream -- with picchio's fp32 chains (bit-identical to
quant.h) timed beside it under "other_arithmetic"; --dot 0 swaps them.

value = algorithmic HBM bytes per token (experts + router + x/out) x tokens/s
(the integer dot reads the same weight bytes; its input and output records
differ from the fp32 rows by under 0.01 % of them).
roofline = the dominant kernel (the experts launch): its algorithmic bytes per
launch / its mean duration (graph replays with HIP events on the engine
stream: router + experts, minus the router launches alone).
cpu_baseline = picchio's MoE layer on the host cores (oracle/_ref build of
the reference when present, else the C restatement).
"""
import os

# picchio's CPU baseline runs under OpenMP with threads bound to cores (the
# conditions its published CPU figures were taken under); set before any
# OpenMP runtime starts
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")

import argparse
import json
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
FFN_BYTES = EXPERT_BYTES + 2 * D * 4               # config 0: one expert, x in, y out: 14,054,400
TOKENS_PER_STEP = 1000                              # config 1: "time 1000 fresh seeded tokens"

# HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE, then
# WRITE_SIZE, in passes of their own), scaled by what the two counters read
# for a 1 GiB device copy in the same call (x 2.000 and x 1.000):
#  * k_moe_ffn (the default, profiles/k_moe_ffn_moe_config1.txt), measured on
#    commit afc7a2d: FETCH_SIZE 27791.47 KiB x 2 + WRITE_SIZE 168.84 KiB;
#  * k_i4_gemv<SWIGLU> gate_up of the two-launch experts
#    (pk_set_moe_fused(e, 0)), measured on commit 0a0ca63: FETCH_SIZE
#    18425.54 KiB x 2 + WRITE_SIZE 45.04 KiB;
#  * k_i4_gemv_stream<SWIGLU, integer dot>, 32 experts' gate_up
#    (profiles/k_i4_gemv_stream_gate_up32.txt), commit afc7a2d: FETCH_SIZE
#    149022.55 KiB x 2 + WRITE_SIZE 630.00 KiB;
#  * measured again on commit 85f4c9b (passes over --mode decode and
#    --mode kernels): k_moe_ffn FETCH_SIZE 27790.06 KiB x 2 + WRITE_SIZE
#    168.84 KiB = 57,085,388 B (the constant above within 0.01 %);
#    k_lm_head<fp32> FETCH_SIZE 1131188.06 KiB x 2 + WRITE_SIZE 2358.62 KiB;
#    config 0's expert FFN, k_i4_gemv<SWIGLU> FETCH_SIZE 4726.50 KiB x 2 +
#    WRITE_SIZE 11.25 KiB, then k_i4_gemv<PLAIN> 2433.75 KiB x 2 + 11.25 KiB;
#  * k_moe_f16<SWIGLU>, config 3's gate_up
#    (profiles/k_moe_f16_prefill_config3.txt, commit 73774fc): FETCH_SIZE
#    369465.17 KiB x 2 + WRITE_SIZE 92160.00 KiB.
#  * k_moe_ffn<integer dot>, config 1's default (passes over --mode kernels,
#    profiles/k_moe_ffn_moe_config1.txt): FETCH_SIZE 27700.78 KiB x 2 +
#    WRITE_SIZE 146.34 KiB.
MOE_FFN_TRAFFIC = 57088267
MOE_FFN_DOT_TRAFFIC = 56879493
GATE_UP_TRAFFIC = 37780589
STREAM_DOT_TRAFFIC = 305834925
LM_HEAD_TRAFFIC = 2319025051
FFN_TRAFFIC = 9691127 + 4995704
F16_GATE_UP_TRAFFIC = 851036516


# the batch-1 expert arithmetic of a run: --dot 1 (and the default) the
# integer dot -- inputs as exact base-16 digit records, exact int32 group sums,
# within 2e-5 of picchio's fp32 per layer and the same 256-step greedy stream;
# --dot 0 picchio's fp32 chains, bit-identical to quant.h. The default run
# times the other one beside the headline.
ARITH = {True: "integer-dot (exact int32 group sums)", False: "fp32 chains (bit-exact with quant.h)"}


def run_dot(args):
    return args.dot != 0


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


# read before any OpenMP runtime binds this thread to one core
HOST = host_info()


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


def cpu_threads():
    return int(os.environ.get("OMP_NUM_THREADS", "0")) or HOST["threads_available"]


def timed_loop(fn, budget_s):
    """fn(i) for i = 0, 1, ... until budget_s seconds have passed (after one
    untimed call that pages the model in); returns (calls, seconds)."""
    fn(0)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        fn(n)
        n += 1
    return n, time.perf_counter() - t0


def cpu_moe_baselines(x1, x0, seed, budget1_s, budget0_s):
    """picchio on the host cores, on one 20B-shaped MoE layer (32 experts
    resident in RAM, the same seeded weights as the GPU store's layer 0):
    moe_forward over config 1's tokens (time-bounded sample), and
    expert_apply over config 0's inputs, one expert after another."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_ffi import Oracle, Reference, reference_available, make_cfg
    o = Oracle()
    threads = cpu_threads()
    cfg = make_cfg(n_layers=1, n_experts=E, ctx_len=16, vocab=64)
    model = o.model_build(cfg, seed, threads)
    kind = "port"
    if reference_available():
        ref = Reference()
        ref.attach(model, cfg)
        moe = lambda xt, out: ref.moe_forward(0, xt, out)
        ffn = lambda e, xt, dst: ref.expert_apply(0, e, xt, dst, 1.0)
        kind = "reference"
    else:
        sel = np.empty(K, np.int32)
        w = np.empty(K, np.float32)
        moe = lambda xt, out: o.moe_forward(model, 0, xt, out, sel, w, None)
        ffn = lambda e, xt, dst: o.expert_apply(model, 0, e, xt, dst, 1.0)
    out = np.empty(D, np.float32)
    n1, dt1 = timed_loop(lambda i: moe(x1[i % len(x1)], out), budget1_s)
    dst = np.zeros(D, np.float32)
    n0, dt0 = timed_loop(lambda i: ffn(i % E, x0[i % len(x0)], dst), budget0_s)
    o.model_free(model)
    c1 = {"value": round(n1 * TOKEN_BYTES / dt1 / 1e9, 3), "unit": "GB/s", "cores": threads,
          "kind": kind, "tokens_per_s": round(n1 / dt1, 2),
          "sample": f"{n1} tokens of the same MoE layer (1 layer, 32 experts resident in RAM), "
                    f"{dt1:.1f} s, OpenMP {threads} threads"}
    c0 = {"value": round(n0 * FFN_BYTES / dt0 / 1e9, 3), "unit": "GB/s", "cores": threads,
          "kind": kind, "us_per_ffn": round(dt0 / n0 * 1e6, 1),
          "sample": f"{n0} expert_apply calls (the 32 experts of one layer in turn), {dt0:.1f} s, "
                    f"OpenMP {threads} threads"}
    return c1, c0


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


def cpu_decode_baseline(cfg, seed, budget_s, prompt, pos0):
    """picchio's forward_token on the host cores for the same model (same
    seeded weights), time-bounded, at positions pos0, pos0 + 1, ... like the
    GPU's decode steps. The KV rows below pos0 stay zero: the attention loops
    do the same work whatever the rows hold."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_ffi import Oracle, Reference, reference_available
    o = Oracle()
    threads = cpu_threads()
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
    n, dt = timed_loop(lambda i: step(int(prompt[i % len(prompt)]), pos0 + i), budget_s)
    o.model_free(model)
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": threads, "kind": kind,
            "sample": f"{n} forward_token steps at positions {pos0}..{pos0 + n} of the same "
                      f"{cfg.n_layers}-layer model ({cfg.n_experts} experts per layer resident in RAM, "
                      f"fp32 lm_head), {dt:.1f} s, OpenMP {threads} threads; model build {build_s:.0f} s"}


def cpu_decode120_baseline(seed, budget_s, prompt, pos0):
    """picchio's forward_token for the 120B shape, from a host model that
    fits the run: every layer at full width (128 experts, the same seeded
    weights as the GPU model's layers 0 and 1) but two layers deep (one
    sliding-window, one full-context layer, as the 36 alternate) and a
    64-entry vocabulary; the 201,088 x 2880 fp32 lm_head GEMV (matmul_f32,
    picchio.c:1744) is timed on its own. Per token at 36 layers:
    18 x t(two layers) + t(lm_head)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_ffi import Oracle, Reference, reference_available, make_cfg
    o = Oracle()
    threads = cpu_threads()
    cfg = make_cfg(n_layers=2, n_experts=128, ctx_len=pos0 + 4096, vocab=64)
    t0 = time.perf_counter()
    model = o.model_build(cfg, seed, threads)
    build_s = time.perf_counter() - t0
    V = 201088
    y = np.empty(V, np.float32)
    xl = np.random.default_rng(seed).standard_normal(D).astype(np.float32)
    # the GEMV's work does not depend on the weight values: a constant matrix
    W = np.full((V, D), 0.01, np.float32)
    if reference_available():
        ref = Reference()
        ref.attach(model, cfg)
        ref.reset_kv()
        step = lambda tok, pos: ref.forward_token(tok, pos)
        lm = lambda: ref.matmul_f32(y, xl, W, 1, D, V)
        kind = "reference"
    else:
        step = lambda tok, pos: o.forward_token(model, tok, pos, None)
        lm = lambda: o.matmul_f32(y, xl, W, 1, D, V)
        kind = "port"
    n2, dt2 = timed_loop(lambda i: step(int(prompt[i % len(prompt)]) % 64, pos0 + i), budget_s)
    nl, dtl = timed_loop(lambda i: lm(), budget_s / 3)
    o.model_free(model)
    del W
    t2, tl = dt2 / n2, dtl / nl
    t36 = 18 * t2 + tl
    return {"value": round(1.0 / t36, 3), "unit": "tok/s", "cores": threads, "kind": kind,
            "ms_per_token_36_layers": round(t36 * 1e3, 1),
            "ms_two_layers": round(t2 * 1e3, 2), "ms_lm_head": round(tl * 1e3, 2),
            "batch32_tok_s": round(1.0 / t36, 3),
            "sample": f"{n2} forward_token steps at positions {pos0}..{pos0 + n2} of a two-layer "
                      f"120B-width model (128 experts per layer resident in RAM, KV rows below {pos0} "
                      f"zero) in {dt2:.1f} s, and {nl} fp32 lm_head GEMVs (201088 x 2880) in "
                      f"{dtl:.1f} s; 36 layers = 18 x two layers + lm_head; OpenMP {threads} threads; "
                      f"model build {build_s:.0f} s; picchio decodes one sequence at a time, so its "
                      f"batch-32 rate is its batch-1 rate"}


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
    main_dot = run_dot(args)
    eng.set_i4_dot(main_dot)
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
    # the same steps on the other expert arithmetic: rate and whether the
    # greedy stream is the same
    alt = None
    if not sampling and args.dot < 0:
        eng.set_i4_dot(not main_dot)
        eng.decode_replay(nxt, n_prompt, max(warmup, 1))
        ev0.record(eng.stream)
        toks_alt = eng.decode_replay(nxt, n_prompt, steps)
        ev1.record(eng.stream)
        ev1.synchronize()
        alt = {"expert_arithmetic": ARITH[not main_dot],
               "tok_s": round(steps / (ev0.elapsed_time(ev1) * 1e-3), 2),
               "same_stream": bool(list(toks_alt) == list(toks))}
        eng.set_i4_dot(main_dot)
    eng.close()
    tok_s = steps / (ms * 1e-3)
    bpt = sum(decode_bytes_per_token(cfg, n_prompt + i) for i in range(steps)) / steps
    lm_bytes = cfg.vocab * cfg.hidden * 4 + cfg.hidden * 4 + cfg.vocab * 4
    cpu = None
    if cpu_on:
        cpu = cpu_decode_baseline(cfg, args.seed, args.cpu_seconds, prompt, n_prompt)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)
    print(f"[bench] config 2: {tok_s:.1f} tok/s ({ms / steps * 1e3:.1f} us/token), prefill "
          f"{prefill_s:.3f} s; experts on the {ARITH[main_dot]}; other arithmetic {alt}", file=sys.stderr,
          flush=True)
    line = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms / steps, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "config2: GPT-OSS-20B-shaped " + ("sampled" if sampling else "greedy") +
                               f" decode, batch 1, 512-token random-id prompt then {steps} steps, all "
                               "experts HBM-resident",
                   "sampling": ({"temperature": sampling[0], "top_p": sampling[1], "top_k": sampling[2],
                                 "rep_penalty": sampling[3], "seed": args.seed} if sampling else "greedy"),
                   "layers": cfg.n_layers, "experts": cfg.n_experts, "vocab": cfg.vocab,
                   "lm_head": "fp32", "bytes_per_token": int(bpt),
                   "hbm_gbps": round(bpt * tok_s / 1e9, 1),
                   "hbm_frac": round(bpt * tok_s / 1e9 / HBM_PEAK_GBPS, 4),
                   "prefill_s": round(prefill_s, 3), "prefill_tok_s": round(n_prompt / prefill_s, 1),
                   "attention_us_per_layer": round(att_ms / max(att_n, 1) * 1e3, 2),
                   "expert_arithmetic": ARITH[main_dot], "other_arithmetic": alt,
                   "first_tokens": [int(nxt)] + [int(t) for t in toks[:8]]},
        "roofline": {"bound": "hbm", "achieved": round(lm_bytes / (lm_ms * 1e-3) / 1e9, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(lm_bytes / (lm_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                     "traffic": LM_HEAD_TRAFFIC, "kernel": "k_lm_head<fp32> (201088 x 2880 GEMV, per-block maxima)",
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
    main_dot = run_dot(args)
    eng.set_i4_dot(main_dot)
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
    # batch 1 on the other expert arithmetic (the same state: the KV rows the
    # steps above wrote are rewritten by the same positions' steps)
    alt1 = None
    if args.dot < 0:
        eng.set_i4_dot(not main_dot)
        eng.decode_replay(tok, ctx, max(warmup, 1))
        ev0.record(eng.stream)
        toks_alt = eng.decode_replay(tok, ctx, steps)
        ev1.record(eng.stream)
        ev1.synchronize()
        diff = [i for i, (a, b) in enumerate(zip(toks_alt, toks1)) if int(a) != int(b)]
        alt1 = {"expert_arithmetic": ARITH[not main_dot],
                "tok_s": round(steps / (ev0.elapsed_time(ev1) * 1e-3), 2),
                "same_stream": not diff, "first_departure_step": diff[0] if diff else None,
                "note": "the two arithmetics differ by at most 2e-5 relative per layer; over 36 layers of "
                        "synthetic weights a routing or top-2 near-tie can separate their greedy streams "
                        "(tests/test_gpu_configs.py traces each departure from the oracle's stream to one)"}
        eng.set_i4_dot(main_dot)
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
        cpu = cpu_decode120_baseline(args.seed, args.cpu_seconds, first, ctx)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)
    print(f"[bench] config 4: batch 1 {tok1:.1f} tok/s ({ARITH[main_dot]}; other arithmetic {alt1}), "
          f"batch 32 {tok32:.1f} tok/s", file=sys.stderr, flush=True)
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
                   "batch1_expert_arithmetic": ARITH[main_dot], "batch1_other_arithmetic": alt1,
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
                     "frac": round(lm_bytes / (lm_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "traffic": LM_HEAD_TRAFFIC,
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


def measure_prefill(args, steps, warmup, cpu_on):
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
    for _ in range(max(warmup, 1)):
        eng.moe_forward_grouped(0, xd, out, sd, wd)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(eng.stream)
    for _ in range(steps):
        eng.moe_forward_grouped(0, xd, out, sd, wd)
    ev1.record(eng.stream)
    ev1.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
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
    if cpu_on:
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
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 5),
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
                     "frac": round(gu_flops / (gu_ms * 1e-3) / 1e12 / peak, 4),
                     "traffic": F16_GATE_UP_TRAFFIC if f16 else None,
                     "kernel": kern + " (gate_up, algorithmic flops vs the dense " +
                               ("fp16" if f16 else "int8") + " peak)",
                     "flops_per_launch": gu_flops, "mean_us": round(gu_ms * 1e3, 2)},
        "cpu_baseline": cpu,
    }
    print(f"[bench] config 3: {ms:.3f} ms per layer, {tfs:.1f} TFLOP/s; gate_up {gu_ms * 1e3:.1f} us, "
          f"down {dn_ms * 1e3:.1f} us", file=sys.stderr, flush=True)
    return line


def capture(eng, lo, hi, enqueue):
    """One executable graph of enqueue(t) for t in lo..hi-1."""
    eng.capture_begin()
    for t in range(lo, hi):
        enqueue(t)
    return eng.capture_end()


def measure_moe_layer(args):
    """the batch-1 MoE layer over fresh seeded tokens, each
    step 1000 of them; and, on the same expert store, config 0: one expert's
    FFN at a time over every distinct expert of the store."""
    import torch
    import picchio_amd as pa

    L = args.layers
    cfg = pa.gptoss_cfg(n_layers=L, n_experts=E, ctx_len=16, vocab=64)
    eng = pa.Engine(cfg)
    dot_on = run_dot(args)
    eng.set_i4_dot(dot_on)
    t0 = time.perf_counter()
    eng.build_synthetic(args.seed, what=1)
    build_s = time.perf_counter() - t0
    print(f"[bench] store built: {L} layers x {E} experts, {eng.device_bytes() / 1e9:.2f} GB in "
          f"{build_s:.1f} s", file=sys.stderr, flush=True)

    W, S, T = args.warmup, args.steps, TOKENS_PER_STEP
    n_tok = (W + S) * T
    x = token_inputs(n_tok, 1000 + args.seed)
    xd = eng.to_dev(x)
    od = eng.empty((n_tok, D), torch.float32)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)

    # timed region: S steps of T tokens, each token the router launch and the
    # experts launch; one graph per step, the steps' graphs replayed back to back
    def enqueue(t):
        eng.moe_forward(t % L, xd[t], od[t])
    graphs = [capture(eng, s * T, (s + 1) * T, enqueue) for s in range(W + S)]
    for g in graphs[:W]:
        eng.graph_launch(g)
    eng.sync()
    torch.cuda.synchronize()
    ev0.record(eng.stream)
    for g in graphs[W:]:
        eng.graph_launch(g)
    ev1.record(eng.stream)
    ev1.synchronize()
    ms = ev0.elapsed_time(ev1)
    for g in graphs:
        eng.graph_destroy(g)

    # the router launch alone over the same tokens, replayed the same way:
    # the experts launch's duration is the difference of the two
    lg = eng.empty(E, torch.float32)
    graphs = [capture(eng, s * T, (s + 1) * T, lambda t: eng.router_logits(t % L, xd[t], lg))
              for s in range(W, W + S)]
    eng.graph_launch(graphs[0])
    eng.sync()
    ev0.record(eng.stream)
    for g in graphs:
        eng.graph_launch(g)
    ev1.record(eng.stream)
    ev1.synchronize()
    ms_router = ev0.elapsed_time(ev1)
    for g in graphs:
        eng.graph_destroy(g)

    # the same tokens on the other expert arithmetic, timed the same way over
    # fewer steps (default run)
    alt = None
    if args.dot < 0:
        eng.set_i4_dot(not dot_on)
        S2 = min(S, 5)

        def replay(steps, fn):
            gs = [capture(eng, s * T, (s + 1) * T, fn) for s in steps]
            eng.graph_launch(gs[0])
            eng.sync()
            ev0.record(eng.stream)
            for g in gs:
                eng.graph_launch(g)
            ev1.record(eng.stream)
            ev1.synchronize()
            for g in gs:
                eng.graph_destroy(g)
            return ev0.elapsed_time(ev1)
        steps2 = range(W, W + S2)
        ms2 = replay(steps2, enqueue)
        ms2_router = replay(steps2, lambda t: eng.router_logits(t % L, xd[t], lg))
        eng.set_i4_dot(dot_on)
        n2 = S2 * T
        moe2 = (ms2 - ms2_router) / n2
        alt = {"expert_arithmetic": ARITH[not dot_on], "tokens_timed": n2,
               "us_per_token": round(ms2 / n2 * 1e3, 3),
               "gbps": round(TOKEN_BYTES / (ms2 / n2 * 1e-3) / 1e9, 1),
               "kernel_us": {"router": round(ms2_router / n2 * 1e3, 3), "moe_ffn": round(moe2 * 1e3, 3)},
               "moe_ffn_gbps": round((gate_up_bytes(K) + down_bytes(K)) / (moe2 * 1e-3) / 1e9, 1)}
        print(f"[bench] config 1 on the {ARITH[not dot_on]}: {alt['us_per_token']:.2f} us/token, "
              f"{alt['gbps']:.1f} GB/s; "
              f"moe_ffn {alt['kernel_us']['moe_ffn']:.2f} us = {alt['moe_ffn_gbps']:.1f} GB/s", file=sys.stderr,
              flush=True)

    # the launches of an eager pass with HIP events on the engine stream around
    # each (tells the one-launch experts from the two-launch ones; the eager
    # events add the dispatch to each launch, so the graph difference above is
    # the experts launch's duration)
    n_prof = max(min(args.profile_tokens, S * T), 1)
    eng.profile(True)
    for t in range(W * T, W * T + n_prof):
        enqueue(t)
    eager = {}
    for name, kind in (("router", pa.PROF_ROUTER), ("moe_ffn", pa.PROF_MOE_FFN),
                       ("gate_up", pa.PROF_EXPERT_GATE_UP), ("down_combine", pa.PROF_EXPERT_DOWN)):
        tot, cnt = eng.profile_read(kind)
        if cnt:
            eager[name] = tot / cnt
    eng.profile(False)
    n_timed = S * T
    fused = "moe_ffn" in eager
    if fused:
        kern = {"router": ms_router / n_timed, "moe_ffn": (ms - ms_router) / n_timed}
    else:
        kern = dict(eager)
    # streaming shape: all 32 experts of a layer copy in one gate_up launch,
    # on picchio's fp32 chains and on the integer dot (input records made
    # once per token, outside the timed launches: the GEMV's input format)
    act = eng.empty((E, HALF), torch.float32)
    all_e = eng.to_dev(np.arange(E, dtype=np.int32))
    st_ms = replay_ms(eng, ev0, ev1, L, lambda t: eng.expert_gate_up(t, all_e, xd[t], act), reps=5)
    rec = eng.empty((L, (D // 32) * 24), torch.int32)
    for t in range(L):
        eng.act_records(xd[t], rec[t])
    arec = eng.empty((E, (INTER // 64) * 24), torch.int32)
    st_dot_ms = replay_ms(eng, ev0, ev1, L, lambda t: eng.expert_gate_up_dot(t, all_e, rec[t], act, arec), reps=5)

    # config 0: one expert FFN after another (gate_up + bias + SwiGLU, then
    # down + bias), FFN i on expert (i // L) % E of layer copy i % L: all
    # L x E distinct experts (10.8 GB) before any repeats; x ~ N(0,1)
    n_ffn = L * E
    x0 = np.random.default_rng(2000 + args.seed).standard_normal((n_ffn, D)).astype(np.float32)
    x0d = eng.to_dev(x0)
    act0 = eng.empty(HALF, torch.float32)
    y0 = eng.empty((n_ffn, D), torch.float32)
    eid = lambda i: all_e[(i // L) % E:(i // L) % E + 1]

    def ffn(i):
        eng.expert_gate_up(i % L, eid(i), x0d[i], act0)
        eng.expert_down(i % L, eid(i), act0, y0[i])
    ffn_ms = replay_ms(eng, ev0, ev1, n_ffn, ffn)
    ffn_gu_ms = replay_ms(eng, ev0, ev1, n_ffn, lambda i: eng.expert_gate_up(i % L, eid(i), x0d[i], act0))

    arith = ARITH[dot_on]
    eng.close()

    ms_tok = ms / n_timed
    gbps = TOKEN_BYTES / (ms_tok * 1e-3) / 1e9
    if fused:
        # the dominant kernel: all routed experts of the token in one launch
        dom, dom_bytes = "moe_ffn", gate_up_bytes(K) + down_bytes(K)
        dom_name = (f"k_moe_ffn<{'integer dot' if dot_on else 'fp32 chains'}> (gate_up + bias + SwiGLU, "
                    "then down + bias + routing-weighted combine, "
                    "the token's 4 routed experts selected in the launch)")
        traffic = MOE_FFN_DOT_TRAFFIC if dot_on else MOE_FFN_TRAFFIC
    else:
        dom, dom_bytes = "gate_up", gate_up_bytes(K)
        dom_name = ("k_i4_gemv<SWIGLU> (gate_up + bias + SwiGLU, the layer's 4 routed experts "
                    "per launch, top-4 selected in the launch)")
        traffic = GATE_UP_TRAFFIC
    achieved = dom_bytes / (kern[dom] * 1e-3) / 1e9
    ffn_gbps = FFN_BYTES / (ffn_ms * 1e-3) / 1e9
    print(f"[bench] config 1: {n_timed} tokens in {ms:.2f} ms: {ms_tok * 1e3:.2f} us/token, {gbps:.1f} GB/s; "
          f"kernels (us) " + ", ".join(f"{k} {v * 1e3:.2f}" for k, v in kern.items()) +
          f"; {dom} {achieved:.1f} GB/s ({arith})", file=sys.stderr, flush=True)
    print(f"[bench] config 0: {ffn_ms * 1e3:.2f} us per expert FFN ({ffn_gu_ms * 1e3:.2f} gate_up), "
          f"{ffn_gbps:.1f} GB/s", file=sys.stderr, flush=True)
    cpu = cpu0 = None
    if not args.no_cpu:
        cpu, cpu0 = cpu_moe_baselines(x[:4000], x0, args.seed, args.cpu_seconds, args.cpu_seconds * 0.6)
        cpu.update(HOST)
        print(f"[bench] cpu baselines: config 1 {cpu}; config 0 {cpu0}", file=sys.stderr, flush=True)
    st_gbps = gate_up_bytes(E) / (st_ms * 1e-3) / 1e9
    st_dot_gbps = gate_up_bytes(E) / (st_dot_ms * 1e-3) / 1e9
    print(f"[bench] INT4 GEMV streaming (gate_up of 32 experts per launch): integer dot {st_dot_ms * 1e3:.2f} us "
          f"= {st_dot_gbps:.1f} GB/s; fp32 chains {st_ms * 1e3:.2f} us = {st_gbps:.1f} GB/s", file=sys.stderr,
          flush=True)
    streaming = {
        "workload": "INT4 gs64 expert GEMV at its streaming shape: gate_up + bias + SwiGLU of all 32 experts of "
                    "a layer in one launch (32 x 5760 x 2880, 299 MB), one input row, over the 24 layer copies "
                    "(graph replay)",
        "bytes_per_launch": gate_up_bytes(E),
        "roofline": {"bound": "hbm", "achieved": round(st_dot_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(st_dot_gbps / HBM_PEAK_GBPS, 4), "traffic": STREAM_DOT_TRAFFIC,
                     "kernel": "k_i4_gemv_stream<SWIGLU, integer dot> (one workgroup per CU-share of row "
                               "blocks, next row block in flight)",
                     "bytes_per_launch": gate_up_bytes(E), "mean_us": round(st_dot_ms * 1e3, 3)},
        "fp32_chains": {"achieved": round(st_gbps, 1), "frac": round(st_gbps / HBM_PEAK_GBPS, 4),
                        "mean_us": round(st_ms * 1e3, 3),
                        "kernel": "k_i4_gemv_stream<SWIGLU, fp32 chains> (bit-exact with quant.h)"},
    }
    config0 = {
        "workload": "config0: one GPT-OSS-20B-shaped expert FFN at batch 1 (gate_up 5760x2880 + bias, "
                    "clamped SwiGLU, down 2880x2880 + bias; INT4 gs64), x ~ N(0,1); FFNs one after another "
                    f"over all {n_ffn} distinct experts of the store (10.8 GB), replayed from a HIP graph",
        "us_per_ffn": round(ffn_ms * 1e3, 3), "bytes_per_ffn": FFN_BYTES,
        "gbps": round(ffn_gbps, 1), "hbm_frac": round(ffn_gbps / HBM_PEAK_GBPS, 4),
        "gate_up_us": round(ffn_gu_ms * 1e3, 3), "down_us": round((ffn_ms - ffn_gu_ms) * 1e3, 3),
        "roofline": {"bound": "hbm", "achieved": round(ffn_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(ffn_gbps / HBM_PEAK_GBPS, 4), "traffic": FFN_TRAFFIC,
                     "kernel": "k_i4_gemv<SWIGLU> (gate_up) then k_i4_gemv<PLAIN> (down), one expert, "
                               "fp32 chains (expert_apply's arithmetic, bit-exact with quant.h)",
                     "bytes_per_launch": FFN_BYTES, "mean_us": round(ffn_ms * 1e3, 3)},
        "cpu_baseline": cpu0,
    }
    return {
        "metric": METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": S,
        "warmup": W,
        "ms_per_step": round(ms / S, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32" if dot_on else "fp32",
        "data": "synthetic",
        "config": {"workload": "config1: GPT-OSS-20B MoE layer, batch-1 decode, top-4 of 32 "
                               f"INT4 gs64 experts; a step = {T} fresh seeded tokens one after another",
                   "tokens_per_step": T, "tokens_timed": n_timed,
                   "layer_copies": L, "experts": E, "topk": K, "hidden": D, "weights": "int4-gs64",
                   "expert_arithmetic": arith, "experts_one_launch": fused,
                   "bytes_per_token": TOKEN_BYTES, "us_per_token": round(ms_tok * 1e3, 3),
                   "tokens_per_s": round(1e3 / ms_tok, 1),
                   "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4), "chained": True,
                   "kernel_us": {k: round(v * 1e3, 3) for k, v in kern.items()},
                   "kernel_us_method": ("graph replays: router launches alone, and router + expert "
                                        "launches; the expert launch = the difference" if fused else
                                        "HIP events around each launch of an eager pass"),
                   "other_arithmetic": alt,
                   "int4_gemv_streaming": streaming,
                   "config0_expert_ffn": config0},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": dom_name, "bytes_per_launch": dom_bytes, "mean_us": round(kern[dom] * 1e3, 3)},
        "cpu_baseline": cpu,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20,
                    help="timed steps: config 1 steps of 1000 tokens (default run, kernels); decode or "
                         "prefill steps in the single-config modes")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=24, help="distinct MoE layer copies (configs 0 and 1)")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile-tokens", type=int, default=400)
    ap.add_argument("--dot", type=int, default=-1,
                    help="batch-1 expert arithmetic of configs 1, 2 and 4: 1 integer dot, 0 picchio's fp32 "
                         "chains; -1 (default) the integer dot, with the fp32 chains timed beside it")
    ap.add_argument("--grouped", choices=["f16", "int8"], default="f16",
                    help="config 3 arithmetic: f16 hi/lo activation pairs (default) or exact int8 limbs")
    ap.add_argument("--decode-steps", type=int, default=256,
                    help="default run: config 2's greedy decode steps (the config names 256)")
    ap.add_argument("--decode120-steps", type=int, default=128,
                    help="default run: config 4's decode steps (the config names 128)")
    ap.add_argument("--prefill-steps", type=int, default=10, help="default run: config 3's timed layers")
    ap.add_argument("--sample", default="",
                    help="decode mode: draw tokens on the device with T,top_p,top_k,rep "
                         "(e.g. 1.0,0.95,50,1.1, picchio's defaults) instead of greedy")
    ap.add_argument("--mode", choices=["all", "kernels", "decode", "prefill", "decode120b"], default="all",
                    help="all (default): config 1 headline with configs 0, 2, 3 and 4 under config; "
                         "kernels: configs 1 and 0 only; decode: config 2 (use --steps 256); prefill: "
                         "config 3, grouped MFMA MoE; decode120b: config 4 (use --steps 128)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the expert path is built and timed on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured configuration).", file=sys.stderr)
        sys.exit(2)
    cpu_on = not args.no_cpu
    if args.mode == "decode":
        print(json.dumps(measure_decode20b(args, args.steps, args.warmup, cpu_on)))
        return
    if args.mode == "prefill":
        print(json.dumps(measure_prefill(args, args.steps, args.warmup, cpu_on)))
        return
    if args.mode == "decode120b":
        print(json.dumps(measure_decode120b(args, args.steps, args.warmup, cpu_on)))
        return
    line = measure_moe_layer(args)
    if args.mode == "all":
        # configs 2, 3 and 4 in the same run, each with its roofline and CPU baseline
        ds, ds4 = args.decode_steps, args.decode120_steps
        d20 = measure_decode20b(args, ds, 8, cpu_on)
        pf = measure_prefill(args, args.prefill_steps, 2, cpu_on)
        d120 = measure_decode120b(args, ds4, 4, cpu_on)
        line["config"]["decode_20b"] = {"tok_s": d20["value"], "ms_per_token": d20["ms_per_step"],
                                        "steps": ds, **{k: d20["config"][k] for k in
                                                        ("workload", "bytes_per_token", "hbm_gbps", "hbm_frac",
                                                         "prefill_tok_s", "attention_us_per_layer",
                                                         "expert_arithmetic", "other_arithmetic")},
                                        "lm_head_roofline": d20["roofline"], "cpu_baseline": d20["cpu_baseline"]}
        line["config"]["prefill_grouped"] = {"tflops": pf["value"], "ms_per_layer": pf["ms_per_step"],
                                             "steps": pf["steps"], "dtype": pf["dtype"],
                                             **{k: pf["config"][k] for k in
                                                ("workload", "pairs", "gate_up_ms", "down_ms")},
                                             "roofline": pf["roofline"], "cpu_baseline": pf["cpu_baseline"]}
        line["config"]["decode_120b"] = {"batch1_tok_s": d120["config"]["batch1_tok_s"],
                                         "steps": ds4, **{k: d120["config"][k] for k in
                                                          ("workload", "batch1_bytes_per_token", "batch1_hbm_gbps",
                                                           "batch1_expert_arithmetic", "batch1_other_arithmetic",
                                                           "batch32_tok_s", "batch32_ms_per_step",
                                                           "batch32_hbm_gbps")},
                                         "lm_head_roofline": d120["roofline"],
                                         "cpu_baseline": d120["cpu_baseline"]}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
