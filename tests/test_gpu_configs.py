"""BASELINE configs 1, 3 and 4 at their own shapes.

Config 1: one GPT-OSS-20B MoE layer with all 32 experts at batch-1 decode
(router launch + one-launch experts) against the oracle's moe_forward, the
4th / 5th router-logit margin of every token logged, both arithmetics.

Config 3: one GPT-OSS-20B MoE layer (32 experts) over T = 2048 tokens with
the Zipf(1.1) routing of the benchmark (8192 (token, expert) pairs, 16..512
pairs per expert), through the expert-grouped MFMA GEMMs
(pk_moe_forward_grouped), both arithmetics. Int8 limbs: activation limbs
and exponents of all rows bit-exact with the oracle's restatement; sampled
pairs' down outputs bit-exact given the same activations. Half-precision
pairs (the default): sampled pairs' SwiGLU activations and down outputs
within relative L2 2e-6 of picchio's fp32 GEMV (matmul_i4_gs). Both:
per-token outputs of 160 sampled tokens within relative L2 1e-5 of picchio's
fp32 expert_apply arithmetic in forward_prefill's first-request expert order
(picchio.c:1829-1916).

Config 4: the GPT-OSS-120B shape (36 layers, 128 experts) with 4096-position
synthetic KV contexts, at batch 1 (the replayed decode step) and batch 32
(pk_decode_batch, the MoE on the integer-dot arithmetic): each batch-32
row's ids = forward_token's eager chain over that row's context, and on a
128-expert, 4096-position model with 2 layers = the oracle's chain, every
departure explained by a traced routing near-tie (picchio.c:504-623,
:1327-1339, :1655-1756).
"""
import numpy as np
import pytest

from helpers import bits_equal, first_mismatch, rel_l2, upload_model

pytestmark = pytest.mark.gpu

GOLDEN = 0x9E3779B97F4A7C15
M64 = (1 << 64) - 1


def _seq0_seed_like(seed, s):
    """pk_kv_fill_synthetic seeds layer l of sequence s with
    seed*GOLDEN + (s*1024 + l)*2: the seed that gives sequence 0 the rows of
    sequence s."""
    return ((seed * GOLDEN + s * 2048) * pow(GOLDEN, -1, 1 << 64)) & M64


def _margin(lg):
    top = np.sort(lg)[-2:]
    return float(top[1] - top[0]), float(abs(top[1]))


# ───────────────────────────── config 1 ─────────────────────────────

@pytest.mark.parametrize("dot", [0, 1], ids=["fp32", "dot"])
def test_config1_moe_layer_32_experts(gpu, oracle, dot):
    """Config 1 at its own shape: one GPT-OSS-20B MoE layer with all 32
    experts (router 32 x 2880 + bias), batch-1 tokens through pk_moe_forward
    (router launch, then the one-launch experts) against the oracle's
    moe_forward (picchio.c:1309-1466). Every token's 4th / 5th router-logit
    margin is logged; the selected experts are identical wherever that
    margin exceeds the router sums' difference (the GPU router adds in a
    fixed tree, picchio in order: within 1e-5), and the layer output is
    within relative L2 1e-4 (fp32 chains: ~3e-6, from the routing weights;
    integer dot: ~2e-5)."""
    import torch
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=32, ctx_len=16, vocab=64)
    D, E, K = cfg.hidden, cfg.n_experts, cfg.topk
    model = oracle.model_build(cfg, 31337, 0)
    eng = pa.Engine(cfg)
    try:
        for e in range(E):
            eng.store_expert(0, e, *oracle.expert_arrays(model, 0, e, cfg))
        eng.store_router(0, oracle.tensor(model, 6, 0, E * D), oracle.tensor(model, 7, 0, E))
        eng.set_i4_dot(dot)
        margins, worst, hist = [], 0.0, np.zeros(E, np.int64)
        for t in range(40):
            x = oracle.normal(4242, 1, t, 0, D)
            xn = np.empty_like(x)
            oracle.rmsnorm(xn, x, np.ones(D, np.float32), D, 1e-5)
            out_ref = np.empty(D, np.float32)
            sel_ref = np.empty(K, np.int32)
            w_ref = np.empty(K, np.float32)
            logits = np.empty(E, np.float32)
            oracle.moe_forward(model, 0, xn, out_ref, sel_ref, w_ref, logits)
            od = eng.empty(D, torch.float32)
            sel, w = eng.moe_forward(0, eng.to_dev(xn), od, want_routing=True)
            m = _route_margin(logits, K)
            margins.append(m)
            hist[list(sel_ref)] += 1
            if m > 1e-5:
                assert list(sel) == list(sel_ref), (t, list(sel), list(sel_ref), m)
                err = rel_l2(eng.to_host(od), out_ref)
                worst = max(worst, err)
                assert err < 1e-4, (t, err)
        eng.sync()
        print(f"config 1 ({'integer dot' if dot else 'fp32 chains'}): 40 tokens, 4th/5th router margins min "
              f"{min(margins):.2e} median {np.median(margins):.2e}; experts hit {int((hist > 0).sum())} of {E}; "
              f"worst rel-L2 {worst:.2e}", flush=True)
        assert (hist > 0).sum() >= 24                       # the tokens spread over the experts
        # fp32 chains: the experts are picchio's bits; what differs is the
        # routing weights' softmax of the fixed-tree router logits (~1e-6)
        assert worst < (1e-5 if not dot else 1e-4)
    finally:
        eng.set_i4_dot(0)
        eng.close()
        oracle.model_free(model)


# ───────────────────────────── config 3 ─────────────────────────────

@pytest.mark.parametrize("f16", [True, False], ids=["f16", "int8"])
def test_config3_grouped_prefill_full_shape(gpu, oracle, f16):
    import torch
    import picchio_amd as pa
    from bench import zipf_routing
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=32, ctx_len=16, vocab=64)
    D, K, E, half = cfg.hidden, cfg.topk, cfg.n_experts, cfg.moe_inter // 2
    T = 2048
    model = oracle.model_build(cfg, 3, 0)
    eng = pa.Engine(cfg)
    try:
        upload_model(eng, oracle, model, cfg, dense=False, globals_=False)
        sel, w, counts = zipf_routing(T, E, K, 3)
        assert sel.size == 8192 and counts.min() >= 16 and counts.max() <= 512
        x = np.random.default_rng(10).standard_normal((T, D)).astype(np.float32)
        xd = eng.to_dev(x)
        out = eng.empty((T, D), torch.float32)
        act = eng.empty((T * K, half), torch.float32)
        eo = eng.empty((T * K, D), torch.float32)
        eng.set_grouped_f16(f16)
        eng.moe_forward_grouped(0, xd, out, eng.to_dev(sel), eng.to_dev(w), act, eo)
        out, act, eo = eng.to_host(out), eng.to_host(act), eng.to_host(eo)
        pairs = [0, 5, 1023, 2048, 4097, 6000, 8191, 7777]
        experts = {}
        if f16:
            # sampled pairs against picchio's fp32 GEMV on the same inputs
            for p in pairs:
                t, k = divmod(p, K)
                e = int(sel[t, k])
                if e not in experts:
                    experts[e] = oracle.expert_arrays(model, 0, e, cfg)
                gq, gs, dq, ds, gb, db = experts[e]
                y = np.empty(cfg.moe_inter, np.float32)
                oracle.matmul_i4_gs(y, np.ascontiguousarray(x[t]), gq, gs, 1, D, cfg.moe_inter, cfg.group_size)
                y += gb
                oracle.swiglu_clamped(y, cfg.moe_inter, cfg.swiglu_limit, cfg.swiglu_alpha)
                assert rel_l2(act[p], y[:half]) < 2e-6, p
                eo_ref = np.empty(D, np.float32)
                oracle.matmul_i4_gs(eo_ref, np.ascontiguousarray(act[p]), dq, ds, 1, half, D, cfg.group_size)
                eo_ref += db
                assert rel_l2(eo[p], eo_ref) < 2e-6, p
            pairs = []

        # activation limbs of every row
        if f16:
            xl = xe = None
        else:
            limbs = eng.empty((3, T, D), torch.int8)
            exps = eng.empty(T, torch.int32)
            eng.quantize_act_i8x3(xd, limbs, exps)
            xl = np.empty((3, T, D), np.int8)
            xe = np.empty(T, np.int32)
            oracle.act_limbs(x, T, D, xl, xe)
            assert np.array_equal(eng.to_host(exps), xe)
            assert np.array_equal(eng.to_host(limbs), xl)

        # sampled pairs: the integer path restated (gate_up to 1e-6, down bit-exact)
        for p in pairs:
            t, k = divmod(p, K)
            e = int(sel[t, k])
            if e not in experts:
                experts[e] = oracle.expert_arrays(model, 0, e, cfg)
            gq, gs, dq, ds, gb, db = experts[e]
            y = np.empty(cfg.moe_inter, np.float32)
            oracle.mfma_matvec(gq, gs, gb, cfg.moe_inter, D, xl[0, t], xl[1, t], xl[2, t], int(xe[t]), y)
            oracle.swiglu_clamped(y, cfg.moe_inter, cfg.swiglu_limit, cfg.swiglu_alpha)
            assert rel_l2(act[p], y[:half]) < 1e-6, p
            al = np.empty((3, 1, half), np.int8)
            ae = np.empty(1, np.int32)
            oracle.act_limbs(np.ascontiguousarray(act[p]), 1, half, al, ae)
            eo_ref = np.empty(D, np.float32)
            oracle.mfma_matvec(dq, ds, db, D, half, al[0, 0], al[1, 0], al[2, 0], int(ae[0]), eo_ref)
            assert bits_equal(eo[p], eo_ref), (p, first_mismatch(eo[p], eo_ref))

        # per-token outputs against picchio's fp32 arithmetic, first-request order
        rank = {}
        for e in sel.ravel():
            rank.setdefault(int(e), len(rank))
        worst = 0.0
        for t in np.random.default_rng(11).choice(T, 160, replace=False):
            acc = np.zeros(D, np.float32)
            for k in sorted(range(K), key=lambda k: rank[int(sel[t, k])]):
                oracle.expert_apply(model, 0, int(sel[t, k]), x[t], acc, float(w[t, k]))
            err = rel_l2(out[t], acc)
            worst = max(worst, err)
            assert err < 1e-5, (int(t), err)
        print(f"config 3 ({'f16' if f16 else 'int8'}): worst token rel-L2 {worst:.2e} over 160 tokens",
              flush=True)
    finally:
        eng.close()
        oracle.model_free(model)


# ───────────────────────────── config 4 ─────────────────────────────
#
# Lockstep rows (pk_decode_batch) run other fp32 operation orders than the
# chain they are checked against (integer-dot experts and skinny GEMMs
# against forward_token's fp32 chains, or against the oracle): their hidden
# states differ by the arithmetic alone, ~1e-6 relative. A routing decision
# whose 4th and 5th router logits lie closer than that can go the other way
# and change that row's later ids. So every row is followed with the router
# logits of both chains (pk_set_router_trace, po_set_router_trace), and
# every departure must be explained:
#  * until the row's first routing flip, every router logit of the two
#    chains agrees within ROUTER_DELTA (the arithmetic difference), and
#  * at a departing step either a routing flip happened at that step or an
#    earlier one, at a 4th / 5th logit margin below 2 x ROUTER_DELTA (a
#    near-tie the arithmetic difference can reorder), or, with no flip, the
#    reference chain's top-2 logits lie within TOP2_REL of each other.
# No count of departures is allowed beyond that.

# |router logit difference| before any flip. The router logits are ~N(0, 1);
# the integer-dot MoE layer is within 2e-5 relative of picchio's arithmetic,
# and over 36 layers the two residual streams drift apart to ~1e-4 of the
# logits (measured 1.04e-4 by layer 16 of row 0): 1e-3 leaves room for that
# drift while any wrong weight, expert or position shows up as O(0.1).
ROUTER_DELTA = 1e-3
TOP2_REL = 2e-3          # top-2 logit margin / max(|top logit|, 1) that the lm_head's order may flip


def _route(lg, K):
    """moe_forward's top-k (picchio.c:1327-1339): repeated argmax with strict
    '>', the lowest index winning a tie."""
    return tuple(np.lexsort((np.arange(len(lg)), -lg.astype(np.float64)))[:K])


def _route_margin(lg, K):
    srt = np.sort(lg.astype(np.float64))[::-1]
    return float(srt[K - 1] - srt[K])


def _explain_row(s, got_ids, ref_ids, ref_top2, got_tr, ref_tr, K):
    """One row: got_tr / ref_tr [steps][layers][E] router logits of the
    checked and the reference chain (over the steps both ran), got_ids /
    ref_ids the ids, ref_top2 the reference's (gap, |top|) per step.
    Returns (equal steps, flips, departure or None); asserts the rules."""
    flips, first_flip = [], None
    equal = 0
    for i in range(len(ref_ids)):
        for l in range(ref_tr.shape[1]):
            if first_flip is not None:
                break
            a, b = ref_tr[i, l], got_tr[i, l]
            delta = float(np.max(np.abs(a.astype(np.float64) - b)))
            assert delta <= ROUTER_DELTA, ("router logits apart beyond the arithmetic", s, i, l, delta)
            if set(_route(a, K)) != set(_route(b, K)):
                m = _route_margin(a, K)
                flips.append((i, l, m, delta))
                first_flip = (i, l)
                assert m < 2 * ROUTER_DELTA, ("routing flip at a clear margin", s, i, l, m, delta)
        if int(got_ids[i]) != int(ref_ids[i]):
            gap, top = ref_top2[i]
            explained = first_flip is not None and first_flip[0] <= i
            assert explained or gap < TOP2_REL * max(top, 1.0), \
                ("departure without a near-tie", s, i, int(got_ids[i]), int(ref_ids[i]), gap, flips)
            return equal, flips, (i, int(got_ids[i]), int(ref_ids[i]), round(gap, 5), first_flip)
        equal += 1
    return equal, flips, None


def test_config4_full_shape_batch_rows_equal_eager_chains(gpu):
    """36 layers x 128 experts (64.7 GB of experts) resident; 32 sequences
    with their own 4096-position contexts decoded in lockstep (the router
    logits of every row and layer traced); then each sequence's context is
    placed in sequence 0 and forward_token (eager, picchio's fp32 expert
    chains) walks the same ids with its router logits traced. Every
    departure is explained by a measured near-tie (rules above). Batch 1:
    the replayed decode step equals the eager chain exactly (same
    arithmetic)."""
    import torch
    import picchio_amd as pa
    ctx, steps, B, seed, kv_seed = 4096, 4, 32, 404, 77
    cfg = pa.gptoss_cfg(n_layers=36, n_experts=128, ctx_len=ctx + 8 + 1)
    L, E, K = cfg.n_layers, cfg.n_experts, cfg.topk
    eng = pa.Engine(cfg)
    try:
        eng.build_synthetic(seed, what=7)
        eng.batch_reserve(B)
        for s in range(B):
            eng.kv_fill_synthetic(s, ctx, kv_seed)
        first = np.random.default_rng(5).integers(0, cfg.vocab, B).astype(np.int32)
        tr = eng.empty(steps * L * B * E, torch.float32)
        eng.set_router_trace(tr)
        got = eng.decode_batch(first, ctx, steps)
        assert eng.router_trace_used() == steps * L * B * E
        got_tr = eng.to_host(tr).reshape(steps, L, B, E)
        etr = eng.empty(steps * L * E, torch.float32)
        lg = eng.empty(cfg.vocab, torch.float32)
        compared, all_flips, departures = 0, [], []
        for s in range(B):
            eng.kv_fill_synthetic(0, ctx, _seq0_seed_like(kv_seed, s))
            eng.set_router_trace(etr)
            tok, ref_ids, top2 = int(first[s]), [], []
            for i in range(steps):
                nxt = eng.forward_token(tok, ctx + i, lg)
                ref_ids.append(nxt)
                top2.append(_margin(eng.to_host(lg)))
                if int(got[i, s]) != nxt:
                    break
                tok = nxt
            n = len(ref_ids)
            ref_tr = eng.to_host(etr)[:n * L * E].reshape(n, L, E)
            eq, flips, dep = _explain_row(s, got[:n, s], ref_ids, top2, got_tr[:n, :, s], ref_tr, K)
            compared += eq
            all_flips += [(s, i, l, f"{m:.2e}", f"{d:.2e}") for i, l, m, d in flips]
            if dep:
                departures.append((s,) + dep)
        eng.set_router_trace(None)
        print(f"config 4 batch 32: {compared} of {B * steps} (row, step) ids equal; routing flips (row, step, "
              f"layer, eager 4th/5th margin, router logit difference) {all_flips}; departures (row, step, got, "
              f"eager, eager top-2 gap, first flip) {departures}", flush=True)
        # batch 1: the replayed step graph over sequence 0's context
        eng.kv_fill_synthetic(0, ctx, kv_seed)
        rep = [int(v) for v in eng.decode_replay(int(first[0]), ctx, 8)]
        eng.kv_fill_synthetic(0, ctx, kv_seed)
        tok, eager = int(first[0]), []
        for i in range(8):
            tok = eng.forward_token(tok, ctx + i, None)
            eager.append(tok)
        assert rep == eager, (rep, eager)
    finally:
        eng.close()


def test_config4_oracle_parity_128_experts_4096_positions(gpu, oracle):
    """All 32 rows of a 128-expert, 2-layer model (every width at its 120B
    size) over 4096-position contexts: decode_batch ids equal the oracle's
    forward_token chains step by step, every departure explained by a
    measured near-tie along that row (router logits of both chains traced;
    rules above); batch 1 (decode_replay) equals the oracle chain."""
    import torch
    import picchio_amd as pa
    ctx, steps, B, seed, kv_seed = 4096, 3, 32, 909, 31
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=128, ctx_len=ctx + 8 + 1, vocab=2000)
    L, E, K = cfg.n_layers, cfg.n_experts, cfg.topk
    model = oracle.model_build(cfg, seed, 0)
    eng = pa.Engine(cfg)
    otr = np.zeros(steps * L * E, np.float32)
    try:
        upload_model(eng, oracle, model, cfg)
        eng.batch_reserve(B)
        for s in range(B):
            eng.kv_fill_synthetic(s, ctx, kv_seed)
        first = np.random.default_rng(6).integers(0, cfg.vocab, B).astype(np.int32)
        tr = eng.empty(steps * L * B * E, torch.float32)
        eng.set_router_trace(tr)
        got = eng.decode_batch(first, ctx, steps)
        eng.set_router_trace(None)
        got_tr = eng.to_host(tr).reshape(steps, L, B, E)
        ref_lg = np.empty(cfg.vocab, np.float32)
        compared, all_flips, departures = 0, [], []
        for s in range(B):
            oracle.model_reset_kv(model)
            for layer in range(L):
                sk = (kv_seed * GOLDEN + (s * 1024 + layer) * 2) & M64
                oracle.model_fill_kv(model, layer, ctx, sk, (sk + 1) & M64)
            oracle.set_router_trace(otr.ctypes.data, otr.size)
            tok, ref_ids, top2 = int(first[s]), [], []
            for i in range(steps):
                nxt = oracle.forward_token(model, tok, ctx + i, ref_lg.ctypes.data)
                ref_ids.append(nxt)
                top2.append(_margin(ref_lg))
                if int(got[i, s]) != nxt:
                    break
                tok = nxt
            oracle.set_router_trace(None, 0)
            n = len(ref_ids)
            eq, flips, dep = _explain_row(s, got[:n, s], ref_ids, top2, got_tr[:n, :, s],
                                          otr[:n * L * E].reshape(n, L, E), K)
            compared += eq
            all_flips += [(s, i, l, f"{m:.2e}", f"{d:.2e}") for i, l, m, d in flips]
            if dep:
                departures.append((s,) + dep)
            if s == 0:
                oracle.model_reset_kv(model)
                for layer in range(L):
                    sk = (kv_seed * GOLDEN + layer * 2) & M64
                    oracle.model_fill_kv(model, layer, ctx, sk, (sk + 1) & M64)
                tok, chain = int(first[0]), []
                for i in range(6):
                    tok = oracle.forward_token(model, tok, ctx + i, None)
                    chain.append(tok)
                eng.kv_fill_synthetic(0, ctx, kv_seed)
                assert [int(v) for v in eng.decode_replay(int(first[0]), ctx, 6)] == chain
        print(f"config 4 (2 layers): {compared} of {B * steps} (row, step) ids equal the oracle's; routing flips "
              f"{all_flips}; departures {departures}", flush=True)
    finally:
        oracle.set_router_trace(None, 0)
        eng.close()
        oracle.model_free(model)
