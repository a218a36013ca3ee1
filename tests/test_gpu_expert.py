"""GPU parity of the INT4 expert path against the oracle (oracle/pk_oracle.c,
itself bit-exact with picchio's quant.h / picchio.c, see test_oracle.py).

Bars: INT4 group-scaled GEMV and the gs64 quantizer bit-exact; fp32 results
of the expert FFN and MoE layer within relative L2 1e-4,
top-k expert ids identical.
"""
import numpy as np
import pytest

from helpers import REL_L2_TOL, bits_equal, first_mismatch, rel_l2

pytestmark = pytest.mark.gpu


def _engine(cfg):
    import picchio_amd
    return picchio_amd.Engine(cfg)


def _rand(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


# ───────────────────────── INT4 GEMV ─────────────────────────

@pytest.mark.parametrize("O,I,S", [(5760, 2880, 1), (2880, 2880, 1), (2880, 2880, 3),
                                   (100, 128, 2), (64, 64, 1), (720, 2880, 1),
                                   (5760, 2880, 8), (2880, 2880, 12), (100, 128, 600)])
def test_i4_gs64_gemv_tiled_bitexact(gpu, oracle, O, I, S):
    """Tiled HBM layout + cvt_off decode reproduce matmul_i4_gs bit for bit;
    the last three shapes have 540-720 row blocks per launch, so they run on
    the persistent streaming kernel (one workgroup per CU walking the row
    blocks with the next block's weights in flight)."""
    import picchio_amd as pa
    import torch
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=4, ctx_len=16, vocab=64)
    w = _rand((O, I), 11 + O + I, 0.02)
    q4, s = oracle.quant_gs(w, 64)
    x = _rand((S, I), 7 + S)
    y_ref = oracle.mm_i4_gs(x, q4, s, O, I, 64)
    with _engine(cfg) as eng:
        qt = eng.qt_upload(pa.FMT_INT4, q4, s, O, I, 64)
        xd = eng.to_dev(x)
        yd = eng.empty((S, O), torch.float32)
        eng.matmul_qt(yd, xd, qt, S)
        y = eng.to_host(yd)
        eng.qt_free(qt)
    assert bits_equal(y, y_ref), first_mismatch(y, y_ref)


@pytest.mark.parametrize("O,I,gs,S", [(37, 200, 64, 2), (16, 101, 32, 2), (5, 50, 64, 3),
                                      (9, 130, 48, 1), (7, 33, 33, 1), (8, 64, 16, 1)])
def test_i4_gs_gemv_ragged_bitexact(gpu, oracle, O, I, gs, S):
    """Shapes outside the tiled layout (short last group, odd width, other
    group sizes) run the reference-layout kernel, still bit-exact."""
    import picchio_amd as pa
    import torch
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=4, ctx_len=16, vocab=64)
    w = _rand((O, I), 100 + O, 0.02)
    q4, s = oracle.quant_gs(w, gs)
    gs_eff = gs if 0 < gs < I else I
    x = _rand((S, I), 3)
    y_ref = oracle.mm_i4_gs(x, q4, s, O, I, gs_eff)
    with _engine(cfg) as eng:
        qt = eng.qt_upload(pa.FMT_INT4, q4, np.ascontiguousarray(s), O, I, gs_eff)
        xd = eng.to_dev(x)
        yd = eng.empty((S, O), torch.float32)
        eng.matmul_qt(yd, xd, qt, S)
        y = eng.to_host(yd)
        eng.qt_free(qt)
    assert bits_equal(y, y_ref), first_mismatch(y, y_ref)


@pytest.mark.parametrize("O,I,gs", [(5760, 2880, 64), (37, 200, 64), (16, 101, 32),
                                    (7, 33, 33), (6, 40, 0), (4, 10, 64)])
def test_quantizer_bitexact(gpu, oracle, O, I, gs):
    """GPU gs64 quantizer == convert.py restatement, bytes and scales."""
    import torch
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=4, ctx_len=16, vocab=64)
    w = _rand((O, I), 5 + I, 0.02)
    w[0, :min(I, 8)] = 0.0                      # an (almost) all-zero group
    q_ref, s_ref = oracle.quant_gs(w, gs)
    ng = s_ref.shape[1]
    with _engine(cfg) as eng:
        wd = eng.to_dev(w)
        qd = eng.empty((O, (I + 1) // 2), torch.uint8)
        sd = eng.empty((O, ng), torch.float32)
        eng.quantize_int4_gs(wd, O, I, gs, qd, sd)
        q = eng.to_host(qd)
        s = eng.to_host(sd)
    assert np.array_equal(q, q_ref)
    assert bits_equal(s, s_ref)


# ───────────────────────── dense matmul_qt ─────────────────────────

@pytest.mark.parametrize("fmt,S", [("f32", 2), ("f32", 7), ("f32", 37), ("q8", 2), ("i4row", 2)])
def test_matmul_qt_formats(gpu, oracle, fmt, S):
    """S >= 4 fp32 rows run the skinny GEMM (one weight read per 32 inputs)."""
    import torch
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=4, ctx_len=16, vocab=64)
    O, I = 300, (2900 if fmt == "f32" else 2880)      # f32: a ragged last 256-column chunk
    x = _rand((S, I), 9)
    y_ref = np.empty((S, O), np.float32)
    W = _rand((O, I), 10, 0.02)
    if fmt == "f32":
        oracle.matmul_f32(y_ref, x, W, S, I, O)
        args = (pa.FMT_F32, W, None, O, I, 0)
    elif fmt == "q8":
        q = np.empty((O, I), np.int8)
        s = np.empty(O, np.float32)
        oracle.quantize_int8_rows(W, O, I, q, s)
        oracle.matmul_q8(y_ref, x, q, s, S, I, O)
        args = (pa.FMT_INT8, q, s, O, I, 0)
    else:
        q = np.empty((O, (I + 1) // 2), np.uint8)
        s = np.empty(O, np.float32)
        oracle.quantize_rows_i4(W, O, I, q, s)
        oracle.matmul_i4(y_ref, x, q, s, S, I, O)
        args = (pa.FMT_INT4, q, s, O, I, 0)
    with _engine(cfg) as eng:
        qt = eng.qt_upload(*args)
        xd = eng.to_dev(x)
        yd = eng.empty((S, O), torch.float32)
        eng.matmul_qt(yd, xd, qt, S)
        y = eng.to_host(yd)
        eng.qt_free(qt)
    if fmt in ("f32", "q8"):                       # quant.h's chains and hsum tree: the same bits
        assert bits_equal(y, y_ref), first_mismatch(y, y_ref)
    else:
        assert rel_l2(y, y_ref) < 1e-6


def test_matmul_qt_dense_golden(gpu):
    """matmul_qt F32 / INT8 on the vectors picchio's own matmul_f32 / matmul_q8
    produced (tests/golden/matmul_dense.npz: ragged I = 13, 37, 4101, I < 8,
    I = 1): bit for bit."""
    import os
    import torch
    import picchio_amd as pa
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "matmul_dense.npz"), allow_pickle=False)
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=4, ctx_len=16, vocab=64)
    with _engine(cfg) as eng:
        for i in range(int(z["n"])):
            S, I, O = (int(v) for v in z[f"c{i}_shape"])
            x = z[f"c{i}_x"]
            for args, ref in [((pa.FMT_F32, z[f"c{i}_W"], None, O, I, 0), z[f"c{i}_yf"]),
                              ((pa.FMT_INT8, z[f"c{i}_q8"], z[f"c{i}_s8"], O, I, 0), z[f"c{i}_y8"])]:
                qt = eng.qt_upload(*args)
                yd = eng.empty((S, O), torch.float32)
                eng.matmul_qt(yd, eng.to_dev(x), qt, S)
                y = eng.to_host(yd)
                eng.qt_free(qt)
                assert bits_equal(y, ref), (i, args[0], first_mismatch(y, ref))


# ───────────────────────── expert FFN / MoE layer ─────────────────────────

@pytest.fixture(scope="module")
def moe_setup(gpu, oracle):
    """One GPT-OSS-20B-shaped MoE layer (8 experts to keep the CPU build
    short; every expert has the full 5760x2880 / 2880x2880 shape)."""
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=8, ctx_len=16, vocab=64)
    model = oracle.model_build(cfg, 20240601, 0)
    eng = pa.Engine(cfg)
    for e in range(cfg.n_experts):
        eng.store_expert(0, e, *oracle.expert_arrays(model, 0, e, cfg))
    D, E = cfg.hidden, cfg.n_experts
    router = oracle.tensor(model, 6, 0, E * D)          # PK_T_ROUTER
    rbias = oracle.tensor(model, 7, 0, E)               # PK_T_ROUTER_B
    eng.store_router(0, router, rbias)
    yield cfg, model, eng
    eng.close()
    oracle.model_free(model)


def _token_x(oracle, cfg, t):
    x = oracle.normal(77, 1, t, 0, cfg.hidden)
    xn = np.empty_like(x)
    oracle.rmsnorm(xn, x, np.ones(cfg.hidden, np.float32), cfg.hidden, 1e-5)
    return xn


def test_expert_apply_parity(moe_setup, oracle):
    import torch
    cfg, model, eng = moe_setup
    D = cfg.hidden
    for eid, w in [(0, 0.25), (5, 1.0), (7, -0.5)]:
        x = _token_x(oracle, cfg, 1000 + eid)
        dst0 = oracle.normal(78, 1, eid, 0, D)
        ref = dst0.copy()
        oracle.expert_apply(model, 0, eid, x, ref, w)
        xd = eng.to_dev(x)
        dd = eng.to_dev(dst0)
        eng.expert_apply(0, eid, xd, dd, w)
        got = eng.to_host(dd)
        assert rel_l2(got - dst0, ref - dst0) < 1e-6


def test_expert_gate_up_down_batched(moe_setup, oracle):
    """gate_up and down over three experts in one launch each give the same
    bits as expert_apply of each expert alone (w = 1 into zeros is exact),
    and match the oracle's expert FFN."""
    import torch
    cfg, model, eng = moe_setup
    D, H = cfg.hidden, cfg.moe_inter // 2
    eids = np.array([6, 1, 3], np.int32)
    x = _token_x(oracle, cfg, 2024)
    xd = eng.to_dev(x)
    act = eng.empty((3, H), torch.float32)
    eo = eng.empty((3, D), torch.float32)
    ed = eng.to_dev(eids)
    eng.expert_gate_up(0, ed, xd, act)
    eng.expert_down(0, ed, act, eo)
    got = eng.to_host(eo)
    for k, eid in enumerate(eids):
        one = eng.to_dev(np.zeros(D, np.float32))
        eng.expert_apply(0, int(eid), xd, one, 1.0)
        assert bits_equal(got[k], eng.to_host(one)), k
        ref = np.zeros(D, np.float32)
        oracle.expert_apply(model, 0, int(eid), x, ref, 1.0)
        assert rel_l2(got[k], ref) < 1e-6


@pytest.mark.parametrize("dot", [0, 1])
def test_expert_gate_up_streaming_matches_tiled(moe_setup, oracle, dot):
    """gate_up over all 8 experts in one launch (720 row blocks: the
    persistent streaming kernel) gives, for experts 6, 1 and 3, the bits of
    gate_up over those three alone (270 row blocks: one workgroup per row
    block), on picchio's fp32 chains and on the integer dot (outputs and
    their records)."""
    import torch
    cfg, model, eng = moe_setup
    D, H, E = cfg.hidden, cfg.moe_inter // 2, cfg.n_experts
    x = _token_x(oracle, cfg, 4711)
    xd = eng.to_dev(x)
    all_e = np.arange(E, dtype=np.int32)[::-1].copy()
    three = np.array([6, 1, 3], np.int32)
    outs = {}
    for name, ids in (("all", all_e), ("three", three)):
        act = eng.empty((len(ids), H), torch.float32)
        if dot:
            rec = eng.empty(((D + 31) // 32) * 24, torch.int32)
            eng.act_records(xd, rec)
            arec = eng.empty((len(ids), (cfg.moe_inter // 64) * 24), torch.int32)
            eng.expert_gate_up_dot(0, eng.to_dev(ids), rec, act, arec)
            outs[name] = (eng.to_host(act), eng.to_host(arec))
        else:
            eng.expert_gate_up(0, eng.to_dev(ids), xd, act)
            outs[name] = (eng.to_host(act), None)
    for k, eid in enumerate(three):
        j = int(np.where(all_e == eid)[0][0])
        assert bits_equal(outs["all"][0][j], outs["three"][0][k]), eid
        if dot:
            assert np.array_equal(outs["all"][1][j], outs["three"][1][k]), eid
    eng.sync()


def test_moe_forward_parity(moe_setup, oracle):
    import torch
    cfg, model, eng = moe_setup
    D, K, E = cfg.hidden, cfg.topk, cfg.n_experts
    worst = 0.0
    for t in range(12):
        x = _token_x(oracle, cfg, t)
        out_ref = np.empty(D, np.float32)
        sel_ref = np.empty(K, np.int32)
        w_ref = np.empty(K, np.float32)
        logits = np.empty(E, np.float32)
        oracle.moe_forward(model, 0, x, out_ref, sel_ref, w_ref, logits)
        xd = eng.to_dev(x)
        od = eng.empty(D, torch.float32)
        # the router launch alone (a fixed-tree sum: within 1e-5 absolute of the in-order one)
        ld = eng.empty(E, torch.float32)
        eng.router_logits(0, xd, ld)
        assert np.allclose(eng.to_host(ld), logits, rtol=1e-5, atol=1e-5), t
        sel, w = eng.moe_forward(0, xd, od, want_routing=True)
        out = eng.to_host(od)
        srt = np.sort(logits)[::-1]
        margin = float(srt[K - 1] - srt[K])           # 4th vs 5th logit
        if margin > 1e-5:
            assert list(sel) == list(sel_ref), (t, sel, sel_ref, margin)
            assert np.allclose(w, w_ref, rtol=1e-5, atol=0)
            err = rel_l2(out, out_ref)
            worst = max(worst, err)
            assert err < REL_L2_TOL, (t, err)
    assert worst < 1e-5


@pytest.mark.parametrize("dot", [0, 1])
def test_moe_one_launch_matches_two(moe_setup, oracle, dot):
    """The batch-1 experts as one launch give the same bits as the gate_up
    launch + down launch, token after token (the hand-over tags advance with
    every launch), on picchio's fp32 chains and on the integer dot: the
    default row-block form (mode 1), the form with every CU streaming the
    same bytes (mode 2, whose row blocks are split between workgroups and
    continued in group order), and mode 1 again after the others; and no
    device-side wait gave up."""
    import torch
    cfg, model, eng = moe_setup
    D = cfg.hidden
    eng.set_i4_dot(dot)
    try:
        for t in range(6):
            x = _token_x(oracle, cfg, 500 + t)
            xd = eng.to_dev(x)
            outs, sels = [], []
            for mode in (1, 0, 2, 1):
                eng.set_moe_fused(mode)
                od = eng.empty(D, torch.float32)
                sel, w = eng.moe_forward(0, xd, od, want_routing=True)
                outs.append(eng.to_host(od))
                sels.append((list(sel), list(w)))
            assert sels[0] == sels[1] == sels[2] == sels[3], (t, sels)
            for m in (0, 2, 3):
                assert np.array_equal(outs[m].view(np.uint32), outs[1].view(np.uint32)), (t, m)
        eng.sync()
    finally:
        eng.set_moe_fused(1)
        eng.set_i4_dot(0)


def test_moe_balanced_launch_runs_here(gpu):
    """Mode 2's ranges hold for the 20B and 120B shapes (top-4) on this
    device's CUs, so that mode runs the balanced launch, not its fallback."""
    import torch
    import picchio_amd as pa
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    assert pa.lib().pk_moe_bal_plan(4, 90, 45, 45, 45, n_cu, None, 0) == 1


def test_moe_one_launch_fits_this_device_only(gpu):
    """The one-launch experts run only where their waiting down tasks leave
    a free workgroup slot: on this device (all its CUs) the 20B shape takes
    that form, on a device partition of 64 CUs it falls back to two launches
    (its 180 down tasks would fill every slot)."""
    import ctypes as C
    import torch
    import picchio_amd as pa
    lib = pa.lib()
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    out = (C.c_int * 360)()
    assert lib.pk_moe_ffn_plan(90, 45, 4, n_cu, 0, out, 360) == 1
    assert lib.pk_moe_ffn_plan(90, 45, 4, n_cu, 1, out, 360) == 1
    assert sorted(out) == list(range(360))
    assert lib.pk_moe_ffn_plan(90, 45, 4, 64, 0, out, 360) == 0
    assert sorted(out) == list(range(360))


def test_router_ties_take_lowest_index(moe_setup, oracle):
    """Equal router logits: the lowest expert index is taken first
    (picchio.c:1327-1339, strict '>' over experts in order), and equal
    logits get equal weights. Rows 2 and 5 of the router are the same, and
    rows 1 and 6, so their logits have the same bits; the top-4 is then
    2, 5, 1, 6 by construction."""
    import torch
    cfg, model, eng = moe_setup
    D, E = cfg.hidden, cfg.n_experts
    router = oracle.tensor(model, 6, 0, E * D)
    rbias = oracle.tensor(model, 7, 0, E)
    x = _token_x(oracle, cfg, 4242)
    R = (router.reshape(E, D) * 0.01).astype(np.float32)
    R[2] = R[5] = x * 0.05
    R[1] = R[6] = x * 0.03
    try:
        eng.store_router(0, np.ascontiguousarray(R).ravel(), np.zeros(E, np.float32))
        xd = eng.to_dev(x)
        od = eng.empty(D, torch.float32)
        sel, w = eng.moe_forward(0, xd, od, want_routing=True)
        assert list(sel) == [2, 5, 1, 6], sel
        assert w[0] == w[1] and w[2] == w[3] and w[0] > w[2], w
    finally:
        eng.store_router(0, router, rbias)


def test_moe_forward_batch_prefill_order(moe_setup, oracle):
    """Batched MoE = forward_prefill's MoE (picchio.c:1829-1916): same routing
    as decode per token; each token sums its experts in the order the batch
    first requested them (restated here with the oracle's expert_apply)."""
    import torch
    import picchio_amd as pa
    cfg, model, eng = moe_setup
    D, K, T = cfg.hidden, cfg.topk, 7
    xs = np.stack([_token_x(oracle, cfg, 50 + t) for t in range(T)])
    xd = eng.to_dev(xs)
    ob = eng.empty((T, D), torch.float32)
    sd = eng.empty((T, K), torch.int32)
    wd = eng.empty((T, K), torch.float32)
    pa.check(eng.L.pk_moe_forward_batch(eng.h, 0, pa.ptr(xd), T, pa.ptr(ob), pa.ptr(sd), pa.ptr(wd)))
    got, sel, w = eng.to_host(ob), eng.to_host(sd), eng.to_host(wd)
    rank = {}
    for e in sel.ravel():
        rank.setdefault(int(e), len(rank))
    od = eng.empty(D, torch.float32)
    for t in range(T):
        s1, w1 = eng.moe_forward(0, xd[t], od, want_routing=True)
        assert list(s1) == list(sel[t])
        acc = np.zeros(D, np.float32)
        for k in sorted(range(K), key=lambda k: rank[int(sel[t, k])]):
            oracle.expert_apply(model, 0, int(sel[t, k]), xs[t], acc, float(w[t, k]))
        assert rel_l2(got[t], acc) < 1e-6, t


def test_missing_expert_is_an_error(gpu, oracle):
    """picchio skips a missing expert silently (picchio.c:1394); the library
    refuses the call instead."""
    import torch
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=4, ctx_len=16, vocab=64)
    with _engine(cfg) as eng:
        xd = eng.to_dev(np.zeros(cfg.hidden, np.float32))
        od = eng.empty(cfg.hidden, torch.float32)
        with pytest.raises(pa.PkError) as ei:
            eng.moe_forward(0, xd, od)
        assert ei.value.code in (-5,)


# ───────────────────────── persistent MoE sequence ─────────────────────────
