"""GPU parity of the single-launch MoE layer (pk_set_moe_fused).

Bars: bit-identical to the three-launch path (router + top-k, gate_up +
SwiGLU, down + combine) on every output and on the routing results, also
when replayed from a HIP graph; moe_forward (picchio.c:1309-1466) of the
oracle within the north star's relative L2 1e-4 with identical top-k ids;
in place inside forward_token (input = residual = output row), and the
greedy streams recorded from picchio's own build on the golden tiny model.
"""
import numpy as np
import pytest

from helpers import REL_L2_TOL, bits_equal, first_mismatch, rel_l2, upload_model

pytestmark = pytest.mark.gpu


def _rows(n, D, seed):
    """RMSNorm'd N(0,1) rows, with a few rows at other scales."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, D)).astype(np.float32)
    x /= np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True)).astype(np.float32)
    x[1] *= 1e-3
    x[2] *= 40.0
    return np.ascontiguousarray(x)


@pytest.mark.parametrize("E", [32, 128])
def test_fused_matches_three_launches_bitwise(gpu, E):
    import torch
    import picchio_amd as pa
    L = 3
    cfg = pa.gptoss_cfg(n_layers=L, n_experts=E, ctx_len=16, vocab=64)
    eng = pa.Engine(cfg)
    try:
        eng.build_synthetic(21 + E, what=1)
        T, D = 24, cfg.hidden
        x = _rows(T, D, E)
        xd = eng.to_dev(x)
        o3 = eng.empty((T, D), torch.float32)
        of = eng.empty((T, D), torch.float32)
        r3 = [eng.moe_forward(t % L, xd[t], o3[t], want_routing=True) for t in range(T)]
        eng.set_moe_fused(True)
        rf = [eng.moe_forward(t % L, xd[t], of[t], want_routing=True) for t in range(T)]
        eng.status()
        a, b = eng.to_host(o3), eng.to_host(of)
        for t in range(T):
            assert list(r3[t][0]) == list(rf[t][0]), (t, r3[t][0], rf[t][0])
            assert bits_equal(r3[t][1], rf[t][1]), t
            assert bits_equal(a[t], b[t]), (t, first_mismatch(a[t], b[t]))
        # the bench's shape: consecutive fused layers replayed from a graph
        og = eng.empty((T, D), torch.float32)
        eng.capture_begin()
        for t in range(T):
            eng.moe_forward(t % L, xd[t], og[t])
        g = eng.capture_end()
        for rep in range(3):
            eng.sync()
            og.fill_(float("nan"))
            torch.cuda.synchronize()
            eng.graph_launch(g)
            eng.sync()
            assert bits_equal(eng.to_host(og), b), rep
        eng.graph_destroy(g)
        eng.status()
    finally:
        eng.close()


@pytest.fixture(scope="module")
def fused_moe(gpu, oracle):
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=8, ctx_len=16, vocab=64)
    model = oracle.model_build(cfg, 313, 0)
    eng = pa.Engine(cfg)
    for e in range(cfg.n_experts):
        eng.store_expert(0, e, *oracle.expert_arrays(model, 0, e, cfg))
    D, E = cfg.hidden, cfg.n_experts
    eng.store_router(0, oracle.tensor(model, 6, 0, E * D), oracle.tensor(model, 7, 0, E))
    eng.set_moe_fused(True)
    yield cfg, model, eng
    eng.close()
    oracle.model_free(model)


def test_fused_moe_forward_matches_oracle(fused_moe, oracle):
    import torch
    cfg, model, eng = fused_moe
    D, K, E = cfg.hidden, cfg.topk, cfg.n_experts
    x = _rows(10, D, 77)
    od = eng.empty(D, torch.float32)
    worst = 0.0
    for t in range(len(x)):
        out_ref = np.empty(D, np.float32)
        sel_ref = np.empty(K, np.int32)
        w_ref = np.empty(K, np.float32)
        logits = np.empty(E, np.float32)
        oracle.moe_forward(model, 0, x[t], out_ref, sel_ref, w_ref, logits)
        sel, w = eng.moe_forward(0, eng.to_dev(x[t]), od, want_routing=True)
        srt = np.sort(logits)[::-1]
        if float(srt[K - 1] - srt[K]) > 1e-5:          # 4th vs 5th logit apart
            assert list(sel) == list(sel_ref), t
            # the x40 row puts weights near 1e-19: relative error there is
            # the logit noise times the logit gap, so an absolute floor
            assert np.allclose(w, w_ref, rtol=1e-5, atol=1e-9)
            err = rel_l2(eng.to_host(od), out_ref)
            worst = max(worst, err)
            assert err < REL_L2_TOL, (t, err)
    eng.status()
    assert worst < 1e-5


def test_fused_decode_in_place_bitwise(gpu):
    """forward_token runs h += moe(rmsnorm(h)) with the norm fused into the
    layer and the combine writing h in place: logits bit-identical to the
    three-launch step, and the same greedy stream from the replayed graph."""
    import torch
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=32, ctx_len=64, vocab=2000)
    eng = pa.Engine(cfg)
    try:
        eng.build_synthetic(8, what=7)
        ids = [int(v) for v in np.random.default_rng(2).integers(0, cfg.vocab, 10)]
        lg = eng.empty(cfg.vocab, torch.float32)
        ref = []
        for pos, tok in enumerate(ids):
            eng.forward_token(tok, pos, lg)
            ref.append(eng.to_host(lg).copy())
        prompt = np.array(ids[:6], np.int32)
        stream3 = list(eng.generate(prompt, 12))
        eng.set_moe_fused(True)
        for pos, tok in enumerate(ids):
            eng.forward_token(tok, pos, lg)
            got = eng.to_host(lg)
            assert bits_equal(got, ref[pos]), (pos, first_mismatch(got, ref[pos]))
        assert list(eng.generate(prompt, 12)) == stream3
        eng.status()
    finally:
        eng.close()


def test_fused_golden_tiny_model(gpu, oracle, monkeypatch):
    """Small widths (2 groups per row, 4 + 2 row blocks): picchio's recorded
    moe_forward outputs and greedy stream with the single-launch layer."""
    import torch
    import picchio_amd as pa
    from test_oracle import cfg_from, load
    z = load("model_tiny.npz")
    cfg = cfg_from(z)
    model = oracle.model_build(cfg, int(z["seed"]), 0)
    eng = pa.Engine(cfg)
    try:
        upload_model(eng, oracle, model, cfg)
        eng.set_moe_fused(True)
        od = eng.empty(cfg.hidden, torch.float32)
        for layer in range(2):
            for t in range(z["moe_x"].shape[1]):
                eng.moe_forward(layer, eng.to_dev(z["moe_x"][layer, t]), od)
                assert rel_l2(eng.to_host(od), z["moe_out"][layer, t]) < REL_L2_TOL, (layer, t)
        prompt = [int(v) for v in z["prompt"]]
        monkeypatch.setenv("PREFILL_BATCH", "1")          # position by position
        assert list(eng.generate(prompt, len(z["stream"]))) == [int(v) for v in z["stream"]]
        monkeypatch.setenv("PREFILL_BATCH", "4")          # forward_prefill in chunks of 4
        assert list(eng.generate(prompt, len(z["prefill_stream"]))) == [int(v) for v in z["prefill_stream"]]
        eng.status()
    finally:
        eng.close()
        oracle.model_free(model)
