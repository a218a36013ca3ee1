"""GPU parity of the expert-grouped MoE on the matrix cores
(pk_moe_forward_grouped, pk_quantize_act_i8x3, pk_set_grouped_f16).

Int8 limbs (pk_set_grouped_f16(e, 0)): activation limbs and exponents
bit-exact with the oracle's restatement; down-projection outputs bit-exact
with the oracle's restatement of the same integer arithmetic given the same
activations; SwiGLU activations within relative L2 1e-6 of it (the device
expf may differ in the last bit).
Half-precision pairs (the default): every pair's SwiGLU activations and
down outputs within relative L2 2e-6 of picchio's fp32 GEMV (matmul_i4_gs)
on the same inputs; the MFMA sums in its own order, so no bit-exact bar.
Both: per-token MoE outputs within relative L2 1e-5 of picchio's fp32
arithmetic (forward_prefill's expert order, oracle expert_apply), i.e. an
order of magnitude inside the north star's 1e-4.
"""
import numpy as np
import pytest

from helpers import REL_L2_TOL, bits_equal, first_mismatch, rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def grp(gpu, oracle):
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=8, ctx_len=16, vocab=64)
    model = oracle.model_build(cfg, 777, 0)
    eng = pa.Engine(cfg)
    for e in range(cfg.n_experts):
        eng.store_expert(0, e, *oracle.expert_arrays(model, 0, e, cfg))
    D, E = cfg.hidden, cfg.n_experts
    eng.store_router(0, oracle.tensor(model, 6, 0, E * D), oracle.tensor(model, 7, 0, E))
    yield cfg, model, eng
    eng.close()
    oracle.model_free(model)


def test_act_limbs_bitexact(grp, oracle):
    import torch
    cfg, model, eng = grp
    rng = np.random.default_rng(5)
    x = rng.standard_normal((9, 2880)).astype(np.float32)
    x[1] = 0.0                                     # all-zero row: k = 0, limbs 0
    x[2] *= 1e-20                                  # tiny values
    x[3] *= 1e20                                   # large values
    x[4, :] = 0.5
    x[4, 7] = 1.0                                  # max an exact power of two
    x[5] = np.round(x[5] * 64) / 64                # many ties after scaling
    x[6, 100] = -np.abs(x[6]).max() * 2            # negative extreme
    limbs = eng.empty((3, 9, 2880), torch.int8)
    exps = eng.empty(9, torch.int32)
    eng.quantize_act_i8x3(eng.to_dev(x), limbs, exps)
    l_ref = np.empty((3, 9, 2880), np.int8)
    e_ref = np.empty(9, np.int32)
    oracle.act_limbs(x, 9, 2880, l_ref, e_ref)
    assert np.array_equal(eng.to_host(exps), e_ref)
    assert np.array_equal(eng.to_host(limbs), l_ref)
    L = l_ref.astype(np.int64)
    A = L[0] * 16384 + L[1] * 128 + L[2]
    assert np.abs(A).max() <= 1 << 20 and l_ref.min() >= -64 and l_ref.max() <= 64
    back = A * np.exp2(e_ref.astype(np.float64) - 20)[:, None]
    scale = np.abs(x).max(axis=1, keepdims=True).astype(np.float64)
    assert np.all(np.abs(back - x) <= scale * 2.0 ** -20 + 1e-45)


def _routing(eng, cfg, xd, T):
    import torch
    sd = eng.empty((T, cfg.topk), torch.int32)
    wd = eng.empty((T, cfg.topk), torch.float32)
    out = eng.empty((T, cfg.hidden), torch.float32)
    eng.moe_forward_batch(0, xd, out, sd, wd)
    return sd, wd, out


def _grouped_run(eng, cfg, x, f16):
    import torch
    D, K, half = cfg.hidden, cfg.topk, cfg.moe_inter // 2
    T = x.shape[0]
    xd = eng.to_dev(x)
    sd, wd, out_exact = _routing(eng, cfg, xd, T)
    out = eng.empty((T, D), torch.float32)
    act = eng.empty((T * K, half), torch.float32)
    eo = eng.empty((T * K, D), torch.float32)
    eng.set_grouped_f16(f16)
    try:
        eng.moe_forward_grouped(0, xd, out, sd, wd, act, eo)
    finally:
        eng.set_grouped_f16(True)
    return tuple(eng.to_host(t) for t in (sd, wd, out, act, eo, out_exact))


def _check_tokens(cfg, model, oracle, x, sel, w, out, out_exact):
    """Per-token outputs against picchio's fp32 arithmetic in the batch's expert order."""
    D, K = cfg.hidden, cfg.topk
    rank = {}
    for e in sel.ravel():
        rank.setdefault(int(e), len(rank))
    worst = 0.0
    for t in range(0, x.shape[0], 9):
        acc = np.zeros(D, np.float32)
        for k in sorted(range(K), key=lambda k: rank[int(sel[t, k])]):
            oracle.expert_apply(model, 0, int(sel[t, k]), x[t], acc, float(w[t, k]))
        err = rel_l2(out[t], acc)
        worst = max(worst, err)
        assert err < 1e-5, (t, err)
    assert rel_l2(out, out_exact) < 1e-5
    return worst


def test_grouped_parity(grp, oracle):
    cfg, model, eng = grp
    D, K, half = cfg.hidden, cfg.topk, cfg.moe_inter // 2
    T = 100                                        # 400 pairs over 8 experts: several tiles each
    x = np.random.default_rng(6).standard_normal((T, D)).astype(np.float32)
    sel, w, out, act, eo, out_exact = _grouped_run(eng, cfg, x, False)

    # integer path restated: a sample of (token, expert) pairs
    xl = np.empty((3, T, D), np.int8)
    xe = np.empty(T, np.int32)
    oracle.act_limbs(x, T, D, xl, xe)
    experts = {}
    for p in [0, 1, 7, 57, 131, 250, 333, 399]:
        t, k = divmod(p, K)
        e = int(sel[t, k])
        if e not in experts:
            experts[e] = oracle.expert_arrays(model, 0, e, cfg)
        gq, gs, dq, ds, gb, db = experts[e]
        y = np.empty(cfg.moe_inter, np.float32)
        oracle.mfma_matvec(gq, gs, gb, cfg.moe_inter, D, xl[0, t], xl[1, t], xl[2, t], int(xe[t]), y)
        a_ref = y.copy()
        oracle.swiglu_clamped(a_ref, cfg.moe_inter, cfg.swiglu_limit, cfg.swiglu_alpha)
        assert rel_l2(act[p], a_ref[:half]) < 1e-6, p
        al = np.empty((3, 1, half), np.int8)
        ae = np.empty(1, np.int32)
        oracle.act_limbs(np.ascontiguousarray(act[p]), 1, half, al, ae)
        eo_ref = np.empty(D, np.float32)
        oracle.mfma_matvec(dq, ds, db, D, half, al[0, 0], al[1, 0], al[2, 0], int(ae[0]), eo_ref)
        assert bits_equal(eo[p], eo_ref), (p, first_mismatch(eo[p], eo_ref))

    worst = _check_tokens(cfg, model, oracle, x, sel, w, out, out_exact)
    print(f"grouped (int8 limbs) vs fp32 reference: worst token rel-L2 {worst:.2e}")


@pytest.mark.parametrize("T", [100, 7, 300])
def test_grouped_f16_parity(grp, oracle, T):
    """The half-precision pair arithmetic against picchio's fp32 GEMV, per
    pair: T = 100 (tiles of 64 and partial halves), 7 (every tile one
    32-pair half), 300 (1200 pairs, full tiles)."""
    cfg, model, eng = grp
    D, K, inter, half, gs = cfg.hidden, cfg.topk, cfg.moe_inter, cfg.moe_inter // 2, cfg.group_size
    rng = np.random.default_rng(60 + T)
    x = rng.standard_normal((T, D)).astype(np.float32)
    x[0] *= 1e-3                                   # a small-magnitude row (its own exponent)
    sel, w, out, act, eo, out_exact = _grouped_run(eng, cfg, x, True)
    experts = {}
    worst_a = worst_e = 0.0
    for p in sorted({0, 1, 3, K * T // 2, K * T - 1} | set(range(5, K * T, max(1, K * T // 40)))):
        t, k = divmod(p, K)
        e = int(sel[t, k])
        if e not in experts:
            experts[e] = oracle.expert_arrays(model, 0, e, cfg)
        gq, gsc, dq, dsc, gb, db = experts[e]
        y = np.empty(inter, np.float32)
        oracle.matmul_i4_gs(y, np.ascontiguousarray(x[t]), gq, gsc, 1, D, inter, gs)
        y += gb
        oracle.swiglu_clamped(y, inter, cfg.swiglu_limit, cfg.swiglu_alpha)
        ea = rel_l2(act[p], y[:half])
        eo_ref = np.empty(D, np.float32)
        oracle.matmul_i4_gs(eo_ref, np.ascontiguousarray(act[p]), dq, dsc, 1, half, D, gs)
        eo_ref += db
        ee = rel_l2(eo[p], eo_ref)
        worst_a, worst_e = max(worst_a, ea), max(worst_e, ee)
        assert ea < 2e-6 and ee < 2e-6, (p, ea, ee)
    worst = _check_tokens(cfg, model, oracle, x, sel, w, out, out_exact)
    print(f"grouped (f16 pairs) T={T}: pair act {worst_a:.2e}, pair down {worst_e:.2e}, "
          f"worst token rel-L2 {worst:.2e}")


def test_grouped_uses_router_when_no_routing_given(grp, oracle):
    import torch
    cfg, model, eng = grp
    T = 37
    x = np.random.default_rng(8).standard_normal((T, cfg.hidden)).astype(np.float32)
    xd = eng.to_dev(x)
    _, _, out_exact = _routing(eng, cfg, xd, T)
    out = eng.empty((T, cfg.hidden), torch.float32)
    eng.moe_forward_grouped(0, xd, out)
    assert rel_l2(eng.to_host(out), eng.to_host(out_exact)) < 1e-5


def test_prefill_on_matrix_cores_matches_oracle(gpu, oracle, monkeypatch):
    """prefill_tokens with PK_PREFILL_MFMA=1 (the chunk MoE as grouped GEMMs)
    then forward_token: next id and logits as the oracle's prefill_tokens."""
    import torch
    import picchio_amd as pa
    from helpers import upload_model
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=8, ctx_len=160, vocab=1000)
    model = oracle.model_build(cfg, 99, 0)
    eng = pa.Engine(cfg)
    try:
        upload_model(eng, oracle, model, cfg)
        monkeypatch.setenv("PREFILL_BATCH", "64")
        monkeypatch.setenv("PK_PREFILL_MFMA", "1")
        prompt = np.random.default_rng(4).integers(0, cfg.vocab, 140).astype(np.int32)
        oracle.model_reset_kv(model)
        nref = oracle.prefill_tokens(model, prompt, len(prompt), 0, 64)
        assert eng.prefill_tokens(prompt) == nref
        ref = np.empty(cfg.vocab, np.float32)
        lg = eng.empty(cfg.vocab, torch.float32)
        oracle.forward_token(model, int(nref), 140, ref.ctypes.data)
        eng.forward_token(int(nref), 140, lg)
        assert rel_l2(eng.to_host(lg), ref) < REL_L2_TOL
    finally:
        eng.close()
        oracle.model_free(model)
