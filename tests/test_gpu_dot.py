"""GPU parity of the opt-in integer-dot expert arithmetic (v_dot8 on the
stored nibbles, inputs as exact five-digit records; not picchio's
arithmetic) against the oracle's restatement of it: records bit-identical,
the down GEMV bit-identical given the same input records, gate_up's SwiGLU
outputs within the device expf's last ulp; and the MoE layer / decode on it
within the north star's bars of picchio's fp32 arithmetic."""
import numpy as np
import pytest

from helpers import REL_L2_TOL, bits_equal, first_mismatch, rel_l2, upload_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dot_setup(gpu, oracle):
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=4, ctx_len=64, vocab=2000)
    model = oracle.model_build(cfg, 557, 0)
    eng = pa.Engine(cfg)
    upload_model(eng, oracle, model, cfg)
    yield cfg, model, eng
    eng.set_i4_dot(False)
    eng.close()
    oracle.model_free(model)


def _records(oracle, x):
    rec = np.zeros(x.size // 32 * 24, np.int32)
    oracle.act_records(np.ascontiguousarray(x, np.float32), x.size, rec)
    return rec


def test_records_bitwise(dot_setup, oracle):
    import torch
    cfg, model, eng = dot_setup
    rng = np.random.default_rng(2)
    for trial in range(4):
        x = (rng.standard_normal(2880) * np.repeat(np.exp2(rng.integers(-12, 12, 90)), 32)).astype(np.float32)
        x[32 * trial:32 * trial + 32] = 0.0
        x[100 + trial] = 2.0 ** trial
        rd = eng.empty(90 * 24, torch.int32)
        eng.act_records(eng.to_dev(x), rd)
        assert np.array_equal(eng.to_host(rd), _records(oracle, x)), trial


def test_expert_gemvs_against_restatement(dot_setup, oracle):
    import torch
    cfg, model, eng = dot_setup
    D, I2 = cfg.hidden, cfg.moe_inter // 2
    rng = np.random.default_rng(3)
    for layer, eid in ((0, 1), (1, 3)):
        gu_q4, gu_s, d_q4, d_s, gu_b, d_b = oracle.expert_arrays(model, layer, eid, cfg)
        x = rng.standard_normal(D).astype(np.float32)
        rec = _records(oracle, x)
        ids = eng.to_dev(np.array([eid], np.int32))
        act = eng.empty(I2, torch.float32)
        arec = eng.empty(cfg.moe_inter // 64 * 24, torch.int32)
        eng.expert_gate_up_dot(layer, ids, eng.to_dev(rec), act, arec)
        y = np.zeros(cfg.moe_inter, np.float32)
        oracle.i4_dot_matvec(gu_q4, gu_s, gu_b.ctypes.data, cfg.moe_inter, D, rec, y)
        g, u = y[0::2], y[1::2]
        g = np.minimum(g, np.float32(cfg.swiglu_limit))
        u = np.clip(u, -np.float32(cfg.swiglu_limit), np.float32(cfg.swiglu_limit))
        a_ref = ((u + 1) * g / (1 + np.exp(-np.float32(cfg.swiglu_alpha) * g))).astype(np.float32)
        a = eng.to_host(act)
        assert np.max(np.abs(a - a_ref) / (np.abs(a_ref) + 1e-30)) < 4e-6, (layer, eid)
        # the epilogue's records of its own outputs
        assert np.array_equal(eng.to_host(arec), _records(oracle, a))
        eo = eng.empty(D, torch.float32)
        eng.expert_down_dot(layer, ids, arec, eo)
        yd = np.zeros(D, np.float32)
        oracle.i4_dot_matvec(d_q4, d_s, d_b.ctypes.data, D, I2, _records(oracle, a), yd)
        got = eng.to_host(eo)
        assert bits_equal(got, yd), first_mismatch(got, yd)


def test_moe_layer_and_decode_within_bars(dot_setup, oracle):
    """moe_forward on the integer dot against picchio's arithmetic (the
    oracle) and the bit-exact path: within 2e-5 relative L2 (the north star:
    1e-4); greedy decode from a prompt: the oracle's stream."""
    import torch
    cfg, model, eng = dot_setup
    D = cfg.hidden
    rng = np.random.default_rng(4)
    out = eng.empty(D, torch.float32)
    worst = 0.0
    for t in range(6):
        x = rng.standard_normal(D).astype(np.float32)
        ref = np.zeros(D, np.float32)
        sel = np.zeros(cfg.topk, np.int32)
        w = np.zeros(cfg.topk, np.float32)
        oracle.moe_forward(model, t % 2, x, ref, sel, w, None)
        eng.set_i4_dot(True)
        s_dot, _ = eng.moe_forward(t % 2, eng.to_dev(x), out, want_routing=True)
        got = eng.to_host(out)
        assert list(s_dot) == list(sel)
        err = rel_l2(got, ref)
        worst = max(worst, err)
        assert err < 2e-5, (t, err)
    eng.set_i4_dot(True)
    prompt = np.random.default_rng(13).integers(0, cfg.vocab, 20).astype(np.int32)
    n = 12
    oracle.model_reset_kv(model)
    lg = np.empty(cfg.vocab, np.float32)
    stream = [oracle.prefill_tokens(model, prompt, len(prompt), 0, 64)]
    for i in range(n - 1):
        stream.append(oracle.forward_token(model, stream[-1], len(prompt) + i, None))
    got = [int(v) for v in eng.generate(prompt, n)]
    eng.set_i4_dot(False)
    assert got == stream


def test_batched_decode_on_integer_dot(gpu, oracle, monkeypatch):
    """decode_batch (the per-pair expert GEMV of several sequences, with the
    prompts' prefill chunks) on the integer-dot arithmetic: each sequence's
    stream is the oracle's prefill_tokens + forward_token stream."""
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=8, ctx_len=128, vocab=1000)
    model = oracle.model_build(cfg, 1235, 0)
    eng = pa.Engine(cfg)
    try:
        upload_model(eng, oracle, model, cfg)
        eng.set_i4_dot(True)
        monkeypatch.setenv("PREFILL_BATCH", "64")
        eng.batch_reserve(3)
        rng = np.random.default_rng(78)
        prompts = [rng.integers(0, cfg.vocab, 40).astype(np.int32) for _ in range(3)]
        first = [eng.prefill_seq(s, prompts[s]) for s in range(3)]
        got = eng.decode_batch(first, 40, 10)
        for s in range(3):
            oracle.model_reset_kv(model)
            ref = [oracle.prefill_tokens(model, prompts[s], 40, 0, 64)]
            for i in range(10):
                ref.append(oracle.forward_token(model, ref[-1], 40 + i, None))
            assert ref[0] == first[s]
            assert list(got[:, s]) == ref[1:], s
    finally:
        eng.close()
        oracle.model_free(model)


def test_expert_tiles_match_per_pair_launches(gpu, oracle, monkeypatch):
    """The batched MoE on the integer dot with pairs grouped by expert (each
    expert block loaded once per tile of up to 4 pairs) gives the per-pair
    launches' values bit for bit: 48 tokens over 8 experts, so most experts
    carry several tiles."""
    import torch
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=8, ctx_len=16, vocab=64)
    model = oracle.model_build(cfg, 99, 0)
    outs = []
    try:
        for tiles in ("1", "0"):
            monkeypatch.setenv("PK_DOT_TILES", tiles)
            eng = pa.Engine(cfg)
            try:
                upload_model(eng, oracle, model, cfg, globals_=False)
                eng.set_i4_dot(True)
                T = 48
                x = np.random.default_rng(5).standard_normal((T, cfg.hidden)).astype(np.float32)
                out = eng.empty((T, cfg.hidden), torch.float32)
                eng.moe_forward_batch(0, eng.to_dev(x), out)
                outs.append(eng.to_host(out))
            finally:
                eng.close()
    finally:
        oracle.model_free(model)
    assert bits_equal(outs[0], outs[1]), first_mismatch(outs[0].ravel(), outs[1].ravel())
