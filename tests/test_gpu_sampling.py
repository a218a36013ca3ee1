"""GPU parity of the device sampler (pk_sample_logits, and the decode step's
draw) against the oracle's restatement of sample_logits
(picchio.c:1509-1649), itself pinned bitwise to the reference's function.

Bars: token ids identical; the xorshift64 state and the repetition-penalty
history identical; the array left behind identical in which entries are 0,
bitwise after a greedy pick (penalised logits: correctly rounded divisions
and products), and within 4e-6 relative elsewhere: the device expf may
differ from the host libm in the last ulp, and the sums follow the
reference's order exactly, so a few ulps is all that can differ. A draw
lands within those few ulps of a boundary with probability about 1e-6.
"""
import ctypes as C

import numpy as np
import pytest

from test_sampling import CASES

pytestmark = pytest.mark.gpu

PROB_RTOL = 4e-6


def _put(eng, dev, x):
    """Host array into a device tensor on the engine's stream, then wait."""
    import torch
    with torch.cuda.stream(eng.stream):
        dev.copy_(torch.from_numpy(x))
    eng.stream.synchronize()


@pytest.fixture(scope="module")
def samp_eng(gpu):
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=4, ctx_len=16, vocab=201088)
    eng = pa.Engine(cfg)
    yield eng
    eng.close()


def _check_draws(eng, oracle, case, V, draws, logits_fn, seed=777, fast=False):
    """fast: the library's exact-sum option against the oracle's restatement
    of that arithmetic (po_sample_logits_fx); else the reference's order
    against po_sample_logits."""
    import torch
    t, p, k, rep = case
    eng.set_sampling_fast_sums(fast)
    eng.set_sampling(t, p, k, rep, seed)
    st = oracle.sampler(t, p, k, rep, seed)
    draw = oracle.sample_logits_fx if fast else oracle.sample_logits
    dev = eng.empty(V, torch.float32)
    for step in range(draws):
        lg = logits_fn(step)
        ref = lg.copy()
        tok_ref = draw(st, ref)
        _put(eng, dev, lg)
        tok = eng.sample_logits(dev, V)
        got = eng.to_host(dev)
        assert tok == tok_ref, (case, V, step, tok, tok_ref)
        rng, hist = eng.sampler_state()
        rng_ref, hist_ref = oracle.sampler_state(st)
        assert rng == rng_ref, (case, V, step)
        assert np.array_equal(hist, hist_ref), (case, V, step)
        if t < 1e-6:
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (case, V, step)
        else:
            assert np.array_equal(got == 0, ref == 0), (case, V, step)
            assert np.allclose(got, ref, rtol=PROB_RTOL, atol=0), (case, V, step,
                                                                   float(np.max(np.abs(got - ref))))
    eng.set_sampling_fast_sums(False)


@pytest.mark.parametrize("case", CASES)
def test_sampler_matches_oracle(samp_eng, oracle, case):
    """picchio's defaults and five other settings, at vocabularies 64, 5000
    and GPT-OSS's 201088, with the state carried over draws (history grows,
    the penalty applies to earlier picks)."""
    rng = np.random.default_rng(5)
    for V, draws in ((64, 30), (5000, 20), (201088, 8)):
        _check_draws(samp_eng, oracle, case, V, draws,
                     lambda s: (rng.standard_normal(V) * 2.5).astype(np.float32))


def test_sampler_ties(samp_eng, oracle):
    """Few distinct logit values: ties at the top-k threshold stay, and
    equal probabilities sort by index in the top-p cut."""
    rng = np.random.default_rng(6)
    for case in ((1.0, 0.6, 40, 1.0), (0.9, 0.3, 0, 1.0), (1.0, 0.95, 50, 1.2)):
        _check_draws(samp_eng, oracle, case, 5000, 15,
                     lambda s: (rng.integers(0, 6, 5000) * 0.75).astype(np.float32))


def test_sampler_top_k_paths(samp_eng, oracle):
    """Top-k whose threshold bucket (same sign and exponent) holds more than
    the 4096 candidates LDS takes: the selection stays in global memory; and a
    threshold of exactly 0 with -0.0 entries, which the reference keeps
    (-0.0 < 0 is false) although their keys sort below +0."""
    rng = np.random.default_rng(11)
    _check_draws(samp_eng, oracle, (1.0, 0.9, 50, 1.0), 201088, 3,
                 lambda s: rng.uniform(1.0, 1.999, 201088).astype(np.float32))

    def zeros(step):
        x = np.zeros(5000, np.float32)
        x[rng.choice(5000, 30, replace=False)] = rng.uniform(0.5, 3.0, 30).astype(np.float32)
        x[rng.choice(5000, 200, replace=False)] = np.float32(-0.0)
        x[:10] = -1.0
        return x
    _check_draws(samp_eng, oracle, (1.0, 1.0, 40, 1.0), 5000, 6, zeros)


def test_sampler_large_top_p_set(samp_eng, oracle):
    """Top-p without top-k over a flat vocabulary: the cut lies tens of
    thousands of entries down the descending order, so the candidates are
    sorted chunk after chunk (radix select of each chunk's bound, LDS sort)
    with the running sum carried across; and a top-k of 20000 (more kept
    entries than the LDS path holds)."""
    rng = np.random.default_rng(7)
    _check_draws(samp_eng, oracle, (1.0, 0.9, 0, 1.0), 201088, 3,
                 lambda s: (rng.standard_normal(201088) * 0.3).astype(np.float32))
    _check_draws(samp_eng, oracle, (1.0, 0.5, 20000, 1.0), 201088, 3,
                 lambda s: (rng.standard_normal(201088) * 0.3).astype(np.float32))


@pytest.mark.parametrize("case", [(0.7, 1.0, 0, 1.0), (1.3, 0.5, 0, 1.0), (1.0, 0.9, 0, 1.1),
                                  (1.0, 0.95, 50, 1.1)])
def test_sampler_fast_sums(samp_eng, oracle, case):
    """The exact-sum option against the oracle's restatement of it (which
    equals the reference's order up to 4096 kept entries), at 5000 and
    201088 entries, with ties in the second half of the draws."""
    rng = np.random.default_rng(10)
    for V, draws in ((5000, 12), (201088, 6)):
        _check_draws(samp_eng, oracle, case, V, draws,
                     lambda s: ((rng.standard_normal(V) * 2.0) if s < draws // 2 else
                                (rng.integers(0, 30, V) * 0.1)).astype(np.float32), fast=True)


def test_repetition_penalty_repeated_tokens(samp_eng, oracle):
    """Greedy with a penalty while one token keeps winning: the history holds
    it several times and each occurrence divides (or multiplies) again."""
    rng = np.random.default_rng(8)
    V = 5000

    def lg(step):
        x = rng.standard_normal(V).astype(np.float32)
        x[17] = 40.0                                  # wins though penalised up to 9 times
        x[23] = -3.0 if step % 2 else 3.0
        return x
    _check_draws(samp_eng, oracle, (0.0, 1.0, 0, 1.5), V, 10, lg)
    _check_draws(samp_eng, oracle, (0.8, 0.9, 8, 1.5), V, 10, lg)


def test_draw_of_zero_and_turn_clamp(samp_eng, oracle):
    """Seed 0 keeps xorshift64 at 0: every draw is r = 0, which picks token 0
    whatever its probability (the reference's first cum >= r). A TURN's
    settings are clamped as picchio clamps them and keep rng and history."""
    import torch
    V = 64
    eng = samp_eng
    eng.set_sampling(1.0, 0.9, 5, 1.0, 0)
    lg = np.zeros(V, np.float32)
    lg[40] = 9.0
    dev = eng.empty(V, torch.float32)
    _put(eng, dev, lg)
    assert eng.sample_logits(dev, V) == 0
    eng.set_sampling(1.0, 1.0, 0, 1.1, 99)
    _put(eng, dev, lg)
    first = eng.sample_logits(dev, V)
    rng0, hist0 = eng.sampler_state()
    eng.set_turn_sampling(9.0, 1.5, -3)                # -> 5.0, 1.0, 0
    rng1, hist1 = eng.sampler_state()
    assert (rng1, list(hist1)) == (rng0, list(hist0)) and list(hist0) == [first]
    st = oracle.sampler(1.0, 1.0, 0, 1.1, 99)
    assert oracle.sample_logits(st, lg.copy()) == first
    C.c_float.from_buffer(st, 0).value = 5.0           # the clamped temperature
    for _ in range(5):
        x = np.random.default_rng(9).standard_normal(V).astype(np.float32)
        _put(eng, dev, x)
        assert eng.sample_logits(dev, V) == oracle.sample_logits(st, x.copy())
    eng.reset_history()
    assert len(eng.sampler_state()[1]) == 0


@pytest.fixture(scope="module")
def gen_setup(gpu, oracle):
    import picchio_amd as pa
    from helpers import upload_model
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=4, ctx_len=128, vocab=2000)
    model = oracle.model_build(cfg, 556, 0)
    eng = pa.Engine(cfg)
    upload_model(eng, oracle, model, cfg)
    yield cfg, model, eng
    eng.close()
    oracle.model_free(model)


@pytest.mark.parametrize("case", [(0.8, 0.9, 40, 1.1), (1.0, 1.0, 0, 1.0)])
def test_sampled_generation_matches_oracle(gen_setup, oracle, monkeypatch, case):
    """generate() with sampling on: the 70-token prompt in chunks of 64 (the
    penalty history seeded with the prompt, one draw per chunk, as
    prefill_tokens and forward_prefill do), then the replayed step graph
    drawing each token on the device. Reference stream: the oracle's logits
    at the chunk ends and each step, drawn by the oracle's sampler. The
    logits agree to fp32 noise (1e-4 relative), so a draw differs only when
    it falls within that of a boundary (about 1e-4 per draw)."""
    cfg, model, eng = gen_setup
    monkeypatch.setenv("PREFILL_BATCH", "64")
    t, p, k, rep = case
    prompt = np.random.default_rng(12).integers(0, cfg.vocab, 70).astype(np.int32)
    n = 16
    st = oracle.sampler(t, p, k, rep, 4242)
    if rep > 1.0:
        oracle.sampler_push_history(st, prompt, cfg.vocab)
    oracle.model_reset_kv(model)
    lg = np.empty(cfg.vocab, np.float32)
    nxt = None
    for pos, tok in enumerate(prompt):
        oracle.forward_token(model, int(tok), pos, lg.ctypes.data)
        if pos in (63, 69):
            nxt = oracle.sample_logits(st, lg.copy())
    ref = [nxt]
    for i in range(n - 1):
        oracle.forward_token(model, ref[-1], len(prompt) + i, lg.ctypes.data)
        ref.append(oracle.sample_logits(st, lg.copy()))
    eng.set_sampling(t, p, k, rep, 4242)
    try:
        got = [int(v) for v in eng.generate(prompt, n)]
        assert got == ref
        rng, hist = eng.sampler_state()
        rng_ref, hist_ref = oracle.sampler_state(st)
        assert rng == rng_ref and np.array_equal(hist, hist_ref)
    finally:
        eng.set_sampling(0.0, 1.0, 0, 1.0, 0)          # back to greedy for other users


def test_batched_decode_rejects_sampling(gen_setup):
    import picchio_amd as pa
    cfg, model, eng = gen_setup
    eng.set_sampling(1.0, 0.9, 10, 1.0, 1)
    try:
        eng.batch_reserve(2)
        with pytest.raises(pa.PkError) as ei:
            eng.decode_batch([1, 2], 0, 1)
        assert ei.value.code == -4
    finally:
        eng.set_sampling(0.0, 1.0, 0, 1.0, 0)
