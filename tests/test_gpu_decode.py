"""GPU parity of the decode path (gqa_attention, forward_token, generate)
against the oracle, on a GPT-OSS-shaped model with every width at its 20B
size (hidden 2880, 64 query / 8 KV heads of 64, experts 5760x2880 and
2880x2880) but 2 layers, 4 experts and a 2000-token vocabulary so the CPU
oracle stays fast. Layer 0 is sliding-window (128), layer 1 full causal.

Bars: fp32 outputs within relative L2 1e-4; token ids
identical wherever the reference's top-2 logit margin exceeds the fp32 noise.
"""
import numpy as np
import pytest

from helpers import REL_L2_TOL, rel_l2, upload_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dec_setup(gpu, oracle):
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=4, ctx_len=256, vocab=2000)
    model = oracle.model_build(cfg, 555, 0)
    eng = pa.Engine(cfg)
    upload_model(eng, oracle, model, cfg)
    yield cfg, model, eng
    eng.close()
    oracle.model_free(model)


def _x(oracle, cfg, i):
    x = oracle.normal(91, 1, i, 0, cfg.hidden)
    xn = np.empty_like(x)
    oracle.rmsnorm(xn, x, np.ones(cfg.hidden, np.float32), cfg.hidden, 1e-5)
    return xn


def test_gqa_attention_parity(dec_setup, oracle):
    """Sliding and full layers over positions 0..139 (crosses the 128 window)."""
    import torch
    cfg, model, eng = dec_setup
    D = cfg.hidden
    oracle.model_reset_kv(model)
    worst = 0.0
    od = eng.empty(D, torch.float32)
    for pos in range(140):
        for layer in (0, 1):
            x = _x(oracle, cfg, pos * 2 + layer)
            ref = np.empty(D, np.float32)
            oracle.gqa_attention(model, layer, x, pos, ref)
            eng.gqa_attention(layer, eng.to_dev(x), pos, od)
            err = rel_l2(eng.to_host(od), ref)
            worst = max(worst, err)
            assert err < REL_L2_TOL, (pos, layer, err)
    assert worst < 1e-5, worst


def test_gqa_attention_long_context(gpu, oracle):
    """Windows of 16, 17, 32 and 33 chunks of 128 positions (the full layer)
    and 1-2 chunks (the sliding layer) over a 4100-position synthetic
    context that the engine (pk_kv_fill_synthetic) and the oracle fill from
    the same generator streams: the chunk partials and their combine by the
    last-arriving block against gqa_attention's single pass."""
    import torch
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=4, ctx_len=4224, vocab=2000)
    model = oracle.model_build(cfg, 556, 0)
    eng = pa.Engine(cfg)
    try:
        upload_model(eng, oracle, model, cfg)
        n_ctx, seed, M = 4100, 17, (1 << 64) - 1
        eng.kv_fill_synthetic(0, n_ctx, seed)
        for layer in (0, 1):
            s = (seed * 0x9E3779B97F4A7C15 + layer * 2) & M
            oracle.model_fill_kv(model, layer, n_ctx, s, (s + 1) & M)
        D = cfg.hidden
        od = eng.empty(D, torch.float32)
        for i, pos in enumerate((2047, 2048, 4095, 4099)):
            for layer in (0, 1):
                x = _x(oracle, cfg, 700 + 2 * i + layer)
                ref = np.empty(D, np.float32)
                oracle.gqa_attention(model, layer, x, pos, ref)
                eng.gqa_attention(layer, eng.to_dev(x), pos, od)
                err = rel_l2(eng.to_host(od), ref)
                assert err < 1e-5, (pos, layer, err)
    finally:
        eng.close()
        oracle.model_free(model)


def test_replay_graph_recaptured_past_its_position_bound(gpu):
    """The replayed step graph's attention grids cover positions up to a
    bound (1024 positions, doubled as needed); a replay that goes past it
    captures the step again. Tokens across the 1024 boundary equal the
    eager forward_token chain's over the same synthetic context."""
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=4, ctx_len=2100, vocab=2000)
    eng = pa.Engine(cfg)
    try:
        eng.build_synthetic(5, what=7)
        eng.kv_fill_synthetic(0, 1000, 9)
        a = eng.decode_replay(7, 990, 8)                 # positions 990..997: bound 1023
        b = eng.decode_replay(int(a[-1]), 998, 40)       # to 1037: captured again (2047)
        c = eng.decode_replay(int(b[-1]), 1038, 10)      # within the bound
        eng.kv_fill_synthetic(0, 1000, 9)
        ref, tok = [], 7
        for pos in range(990, 1048):
            tok = eng.forward_token(tok, pos)
            ref.append(tok)
        assert list(a) + list(b) + list(c) == ref
    finally:
        eng.close()


def test_attention_one_launch_matches_two(gpu):
    """Decode attention and its output projection as one launch (the
    projection's workgroups waiting on the attention row's tagged words)
    give the same bits as the two launches: forward_token's logits over
    one-chunk and eight-chunk windows (layer 0 sliding, layer 1 full), and
    the replayed step graph's tokens; no device-side wait gave up."""
    import torch
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=4, ctx_len=2100, vocab=2000)
    eng = pa.Engine(cfg)
    try:
        eng.build_synthetic(5, what=7)
        lg = eng.empty(cfg.vocab, torch.float32)
        for n_ctx in (40, 1000):
            eng.kv_fill_synthetic(0, n_ctx, 9)
            for i in range(3):
                outs = []
                for fused in (1, 0, 1):
                    eng.set_attn_fused(fused)
                    nxt = eng.forward_token(7 + i, n_ctx + i, lg)
                    outs.append((nxt, eng.to_host(lg)))
                for nxt, v in outs[1:]:
                    assert nxt == outs[0][0], (n_ctx, i)
                    assert np.array_equal(v.view(np.uint32), outs[0][1].view(np.uint32)), (n_ctx, i)
        streams = []
        for fused in (1, 0):
            eng.set_attn_fused(fused)
            eng.kv_fill_synthetic(0, 1000, 9)
            streams.append(list(eng.decode_replay(7, 990, 12)))
        assert streams[0] == streams[1]
        eng.sync()
    finally:
        eng.close()


def test_forward_token_parity(dec_setup, oracle):
    import torch
    cfg, model, eng = dec_setup
    oracle.model_reset_kv(model)
    ids = [int(v) for v in np.random.default_rng(3).integers(0, cfg.vocab, 24)]
    lg_dev = eng.empty(cfg.vocab, torch.float32)
    ref_lg = np.empty(cfg.vocab, np.float32)
    for pos, tok in enumerate(ids):
        nxt_ref = oracle.forward_token(model, tok, pos, ref_lg.ctypes.data)
        nxt = eng.forward_token(tok, pos, lg_dev)
        lg = eng.to_host(lg_dev)
        assert rel_l2(lg, ref_lg) < REL_L2_TOL, pos
        srt = np.sort(ref_lg)[::-1]
        if srt[0] - srt[1] > 1e-4 * max(abs(srt[0]), 1e-3):
            assert nxt == nxt_ref, (pos, nxt, nxt_ref)


def test_router_trace_and_numeric_trace(dec_setup, oracle, capfd):
    """Diagnostics. pk_set_router_trace: forward_token appends each layer's
    router logits (n_layers rows per token), which agree with the oracle's
    in-order router along the same chain (po_set_router_trace) within the
    fixed-tree sum's 1e-5, with the same top-4 wherever the 4th / 5th margin
    exceeds that; a launch past the buffer's capacity is not kept. With the
    numeric trace on, forward_token prints picchio's TRACE_NUMERIC lines
    (picchio.c:251-288): stage statistics, the routing with its margin, the
    top-10 logits led by the greedy id."""
    import re
    import torch
    cfg, model, eng = dec_setup
    L, E, K = cfg.n_layers, cfg.n_experts, cfg.topk
    ids = [int(v) for v in np.random.default_rng(8).integers(0, cfg.vocab, 3)]
    tr = eng.empty(3 * L * E + E - 1, torch.float32)
    otr = np.zeros(3 * L * E, np.float32)
    oracle.model_reset_kv(model)
    eng.set_router_trace(tr)
    oracle.set_router_trace(otr.ctypes.data, otr.size)
    try:
        for pos, tok in enumerate(ids):
            eng.forward_token(tok, pos, None)
            oracle.forward_token(model, tok, pos, None)
        assert eng.router_trace_used() == 3 * L * E
        assert oracle.router_trace_used() == 3 * L * E
        eng.forward_token(ids[-1], 3, None)               # does not fit: not kept
        assert eng.router_trace_used() == 3 * L * E
    finally:
        eng.set_router_trace(None)
        oracle.set_router_trace(None, 0)
    got = eng.to_host(tr)[:3 * L * E].reshape(3 * L, E)
    ref = otr.reshape(3 * L, E)
    assert np.max(np.abs(got - ref)) < 1e-5
    for g, r in zip(got, ref):
        srt = np.sort(r)[::-1]
        if E == K or srt[K - 1] - srt[K] > 1e-5:
            assert set(np.argsort(-g)[:K]) == set(np.argsort(-r)[:K])

    capfd.readouterr()
    eng.set_numeric_trace(True)
    try:
        lg = eng.empty(cfg.vocab, torch.float32)
        nxt = eng.forward_token(ids[0], 4, lg)
    finally:
        eng.set_numeric_trace(False)
    err = capfd.readouterr().err
    assert "numeric L=-1 embedding" in err and "bad=0" in err
    for l in range(L):
        assert f"numeric L={l} post_attention" in err and f"numeric L={l} post_moe" in err
        # (the 4th / 5th margin only where the layer has a 5th expert)
        m = re.search(rf"numeric route L={l}:((?: e\d+=[^ \n]+)+)( margin4/5=(\S+))?\n", err)
        assert m, err
        assert len(re.findall(r"e\d+=", m.group(1))) == K
        assert (m.group(3) is not None) == (E > K) and (E == K or float(m.group(3)) >= 0.0)
    top = re.search(r"numeric logits bad=0 top10: (\d+)=", err)
    assert top and int(top.group(1)) == nxt, err
    assert int(np.argmax(eng.to_host(lg))) == nxt


def test_out_of_range_token_embeds_zero(dec_setup, oracle):
    """embed_token gives a zero row for ids outside the vocabulary (picchio.c:1476-1480)."""
    import torch
    cfg, model, eng = dec_setup
    oracle.model_reset_kv(model)
    ref_lg = np.empty(cfg.vocab, np.float32)
    lg_dev = eng.empty(cfg.vocab, torch.float32)
    for pos, tok in enumerate([5, cfg.vocab + 7, -1]):
        oracle.forward_token(model, tok, pos, ref_lg.ctypes.data)
        eng.forward_token(tok, pos, lg_dev)
        assert rel_l2(eng.to_host(lg_dev), ref_lg) < REL_L2_TOL


def test_generate_stream_matches_oracle(dec_setup, oracle):
    """The prompt through prefill_tokens (chunks of 64, as picchio runs it),
    then greedy decode from the replayed step graph: the oracle's stream."""
    cfg, model, eng = dec_setup
    prompt = np.random.default_rng(11).integers(0, cfg.vocab, 70).astype(np.int32)
    n = 20
    oracle.model_reset_kv(model)
    ref = [oracle.prefill_tokens(model, prompt, len(prompt), 0, 64)]
    for i in range(n - 1):
        ref.append(oracle.forward_token(model, ref[-1], len(prompt) + i, None))
    got = list(eng.generate(prompt, n))
    assert got == ref


def test_prefill_chunks_match_oracle(dec_setup, oracle, monkeypatch):
    """prefill_tokens over 150 positions in chunks of 64 (crossing the
    128-position window), then forward_token: next id and logits as the
    oracle's prefill_tokens + forward_token (the KV written by the prompt
    path is what the decode step reads)."""
    import torch
    cfg, model, eng = dec_setup
    monkeypatch.setenv("PREFILL_BATCH", "64")
    prompt = np.random.default_rng(21).integers(0, cfg.vocab, 150).astype(np.int32)
    oracle.model_reset_kv(model)
    nref = oracle.prefill_tokens(model, prompt, len(prompt), 0, 64)
    assert eng.prefill_tokens(prompt) == nref
    ref = np.empty(cfg.vocab, np.float32)
    lg = eng.empty(cfg.vocab, torch.float32)
    for i, tok in enumerate([nref, 7, 1999]):
        oracle.forward_token(model, int(tok), 150 + i, ref.ctypes.data)
        eng.forward_token(int(tok), 150 + i, lg)
        assert rel_l2(eng.to_host(lg), ref) < REL_L2_TOL, i


def test_context_full_is_an_error(dec_setup):
    import picchio_amd as pa
    cfg, model, eng = dec_setup
    with pytest.raises(pa.PkError) as ei:
        eng.forward_token(1, cfg.ctx_len, None)
    assert ei.value.code == -6


def test_reference_golden_tiny_model(gpu, oracle):
    """The GPU path against picchio's own outputs (tests/golden/model_tiny.npz,
    recorded from the reference build): moe_forward and gqa_attention outputs,
    and the greedy token stream of forward_token."""
    import os
    import torch
    import picchio_amd as pa
    from test_oracle import cfg_from, load
    z = load("model_tiny.npz")
    cfg = cfg_from(z)
    model = oracle.model_build(cfg, int(z["seed"]), 0)
    eng = pa.Engine(cfg)
    try:
        upload_model(eng, oracle, model, cfg)
        D = cfg.hidden
        od = eng.empty(D, torch.float32)
        for layer in range(2):
            for t in range(z["moe_x"].shape[1]):
                eng.moe_forward(layer, eng.to_dev(z["moe_x"][layer, t]), od)
                assert rel_l2(eng.to_host(od), z["moe_out"][layer, t]) < REL_L2_TOL, (layer, t)
        for pos in range(z["att_x"].shape[0]):
            for layer in range(2):
                eng.gqa_attention(layer, eng.to_dev(z["att_x"][pos, layer]), pos, od)
                assert rel_l2(eng.to_host(od), z["att_out"][pos, layer]) < REL_L2_TOL, (pos, layer)
        prompt = [int(v) for v in z["prompt"]]
        os.environ["PREFILL_BATCH"] = "1"            # position by position
        assert list(eng.generate(prompt, len(z["stream"]))) == [int(v) for v in z["stream"]]
        os.environ["PREFILL_BATCH"] = "4"            # forward_prefill in chunks of 4
        got = list(eng.generate(prompt, len(z["prefill_stream"])))
        assert got == [int(v) for v in z["prefill_stream"]]
    finally:
        os.environ.pop("PREFILL_BATCH", None)
        eng.close()
        oracle.model_free(model)


def test_synthetic_build_matches_oracle_model(gpu, oracle):
    """pk_engine_build_synthetic (generator + INT4 quantizer on the GPU) gives
    the model po_model_build gives on the CPU for the same seed: MoE outputs
    match an engine loaded from the oracle's tensors (the device libm may
    round about one generated weight in 1e9 differently, hence a relative
    bar rather than bits), and logits match the oracle within the fp32 bar."""
    import torch
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=4, ctx_len=32, vocab=512)
    model = oracle.model_build(cfg, 31, 0)
    a, b = pa.Engine(cfg), pa.Engine(cfg)
    try:
        a.build_synthetic(31, what=7)
        upload_model(b, oracle, model, cfg)
        D = cfg.hidden
        oa, ob = a.empty(D, torch.float32), b.empty(D, torch.float32)
        for t in range(4):
            x = _x(oracle, cfg, 500 + t)
            a.moe_forward(1, a.to_dev(x), oa)
            b.moe_forward(1, b.to_dev(x), ob)
            assert rel_l2(a.to_host(oa), b.to_host(ob)) < 1e-6
        oracle.model_reset_kv(model)
        ref = np.empty(cfg.vocab, np.float32)
        lg = a.empty(cfg.vocab, torch.float32)
        for pos, tok in enumerate([3, 77, 400, 12]):
            nref = oracle.forward_token(model, tok, pos, ref.ctypes.data)
            n = a.forward_token(tok, pos, lg)
            assert rel_l2(a.to_host(lg), ref) < REL_L2_TOL
    finally:
        a.close()
        b.close()
        oracle.model_free(model)


def test_batched_sequences_match_separate_streams(gpu, oracle, monkeypatch):
    """Three sequences with different prompts: prefill_seq into their own
    caches, then decode_batch of all three in lockstep; each stream equals
    the oracle's prefill_tokens + forward_token stream for that prompt."""
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=8, ctx_len=128, vocab=1000)
    model = oracle.model_build(cfg, 1234, 0)
    eng = pa.Engine(cfg)
    try:
        upload_model(eng, oracle, model, cfg)
        monkeypatch.setenv("PREFILL_BATCH", "64")
        eng.batch_reserve(3)
        rng = np.random.default_rng(77)
        prompts = [rng.integers(0, cfg.vocab, 40).astype(np.int32) for _ in range(3)]
        first = [eng.prefill_seq(s, prompts[s]) for s in range(3)]
        got = eng.decode_batch(first, 40, 12)
        for s in range(3):
            oracle.model_reset_kv(model)
            ref = [oracle.prefill_tokens(model, prompts[s], 40, 0, 64)]
            for i in range(12):
                ref.append(oracle.forward_token(model, ref[-1], 40 + i, None))
            assert ref[0] == first[s]
            assert list(got[:, s]) == ref[1:], s
    finally:
        eng.close()
        oracle.model_free(model)


def test_batched_sequences_over_long_contexts(gpu, oracle):
    """Three sequences, each with its own 1100-position synthetic context
    (pk_kv_fill_synthetic; the oracle's caches filled from the same
    generator streams), decoded in lockstep: every row's attention spans 9
    chunks of 128 positions on the full layer. Each stream equals the
    oracle's forward_token stream over that sequence's context."""
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=8, ctx_len=1200, vocab=1000)
    model = oracle.model_build(cfg, 4321, 0)
    eng = pa.Engine(cfg)
    try:
        upload_model(eng, oracle, model, cfg)
        n_ctx, steps, seed, M = 1100, 8, 23, (1 << 64) - 1
        eng.batch_reserve(3)
        for s in range(3):
            eng.kv_fill_synthetic(s, n_ctx, seed)
        first = [5, 17, 99]
        got = eng.decode_batch(first, n_ctx, steps)
        for s in range(3):
            oracle.model_reset_kv(model)
            for layer in range(cfg.n_layers):
                sk = (seed * 0x9E3779B97F4A7C15 + (s * 1024 + layer) * 2) & M
                oracle.model_fill_kv(model, layer, n_ctx, sk, (sk + 1) & M)
            ref, tok = [], first[s]
            for i in range(steps):
                tok = oracle.forward_token(model, tok, n_ctx + i, None)
                ref.append(tok)
            assert list(got[:, s]) == ref, s
    finally:
        eng.close()
        oracle.model_free(model)


def test_batched_decode_on_matrix_cores(gpu, oracle, monkeypatch):
    """With PK_BATCH_MFMA_MIN=16, decode_batch of 16 sequences runs the MoE
    as the expert-grouped int8 MFMA GEMM (exact activation limbs, sums in
    another order than the per-pair GEMV): each stream follows the oracle's
    forward_token while the oracle's top-2 logit margin is clear of the
    last-bit differences; a stream is compared up to its first step with a
    margin below 1e-3."""
    import picchio_amd as pa
    monkeypatch.setenv("PK_BATCH_MFMA_MIN", "16")
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=8, ctx_len=128, vocab=1000)
    model = oracle.model_build(cfg, 4321, 0)
    eng = pa.Engine(cfg)
    n_seq, n_prompt, steps = 16, 24, 8
    try:
        upload_model(eng, oracle, model, cfg)
        eng.batch_reserve(n_seq)
        rng = np.random.default_rng(99)
        prompts = [rng.integers(0, cfg.vocab, n_prompt).astype(np.int32) for _ in range(n_seq)]
        first = [eng.prefill_seq(s, prompts[s]) for s in range(n_seq)]
        got = eng.decode_batch(first, n_prompt, steps)
        compared = 0
        logits = np.empty(cfg.vocab, np.float32)
        for s in range(n_seq):
            oracle.model_reset_kv(model)
            tok = oracle.prefill_tokens(model, prompts[s], n_prompt, 0, 64)
            assert tok == first[s], s
            for i in range(steps):
                ref = oracle.forward_token(model, tok, n_prompt + i, logits.ctypes.data)
                top2 = np.sort(logits)[-2:]
                if top2[1] - top2[0] < 1e-3:
                    break
                assert got[i, s] == ref, (s, i, got[i, s], ref)
                compared += 1
                tok = ref
        assert compared >= n_seq * steps // 2, compared
    finally:
        eng.close()
        oracle.model_free(model)


def _greedy_rule(lg):
    """picchio's greedy pick (picchio.c:1555-1560): start at index 0, move on
    a strictly greater value only (a NaN at index 0 keeps 0; later NaNs never win)."""
    best = 0
    for i in range(1, lg.size):
        if lg[i] > lg[best]:
            best = i
    return best


@pytest.mark.parametrize("nan_rows", [(0,), (7,), (0, 3)])
def test_greedy_with_nan_logits(gpu, oracle, nan_rows):
    """lm_head rows made NaN: forward_token's argmax (per-block maxima) and
    decode_batch's per-row argmax both follow the reference's scan."""
    import torch
    import picchio_amd as pa
    from helpers import T_EMBED, T_LM_HEAD
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=4, ctx_len=32, vocab=600)
    model = oracle.model_build(cfg, 808, 0)
    eng = pa.Engine(cfg)
    try:
        upload_model(eng, oracle, model, cfg, globals_=False)
        D, V = cfg.hidden, cfg.vocab
        lm = oracle.tensor(model, T_LM_HEAD, 0, V * D).reshape(V, D)
        for r in nan_rows:
            lm[r] = np.nan
        eng.store_globals(oracle.tensor(model, T_EMBED, 0, V * D), lm.ravel(), oracle.tensor(model, 0, 0, D))
        lg_dev = eng.empty(V, torch.float32)
        for pos, tok in enumerate([3, 11, 5]):
            nxt = eng.forward_token(tok, pos, lg_dev)
            lg = eng.to_host(lg_dev)
            assert all(np.isnan(lg[r]) for r in nan_rows)
            assert nxt == _greedy_rule(lg), (pos, nxt, _greedy_rule(lg))
        # the batched decode's per-row argmax on the same weights
        eng.batch_reserve(2)
        got = eng.decode_batch([3, 3], 0, 2)
        if 0 in nan_rows:
            assert (got == 0).all(), got
        else:
            assert (got != nan_rows[0]).all(), got
    finally:
        eng.close()
        oracle.model_free(model)
