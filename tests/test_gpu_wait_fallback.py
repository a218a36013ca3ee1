"""The one-launch forms (k_moe_ffn, k_attn_oproj) hand values between
workgroups of one launch and wait for them with bounded polls. When a wait
reaches its bound (on a device shared with other work), the engine switches
to the separate launches, which wait for nothing, and redoes the call: the
results equal a normal engine's bit for bit, and pk_wait_fallbacks counts the
switch.

pk_set_poll_bound(1) forces the path from the host: the waits give up after
one poll, every wave still ends, and what a wave reads after giving up is
only ever arithmetic data (activations, rows, records), never an index.
GPT-OSS-20B widths, 2 layers (sliding window, full), 32 experts, synthetic
weights built on the GPU from one seed for both engines."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SEED = 21


def _cfg(pa):
    return pa.gptoss_cfg(n_layers=2, n_experts=32, ctx_len=512, vocab=2000)


def _engine(pa, cfg):
    eng = pa.Engine(cfg)
    eng.build_synthetic(SEED, what=7)
    return eng


def test_generate_and_replay_redone_with_separate_launches(gpu):
    import picchio_amd as pa
    cfg = _cfg(pa)
    ref, ev = _engine(pa, cfg), _engine(pa, cfg)
    try:
        prompt = (np.arange(1, 40, dtype=np.int64) * 37 % cfg.vocab).astype(np.int32)
        want = ref.generate(prompt, 24)
        ev.set_poll_bound(1)
        got = ev.generate(prompt, 24)
        print(f"generate: {ev.wait_fallbacks()} switch(es), tokens {list(got[:8])}...", flush=True)
        assert ev.wait_fallbacks() == 1
        assert list(got) == list(want)
        # the engine stays on the separate launches: a replayed continuation
        # matches and needs no further switch
        pos = len(prompt) + len(want) - 1
        want_r = ref.decode_replay(int(want[-1]), pos, 16)
        got_r = ev.decode_replay(int(got[-1]), pos, 16)
        assert list(got_r) == list(want_r)
        assert ev.wait_fallbacks() == 1
        assert ref.wait_fallbacks() == 0
    finally:
        ref.close()
        ev.close()


def test_forward_token_and_moe_forward_redone(gpu):
    import picchio_amd as pa
    import torch
    cfg = _cfg(pa)
    ref, ev = _engine(pa, cfg), _engine(pa, cfg)
    try:
        ev.set_poll_bound(1)
        lr = ref.empty(cfg.vocab, torch.float32)
        le = ev.empty(cfg.vocab, torch.float32)
        tr = te = 7
        for pos in range(6):
            tr = ref.forward_token(tr, pos, lr)
            te = ev.forward_token(te, pos, le)
            assert te == tr, pos
            assert np.array_equal(ev.to_host(le), ref.to_host(lr)), pos
        print(f"forward_token: {ev.wait_fallbacks()} switch(es)", flush=True)
        assert ev.wait_fallbacks() == 1
    finally:
        ref.close()
        ev.close()
    ref, ev = _engine(pa, cfg), _engine(pa, cfg)
    try:
        ev.set_poll_bound(1)
        x = np.random.default_rng(3).standard_normal(cfg.hidden).astype(np.float32)
        xr, xe = ref.to_dev(x), ev.to_dev(x)
        orr = ref.empty(cfg.hidden, torch.float32)
        oe = ev.empty(cfg.hidden, torch.float32)
        sr, wr = ref.moe_forward(1, xr, orr, want_routing=True)
        se, we = ev.moe_forward(1, xe, oe, want_routing=True)
        print(f"moe_forward: {ev.wait_fallbacks()} switch(es), experts {list(se)}", flush=True)
        assert ev.wait_fallbacks() == 1
        assert list(se) == list(sr) and np.array_equal(we, wr)
        assert np.array_equal(ev.to_host(oe), ref.to_host(orr))
    finally:
        ref.close()
        ev.close()
