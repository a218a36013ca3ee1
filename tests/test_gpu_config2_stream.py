"""BASELINE config 2 at full size: the GPT-OSS-20B-shaped model (24 layers,
32 experts, vocab 201088) from seed 2025, a 512-token prompt of uniform
random ids through prefill_tokens (chunks of 64, picchio's default), then
256 greedy steps. The expected stream and the logits of two decode steps
come from picchio's own prefill_tokens / forward_token (oracle/_ref, built
from the reference sources) on the same weights, committed as
tests/golden/config2_stream.npz by tests/golden/make_golden.py config2.

Bars: an identical greedy token stream over 256 steps;
fp32 logits of the full 201,088-row lm_head within relative L2 1e-4.
"""
import os

import numpy as np
import pytest

from helpers import REL_L2_TOL, rel_l2

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config2_stream.npz")


def _fixture():
    return np.load(FIXTURE, allow_pickle=False)


def _cfg(z):
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(ctx_len=int(z["cfg_ctx_len"]))
    for name, _ in cfg._fields_:
        if name == "layer_type":
            assert list(cfg.layer_type) == list(z["cfg_layer_type"])
        else:
            assert np.isclose(getattr(cfg, name), z[f"cfg_{name}"]), name
    return cfg


@pytest.fixture(scope="module")
def c2_engine(gpu):
    import picchio_amd as pa
    z = _fixture()
    eng = pa.Engine(_cfg(z))
    eng.build_synthetic(int(z["seed"]), what=7)
    yield z, eng
    eng.close()


@pytest.mark.parametrize("dot", [False, True], ids=["fp32-chains", "integer-dot"])
def test_config2_greedy_stream_256(c2_engine, dot):
    """pk_generate (prefill chunks + the replayed decode step): picchio's 256 ids."""
    z, eng = c2_engine
    eng.set_i4_dot(dot)
    try:
        got = [int(v) for v in eng.generate(z["prompt"], len(z["stream"]))]
    finally:
        eng.set_i4_dot(False)
    ref = [int(v) for v in z["stream"]]
    first = next((i for i, (a, b) in enumerate(zip(got, ref)) if a != b), None)
    assert first is None, (f"stream diverges at step {first}: {got[first:first + 4]} vs {ref[first:first + 4]}"
                           f" (picchio's top-2 margin there {float(z['margins'][first]):.3g})")


def test_config2_eager_logits_full_vocab(c2_engine):
    """prefill_tokens, then forward_token step by step (the eager lm_head +
    argmax path): every id equals picchio's, and the full-vocabulary logits
    of the kept steps are within relative L2 1e-4 of picchio's."""
    import torch
    z, eng = c2_engine
    prompt, ref = z["prompt"], [int(v) for v in z["stream"]]
    n_prompt = len(prompt)
    assert eng.prefill_tokens(prompt) == ref[0]
    keep = set(int(k) for k in z["logit_steps"])
    lg_dev = eng.empty(int(z["cfg_vocab"]), torch.float32)
    for k in range(1, len(ref)):
        nxt = eng.forward_token(ref[k - 1], n_prompt + k - 1, lg_dev if k in keep else None)
        assert nxt == ref[k], (k, nxt, ref[k])
        if k in keep:
            err = rel_l2(eng.to_host(lg_dev), z[f"logits_step{k}"])
            print(f"step {k}: logits rel-L2 {err:.2e}", flush=True)
            assert err < REL_L2_TOL, (k, err)
