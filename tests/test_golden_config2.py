"""Consistency of the config-2 fixture written from picchio's own code
(tests/golden/make_golden.py config2): the recorded logits of a kept step
select that step's id by picchio's greedy rule, the margins are the top-2
gaps of those logits, and the prompt is the seeded uniform draw the GPU test
feeds. (The ids themselves are picchio's; the GPU test compares against them.)
"""
import os

import numpy as np

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config2_stream.npz")


def test_config2_fixture_is_consistent():
    z = np.load(FIXTURE, allow_pickle=False)
    V = int(z["cfg_vocab"])
    assert V == 201088 and int(z["cfg_n_layers"]) == 24 and int(z["cfg_n_experts"]) == 32
    prompt, stream, margins = z["prompt"], z["stream"], z["margins"]
    assert len(prompt) == 512 and len(stream) == 256 and len(margins) == 256
    assert np.array_equal(prompt, np.random.default_rng(int(z["seed"])).integers(0, V, 512).astype(np.int32))
    assert ((stream >= 0) & (stream < V)).all()
    assert np.isnan(margins[0]) and (margins[1:] >= 0).all()
    for k in z["logit_steps"]:
        lg = z[f"logits_step{int(k)}"]
        assert lg.shape == (V,) and np.isfinite(lg).all()
        best = int(np.argmax(lg))                   # first maximum = picchio's strict '>' scan
        assert best == int(stream[int(k)])
        top = np.sort(lg)[-2:]
        assert np.isclose(float(top[1]) - float(top[0]), float(margins[int(k)]), rtol=0, atol=1e-6)
