"""The oracle's restatement of sample_logits (picchio.c:1509-1649), pinned
against the reference's own function (oracle/_ref, where the reference tree
was present at build time) and against closed forms: the xorshift64 draw,
greedy = first maximum, top-k 1 and a tiny top-p = the maximum."""
import ctypes as C

import numpy as np
import pytest

CASES = [  # temperature, top_p, top_k, rep_penalty
    (1.0, 0.95, 50, 1.1),         # picchio's defaults (picchio.c:1510-1513)
    (0.7, 1.0, 0, 1.0),           # temperature only
    (1.3, 0.5, 0, 1.0),           # top-p only
    (0.8, 1.0, 5, 1.3),           # top-k only, with the penalty
    (0.0, 0.95, 50, 1.2),         # greedy after the penalty
    (1.0, 0.9, 1, 1.0),           # top-k 1
]


def _xorshift(state):
    m = (1 << 64) - 1
    x = state
    x ^= (x << 13) & m
    x ^= x >> 7
    x ^= (x << 17) & m
    return x, np.float32(np.float32(x >> 33) / np.float32(1 << 31))


def test_rng_closed_form(oracle):
    st = C.c_uint64(1234567890123456789)
    x = 1234567890123456789
    for _ in range(1000):
        x, r = _xorshift(x)
        assert oracle.rng_float(C.byref(st)) == r
        assert st.value == x


@pytest.mark.parametrize("case", CASES)
def test_sampler_closed_forms(oracle, case):
    t, p, k, rep = case
    rng = np.random.default_rng(1)
    for trial in range(20):
        lg = (rng.standard_normal(1000) * 3).astype(np.float32)
        st = oracle.sampler(t, p, k, 1.0, 42 + trial)      # no history: no penalty effect
        tok = oracle.sample_logits(st, lg.copy())
        if t == 0.0 or k == 1:
            assert tok == int(np.argmax(lg))               # first maximum
        else:
            assert 0 <= tok < lg.size
    lg = np.zeros(16, np.float32)
    lg[7] = 5.0
    assert oracle.sample_logits(oracle.sampler(1.0, 1e-6, 0, 1.0, 9), lg.copy()) == 7


@pytest.mark.parametrize("case", CASES)
def test_sampler_matches_reference(oracle, case):
    from oracle_ffi import reference_available, Reference
    if not reference_available():
        pytest.skip("oracle/_ref not built (no reference tree at build time)")
    ref = Reference()
    t, p, k, rep = case
    rng = np.random.default_rng(2)
    for V in (64, 5000, 201088):
        st = oracle.sampler(t, p, k, rep, 777)
        state = C.c_uint64(777)
        hist = []
        for step in range(6 if V == 201088 else 25):
            lg = (rng.standard_normal(V) * 2.5).astype(np.float32)
            a, b = lg.copy(), lg.copy()
            ta = oracle.sample_logits(st, a)
            h = np.array(hist + [0], np.int32)
            tb = ref.sample_logits(b, V, t, p, k, rep, C.byref(state), h, len(hist))
            assert ta == tb, (V, step)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (V, step)
            hist.append(tb)
