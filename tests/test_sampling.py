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


def test_sampler_matches_reference_fixtures(oracle):
    """The oracle against sample_logits sequences recorded from the
    reference's own function (tests/golden/sample_logits.npz, written by
    make_golden.py sampling from oracle/_ref): ids, the arrays as the
    function leaves them, the rng after each draw, for every case at V = 64
    and 700; the history is the ids drawn so far."""
    import os
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "sample_logits.npz"))
    seed = int(z["seed"])
    for ci, (t, p, k, rep) in enumerate(z["cases"]):
        for V in (64, 700):
            key = f"c{ci}_v{V}"
            st = oracle.sampler(float(t), float(p), int(k), float(rep), seed)
            for i, lg in enumerate(z[f"{key}_in"]):
                a = lg.copy()
                assert oracle.sample_logits(st, a) == z[f"{key}_ids"][i], (key, i)
                assert np.array_equal(a.view(np.uint32), z[f"{key}_out"][i].view(np.uint32)), (key, i)
                assert oracle.sampler_state(st)[0] == int(z[f"{key}_rng"][i]), (key, i)


def _draw_r(state):
    return _xorshift(state)[1]


@pytest.mark.parametrize("case", CASES)
def test_fx_variant_is_the_reference_order_up_to_4096_kept(oracle, case):
    """With at most 4096 kept entries the library's arithmetic is the
    reference's own order: po_sample_logits_fx equals po_sample_logits bit
    for bit (tokens, arrays, rng, history)."""
    t, p, k, rep = case
    rng = np.random.default_rng(3)
    for V in (64, 3000):
        a = oracle.sampler(t, p, k, rep, 91)
        b = oracle.sampler(t, p, k, rep, 91)
        for step in range(20):
            lg = (rng.standard_normal(V) * 2.0).astype(np.float32)
            x, y = lg.copy(), lg.copy()
            assert oracle.sample_logits(a, x) == oracle.sample_logits_fx(b, y)
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
        assert oracle.sampler_state(a)[0] == oracle.sampler_state(b)[0]
        assert np.array_equal(oracle.sampler_state(a)[1], oracle.sampler_state(b)[1])


@pytest.mark.parametrize("case", [(0.7, 1.0, 0, 1.0), (1.0, 0.6, 0, 1.1), (1.0, 0.9, 6000, 1.0)])
def test_fx_variant_exact_sums(oracle, case):
    """Beyond 4096 kept entries: the pick is the first index whose exact
    (rational) cumulative sum reaches the draw, the top-p cut the shortest
    descending prefix whose exact sum reaches top_p (checked with Python
    fractions, independent of the 64-bit fixed point); and the result agrees
    with the reference's float-by-float order up to that order's rounding
    (probabilities within 3e-4, a top-p cut moved by at most an entry)."""
    from fractions import Fraction
    t, p, k, rep = case
    V = 20000
    rng = np.random.default_rng(4)
    st = oracle.sampler(t, p, k, rep, 2024)
    ref = oracle.sampler(t, p, k, rep, 2024)
    worst = 0.0
    same = 0
    for step in range(12):
        lg = rng.standard_normal(V).astype(np.float32)
        state = oracle.sampler_state(st)[0]
        x, y = lg.copy(), lg.copy()
        tok = oracle.sample_logits_fx(st, x)
        tok_ref = oracle.sample_logits(ref, y)
        same += tok == tok_ref
        # the reference's float-by-float rounding can move a top-p cut by an entry
        assert int(np.sum((x != 0) != (y != 0))) <= 2, step
        nz = (y != 0) & (x != 0)
        worst = max(worst, float(np.max(np.abs(x[nz] - y[nz]) / y[nz])))
        C.memmove(st, ref, C.sizeof(ref))        # same history from here on, whichever was picked
        # the pick against exact rational prefix sums of the array left behind
        r = Fraction(float(_draw_r(state)))
        fr = [Fraction(float(v)) for v in x]
        cum = Fraction(0)
        want = None
        for i, v in enumerate(fr):
            cum += v
            if cum >= r:
                want = i
                break
        assert tok == want, (step, tok, want)
    # over this flat distribution (thousands of entries near the cut) the
    # reference's rounding flips a draw now and then; the exact sums do not
    assert same >= 9, same
    assert worst < 3e-4, worst


def test_fx_variant_top_p_cut_is_exact(oracle):
    """Top-p beyond 4096 entries: the kept set is the shortest descending
    prefix (ties by index) whose exact sum reaches top_p, the others 0."""
    from fractions import Fraction
    V = 9000
    rng = np.random.default_rng(5)
    for top_p in (0.3, 0.75, 0.999):
        st = oracle.sampler(1.0, top_p, 0, 1.0, 77)
        lg = (rng.integers(0, 40, V) * 0.05).astype(np.float32)     # many ties
        x = lg.copy()
        oracle.sample_logits_fx(st, x)
        # the probabilities before the cut: softmax with the exact sum rounded once
        e = np.exp(lg.astype(np.float64) - lg.max()).astype(np.float32)
        kept = x != 0
        order = sorted(range(V), key=lambda i: (-float(lg[i]), i))
        n_keep = int(kept.sum())
        assert all(kept[i] for i in order[:n_keep]) and not any(kept[i] for i in order[n_keep:])
        # the kept prefix reaches top_p exactly, one fewer does not (values before renormalising)
        pre = [Fraction(float(v)) for v in (e / np.float32(e.astype(np.float64).sum()))]
        s_all = sum(pre[i] for i in order[:n_keep])
        s_less = s_all - pre[order[n_keep - 1]]
        assert s_all >= Fraction(top_p) - Fraction(1, 10 ** 6)
        assert s_less < Fraction(top_p) + Fraction(1, 10 ** 6)
