"""The oracle's restatement of the library's opt-in integer-dot expert
arithmetic (po_act_records, po_i4_dot_matvec; not reference functions),
pinned by what the definitions fix: the records rebuild A = rint(x 2^(18-k))
with k the frexp exponent of the half-group's largest magnitude, the group
sums are the exact integer dot products, and the matvec equals the float64
product of the weights with the quantized inputs to fp32 rounding and the
unquantized product to the grid's resolution."""
import numpy as np
import pytest


def _rebuild(rec):
    """A and k of each half-group from its record (independent decoding)."""
    rec = rec.reshape(-1, 24)
    A = np.zeros((rec.shape[0], 32), np.int64)
    for i in range(5):
        for w in range(4):
            word = rec[:, 4 * i + w].astype(np.int64) & 0xffffffff
            for n in range(8):
                d = (word >> (4 * n)) & 15
                d = np.where(d >= 8, d - 16, d)
                A[:, 8 * w + n] += d * 16 ** i
    return A, rec[:, 20].astype(np.int64)


def _records(oracle, x):
    rec = np.zeros(x.size // 32 * 24, np.int32)
    oracle.act_records(np.ascontiguousarray(x, np.float32), x.size, rec)
    return rec


def test_records_rebuild_the_grid(oracle):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(32 * 40) * np.repeat(np.exp2(rng.integers(-20, 20, 40)), 32)).astype(np.float32)
    x[32 * 3:32 * 4] = 0.0                                  # an all-zero half-group: k = 0
    x[32 * 5 + 7] = 4.0                                     # maximum an exact power of two
    x[32 * 6:32 * 7] = -x[32 * 6:32 * 7]
    x[32 * 8 + 1] = np.float32(np.nextafter(np.float32(8.0), np.float32(0)))   # A rounds up to 2^18
    A, k = _rebuild(_records(oracle, x))
    xs = x.reshape(-1, 32).astype(np.float64)
    m = np.abs(xs).max(1)
    k_ref = np.where(m > 0, np.frexp(m)[1], 0)
    assert np.array_equal(k, k_ref)
    assert np.array_equal(A, np.rint(np.ldexp(xs, (18 - k_ref)[:, None])).astype(np.int64))
    assert np.abs(A).max() <= 2 ** 18 and A[8].max() == 2 ** 18
    assert not A[3].any() and k[3] == 0
    assert A[5, 7] == 2 ** 17                               # 4 = 0.5 * 2^3: k = 3


@pytest.mark.parametrize("O,I", [(8, 128), (64, 2880), (130, 640)])
def test_dot_matvec_is_the_exact_product(oracle, O, I):
    rng = np.random.default_rng(O + I)
    q4 = rng.integers(0, 256, (O, I // 2)).astype(np.uint8)
    s = rng.uniform(1e-3, 0.1, (O, I // 64)).astype(np.float32)
    bias = rng.standard_normal(O).astype(np.float32)
    x = rng.standard_normal(I).astype(np.float32)
    rec = _records(oracle, x)
    y = np.zeros(O, np.float32)
    oracle.i4_dot_matvec(q4, s, bias.ctypes.data, O, I, rec, y)
    q = np.zeros((O, I), np.int64)
    q[:, 0::2] = q4 & 15
    q[:, 1::2] = q4 >> 4
    A, k = _rebuild(rec)
    xq = (A * np.exp2(k - 18.0)[:, None]).reshape(-1)       # the quantized inputs, exactly
    w = (q - 8) * np.repeat(s.astype(np.float64), 64, axis=1)
    exact = w @ xq + bias
    assert np.max(np.abs(y - exact) / (np.abs(w) @ np.abs(xq) + np.abs(bias))) < 1e-6
    direct = w @ x.astype(np.float64) + bias
    assert np.linalg.norm(y - direct) / np.linalg.norm(direct) < 2e-5


def test_dot_matvec_catches_a_wrong_exponent(oracle):
    """A record with its exponent off by one moves the result by 2x: the
    float64 check above would fail (the test checks what it claims)."""
    rng = np.random.default_rng(9)
    O, I = 4, 64
    q4 = rng.integers(0, 256, (O, I // 2)).astype(np.uint8)
    s = np.full((O, 1), 0.05, np.float32)
    x = rng.standard_normal(I).astype(np.float32)
    rec = _records(oracle, x)
    y0 = np.zeros(O, np.float32)
    oracle.i4_dot_matvec(q4, s, None, O, I, rec, y0)
    rec[20] += 1
    rec[24 + 20] += 1
    y1 = np.zeros(O, np.float32)
    oracle.i4_dot_matvec(q4, s, None, O, I, rec, y1)
    assert np.allclose(y1, 2 * y0, rtol=1e-6)
