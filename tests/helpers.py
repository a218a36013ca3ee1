"""Shared helpers for the parity tests."""
import numpy as np


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def first_mismatch(a, b):
    a = np.ascontiguousarray(a, np.float32).ravel()
    b = np.ascontiguousarray(b, np.float32).ravel()
    idx = np.nonzero(a.view(np.uint32) != b.view(np.uint32))[0]
    if len(idx) == 0:
        return None
    i = int(idx[0])
    return f"{len(idx)} mismatches; first at {i}: {a[i]!r} vs {b[i]!r}"


# fp32 outputs within relative L2 error 1e-4 per layer.
REL_L2_TOL = 1e-4
