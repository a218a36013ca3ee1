"""pk_moe_forward_batch_noalloc: the batched MoE on the fixed per-GPU scratch
array. Called through the C ABI, it gives the bits of pk_moe_forward_batch
(the same kernels) on two calls in a row, the second smaller; it refuses a
batch whose scratch would not fit; and it runs inside a captured HIP graph on
an engine that has never allocated batch scratch (pk_moe_forward_batch would
have to allocate there), every replay equal to the eager result."""
import ctypes as C

import numpy as np
import pytest

from helpers import bits_equal, first_mismatch

pytestmark = pytest.mark.gpu


def _call(eng, layer, xd, out, sd, wd):
    import picchio_amd as pa
    return eng.L.pk_moe_forward_batch_noalloc(eng.h, layer, pa.ptr(xd), xd.shape[0], pa.ptr(out), pa.ptr(sd),
                                              pa.ptr(wd))


def test_noalloc_matches_allocating_entry_point(gpu):
    import torch
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=32, ctx_len=16, vocab=64)
    D, K = cfg.hidden, cfg.topk
    with pa.Engine(cfg) as eng:
        eng.build_synthetic(77, what=1)
        for T, seed in [(64, 1), (17, 2)]:
            x = np.random.default_rng(seed).standard_normal((T, D)).astype(np.float32)
            xd = eng.to_dev(x)
            outs = []
            for noalloc in (True, False):
                out = eng.empty((T, D), torch.float32)
                sd = eng.empty((T, K), torch.int32)
                wd = eng.empty((T, K), torch.float32)
                if noalloc:
                    pa.check(_call(eng, 0, xd, out, sd, wd))
                else:
                    eng.moe_forward_batch(0, xd, out, sd, wd)
                outs.append((eng.to_host(out), eng.to_host(sd), eng.to_host(wd)))
            (o1, s1, w1), (o2, s2, w2) = outs
            assert np.array_equal(s1, s2), T
            assert bits_equal(w1, w2), T
            assert bits_equal(o1, o2), (T, first_mismatch(o1, o2))


def test_noalloc_refuses_too_many_tokens(gpu):
    import torch
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=32, ctx_len=16, vocab=64)
    with pa.Engine(cfg) as eng:
        eng.build_synthetic(77, what=1)
        T = 400
        xd = eng.empty((T, cfg.hidden), torch.float32)
        out = eng.empty((T, cfg.hidden), torch.float32)
        rc = eng.L.pk_moe_forward_batch_noalloc(eng.h, 0, pa.ptr(xd), T, pa.ptr(out), None, None)
        assert rc == -4, rc
        assert b"scratch" in eng.L.pk_last_error()


def test_noalloc_inside_a_captured_graph(gpu):
    import torch
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=32, ctx_len=16, vocab=64)
    D, K, T = cfg.hidden, cfg.topk, 48
    with pa.Engine(cfg) as eng:
        eng.build_synthetic(78, what=1)
        x = np.random.default_rng(3).standard_normal((T, D)).astype(np.float32)
        xd = eng.to_dev(x)
        out = eng.empty((T, D), torch.float32)
        sd = eng.empty((T, K), torch.int32)
        wd = eng.empty((T, K), torch.float32)
        eng.capture_begin()
        rc = _call(eng, 0, xd, out, sd, wd)
        g = eng.capture_end()
        pa.check(rc)
        ref = eng.empty((T, D), torch.float32)
        pa.check(_call(eng, 0, xd, ref, sd, wd))
        ref_h = eng.to_host(ref)
        for rep in range(3):
            out.zero_()
            torch.cuda.synchronize()
            eng.graph_launch(g)
            eng.sync()
            got = eng.to_host(out)
            assert bits_equal(got, ref_h), (rep, first_mismatch(got, ref_h))
            # eager work between replays: the same call on other rows
            y = np.random.default_rng(10 + rep).standard_normal((T, D)).astype(np.float32)
            tmp = eng.empty((T, D), torch.float32)
            pa.check(_call(eng, 0, eng.to_dev(y), tmp, sd, wd))
            eng.sync()
        eng.graph_destroy(g)
