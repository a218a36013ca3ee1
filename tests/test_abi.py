"""The C-ABI library on the CPU: it loads, exports every entry point that
include/picchio_hip.h declares, its structs have the header's layout on the
Python side, and its argument checks return error codes (no device work)."""
import ctypes as C
import os
import re
import subprocess
import tempfile

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "picchio_hip.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(pk_[a-z0-9_]+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    import picchio_amd
    return picchio_amd.lib()


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_declared_symbols():
    import picchio_amd
    src = open(picchio_amd.__file__).read()
    bound = set(re.findall(r'"(pk_[a-z0-9_]+)"', src))
    assert set(declared_functions()) <= bound | {"pk_version", "pk_last_error"}


def _c_layout():
    prog = r"""
#include <stdio.h>
#include <stddef.h>
#include "picchio_hip.h"
#define F(T, m) printf(#T " " #m " %zu\n", offsetof(T, m));
int main(void) {
  printf("pk_cfg size %zu\n", sizeof(pk_cfg));
  printf("pk_qt_host size %zu\n", sizeof(pk_qt_host));
  printf("pk_layer_host size %zu\n", sizeof(pk_layer_host));
  F(pk_cfg, eps) F(pk_cfg, rope_original_ctx) F(pk_cfg, rope_attn_factor)
  F(pk_cfg, group_size) F(pk_cfg, lm_head_fmt) F(pk_cfg, layer_type)
  F(pk_qt_host, data) F(pk_qt_host, s) F(pk_qt_host, O) F(pk_qt_host, block_size)
  F(pk_layer_host, wq) F(pk_layer_host, wo) F(pk_layer_host, bq) F(pk_layer_host, sinks)
  F(pk_layer_host, router_bias)
  return 0;
}
"""
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "l.c")
        open(c, "w").write(prog)
        exe = os.path.join(d, "l")
        subprocess.check_call(["gcc", "-I", os.path.join(ROOT, "include"), c, "-o", exe])
        out = subprocess.check_output([exe], text=True)
    return {(a, b): int(v) for a, b, v in (l.split() for l in out.splitlines())}


def test_struct_layout_matches_header():
    import picchio_amd as pa
    lay = _c_layout()
    assert lay[("pk_cfg", "size")] == C.sizeof(pa.PkCfg)
    assert lay[("pk_qt_host", "size")] == C.sizeof(pa.PkQtHost)
    assert lay[("pk_layer_host", "size")] == C.sizeof(pa.PkLayerHost)
    for (t, m), off in lay.items():
        if m == "size":
            continue
        cls = {"pk_cfg": pa.PkCfg, "pk_qt_host": pa.PkQtHost, "pk_layer_host": pa.PkLayerHost}[t]
        assert getattr(cls, m).offset == off, (t, m)


def test_version_and_error_strings(lib):
    assert b"gfx950" in lib.pk_version()
    assert lib.pk_last_error() is not None


def test_null_arguments_are_errors_not_crashes(lib):
    import picchio_amd as pa
    h = C.c_void_p()
    assert lib.pk_engine_create(None, 0, C.byref(h)) == -1
    assert b"null" in lib.pk_last_error().lower() or lib.pk_last_error()
    for fn, args in (("pk_moe_forward", [None, 0, None, None, None, None]),
                     ("pk_forward_token", [None, 0, 0, None, None]),
                     ("pk_gqa_attention", [None, 0, None, 0, None]),
                     ("pk_expert_apply", [None, 0, 0, None, None, 1.0]),
                     ("pk_expert_gate_up", [None, 0, None, 1, None, None]),
                     ("pk_matmul_qt", [None, None, None, None, 1])):
        assert getattr(lib, fn)(*args) == -1, fn
    assert lib.pk_engine_destroy(None) in (0, -1)


def test_bad_config_is_rejected(lib):
    import picchio_amd as pa
    h = C.c_void_p()
    for kw in ({"group_size": 32}, {"hidden": 2890}, {"topk": 0}, {"head_dim": 256},
               {"n_experts": 129}):
        cfg = pa.gptoss_cfg(n_layers=1, **kw)
        rc = lib.pk_engine_create(C.byref(cfg), 0, C.byref(h))
        assert rc in (-1, -4), (kw, rc)


def test_rope_attn_factor_default():
    """picchio.c:380-381: attn_factor = 0.1 * ln(factor) + 1 for factor > 1."""
    import math
    import picchio_amd as pa
    assert abs(pa.gptoss_cfg().rope_attn_factor - (0.1 * math.log(32.0) + 1.0)) < 1e-6
    assert pa.gptoss_cfg(rope_factor=1.0).rope_attn_factor == 1.0


@pytest.mark.parametrize("n_cu", [1, 32, 64, 104, 128, 179, 180, 255, 256, 304, 512])
@pytest.mark.parametrize("gu_rb,dn_rb,k", [(90, 45, 4), (90, 45, 2), (90, 45, 1), (8, 4, 3)])
def test_moe_ffn_down_tasks_are_a_permutation(lib, n_cu, gu_rb, dn_rb, k):
    """k_moe_ffn's workgroup -> down-task placement is a permutation of the
    grid for every CU count, so every down task is taken exactly once and no
    task index is negative (device partitions report 32/64/128 CUs)."""
    grid = gu_rb * k
    out = (C.c_int * grid)()
    rc = lib.pk_moe_ffn_plan(gu_rb, dn_rb, k, n_cu, 0, out, grid)
    assert rc in (0, 1)
    got = list(out)
    assert sorted(got) == list(range(grid)), (n_cu, min(got))
    # with a CU to spare for some workgroups, the down tasks go to those first
    n2 = max(grid - n_cu, 0)
    if 0 < n2 < n_cu:
        alone = range(n2, n_cu)
        assert all(got[t] < n_cu - n2 for t in alone)


@pytest.mark.parametrize("ctx,kvh,hd", [(16, 8, 64), (128, 2, 64), (200, 3, 32), (4105, 8, 64), (1200, 1, 128)])
def test_kv_layout_k_chunks(lib, ctx, kvh, hd):
    """The device K cache layout: a permutation of the region; inside each
    128-position chunk a head's float4 column of consecutive positions is
    contiguous (one lane per position reads one contiguous run), and a
    position's four values of a column are adjacent."""
    n = ctx * kvh * hd
    off = np.zeros(n, np.int64)
    assert lib.pk_kv_layout(ctx, kvh, hd, off.ctypes.data, n) == 0
    assert np.array_equal(np.sort(off), np.arange(n))
    o = off.reshape(ctx, kvh, hd // 4, 4)
    assert np.all(np.diff(o, axis=3) == 1)
    for c0 in range(0, ctx, 128):
        cs = min(128, ctx - c0)
        blk = o[c0:c0 + cs, :, :, 0]                       # [pos][head][column]
        assert np.all(np.diff(blk, axis=0) == 4)           # neighbouring positions 16 bytes apart
        assert blk.min() == c0 * kvh * hd and blk.max() == (c0 + cs) * kvh * hd - 4
        assert np.all(np.diff(blk[0].reshape(-1)) == 4 * cs)   # columns, then heads, cs positions apart


def test_kv_layout_checks_arguments(lib):
    out = np.zeros(16, np.int64)
    assert lib.pk_kv_layout(0, 8, 64, out.ctypes.data, 16) < 0
    assert lib.pk_kv_layout(4, 1, 6, out.ctypes.data, 16) < 0         # head_dim not a multiple of 4
    assert lib.pk_kv_layout(4, 1, 8, out.ctypes.data, 16) < 0         # too few outputs


def test_moe_ffn_plan_checks_arguments(lib):
    out = (C.c_int * 4)()
    assert lib.pk_moe_ffn_plan(0, 45, 4, 256, 0, None, 0) == -1
    assert lib.pk_moe_ffn_plan(90, 45, 4, 0, 0, None, 0) == -1
    assert lib.pk_moe_ffn_plan(90, 45, 4, 256, 0, out, 4) == -1   # too few outputs


@pytest.mark.parametrize("W", [256, 240, 304, 200])
@pytest.mark.parametrize("K", [4, 3, 2])
def test_moe_balanced_ranges_partition_the_tiles(lib, W, K):
    """The balanced experts launch's ranges (the same function the kernel
    evaluates): each workgroup's gate_up and down ranges are contiguous and
    together cover every (item, row block, group) tile once; down ranges
    start and end on thirds of a row block; every workgroup holds about the
    same number of tiles; no row block spans more than two workgroups."""
    gu_rb, ng, dn_rb = 90, 45, 45
    out = (C.c_int * (4 * W))()
    ok = lib.pk_moe_bal_plan(K, gu_rb, ng, dn_rb, ng, W, out, 4 * W)
    r = np.array(list(out)).reshape(W, 4)
    Ug, Ud = K * gu_rb * ng, K * dn_rb * ng
    assert r[0, 0] == 0 and r[0, 2] == 0 and r[-1, 1] == Ug and r[-1, 3] == Ud
    assert np.all(r[1:, 0] == r[:-1, 1]) and np.all(r[1:, 2] == r[:-1, 3])
    assert np.all(r[:, 2] % 15 == 0) and np.all(r[:, 3] % 15 == 0)
    tot = (r[:, 1] - r[:, 0]) + (r[:, 3] - r[:, 2])
    assert tot.max() - tot.min() <= 1
    if ok == 1:
        for lo, hi, NG in ((0, 1, ng), (2, 3, ng)):
            owners = {}
            for c in range(W):
                for u in (r[c, lo], r[c, hi] - 1):
                    if r[c, hi] > r[c, lo]:
                        owners.setdefault(u // NG, set()).add(c)
            for R, cs in owners.items():
                assert max(cs) - min(cs) <= 1, (R, cs)


def test_moe_balanced_plan_refuses_what_does_not_fit(lib):
    # 128 CUs: ~190 tiles per workgroup, beyond the kernel's 80 + 48 slots
    assert lib.pk_moe_bal_plan(4, 90, 45, 45, 45, 128, None, 0) == 0
    # a down input that does not split in thirds
    assert lib.pk_moe_bal_plan(4, 90, 45, 45, 44, 256, None, 0) == 0
    assert lib.pk_moe_bal_plan(0, 90, 45, 45, 45, 256, None, 0) == -1
