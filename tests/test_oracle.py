"""Pins the oracle (oracle/pk_oracle.c, the CPU restatement the GPU path is
checked against) three ways, on the CPU:

1. golden vectors: outputs of picchio's own C functions (quant.h kernels,
   moe_forward, gqa_attention, RoPE/YaRN, forward_token, prefill_tokens)
   recorded by tests/golden/make_golden.py from oracle/_ref — bit-identical;
2. the reference's own known-answer tests (picchio.c:2249-2371 self-test,
   test_forward.py:95-120 component asserts);
3. what the mathematics fixes: the gs64 quantizer of convert.py:45-93
   restated in numpy, an exhaustive nibble decode, and float64 brute-force
   restatements of the INT4 GEMV, the expert FFN / router / top-k / combine,
   and sink attention with YaRN RoPE.
Where oracle/_ref is present (development container) it is also compared
live with the oracle on fresh inputs.
"""
import ctypes as C
import math
import os

import numpy as np
import pytest

from helpers import T_BK, T_BO, T_BQ, T_BV, T_SINKS, T_WK, T_WO, T_WQ, T_WV, bits_equal, rel_l2

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def cfg_from(z):
    from oracle_ffi import make_cfg
    names = [k[4:] for k in z.files if k.startswith("cfg_") and k != "cfg_layer_type"]
    c = make_cfg(**{n: z["cfg_" + n].item() for n in names})
    for i, v in enumerate(z["cfg_layer_type"]):
        c.layer_type[i] = int(v)
    return c


# ───────────────────────── 1. golden vectors ─────────────────────────

def test_golden_matmul_i4_gs(oracle):
    z = load("matmul_i4_gs.npz")
    for i in range(int(z["n"])):
        O, I, gs, S = (int(v) for v in z[f"c{i}_shape"])
        y = np.empty((S, O), np.float32)
        oracle.matmul_i4_gs(y, z[f"c{i}_x"], z[f"c{i}_q4"], z[f"c{i}_s"], S, I, O, gs)
        assert bits_equal(y, z[f"c{i}_y"]), (O, I, gs, S)


def test_golden_matmul_dense(oracle):
    z = load("matmul_dense.npz")
    for i in range(int(z["n"])):
        S, I, O = (int(v) for v in z[f"c{i}_shape"])
        x = z[f"c{i}_x"]
        for fn, args, key in ((oracle.matmul_f32, (z[f"c{i}_W"],), "yf"),
                              (oracle.matmul_q8, (z[f"c{i}_q8"], z[f"c{i}_s8"]), "y8"),
                              (oracle.matmul_i4, (z[f"c{i}_q4"], z[f"c{i}_s4"]), "y4")):
            y = np.empty((S, O), np.float32)
            fn(y, x, *args, S, I, O)
            assert bits_equal(y, z[f"c{i}_{key}"]), (key, S, I, O)


def test_golden_quantize_rows_i4(oracle):
    z = load("quantize_rows_i4.npz")
    for i in range(int(z["n"])):
        w = z[f"c{i}_w"]
        O, I = w.shape
        q4 = np.empty((O, (I + 1) // 2), np.uint8)
        s = np.empty(O, np.float32)
        oracle.quantize_rows_i4(w, O, I, q4, s)
        assert np.array_equal(q4, z[f"c{i}_q4"]) and bits_equal(s, z[f"c{i}_s"])


def test_golden_rmsnorm_softmax(oracle):
    z = load("norm_softmax.npz")
    for i in range(int(z["n"])):
        x, w = z[f"c{i}_x"], z[f"c{i}_w"]
        o = np.empty_like(x)
        oracle.rmsnorm(o, x, w, x.size, 1e-5)
        assert bits_equal(o, z[f"c{i}_rms"])
        sm = x.copy()
        oracle.softmax(sm, sm.size)
        assert bits_equal(sm, z[f"c{i}_softmax"])


def test_golden_rope_yarn(oracle):
    z = load("rope_yarn.npz")
    cfg = cfg_from(z)
    inv = np.array([oracle.yarn_inv_freq(cfg, j) for j in range(cfg.head_dim // 2)], np.float32)
    assert bits_equal(inv, z["inv_freq"])
    for i, p in enumerate(z["pos"]):
        q, k = z["q_in"][i].copy(), z["k_in"][i].copy()
        oracle.rope_apply(cfg, q, k, int(p))
        assert bits_equal(q, z["q_out"][i]) and bits_equal(k, z["k_out"][i]), int(p)


@pytest.fixture(scope="module")
def tiny(oracle):
    z = load("model_tiny.npz")
    cfg = cfg_from(z)
    model = oracle.model_build(cfg, int(z["seed"]), 0)
    yield z, cfg, model
    oracle.model_free(model)


def test_golden_moe_forward(tiny, oracle):
    z, cfg, model = tiny
    for layer in range(2):
        for t in range(z["moe_x"].shape[1]):
            out = np.empty(cfg.hidden, np.float32)
            oracle.moe_forward(model, layer, z["moe_x"][layer, t], out, None, None, None)
            assert bits_equal(out, z["moe_out"][layer, t]), (layer, t)


def test_golden_gqa_attention(tiny, oracle):
    z, cfg, model = tiny
    oracle.model_reset_kv(model)
    for pos in range(z["att_x"].shape[0]):
        for layer in range(2):
            out = np.empty(cfg.hidden, np.float32)
            oracle.gqa_attention(model, layer, z["att_x"][pos, layer], pos, out)
            assert bits_equal(out, z["att_out"][pos, layer]), (pos, layer)


def test_golden_greedy_stream(tiny, oracle):
    z, cfg, model = tiny
    prompt = [int(v) for v in z["prompt"]]
    oracle.model_reset_kv(model)
    nxt = None
    for pos, tok in enumerate(prompt):
        nxt = oracle.forward_token(model, tok, pos, None)
    got = [nxt]
    for i in range(len(z["stream"]) - 1):
        got.append(oracle.forward_token(model, got[-1], len(prompt) + i, None))
    assert got == [int(v) for v in z["stream"]]


def test_golden_prefill_stream(tiny, oracle):
    z, cfg, model = tiny
    prompt = np.ascontiguousarray(z["prompt"], np.int32)
    oracle.model_reset_kv(model)
    got = [oracle.prefill_tokens(model, prompt, len(prompt), 0, 4)]
    for i in range(len(z["prefill_stream"]) - 1):
        got.append(oracle.forward_token(model, got[-1], len(prompt) + i, None))
    assert got == [int(v) for v in z["prefill_stream"]]


def test_live_reference_matmul_i4_gs(oracle, reference):
    """Fresh shapes, oracle vs picchio's own matmul_i4_gs (dev container only)."""
    rng = np.random.default_rng(99)
    for O, I, gs, S in [(64, 2880, 64, 1), (11, 150, 64, 4), (5, 96, 16, 2)]:
        x = rng.standard_normal((S, I)).astype(np.float32)
        q4 = rng.integers(0, 256, (O, (I + 1) // 2), dtype=np.uint8)
        s = rng.random((O, (I + gs - 1) // gs)).astype(np.float32)
        a, b = np.empty((S, O), np.float32), np.empty((S, O), np.float32)
        oracle.matmul_i4_gs(a, x, q4, s, S, I, O, gs)
        reference.matmul_i4_gs(b, x, q4, s, S, I, O, gs)
        assert bits_equal(a, b)


# ─────────────── 2. the reference's own known-answer tests ───────────────

def test_kat_rmsnorm(oracle):
    x = np.array([1, 2, 3, 4], np.float32)
    o = np.empty(4, np.float32)
    oracle.rmsnorm(o, x, np.ones(4, np.float32), 4, 1e-5)
    assert abs(o[0] - 1.0 / math.sqrt(7.5)) < 1e-4                 # picchio.c:2251-2264
    assert abs(o[0] - 1.0 / math.sqrt(7.5 + 1e-5)) < 1e-5          # test_forward.py:99-101


def test_kat_softmax(oracle):
    x = np.array([1, 2, 3], np.float32)
    oracle.softmax(x, 3)
    assert abs(x.sum() - 1.0) < 1e-5 and x[2] > x[1] > x[0]        # picchio.c:2266-2280


def test_kat_matmul_f32(oracle):
    y = np.zeros((1, 2), np.float32)
    oracle.matmul_f32(y, np.array([[1, 2, 3, 4]], np.float32),
                      np.array([1, 0, 0, 0, 0, 1, 0, 0], np.float32), 1, 4, 2)
    assert abs(y[0, 0] - 1) < 1e-5 and abs(y[0, 1] - 2) < 1e-5     # picchio.c:2282-2294


def test_kat_swiglu_silu(oracle):
    # gate = 0 -> 0; gate = 1, up = 0 -> silu(1) (picchio.c:2296-2310)
    gu = np.array([0.0, 3.0, 1.0, 0.0], np.float32)
    oracle.swiglu_clamped(gu, 4, 7.0, 1.0)
    assert abs(gu[0]) < 1e-6 and abs(gu[1] - 1.0 / (1.0 + math.exp(-1.0))) < 1e-5


def test_kat_rope_pos0_identity(oracle):
    from oracle_ffi import make_cfg
    c = make_cfg(head_dim=8, n_heads=2, n_kv_heads=1, theta=10000.0, rope_factor=1.0,
                 rope_attn_factor=1.0)
    q = np.arange(1, 17, dtype=np.float32)
    k = np.arange(1, 9, dtype=np.float32)
    q0, k0 = q.copy(), k.copy()
    oracle.rope_apply(c, q, k, 0)                                  # picchio.c:2312-2339
    assert np.allclose(q, q0, atol=1e-5) and np.allclose(k, k0, atol=1e-5)


def test_kat_int4_quant_matmul(oracle):
    O, I = 4, 8                                                    # picchio.c:2341-2371
    W = ((np.arange(32, dtype=np.float32) - 16) * np.float32(0.1)).reshape(O, I)
    q4 = np.empty((O, I // 2), np.uint8)
    s = np.empty(O, np.float32)
    oracle.quantize_rows_i4(W, O, I, q4, s)
    x = np.ones((1, I), np.float32)
    yr, yq = np.empty((1, O), np.float32), np.empty((1, O), np.float32)
    oracle.matmul_f32(yr, x, W, 1, I, O)
    oracle.matmul_i4(yq, x, q4, s, 1, I, O)
    assert np.abs(yr - yq).max() <= 2.0


# ─────────────── 3. closed forms and brute force ───────────────

def np_quantize_int4(w, gs):
    """convert.py:45-93 restated in numpy: fp32 amax/7 (1e-8 floor), round
    half to even, clip [-8, 7], pack (q+8) low nibble = even column."""
    O, I = w.shape
    if gs <= 0 or gs >= I:
        bounds = [(0, I)]
    else:
        bounds = [(g, min(g + gs, I)) for g in range(0, I, gs)]
    q = np.empty((O, I), np.int16)
    scales = np.empty((O, len(bounds)), np.float32)
    for gi, (a, b) in enumerate(bounds):
        amax = np.abs(w[:, a:b]).max(axis=1)
        sc = np.where(amax > np.float32(1e-8), amax / np.float32(7.0),
                      np.float32(1e-8)).astype(np.float32)
        scales[:, gi] = sc
        q[:, a:b] = np.clip(np.round(w[:, a:b] / sc[:, None]), -8, 7)
    nib = (q + 8).astype(np.uint8)
    if I % 2:
        nib = np.concatenate([nib, np.full((O, 1), 0, np.uint8)], axis=1)
        nib[:, -1] = 0
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    return packed, scales


@pytest.mark.parametrize("O,I,gs", [(16, 2880, 64), (7, 200, 64), (5, 33, 33), (6, 101, 32),
                                    (3, 40, 0), (4, 10, 64), (2, 129, 64)])
def test_quantizer_matches_numpy_restatement(oracle, O, I, gs):
    rng = np.random.default_rng(O * 1000 + I)
    w = (rng.standard_normal((O, I)) * 0.02).astype(np.float32)
    w[0, : min(I, 64)] = 0.0                       # an all-zero group
    if O > 2:
        w[2, :5] = np.float32(3e-9)                # amax <= 1e-8 in a row's first group
    ref_p, ref_s = np_quantize_int4(w, gs)
    p, s = oracle.quant_gs(w, gs)
    assert np.array_equal(p, ref_p)
    assert bits_equal(s, ref_s)


def test_quantizer_known_answers(oracle):
    w = np.zeros((2, 64), np.float32)
    w[0, :8] = [7.0, 2.5, 3.5, -2.5, -0.5, 0.5, 1.5, -1.5]   # amax 7 -> scale exactly 1
    p, s = oracle.quant_gs(w, 64)
    assert s[0, 0] == 1.0 and s[1, 0] == np.float32(1e-8)
    # round half to even: 2.5->2, 3.5->4, -2.5->-2, +-0.5->0, 1.5->2, -1.5->-2
    assert list(p[0, :4]) == [0xAF, 0x6C, 0x88, 0x6A]
    assert np.all(p[0, 4:] == 0x88) and np.all(p[1] == 0x88)    # zero -> nibble 8


def test_int8_row_quantizer_matches_numpy_restatement(oracle):
    """convert.py:106-126: per-row fp32 amax/127 (1.0 for an all-zero row),
    round half to even, clip [-127, 127]."""
    rng = np.random.default_rng(12)
    w = (rng.standard_normal((9, 333)) * 0.05).astype(np.float32)
    w[3] = 0.0
    w[4, :3] = [127.0, 0.5, -1.5]                  # scale exactly 1: ties to even
    w[4, 3:] = 0.0
    amax = np.abs(w).max(axis=1)
    s_ref = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q_ref = np.clip(np.rint(w / s_ref[:, None]), -127, 127).astype(np.int8)
    q = np.empty_like(q_ref)
    s = np.empty(9, np.float32)
    oracle.quantize_int8_rows(w, 9, 333, q, s)
    assert np.array_equal(q, q_ref) and bits_equal(s, s_ref)
    assert list(q[4, :3]) == [127, 0, -2] and s[3] == 1.0 and np.all(q[3] == 0)


def test_nibble_decode_exhaustive(oracle):
    """Every byte value, both nibbles: matmul_i4_gs with x = identity gives
    (nib - 8) * scale exactly, low nibble = even column."""
    I = 512
    q4 = np.arange(256, dtype=np.uint8).reshape(1, 256)
    s = np.full((1, I // 64), 0.5, np.float32)
    y = np.empty((I, 1), np.float32)
    oracle.matmul_i4_gs(y, np.eye(I, dtype=np.float32), q4, s, I, I, 1, 64)
    b = np.arange(256)
    want = np.empty(I, np.float32)
    want[0::2] = ((b & 15) - 8) * 0.5
    want[1::2] = ((b >> 4) - 8) * 0.5
    assert np.array_equal(y[:, 0], want)


def dequant(q4, s, I, gs):
    lo = (q4 & 15).astype(np.float64) - 8
    hi = (q4 >> 4).astype(np.float64) - 8
    q = np.empty((q4.shape[0], q4.shape[1] * 2))
    q[:, 0::2], q[:, 1::2] = lo, hi
    q = q[:, :I]
    return q * np.repeat(s.astype(np.float64), gs, axis=1)[:, :I]


def test_matmul_i4_gs_vs_float64(oracle):
    rng = np.random.default_rng(7)
    O, I = 5760, 2880
    w = (rng.standard_normal((O, I)) * 0.02).astype(np.float32)
    p, s = oracle.quant_gs(w, 64)
    x = rng.standard_normal((1, I)).astype(np.float32)
    y = oracle.mm_i4_gs(x, p, s, O, I, 64)
    exact = dequant(p, s, I, 64) @ x[0].astype(np.float64)
    assert rel_l2(y[0], exact) < 1e-6


def np_swiglu(gu, lim, alpha):
    g, u = gu[0::2].copy(), gu[1::2].copy()
    g = np.minimum(g, lim)
    u = np.clip(u, -lim, lim)
    return (u + 1.0) * g / (1.0 + np.exp(-alpha * g))


def test_swiglu_clamps(oracle):
    gu = np.array([9.0, 9.0, 7.5, -8.0, -3.0, 0.25, 2.0, -9.0, -20.0, 5.0], np.float32)
    want = np_swiglu(gu.astype(np.float64), 7.0, 1.702)
    oracle.swiglu_clamped(gu, gu.size, 7.0, 1.702)
    assert np.allclose(gu[: gu.size // 2], want, rtol=1e-6, atol=1e-7)


def test_argmax_first_max(oracle):
    assert oracle.argmax(np.array([1, 3, 3, 2], np.float32), 4) == 1   # picchio.c:1557-1559
    assert oracle.argmax(np.array([-5, -5], np.float32), 2) == 0


def test_moe_layer_vs_float64(tiny, oracle):
    """Router dot + bias, top-k by repeated strict argmax (lowest index on
    ties), softmax of the k logits, routed_scale, expert FFN with clamped
    SwiGLU, combine in routing order — float64, from the dequantized weights."""
    z, cfg, model = tiny
    D, E, K, gs = cfg.hidden, cfg.n_experts, cfg.topk, cfg.group_size
    half = cfg.moe_inter // 2
    from helpers import T_ROUTER, T_ROUTER_B
    R = oracle.tensor(model, T_ROUTER, 0, E * D).reshape(E, D).astype(np.float64)
    rb = oracle.tensor(model, T_ROUTER_B, 0, E).astype(np.float64)
    experts = []
    for e in range(E):
        gq, gsc, dq, dsc, gb, db = oracle.expert_arrays(model, 0, e, cfg)
        experts.append((dequant(gq, gsc, D, gs), dequant(dq, dsc, half, gs), gb, db))
    rng = np.random.default_rng(3)
    for t in range(6):
        x = rng.standard_normal(D).astype(np.float32)
        out = np.empty(D, np.float32)
        sel = np.empty(K, np.int32)
        w = np.empty(K, np.float32)
        lg = np.empty(E, np.float32)
        oracle.moe_forward(model, 0, x, out, sel, w, lg)
        x64 = x.astype(np.float64)
        lg64 = R @ x64 + rb
        assert np.allclose(lg, lg64, rtol=1e-5, atol=1e-6)
        order = sorted(range(E), key=lambda e: (-lg[e], e))[:K]
        assert list(sel) == order
        ws = np.exp(lg64[sel] - lg64[sel].max())
        ws /= ws.sum()
        assert np.allclose(w, ws, rtol=1e-5)
        acc = np.zeros(D)
        for k in range(K):
            gw, dw, gb, db = experts[sel[k]]
            a = np_swiglu(gw @ x64 + gb, cfg.swiglu_limit, cfg.swiglu_alpha)
            acc += ws[k] * cfg.routed_scale * (dw @ a + db)
        assert rel_l2(out, acc) < 1e-5


def np_yarn_inv_freq(cfg, j):
    dim = cfg.head_dim
    extrap = 1.0 / cfg.theta ** (2.0 * j / dim)
    if cfg.rope_factor <= 1.0:
        return extrap
    lg = math.log(cfg.theta)
    low = dim * math.log(cfg.rope_original_ctx / (cfg.rope_beta_fast * 2 * math.pi)) / (2 * lg)
    high = dim * math.log(cfg.rope_original_ctx / (cfg.rope_beta_slow * 2 * math.pi)) / (2 * lg)
    if cfg.rope_truncate:
        low, high = math.floor(low), math.ceil(high)
    low, high = max(low, 0.0), min(high, dim - 1.0)
    if low == high:
        high += 0.001
    ramp = min(max((j - low) / (high - low), 0.0), 1.0)
    return extrap / cfg.rope_factor * ramp + extrap * (1.0 - ramp)


def test_yarn_inv_freq_closed_form(oracle):
    from oracle_ffi import make_cfg
    for kw in ({}, {"rope_truncate": 1}, {"rope_factor": 1.0}, {"head_dim": 128}):
        c = make_cfg(**kw)
        for j in range(c.head_dim // 2):
            assert math.isclose(oracle.yarn_inv_freq(c, j), np_yarn_inv_freq(c, j),
                                rel_tol=2e-6), (kw, j)


class Attn64:
    """gqa_attention (picchio.c:504-623) in float64: projections + bias, YaRN
    RoPE (angle pos*inv_freq rounded to fp32 as the reference computes it),
    KV store, window on sliding layers, sink softmax, output projection."""

    def __init__(self, oracle, model, cfg):
        D, H, KVH, hd = cfg.hidden, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        self.c, self.L = cfg, []
        inv = np.array([oracle.yarn_inv_freq(cfg, j) for j in range(hd // 2)], np.float32)
        self.inv = inv
        for l in range(cfg.n_layers):
            t = lambda k, n: oracle.tensor(model, k, l, n).astype(np.float64)
            self.L.append(dict(wq=t(T_WQ, H * hd * D).reshape(H * hd, D),
                               wk=t(T_WK, KVH * hd * D).reshape(KVH * hd, D),
                               wv=t(T_WV, KVH * hd * D).reshape(KVH * hd, D),
                               wo=t(T_WO, D * H * hd).reshape(D, H * hd),
                               bq=t(T_BQ, H * hd), bk=t(T_BK, KVH * hd), bv=t(T_BV, KVH * hd),
                               bo=t(T_BO, D), sinks=t(T_SINKS, H), K={}, V={}))

    def rope(self, v, heads, pos):
        hd = self.c.head_dim
        ang = (np.float32(pos) * self.inv).astype(np.float64)
        cs = np.cos(ang) * self.c.rope_attn_factor
        sn = np.sin(ang) * self.c.rope_attn_factor
        v = v.reshape(heads, hd).copy()
        a, b = v[:, : hd // 2].copy(), v[:, hd // 2:].copy()
        v[:, : hd // 2] = a * cs - b * sn
        v[:, hd // 2:] = a * sn + b * cs
        return v

    def __call__(self, layer, x, pos):
        c, P = self.c, self.L[layer]
        H, KVH, hd = c.n_heads, c.n_kv_heads, c.head_dim
        x = x.astype(np.float64)
        q = self.rope(P["wq"] @ x + P["bq"], H, pos)
        k = self.rope(P["wk"] @ x + P["bk"], KVH, pos)
        P["K"][pos], P["V"][pos] = k, (P["wv"] @ x + P["bv"]).reshape(KVH, hd)
        start = max(0, pos - c.sliding_window + 1) if c.layer_type[layer] == 0 else 0
        Ks = np.stack([P["K"][t] for t in range(start, pos + 1)])
        Vs = np.stack([P["V"][t] for t in range(start, pos + 1)])
        o = np.empty((H, hd))
        for h in range(H):
            kv = h // (H // KVH)
            s = Ks[:, kv] @ q[h] / math.sqrt(hd)
            m = max(P["sinks"][h], s.max())
            e = np.exp(s - m)
            o[h] = (e / (math.exp(P["sinks"][h] - m) + e.sum())) @ Vs[:, kv]
        return P["wo"] @ o.ravel() + P["bo"]


def test_gqa_attention_vs_float64(tiny, oracle):
    z, cfg, model = tiny
    ref = Attn64(oracle, model, cfg)
    oracle.model_reset_kv(model)
    rng = np.random.default_rng(8)
    for pos in range(24):                       # crosses the 16-position window
        for layer in range(2):
            x = rng.standard_normal(cfg.hidden).astype(np.float32)
            out = np.empty(cfg.hidden, np.float32)
            oracle.gqa_attention(model, layer, x, pos, out)
            assert rel_l2(out, ref(layer, x, pos)) < 1e-5, (pos, layer)


def test_sink_minus_inf_is_plain_softmax(oracle):
    """With every sink at -inf the sink term vanishes: plain causal softmax."""
    z = load("model_tiny.npz")
    cfg = cfg_from(z)
    model = oracle.model_build(cfg, 77, 0)
    try:
        for l in range(cfg.n_layers):
            p = oracle.model_tensor(model, T_SINKS, l, None)
            arr = np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(cfg.n_heads,))
            arr[:] = -np.inf
        ref = Attn64(oracle, model, cfg)
        oracle.model_reset_kv(model)
        rng = np.random.default_rng(9)
        for pos in range(6):
            x = rng.standard_normal(cfg.hidden).astype(np.float32)
            out = np.empty(cfg.hidden, np.float32)
            oracle.gqa_attention(model, 1, x, pos, out)
            assert rel_l2(out, ref(1, x, pos)) < 1e-5
    finally:
        oracle.model_free(model)


# ── the grouped MFMA path's arithmetic (not a reference function) ──
# po_act_limbs / po_mfma_matvec restate what the library's int8 matrix-core
# prefill computes. They are pinned here by what the mathematics fixes: the
# exponent's definition, limb ranges, the rounding bound and ties-to-even of
# the scaled grid, exactness on grid points, and a float64 brute force with
# exact int64 group sums for the GEMV. A wrong shift, sign, nibble order or
# limb weight fails one of these.

def _limb_rows():
    rng = np.random.default_rng(71)
    cols = 192
    x = rng.standard_normal((10, cols)).astype(np.float32)
    x[1] = 0.0                                          # all zero: k = 0, limbs 0
    x[2] *= np.float32(1e-30)                           # tiny magnitudes
    x[3] *= np.float32(1e30)                            # huge magnitudes
    x[4] = np.float32(0.25)
    x[4, 5] = np.float32(1.0)                           # max an exact power of two: k = 1
    k5 = 3                                              # a row on the grid of exponent 3
    j = rng.integers(-(1 << 20), 1 << 20, cols)
    j[0] = 1 << 20 - 1
    x[5] = (j * 2.0 ** (k5 - 20)).astype(np.float32)
    x[5, 0] = np.float32(7.5)                           # max in [4, 8): k = 3
    half = rng.integers(-(1 << 18), 1 << 18, cols) + 0.5  # ties on the grid of x[6]
    x[6] = (half * 2.0 ** (2 - 20)).astype(np.float32)
    x[6, 0] = np.float32(3.0)                           # max in [2, 4): k = 2
    x[7, :] = np.float32(-5.0)                          # negative extreme, constant row
    # limb boundaries (k = 0, step 2^-20): A = 2^20 gives a0 = 64, A = 8191
    # gives a1 = 64, A = +-8192 gives a1 = -64
    x[8, 1::4] = np.float32(8191 * 2.0 ** -20)
    x[8, 2::4] = np.float32(8192 * 2.0 ** -20)
    x[8, 3::4] = np.float32(-8192 * 2.0 ** -20)
    x[8, 4::4] = np.float32(-8191 * 2.0 ** -20)
    x[8, 0] = np.nextafter(np.float32(1.0), np.float32(0.0))
    return x


def test_act_limbs_definition_and_bounds(oracle):
    x = _limb_rows()
    rows, cols = x.shape
    limbs = np.empty((3, rows, cols), np.int8)
    exps = np.empty(rows, np.int32)
    oracle.act_limbs(x, rows, cols, limbs, exps)
    L = limbs.astype(np.int64)
    A = L[0] * 16384 + L[1] * 128 + L[2]
    assert L[0].min() >= -64 and L[0].max() <= 64
    assert L[1].min() >= -64 and L[1].max() <= 64
    assert L[2].min() >= -64 and L[2].max() <= 63
    for r in range(rows):
        m = float(np.abs(x[r].astype(np.float64)).max())
        if m == 0.0:
            assert exps[r] == 0 and not A[r].any()
            continue
        k = int(exps[r])
        assert 2.0 ** (k - 1) <= m < 2.0 ** k, (r, k, m)          # frexp exponent of max|x|
        step = 2.0 ** (k - 20)
        err = np.abs(A[r] * step - x[r].astype(np.float64))
        assert err.max() <= step / 2, r                          # nearest grid point
        assert np.abs(A[r]).max() <= 1 << 20
    assert exps[4] == 1 and exps[5] == 3 and exps[6] == 2 and exps[8] == 0
    assert A[8, 0] == 1 << 20 and L[0, 8, 0] == 64
    assert L[1, 8].max() == 64 and L[1, 8].min() == -64
    # on the grid: exact
    assert np.array_equal(A[5] * 2.0 ** (3 - 20), x[5].astype(np.float64)[:])
    # ties round to the even neighbour
    t = x[6].astype(np.float64) * 2.0 ** (20 - 2)
    tie = (t - np.floor(t)) == 0.5
    assert tie.sum() > 100 and np.all(A[6][tie] % 2 == 0)


@pytest.mark.parametrize("O,I,scale", [(96, 256, 1.0), (64, 192, 1e-6), (130, 320, 3e4)])
def test_mfma_matvec_against_float64(oracle, O, I, scale):
    rng = np.random.default_rng(O + I)
    w = (rng.standard_normal((O, I)) * 0.02).astype(np.float32)
    w[3, :64] = 0.0                                       # a zero group
    q4, s = oracle.quant_gs(w, 64)
    bias = (rng.standard_normal(O) * 0.02).astype(np.float32)
    x = (rng.standard_normal((3, I)) * scale).astype(np.float32)
    x[1, 10] = np.float32(-40.0 * scale)                  # one dominant element
    x[2] = np.float32(0.0)                                 # zero row: y = bias
    limbs = np.empty((3, 3, I), np.int8)
    exps = np.empty(3, np.int32)
    oracle.act_limbs(x, 3, I, limbs, exps)
    A = limbs.astype(np.int64)
    A = A[0] * 16384 + A[1] * 128 + A[2]                   # [3][I]
    nib = np.empty((O, I), np.int64)
    nib[:, 0::2] = q4 & 15
    nib[:, 1::2] = q4 >> 4
    q = nib - 8                                            # int4 values
    ng = I // 64
    for r in range(3):
        y = np.empty(O, np.float32)
        oracle.mfma_matvec(q4, s, bias, O, I, limbs[0, r], limbs[1, r], limbs[2, r], int(exps[r]), y)
        # exact group sums C_g = sum A q (int64), then float64 terms
        C = (q.reshape(O, ng, 64) * A[r].reshape(1, ng, 64)).sum(axis=2)
        term = 16.0 * s.astype(np.float64) * C * 2.0 ** (int(exps[r]) - 24)
        y64 = term.sum(axis=1) + bias
        bound = (ng + 2) * 2.0 ** -24 * (np.abs(term).sum(axis=1) + np.abs(bias)) + 1e-45
        assert np.all(np.abs(y.astype(np.float64) - y64) <= bound), r
        if r == 2:
            assert bits_equal(y, bias)
