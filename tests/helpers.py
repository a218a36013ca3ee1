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


# pk_synth kinds (picchio_amd/csrc/pk_synth.h)
T_ROUTER, T_ROUTER_B, T_WQ, T_WK, T_WV, T_WO = 6, 7, 8, 9, 10, 11
T_BQ, T_BK, T_BV, T_BO, T_SINKS, T_EMBED, T_LM_HEAD = 12, 13, 14, 15, 16, 17, 18


def upload_model(eng, oracle, model, cfg, experts=True, dense=True, globals_=True):
    """Copies every tensor of an oracle-built model into the engine's HBM store."""
    D, E, H, KVH, hd = cfg.hidden, cfg.n_experts, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    for l in range(cfg.n_layers):
        if experts:
            for e in range(E):
                eng.store_expert(l, e, *oracle.expert_arrays(model, l, e, cfg))
        t = lambda kind, n: oracle.tensor(model, kind, l, n)
        if dense:
            eng.store_layer(l, t(-1, D), t(-2, D), t(T_WQ, H * hd * D), t(T_WK, KVH * hd * D),
                            t(T_WV, KVH * hd * D), t(T_WO, D * H * hd), t(T_BQ, H * hd),
                            t(T_BK, KVH * hd), t(T_BV, KVH * hd), t(T_BO, D), t(T_SINKS, H),
                            t(T_ROUTER, E * D), t(T_ROUTER_B, E))
        elif experts:
            eng.store_router(l, t(T_ROUTER, E * D), t(T_ROUTER_B, E))
    if globals_:
        assert cfg.lm_head_fmt == 0
        eng.store_globals(oracle.tensor(model, T_EMBED, 0, cfg.vocab * D),
                          oracle.tensor(model, T_LM_HEAD, 0, cfg.vocab * D),
                          oracle.tensor(model, 0, 0, D))
