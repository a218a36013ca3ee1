"""The INT8 per-row lm_head (what converted checkpoints carry: convert.py
:106-126 rows, matmul_q8 at quant.h:152-186, called from forward_token at
picchio.c:1744) inside pk_forward_token / pk_generate at the full GPT-OSS
vocabulary of 201,088 rows, against the oracle's forward_token on the same
INT8 rows and scales (the oracle's matmul_q8 is pinned to picchio's by the
golden vectors). Model: every width at its 20B size, 2 layers, 4 experts.

Bars: logits within relative L2 1e-4; greedy ids identical.
"""
import ctypes as C

import numpy as np
import pytest

from helpers import REL_L2_TOL, T_EMBED, T_LM_HEAD, rel_l2, upload_model

pytestmark = pytest.mark.gpu


def _int8_lm_head(oracle, model, cfg):
    """Copies of the oracle model's INT8 lm_head rows and per-row scales."""
    sp = C.c_void_p()
    q = oracle.model_tensor(model, T_LM_HEAD, 0, C.byref(sp))
    V, D = cfg.vocab, cfg.hidden
    q8 = np.ctypeslib.as_array(C.cast(q, C.POINTER(C.c_int8)), shape=(V * D,)).copy()
    s = np.ctypeslib.as_array(C.cast(sp, C.POINTER(C.c_float)), shape=(V,)).copy()
    return q8, s


@pytest.fixture(scope="module")
def q8_setup(gpu, oracle):
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=4, ctx_len=96, lm_head_fmt=pa.FMT_INT8)
    assert cfg.vocab == 201088
    model = oracle.model_build(cfg, 31337, 0)
    eng = pa.Engine(cfg)
    upload_model(eng, oracle, model, cfg, globals_=False)
    q8, s = _int8_lm_head(oracle, model, cfg)
    eng.store_globals(oracle.tensor(model, T_EMBED, 0, cfg.vocab * cfg.hidden), q8,
                      oracle.tensor(model, 0, 0, cfg.hidden), lm_scales=s)
    yield cfg, model, eng
    eng.close()
    oracle.model_free(model)


def test_int8_lm_head_forward_token(q8_setup, oracle):
    import torch
    cfg, model, eng = q8_setup
    oracle.model_reset_kv(model)
    ref_lg = np.empty(cfg.vocab, np.float32)
    lg_dev = eng.empty(cfg.vocab, torch.float32)
    tok = 1234
    for pos in range(8):
        nxt_ref = oracle.forward_token(model, tok, pos, ref_lg.ctypes.data)
        nxt = eng.forward_token(tok, pos, lg_dev)
        err = rel_l2(eng.to_host(lg_dev), ref_lg)
        assert err < REL_L2_TOL, (pos, err)
        srt = np.sort(ref_lg)[::-1]
        assert srt[0] - srt[1] > 1e-5, "top-2 logits too close for an id check"
        assert nxt == nxt_ref, (pos, nxt, nxt_ref)
        tok = nxt_ref


def test_int8_lm_head_generate(q8_setup, oracle):
    """Prompt through prefill_tokens (chunks of 64), then 24 replayed decode
    steps: the oracle's ids."""
    cfg, model, eng = q8_setup
    prompt = np.random.default_rng(8).integers(0, cfg.vocab, 66).astype(np.int32)
    oracle.model_reset_kv(model)
    ref = [oracle.prefill_tokens(model, prompt, len(prompt), 0, 64)]
    for i in range(23):
        ref.append(oracle.forward_token(model, ref[-1], len(prompt) + i, None))
    assert list(eng.generate(prompt, 24)) == ref
