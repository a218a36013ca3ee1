"""Converted checkpoints into the HBM store (pk_load_container): a container
written in the converter's format from the oracle's model gives the
oracle's greedy stream; the other layouts the reference reads (per-expert
names and biases, INT8 embedding and lm_head, BF16 / F16 / INT8 / INT4
attention, embedding and lm_head) give the same bits as the values the
reference's loader makes of them uploaded directly."""
import numpy as np
import pytest

from container_writer import oracle_tensors, quantize_int8_rows, write_container
from helpers import upload_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ckpt(gpu, oracle, tmp_path_factory):
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=8, ctx_len=128, vocab=1000)
    model = oracle.model_build(cfg, 2468, 0)
    dense, experts = oracle_tensors(oracle, model, cfg)
    yield cfg, model, dense, experts, tmp_path_factory
    oracle.model_free(model)


def test_container_stream_matches_oracle(ckpt, oracle):
    import picchio_amd as pa
    cfg, model, dense, experts, tmpf = ckpt
    path = str(tmpf.mktemp("conv"))
    write_container(path, cfg, dense, experts)
    c = pa.cfg_from_container(path, ctx_len=cfg.ctx_len)
    for f in ("hidden", "n_layers", "n_experts", "moe_inter", "vocab", "group_size", "lm_head_fmt"):
        assert getattr(c, f) == getattr(cfg, f), f
    eng = pa.Engine(c)
    try:
        eng.load_container(path, threads=4)
        prompt = np.random.default_rng(5).integers(0, cfg.vocab, 30).astype(np.int32)
        n = 12
        oracle.model_reset_kv(model)
        ref = [oracle.prefill_tokens(model, prompt, len(prompt), 0, 64)]
        for i in range(n - 1):
            ref.append(oracle.forward_token(model, ref[-1], len(prompt) + i, None))
        assert list(eng.generate(prompt, n)) == ref
    finally:
        eng.close()


def test_container_layouts_match_direct_upload(ckpt, oracle):
    """Per-expert tensor names and biases (expert_load's second spelling,
    load_expert_bias's per-expert name), INT8 rows for the embedding
    (dequantized as embed_token does) and the lm_head: the logits of
    forward_token equal, bit for bit, those of an engine given the same
    tensors through pk_store_*."""
    import torch
    import picchio_amd as pa
    cfg, model, dense, experts, tmpf = ckpt
    V, D = cfg.vocab, cfg.hidden
    lm_q = quantize_int8_rows(dense["lm_head.weight"])
    em_q = quantize_int8_rows(dense["model.embed_tokens.weight"])
    path = str(tmpf.mktemp("conv_b"))
    write_container(path, cfg, dense, experts, per_expert_names=True, lm_int8=lm_q, embed_int8=em_q,
                    expert_shards=3)
    c = pa.cfg_from_container(path, ctx_len=cfg.ctx_len)
    assert c.lm_head_fmt == pa.FMT_INT8
    a, b = pa.Engine(c), pa.Engine(c)
    try:
        a.load_container(path, threads=3)
        upload_model(b, oracle, model, cfg, globals_=False)
        emb = (em_q[0].astype(np.float32) * em_q[1][:, None]).astype(np.float32)
        b.store_globals(np.ascontiguousarray(emb), np.ascontiguousarray(lm_q[0]), dense["model.norm.weight"],
                        lm_scales=lm_q[1])
        la, lb = a.empty(V, torch.float32), b.empty(V, torch.float32)
        tok = 17
        for pos in range(6):
            na = a.forward_token(tok, pos, la)
            nb = b.forward_token(tok, pos, lb)
            assert na == nb, pos
            ga, gb = a.to_host(la), b.to_host(lb)
            assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), pos
            tok = na
    finally:
        a.close()
        b.close()


def test_container_rejects_fp32_experts(ckpt, oracle):
    """F32 experts (the reference's fmt-0 path) are not held by the INT4
    store: PK_ERR_UNSUPPORTED, not a silent conversion."""
    import picchio_amd as pa
    from safetensors.numpy import save_file
    cfg, model, dense, experts, tmpf = ckpt
    path = str(tmpf.mktemp("conv_f32"))
    write_container(path, cfg, dense, experts)
    save_file({"model.layers.0.mlp.experts.gate_up_proj.0":
               np.zeros((cfg.moe_inter, cfg.hidden), np.float32)}, path + "/dense.safetensors")
    eng = pa.Engine(pa.cfg_from_container(path, ctx_len=cfg.ctx_len))
    try:
        with pytest.raises(pa.PkError) as e:
            eng.load_container(path)
        assert e.value.code == -4
    finally:
        eng.close()


# ── load_qt_i4's other forms (picchio.c:2443-2531) for attention, embedding
#    and lm_head. Expected values: BF16 / F16 to fp32 by load_f32_tensor's
#    rules, then the oracle's quantize_rows_i4 (golden-pinned); INT8 / INT4
#    as (float)q * scale, embed_token's product. ──

_ATT = ("q_proj", "k_proj", "v_proj", "o_proj")
_KIND = {"q_proj": 8, "k_proj": 9, "v_proj": 10, "o_proj": 11}      # helpers.T_WQ..T_WO


def _rows_i4(oracle, f):
    from container_writer import unpack_i4
    O, I = f.shape
    q4, s = np.empty((O, (I + 1) // 2), np.uint8), np.empty(O, np.float32)
    oracle.quantize_rows_i4(np.ascontiguousarray(f, np.float32), O, I, q4, s)
    return unpack_i4(q4, I), s


def _deq(q, s):
    s = s.reshape(q.shape[0], -1)
    return (q.astype(np.float32) * np.repeat(s, -(-q.shape[1] // s.shape[1]), axis=1)[:, :q.shape[1]]
            ).astype(np.float32)


def _forms(case, oracle, dense):
    """(tensors to store, fp32 values the engine must hold for the attention
    and the embedding, lm_head as ("INT8", q, s) or ("F32", values))."""
    from container_writer import BF16, f16_to_f32, pack_i4, quantize_int8_rows, unpack_i4
    store, expect = {}, {}
    emb, lm = dense["model.embed_tokens.weight"], dense["lm_head.weight"]
    if case == "bf16_f16":
        for l in range(2):
            for a in _ATT:
                n = f"model.layers.{l}.self_attn.{a}.weight"
                if l == 0:
                    b = BF16(dense[n])
                    store[n], f = b, b.to_f32()
                else:
                    h = dense[n].astype(np.float16)
                    store[n], f = h, f16_to_f32(h)
                expect[n] = _deq(*_rows_i4(oracle, f))
        b = BF16(emb)
        store["model.embed_tokens.weight"] = b
        expect["model.embed_tokens.weight"] = _deq(*_rows_i4(oracle, b.to_f32()))
        b = BF16(lm)
        store["lm_head.weight"] = b
        return store, expect, ("INT8",) + _rows_i4(oracle, b.to_f32())
    if case == "int4_int8":
        for l in range(2):
            for a in _ATT:
                n = f"model.layers.{l}.self_attn.{a}.weight"
                if l == 0:                                   # INT4 groups of 64
                    q4, s = oracle.quant_gs(dense[n], 64)
                    store[n], store[n + ".qs"] = q4, s.ravel()
                    expect[n] = _deq(unpack_i4(q4, dense[n].shape[1]), s)
                else:                                        # INT8 rows
                    q, s = quantize_int8_rows(dense[n])
                    store[n], store[n + ".qs"] = q, s
                    expect[n] = _deq(q, s)
        q4, s = oracle.quant_gs(emb, 32)                     # INT4 groups of 32
        store["model.embed_tokens.weight"], store["model.embed_tokens.weight.qs"] = q4, s.ravel()
        expect["model.embed_tokens.weight"] = _deq(unpack_i4(q4, emb.shape[1]), s)
        q, s = _rows_i4(oracle, lm)                          # INT4 rows
        store["lm_head.weight"], store["lm_head.weight.qs"] = pack_i4(q), s
        return store, expect, ("INT8", q, s)
    assert case == "int4_groups_lm"
    q = np.clip(np.rint(emb / np.float32(0.01)), -8, 7).astype(np.int8)
    store["model.embed_tokens.weight"] = pack_i4(q)          # no .qs: scale 1.0
    expect["model.embed_tokens.weight"] = q.astype(np.float32)
    q4, s = oracle.quant_gs(lm, 64)
    store["lm_head.weight"], store["lm_head.weight.qs"] = q4, s.ravel()
    return store, expect, ("F32", _deq(unpack_i4(q4, lm.shape[1]), s))


@pytest.mark.parametrize("case", ["bf16_f16", "int4_int8", "int4_groups_lm"])
def test_container_dense_forms(ckpt, oracle, case):
    """Each form loads to the values the reference's loader gives: the
    logits equal, bit for bit, those of an engine given those values
    through pk_store_*, and the greedy stream is the oracle's on the same
    values."""
    import ctypes as C
    import torch
    import picchio_amd as pa
    from helpers import T_EMBED, T_LM_HEAD
    cfg, _, dense, experts, tmpf = ckpt
    V, D = cfg.vocab, cfg.hidden
    store, expect, lm = _forms(case, oracle, dense)
    path = str(tmpf.mktemp("conv_" + case))
    write_container(path, cfg, {**{k: v for k, v in dense.items() if k not in store}, **store}, experts)
    c = pa.cfg_from_container(path, ctx_len=cfg.ctx_len)
    assert c.lm_head_fmt == getattr(pa, "FMT_" + lm[0])
    # the oracle's model with the expected values in place
    model = oracle.model_build(c, 2468, 0)
    try:
        def put(kind, layer, arr):
            C.memmove(oracle.model_tensor(model, kind, layer, None), arr.ctypes.data, arr.nbytes)
        for l in range(cfg.n_layers):
            for a in _ATT:
                n = f"model.layers.{l}.self_attn.{a}.weight"
                if n in expect:
                    put(_KIND[a], l, np.ascontiguousarray(expect[n]))
        emb = np.ascontiguousarray(expect["model.embed_tokens.weight"])
        put(T_EMBED, 0, emb)
        if lm[0] == "INT8":
            sp = C.c_void_p()
            C.memmove(oracle.model_tensor(model, T_LM_HEAD, 0, C.byref(sp)), lm[1].ctypes.data, V * D)
            C.memmove(sp, lm[2].ctypes.data, V * 4)
        else:
            put(T_LM_HEAD, 0, np.ascontiguousarray(lm[1]))
        a, b = pa.Engine(c), pa.Engine(c)
        try:
            a.load_container(path, threads=4)
            upload_model(b, oracle, model, c, globals_=False)
            if lm[0] == "INT8":
                b.store_globals(emb, np.ascontiguousarray(lm[1]), dense["model.norm.weight"], lm_scales=lm[2])
            else:
                b.store_globals(emb, np.ascontiguousarray(lm[1]), dense["model.norm.weight"])
            la, lb = a.empty(V, torch.float32), b.empty(V, torch.float32)
            tok = 17
            for pos in range(4):
                na, nb = a.forward_token(tok, pos, la), b.forward_token(tok, pos, lb)
                assert na == nb, (case, pos)
                assert np.array_equal(a.to_host(la).view(np.uint32), b.to_host(lb).view(np.uint32)), (case, pos)
                tok = na
            # generate rewrites every KV position it reads (prefill from 0)
            prompt = np.random.default_rng(6).integers(0, V, 20).astype(np.int32)
            n = 8
            oracle.model_reset_kv(model)
            ref = [oracle.prefill_tokens(model, prompt, len(prompt), 0, 64)]
            for i in range(n - 1):
                ref.append(oracle.forward_token(model, ref[-1], len(prompt) + i, None))
            assert list(a.generate(prompt, n)) == ref, case
        finally:
            a.close()
            b.close()
    finally:
        oracle.model_free(model)
