"""Converted checkpoints into the HBM store (pk_load_container): a container
written in the converter's format from the oracle's model gives the
oracle's greedy stream; the other layouts the reference reads (per-expert
names and biases, INT8 embedding and lm_head) give the same bits as the
same tensors uploaded directly."""
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
