"""Converted-checkpoint reading on the host (pk_cfg_from_container): config.json
with cfg_load's keys and defaults (picchio.c:349-420), the shard index, and
what is inferred from the shards (group size, picchio.c:781-784; lm_head
format). The tensor loading itself needs a GPU (tests/test_gpu_container.py)."""
import json
import os

import numpy as np
import pytest

from container_writer import config_json, write_container


def _tiny(pa):
    return pa.gptoss_cfg(hidden=128, n_layers=3, n_heads=4, n_kv_heads=2, head_dim=32, n_experts=4,
                         topk=2, moe_inter=256, vocab=64, ctx_len=64, layer_type=[0, 1, 1])


def _random_experts(cfg, rng):
    D, I, Id = cfg.hidden, cfg.moe_inter, cfg.moe_inter // 2
    ex = []
    for _ in range(cfg.n_layers):
        ex.append([(rng.integers(0, 256, (I, D // 2), dtype=np.uint8), rng.random((I, D // 64), np.float32),
                    rng.integers(0, 256, (D, Id // 2), dtype=np.uint8), rng.random((D, Id // 64), np.float32),
                    rng.random(I, np.float32), rng.random(D, np.float32)) for _ in range(cfg.n_experts)])
    return ex


def test_cfg_from_converted_container(tmp_path):
    import picchio_amd as pa
    from container_writer import quantize_int8_rows
    cfg = _tiny(pa)
    rng = np.random.default_rng(3)
    lm = rng.standard_normal((cfg.vocab, cfg.hidden)).astype(np.float32)
    dense = {"lm_head.weight": lm, "model.norm.weight": np.ones(cfg.hidden, np.float32)}
    write_container(str(tmp_path), cfg, dense, _random_experts(cfg, rng), lm_int8=quantize_int8_rows(lm))
    got = pa.cfg_from_container(str(tmp_path), ctx_len=96)
    for f in ("hidden", "n_layers", "n_heads", "n_kv_heads", "head_dim", "n_experts", "topk", "moe_inter",
              "vocab", "sliding_window", "rope_original_ctx", "rope_truncate"):
        assert getattr(got, f) == getattr(cfg, f), f
    for f in ("eps", "theta", "rope_factor", "rope_beta_fast", "rope_beta_slow", "swiglu_limit",
              "routed_scale", "swiglu_alpha"):
        assert np.float32(getattr(got, f)) == np.float32(getattr(cfg, f)), f
    assert got.ctx_len == 96
    assert got.group_size == 64                       # 256 x 128 / 512 scales
    assert got.lm_head_fmt == pa.FMT_INT8
    assert list(got.layer_type[:3]) == [0, 1, 1]
    # 0.1f * logf(32) + 1.0f (picchio.c:380-381)
    assert abs(got.rope_attn_factor - (0.1 * np.log(32.0) + 1.0)) < 1e-6
    assert pa.cfg_from_container(str(tmp_path)).ctx_len == 131072   # max_position_embeddings


def test_cfg_defaults_of_the_reference_test_model(tmp_path):
    """The mini model of the reference's make_test_model.py (its values:
    D 64, 2 layers, 4 heads / 2 KV heads of 16, 4 experts top-2,
    intermediate 128, vocab 32, 64 positions, window 16, theta 1e4, no
    rope_scaling): the YaRN fields take cfg_load's defaults (factor 1 ->
    attention factor 1, original context = max_position_embeddings,
    truncate on)."""
    import picchio_amd as pa
    conf = {"hidden_size": 64, "num_hidden_layers": 2, "num_attention_heads": 4, "num_key_value_heads": 2,
            "head_dim": 16, "intermediate_size": 128, "num_local_experts": 4, "num_experts_per_tok": 2,
            "vocab_size": 32, "max_position_embeddings": 64, "sliding_window": 16, "rms_norm_eps": 1e-5,
            "rope_theta": 10000.0, "attention_bias": True,
            "layer_types": ["sliding_attention", "full_attention"], "routed_scaling_factor": 1.0}
    with open(tmp_path / "config.json", "w") as f:
        json.dump(conf, f)
    from safetensors.numpy import save_file
    save_file({"lm_head.weight": np.zeros((32, 64), np.float32)}, str(tmp_path / "model.safetensors"))
    c = pa.cfg_from_container(str(tmp_path))
    assert (c.hidden, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim) == (64, 2, 4, 2, 16)
    assert (c.n_experts, c.topk, c.moe_inter, c.vocab, c.ctx_len) == (4, 2, 256, 32, 64)
    assert c.sliding_window == 16 and c.rope_factor == 1.0 and c.rope_attn_factor == 1.0
    assert c.rope_original_ctx == 64 and c.rope_truncate == 1
    assert c.swiglu_limit == 7.0 and np.float32(c.swiglu_alpha) == np.float32(1.702)
    assert c.lm_head_fmt == pa.FMT_F32 and c.group_size == 64
    assert list(c.layer_type[:2]) == [0, 1]


def test_container_errors(tmp_path):
    import picchio_amd as pa
    with pytest.raises(pa.PkError) as e:
        pa.cfg_from_container(str(tmp_path / "nowhere"))
    assert e.value.code == -5
    cfg = _tiny(pa)
    with open(tmp_path / "config.json", "w") as f:
        json.dump(config_json(cfg), f)
    with pytest.raises(pa.PkError) as e:                       # no shard at all
        pa.cfg_from_container(str(tmp_path))
    assert e.value.code == -5
    with open(tmp_path / "model-00000.safetensors", "wb") as f:   # header length past the file
        f.write((1 << 20).to_bytes(8, "little") + b"{}")
    with pytest.raises(pa.PkError) as e:
        pa.cfg_from_container(str(tmp_path))
    assert e.value.code == -1
    with open(tmp_path / "model-00000.safetensors", "wb") as f:   # not JSON
        f.write((4).to_bytes(8, "little") + b"{x:1")
    with pytest.raises(pa.PkError) as e:
        pa.cfg_from_container(str(tmp_path))
    assert e.value.code == -1


def _lm_head_variants(cfg, rng):
    """lm_head.weight in each form load_qt_i4 accepts (picchio.c:2443-2531),
    with the engine format it maps to."""
    from container_writer import BF16, pack_i4
    V, D = cfg.vocab, cfg.hidden
    lm = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
    q = rng.integers(-8, 8, (V, D)).astype(np.int8)
    return [({"lm_head.weight": BF16(lm)}, "INT8"),
            ({"lm_head.weight": lm.astype(np.float16)}, "INT8"),
            ({"lm_head.weight": pack_i4(q), "lm_head.weight.qs": rng.random(V, np.float32)}, "INT8"),
            ({"lm_head.weight": pack_i4(q)}, "INT8"),                        # no .qs: scales 1.0
            ({"lm_head.weight": pack_i4(q), "lm_head.weight.qs": rng.random(V * D // 32, np.float32)}, "F32"),
            ({"lm_head.weight": lm}, "F32")]


def test_cfg_lm_head_format_of_each_form(tmp_path):
    """INT4 or INT8 rows become the INT8-row lm_head (BF16 / F16 are
    quantized to INT4 rows by load_qt_i4), F32 and group-scaled INT4 the F32
    one."""
    import picchio_amd as pa
    cfg = _tiny(pa)
    rng = np.random.default_rng(8)
    ex = _random_experts(cfg, rng)
    for i, (lm, fmt) in enumerate(_lm_head_variants(cfg, rng)):
        d = str(tmp_path / f"v{i}")
        write_container(d, cfg, {**lm, "model.norm.weight": np.ones(cfg.hidden, np.float32)}, ex)
        assert pa.cfg_from_container(d).lm_head_fmt == getattr(pa, "FMT_" + fmt), i


def test_cfg_rejects_inconsistent_int4_scales(tmp_path):
    """A U8 lm_head whose .qs count is neither the row count nor a whole
    number of groups per row is an error, not a read past the scales."""
    import picchio_amd as pa
    from container_writer import pack_i4
    cfg = _tiny(pa)
    rng = np.random.default_rng(9)
    q = rng.integers(-8, 8, (cfg.vocab, cfg.hidden)).astype(np.int8)
    for ns in (cfg.vocab - 1, cfg.vocab * 3):
        d = str(tmp_path / f"n{ns}")
        write_container(d, cfg, {"lm_head.weight": pack_i4(q), "lm_head.weight.qs": np.ones(ns, np.float32)},
                        _random_experts(cfg, rng))
        with pytest.raises(pa.PkError) as e:
            pa.cfg_from_container(d)
        assert e.value.code == -1, ns


@pytest.mark.parametrize("I", [64, 128, 2880])
def test_int4_rows_product_is_the_int8_row_product(oracle, I):
    """The INT8-row lm_head holds INT4 rows as q = nibble - 8 with the row
    scale: matmul_i4 (quant.h:191-257) and matmul_q8 (quant.h:152-186) sum
    x * q in the same eight chains and scale once, so for I a multiple of 16
    the two agree bit for bit."""
    from container_writer import unpack_i4
    rng = np.random.default_rng(I)
    O = 24
    w = rng.standard_normal((O, I)).astype(np.float32)
    q4, s = np.empty((O, I // 2), np.uint8), np.empty(O, np.float32)
    oracle.quantize_rows_i4(w, O, I, q4, s)
    x = rng.standard_normal((3, I)).astype(np.float32)
    y4, y8 = np.empty((3, O), np.float32), np.empty((3, O), np.float32)
    oracle.matmul_i4(y4, x, q4, s, 3, I, O)
    oracle.matmul_q8(y8, x, np.ascontiguousarray(unpack_i4(q4, I)), s, 3, I, O)
    assert np.array_equal(y4.view(np.uint32), y8.view(np.uint32))


@pytest.mark.parametrize("gs", [0, 64])
def test_int4_attention_as_fp32_values(oracle, gs):
    """Attention in INT4 is held as its fp32 values q * s: sum(x * q * s)
    against matmul_i4's sum(x * q) * s (or matmul_i4_gs's per group) differs
    by rounding only, bounded here by 1e-6 of sum |x * q * s|."""
    from container_writer import unpack_i4
    rng = np.random.default_rng(11 + gs)
    O, I = 64, 2880
    w = (rng.standard_normal((O, I)) * 0.02).astype(np.float32)
    if gs:
        q4, s = oracle.quant_gs(w, gs)
    else:
        q4, s = np.empty((O, I // 2), np.uint8), np.empty(O, np.float32)
        oracle.quantize_rows_i4(w, O, I, q4, s)
    s = s.reshape(O, -1)
    q = unpack_i4(q4, I).astype(np.float32)
    deq = (q * np.repeat(s, I // s.shape[1], axis=1)).astype(np.float32)
    x = rng.standard_normal((2, I)).astype(np.float32)
    yq, yf = np.empty((2, O), np.float32), np.empty((2, O), np.float32)
    if gs:
        oracle.matmul_i4_gs(yq, x, q4, s, 2, I, O, gs)
    else:
        oracle.matmul_i4(yq, x, q4, s.ravel(), 2, I, O)
    oracle.matmul_f32(yf, x, deq, 2, I, O)
    bound = 1e-6 * (np.abs(x.astype(np.float64)) @ np.abs(deq.astype(np.float64)).T)
    assert (np.abs(yq.astype(np.float64) - yf) <= bound).all()
    assert not np.array_equal(yq, yf)                     # the two orders do differ
