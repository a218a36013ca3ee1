"""Writes checkpoint directories in the converter's output format
(convert.py:216-334, :440-470): config.json with Hugging Face keys, and
safetensors shards holding F32 norms / biases / router / sinks / attention,
F32 or INT8-per-row (+ ".qs" row scales) embedding and lm_head, INT4 experts
as uint8 [O][I/2] + ".qs" group scales, and F32 expert biases (aggregated
[E][n] or per expert). Dense tensors may also be BF16 / F16 / INT8 / INT4
(load_qt_i4's other inputs, picchio.c:2443-2531). Test infrastructure: the
tensors come from the oracle's model or from numpy."""
import json
import os
import struct

import numpy as np

_ST_DTYPE = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16", np.dtype(np.int8): "I8",
             np.dtype(np.uint8): "U8", np.dtype(np.int32): "I32", np.dtype(np.float64): "F64"}


class BF16:
    """A tensor to be stored as BF16: fp32 values rounded to nearest even."""

    def __init__(self, f32):
        f32 = np.ascontiguousarray(f32, np.float32)
        u = f32.view(np.uint32).astype(np.uint64)
        self.bits = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        self.shape = f32.shape

    def to_f32(self):
        """load_f32_tensor's BF16 rule (picchio.c:2404-2411): the high half."""
        return (self.bits.astype(np.uint32) << 16).view(np.float32).reshape(self.shape)


def f16_to_f32(h):
    """load_f32_tensor's F16 rule (picchio.c:2412-2429): subnormals become
    signed zero."""
    f = np.asarray(h, np.float16).astype(np.float32)
    sub = (np.asarray(h, np.float16).view(np.uint16) & 0x7C00) == 0
    return np.where(sub, np.copysign(np.float32(0), f), f).astype(np.float32)


def save_shard(path, tensors):
    """A safetensors file: u64 header length, JSON header (dtype, shape,
    data_offsets), then the tensors' bytes in order."""
    header, blobs, off = {}, [], 0
    for name, v in tensors.items():
        if isinstance(v, BF16):
            dt, shape, raw = "BF16", v.shape, v.bits.tobytes()
        else:
            v = np.ascontiguousarray(v)
            dt, shape, raw = _ST_DTYPE[v.dtype], v.shape, v.tobytes()
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def pack_i4(q):
    """Signed values in [-8, 7] of [O][I] as picchio's nibbles (value + 8,
    even index in the low half, quant.h:386-390)."""
    q = np.asarray(q, np.int16) + 8
    O, I = q.shape
    if I % 2:
        q = np.concatenate([q, np.full((O, 1), 8, np.int16)], axis=1)
    return (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)


def unpack_i4(packed, I):
    """pack_i4's inverse: signed int8 values [O][I]."""
    lo = (packed & 0x0F).astype(np.int8) - 8
    hi = (packed >> 4).astype(np.int8) - 8
    out = np.empty((packed.shape[0], packed.shape[1] * 2), np.int8)
    out[:, 0::2], out[:, 1::2] = lo, hi
    return out[:, :I]


def config_json(cfg):
    """Hugging Face config.json keys that picchio's cfg_load reads
    (picchio.c:349-420) for a pk_cfg."""
    lt = ["full_attention" if cfg.layer_type[i] else "sliding_attention" for i in range(cfg.n_layers)]
    return {
        "architectures": ["GptOssForCausalLM"],
        "model_type": "gpt_oss",
        "hidden_size": cfg.hidden,
        "num_hidden_layers": cfg.n_layers,
        "num_attention_heads": cfg.n_heads,
        "num_key_value_heads": cfg.n_kv_heads,
        "head_dim": cfg.head_dim,
        "num_local_experts": cfg.n_experts,
        "num_experts_per_tok": cfg.topk,
        "intermediate_size": cfg.moe_inter // 2,
        "vocab_size": cfg.vocab,
        "max_position_embeddings": 131072,
        "sliding_window": cfg.sliding_window,
        "rms_norm_eps": cfg.eps,
        "rope_theta": cfg.theta,
        "rope_scaling": {"rope_type": "yarn", "factor": cfg.rope_factor,
                         "beta_fast": cfg.rope_beta_fast, "beta_slow": cfg.rope_beta_slow,
                         "original_max_position_embeddings": cfg.rope_original_ctx,
                         "truncate": bool(cfg.rope_truncate)},
        "swiglu_limit": cfg.swiglu_limit,
        "attention_bias": True,
        "layer_types": lt,
        "tie_word_embeddings": False,
    }


def quantize_int8_rows(w):
    """Per-row symmetric INT8 (convert.py:106-126): s = amax / 127 (1.0 for
    an all-zero row, convert.py:123), q = clip(round(w / s), -127, 127)."""
    amax = np.abs(w).max(axis=1).astype(np.float32)
    s = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(w / s[:, None]), -127, 127).astype(np.int8)
    return q, s


def write_container(path, cfg, tensors, experts, per_expert_names=False, lm_int8=None,
                    embed_int8=None, expert_shards=2):
    """tensors: dict of dense fp32 arrays by picchio name (without the
    experts); experts[l][e] = (gu_q4, gu_s, d_q4, d_s, gu_b, d_b) in picchio's
    host layout. lm_int8 / embed_int8: (q, s) to store INT8 rows instead of
    the F32 tensor. Experts of each layer go to `expert_shards` shards."""
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(config_json(cfg), f, indent=2)
    dense = dict(tensors)
    if lm_int8 is not None:
        dense["lm_head.weight"], dense["lm_head.weight.qs"] = lm_int8
    if embed_int8 is not None:
        dense["model.embed_tokens.weight"], dense["model.embed_tokens.weight.qs"] = embed_int8
    save_shard(os.path.join(path, "model-00000.safetensors"), dense)
    E = cfg.n_experts
    shards = [dict() for _ in range(expert_shards)]
    for l, layer in enumerate(experts):
        p = f"model.layers.{l}.mlp.experts"
        if not per_expert_names:
            # the converter's aggregated biases (F32 [E][n])
            shards[0][f"{p}.gate_up_proj_bias"] = np.stack([layer[e][4] for e in range(E)])
            shards[0][f"{p}.down_proj_bias"] = np.stack([layer[e][5] for e in range(E)])
        for e in range(E):
            gq, gs, dq, ds, gb, db = layer[e]
            sh = shards[e % expert_shards]
            if per_expert_names:
                sh[f"{p}.{e}.gate_up_proj"], sh[f"{p}.{e}.gate_up_proj.qs"] = gq, gs
                sh[f"{p}.{e}.down_proj"], sh[f"{p}.{e}.down_proj.qs"] = dq, ds
                sh[f"{p}.{e}.gate_up_proj_bias"], sh[f"{p}.{e}.down_proj_bias"] = gb, db
            else:
                sh[f"{p}.gate_up_proj.{e}"], sh[f"{p}.gate_up_proj.{e}.qs"] = gq, gs
                sh[f"{p}.down_proj.{e}"], sh[f"{p}.down_proj.{e}.qs"] = dq, ds
    for i, sh in enumerate(shards):
        if sh:
            save_shard(os.path.join(path, f"model-{i + 1:05d}.safetensors"), sh)


def oracle_tensors(oracle, model, cfg):
    """Dense tensors of an oracle-built model by picchio name, and its
    experts in picchio's host layout."""
    from helpers import (T_ROUTER, T_ROUTER_B, T_WQ, T_WK, T_WV, T_WO, T_BQ, T_BK, T_BV, T_BO,
                         T_SINKS, T_EMBED, T_LM_HEAD)
    D, E, H, KVH, hd, V = cfg.hidden, cfg.n_experts, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.vocab
    t = {"model.embed_tokens.weight": oracle.tensor(model, T_EMBED, 0, V * D).reshape(V, D),
         "lm_head.weight": oracle.tensor(model, T_LM_HEAD, 0, V * D).reshape(V, D),
         "model.norm.weight": oracle.tensor(model, 0, 0, D)}
    experts = []
    for l in range(cfg.n_layers):
        g = lambda kind, n: oracle.tensor(model, kind, l, n)
        p = f"model.layers.{l}"
        t[f"{p}.input_layernorm.weight"] = g(-1, D)
        t[f"{p}.post_attention_layernorm.weight"] = g(-2, D)
        t[f"{p}.self_attn.q_proj.weight"] = g(T_WQ, H * hd * D).reshape(H * hd, D)
        t[f"{p}.self_attn.k_proj.weight"] = g(T_WK, KVH * hd * D).reshape(KVH * hd, D)
        t[f"{p}.self_attn.v_proj.weight"] = g(T_WV, KVH * hd * D).reshape(KVH * hd, D)
        t[f"{p}.self_attn.o_proj.weight"] = g(T_WO, D * H * hd).reshape(D, H * hd)
        t[f"{p}.self_attn.q_proj.bias"] = g(T_BQ, H * hd)
        t[f"{p}.self_attn.k_proj.bias"] = g(T_BK, KVH * hd)
        t[f"{p}.self_attn.v_proj.bias"] = g(T_BV, KVH * hd)
        t[f"{p}.self_attn.o_proj.bias"] = g(T_BO, D)
        t[f"{p}.self_attn.sinks"] = g(T_SINKS, H)
        t[f"{p}.mlp.router.weight"] = g(T_ROUTER, E * D).reshape(E, D)
        t[f"{p}.mlp.router.bias"] = g(T_ROUTER_B, E)
        experts.append([tuple(np.asarray(a) for a in oracle.expert_arrays(model, l, e, cfg))
                        for e in range(E)])
    return t, experts
