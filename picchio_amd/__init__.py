"""picchio_amd — MI355X (gfx950) quantized-MoE expert path of picchio.

The product is the C-ABI library libpicchio_hip.so (include/picchio_hip.h).
This module binds it with ctypes for tests and benchmarks; there is no
Python or CPU fallback: loading fails loudly when the library is missing.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libpicchio_hip.so")
HEADER = os.path.join(ROOT, "include", "picchio_hip.h")

PK_OK = 0
ERRORS = {-1: "PK_ERR_ARG", -2: "PK_ERR_HIP", -3: "PK_ERR_OOM", -4: "PK_ERR_UNSUPPORTED",
          -5: "PK_ERR_MISSING", -6: "PK_ERR_CONTEXT_FULL"}
FMT_F32, FMT_INT8, FMT_INT4 = 0, 1, 2
PROF_EXPERT_GATE_UP, PROF_EXPERT_DOWN, PROF_ROUTER, PROF_COMBINE = 0, 1, 2, 3
PROF_MOE_FFN, PROF_LM_HEAD, PROF_ATTENTION = 4, 5, 6


class PkError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{ERRORS.get(code, code)}: {msg}")
        self.code = code


class PkCfg(C.Structure):
    """pk_cfg (include/picchio_hip.h)."""
    _fields_ = [
        ("hidden", C.c_int32), ("n_layers", C.c_int32), ("n_heads", C.c_int32),
        ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("n_experts", C.c_int32),
        ("topk", C.c_int32), ("moe_inter", C.c_int32), ("vocab", C.c_int32),
        ("ctx_len", C.c_int32), ("sliding_window", C.c_int32),
        ("eps", C.c_float), ("theta", C.c_float), ("rope_factor", C.c_float),
        ("rope_beta_fast", C.c_float), ("rope_beta_slow", C.c_float),
        ("rope_original_ctx", C.c_int32), ("rope_truncate", C.c_int32),
        ("rope_attn_factor", C.c_float), ("swiglu_limit", C.c_float),
        ("swiglu_alpha", C.c_float), ("routed_scale", C.c_float),
        ("group_size", C.c_int32), ("lm_head_fmt", C.c_int32),
        ("layer_type", C.c_int8 * 128),
    ]


class PkQtHost(C.Structure):
    """pk_qt_host == picchio's QT (quant.h:32-40), host pointers."""
    _fields_ = [("fmt", C.c_int32), ("data", C.c_void_p), ("s", C.c_void_p),
                ("O", C.c_int32), ("I", C.c_int32), ("block_size", C.c_int32)]


class PkLayerHost(C.Structure):
    _fields_ = [("in_ln", C.c_void_p), ("post_ln", C.c_void_p),
                ("wq", PkQtHost), ("wk", PkQtHost), ("wv", PkQtHost), ("wo", PkQtHost),
                ("bq", C.c_void_p), ("bk", C.c_void_p), ("bv", C.c_void_p), ("bo", C.c_void_p),
                ("sinks", C.c_void_p), ("router", C.c_void_p), ("router_bias", C.c_void_p)]


def gptoss_cfg(**kw):
    """GPT-OSS-20B-shaped configuration; keywords override.
    Defaults follow picchio's cfg_load (picchio.c:363-392) with the YaRN
    fields of GPT-OSS set explicitly (factor 32, original ctx 4096)."""
    import math
    import numpy as np
    d = dict(hidden=2880, n_layers=24, n_heads=64, n_kv_heads=8, head_dim=64,
             n_experts=32, topk=4, moe_inter=5760, vocab=201088, ctx_len=1024,
             sliding_window=128, eps=1e-5, theta=150000.0, rope_factor=32.0,
             rope_beta_fast=32.0, rope_beta_slow=1.0, rope_original_ctx=4096,
             rope_truncate=0, swiglu_limit=7.0, swiglu_alpha=1.702,
             routed_scale=1.0, group_size=64, lm_head_fmt=FMT_F32)
    lt = kw.pop("layer_type", None)
    d.update(kw)
    if "rope_attn_factor" not in d:
        f = np.float32(d["rope_factor"])
        # picchio.c:380-381: 0.1f * logf(factor) + 1.0f
        d["rope_attn_factor"] = float(np.float32(np.float32(0.1) * np.float32(math.log(f)))
                                      + np.float32(1.0)) if f > 1 else 1.0
    c = PkCfg(**d)
    for i in range(128):
        c.layer_type[i] = lt[i] if lt is not None and i < len(lt) else i % 2
    return c


def cfg_from_container(path, ctx_len=0):
    """pk_cfg of a converted checkpoint directory (config.json + shards)."""
    c = PkCfg()
    check(lib().pk_cfg_from_container(os.fsencode(path), ctx_len, C.byref(c)))
    return c


_lib = None


def lib():
    """The native library (loaded once). Raises if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: run `python -m picchio_amd.build` "
                           "(the expert path has no CPU fallback)")
    L = C.CDLL(LIB_PATH)
    vp, i32, i64, f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_float
    sig = {
        "pk_last_error": (C.c_char_p, []),
        "pk_version": (C.c_char_p, []),
        "pk_engine_create": (C.c_int, [C.POINTER(PkCfg), C.c_int, C.POINTER(vp)]),
        "pk_engine_destroy": (C.c_int, [vp]),
        "pk_engine_stream": (vp, [vp]),
        "pk_engine_sync": (C.c_int, [vp]),
        "pk_engine_device_bytes": (i64, [vp]),
        "pk_store_expert": (C.c_int, [vp, C.c_int, C.c_int, C.POINTER(PkQtHost),
                                      C.POINTER(PkQtHost), vp, vp]),
        "pk_store_layer": (C.c_int, [vp, C.c_int, C.POINTER(PkLayerHost)]),
        "pk_store_globals": (C.c_int, [vp, C.POINTER(PkQtHost), C.POINTER(PkQtHost), vp]),
        "pk_engine_build_synthetic": (C.c_int, [vp, C.c_uint64, C.c_int, C.c_int]),
        "pk_cfg_from_container": (C.c_int, [C.c_char_p, C.c_int, C.POINTER(PkCfg)]),
        "pk_load_container": (C.c_int, [vp, C.c_char_p, C.c_int]),
        "pk_set_sampling": (C.c_int, [vp, f32, f32, C.c_int, f32, C.c_uint64]),
        "pk_set_turn_sampling": (C.c_int, [vp, f32, f32, C.c_int]),
        "pk_reset_history": (C.c_int, [vp]),
        "pk_set_sampling_fast_sums": (C.c_int, [vp, C.c_int]),
        "pk_set_i4_dot": (C.c_int, [vp, C.c_int]),
        "pk_set_grouped_f16": (C.c_int, [vp, C.c_int]),
        "pk_set_moe_fused": (C.c_int, [vp, C.c_int]),
        "pk_moe_ffn_plan": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp, C.c_int]),
        "pk_kv_layout": (C.c_int, [C.c_int, C.c_int, C.c_int, vp, C.c_int64]),
        "pk_moe_bal_plan": (C.c_int, [C.c_int] * 6 + [vp, C.c_int]),
        "pk_set_router_trace": (C.c_int, [vp, vp, C.c_int64]),
        "pk_router_trace_used": (C.c_int64, [vp]),
        "pk_set_numeric_trace": (C.c_int, [vp, C.c_int]),
        "pk_set_poll_bound": (C.c_int, [vp, C.c_uint32]),
        "pk_wait_fallbacks": (C.c_int64, [vp]),
        "pk_set_attn_fused": (C.c_int, [vp, C.c_int]),
        "pk_router_logits": (C.c_int, [vp, C.c_int, vp, vp]),
        "pk_act_records": (C.c_int, [vp, vp, C.c_int, vp]),
        "pk_expert_gate_up_dot": (C.c_int, [vp, C.c_int, vp, C.c_int, vp, vp, vp]),
        "pk_expert_down_dot": (C.c_int, [vp, C.c_int, vp, C.c_int, vp, vp]),
        "pk_sample_logits": (C.c_int, [vp, vp, C.c_int, C.POINTER(i32)]),
        "pk_sampler_state": (C.c_int, [vp, C.POINTER(C.c_uint64), vp, C.c_int, C.POINTER(C.c_int)]),
        "pk_quantize_int4_gs": (C.c_int, [vp, vp, C.c_int, C.c_int, C.c_int, vp, vp]),
        "pk_qt_upload": (C.c_int, [vp, C.POINTER(PkQtHost), C.POINTER(vp)]),
        "pk_qt_free": (C.c_int, [vp, vp]),
        "pk_matmul_qt": (C.c_int, [vp, vp, vp, vp, C.c_int]),
        "pk_expert_apply": (C.c_int, [vp, C.c_int, C.c_int, vp, vp, f32]),
        "pk_expert_gate_up": (C.c_int, [vp, C.c_int, vp, C.c_int, vp, vp]),
        "pk_expert_down": (C.c_int, [vp, C.c_int, vp, C.c_int, vp, vp]),
        "pk_moe_forward": (C.c_int, [vp, C.c_int, vp, vp, vp, vp]),
        "pk_moe_forward_batch": (C.c_int, [vp, C.c_int, vp, C.c_int, vp, vp, vp]),
        "pk_moe_forward_batch_noalloc": (C.c_int, [vp, C.c_int, vp, C.c_int, vp, vp, vp]),
        "pk_moe_forward_grouped": (C.c_int, [vp, C.c_int, vp, C.c_int, vp, vp, vp, vp, vp]),
        "pk_quantize_act_i8x3": (C.c_int, [vp, vp, C.c_int, C.c_int, vp, vp]),
        "pk_gqa_attention": (C.c_int, [vp, C.c_int, vp, C.c_int, vp]),
        "pk_forward_token": (C.c_int, [vp, C.c_int, C.c_int, vp, vp]),
        "pk_prefill_tokens": (C.c_int, [vp, vp, C.c_int, C.c_int, vp]),
        "pk_generate": (C.c_int, [vp, vp, C.c_int, C.c_int, vp]),
        "pk_engine_profile": (C.c_int, [vp, C.c_int]),
        "pk_engine_profile_read": (C.c_int, [vp, C.c_int, C.POINTER(C.c_double), C.POINTER(i64)]),
        "pk_engine_stall": (C.c_int, [vp, C.c_int]),
        "pk_decode_replay": (C.c_int, [vp, C.c_int, C.c_int, C.c_int, vp]),
        "pk_batch_reserve": (C.c_int, [vp, C.c_int]),
        "pk_kv_fill_synthetic": (C.c_int, [vp, C.c_int, C.c_int, C.c_uint64]),
        "pk_prefill_seq": (C.c_int, [vp, C.c_int, vp, C.c_int, C.c_int, vp]),
        "pk_decode_batch": (C.c_int, [vp, C.c_int, vp, C.c_int, C.c_int, vp]),
        "pk_capture_begin": (C.c_int, [vp]),
        "pk_capture_end": (C.c_int, [vp, C.POINTER(vp)]),
        "pk_graph_launch": (C.c_int, [vp, vp]),
        "pk_graph_destroy": (C.c_int, [vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(rc):
    if rc != PK_OK:
        raise PkError(rc, lib().pk_last_error().decode())
    return rc


def ptr(a):
    """Raw address of a numpy array or torch tensor."""
    if hasattr(a, "data_ptr"):
        return C.c_void_p(a.data_ptr())
    return C.c_void_p(a.ctypes.data)


class Engine:
    """One pk_engine: GPU, stream and HBM store. Device buffers are torch
    tensors allocated on the engine's stream so that the order of torch
    copies and library kernels is the stream order."""

    def __init__(self, cfg, device=0):
        import torch
        self.cfg = cfg
        self.L = lib()
        h = C.c_void_p()
        check(self.L.pk_engine_create(C.byref(cfg), device, C.byref(h)))
        self.h = h
        self.device = torch.device("cuda", device)
        self.stream = torch.cuda.ExternalStream(self.L.pk_engine_stream(h), device=self.device)

    def close(self):
        if self.h:
            self.L.pk_engine_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def sync(self):
        check(self.L.pk_engine_sync(self.h))

    def device_bytes(self):
        return self.L.pk_engine_device_bytes(self.h)

    def profile(self, enable):
        check(self.L.pk_engine_profile(self.h, 1 if enable else 0))

    def profile_read(self, kernel):
        ms = C.c_double()
        n = C.c_int64()
        check(self.L.pk_engine_profile_read(self.h, kernel, C.byref(ms), C.byref(n)))
        return ms.value, n.value

    def stall(self, usec):
        check(self.L.pk_engine_stall(self.h, int(usec)))

    def capture_begin(self):
        check(self.L.pk_capture_begin(self.h))

    def capture_end(self):
        g = C.c_void_p()
        check(self.L.pk_capture_end(self.h, C.byref(g)))
        return g

    def graph_launch(self, g):
        check(self.L.pk_graph_launch(self.h, g))

    def graph_destroy(self, g):
        check(self.L.pk_graph_destroy(g))

    # torch helpers on the engine stream
    def to_dev(self, arr, dtype=None):
        import torch
        with torch.cuda.stream(self.stream):
            t = torch.as_tensor(arr).to(self.device, non_blocking=False)
            if dtype is not None:
                t = t.to(dtype)
        self.stream.synchronize()
        return t.contiguous()

    def empty(self, shape, dtype):
        import torch
        with torch.cuda.stream(self.stream):
            return torch.empty(shape, dtype=dtype, device=self.device)

    def to_host(self, t):
        self.sync()
        return t.cpu().numpy()

    # library calls
    def build_synthetic(self, seed, what=7, threads=0):
        check(self.L.pk_engine_build_synthetic(self.h, seed, what, threads))

    def load_container(self, path, threads=8):
        """Every tensor of a converted checkpoint directory (pk_load_container)."""
        check(self.L.pk_load_container(self.h, os.fsencode(path), threads))

    def set_sampling(self, temperature, top_p, top_k, rep_penalty, seed):
        """Sampling parameters, seed and an empty history (the TEMPERATURE /
        TOPP / TOPK / REP / SEED start-up settings, picchio.c:3033-3037)."""
        check(self.L.pk_set_sampling(self.h, temperature, top_p, top_k, rep_penalty, seed))

    def set_turn_sampling(self, temperature, top_p, top_k):
        """A TURN's per-request temperature / top-p / top-k with the
        reference's clamp; rng and history carry on (picchio.c:2737-2743)."""
        check(self.L.pk_set_turn_sampling(self.h, temperature, top_p, top_k))

    def set_i4_dot(self, on):
        """Batch-1 MoE experts on the integer-dot arithmetic, or on picchio's
        fp32 chains, bit-identical (the default) (pk_set_i4_dot)."""
        check(self.L.pk_set_i4_dot(self.h, 1 if on else 0))

    def set_grouped_f16(self, on):
        """Grouped MoE arithmetic: f16 hi/lo activations on the f16 MFMA (the
        default) or the exact int8 limbs (pk_set_grouped_f16)."""
        check(self.L.pk_set_grouped_f16(self.h, 1 if on else 0))

    def set_router_trace(self, buf_dev):
        """Every MoE router launch appends its logits to buf_dev (a float32
        device tensor; None: off) until it is full (pk_set_router_trace)."""
        check(self.L.pk_set_router_trace(self.h, ptr(buf_dev) if buf_dev is not None else None,
                                         buf_dev.numel() if buf_dev is not None else 0))

    def router_trace_used(self):
        return int(self.L.pk_router_trace_used(self.h))

    def set_poll_bound(self, polls):
        """Polls a device-side wait makes before it gives up (0: the default;
        pk_set_poll_bound)."""
        check(self.L.pk_set_poll_bound(self.h, int(polls)))

    def wait_fallbacks(self):
        """Calls redone with the separate launches after a wait gave up."""
        return int(self.L.pk_wait_fallbacks(self.h))

    def set_numeric_trace(self, on):
        """picchio's TRACE_NUMERIC lines on stderr for eager forward_token."""
        check(self.L.pk_set_numeric_trace(self.h, 1 if on else 0))

    def set_moe_fused(self, mode):
        """How a batch-1 MoE layer runs its experts (pk_set_moe_fused): 1 one
        launch of row-block workgroups (default), 2 one launch with every CU
        streaming the same bytes, 0 a gate_up launch and a down launch; same
        results. True / False mean 1 / 0."""
        check(self.L.pk_set_moe_fused(self.h, int(mode)))

    def set_attn_fused(self, on):
        """Batch-1 decode attention and its output projection as one launch
        (default) or two; same results (pk_set_attn_fused)."""
        check(self.L.pk_set_attn_fused(self.h, 1 if on else 0))

    def act_records(self, x_dev, rec_dev):
        """Half-group records of the integer-dot arithmetic for a device row."""
        check(self.L.pk_act_records(self.h, ptr(x_dev), x_dev.numel(), ptr(rec_dev)))

    def expert_gate_up_dot(self, layer, eids_dev, rec_dev, act_dev, act_rec_dev=None):
        check(self.L.pk_expert_gate_up_dot(self.h, layer, ptr(eids_dev), eids_dev.numel(), ptr(rec_dev),
                                           ptr(act_dev), ptr(act_rec_dev) if act_rec_dev is not None else None))

    def expert_down_dot(self, layer, eids_dev, act_rec_dev, eo_dev):
        check(self.L.pk_expert_down_dot(self.h, layer, ptr(eids_dev), eids_dev.numel(), ptr(act_rec_dev),
                                        ptr(eo_dev)))

    def set_sampling_fast_sums(self, on):
        """Exact integer sums instead of the reference's float order for
        draws keeping more than 4096 entries (pk_set_sampling_fast_sums)."""
        check(self.L.pk_set_sampling_fast_sums(self.h, 1 if on else 0))

    def reset_history(self):
        """RESET's history clear (picchio.c:2711-2716)."""
        check(self.L.pk_reset_history(self.h))

    def sample_logits(self, logits_dev, vocab=None):
        """sample_logits on a device fp32 vector, modified in place as the
        reference modifies its array; returns the token id."""
        tok = C.c_int32()
        n = logits_dev.numel() if vocab is None else vocab
        check(self.L.pk_sample_logits(self.h, ptr(logits_dev), n, C.byref(tok)))
        return tok.value

    def sampler_state(self):
        """(rng state, repetition-penalty history) of the device sampler."""
        import numpy as np
        rng = C.c_uint64()
        n = C.c_int()
        hist = np.zeros(4096, np.int32)
        check(self.L.pk_sampler_state(self.h, C.byref(rng), ptr(hist), len(hist), C.byref(n)))
        return rng.value, hist[:n.value].copy()

    def store_expert(self, layer, eid, gu_q4, gu_s, d_q4, d_s, gu_b, d_b):
        c = self.cfg
        gu = PkQtHost(FMT_INT4, gu_q4.ctypes.data, gu_s.ctypes.data, c.moe_inter, c.hidden, c.group_size)
        dn = PkQtHost(FMT_INT4, d_q4.ctypes.data, d_s.ctypes.data, c.hidden, c.moe_inter // 2, c.group_size)
        check(self.L.pk_store_expert(self.h, layer, eid, C.byref(gu), C.byref(dn),
                                     ptr(gu_b), ptr(d_b)))

    def store_router(self, layer, router, bias):
        lh = PkLayerHost()
        lh.router = router.ctypes.data
        lh.router_bias = bias.ctypes.data
        check(self.L.pk_store_layer(self.h, layer, C.byref(lh)))

    def router_logits(self, layer, x_dev, logits_dev):
        """moe_forward's router launch alone: logits_dev[E] = R x + b."""
        check(self.L.pk_router_logits(self.h, layer, ptr(x_dev), ptr(logits_dev)))

    def moe_forward(self, layer, x_dev, out_dev, want_routing=False):
        import numpy as np
        if want_routing:
            sel = np.empty(self.cfg.topk, np.int32)
            w = np.empty(self.cfg.topk, np.float32)
            check(self.L.pk_moe_forward(self.h, layer, ptr(x_dev), ptr(out_dev), ptr(sel), ptr(w)))
            return sel, w
        check(self.L.pk_moe_forward(self.h, layer, ptr(x_dev), ptr(out_dev), None, None))
        return None

    def store_layer(self, layer, in_ln, post_ln, wq, wk, wv, wo, bq, bk, bv, bo, sinks,
                    router=None, router_bias=None):
        """Dense tensors of one layer (host fp32 numpy arrays)."""
        c = self.cfg
        H, KVH, hd, D = c.n_heads, c.n_kv_heads, c.head_dim, c.hidden
        lh = PkLayerHost()
        keep = [in_ln, post_ln, wq, wk, wv, wo, bq, bk, bv, bo, sinks, router, router_bias]
        lh.in_ln, lh.post_ln = in_ln.ctypes.data, post_ln.ctypes.data
        lh.wq = PkQtHost(FMT_F32, wq.ctypes.data, None, H * hd, D, 0)
        lh.wk = PkQtHost(FMT_F32, wk.ctypes.data, None, KVH * hd, D, 0)
        lh.wv = PkQtHost(FMT_F32, wv.ctypes.data, None, KVH * hd, D, 0)
        lh.wo = PkQtHost(FMT_F32, wo.ctypes.data, None, D, H * hd, 0)
        lh.bq, lh.bk, lh.bv, lh.bo = bq.ctypes.data, bk.ctypes.data, bv.ctypes.data, bo.ctypes.data
        lh.sinks = sinks.ctypes.data
        if router is not None:
            lh.router, lh.router_bias = router.ctypes.data, router_bias.ctypes.data
        check(self.L.pk_store_layer(self.h, layer, C.byref(lh)))
        del keep

    def store_globals(self, embed, lm_head, final_norm, lm_scales=None):
        c = self.cfg
        emb = PkQtHost(FMT_F32, embed.ctypes.data, None, c.vocab, c.hidden, 0)
        if lm_scales is None:
            lm = PkQtHost(FMT_F32, lm_head.ctypes.data, None, c.vocab, c.hidden, 0)
        else:
            lm = PkQtHost(FMT_INT8, lm_head.ctypes.data, lm_scales.ctypes.data, c.vocab, c.hidden, 0)
        check(self.L.pk_store_globals(self.h, C.byref(emb), C.byref(lm), ptr(final_norm)))

    def forward_token(self, tok, pos, logits_dev=None):
        nxt = C.c_int32()
        check(self.L.pk_forward_token(self.h, tok, pos, C.byref(nxt),
                                      ptr(logits_dev) if logits_dev is not None else None))
        return nxt.value

    def gqa_attention(self, layer, x_dev, pos, out_dev):
        check(self.L.pk_gqa_attention(self.h, layer, ptr(x_dev), pos, ptr(out_dev)))

    def generate(self, prompt, n_steps):
        import numpy as np
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(max(n_steps, 1), np.int32)
        check(self.L.pk_generate(self.h, ptr(p), len(p), n_steps, ptr(out)))
        return out[:n_steps]

    def prefill_tokens(self, ids, pos_base=0):
        import numpy as np
        p = np.ascontiguousarray(ids, np.int32)
        nxt = C.c_int32()
        check(self.L.pk_prefill_tokens(self.h, ptr(p), len(p), pos_base, C.byref(nxt)))
        return nxt.value

    def batch_reserve(self, n_seq):
        check(self.L.pk_batch_reserve(self.h, n_seq))

    def kv_fill_synthetic(self, seq, n_pos, seed):
        check(self.L.pk_kv_fill_synthetic(self.h, seq, n_pos, seed))

    def prefill_seq(self, seq, ids, pos_base=0):
        import numpy as np
        p = np.ascontiguousarray(ids, np.int32)
        nxt = C.c_int32()
        check(self.L.pk_prefill_seq(self.h, seq, ptr(p), len(p), pos_base, C.byref(nxt)))
        return nxt.value

    def decode_batch(self, toks, pos, n_steps):
        import numpy as np
        t = np.ascontiguousarray(toks, np.int32)
        out = np.empty((n_steps, len(t)), np.int32)
        check(self.L.pk_decode_batch(self.h, len(t), ptr(t), pos, n_steps, ptr(out)))
        return out

    def decode_replay(self, tok, pos, n_steps):
        import numpy as np
        out = np.empty(n_steps, np.int32)
        check(self.L.pk_decode_replay(self.h, tok, pos, n_steps, ptr(out)))
        return out

    def expert_apply(self, layer, eid, x_dev, dst_dev, w):
        check(self.L.pk_expert_apply(self.h, layer, eid, ptr(x_dev), ptr(dst_dev), w))

    def moe_forward_batch(self, layer, x_dev, out_dev, sel_dev=None, w_dev=None):
        T = x_dev.shape[0]
        check(self.L.pk_moe_forward_batch(self.h, layer, ptr(x_dev), T, ptr(out_dev),
                                          ptr(sel_dev) if sel_dev is not None else None,
                                          ptr(w_dev) if w_dev is not None else None))

    def moe_forward_grouped(self, layer, x_dev, out_dev, sel_dev=None, w_dev=None, act_dev=None,
                            eo_dev=None):
        T = x_dev.shape[0]
        opt = lambda t: ptr(t) if t is not None else None
        check(self.L.pk_moe_forward_grouped(self.h, layer, ptr(x_dev), T, opt(sel_dev), opt(w_dev),
                                            ptr(out_dev), opt(act_dev), opt(eo_dev)))

    def quantize_act_i8x3(self, x_dev, limbs_dev, exps_dev):
        rows, cols = x_dev.shape
        check(self.L.pk_quantize_act_i8x3(self.h, ptr(x_dev), rows, cols, ptr(limbs_dev), ptr(exps_dev)))

    def expert_gate_up(self, layer, eids_dev, x_dev, act_dev):
        check(self.L.pk_expert_gate_up(self.h, layer, ptr(eids_dev), eids_dev.numel(),
                                       ptr(x_dev), ptr(act_dev)))

    def expert_down(self, layer, eids_dev, act_dev, eo_dev):
        check(self.L.pk_expert_down(self.h, layer, ptr(eids_dev), eids_dev.numel(),
                                    ptr(act_dev), ptr(eo_dev)))

    def qt_upload(self, fmt, data, scales, O, I, block_size=0):
        q = PkQtHost(fmt, data.ctypes.data, scales.ctypes.data if scales is not None else None,
                     O, I, block_size)
        h = C.c_void_p()
        check(self.L.pk_qt_upload(self.h, C.byref(q), C.byref(h)))
        return h

    def qt_free(self, h):
        check(self.L.pk_qt_free(self.h, h))

    def matmul_qt(self, y_dev, x_dev, qt, S):
        check(self.L.pk_matmul_qt(self.h, ptr(y_dev), ptr(x_dev), qt, S))

    def quantize_int4_gs(self, w_dev, O, I, gs, packed_dev, scales_dev):
        check(self.L.pk_quantize_int4_gs(self.h, ptr(w_dev), O, I, gs, ptr(packed_dev), ptr(scales_dev)))
