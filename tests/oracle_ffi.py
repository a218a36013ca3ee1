"""ctypes bindings for the CPU parity checker (oracle/liboracle.so) and, where
it was built, picchio's own code (oracle/_ref/libpicchio_ref.so).

Test infrastructure: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py only.
"""
import ctypes as C
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "liboracle.so")
REF_SO = os.path.join(ORACLE_DIR, "_ref", "libpicchio_ref.so")

def _nd(dtype):
    """ndpointer that also accepts None (optional outputs)."""
    base = np.ctypeslib.ndpointer(dtype, flags="C_CONTIGUOUS")

    def from_param(cls, obj):
        if obj is None:
            return None
        return base.from_param(obj)
    return type(f"nd_{np.dtype(dtype).name}", (base,), {"from_param": classmethod(from_param)})


f32p = _nd(np.float32)
u8p = _nd(np.uint8)
i8p = _nd(np.int8)
i32p = _nd(np.int32)


from picchio_amd import PkCfg, gptoss_cfg  # noqa: E402  (struct layout only)


def make_cfg(**kw):
    """GPT-OSS-20B-shaped configuration; keywords override."""
    return gptoss_cfg(**kw)


def _bind(lib, name, res, *args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = list(args)
    return fn


class Oracle:
    """The C restatement (pk_oracle.c)."""

    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            subprocess.check_call(["make", "-s", "-C", ORACLE_DIR, "oracle"])
        self.lib = L = C.CDLL(path)
        vp = C.c_void_p
        self.quantize_int4_gs = _bind(L, "po_quantize_int4_gs", None, f32p, C.c_int, C.c_int, C.c_int, u8p, f32p)
        self.quantize_int8_rows = _bind(L, "po_quantize_int8_rows", None, f32p, C.c_int, C.c_int, i8p, f32p)
        self.quantize_rows_i4 = _bind(L, "po_quantize_rows_i4", None, f32p, C.c_int, C.c_int, u8p, f32p)
        self.matmul_f32 = _bind(L, "po_matmul_f32", None, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int)
        self.matmul_q8 = _bind(L, "po_matmul_q8", None, f32p, f32p, i8p, f32p, C.c_int, C.c_int, C.c_int)
        self.matmul_i4 = _bind(L, "po_matmul_i4", None, f32p, f32p, u8p, f32p, C.c_int, C.c_int, C.c_int)
        self.matmul_i4_gs = _bind(L, "po_matmul_i4_gs", None, f32p, f32p, u8p, f32p, C.c_int, C.c_int, C.c_int, C.c_int)
        self.rmsnorm = _bind(L, "po_rmsnorm", None, f32p, f32p, f32p, C.c_int, C.c_float)
        self.softmax = _bind(L, "po_softmax", None, f32p, C.c_int)
        self.swiglu_clamped = _bind(L, "po_swiglu_clamped", None, f32p, C.c_int, C.c_float, C.c_float)
        self.model_build = _bind(L, "po_model_build", vp, C.POINTER(PkCfg), C.c_uint64, C.c_int)
        self.model_free = _bind(L, "po_model_free", None, vp)
        self.model_reset_kv = _bind(L, "po_model_reset_kv", None, vp)
        self.model_fill_kv = _bind(L, "po_model_fill_kv", None, vp, C.c_int, C.c_int, C.c_uint64, C.c_uint64)
        self.model_tensor = _bind(L, "po_model_tensor", vp, vp, C.c_int, C.c_int, C.POINTER(vp))
        self._model_expert = _bind(L, "po_model_expert", C.c_int, vp, C.c_int, C.c_int,
                                   *([C.POINTER(vp)] * 6))
        self._fill_normal = _bind(L, "po_fill_normal", None, C.c_uint64, C.c_int, C.c_int, C.c_int,
                                  C.c_int64, C.c_int64, C.c_float, f32p)
        self.expert_apply = _bind(L, "po_expert_apply", None, vp, C.c_int, C.c_int, f32p, f32p, C.c_float)
        self.moe_forward = _bind(L, "po_moe_forward", None, vp, C.c_int, f32p, f32p, i32p, f32p, f32p)
        self.gqa_attention = _bind(L, "po_gqa_attention", None, vp, C.c_int, f32p, C.c_int, f32p)
        self.rope_apply = _bind(L, "po_rope_apply", None, C.POINTER(PkCfg), f32p, f32p, C.c_int)
        self.yarn_inv_freq = _bind(L, "po_yarn_inv_freq", C.c_float, C.POINTER(PkCfg), C.c_int)
        self.forward_token = _bind(L, "po_forward_token", C.c_int, vp, C.c_int, C.c_int, vp)
        self.set_router_trace = _bind(L, "po_set_router_trace", None, vp, C.c_int64)
        self.router_trace_used = _bind(L, "po_router_trace_used", C.c_int64)
        self.forward_prefill = _bind(L, "po_forward_prefill", C.c_int, vp, i32p, C.c_int, C.c_int)
        self.prefill_tokens = _bind(L, "po_prefill_tokens", C.c_int, vp, i32p, C.c_int, C.c_int, C.c_int)
        self.argmax = _bind(L, "po_argmax", C.c_int, f32p, C.c_int)
        self._sampler_init = _bind(L, "po_sampler_init", None, C.c_void_p, C.c_float, C.c_float, C.c_int,
                                   C.c_float, C.c_uint64)
        self._sample_logits = _bind(L, "po_sample_logits", C.c_int, C.c_void_p, f32p, C.c_int)
        self._sample_logits_fx = _bind(L, "po_sample_logits_fx", C.c_int, C.c_void_p, f32p, C.c_int)
        self.act_records = _bind(L, "po_act_records", None, f32p, C.c_int, i32p)
        self.i4_dot_matvec = _bind(L, "po_i4_dot_matvec", None, u8p, f32p, C.c_void_p, C.c_int, C.c_int,
                                   i32p, f32p)
        self.rng_float = _bind(L, "po_rng_float", C.c_float, C.POINTER(C.c_uint64))
        self.act_limbs = _bind(L, "po_act_limbs", None, f32p, C.c_int, C.c_int, i8p, i32p)
        self.mfma_matvec = _bind(L, "po_mfma_matvec", None, u8p, f32p, _nd(np.float32), C.c_int, C.c_int,
                                 i8p, i8p, i8p, C.c_int, f32p)

    def normal(self, seed, kind, layer, idx, n, std=1.0, first=0):
        out = np.empty(n, np.float32)
        self._fill_normal(seed, kind, layer, idx, first, n, std, out)
        return out

    def quant_gs(self, w, gs=64):
        O, I = w.shape
        ng = 1 if (gs <= 0 or gs >= I) else (I + gs - 1) // gs
        packed = np.empty((O, (I + 1) // 2), np.uint8)
        scales = np.empty((O, ng), np.float32)
        self.quantize_int4_gs(np.ascontiguousarray(w, np.float32), O, I, gs, packed, scales)
        return packed, scales

    def mm_i4_gs(self, x, q4, s, O, I, gs):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, I)
        y = np.empty((x.shape[0], O), np.float32)
        self.matmul_i4_gs(y, x, np.ascontiguousarray(q4), np.ascontiguousarray(s, np.float32),
                          x.shape[0], I, O, gs)
        return y

    def expert_arrays(self, model, layer, eid, cfg):
        """Copies of one expert's tensors (reference layout) from a po_model."""
        ptrs = [C.c_void_p() for _ in range(6)]
        rc = self._model_expert(model, layer, eid, *[C.byref(p) for p in ptrs])
        assert rc == 0
        D, inter, gs = cfg.hidden, cfg.moe_inter, cfg.group_size
        half = inter // 2

        def arr(p, ctype, n, dt):
            return np.ctypeslib.as_array(C.cast(p, C.POINTER(ctype)), shape=(n,)).astype(dt, copy=True)
        gu_q4 = arr(ptrs[0], C.c_uint8, inter * ((D + 1) // 2), np.uint8).reshape(inter, -1)
        gu_s = arr(ptrs[1], C.c_float, inter * ((D + gs - 1) // gs), np.float32).reshape(inter, -1)
        d_q4 = arr(ptrs[2], C.c_uint8, D * ((half + 1) // 2), np.uint8).reshape(D, -1)
        d_s = arr(ptrs[3], C.c_float, D * ((half + gs - 1) // gs), np.float32).reshape(D, -1)
        gu_b = arr(ptrs[4], C.c_float, inter, np.float32)
        d_b = arr(ptrs[5], C.c_float, D, np.float32)
        return gu_q4, gu_s, d_q4, d_s, gu_b, d_b

    def sampler(self, temperature, top_p, top_k, rep_penalty, seed):
        """po_sampler state (sample_logits' globals), as a ctypes buffer."""
        st = (C.c_byte * (4 * 4 + 8 + 4 + 4 * 4096 + 4))()
        self._sampler_init(C.cast(st, C.c_void_p), temperature, top_p, top_k, rep_penalty, seed)
        return st

    def sample_logits(self, st, logits):
        return self._sample_logits(C.cast(st, C.c_void_p), logits, logits.size)

    def sample_logits_fx(self, st, logits):
        return self._sample_logits_fx(C.cast(st, C.c_void_p), logits, logits.size)

    @staticmethod
    def sampler_state(st):
        """(rng, history) of a po_sampler buffer (rng at byte 16, history_len
        at 24, history from 28)."""
        raw = bytes(st)
        rng = int.from_bytes(raw[16:24], "little")
        n = int.from_bytes(raw[24:28], "little", signed=True)
        return rng, np.frombuffer(raw[28:28 + 4 * n], np.int32).copy()

    @staticmethod
    def sampler_push_history(st, ids, vocab):
        """Append ids to a po_sampler's history as prefill_tokens seeds it
        (picchio.c:1960-1967): valid ids only, up to 4096 entries."""
        n = int.from_bytes(bytes(st)[24:28], "little", signed=True)
        hist = (C.c_int32 * 4096).from_buffer(st, 28)
        for t in ids:
            if n < 4096 and 0 <= int(t) < vocab:
                hist[n] = int(t)
                n += 1
        C.c_int32.from_buffer(st, 24).value = n

    def tensor(self, model, kind, layer, n):
        p = self.model_tensor(model, kind, layer, None)
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(n,)).copy()


class Reference:
    """picchio's own functions via oracle/_ref (only where the reference tree
    was present when it was built)."""

    def __init__(self, path=REF_SO):
        self.lib = L = C.CDLL(path)
        vp = C.c_void_p
        self.matmul_f32 = _bind(L, "ref_matmul_f32", None, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int)
        self.matmul_q8 = _bind(L, "ref_matmul_q8", None, f32p, f32p, i8p, f32p, C.c_int, C.c_int, C.c_int)
        self.matmul_i4 = _bind(L, "ref_matmul_i4", None, f32p, f32p, u8p, f32p, C.c_int, C.c_int, C.c_int)
        self.matmul_i4_gs = _bind(L, "ref_matmul_i4_gs", None, f32p, f32p, u8p, f32p, C.c_int, C.c_int, C.c_int, C.c_int)
        self.quantize_rows_i4 = _bind(L, "ref_quantize_rows_i4", None, f32p, u8p, f32p, C.c_int, C.c_int)
        self.rmsnorm = _bind(L, "ref_rmsnorm", None, f32p, f32p, f32p, C.c_int, C.c_float)
        self.softmax = _bind(L, "ref_softmax", None, f32p, C.c_int)
        self.attach = _bind(L, "ref_attach", C.c_int, vp, C.POINTER(PkCfg))
        self.reset_kv = _bind(L, "ref_reset_kv", None)
        self.moe_forward = _bind(L, "ref_moe_forward", C.c_int, C.c_int, f32p, f32p)
        self.expert_apply = _bind(L, "ref_expert_apply", C.c_int, C.c_int, C.c_int, f32p, f32p, C.c_float)
        self.gqa_attention = _bind(L, "ref_gqa_attention", C.c_int, C.c_int, f32p, C.c_int, f32p)
        self.rope_apply = _bind(L, "ref_rope_apply", None, C.POINTER(PkCfg), f32p, f32p, C.c_int)
        self.yarn_inv_freq = _bind(L, "ref_yarn_inv_freq", C.c_float, C.POINTER(PkCfg), C.c_int)
        self.forward_token = _bind(L, "ref_forward_token", C.c_int, C.c_int, C.c_int)
        self.prefill_tokens = _bind(L, "ref_prefill_tokens", C.c_int, i32p, C.c_int, C.c_int, C.c_int)
        self.set_dump_dir = _bind(L, "ref_set_dump_dir", None, C.c_char_p)
        self.sample_logits = _bind(L, "ref_sample_logits", C.c_int, f32p, C.c_int, C.c_float, C.c_float,
                                   C.c_int, C.c_float, C.POINTER(C.c_uint64), i32p, C.c_int)


def reference_available():
    return os.path.exists(REF_SO)
