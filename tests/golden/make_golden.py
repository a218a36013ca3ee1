#!/usr/bin/env python3
"""Writes the golden vectors under tests/golden/ from picchio's own C code.

Run in the development container only (it needs oracle/_ref, built from the
reference sources by `make -C oracle ref`). Every fixture is data: seeded
inputs and the outputs picchio's functions produced for them, as .npz
(numpy arrays, no pickles). Model-level fixtures record the configuration and
seed; the tests rebuild the same weights with the oracle's generator
(po_model_build), which is also what the reference ran on here.

    python tests/golden/make_golden.py            # kernel and tiny-model vectors
    python tests/golden/make_golden.py config2    # config-2 stream (~18 GB RAM)
    python tests/golden/make_golden.py sampling   # sample_logits sequences
"""
import os
import shutil
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle_ffi import Oracle, Reference, make_cfg  # noqa: E402

# Small model geometry used by the model-level fixtures (every width a
# multiple of 64 so the GPU tiled path can load the same model).
TINY = dict(hidden=128, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=32, n_experts=8,
            topk=4, moe_inter=256, vocab=300, ctx_len=64, sliding_window=16)
TINY_SEED = 4242


def cfg_array(cfg):
    """pk_cfg as a flat record of its scalar fields (+ layer_type)."""
    names = [f for f, _ in cfg._fields_ if f != "layer_type"]
    return {f"cfg_{n}": np.array(getattr(cfg, n)) for n in names} | \
        {"cfg_layer_type": np.array(list(cfg.layer_type), np.int8)}


def save(name, **arrs):
    path = os.path.join(HERE, name)
    np.savez_compressed(path, **arrs)
    print(f"{name}: {os.path.getsize(path)} bytes")


def kernels(ref, rng):
    # INT4 group-scaled matmul (quant.h:259-319): random nibbles and scales, ragged shapes
    cases = [(37, 200, 64, 2), (16, 101, 32, 2), (5, 50, 64, 3), (9, 130, 48, 1),
             (7, 33, 33, 1), (8, 2880, 64, 1), (3, 17, 64, 2)]
    out = {}
    for i, (O, I, gs, S) in enumerate(cases):
        ng = (I + gs - 1) // gs
        x = rng.standard_normal((S, I)).astype(np.float32)
        q4 = rng.integers(0, 256, (O, (I + 1) // 2), dtype=np.uint8)
        s = (rng.random((O, ng)) * 0.01 + 1e-4).astype(np.float32)
        y = np.empty((S, O), np.float32)
        ref.matmul_i4_gs(y, x, q4, s, S, I, O, gs)
        out.update({f"c{i}_shape": np.array([O, I, gs, S]), f"c{i}_x": x, f"c{i}_q4": q4,
                    f"c{i}_s": s, f"c{i}_y": y})
    save("matmul_i4_gs.npz", n=np.array(len(cases)), **out)

    # fp32, int8-row, int4-row matmuls (quant.h:117-148, :152-186, :191-253)
    out = {}
    cases = [(1, 13, 5), (2, 2880, 7), (3, 37, 4), (1, 8, 3), (2, 1, 2), (1, 4101, 3)]
    for i, (S, I, O) in enumerate(cases):
        x = rng.standard_normal((S, I)).astype(np.float32)
        W = (rng.standard_normal((O, I)) * 0.02).astype(np.float32)
        q8 = rng.integers(-127, 128, (O, I), dtype=np.int8)
        s8 = (rng.random(O) * 0.01 + 1e-4).astype(np.float32)
        q4 = rng.integers(0, 256, (O, (I + 1) // 2), dtype=np.uint8)
        s4 = (rng.random(O) * 0.01 + 1e-4).astype(np.float32)
        yf, y8, y4 = (np.empty((S, O), np.float32) for _ in range(3))
        ref.matmul_f32(yf, x, W, S, I, O)
        ref.matmul_q8(y8, x, q8, s8, S, I, O)
        ref.matmul_i4(y4, x, q4, s4, S, I, O)
        out.update({f"c{i}_shape": np.array([S, I, O]), f"c{i}_x": x, f"c{i}_W": W,
                    f"c{i}_q8": q8, f"c{i}_s8": s8, f"c{i}_q4": q4, f"c{i}_s4": s4,
                    f"c{i}_yf": yf, f"c{i}_y8": y8, f"c{i}_y4": y4})
    save("matmul_dense.npz", n=np.array(len(cases)), **out)

    # per-row INT4 quantizer (quant.h:366-392), incl. the self-test matrix and a zero row
    W0 = ((np.arange(32, dtype=np.float32) - 16) * np.float32(0.1)).reshape(4, 8)
    W1 = (rng.standard_normal((6, 45)) * 0.02).astype(np.float32)
    W1[2] = 0.0
    out = {}
    for i, W in enumerate((W0, W1)):
        O, I = W.shape
        q4 = np.empty((O, (I + 1) // 2), np.uint8)
        s = np.empty(O, np.float32)
        ref.quantize_rows_i4(W, q4, s, O, I)
        out.update({f"c{i}_w": W, f"c{i}_q4": q4, f"c{i}_s": s})
    save("quantize_rows_i4.npz", n=np.array(2), **out)

    # rmsnorm (quant.h:396-402) and softmax (quant.h:406-412)
    xs = [np.array([1, 2, 3, 4], np.float32), rng.standard_normal(2880).astype(np.float32),
          (rng.standard_normal(37) * 50).astype(np.float32)]
    out = {}
    for i, x in enumerate(xs):
        w = (1 + 0.1 * rng.standard_normal(x.size)).astype(np.float32)
        o = np.empty_like(x)
        ref.rmsnorm(o, x, w, x.size, 1e-5)
        sm = x.copy()
        ref.softmax(sm, sm.size)
        out.update({f"c{i}_x": x, f"c{i}_w": w, f"c{i}_rms": o, f"c{i}_softmax": sm})
    save("norm_softmax.npz", n=np.array(len(xs)), **out)


def rope(ref):
    # YaRN inverse frequencies and RoPE (picchio.c:431-473), GPT-OSS settings
    cfg = make_cfg()
    hd = cfg.head_dim
    inv = np.array([ref.yarn_inv_freq(cfg, j) for j in range(hd // 2)], np.float32)
    rng = np.random.default_rng(5)
    pos = np.array([0, 1, 7, 127, 1000, 4095, 70000], np.int32)
    q_in = rng.standard_normal((len(pos), cfg.n_heads * hd)).astype(np.float32)
    k_in = rng.standard_normal((len(pos), cfg.n_kv_heads * hd)).astype(np.float32)
    q_out, k_out = q_in.copy(), k_in.copy()
    for i, p in enumerate(pos):
        ref.rope_apply(cfg, q_out[i], k_out[i], int(p))
    save("rope_yarn.npz", inv_freq=inv, pos=pos, q_in=q_in, k_in=k_in, q_out=q_out,
         k_out=k_out, **cfg_array(cfg))


def model_level(oracle, ref):
    cfg = make_cfg(**TINY)
    model = oracle.model_build(cfg, TINY_SEED, 0)
    assert ref.attach(model, cfg) == 0
    D = cfg.hidden
    rng = np.random.default_rng(17)

    # moe_forward (picchio.c:1309-1466) on 8 tokens of each layer
    xs = rng.standard_normal((2, 8, D)).astype(np.float32)
    moe = np.empty_like(xs)
    for layer in range(2):
        for t in range(8):
            assert ref.moe_forward(layer, xs[layer, t], moe[layer, t]) == 0

    # gqa_attention (picchio.c:504-623), positions 0..39 on both layers
    # (layer 0 sliding window 16, layer 1 full), KV written as it goes
    ref.reset_kv()
    ax = rng.standard_normal((40, 2, D)).astype(np.float32)
    att = np.empty_like(ax)
    for pos in range(40):
        for layer in range(2):
            assert ref.gqa_attention(layer, ax[pos, layer], pos, att[pos, layer]) == 0

    # greedy decode (forward_token, picchio.c:1655-1756): 6-token prompt, 24 steps
    ref.reset_kv()
    prompt = rng.integers(0, cfg.vocab, 6).astype(np.int32)
    nxt = None
    for pos, tok in enumerate(prompt):
        nxt = ref.forward_token(int(tok), pos)
    stream = [nxt]
    for i in range(23):
        stream.append(ref.forward_token(stream[-1], len(prompt) + i))

    # batched prefill (prefill_tokens, picchio.c:1936-1975, chunks of 4) then decode
    ref.reset_kv()
    nxt_p = ref.prefill_tokens(prompt, len(prompt), 0, 4)
    stream_p = [nxt_p]
    for i in range(7):
        stream_p.append(ref.forward_token(stream_p[-1], len(prompt) + i))

    save("model_tiny.npz", seed=np.array(TINY_SEED), moe_x=xs, moe_out=moe, att_x=ax,
         att_out=att, prompt=prompt, stream=np.array(stream, np.int32),
         prefill_stream=np.array(stream_p, np.int32), **cfg_array(cfg))
    oracle.model_free(model)


# GPT-OSS-20B shape, 512-token prompt, 256 greedy tokens.
C2_PROMPT, C2_STEPS, C2_SEED = 512, 256, 2025
C2_LOGIT_STEPS = (1, 255)       # decode steps whose full logits are kept


def config2_stream(oracle, ref, small=None, out="config2_stream.npz"):
    """picchio's own greedy stream on the full-size config-2 model: the
    prompt through prefill_tokens (chunks of 64), then forward_token; the
    logits of every decode step come from picchio's ORACLE_DIR dump
    (picchio.c:1746). Keeps the ids, each step's top-1 minus top-2 logit and
    the whole logit vector of the steps in C2_LOGIT_STEPS. About 18 GB of
    host memory and a few minutes of CPU."""
    cfg = make_cfg(**dict(small or {}, ctx_len=C2_PROMPT + C2_STEPS + 1))
    model = oracle.model_build(cfg, C2_SEED, 0)
    assert ref.attach(model, cfg) == 0
    ref.reset_kv()
    prompt = np.random.default_rng(C2_SEED).integers(0, cfg.vocab, C2_PROMPT).astype(np.int32)
    ids = [ref.prefill_tokens(prompt, C2_PROMPT, 0, 64)]
    margins = [np.nan]
    kept = {}
    dump = tempfile.mkdtemp(prefix="pk_c2_")
    dump_c = dump.encode()          # picchio keeps the pointer: keep the bytes alive
    try:
        ref.set_dump_dir(dump_c)
        for i in range(C2_STEPS - 1):
            ids.append(ref.forward_token(ids[-1], C2_PROMPT + i))
            lg = np.load(os.path.join(dump, "logits.npy"), allow_pickle=False).reshape(-1)
            assert lg.size == cfg.vocab and int(np.argmax(lg)) == ids[-1]
            top = np.sort(lg)[-2:]
            margins.append(float(top[1]) - float(top[0]))
            if len(ids) - 1 in C2_LOGIT_STEPS:
                kept[f"logits_step{len(ids) - 1}"] = lg.astype(np.float32)
            if i % 32 == 0:
                print(f"config2: step {len(ids) - 1} id {ids[-1]} margin {margins[-1]:.3g}", flush=True)
    finally:
        ref.set_dump_dir(None)
        shutil.rmtree(dump, ignore_errors=True)
    save(out, seed=np.array(C2_SEED), prompt=prompt, stream=np.array(ids, np.int32),
         margins=np.array(margins, np.float32), logit_steps=np.array(C2_LOGIT_STEPS, np.int32),
         **kept, **cfg_array(cfg))
    oracle.model_free(model)


SAMPLE_CASES = [  # temperature, top_p, top_k, rep_penalty (the sampler tests' cases)
    (1.0, 0.95, 50, 1.1), (0.7, 1.0, 0, 1.0), (1.3, 0.5, 0, 1.0), (0.8, 1.0, 5, 1.3),
    (0.0, 0.95, 50, 1.2), (1.0, 0.9, 1, 1.0)]


def sampling(ref):
    """sample_logits (picchio.c:1509-1649) sequences per case: the logits in,
    the arrays as the function leaves them, the ids, the rng state after
    each draw; the history is the ids drawn so far (as the caller keeps it)."""
    import ctypes as C
    rng = np.random.default_rng(20261202)
    out = {}
    for ci, (t, p, k, rep) in enumerate(SAMPLE_CASES):
        for V, steps in ((64, 25), (700, 10)):
            state = C.c_uint64(777)
            hist, ins, outs, ids, states = [], [], [], [], []
            for _ in range(steps):
                lg = (rng.standard_normal(V) * 2.5).astype(np.float32)
                b = lg.copy()
                h = np.array(hist + [0], np.int32)
                tok = ref.sample_logits(b, V, t, p, k, rep, C.byref(state), h, len(hist))
                ins.append(lg)
                outs.append(b)
                ids.append(tok)
                states.append(state.value)
                hist.append(tok)
            key = f"c{ci}_v{V}"
            out.update({f"{key}_in": np.stack(ins), f"{key}_out": np.stack(outs),
                        f"{key}_ids": np.array(ids, np.int32), f"{key}_rng": np.array(states, np.uint64)})
    out["cases"] = np.array(SAMPLE_CASES, np.float64)
    out["seed"] = np.array(777, np.uint64)
    save("sample_logits.npz", **out)


def main():
    oracle, ref = Oracle(), Reference()
    if sys.argv[1:] == ["sampling"]:
        sampling(ref)
        return
    if sys.argv[1:] == ["config2"]:
        config2_stream(oracle, ref)
        return
    if sys.argv[1:] == ["config2-dry"]:     # the same recipe on a small model, not kept
        config2_stream(oracle, ref, small=TINY, out="_dry.npz")
        os.remove(os.path.join(HERE, "_dry.npz"))
        return
    rng = np.random.default_rng(20261201)
    kernels(ref, rng)
    rope(ref)
    model_level(oracle, ref)


if __name__ == "__main__":
    main()
