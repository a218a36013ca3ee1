"""BASELINE config 2 at full size: the GPT-OSS-20B-shaped model (24 layers,
32 experts, vocab 201088), a 512-token prompt of uniform random ids through
prefill_tokens (chunks of 64, picchio's default), then 256 greedy steps —
the GPU stream must equal the oracle's (itself bit-exact with picchio).

The CPU side builds the 18 GB model and runs 768 positions (about three
minutes on 16 host cores), so this test runs only with PK_FULL_STREAM=1;
the same path is covered at reduced depth by test_gpu_decode.py on every run.
"""
import os
import time

import numpy as np
import pytest

from helpers import upload_model

pytestmark = pytest.mark.gpu

N_PROMPT, N_STEPS, SEED = 512, 256, 2025


@pytest.mark.skipif(os.environ.get("PK_FULL_STREAM") != "1",
                    reason="full-size 20B stream check: set PK_FULL_STREAM=1 (about 3 min of CPU)")
def test_config2_greedy_stream_256(gpu, oracle):
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(ctx_len=N_PROMPT + N_STEPS + 1)
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    t0 = time.time()
    model = oracle.model_build(cfg, SEED, threads)
    print(f"oracle model built in {time.time() - t0:.0f} s", flush=True)
    eng = pa.Engine(cfg)
    try:
        t0 = time.time()
        upload_model(eng, oracle, model, cfg)
        print(f"uploaded in {time.time() - t0:.0f} s", flush=True)
        prompt = np.random.default_rng(SEED).integers(0, cfg.vocab, N_PROMPT).astype(np.int32)
        t0 = time.time()
        got = [int(v) for v in eng.generate(prompt, N_STEPS)]
        print(f"GPU stream in {time.time() - t0:.1f} s: {got[:12]}", flush=True)
        t0 = time.time()
        oracle.model_reset_kv(model)
        ref = [oracle.prefill_tokens(model, prompt, N_PROMPT, 0, 64)]
        for i in range(N_STEPS - 1):
            ref.append(oracle.forward_token(model, ref[-1], N_PROMPT + i, None))
        print(f"oracle stream in {time.time() - t0:.0f} s: {ref[:12]}", flush=True)
        first = next((i for i, (a, b) in enumerate(zip(got, ref)) if a != b), None)
        assert first is None, f"streams diverge at step {first}: {got[first:first + 4]} vs {ref[first:first + 4]}"
    finally:
        eng.close()
        oracle.model_free(model)
