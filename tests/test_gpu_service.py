"""picchio's SERVICE=1 loop (picchio.c:2697-2795) as the C program
picchio_amd/picchio_service over the C-ABI: TURN lines piped to it on a
converted checkpoint give the oracle's token stream (prefill_tokens, then
forward_token per emitted token), with the reference's frames for prefix
reuse, BAD_RANGE / BAD_TOKEN (session intact), CONTEXT_FULL, RESET,
SHUTDOWN, BAD_COMMAND and the RETURN / CALL stop ids."""
import os
import select
import subprocess
import time

import numpy as np
import pytest

from container_writer import oracle_tensors, write_container

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "picchio_amd", "picchio_service")


class Service:
    """The program with pipes; lines read against a deadline."""

    def __init__(self, model_dir, cap, seed=1):
        if not os.path.exists(BIN):
            pytest.fail("picchio_service is not built (python -m picchio_amd.build)")
        env = dict(os.environ, SERVICE="1", MODEL=model_dir, CTX=str(cap), TEMPERATURE="0", TOPP="1",
                   TOPK="0", REP="1", SEED=str(seed), IO_THREADS="4", PREFILL_BATCH="64")
        self.p = subprocess.Popen([BIN], stdin=subprocess.PIPE, stdout=subprocess.PIPE,
                                  stderr=subprocess.PIPE, env=env, bufsize=0)
        self.buf = b""

    def line(self, timeout=120.0):
        end = time.time() + timeout
        while b"\n" not in self.buf:
            left = end - time.time()
            if left <= 0:
                raise TimeoutError("no line from picchio_service")
            r, _, _ = select.select([self.p.stdout], [], [], left)
            if r:
                chunk = os.read(self.p.stdout.fileno(), 65536)
                if not chunk:
                    raise EOFError("picchio_service closed stdout: " + self.p.stderr.read().decode()[-2000:])
                self.buf += chunk
        ln, self.buf = self.buf.split(b"\n", 1)
        return ln.decode()

    def send(self, text):
        self.p.stdin.write((text + "\n").encode())
        self.p.stdin.flush()

    def turn(self, max_new, keep, ids, temp=0.0, top_p=1.0, top_k=0):
        """Sends a TURN; returns (tokens, final frame split)."""
        self.send(f"TURN {max_new} {keep} {temp} {top_p} {top_k} {len(ids)} " + " ".join(str(int(i)) for i in ids))
        toks = []
        while True:
            f = self.line().split()
            if f[0] == "TOKEN":
                toks.append(int(f[1]))
            else:
                return toks, f

    def close(self, timeout=60):
        try:
            return self.p.wait(timeout=timeout)
        finally:
            if self.p.poll() is None:
                self.p.kill()
                self.p.wait()


@pytest.fixture(scope="module")
def ckpt(gpu, oracle, tmp_path_factory):
    import picchio_amd as pa
    cfg = pa.gptoss_cfg(n_layers=2, n_experts=8, ctx_len=128, vocab=1000)
    model = oracle.model_build(cfg, 8642, 0)
    dense, experts = oracle_tensors(oracle, model, cfg)
    path = str(tmp_path_factory.mktemp("svc"))
    write_container(path, cfg, dense, experts)
    yield cfg, model, path
    oracle.model_free(model)


def _oracle_turn(oracle, model, ids, keep, max_new, cap):
    """service_loop's turn on the oracle: (emitted tokens, reason, produced, pos)."""
    pos = keep
    tok = oracle.prefill_tokens(model, np.asarray(ids, np.int32), len(ids), pos, 64)
    pos += len(ids)
    out = []
    while True:
        if len(out) >= max_new:
            return out, "MAX_TOKENS", len(out), pos
        if pos >= cap:
            return out, "CONTEXT_FULL", len(out), pos
        out.append(tok)
        nxt = oracle.forward_token(model, tok, pos, None)
        pos += 1
        tok = nxt if 0 <= nxt < 1000 else 0


def test_service_turns_match_oracle(ckpt, oracle):
    cfg, model, path = ckpt
    cap = 48
    s = Service(path, cap)
    try:
        assert s.line().split() == ["READY", str(cap), str(cfg.vocab), "200002", "200012"]
        oracle.model_reset_kv(model)
        rng = np.random.default_rng(11)
        # turn 1: a fresh prompt
        ids = rng.integers(0, cfg.vocab, 10)
        toks, done = s.turn(5, 0, ids)
        ref, reason, produced, pos = _oracle_turn(oracle, model, ids, 0, 5, cap)
        assert toks == ref and done == ["DONE", reason, str(produced), str(pos)], (toks, ref, done)
        assert pos == 15
        # turn 2: keep the whole prefix
        ids2 = rng.integers(0, cfg.vocab, 4)
        toks, done = s.turn(3, 15, ids2)
        ref, reason, produced, pos = _oracle_turn(oracle, model, ids2, 15, 3, cap)
        assert toks == ref and done == ["DONE", reason, str(produced), str(pos)]
        # turn 3: keep only part of it (positions 12.. are rewritten)
        ids3 = rng.integers(0, cfg.vocab, 6)
        toks, done = s.turn(4, 12, ids3)
        ref, reason, produced, pos = _oracle_turn(oracle, model, ids3, 12, 4, cap)
        assert toks == ref and done == ["DONE", reason, str(produced), str(pos)]
        assert pos == 22
        # BAD_RANGE (keep beyond pos): an ERROR frame, nothing changes
        assert s.turn(2, 30, [1, 2])[1] == "ERROR BAD_RANGE 0 keep/n_ids out of bounds (pos=22 cap=48)".split()
        # BAD_TOKEN: an ERROR frame, nothing changes
        assert s.turn(2, 22, [3, cfg.vocab + 5])[1] == "ERROR BAD_TOKEN 0 ID out of vocabulary".split()
        # the session is intact: continue at 22 and run into the capacity
        ids4 = rng.integers(0, cfg.vocab, 3)
        toks, done = s.turn(100, 22, ids4)
        ref, reason, produced, pos = _oracle_turn(oracle, model, ids4, 22, 100, cap)
        assert reason == "CONTEXT_FULL" and pos == cap
        assert toks == ref and done == ["DONE", reason, str(produced), str(pos)]
        # RESET: positions from 0 again, keep > 0 is out of range
        s.send("RESET")
        assert s.line().split() == ["DONE", "RESET", "0", "0"]
        assert s.turn(1, 1, [5])[1][:2] == ["ERROR", "BAD_RANGE"]
        oracle.model_reset_kv(model)
        ids5 = rng.integers(0, cfg.vocab, 8)
        toks, done = s.turn(4, 0, ids5)
        ref, reason, produced, pos = _oracle_turn(oracle, model, ids5, 0, 4, cap)
        assert toks == ref and done == ["DONE", reason, str(produced), str(pos)]
        # a zero-token turn: prefill only
        toks, done = s.turn(0, pos, [7])
        assert toks == [] and done == ["DONE", "MAX_TOKENS", "0", str(pos + 1)]
        s.send("SHUTDOWN")
        assert s.close() == 0
    finally:
        s.close(5)


def test_service_bad_command_and_header(ckpt):
    cfg, model, path = ckpt
    s = Service(path, 32)
    try:
        assert s.line().split()[0] == "READY"
        s.send("HELLO")
        assert s.line() == "ERROR BAD_COMMAND 1 unknown command"
        assert s.close() == 1
    finally:
        s.close(5)
    s = Service(path, 32)
    try:
        assert s.line().split()[0] == "READY"
        s.send("TURN 1 0 x")
        assert s.line() == "ERROR BAD_HEADER 1 unreadable TURN header"
        assert s.close() == 1
    finally:
        s.close(5)


def test_service_stop_ids(gpu, oracle, tmp_path_factory):
    """A checkpoint whose vocabulary holds the stop ids: its INT8 lm_head is
    zero but for <|return|> (+1 in every column) and <|call|> (-1), so the
    greedy token is one of them; the turn ends there with RETURN or CALL."""
    import picchio_amd as pa
    V = 200016
    small = pa.gptoss_cfg(n_layers=1, n_experts=4, ctx_len=32, vocab=64)
    model = oracle.model_build(small, 97, 0)
    dense, experts = oracle_tensors(oracle, model, small)
    oracle.model_free(model)
    cfg = pa.gptoss_cfg(n_layers=1, n_experts=4, ctx_len=32, vocab=V)
    D = cfg.hidden
    rng = np.random.default_rng(3)
    emb = (rng.integers(-127, 128, (V, D), dtype=np.int8), np.full(V, 0.01, np.float32))
    lm = np.zeros((V, D), np.int8)
    lm[200002] = 1
    lm[200012] = -1
    del dense["model.embed_tokens.weight"], dense["lm_head.weight"]
    path = str(tmp_path_factory.mktemp("svc_stop"))
    write_container(path, cfg, dense, experts, lm_int8=(lm, np.ones(V, np.float32)), embed_int8=emb)
    del emb, lm
    s = Service(path, 32)
    try:
        assert s.line().split() == ["READY", "32", str(V), "200002", "200012"]
        for ids in ([1, 2, 3], [40000, 5]):
            toks, done = s.turn(5, 0, ids)
            assert len(toks) == 1 and toks[0] in (200002, 200012), toks
            reason = "RETURN" if toks[0] == 200002 else "CALL"
            assert done == ["DONE", reason, "1", str(len(ids) + 1)], done
        s.send("SHUTDOWN")
        assert s.close() == 0
    finally:
        s.close(5)
