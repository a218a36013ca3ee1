/* picchio_service.c — picchio's SERVICE=1 mode over the C-ABI of
 * libpicchio_hip.so: a persistent multi-turn session on one GPU, speaking
 * service_loop's protocol (picchio.c:2697-2795) on stdin / stdout.
 *
 *   start-up (picchio.c main, :2800-3082): MODEL (or argv[1]) = the converted
 *   checkpoint directory; CTX = KV capacity in positions (default 512, at
 *   most the config's max_position_embeddings, :2931-2936); TEMPERATURE,
 *   TOPP, TOPK, REP, SEED = the sampler's settings (defaults 1.0 / 0.95 / 50
 *   / 1.1 and a time seed, :1510-1513, :3031-3038). SERVICE must be set to a
 *   non-zero value: the interactive and batch modes of picchio's main (the
 *   tokenizer, the chat template) are not part of this program.
 *
 *   protocol (stdout carries only the protocol, stderr diagnostics):
 *     READY <cap> <vocab> <stop0> <stop1>
 *     TURN <max_new> <keep> <temp> <top_p> <top_k> <n_ids> <id>...
 *         -> TOKEN <id> ... then DONE <MAX_TOKENS|CONTEXT_FULL|RETURN|CALL>
 *            <produced> <pos>
 *         -> ERROR BAD_RANGE 0 ... / ERROR BAD_TOKEN 0 ... (session intact)
 *     RESET    -> DONE RESET 0 0
 *     SHUTDOWN -> exit 0
 *     anything else -> ERROR BAD_COMMAND 1 ..., exit 1; an unreadable TURN
 *     header -> ERROR BAD_HEADER 1 ..., exit 1.
 *   The TURN's sampling is applied (with its clamp) before the range check,
 *   and nothing in the KV cache changes before the ids are validated, as in
 *   the reference. `keep` positions of the cache are reused: the turn's ids
 *   go in at pos = keep.
 *
 *   No reference counterpart: a failing GPU call prints
 *   ERROR ENGINE 1 <message> and exits 1 (the CPU reference cannot fail
 *   there). */
#include <limits.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "picchio_hip.h"

/* picchio.c:410-412: <|return|>, <|call|> */
enum { STOP_RETURN = 200002, STOP_CALL = 200012 };

static int engine_failed(const char *what) {
    printf("ERROR ENGINE 1 %s: %s\n", what, pk_last_error());
    fflush(stdout);
    return 1;
}

static float env_f(const char *name, float def) {
    const char *v = getenv(name);
    return v ? (float)atof(v) : def;
}

static int service_loop(pk_engine *e, const pk_cfg *c, int cap) {
    int pos = 0;
    printf("READY %d %d %d %d\n", cap, c->vocab, STOP_RETURN, STOP_CALL);
    fflush(stdout);

    char cmd[32];
    while (scanf("%31s", cmd) == 1) {
        if (strcmp(cmd, "SHUTDOWN") == 0) break;

        if (strcmp(cmd, "RESET") == 0) {
            /* positions are overwritten from 0 on; the penalty history empties */
            pos = 0;
            if (pk_reset_history(e) != PK_OK) return engine_failed("reset");
            printf("DONE RESET 0 0\n");
            fflush(stdout);
            continue;
        }

        if (strcmp(cmd, "TURN") != 0) {
            printf("ERROR BAD_COMMAND 1 unknown command\n");
            fflush(stdout);
            return 1;
        }

        long max_new = 0, keep = 0, n_ids = 0, t_topk = 0;
        float t_temp = 0.0f, t_topp = 0.0f;
        if (scanf("%ld %ld %f %f %ld %ld", &max_new, &keep, &t_temp, &t_topp, &t_topk, &n_ids) != 6) {
            printf("ERROR BAD_HEADER 1 unreadable TURN header\n");
            fflush(stdout);
            return 1;
        }
        /* the turn's sampling, clamped by the engine as picchio.c:2737-2743 */
        if (pk_set_turn_sampling(e, t_temp, t_topp, t_topk > INT_MAX ? INT_MAX : (int)t_topk) != PK_OK)
            return engine_failed("sampling");
        if (max_new < 0 || keep < 0 || keep > pos || n_ids <= 0 || keep + n_ids > cap || n_ids > cap) {
            printf("ERROR BAD_RANGE 0 keep/n_ids out of bounds (pos=%d cap=%d)\n", pos, cap);
            fflush(stdout);
            /* nothing changed: discard the turn's ids, the session stays usable */
            for (long i = 0; i < n_ids; i++) {
                long skip;
                if (scanf("%ld", &skip) != 1) return 1;
            }
            continue;
        }

        int32_t *ids = (int32_t *)malloc((size_t)n_ids * sizeof(int32_t));
        if (!ids) return 1;
        int valid = 1;
        for (long i = 0; i < n_ids; i++) {
            long value;
            if (scanf("%ld", &value) != 1) {
                free(ids);
                return 1;
            }
            if (value < 0 || value >= c->vocab) valid = 0;
            ids[i] = (int32_t)value;
        }
        if (!valid) {
            free(ids);
            printf("ERROR BAD_TOKEN 0 ID out of vocabulary\n");
            fflush(stdout);
            continue;
        }

        /* the prefix up to `keep` stays; the turn's ids overwrite from there */
        pos = (int)keep;
        int32_t next = 0;
        const int rc = pk_prefill_tokens(e, ids, (int)n_ids, pos, &next);
        free(ids);
        if (rc != PK_OK) return engine_failed("prefill");
        pos += (int)n_ids;

        const char *reason = "MAX_TOKENS";
        int produced = 0;
        int tok = next;
        while (1) {
            if (produced >= max_new) { reason = "MAX_TOKENS"; break; }
            if (pos >= cap) { reason = "CONTEXT_FULL"; break; }
            printf("TOKEN %d\n", tok);
            fflush(stdout);
            produced++;
            int32_t following = 0;
            if (pk_forward_token(e, tok, pos, &following, NULL) != PK_OK) return engine_failed("forward");
            pos++;
            if (tok == STOP_RETURN) { reason = "RETURN"; break; }
            if (tok == STOP_CALL) { reason = "CALL"; break; }
            tok = (following < 0 || following >= c->vocab) ? 0 : following;
        }
        printf("DONE %s %d %d\n", reason, produced, pos);
        fflush(stdout);
    }
    return 0;
}

int main(int argc, char **argv) {
    const char *model = getenv("MODEL");
    if (!model && argc > 1) model = argv[1];
    const char *svc = getenv("SERVICE");
    if (!model || !svc || atoi(svc) == 0) {
        fprintf(stderr, "usage: SERVICE=1 MODEL=/path/to/checkpoint %s  (or SERVICE=1 %s /path)\n", argv[0],
                argv[0]);
        return 1;
    }

    pk_cfg cfg;
    if (pk_cfg_from_container(model, 0, &cfg) != PK_OK) {
        fprintf(stderr, "error: %s\n", pk_last_error());
        return 1;
    }
    int cap = 512;
    const char *ctx = getenv("CTX");
    if (ctx) cap = atoi(ctx);
    if (cap > cfg.ctx_len) cap = cfg.ctx_len;
    if (cap < 1) {
        fprintf(stderr, "error: KV capacity %d\n", cap);
        return 1;
    }
    cfg.ctx_len = cap;

    pk_engine *e = NULL;
    const char *dev = getenv("PK_DEVICE");
    if (pk_engine_create(&cfg, dev ? atoi(dev) : 0, &e) != PK_OK) {
        fprintf(stderr, "error: %s\n", pk_last_error());
        return 1;
    }
    const char *io = getenv("IO_THREADS");
    const clock_t t0 = clock();
    if (pk_load_container(e, model, io ? atoi(io) : 8) != PK_OK) {
        fprintf(stderr, "error: %s\n", pk_last_error());
        pk_engine_destroy(e);
        return 1;
    }
    fprintf(stderr, "loaded %s: %d layers, %d experts, vocab %d, %.2f GB resident (%.1f s cpu)\n", model,
            cfg.n_layers, cfg.n_experts, cfg.vocab, (double)pk_engine_device_bytes(e) / 1e9,
            (double)(clock() - t0) / CLOCKS_PER_SEC);

    const char *seed = getenv("SEED");
    const uint64_t s = seed ? (uint64_t)atoll(seed) : (uint64_t)time(NULL);
    const char *topk = getenv("TOPK");
    if (pk_set_sampling(e, env_f("TEMPERATURE", 1.0f), env_f("TOPP", 0.95f), topk ? atoi(topk) : 50,
                        env_f("REP", 1.1f), s) != PK_OK) {
        fprintf(stderr, "error: %s\n", pk_last_error());
        pk_engine_destroy(e);
        return 1;
    }
    fprintf(stderr, "service: persistent session, KV capacity %d positions\n", cap);
    const int rc = service_loop(e, &cfg, cap);
    pk_engine_destroy(e);
    return rc;
}
