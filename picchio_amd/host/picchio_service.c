/* picchio_service.c — a persistent multi-turn session on one GPU, speaking
 * the wire protocol of picchio's SERVICE=1 mode (picchio.c:2697-2795) on
 * stdin / stdout, over the C-ABI of libpicchio_hip.so.
 *
 * Start-up (the parts of picchio.c main, :2800-3082, that this mode uses):
 *   MODEL (or argv[1])  converted checkpoint directory
 *   CTX                 KV capacity in positions (default 512, at most the
 *                       config's max_position_embeddings, :2931-2936)
 *   TEMPERATURE, TOPP, TOPK, REP, SEED
 *                       sampler settings (defaults 1.0 / 0.95 / 50 / 1.1
 *                       and a time seed, :1510-1513, :3031-3038)
 *   SERVICE             must be non-zero: the interactive and batch modes
 *                       (tokenizer, chat template) are not part of this
 *                       program.
 *
 * Protocol. stdout carries protocol frames only (one line each, flushed),
 * stderr diagnostics. The input is a stream of whitespace-separated fields;
 * a command is one field followed by its arguments:
 *
 *   (on start)  READY <cap> <vocab> <stop_return> <stop_call>
 *   TURN <max_new> <keep> <temp> <top_p> <top_k> <n_ids> <id>*n_ids
 *               TOKEN <id> per emitted token, then
 *               DONE <MAX_TOKENS|CONTEXT_FULL|RETURN|CALL> <produced> <pos>
 *               or ERROR BAD_RANGE 0 ... / ERROR BAD_TOKEN 0 ...
 *               (the session is unchanged and continues)
 *   RESET       DONE RESET 0 0
 *   SHUTDOWN    exit status 0 (so does the end of the input)
 *   other       ERROR BAD_COMMAND 1 ..., exit status 1; a TURN header that
 *               does not parse: ERROR BAD_HEADER 1 ..., exit status 1; the
 *               input ending inside a TURN's ids: exit status 1.
 *
 * Semantics a client relies on (the reference's):
 *  - the turn's sampling settings take effect (clamped) even when the turn
 *    is then refused;
 *  - a turn is refused before anything changes: BAD_RANGE when the counts do
 *    not fit the session (max_new < 0, keep outside [0, pos], n_ids outside
 *    [1, cap - keep]), its ids still consumed; BAD_TOKEN when any id is
 *    outside the vocabulary;
 *  - `keep` positions of the cache are reused and the ids go in at keep;
 *  - each emitted token is also fed forward, so after DONE `pos` counts the
 *    cache's valid positions; a stop id is emitted, fed, then ends the turn;
 *  - an out-of-vocabulary prediction continues as token 0.
 *
 * No reference counterpart: a failing GPU call answers
 * ERROR ENGINE 1 <message> and exits with status 1. */
#include <ctype.h>
#include <errno.h>
#include <limits.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "picchio_hip.h"

/* the stop ids of the GPT-OSS vocabulary: <|return|>, <|call|> (picchio.c:410-412) */
#define STOP_RETURN 200002
#define STOP_CALL 200012

/* ───────────── input: whitespace-separated fields ───────────── */

typedef struct {
    FILE *in;
    char field[64];   /* the current field, NUL-terminated (longer fields are cut) */
} field_reader;

/* Next field into r->field; 0 at the end of the input. */
static int next_field(field_reader *r) {
    int ch;
    do {
        ch = getc(r->in);
    } while (ch != EOF && isspace(ch));
    if (ch == EOF) return 0;
    size_t n = 0;
    while (ch != EOF && !isspace(ch)) {
        if (n + 1 < sizeof r->field) r->field[n++] = (char)ch;
        ch = getc(r->in);
    }
    r->field[n] = '\0';
    return 1;
}

/* The next field as an integer / a float; 0 if missing or malformed. */
static int field_long(field_reader *r, long *v) {
    if (!next_field(r)) return 0;
    char *end = NULL;
    errno = 0;
    *v = strtol(r->field, &end, 10);
    return end != r->field && *end == '\0' && errno == 0;
}

static int field_float(field_reader *r, float *v) {
    if (!next_field(r)) return 0;
    char *end = NULL;
    *v = strtof(r->field, &end);
    return end != r->field && *end == '\0';
}

/* ───────────── output: one flushed frame per call ───────────── */

static void frame(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vfprintf(stdout, fmt, ap);
    va_end(ap);
    fputc('\n', stdout);
    fflush(stdout);
}

/* ───────────── the session ───────────── */

typedef struct {
    pk_engine *engine;
    int vocab;
    int cap;            /* KV capacity in positions */
    int pos;            /* valid positions in the KV cache */
    int32_t *ids;       /* the current turn's ids (grown on demand) */
    long ids_cap;
    field_reader rd;
} session;

/* what a handler tells the command loop */
typedef enum { NEXT_COMMAND, END_OK, END_FAIL } outcome;

static outcome engine_failure(const char *what) {
    frame("ERROR ENGINE 1 %s: %s", what, pk_last_error());
    return END_FAIL;
}

/* The TURN header: the six fields after the command word. */
typedef struct {
    long max_new, keep, top_k, n_ids;
    float temp, top_p;
} turn_header;

static int read_turn_header(field_reader *r, turn_header *h) {
    return field_long(r, &h->max_new) && field_long(r, &h->keep) && field_float(r, &h->temp) &&
           field_float(r, &h->top_p) && field_long(r, &h->top_k) && field_long(r, &h->n_ids);
}

/* Whether the turn's counts fit the session (nothing changes otherwise). */
static int turn_fits(const session *s, const turn_header *h) {
    const long room = (long)s->cap - h->keep;   /* positions left after the kept prefix */
    return h->max_new >= 0 && h->keep >= 0 && h->keep <= s->pos && h->n_ids >= 1 && h->n_ids <= room &&
           h->n_ids <= s->cap;
}

/* Reads n ids into s->ids; returns the number outside the vocabulary, or -1
 * if the input ended first (or memory ran out). */
static long read_ids(session *s, long n) {
    if (n > s->ids_cap) {
        int32_t *grown = (int32_t *)realloc(s->ids, (size_t)n * sizeof(int32_t));
        if (!grown) return -1;
        s->ids = grown;
        s->ids_cap = n;
    }
    long outside = 0;
    for (long i = 0; i < n; ++i) {
        long v;
        if (!field_long(&s->rd, &v)) return -1;
        outside += v < 0 || v >= s->vocab;
        s->ids[i] = (int32_t)v;
    }
    return outside;
}

/* Skips n ids of a refused turn; 0 if the input ended first. */
static int skip_ids(session *s, long n) {
    for (long i = 0; i < n; ++i) {
        long v;
        if (!field_long(&s->rd, &v)) return 0;
    }
    return 1;
}

/* Why a turn that has `produced` tokens out stops before the next emission
 * (NULL: it goes on). The token budget is checked before the cache room. */
static const char *budget_stop(const session *s, long produced, long max_new) {
    if (produced >= max_new) return "MAX_TOKENS";
    if (s->pos >= s->cap) return "CONTEXT_FULL";
    return NULL;
}

/* Why an emitted (and already fed) token ends the turn (NULL: it does not). */
static const char *stop_token(int32_t tok) {
    switch (tok) {
    case STOP_RETURN: return "RETURN";
    case STOP_CALL: return "CALL";
    default: return NULL;
    }
}

/* Emits tokens from `tok` on: each is announced, then fed at the next
 * position; the prediction of the last fed token is the next candidate. */
static outcome generate(session *s, int32_t tok, long max_new) {
    long produced = 0;
    const char *why;
    while ((why = budget_stop(s, produced, max_new)) == NULL) {
        frame("TOKEN %d", tok);
        ++produced;
        int32_t predicted = 0;
        if (pk_forward_token(s->engine, tok, s->pos, &predicted, NULL) != PK_OK) return engine_failure("forward");
        ++s->pos;
        if ((why = stop_token(tok)) != NULL) break;
        tok = predicted >= 0 && predicted < s->vocab ? predicted : 0;
    }
    frame("DONE %s %ld %d", why, produced, s->pos);
    return NEXT_COMMAND;
}

static outcome cmd_turn(session *s) {
    turn_header h;
    if (!read_turn_header(&s->rd, &h)) {
        frame("ERROR BAD_HEADER 1 unreadable TURN header");
        return END_FAIL;
    }
    /* the turn's sampling holds from here on, refused or not (the engine
     * clamps it as picchio.c:2737-2743 does) */
    const int top_k = h.top_k > INT_MAX ? INT_MAX : h.top_k < INT_MIN ? INT_MIN : (int)h.top_k;
    if (pk_set_turn_sampling(s->engine, h.temp, h.top_p, top_k) != PK_OK) return engine_failure("sampling");
    if (!turn_fits(s, &h)) {
        frame("ERROR BAD_RANGE 0 keep/n_ids out of bounds (pos=%d cap=%d)", s->pos, s->cap);
        return skip_ids(s, h.n_ids) ? NEXT_COMMAND : END_FAIL;
    }
    const long outside = read_ids(s, h.n_ids);
    if (outside < 0) return END_FAIL;
    if (outside > 0) {
        frame("ERROR BAD_TOKEN 0 ID out of vocabulary");
        return NEXT_COMMAND;
    }
    /* the prompt overwrites the cache from `keep` on */
    int32_t first = 0;
    if (pk_prefill_tokens(s->engine, s->ids, (int)h.n_ids, (int)h.keep, &first) != PK_OK)
        return engine_failure("prefill");
    s->pos = (int)(h.keep + h.n_ids);
    return generate(s, first, h.max_new);
}

static outcome cmd_reset(session *s) {
    /* positions are rewritten from 0; the penalty history empties */
    s->pos = 0;
    if (pk_reset_history(s->engine) != PK_OK) return engine_failure("reset");
    frame("DONE RESET 0 0");
    return NEXT_COMMAND;
}

static outcome cmd_shutdown(session *s) {
    (void)s;
    return END_OK;
}

static const struct {
    const char *word;
    outcome (*run)(session *);
} COMMANDS[] = {
    {"TURN", cmd_turn},
    {"RESET", cmd_reset},
    {"SHUTDOWN", cmd_shutdown},
};

/* Runs commands until SHUTDOWN, the end of the input or a fatal error;
 * returns the exit status. */
static int serve(session *s) {
    frame("READY %d %d %d %d", s->cap, s->vocab, STOP_RETURN, STOP_CALL);
    while (next_field(&s->rd)) {
        outcome (*run)(session *) = NULL;
        for (size_t i = 0; i < sizeof COMMANDS / sizeof COMMANDS[0]; ++i)
            if (strcmp(s->rd.field, COMMANDS[i].word) == 0) run = COMMANDS[i].run;
        if (!run) {
            frame("ERROR BAD_COMMAND 1 unknown command");
            return 1;
        }
        const outcome o = run(s);
        if (o != NEXT_COMMAND) return o == END_OK ? 0 : 1;
    }
    return 0;
}

/* ───────────── start-up ───────────── */

static float env_float(const char *name, float fallback) {
    const char *v = getenv(name);
    return v ? (float)atof(v) : fallback;
}

static int env_int(const char *name, int fallback) {
    const char *v = getenv(name);
    return v ? atoi(v) : fallback;
}

static int fail_startup(pk_engine *e) {
    fprintf(stderr, "error: %s\n", pk_last_error());
    if (e) pk_engine_destroy(e);
    return 1;
}

int main(int argc, char **argv) {
    const char *model = getenv("MODEL");
    if (!model && argc > 1) model = argv[1];
    if (!model || env_int("SERVICE", 0) == 0) {
        fprintf(stderr, "usage: SERVICE=1 MODEL=/path/to/checkpoint %s  (or SERVICE=1 %s /path)\n", argv[0],
                argv[0]);
        return 1;
    }

    pk_cfg cfg;
    if (pk_cfg_from_container(model, 0, &cfg) != PK_OK) return fail_startup(NULL);
    int cap = env_int("CTX", 512);
    if (cap > cfg.ctx_len) cap = cfg.ctx_len;
    if (cap < 1) {
        fprintf(stderr, "error: KV capacity %d\n", cap);
        return 1;
    }
    cfg.ctx_len = cap;

    pk_engine *e = NULL;
    if (pk_engine_create(&cfg, env_int("PK_DEVICE", 0), &e) != PK_OK) return fail_startup(NULL);
    const clock_t t0 = clock();
    if (pk_load_container(e, model, env_int("IO_THREADS", 8)) != PK_OK) return fail_startup(e);
    fprintf(stderr, "loaded %s: %d layers, %d experts, vocab %d, %.2f GB resident (%.1f s cpu)\n", model,
            cfg.n_layers, cfg.n_experts, cfg.vocab, (double)pk_engine_device_bytes(e) / 1e9,
            (double)(clock() - t0) / CLOCKS_PER_SEC);

    const char *seed = getenv("SEED");
    const uint64_t rng_seed = seed ? (uint64_t)atoll(seed) : (uint64_t)time(NULL);
    if (pk_set_sampling(e, env_float("TEMPERATURE", 1.0f), env_float("TOPP", 0.95f), env_int("TOPK", 50),
                        env_float("REP", 1.1f), rng_seed) != PK_OK)
        return fail_startup(e);
    fprintf(stderr, "service: persistent session, KV capacity %d positions\n", cap);

    session s = {0};
    s.engine = e;
    s.vocab = cfg.vocab;
    s.cap = cap;
    s.rd.in = stdin;
    const int status = serve(&s);
    free(s.ids);
    pk_engine_destroy(e);
    return status;
}
