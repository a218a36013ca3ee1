// pk_decode.hip — GQA decode attention and the forward_token driver.
#include "pk_engine.h"

extern "C" int pk_gqa_attention(pk_engine *e, int layer, const float *x_dev, int pos,
                                float *out_dev) {
    (void)e; (void)layer; (void)x_dev; (void)pos; (void)out_dev;
    pk_set_error("gqa_attention: not built yet");
    return PK_ERR_UNSUPPORTED;
}

extern "C" int pk_forward_token(pk_engine *e, int tok, int pos, int32_t *next_host,
                                float *logits_dev) {
    (void)e; (void)tok; (void)pos; (void)next_host; (void)logits_dev;
    pk_set_error("forward_token: not built yet");
    return PK_ERR_UNSUPPORTED;
}

extern "C" int pk_prefill_tokens(pk_engine *e, const int32_t *ids, int n, int pos_base,
                                 int32_t *next_host) {
    (void)e; (void)ids; (void)n; (void)pos_base; (void)next_host;
    pk_set_error("prefill_tokens: not built yet");
    return PK_ERR_UNSUPPORTED;
}

extern "C" int pk_generate(pk_engine *e, const int32_t *prompt, int n_prompt, int n_steps,
                           int32_t *out) {
    (void)e; (void)prompt; (void)n_prompt; (void)n_steps; (void)out;
    pk_set_error("generate: not built yet");
    return PK_ERR_UNSUPPORTED;
}
