/*
 * g3backend.c - the engine's GPU backend hook (gemma3_transformer.c:17-31)
 * defined over libg3attn.  Each function forwards to the g3attn entry point
 * that replaces it; the context is the g3attn context itself.
 */
#include "g3backend.h"

#include <hip/hip_runtime_api.h>
#include <stdlib.h>

struct gemma3_metal_context {
    g3attn_ctx *attn;
};

static g3attn_ctx *attn_of(gemma3_metal_context *ctx) { return ctx ? ctx->attn : NULL; }

int gemma3_metal_available(void) {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess && n > 0;
}

gemma3_metal_context *gemma3_metal_init(const g3attn_config *cfg, int max_context) {
    g3attn_ctx *attn = g3attn_create(cfg, max_context, NULL, NULL);
    if (!attn) return NULL;
    gemma3_metal_context *ctx = (gemma3_metal_context *)calloc(1, sizeof *ctx);
    if (!ctx) {
        g3attn_destroy(attn);
        return NULL;
    }
    ctx->attn = attn;
    return ctx;
}

void gemma3_metal_free(gemma3_metal_context *ctx) {
    if (!ctx) return;
    g3attn_destroy(ctx->attn);
    free(ctx);
}

int gemma3_metal_upload_weights(gemma3_metal_context *ctx, const void *weights) {
    return g3attn_upload_weights(attn_of(ctx), weights);
}

int gemma3_metal_upload_rope(gemma3_metal_context *ctx, const float *rope_local, const float *rope_global,
                             int max_context, int head_dim) {
    return g3attn_upload_rope(attn_of(ctx), rope_local, rope_global, max_context, head_dim);
}

int gemma3_metal_forward_token(gemma3_metal_context *ctx, int token_id, int pos, float *logits,
                               int compute_logits) {
    return g3attn_forward_token(attn_of(ctx), token_id, pos, logits, compute_logits);
}

int gemma3_metal_prefill(gemma3_metal_context *ctx, const int *tokens, int num_tokens, int start_pos,
                         float *logits) {
    return g3attn_prefill_tokens(attn_of(ctx), tokens, num_tokens, start_pos, logits);
}

void gemma3_metal_reset_cache(gemma3_metal_context *ctx) { g3attn_reset(attn_of(ctx)); }
