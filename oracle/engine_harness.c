/*
 * engine_harness.c - the reference engine with its GPU backend hook switched
 * on, driving libg3attn through libg3backend.so.  TEST INFRASTRUCTURE: built
 * into oracle/_ref/ by oracle/Makefile only where /root/reference exists.
 *
 * gemma3_transformer.c is compiled in place with -DUSE_MPS, so its own
 * backend declarations (gemma3_transformer.c:17-31) and calls (create
 * :889-905, destroy :912-914, forward_token :931-935, prefill_tokens
 * :954-958, reset :974-978) are what run; libg3backend.so defines the eight
 * functions they name.  Nothing of the engine is restated here: eng_run only
 * builds the harness model (ref_harness.c) and calls the engine's public API.
 * When the backend is unavailable (no GPU, or a G3ATTN_FAULT site) the engine
 * falls back to its CPU path by its own logic, which is what the fallback
 * tests check.
 */
#include "ref_harness.c"

#include <stddef.h>

#include "g3attn.h"

/* g3attn_upload_weights reads the engine's gemma3_weights_t as a
 * g3attn_weights: the two must have one layout. */
_Static_assert(sizeof(gemma3_weights_t) == sizeof(g3attn_weights), "weights size");
_Static_assert(offsetof(gemma3_weights_t, norm) == offsetof(g3attn_weights, norm), "norm");
_Static_assert(offsetof(gemma3_weights_t, layers[1].input_layernorm) ==
                   offsetof(g3attn_weights, layers[1].input_layernorm), "layer stride");
_Static_assert(offsetof(gemma3_weights_t, layers[0].q_norm) == offsetof(g3attn_weights, layers[0].q_norm),
               "q_norm");
_Static_assert(offsetof(gemma3_weights_t, layers[0].post_feedforward_layernorm) ==
                   offsetof(g3attn_weights, layers[0].post_feedforward_layernorm), "last tensor");
_Static_assert(sizeof(gemma3_config) == sizeof(g3attn_config), "config size");

/* gemma3_transformer_create on the harness model, then `passes` runs of the
 * token sequence with gemma3_transformer_reset between runs.  Each run
 * prefills tokens[0..n_prefill) with gemma3_transformer_prefill_tokens (its
 * logits are the last prefilled token's) and decodes the rest one by one with
 * gemma3_transformer_forward_token.  Run p writes token i's logits at
 * logits + (p * n + i) * vocab (rows the engine does not return are left as
 * they are).  *on_gpu is 1 when the engine kept its backend context after
 * create.  Returns 0, the first nonzero engine return code, or -4 when create
 * fails. */
int eng_run(float *logits, int *on_gpu, const int *tokens, int n, int n_prefill, int passes,
            const uint16_t *embed, const uint16_t *const *layer_w, const uint16_t *norm, int vocab,
            int hidden, int inter, int num_layers, int hq, int hkv, int max_context, int window) {
    if (num_layers < 1 || num_layers > GEMMA3_NUM_LAYERS || n < 1 || n_prefill < 0 || n_prefill > n ||
        n > max_context || passes < 1)
        return -1;
    gemma3_config cfg;
    gemma3_weights_t w;
    harness_model(&cfg, &w, embed, layer_w, norm, vocab, hidden, inter, num_layers, hq, hkv, max_context,
                  window);
    gemma3_transformer *t = gemma3_transformer_create(&w, &cfg, max_context);
    if (!t) return -4;
    *on_gpu = t->metal_ctx != NULL;
    int rc = 0;
    for (int p = 0; p < passes && !rc; p++) {
        float *lg = logits + (size_t)p * n * vocab;
        if (p > 0) gemma3_transformer_reset(t);
        if (n_prefill > 0)
            rc = gemma3_transformer_prefill_tokens(t, tokens, n_prefill, 0, lg + (size_t)(n_prefill - 1) * vocab);
        for (int i = n_prefill; i < n && !rc; i++)
            rc = gemma3_transformer_forward_token(t, tokens[i], i, lg + (size_t)i * vocab);
    }
    gemma3_transformer_destroy(t);
    return rc;
}
