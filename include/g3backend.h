/*
 * g3backend.h - the reference engine's GPU backend hook, served by libg3attn.
 *
 * gemma3.c's transformer calls an optional GPU backend through eight C
 * functions, declared in gemma3_transformer.c:17-31 (and gemma3_metal.h)
 * under USE_MPS and called at gemma3_transformer.c:889-905 (create),
 * 912-914 (destroy), 931-935 (forward_token), 954-958 (prefill_tokens) and
 * 974-978 (reset).  libg3backend.so defines those functions on top of
 * libg3attn.so, so the engine's existing backend hook runs on an MI355X with
 * no source change: build gemma3_transformer.c with -DUSE_MPS and link
 * libg3backend.so in place of gemma3_metal.o.  Every call keeps the Metal
 * backend's contract: init returns NULL when no GPU is usable (the engine then
 * stays on the CPU), uploads and forwards return 0 or a negative gemma3_error.
 *
 * The prototypes use g3attn_config where the reference writes gemma3_config;
 * the two have one layout (tests/test_abi.py checks every field offset), and
 * C symbols carry no types, so the engine's own declarations link to these.
 */
#ifndef G3BACKEND_H
#define G3BACKEND_H

#include "g3attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The engine's opaque backend context (gemma3_transformer.c:19). */
typedef struct gemma3_metal_context gemma3_metal_context;

/* gemma3_metal_available (gemma3_metal.h:22): 1 if a HIP device is visible. */
int gemma3_metal_available(void);

/* gemma3_metal_init (gemma3_transformer.c:20, called at :890): a g3attn
 * context for cfg with its device KV cache; the RoPE tables follow through
 * gemma3_metal_upload_rope.  NULL when no device is usable or an allocation
 * fails (message in g3attn_last_error). */
gemma3_metal_context *gemma3_metal_init(const g3attn_config *cfg, int max_context);

/* gemma3_metal_free (:21, called at :897 and :913). */
void gemma3_metal_free(gemma3_metal_context *ctx);

/* gemma3_metal_upload_weights (:22, called at :892): weights is the engine's
 * gemma3_weights_t (gemma3_transformer.c:55-73); see g3attn_upload_weights.
 * 0, or -1 / -4 (the engine then frees the context and uses the CPU). */
int gemma3_metal_upload_weights(gemma3_metal_context *ctx, const void *weights);

/* gemma3_metal_upload_rope (:23-25, called at :893-895); see g3attn_upload_rope. */
int gemma3_metal_upload_rope(gemma3_metal_context *ctx, const float *rope_local, const float *rope_global,
                             int max_context, int head_dim);

/* gemma3_metal_forward_token (:26-27, called at :933): one token through the
 * model at pos; logits [vocab_size] on the host when compute_logits. */
int gemma3_metal_forward_token(gemma3_metal_context *ctx, int token_id, int pos, float *logits,
                               int compute_logits);

/* gemma3_metal_prefill (:28-29, called at :956): num_tokens tokens at
 * start_pos.., logits of the last one (may be NULL). */
int gemma3_metal_prefill(gemma3_metal_context *ctx, const int *tokens, int num_tokens, int start_pos,
                         float *logits);

/* gemma3_metal_reset_cache (:30, called at :976). */
void gemma3_metal_reset_cache(gemma3_metal_context *ctx);

#ifdef __cplusplus
}
#endif

#endif /* G3BACKEND_H */
