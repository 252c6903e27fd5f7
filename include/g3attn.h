/*
 * g3attn.h - MI355X (gfx950) attention path for gemma3.c, as a C-ABI library
 * (libg3attn.so).  Plain C types only; every pointer is a caller-owned buffer.
 *
 * The library owns a GPU-resident fp32 KV cache per layer and runs the
 * attention block that follows the Q/K/V projections: per-head QK-RMSNorm,
 * RoPE from the caller's precomputed table, the KV-cache write and GQA
 * attention (decode: one token; prefill: a causal / sliding-window batch).
 * The surrounding engine (loader, tokenizer, sampler) is untouched; a
 * transformer built with -DUSE_HIP calls these entry points where the
 * reference runs its CPU attention, and optionally the projection, forward
 * and batched-prefill entry points below for the rest of a token's layers.
 *
 * Conventions kept from the reference:
 *   - 0 on success, a negative gemma3_error code on failure (gemma3.h:57-67):
 *     -1 invalid argument or GPU runtime error, -4 device allocation failed,
 *     -8 position >= max_context.  The message is thread-local
 *     (g3attn_last_error), as gemma3.c:30-41 keeps it.
 *   - create returns NULL on failure so the caller keeps its CPU path
 *     (gemma3_transformer.c:889-905 does this for Metal).
 *   - Not re-entrant per context: one host thread drives a context, as the
 *     reference drives its transformer (gemma3_transformer.c:38-49).
 *
 * Entry points ending in _device take device pointers, enqueue on the
 * context's stream and return without waiting; all others take host
 * pointers and return when the result is in the caller's buffer.
 */
#ifndef G3ATTN_H
#define G3ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Field-for-field the layout of gemma3_config (gemma3.h:82-95), so a caller
 * may pass (const g3attn_config *)&its_gemma3_config.  The attention path
 * reads num_layers, num_heads, num_kv_heads, head_dim, sliding_window,
 * rmsnorm_eps; supported: head_dim 256, num_heads / num_kv_heads in {1, 2, 4}. */
typedef struct {
    int vocab_size;
    int hidden_size;
    int intermediate_size;
    int num_layers;
    int num_heads;
    int num_kv_heads;
    int head_dim;
    int max_context;
    int sliding_window;
    float rmsnorm_eps;
    float rope_theta_local;
    float rope_theta_global;
} g3attn_config;

typedef struct g3attn_ctx g3attn_ctx;

/* Gemma 3 4B defaults (gemma3.h:36-51; gemma3.c:94-109). */
void g3attn_default_config(g3attn_config *cfg);

/* 1 if layer `layer` uses global attention: (layer + 1) % 6 == 0
 * (gemma3_is_global_layer, gemma3.h:347-350). */
int g3attn_is_global_layer(int layer);

/* RoPE table [max_pos][head_dim/2][cos, sin] with the reference expression
 * (gemma3_rope_precompute, gemma3_kernels.c:455-468), computed on the host in
 * fp32 with libm so the GPU sees bit-identical angles. */
void g3attn_rope_precompute(float *freqs, int max_pos, int head_dim, float theta);

/* Allocates the device KV cache for every layer (gemma3_kv_cache_alloc,
 * gemma3_transformer.c:180-214: max_context rows on global layers, a
 * sliding_window ring on local ones) and uploads both RoPE tables
 * ([max_context][head_dim/2][2], from gemma3_transformer.c:870-883; the Metal
 * backend uploads them the same way, gemma3_metal.m:603-614).  Replaces
 * gemma3_metal_init + gemma3_metal_upload_rope (gemma3_metal.h:26, 37-39).
 * Both tables may be NULL, as gemma3_metal_init takes none: they are then
 * uploaded with g3attn_upload_rope, and the attention calls return -1 until
 * they are.  Returns NULL on failure (message in g3attn_last_error).
 *
 * Failure injection, for testing a caller's fallback: the environment
 * variable G3ATTN_FAULT, a comma-separated list read at each call, makes the
 * listed sites fail before any GPU work: "create" (g3attn_create returns
 * NULL), "upload" (g3attn_upload_weights returns -4, as a failed device
 * allocation does) and "forward" (g3attn_forward_token[_device] and
 * g3attn_prefill_tokens return -1, as a GPU runtime error does). */
g3attn_ctx *g3attn_create(const g3attn_config *cfg, int max_context,
                          const float *rope_local, const float *rope_global);

/* gemma3_metal_upload_rope (gemma3_metal.h:37-39, called at
 * gemma3_transformer.c:893-895): copies the engine's local and global RoPE
 * tables [max_context][head_dim/2][2] to the device, replacing the context's.
 * max_context must equal the context's and head_dim must be 256, else -1. */
int g3attn_upload_rope(g3attn_ctx *ctx, const float *rope_local, const float *rope_global,
                       int max_context, int head_dim);

/* gemma3_kv_cache_free (gemma3_transformer.c:216-223) + gemma3_metal_free. */
void g3attn_destroy(g3attn_ctx *ctx);

/* gemma3_kv_cache_reset (gemma3_transformer.c:225-233): positions only.
 * The cache holds no position state (the caller passes pos), so this waits
 * for queued work and leaves the rows as they are, like the reference. */
void g3attn_reset(g3attn_ctx *ctx);

/* One decode step of one layer: the attention section of layer_attention
 * (gemma3_transformer.c:294-352).  q [num_heads*256], k, v [num_kv_heads*256]
 * are the raw projections (pre-norm); q_norm / k_norm are the layer's bf16
 * QK-norm weights [256] (both NULL: no norm, as :295).  Normalises + RoPEs q
 * and k at pos, writes k, v to slot pos (global) or pos % sliding_window
 * (local), attends over pos+1 (global) or min(pos+1, window) (local) cached
 * rows, and writes attn_out [num_heads*256].  Blocking. */
int g3attn_decode(g3attn_ctx *ctx, int layer, int pos,
                  const float *q, const float *k, const float *v,
                  const uint16_t *q_norm, const uint16_t *k_norm, float *attn_out);

/* Prefill of n tokens at positions start_pos..start_pos+n-1 of one layer: the
 * per-token attention loop of gemma3_transformer_prefill_batched
 * (gemma3_transformer.c:641-692), batched.  Q [n][num_heads*256],
 * K, V [n][num_kv_heads*256] (pre-norm), attn_out [n][num_heads*256].
 * Token i sees exactly the keys the sequential loop gives it: positions
 * [0, pos] (global) or [pos-window+1, pos] (local), including keys cached by
 * earlier calls when start_pos > 0.  Blocking.
 * Scores use fp16 q_hi k_hi plus the cross terms q_lo k_hi + q_hi k_lo as
 * scaled fp8 products (per-key and per-query power-of-two scales, so any
 * input range fp16 holds keeps its precision): about 4e-4 x output RMS
 * against the reference at the configs, against the path's 2e-3 bar.  The
 * environment variable G3ATTN_PREFILL_QK=exact, read at g3attn_create,
 * selects three fp16 passes instead (about 1e-4).  The whole-model batched
 * prefill (g3attn_prefill_forward_device, g3attn_prefill_tokens) always
 * uses the exact scores: its logits are held to 1e-4 x RMS. */
int g3attn_prefill(g3attn_ctx *ctx, int layer, int start_pos, int n,
                   const float *Q, const float *K, const float *V,
                   const uint16_t *q_norm, const uint16_t *k_norm, float *attn_out);

/* Device-pointer forms of decode / prefill (same arguments, device memory),
 * enqueued on the context stream.  For callers whose projections already
 * live on the GPU, and for timing with inputs resident in HBM. */
int g3attn_decode_device(g3attn_ctx *ctx, int layer, int pos,
                         const float *q, const float *k, const float *v,
                         const uint16_t *q_norm, const uint16_t *k_norm, float *attn_out);
int g3attn_prefill_device(g3attn_ctx *ctx, int layer, int start_pos, int n,
                          const float *Q, const float *K, const float *V,
                          const uint16_t *q_norm, const uint16_t *k_norm, float *attn_out);

/* K-norm + RoPE + cache_kv for n tokens without attention: the key/value half
 * of the prefill loop (gemma3_transformer.c:650-671).  K, V [n][num_kv_heads*256]
 * pre-norm (host / device pointers respectively). */
int g3attn_kv_append(g3attn_ctx *ctx, int layer, int start_pos, int n,
                     const float *K, const float *V, const uint16_t *k_norm);
int g3attn_kv_append_device(g3attn_ctx *ctx, int layer, int start_pos, int n,
                            const float *K, const float *V, const uint16_t *k_norm);

/* Raw access to cache rows (layer_kv_cache.k / .v, gemma3_transformer.c:77-81):
 * rows slot..slot+n-1 in the reference layout [n][num_kv_heads][256], already
 * normalised and rotated.  Host pointers; blocking. */
int g3attn_kv_write(g3attn_ctx *ctx, int layer, int slot, int n,
                    const float *k_rows, const float *v_rows);
int g3attn_kv_read(g3attn_ctx *ctx, int layer, int slot, int n,
                   float *k_rows, float *v_rows);

/* Same signature and semantics as gemma3_gqa (gemma3_kernels.h:188-191,
 * gemma3_kernels.c:527-597): q [n_heads][head_dim] (final), k_cache / v_cache
 * [seq_len][n_kv_heads][head_dim], optional additive mask [seq_len]; query
 * head h reads KV head h / (n_heads / n_kv_heads).  Any shape the reference
 * computes in bounds: n_kv_heads dividing n_heads (any group), head_dim 1 to
 * 512.  head_dim 256 with groups 1, 2, 4 (the model's shapes) runs the
 * split-K decode kernels; every other shape a general split-K kernel.
 * scores_buf is accepted and unused.  Host pointers, runs on the default
 * device through a process-wide context; for unit parity and for drop-in use
 * where no cache-owning context exists (an engine compiled with
 * -Dgemma3_gqa=g3attn_gqa runs its own attention loop on the GPU this way).
 * Failures leave output untouched and set g3attn_last_error (the reference
 * also returns silently). */
void g3attn_gqa(float *output, const float *q, const float *k_cache, const float *v_cache,
                int n_heads, int n_kv_heads, int seq_len, int head_dim,
                float scale, const float *mask, float *scores_buf);

/* Allocation-free variant of g3attn_gqa.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Every
 * pointer is a DEVICE buffer with g3attn_gqa's shapes (q [n_heads][head_dim],
 * K/V [seq_len][n_kv_heads][head_dim], mask [seq_len] or NULL, output
 * [n_heads][head_dim]); the launch goes on `stream` (a hipStream_t, NULL =
 * the null stream) and the call returns without waiting.  The split partials
 * live in a fixed static device scratch of 4.03 MiB per device, held until
 * the process ends, so n_heads <= G3ATTN_NOALLOC_MAX_HEADS (larger calls
 * return -1 with a message).  Calls that overlap on one GPU (other streams,
 * other threads) race on that scratch; serialise them.  Same splits and
 * kernels as g3attn_gqa (the general kernel's splits are capped to fit
 * the scratch): the results agree bit for bit.  The call enqueues
 * kernel launches only (no allocation, no memset), so it can be recorded into
 * a HIP graph once a first call on the device has run outside capture (that
 * call looks the scratch address up).  Returns 0 or -1. */
#define G3ATTN_NOALLOC_MAX_HEADS 16
int g3attn_gqa_noalloc(float *output, const float *q, const float *k_cache, const float *v_cache,
                       int n_heads, int n_kv_heads, int seq_len, int head_dim, float scale,
                       const float *mask, void *stream);

/* y [M] = A [M][K] . x [K] with A bf16 row-major and fp32 x, y: the same
 * signature and arithmetic as gemma3_matvec_bf16 (gemma3_kernels.h:217-218,
 * gemma3_kernels.c:188-238; fp32 accumulation, summation order differs).
 * scratch is accepted and unused.  Host pointers: A is copied to the device
 * on every call, so this form is for parity and drop-in use; weights that
 * stay on the device go through g3attn_matvec_bf16_device.  Runs on the
 * default device through a process-wide context; failures leave y untouched
 * and set g3attn_last_error (the reference returns void). */
void g3attn_matvec_bf16(float *y, const uint16_t *A, const float *x, int M, int K, float *scratch);

/* Device-pointer form of g3attn_matvec_bf16 on the context stream (replaces
 * matvec_bf16_dispatch, gemma3_transformer.c:38-49, for resident weights).
 * A and x 16-byte aligned with K % 8 == 0 take the vector path. */
int g3attn_matvec_bf16_device(g3attn_ctx *ctx, float *y, const uint16_t *A, const float *x, int M, int K);

/* The Q, K and V projections of layer_attention (gemma3_transformer.c:290-292)
 * in one launch: q [num_heads*head_dim] = wq . x, k / v [num_kv_heads*head_dim]
 * = wk / wv . x, x [hidden_size]; weights bf16 [rows][hidden_size].  Device
 * pointers, on the context stream; feeds g3attn_decode_device directly. */
int g3attn_qkv_proj_device(g3attn_ctx *ctx, const float *x, const uint16_t *wq, const uint16_t *wk,
                           const uint16_t *wv, float *q, float *k, float *v);

/* The whole of layer_attention (gemma3_transformer.c:258-356) for one token
 * at pos: x [hidden_size] -> Q/K/V projections -> QK-norm, RoPE, cache write,
 * GQA -> o_proj -> out [hidden_size].  Weights bf16 (wq [num_heads*head_dim]
 * [hidden], wk / wv [num_kv_heads*head_dim][hidden], wo [hidden]
 * [num_heads*head_dim]), q_norm / k_norm as in g3attn_decode.  Device
 * pointers, on the context stream (four launches, no host round trip). */
int g3attn_layer_attention_device(g3attn_ctx *ctx, int layer, int pos, const float *x,
                                  const uint16_t *wq, const uint16_t *wk, const uint16_t *wv,
                                  const uint16_t *wo, const uint16_t *q_norm, const uint16_t *k_norm,
                                  float *out);

/* Device copies of a model's bf16 tensors, field for field the layout of the
 * reference's gemma3_weights_t (gemma3_transformer.c:56-74; the safetensors
 * loader fills the host one, gemma3_safetensors.c:620-635): a caller that
 * uploaded every tensor can fill this struct with the device addresses in the
 * same places.  Entries of layers beyond cfg.num_layers are ignored. */
#define G3ATTN_MAX_LAYERS 34
typedef struct {
    const uint16_t *input_layernorm;
    const uint16_t *q_proj;
    const uint16_t *k_proj;
    const uint16_t *v_proj;
    const uint16_t *o_proj;
    const uint16_t *q_norm;
    const uint16_t *k_norm;
    const uint16_t *post_attention_layernorm;
    const uint16_t *gate_proj;
    const uint16_t *up_proj;
    const uint16_t *down_proj;
    const uint16_t *pre_feedforward_layernorm;
    const uint16_t *post_feedforward_layernorm;
} g3attn_layer_weights;

typedef struct {
    const uint16_t *embed_tokens;
    g3attn_layer_weights layers[G3ATTN_MAX_LAYERS];
    const uint16_t *norm;
} g3attn_weights;

/* One token through the whole model: gemma3_transformer_forward
 * (gemma3_transformer.c:396-512) on the GPU.  Embedding row * sqrt(hidden);
 * per layer the input RMSNorm, layer_attention (projections, QK-norm, RoPE,
 * cache write at pos, GQA, o_proj), post-attention RMSNorm + residual,
 * pre-feedforward RMSNorm, the GELU-gated MLP and the post-feedforward
 * RMSNorm + residual; then, if compute_logits, the final RMSNorm and the
 * tied-embedding logits [vocab_size].  Norm weights may be NULL where the
 * reference allows it (post-attention, pre- / post-feedforward).  hidden_out
 * (optional, [hidden_size]) receives the final hidden state before the final
 * norm.  weights is a host struct of device pointers; logits / hidden_out are
 * device buffers.  Enqueued on the context stream. */
int g3attn_forward_device(g3attn_ctx *ctx, const g3attn_weights *weights, int token_id, int pos,
                          float *logits, int compute_logits, float *hidden_out);

/* The model on the device, the GPU side of the reference's backend hook
 * (the USE_MPS precedent: gemma3_transformer.c:17-31, 889-905, 931-935,
 * 954-958, 974-978).
 *
 * g3attn_upload_weights replaces gemma3_metal_upload_weights
 * (gemma3_metal.m:560-601): weights points at the host gemma3_weights_t
 * (gemma3_transformer.c:55-73, the layout of g3attn_weights), typically the
 * safetensors mmap (gemma3_safetensors.c:651-712).  Every tensor is copied,
 * sized from the context's config, into one device allocation through pinned
 * staging buffers; NULL optional norms stay NULL.  A second call replaces the
 * model.  Returns 0, -1 (missing embed_tokens / norm, bad config) or -4. */
int g3attn_upload_weights(g3attn_ctx *ctx, const void *weights);

/* The device addresses of the uploaded model, NULL before an upload (for
 * g3attn_forward_device callers that keep their own activations). */
const g3attn_weights *g3attn_device_weights(g3attn_ctx *ctx);

/* gemma3_metal_forward_token (gemma3_metal.m:620-971), the body of
 * gemma3_transformer_forward_token's backend branch (gemma3_transformer.c:
 * 930-935): one token on the uploaded model; logits [vocab_size] is host
 * memory, written when compute_logits and logits are set.  Blocking. */
int g3attn_forward_token(g3attn_ctx *ctx, int token_id, int pos, float *logits, int compute_logits);

/* g3attn_forward_token with device logits ([vocab_size], may be NULL: no
 * logits), enqueued on the context stream without waiting, for engines that
 * sample on the device. */
int g3attn_forward_token_device(g3attn_ctx *ctx, int token_id, int pos, float *logits);

/* gemma3_metal_prefill (gemma3_metal.m:977-987), gemma3_transformer_
 * prefill_tokens' backend branch (:953-958): tokens[0..n-1] at positions
 * start_pos.. through the uploaded model; logits (host, may be NULL) receives
 * the last token's logits.  Tokens and positions are checked before anything
 * is enqueued.  Batches of G3ATTN_PREFILL_BATCH_MIN tokens or more take the
 * batched path (g3attn_prefill_forward_device, the USE_BLAS build's
 * gemma3_transformer_prefill_batched); shorter ones run the token forward
 * back to back.  Blocking. */
#define G3ATTN_PREFILL_BATCH_MIN 16
int g3attn_prefill_tokens(g3attn_ctx *ctx, const int *tokens, int num_tokens, int start_pos, float *logits);

/* The batched prefill's projection, C = X . W^T: the reference's
 * bf16_matrix_to_f32 + cblas_sgemm(RowMajor, NoTrans, Trans, N, M, K, 1, X, K,
 * W_f32, K, 0, C, M) pairs (gemma3_transformer.c:614-639, 694-699, 726-751).
 * X [N][K] fp32, W [M][K] bf16, C [N][M] fp32, device pointers; M a multiple
 * of 4, K of 32.  On MFMA: X is split into bf16 hi + lo planes (relative error
 * <= 2^-17) and both are multiplied by W with fp32 accumulation.  Enqueued on
 * the context stream. */
int g3attn_matmul_bf16_device(g3attn_ctx *ctx, float *C, const uint16_t *W, const float *X, int N, int M, int K);

/* gemma3_transformer_prefill_batched (gemma3_transformer.c:526-787) on the
 * GPU: all num_tokens tokens (host array) through each layer at once, in
 * chunks of up to 8192.  The reference's bf16 -> fp32 conversions and
 * cblas_sgemm calls (:614-639, 694-699, 726-751) become MFMA GEMMs (bf16
 * weights times the fp32 activations as bf16 hi + lo planes, fp32
 * accumulation); the per-token attention loop (:641-692) is g3attn_prefill's
 * kernel; the norms and residuals run per token row.  weights holds device
 * pointers; logits (device, [vocab_size], may be NULL) receives the last
 * token's logits.  Hidden and intermediate sizes must be multiples of 32.
 * Enqueued on the context stream. */
int g3attn_prefill_forward_device(g3attn_ctx *ctx, const g3attn_weights *weights, const int *tokens,
                                  int num_tokens, int start_pos, float *logits);

/* The context's HIP stream (hipStream_t), for callers that interleave their
 * own work; and a wait for everything queued on it. */
void *g3attn_stream(g3attn_ctx *ctx);
int g3attn_synchronize(g3attn_ctx *ctx);

/* Kernel timing for benchmarks (no counterpart in the reference, which has no
 * timers).  While enabled, every decode / prefill call times its main
 * attention kernel (kind 0: the split-K decode kernel, without the split
 * combine; kind 1: the prefill MFMA kernel, without the staging kernels)
 * with a pair of HIP events that the kernel's own dispatch records (begin
 * and end of execution) on the context stream.  g3attn_profile_read waits for the
 * stream and returns, for one kind, the launches bracketed since the last
 * read and their summed duration in milliseconds, then resets that kind. */
int g3attn_profile_enable(g3attn_ctx *ctx, int enable);
int g3attn_profile_read(g3attn_ctx *ctx, int kind, double *total_ms, int *count);

/* The work split the last call of one kind chose (no counterpart in the
 * reference): kind 0, the decode's key splits per KV head (1 = no combine);
 * kind 1, the prefill's key splits per query block (1, 2 or 4; above 1 the
 * last split to arrive merges the parts inside the kernel); kind 2, the
 * decode's query heads per workgroup when its splits were merged inside the
 * kernel by the last to arrive on each XCD, or 0 when a second launch
 * combined them (or there was one split).  0 before the first call of that
 * kind.  For tests and benchmarks that must know which code path a call
 * took. */
int g3attn_last_splits(g3attn_ctx *ctx, int kind, int *splits);

/* Thread-local message of the last failure on this thread ("" if none). */
const char *g3attn_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* G3ATTN_H */
