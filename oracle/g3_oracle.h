/*
 * g3_oracle.h - CPU restatement of the gemma3.c attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product library (libg3attn.so) never links or calls it.
 *
 * Every function restates one piece of robitec97/gemma3.c (paths relative to
 * the reference tree) in plain C11, written fresh, same operation order:
 *
 *   g3o_bf16_to_f32 / g3o_f32_to_bf16_trunc  gemma3_kernels.h:268-283
 *   g3o_rmsnorm_bf16                         gemma3_kernels.c:289-304
 *   g3o_rope_precompute                      gemma3_kernels.c:455-468
 *   g3o_rope_apply                           gemma3_kernels.c:470-484
 *   g3o_softmax                              gemma3_kernels.c:396-415
 *   g3o_causal_mask                          gemma3_kernels.c:613-622
 *   g3o_gqa                                  gemma3_kernels.c:527-597 (non-BLAS)
 *   g3o_cache_kv                             gemma3_transformer.c:236-251
 *   g3o_layer_decode                         gemma3_transformer.c:294-352
 *   g3o_prefill                              gemma3_transformer.c:641-692
 *   g3o_prefill_mt / g3o_prefill_rows        the same loop, tokens in parallel
 *   g3o_is_global_layer / g3o_layer_theta    gemma3.h:347-360
 *   g3o_matvec_bf16                          gemma3_kernels.c:146-238 (AVX2 order)
 *   g3o_gelu_tanh                            gemma3_kernels.c:348-357
 *   g3o_forward_seq, g3o_forward_cached      gemma3_transformer.c:396-512 (+ layer_mlp :362-391)
 *
 * How each function is pinned (tests/test_oracle_*.py):
 *   - against golden vectors written by the real reference sources compiled
 *     in place (oracle/_ref, tests/golden/), and
 *   - against closed forms / invariants / an fp64 brute force.
 *
 * Cache layout is the reference's: [slot][n_kv_heads][head_dim] fp32, with
 * slot = pos on global layers and pos % sliding_window on local layers.
 */
#ifndef G3_ORACLE_H
#define G3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Subset of gemma3_config (gemma3.h:82-95) that the attention path reads. */
typedef struct {
    int num_layers;
    int num_heads;
    int num_kv_heads;
    int head_dim;
    int max_context;
    int sliding_window;
    float rmsnorm_eps;
    float rope_theta_local;
    float rope_theta_global;
} g3o_config;

void g3o_default_config(g3o_config *cfg);

int g3o_is_global_layer(int layer);
float g3o_layer_theta(const g3o_config *cfg, int layer);

float g3o_bf16_to_f32(uint16_t b);
uint16_t g3o_f32_to_bf16_trunc(float f);
/* Round-to-nearest-even; used only by the input generator (not in the reference). */
uint16_t g3o_f32_to_bf16_rne(float f);

void g3o_rmsnorm_bf16(float *y, const float *x, const uint16_t *w, int n, float eps);
void g3o_rope_precompute(float *freqs, int max_pos, int head_dim, float theta);
void g3o_rope_apply(float *x, const float *freqs, int head_dim, int pos);
void g3o_softmax(float *x, int n);
void g3o_causal_mask(float *mask, int seq_len, int query_pos);

/* gemma3_gqa restated.  k/v: [seq][n_kv_heads][head_dim]; rows[i] (optional)
 * names the cache row read at attention index i (NULL: row i).  The
 * reference reads rows 0..seq_len-1; `rows` lets the multi-threaded prefill
 * replay exactly the reference's ring order from a position-indexed array. */
void g3o_gqa(float *out, const float *q, const float *k, const float *v,
             int n_heads, int n_kv_heads, int seq_len, int head_dim,
             float scale, const float *mask, float *scores);
void g3o_gqa_rows(float *out, const float *q, const float *k, const float *v,
                  const int *rows, int n_heads, int n_kv_heads, int seq_len,
                  int head_dim, float scale, const float *mask, float *scores);

/* gemma3_matvec_bf16: y [M] = A [M][K] (bf16 row-major) . x [K], fp32.  The
 * sum follows the reference's AVX2 build (the path its `make fast` flags
 * select): per row, two 8-lane fused multiply-add accumulators over blocks of
 * 16 elements, one over a remaining block of 8, lane sums combined as
 * (acc0 + acc1) -> halves -> pairs -> one, then a scalar tail. */
void g3o_matvec_bf16(float *y, const uint16_t *A, const float *x, int M, int K);

/* gemma3_gelu_tanh_inplace: x = 0.5 x (1 + tanhf(sqrt(2/pi) (x + 0.044715 x^3))). */
void g3o_gelu_tanh(float *x, int n);

/* Shape of a whole model for g3o_forward_seq (gemma3_config fields). */
typedef struct {
    int vocab_size, hidden_size, intermediate_size, num_layers;
    int num_heads, num_kv_heads, head_dim, max_context, sliding_window;
    float rmsnorm_eps, rope_theta_local, rope_theta_global;
} g3o_model;

/* gemma3_transformer_forward for tokens[0..n-1] at positions 0..n-1 from an
 * empty cache: per step the embedding row * sqrt(hidden), then per layer the
 * input RMSNorm, the Q/K/V GEMVs, the attention section (g3o_layer_decode),
 * the o_proj GEMV, post-attention RMSNorm + residual, pre-feedforward RMSNorm
 * (or a copy when absent), gate / up GEMVs, gelu(gate) * up, the down GEMV,
 * post-feedforward RMSNorm + residual; then the final RMSNorm and the
 * tied-embedding logits.  layer_w: num_layers x 13 tensors in the
 * gemma3_weights_t field order (post-attention, pre- and post-feedforward
 * norms may be NULL).  logits [n][vocab]; hidden_last [hidden]. */
/* The same forward for tokens[0..n-1] at positions pos0..pos0+n-1 on
 * caller-owned caches kc / vc [num_layers] (reference layout [rows][kv
 * heads x head_dim], rows = max_context for global layers, sliding_window
 * for local ones; updated as cache_kv does), so a step can start from any
 * cache state.  Logits are computed for the last n_logits tokens only
 * (logits [n_logits][vocab]); hidden_last may be NULL.  The GEMVs split
 * their rows over `threads` threads (same bits for any count). */
int g3o_forward_cached(float *logits, int n_logits, float *hidden_last, const int *tokens, int n, int pos0,
                       const uint16_t *embed, const uint16_t *const *layer_w, const uint16_t *norm,
                       const g3o_model *m, float *const *kc, float *const *vc, int threads);
int g3o_forward_seq(float *logits, float *hidden_last, const int *tokens, int n,
                    const uint16_t *embed, const uint16_t *const *layer_w, const uint16_t *norm,
                    const g3o_model *m);

/* cache_kv: copies k, v (kv_size floats each) into slot pos or pos % window. */
void g3o_cache_kv(float *k_cache, float *v_cache, const float *k, const float *v,
                  int kv_size, int is_global, int window, int pos);

/* Attention section of layer_attention for one token.
 *   q [H_q*d], k [H_kv*d]: pre-norm; normed + RoPE'd in place (as the reference does).
 *   v [H_kv*d]; q_norm/k_norm: bf16 [d] (NULL/NULL skips the norm, as the reference).
 *   k_cache/v_cache: this layer's cache (global: max_context rows; local: window rows).
 *   rope: table for this layer's theta.  attn_out [H_q*d].
 *   work: >= max(max_context, window) floats (mask) + same again (scores).
 * Returns 0, or -8 (GEMMA3_ERR_CONTEXT_OVERFLOW) when pos >= max_context. */
int g3o_layer_decode(float *attn_out, float *q, float *k, const float *v,
                     const uint16_t *q_norm, const uint16_t *k_norm,
                     float *k_cache, float *v_cache, const float *rope,
                     const g3o_config *cfg, int layer, int pos, float *work);

/* Prefill attention loop (gemma3_transformer.c:641-692) for n tokens starting
 * at start_pos: per token, in order, QK-norm -> RoPE -> cache_kv -> GQA.
 *   Q [n][H_q*d], K [n][H_kv*d] are normed/RoPE'd in place; V [n][H_kv*d];
 *   attn_out [n][H_q*d]. */
int g3o_prefill(float *attn_out, float *Q, float *K, const float *V,
                const uint16_t *q_norm, const uint16_t *k_norm,
                float *k_cache, float *v_cache, const float *rope,
                const g3o_config *cfg, int layer, int start_pos, int n, float *work);

/* Same results as g3o_prefill, bit for bit, computed with `threads` workers:
 * the cache writes are replayed first and every token then reads its keys in
 * the exact ring/slot order the sequential loop would have seen.  On return
 * k_cache/v_cache hold the same final state as after g3o_prefill. */
int g3o_prefill_mt(float *attn_out, float *Q, float *K, const float *V,
                   const uint16_t *q_norm, const uint16_t *k_norm,
                   float *k_cache, float *v_cache, const float *rope,
                   const g3o_config *cfg, int layer, int start_pos, int n, int threads);

/* g3o_prefill_mt restricted to the tokens sel[0..n_sel-1] (indices into the
 * batch): attn_out [n_sel][H_q*d] row j is token sel[j].  Q/K are normed +
 * RoPE'd in place and the cache ends in the same state as after g3o_prefill. */
int g3o_prefill_rows(float *attn_out, float *Q, float *K, const float *V,
                     const uint16_t *q_norm, const uint16_t *k_norm,
                     float *k_cache, float *v_cache, const float *rope,
                     const g3o_config *cfg, int layer, int start_pos, int n,
                     const int *sel, int n_sel, int threads);

/* QK-norm + RoPE of n tokens x n_heads vectors in place (X [n][n_heads][d]),
 * token i at position start_pos + i: the same per-vector calls as
 * g3o_layer_decode makes (gemma3_transformer.c:295-312), over `threads`
 * workers.  w == NULL skips the norm.  Used to build long caches. */
void g3o_norm_rope_batch(float *X, int n, int n_heads, int head_dim, const uint16_t *w,
                         const float *rope, int start_pos, float eps, int threads);

/* Seeded input generator: counter-indexed splitmix64, Box-Muller (cos branch)
 * in double, rounded to fp32 then to bf16 (RNE).  Element i of a tensor uses
 * counters 2i and 2i+1 of stream `seed`.  Output floats are bf16-exact.
 * Threads: 0 = auto. */
void g3o_gen_normal_bf16(float *out, size_t n, uint64_t seed, size_t first, int threads);
uint64_t g3o_splitmix64(uint64_t seed, uint64_t counter);

/* FNV-1a 64 over raw bytes: input hashes recorded in the golden fixtures. */
uint64_t g3o_fnv1a64(const void *data, size_t nbytes);

#ifdef __cplusplus
}
#endif
#endif /* G3_ORACLE_H */
