/*
 * g3k.h - the thin C-ABI between the C11 host library (host/g3attn.c) and the
 * HIP kernels (the .hip files in csrc).  Plain pointers, sizes and a hipStream_t passed
 * as void*; every launcher returns a hipError_t value (0 = launched).
 *
 * Device data layouts (all fp32 unless noted):
 *   KV cache, per layer: head-major [n_kv_heads][rows][head_dim]; row r of
 *     head h at base + h*head_stride + r*row_stride (row_stride = head_dim).
 *     rows = max_context (global layer) or sliding_window (local ring).
 *   RoPE table: [max_context][head_dim/2][cos, sin], the reference's layout
 *     (gemma3_kernels.c:455-468), uploaded from the host.
 *   q/k/v of one token: [heads][head_dim] as produced by the reference's GEMVs.
 */
#ifndef G3K_H
#define G3K_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define G3K_HEAD_DIM 256
#define G3K_MAX_SPLITS 256

typedef struct {
    /* query side */
    const float *q;        /* [H_q][D]: pre-norm (fused decode) or final (gqa) */
    const float *k_new;    /* [H_kv][D] pre-norm key of the new token (fused decode) */
    const float *v_new;    /* [H_kv][D] value of the new token (fused decode) */
    const uint16_t *q_norm;/* bf16 [D] or NULL: no QK-norm (fused decode) */
    const uint16_t *k_norm;
    const float *rope_row; /* table row of pos: [D/2][2] (fused decode) */
    float eps;
    /* cache */
    float *kc, *vc;
    long long row_stride, head_stride; /* in floats */
    int n_stream;          /* attention indices streamed from the cache */
    int skip;              /* cache row excluded from the stream (rows >= skip shift by one) */
    int new_slot;          /* cache row receiving the new k/v (fused decode) */
    const float *mask;     /* additive mask per attention index or NULL (gqa) */
    float qscale;          /* softmax scale * log2(e) */
    int rows_per_split;    /* multiple of 64 */
    int n_splits;          /* <= G3K_MAX_SPLITS */
    int n_kv_heads;
    int group;             /* query heads per kv head: 1, 2 or 4 */
    /* outputs */
    float *out;            /* [H_q][D] */
    float *ws_acc;         /* [H_kv][G3K_MAX_SPLITS][group][D] split partials */
    float *ws_ml;          /* [H_kv][G3K_MAX_SPLITS][group][2] (max, sum) */
} g3k_decode_args;

/* QK-norm + RoPE of q (and of the new k), cache write of the new k/v and
 * split-K attention over the cache; with n_splits > 1 a second launch
 * combines the split partials. */
int g3k_decode(const g3k_decode_args *a, int fused, void *stream);

/* Workgroups of the decode kernel that can be resident at once on the
 * current device (occupancy x compute units); 0 if unknown. */
int g3k_decode_capacity(int group, int fused);

/* Batched QK-norm + RoPE + cache write for n tokens (positions start_pos..).
 *   Q [n][H_q][D] (may be NULL) -> q_out head-major [H_q][n][D];
 *   K, V [n][H_kv][D] -> k_dst/v_dst rows: slot = ring ? (pos % ring) : (pos - dst_pos0),
 *   with head stride dst_head_stride floats. */
typedef struct {
    const float *Q, *K, *V;
    const uint16_t *q_norm, *k_norm;
    const float *rope;     /* full table [max_context][D/2][2] */
    float eps;
    int n, start_pos, n_heads, n_kv_heads;
    float *q_out;
    float *k_dst, *v_dst;
    long long dst_head_stride;
    int ring;              /* >0: slot = pos % ring; 0: slot = pos - dst_pos0 */
    int dst_pos0;
} g3k_rope_write_args;

int g3k_rope_write(const g3k_rope_write_args *a, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* G3K_H */
