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
#define G3K_SPLIT_GRAIN 32   /* decode split granularity (rows): one workgroup step at group <= 2 */

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
    int rows_per_split;    /* multiple of G3K_SPLIT_GRAIN */
    int n_splits;          /* <= G3K_MAX_SPLITS */
    int n_kv_heads;
    int group;             /* query heads per kv head: 1, 2 or 4 */
    /* outputs */
    float *out;            /* [H_q][D] */
    float *ws_acc;         /* [H_kv][G3K_MAX_SPLITS][group][D] split partials */
    float *ws_ml;          /* [H_kv][G3K_MAX_SPLITS][group][2] (max, sum) */
    int nt_loads;          /* fused decode: K/V rows through non-temporal buffer loads */
    void *ev0, *ev1;       /* hipEvent_t: begin / end of decode_kernel's dispatch, or NULL */
    /* One-launch form (xm_heads > 0): workgroups of xm_heads query heads,
     * the splits of each (KV head, query-head run) on one XCD, merged there
     * by the last to arrive (G3K_XM_* below); 0: decode + combine launches. */
    int xm_heads;
    unsigned *xm_count;    /* G3K_XM_COUNTERS(H_q) zeroed arrival counters */
} g3k_decode_args;

/* One-launch decode: at most this many splits, and the arrival counters,
 * one per (KV head, query-head run) and G3K_XM_COUNTER_STRIDE apart (their
 * own 256-byte line each), in a zeroed buffer that every launch leaves zero. */
#ifndef G3K_XM_MAX_SPLITS
#define G3K_XM_MAX_SPLITS 32
#endif
#define G3K_XM_COUNTER_STRIDE 64
#define G3K_XM_COUNTERS(n_heads) ((size_t)(n_heads) * G3K_XM_COUNTER_STRIDE)

/* Writes the XCD (hardware register XCC_ID) each workgroup of an n-workgroup
 * launch ran on to xcc[n].  The one-launch decode needs workgroups whose ids
 * agree mod 8 to run on one XCD.  Returns a hipError_t. */
int g3k_xcd_probe(unsigned *xcc, int n, void *stream);

/* QK-norm + RoPE of q (and of the new k), cache write of the new k/v and
 * split-K attention over the cache; with n_splits > 1 a second launch
 * combines the split partials. */
int g3k_decode(const g3k_decode_args *a, int fused, void *stream);

/* Workgroups of the decode kernel that can be resident at once on the
 * current device (occupancy x compute units); 0 if unknown. */
int g3k_decode_capacity(int group, int fused);

/* The current device's fixed split-partial scratch of the allocation-free
 * gqa entry point (a static device array; its address is looked up once per
 * device).  acc holds G3K_NOALLOC_MAX_HEADS * G3K_MAX_SPLITS * head_dim
 * floats in the ws_acc layout of g3k_decode_args, ml the matching (max, sum)
 * pairs.  Allocates nothing. */
#define G3K_NOALLOC_MAX_HEADS 16
int g3k_noalloc_scratch(float **acc, float **ml);

/* gemma3_gqa of any shape the reference computes (gemma3_kernels.c:527-597):
 * q [n_heads][head_dim] final, k / v rows [seq_len][n_kv_heads][head_dim],
 * optional additive mask [seq_len], out [n_heads][head_dim]; query head h
 * reads KV head h / (n_heads / n_kv_heads).  head_dim 1..G3K_GQA_MAX_DIM,
 * any group.  Split-K over n_splits runs of rows_per_split keys; with more
 * than one split the partials go to ws_acc [n_heads][n_splits][head_dim] and
 * ws_ml [n_heads][n_splits][2] and a second launch merges them. */
#define G3K_GQA_MAX_DIM 512
typedef struct {
    const float *q, *k, *v, *mask;
    float *out, *ws_acc, *ws_ml;
    int n_heads, n_kv_heads, seq_len, head_dim;
    int n_splits, rows_per_split;
    float qscale;          /* softmax scale * log2(e) */
} g3k_gqa_args;
int g3k_gqa_generic(const g3k_gqa_args *a, void *stream);

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
    int kv_skip;           /* tokens i < kv_skip are not written to k_dst / v_dst */
    /* optional prefill staging of the rotated keys (bit patterns),
     * kq [n_kv_heads][ldk][2][D], token i at row row0 + i: fp16 hi | lo rows,
     * or, with kscale != NULL, fp16 hi | fp8 cross rows and the row's scale
     * byte in kscale [n_kv_heads][ldk] (see G3K_KROW_X8) */
    uint16_t *kq;
    uint8_t *kscale;
    long long ldk;
    int row0;
} g3k_rope_write_args;

/* Key row formats of the prefill staging (1 KiB per key and KV head).
 * Exact policy: fp16 hi (dim d at bytes 2d) | fp16 lo = fp16(k - hi) (512 +
 * 2d).  Fp8 cross policy (G3K_KROW_X8): fp16 hi as above | 512 bytes of OCP
 * e4m3 in the lane order of the 16x16x128 fp8 MFMA: part p (0: hi / 2^E,
 * 1: lo * 2^11 / 2^E, lo = k - hi in fp32) of dim d = 32 t + 8 g + u at byte
 * 512 + 256 p + 64 (t >> 1) + 16 g + 8 (t & 1) + u, where E = floor(log2
 * max |k|) - 7 over the row (0 for a zero row) keeps every value within
 * +-256; the row's scale byte is the E8M0 code 127 + E. */
#define G3K_KROW_X8 1

int g3k_rope_write(const g3k_rope_write_args *a, void *stream);

/* Cache rows from the reference layout: rows [n][n_kv_heads][D] (device) ->
 * dst + h*head_stride + (slot + i)*D for head h, row i, in one launch for
 * every head (instead of a strided copy per head).  to_rows != 0 runs the
 * other way (cache -> rows). */
int g3k_kv_scatter(float *dst_k, float *dst_v, float *rows_k, float *rows_v, int n, int n_kv_heads,
                   long long head_stride, int slot, int to_rows, void *stream);

/* Prefill staging of key rows kk0..kk0+cnt-1 (key index kk = position -
 * kstart): K (already normed + rotated, fp32) -> key rows of
 * kq [H_kv][ldk][2][D] in the format kscale selects (exact fp16 hi | lo, or
 * fp16 hi | fp8 cross with a scale byte per row, G3K_KROW_X8); V (fp32) ->
 * bf16 hi and lo columns of vt / vt_lo
 * [H_kv][D][ldk] (v = hi + lo to 16 bits).  If any staged V has a nonzero lo
 * part, *v_lo_flag is set to epoch.
 * Source row of key kk (position pos = kstart + kk) for head h:
 *   src + h*head_stride + r*row_stride, r = ring ? pos % ring : pos - row_pos0.
 * k_src == NULL stages V only.  Key indices in [nk, kk0+cnt) are written as
 * zeros (K rows and V columns) without reading the source. */
typedef struct {
    const float *k_src, *v_src;
    long long head_stride, row_stride;
    int ring, row_pos0, kstart;
    int kk0, cnt, nk, n_kv_heads;
    uint16_t *kq, *vt, *vt_lo;
    uint8_t *kscale;       /* NULL: exact key rows; else fp8 cross rows + scale bytes */
    long long ldk;
    int *v_lo_flag;
    int epoch;
} g3k_stage_args;

int g3k_stage(const g3k_stage_args *a, void *stream);

/* g3k_rope_write (without queries: ra->Q == NULL) and g3k_stage of the same
 * batch's values (sa: V only, from ra->V, key indices from the batch's first
 * token on) in one launch; the staging blocks also write the batch's V rows
 * to the cache, so V is read once. */
int g3k_rope_write_stage(const g3k_rope_write_args *ra, const g3k_stage_args *sa, void *stream);

/* Causal / sliding-window prefill attention on MFMA (one launch).
 *   q:  raw (pre-norm) queries [n][n_heads][D] fp32, the reference's Q_all
 *       layout; the kernel applies QK-norm (q_norm, NULL = none) and RoPE
 *       (table row start_pos + i) to token i, whose key index is hist + i.
 *   kq: staged keys [H_kv][ldk][2][D] in the row format kscale selects
 *       (exact or fp8 cross, G3K_KROW_X8); vt / vt_lo: bf16
 *       hi / lo values [H_kv][D][ldk], nk valid key indices, zero padded to
 *       ldk (a multiple of 64).  vt_lo is read only when *v_lo_flag == epoch
 *       (some staged V is not exactly bf16).
 *   Query i attends key indices kk with hist+i-window < kk <= hist+i.
 *   out: [n][H_q][D] fp32 (the reference's attn_out layout). */
typedef struct {
    const float *q;
    const uint16_t *q_norm;
    const float *rope;        /* full table [max_context][D/2][2] */
    float eps;
    int start_pos;
    const uint16_t *kq, *vt, *vt_lo;
    const uint8_t *kscale;    /* NULL: exact key rows; else fp8 cross rows + scale bytes */
    const int *v_lo_flag;
    int epoch;
    float *out;
    long long ldk;
    int n, hist, nk, window;  /* window: INT_MAX / 2 for global layers */
    int n_kv_heads, group;
    float qscale;             /* softmax scale * log2(e) */
    int queries_per_wave;     /* 16 (8 waves, 2 per SIMD) or 32 (4 waves, 1 per SIMD) */
    int schedule;             /* 16 queries per wave: 0 = all waves in phase, 1 = SIMD pairs in opposite phase */
    void *ev0, *ev1;          /* hipEvent_t: begin / end of prefill_kernel's dispatch, or NULL */
    /* Key splits (1, 2 or 4).  With S > 1 every (query block, KV head) runs as
     * S workgroups over consecutive parts of its key tiles; each writes its
     * unnormalised O and (max, sum) per query row to part_o [S][n][H_q][D]
     * and part_ml [S][n][H_q][2], then counts itself in arrive[qb * H_kv +
     * kvh] (an atomic increment that wraps to 0 after S arrivals, so the
     * counters start every call at zero).  The last of the S workgroups to
     * arrive merges the S parts into out, in split order (deterministic).
     * arrive holds G3K_PREFILL_ARRIVE(max_n, H_kv) zeroed counters. */
    int ksplit;
    float *part_o, *part_ml;
    unsigned *arrive;
} g3k_prefill_args;

/* arrival counters a prefill of up to n tokens can index: query blocks of at
 * least 32 positions, one counter per (query block, KV head) */
#define G3K_PREFILL_ARRIVE(n, n_kv) ((((n) + 31) / 32) * (n_kv))

int g3k_prefill(const g3k_prefill_args *a, void *stream);

/* bf16-weight GEMV, y[m] = A[m] . x for up to G3K_MATVEC_MAX matrices that
 * share x (one launch): A[m] [M[m]][K] bf16 row-major, x [K], y[m] [M[m]]
 * fp32. */
#define G3K_MATVEC_MAX 3
typedef struct {
    const float *x;
    int K;
    int n_mat;
    const uint16_t *A[G3K_MATVEC_MAX];
    float *y[G3K_MATVEC_MAX];
    int M[G3K_MATVEC_MAX];
    /* 0: y[m] = A[m] . x.  G3K_MV_GEGLU: n_mat = 2, M[0] == M[1],
     * y[0] = gelu_tanh(A[0] . x) * (A[1] . x)  (gemma3_transformer.c:380-386) */
    int mode;
    /* Residual prologue, taken when pre_t is set (K <= G3K_MATVEC_PRE_MAX).
     * x is then not read: every workgroup forms it in LDS from the step that
     * sits between two GEMVs of the token forward (gemma3_transformer.c:
     * 463-477, 490-496, 444-446):
     *   s = pre_r + rmsnorm(pre_t, pre_w_post)    (pre_r + pre_t without pre_w_post)
     *   x = rmsnorm(s, pre_w_next)                (s without pre_w_next)
     * with rmsnorm as gemma3_rmsnorm_bf16 (gemma3_kernels.c:289-304) at
     * pre_eps, and workgroup 0 stores s to pre_r_out.  pre_r_out must not
     * overlap pre_r: the other workgroups read pre_r while it is written.
     * K % 4 == 0; pre_t, pre_r and pre_r_out 16-byte aligned, the gain rows
     * 8-byte aligned. */
    const float *pre_t, *pre_r;
    const uint16_t *pre_w_post, *pre_w_next;
    float *pre_r_out;
    float pre_eps;
} g3k_matvec_args;
#define G3K_MV_GEGLU 1
#define G3K_MATVEC_PRE_MAX 4096

int g3k_matvec(const g3k_matvec_args *a, void *stream);

/* One-workgroup steps of a token's forward pass on a hidden vector of n
 * floats (n <= G3K_LAYER_MAX_HIDDEN):
 *   G3K_OP_EMBED:    x = bf16(embed[token][.]) * sqrt(n)
 *   G3K_OP_NORM:     y = rmsnorm(x, w_next)
 *   G3K_OP_RESIDUAL: t = rmsnorm(t, w_post) if w_post; x += t;
 *                    then, if y: y = rmsnorm(x, w_next), or a copy of x if
 *                    w_next is NULL
 * rmsnorm(v, w) = v / sqrt(mean(v^2) + eps) * (1 + bf16(w)). */
#define G3K_LAYER_MAX_HIDDEN 8192
enum { G3K_OP_EMBED = 0, G3K_OP_NORM = 1, G3K_OP_RESIDUAL = 2 };
typedef struct {
    int op, n, token;
    float eps;
    const uint16_t *embed, *w_post, *w_next;
    float *x, *t, *y;
} g3k_layer_args;

int g3k_layer_step(const g3k_layer_args *a, void *stream);

/* The same steps over `rows` tokens at once, one workgroup per token row, for
 * the batched prefill.  The normed output goes to two bf16 planes, y = y_hi +
 * y_lo (y_hi = bf16(y), y_lo = bf16(y - y_hi)), the GEMM operand format:
 *   G3K_ROWS_EMBED:    x[r] = bf16(embed[tokens[r]][.]) * sqrt(n);
 *                      y[r] = rmsnorm(x[r], w_next)
 *   G3K_ROWS_RESIDUAL: t' = rmsnorm(t[r], w_post) if w_post, else t[r];
 *                      x[r] += t'; then, if y_hi: y[r] = rmsnorm(x[r], w_next),
 *                      or x[r] itself if w_next is NULL
 *   G3K_ROWS_SPLIT:    y[r] = t[r] (any n; the other ops take n <= G3K_LAYER_MAX_HIDDEN)
 * x is [rows][n] fp32, t [rows][ldt] fp32 (RESIDUAL: the sum of nsplit >= 1
 * partial products at t + s * split_stride), y_hi / y_lo [rows][ldy] bf16;
 * tokens is a device array. */
enum { G3K_ROWS_EMBED = 0, G3K_ROWS_RESIDUAL = 1, G3K_ROWS_SPLIT = 2 };
typedef struct {
    int op, rows, n;
    float eps;
    const int *tokens;
    const uint16_t *embed, *w_post, *w_next;
    float *x;
    const float *t;
    int ldt, nsplit;
    long long split_stride;
    uint16_t *y_hi, *y_lo;
    int ldy;
} g3k_rows_args;

int g3k_rows(const g3k_rows_args *a, void *stream);

/* Batched projection on MFMA: C[n][m] = sum_k X[n][k] W[m][k] for N tokens,
 * X given as bf16 planes x_hi + x_lo [N][ldx], W bf16 [M][K] (K % (32 ksplit)
 * == 0, M % 4 == 0).  mode 0: n_mat (1..3) matrices sharing X, each written
 * to C[j] [N][ldc[j]] fp32; with ksplit S > 1, split s covers k in
 * [s K / S, (s + 1) K / S) and writes its partial product to C[j] +
 * s * split_stride (floats), for the consumer to add.  mode G3K_MV_GEGLU
 * (ksplit 1): W[0] = gate, W[1] = up (same M); gelu_tanh(gate) * up is
 * written as bf16 planes h_hi + h_lo [N][ldh]. */
typedef struct {
    const uint16_t *x_hi, *x_lo;
    int N, K, ldx, n_mat, mode, ksplit;
    long long split_stride;
    const uint16_t *W[G3K_MATVEC_MAX];
    int M[G3K_MATVEC_MAX];
    float *C[G3K_MATVEC_MAX];
    int ldc[G3K_MATVEC_MAX];
    uint16_t *h_hi, *h_lo;
    int ldh;
} g3k_gemm_args;

int g3k_gemm(const g3k_gemm_args *a, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* G3K_H */
