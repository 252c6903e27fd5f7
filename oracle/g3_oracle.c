/*
 * g3_oracle.c - CPU restatement of the gemma3.c attention path (checker only).
 *
 * TEST INFRASTRUCTURE.  Loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py; never by the product library.  Each function
 * cites the reference lines (robitec97/gemma3.c) whose operation order it
 * follows.  The pins for each function are listed in g3_oracle.h.
 */
#define _GNU_SOURCE
#include "g3_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* gemma3.h:36-51 constants; gemma3.c:94-109 fills gemma3_config from them. */
void g3o_default_config(g3o_config *cfg) {
    cfg->num_layers = 34;
    cfg->num_heads = 8;
    cfg->num_kv_heads = 4;
    cfg->head_dim = 256;
    cfg->max_context = 8192;
    cfg->sliding_window = 1024;
    cfg->rmsnorm_eps = 1e-6f;
    cfg->rope_theta_local = 10000.0f;
    cfg->rope_theta_global = 1000000.0f;
}

/* gemma3.h:347-350: every sixth layer (5, 11, 17, ...) is global. */
int g3o_is_global_layer(int layer) { return (layer + 1) % 6 == 0; }

/* gemma3.h:357-360 */
float g3o_layer_theta(const g3o_config *cfg, int layer) {
    return g3o_is_global_layer(layer) ? cfg->rope_theta_global : cfg->rope_theta_local;
}

/* gemma3_kernels.h:268-275: bf16 -> f32 is a 16-bit left shift. */
float g3o_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* gemma3_kernels.h:277-283: f32 -> bf16 truncates. */
uint16_t g3o_f32_to_bf16_trunc(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return (uint16_t)(u >> 16);
}

uint16_t g3o_f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* gemma3_kernels.c:289-304.  Sequential fp32 sum of squares, mean + eps,
 * 1/sqrtf, then x * r * (1 + w). */
void g3o_rmsnorm_bf16(float *y, const float *x, const uint16_t *w, int n, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    ss = ss / n + eps;
    const float r = 1.0f / sqrtf(ss);
    for (int i = 0; i < n; i++) y[i] = x[i] * r * (1.0f + g3o_bf16_to_f32(w[i]));
}

/* gemma3_kernels.c:455-468.  Table layout [pos][head_dim/2][cos, sin]. */
void g3o_rope_precompute(float *freqs, int max_pos, int head_dim, float theta) {
    const int half = head_dim / 2;
    for (int p = 0; p < max_pos; p++) {
        for (int i = 0; i < half; i++) {
            float inv = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
            float ang = (float)p * inv;
            freqs[((size_t)p * half + i) * 2] = cosf(ang);
            freqs[((size_t)p * half + i) * 2 + 1] = sinf(ang);
        }
    }
}

/* gemma3_kernels.c:470-484.  NeoX half-split rotation of (x_i, x_{i+half}). */
void g3o_rope_apply(float *x, const float *freqs, int head_dim, int pos) {
    const int half = head_dim / 2;
    const float *row = freqs + (size_t)pos * half * 2;
    for (int i = 0; i < half; i++) {
        const float c = row[2 * i], s = row[2 * i + 1];
        const float a = x[i], b = x[i + half];
        x[i] = a * c - b * s;
        x[i + half] = a * s + b * c;
    }
}

/* gemma3_kernels.c:146-186 (avx2_bf16_dot) as called by gemma3_matvec_bf16
 * (:188-238) in the reference's AVX2 build.  Lane j of accumulator 0 sums
 * elements 16 b + j, lane j of accumulator 1 elements 16 b + 8 + j (fused
 * multiply-add, one rounding each); a remaining block of 8 goes to
 * accumulator 0.  The horizontal sum adds acc1 into acc0 lane-wise, then lanes
 * l and l + 4, then l and l + 2, then lanes 0 and 1; the tail adds
 * bf16(a) * x one element at a time. */
static float matvec_row(const uint16_t *a, const float *x, int K) {
    float acc0[8] = {0}, acc1[8] = {0};
    int k = 0;
    for (; k + 15 < K; k += 16)
        for (int j = 0; j < 8; j++) {
            acc0[j] = fmaf(g3o_bf16_to_f32(a[k + j]), x[k + j], acc0[j]);
            acc1[j] = fmaf(g3o_bf16_to_f32(a[k + 8 + j]), x[k + 8 + j], acc1[j]);
        }
    for (; k + 7 < K; k += 8)
        for (int j = 0; j < 8; j++) acc0[j] = fmaf(g3o_bf16_to_f32(a[k + j]), x[k + j], acc0[j]);
    float s8[8], s4[4], s2[2];
    for (int j = 0; j < 8; j++) s8[j] = acc0[j] + acc1[j];
    for (int j = 0; j < 4; j++) s4[j] = s8[j] + s8[j + 4];
    for (int j = 0; j < 2; j++) s2[j] = s4[j] + s4[j + 2];
    float r = s2[0] + s2[1];
    for (; k < K; k++) r += g3o_bf16_to_f32(a[k]) * x[k];
    return r;
}

void g3o_matvec_bf16(float *y, const uint16_t *A, const float *x, int M, int K) {
    for (int i = 0; i < M; i++) y[i] = matvec_row(A + (size_t)i * K, x, K);
}

/* gemma3_kernels.c:348-357.  GELU, tanh approximation, in place. */
void g3o_gelu_tanh(float *x, int n) {
    const float c0 = 0.7978845608028654f, c1 = 0.044715f;   /* sqrt(2/pi); the cubic term */
    for (int i = 0; i < n; i++) {
        const float v = x[i];
        x[i] = 0.5f * v * (1.0f + tanhf(c0 * (v + c1 * (v * v * v))));
    }
}

/* gemma3_kernels.c:396-415.  Max, exp(x - max) with running sum, scale by 1/sum. */
void g3o_softmax(float *x, int n) {
    float m = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > m) m = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - m);
        sum += x[i];
    }
    const float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

/* gemma3_kernels.c:613-622 */
void g3o_causal_mask(float *mask, int seq_len, int query_pos) {
    for (int i = 0; i < seq_len; i++) mask[i] = (i <= query_pos) ? 0.0f : -INFINITY;
}

/* gemma3_kernels.c:527-597 (non-BLAS branch).  Per query head h (kv head
 * h / group): scores = (q . k_i) * scale + mask_i; softmax; out = sum_i p_i v_i.
 * Each KV row is streamed once per query head, as in the reference. */
void g3o_gqa_rows(float *out, const float *q, const float *k, const float *v,
                  const int *rows, int n_heads, int n_kv_heads, int seq_len,
                  int head_dim, float scale, const float *mask, float *scores) {
    const int group = n_heads / n_kv_heads;
    const size_t stride = (size_t)n_kv_heads * head_dim;
    int own = 0;
    if (!scores) {
        scores = (float *)malloc((size_t)seq_len * sizeof(float));
        own = 1;
        if (!scores) return;
    }
    for (int h = 0; h < n_heads; h++) {
        const int kvh = h / group;
        const float *qh = q + (size_t)h * head_dim;
        float *oh = out + (size_t)h * head_dim;
        for (int i = 0; i < seq_len; i++) {
            const size_t r = rows ? (size_t)rows[i] : (size_t)i;
            const float *kr = k + r * stride + (size_t)kvh * head_dim;
            float dot = 0.0f;
            for (int d = 0; d < head_dim; d++) dot += qh[d] * kr[d];
            scores[i] = dot * scale;
            if (mask) scores[i] += mask[i];
        }
        g3o_softmax(scores, seq_len);
        memset(oh, 0, (size_t)head_dim * sizeof(float));
        for (int i = 0; i < seq_len; i++) {
            const size_t r = rows ? (size_t)rows[i] : (size_t)i;
            const float *vr = v + r * stride + (size_t)kvh * head_dim;
            const float p = scores[i];
            for (int d = 0; d < head_dim; d++) oh[d] += p * vr[d];
        }
    }
    if (own) free(scores);
}

void g3o_gqa(float *out, const float *q, const float *k, const float *v,
             int n_heads, int n_kv_heads, int seq_len, int head_dim,
             float scale, const float *mask, float *scores) {
    g3o_gqa_rows(out, q, k, v, NULL, n_heads, n_kv_heads, seq_len, head_dim, scale, mask, scores);
}

/* gemma3_transformer.c:236-251: global layers append at slot pos, local
 * layers use a ring of `window` slots. */
void g3o_cache_kv(float *k_cache, float *v_cache, const float *k, const float *v,
                  int kv_size, int is_global, int window, int pos) {
    const size_t slot = is_global ? (size_t)pos : (size_t)(pos % window);
    memcpy(k_cache + slot * kv_size, k, (size_t)kv_size * sizeof(float));
    memcpy(v_cache + slot * kv_size, v, (size_t)kv_size * sizeof(float));
}

/* Attention range of gemma3_transformer.c:318-346: global reads slots
 * [0, pos], local reads min(pos + 1, window) ring slots; the mask is all
 * zeros in both cases. */
static int attn_seq_len(const g3o_config *cfg, int is_global, int pos) {
    if (is_global) return pos + 1;
    return pos < cfg->sliding_window ? pos + 1 : cfg->sliding_window;
}

static void norm_rope_token(float *q, float *k, const uint16_t *q_norm, const uint16_t *k_norm,
                            const float *rope, const g3o_config *cfg, int pos) {
    const int d = cfg->head_dim;
    if (q_norm && k_norm) { /* gemma3_transformer.c:295-304 */
        for (int h = 0; h < cfg->num_heads; h++)
            g3o_rmsnorm_bf16(q + (size_t)h * d, q + (size_t)h * d, q_norm, d, cfg->rmsnorm_eps);
        for (int h = 0; h < cfg->num_kv_heads; h++)
            g3o_rmsnorm_bf16(k + (size_t)h * d, k + (size_t)h * d, k_norm, d, cfg->rmsnorm_eps);
    }
    for (int h = 0; h < cfg->num_heads; h++) /* :307-312 */
        g3o_rope_apply(q + (size_t)h * d, rope, d, pos);
    for (int h = 0; h < cfg->num_kv_heads; h++)
        g3o_rope_apply(k + (size_t)h * d, rope, d, pos);
}

/* gemma3_transformer.c:294-352 (the attention section of layer_attention). */
int g3o_layer_decode(float *attn_out, float *q, float *k, const float *v,
                     const uint16_t *q_norm, const uint16_t *k_norm,
                     float *k_cache, float *v_cache, const float *rope,
                     const g3o_config *cfg, int layer, int pos, float *work) {
    if (pos < 0) return -1;
    if (pos >= cfg->max_context) return -8;
    const int kv_size = cfg->num_kv_heads * cfg->head_dim;
    const int is_global = g3o_is_global_layer(layer);
    const int cap = cfg->max_context > cfg->sliding_window ? cfg->max_context : cfg->sliding_window;
    float *mask = work, *scores = work + cap;

    norm_rope_token(q, k, q_norm, k_norm, rope, cfg, pos);
    g3o_cache_kv(k_cache, v_cache, k, v, kv_size, is_global, cfg->sliding_window, pos);
    const int seq_len = attn_seq_len(cfg, is_global, pos);
    if (is_global)
        g3o_causal_mask(mask, seq_len, pos);
    else
        for (int i = 0; i < seq_len; i++) mask[i] = 0.0f;
    const float scale = 1.0f / sqrtf((float)cfg->head_dim);
    g3o_gqa(attn_out, q, k_cache, v_cache, cfg->num_heads, cfg->num_kv_heads, seq_len,
            cfg->head_dim, scale, mask, scores);
    return 0;
}

/* gemma3_transformer.c:641-692: strictly sequential per token. */
int g3o_prefill(float *attn_out, float *Q, float *K, const float *V,
                const uint16_t *q_norm, const uint16_t *k_norm,
                float *k_cache, float *v_cache, const float *rope,
                const g3o_config *cfg, int layer, int start_pos, int n, float *work) {
    if (start_pos < 0 || n < 0) return -1;
    if (start_pos + n > cfg->max_context) return -8;
    const size_t qs = (size_t)cfg->num_heads * cfg->head_dim;
    const size_t ks = (size_t)cfg->num_kv_heads * cfg->head_dim;
    for (int i = 0; i < n; i++) {
        int rc = g3o_layer_decode(attn_out + i * qs, Q + i * qs, K + i * ks, V + i * ks, q_norm,
                                  k_norm, k_cache, v_cache, rope, cfg, layer, start_pos + i, work);
        if (rc) return rc;
    }
    return 0;
}

/* ---- multi-threaded prefill: same arithmetic, rows replayed in slot order ---- */

typedef struct {
    float *attn_out;
    const float *Q;
    const float *Kc, *Vc; /* [cache rows + n] combined: cache snapshot then batch rows */
    const g3o_config *cfg;
    int is_global, start_pos, n, cache_rows;
    const int *sel; /* tokens to compute (NULL: all n) */
    int n_out;      /* number of output rows */
    int next;       /* work counter (under lock) */
    pthread_mutex_t lock;
} mt_job;

static void *mt_worker(void *arg) {
    mt_job *J = (mt_job *)arg;
    const g3o_config *cfg = J->cfg;
    const int W = cfg->sliding_window;
    const int cap = (J->is_global ? J->start_pos + J->n : W) + 1;
    int *rows = (int *)malloc((size_t)cap * sizeof(int));
    float *mask = (float *)calloc((size_t)cap, sizeof(float));
    float *scores = (float *)malloc((size_t)cap * sizeof(float));
    const size_t qs = (size_t)cfg->num_heads * cfg->head_dim;
    const float scale = 1.0f / sqrtf((float)cfg->head_dim);
    if (!rows || !mask || !scores) goto done;
    for (;;) {
        pthread_mutex_lock(&J->lock);
        const int j = J->next < J->n_out ? J->next++ : -1;
        pthread_mutex_unlock(&J->lock);
        if (j < 0) break;
        const int i = J->sel ? J->sel[j] : j;
        const int pos = J->start_pos + i;
        const int seq_len = attn_seq_len(cfg, J->is_global, pos);
        for (int s = 0; s < seq_len; s++) {
            /* Position whose K/V sits in slot s after token i's cache write. */
            const int p = J->is_global ? s : pos - ((pos - s) % W);
            rows[s] = p >= J->start_pos ? J->cache_rows + (p - J->start_pos) : s;
        }
        g3o_gqa_rows(J->attn_out + (size_t)j * qs, J->Q + (size_t)i * qs, J->Kc, J->Vc, rows,
                     cfg->num_heads, cfg->num_kv_heads, seq_len, cfg->head_dim, scale, mask,
                     scores);
    }
done:
    free(rows);
    free(mask);
    free(scores);
    return NULL;
}

int g3o_prefill_mt(float *attn_out, float *Q, float *K, const float *V,
                   const uint16_t *q_norm, const uint16_t *k_norm,
                   float *k_cache, float *v_cache, const float *rope,
                   const g3o_config *cfg, int layer, int start_pos, int n, int threads) {
    return g3o_prefill_rows(attn_out, Q, K, V, q_norm, k_norm, k_cache, v_cache, rope, cfg, layer,
                            start_pos, n, NULL, n, threads);
}

int g3o_prefill_rows(float *attn_out, float *Q, float *K, const float *V,
                     const uint16_t *q_norm, const uint16_t *k_norm,
                     float *k_cache, float *v_cache, const float *rope,
                     const g3o_config *cfg, int layer, int start_pos, int n,
                     const int *sel, int n_sel, int threads) {
    if (start_pos < 0 || n < 0 || n_sel < 0) return -1;
    if (sel)
        for (int j = 0; j < n_sel; j++)
            if (sel[j] < 0 || sel[j] >= n) return -1;
    if (start_pos + n > cfg->max_context) return -8;
    if (n == 0) return 0;
    const int is_global = g3o_is_global_layer(layer);
    const size_t qs = (size_t)cfg->num_heads * cfg->head_dim;
    const size_t ks = (size_t)cfg->num_kv_heads * cfg->head_dim;
    for (int i = 0; i < n; i++)
        norm_rope_token(Q + i * qs, K + i * ks, q_norm, k_norm, rope, cfg, start_pos + i);

    /* Snapshot of the cache rows older tokens may read, followed by the batch. */
    const int cache_rows = is_global ? start_pos : cfg->sliding_window;
    const size_t total = (size_t)cache_rows + (size_t)n;
    float *Kc = (float *)malloc(total * ks * sizeof(float));
    float *Vc = (float *)malloc(total * ks * sizeof(float));
    if (!Kc || !Vc) {
        free(Kc);
        free(Vc);
        return -4;
    }
    memcpy(Kc, k_cache, (size_t)cache_rows * ks * sizeof(float));
    memcpy(Vc, v_cache, (size_t)cache_rows * ks * sizeof(float));
    memcpy(Kc + (size_t)cache_rows * ks, K, (size_t)n * ks * sizeof(float));
    memcpy(Vc + (size_t)cache_rows * ks, V, (size_t)n * ks * sizeof(float));

    mt_job J;
    J.attn_out = attn_out;
    J.Q = Q;
    J.Kc = Kc;
    J.Vc = Vc;
    J.cfg = cfg;
    J.is_global = is_global;
    J.start_pos = start_pos;
    J.n = n;
    J.cache_rows = cache_rows;
    J.sel = sel;
    J.n_out = sel ? n_sel : n;
    J.next = 0;
    pthread_mutex_init(&J.lock, NULL);
    if (threads <= 0) threads = (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    int started = 0;
    for (int t = 1; t < threads; t++)
        if (pthread_create(&tid[started], NULL, mt_worker, &J) == 0) started++;
    mt_worker(&J);
    for (int t = 0; t < started; t++) pthread_join(tid[t], NULL);
    pthread_mutex_destroy(&J.lock);
    free(Kc);
    free(Vc);

    /* Final cache state, as after the sequential loop's cache_kv calls. */
    for (int i = 0; i < n; i++)
        g3o_cache_kv(k_cache, v_cache, K + i * ks, V + i * ks, (int)ks, is_global,
                     cfg->sliding_window, start_pos + i);
    return 0;
}

/* ---- batch norm + rope ---- */

typedef struct {
    float *X;
    const uint16_t *w;
    const float *rope;
    int n_heads, head_dim, start_pos;
    float eps;
    int lo, hi;
} nr_job;

static void *nr_worker(void *arg) {
    nr_job *J = (nr_job *)arg;
    const size_t ts = (size_t)J->n_heads * J->head_dim;
    for (int i = J->lo; i < J->hi; i++)
        for (int h = 0; h < J->n_heads; h++) {
            float *x = J->X + (size_t)i * ts + (size_t)h * J->head_dim;
            if (J->w) g3o_rmsnorm_bf16(x, x, J->w, J->head_dim, J->eps);
            g3o_rope_apply(x, J->rope, J->head_dim, J->start_pos + i);
        }
    return NULL;
}

void g3o_norm_rope_batch(float *X, int n, int n_heads, int head_dim, const uint16_t *w,
                         const float *rope, int start_pos, float eps, int threads) {
    if (threads <= 0) threads = (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    if (n < 256) threads = 1;
    nr_job jobs[64];
    pthread_t tid[64];
    int started[64] = {0};
    const int chunk = (n + threads - 1) / threads;
    for (int t = 0; t < threads; t++) {
        nr_job j = {X, w, rope, n_heads, head_dim, start_pos, eps, t * chunk,
                    (t + 1) * chunk < n ? (t + 1) * chunk : n};
        if (j.lo > j.hi) j.lo = j.hi;
        jobs[t] = j;
        if (t > 0) started[t] = pthread_create(&tid[t], NULL, nr_worker, &jobs[t]) == 0;
        if (t > 0 && !started[t]) nr_worker(&jobs[t]);
    }
    nr_worker(&jobs[0]);
    for (int t = 1; t < threads; t++)
        if (started[t]) pthread_join(tid[t], NULL);
}

/* ---- generator ---- */

uint64_t g3o_splitmix64(uint64_t seed, uint64_t counter) {
    uint64_t z = seed + (counter + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static float gen_one(uint64_t seed, uint64_t idx) {
    const double u1 = (double)((g3o_splitmix64(seed, 2 * idx) >> 11) + 1) * 0x1.0p-53;
    const double u2 = (double)(g3o_splitmix64(seed, 2 * idx + 1) >> 11) * 0x1.0p-53;
    const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2);
    return g3o_bf16_to_f32(g3o_f32_to_bf16_rne((float)z));
}

typedef struct {
    float *out;
    size_t n, first;
    uint64_t seed;
} gen_job;

static void *gen_worker(void *arg) {
    gen_job *g = (gen_job *)arg;
    for (size_t i = 0; i < g->n; i++) g->out[i] = gen_one(g->seed, g->first + i);
    return NULL;
}

void g3o_gen_normal_bf16(float *out, size_t n, uint64_t seed, size_t first, int threads) {
    if (threads <= 0) threads = (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    if (n < ((size_t)1 << 16)) threads = 1;
    gen_job jobs[64];
    pthread_t tid[64];
    int started[64] = {0};
    const size_t chunk = (n + threads - 1) / threads;
    for (int t = 0; t < threads; t++) {
        const size_t lo = (size_t)t * chunk;
        const size_t hi = lo + chunk < n ? lo + chunk : n;
        jobs[t].out = out + lo;
        jobs[t].n = hi > lo ? hi - lo : 0;
        jobs[t].first = first + lo;
        jobs[t].seed = seed;
        if (t > 0) started[t] = pthread_create(&tid[t], NULL, gen_worker, &jobs[t]) == 0;
        if (t > 0 && !started[t]) gen_worker(&jobs[t]);
    }
    gen_worker(&jobs[0]);
    for (int t = 1; t < threads; t++)
        if (started[t]) pthread_join(tid[t], NULL);
}

uint64_t g3o_fnv1a64(const void *data, size_t nbytes) {
    const unsigned char *p = (const unsigned char *)data;
    uint64_t h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < nbytes; i++) {
        h ^= p[i];
        h *= 0x100000001b3ull;
    }
    return h;
}


/* ---------------------------------------------------------------- token forward */

/* The forward's GEMVs split by rows over a small pool of threads (each row's
 * summation order is g3o_matvec_bf16's, so the result is the same bits for
 * any thread count).  Each product is a new generation the workers wait for;
 * the caller takes part and waits until every worker has done its rows. */
typedef struct {
    pthread_mutex_t lock;
    pthread_cond_t start, done_cv;
    unsigned gen;
    int workers, done, quit;
    float *y;
    const uint16_t *A;
    const float *x;
    int M, K;
} mv_pool;

typedef struct {
    mv_pool *p;
    int idx;
} mv_arg;

static void mv_rows(mv_pool *p, int idx) {
    const int parts = p->workers + 1;
    const int lo = (int)((long long)p->M * idx / parts), hi = (int)((long long)p->M * (idx + 1) / parts);
    for (int i = lo; i < hi; i++) p->y[i] = matvec_row(p->A + (size_t)i * p->K, p->x, p->K);
}

static void *mv_worker(void *arg) {
    mv_arg *a = (mv_arg *)arg;
    mv_pool *p = a->p;
    unsigned seen = 0;
    for (;;) {
        pthread_mutex_lock(&p->lock);
        while (p->gen == seen && !p->quit) pthread_cond_wait(&p->start, &p->lock);
        if (p->quit) {
            pthread_mutex_unlock(&p->lock);
            return NULL;
        }
        seen = p->gen;
        pthread_mutex_unlock(&p->lock);
        mv_rows(p, a->idx);
        pthread_mutex_lock(&p->lock);
        if (++p->done == p->workers) pthread_cond_signal(&p->done_cv);
        pthread_mutex_unlock(&p->lock);
    }
}

static void pool_matvec(mv_pool *p, float *y, const uint16_t *A, const float *x, int M, int K) {
    if (!p || p->workers == 0) {
        g3o_matvec_bf16(y, A, x, M, K);
        return;
    }
    pthread_mutex_lock(&p->lock);
    p->y = y;
    p->A = A;
    p->x = x;
    p->M = M;
    p->K = K;
    p->done = 0;
    p->gen++;
    pthread_cond_broadcast(&p->start);
    pthread_mutex_unlock(&p->lock);
    mv_rows(p, 0);
    pthread_mutex_lock(&p->lock);
    while (p->done < p->workers) pthread_cond_wait(&p->done_cv, &p->lock);
    pthread_mutex_unlock(&p->lock);
}

/* gemma3_transformer.c:396-512 with layer_mlp (:362-391): tokens[0..n-1] at
 * positions pos0.. on caller-owned caches (kc / vc [layer], the reference
 * layout, updated as cache_kv does); logits for the last n_logits tokens. */
int g3o_forward_cached(float *logits, int n_logits, float *hidden_last, const int *tokens, int n, int pos0,
                       const uint16_t *embed, const uint16_t *const *layer_w, const uint16_t *norm,
                       const g3o_model *m, float *const *kc, float *const *vc, int threads) {
    const int H = m->hidden_size, I = m->intermediate_size, V = m->vocab_size, L = m->num_layers;
    const int d = m->head_dim, qs = m->num_heads * d, ks = m->num_kv_heads * d;
    if (n < 1 || n_logits < 0 || n_logits > n || pos0 < 0 || pos0 + n > m->max_context) return -1;
    g3o_config cfg;
    cfg.num_layers = L;
    cfg.num_heads = m->num_heads;
    cfg.num_kv_heads = m->num_kv_heads;
    cfg.head_dim = d;
    cfg.max_context = m->max_context;
    cfg.sliding_window = m->sliding_window;
    cfg.rmsnorm_eps = m->rmsnorm_eps;
    cfg.rope_theta_local = m->rope_theta_local;
    cfg.rope_theta_global = m->rope_theta_global;
    const int cap = m->max_context > m->sliding_window ? m->max_context : m->sliding_window;
    float *x = malloc((size_t)H * 4), *xn = malloc((size_t)H * 4), *proj = malloc((size_t)H * 4);
    float *mlp = malloc((size_t)H * 4), *q = malloc((size_t)qs * 4), *k = malloc((size_t)ks * 4);
    float *v = malloc((size_t)ks * 4), *attn = malloc((size_t)qs * 4);
    float *gate = malloc((size_t)I * 4), *up = malloc((size_t)I * 4);
    float *work = malloc((size_t)2 * cap * 4);
    float *rl = malloc((size_t)m->max_context * d * 4), *rg = malloc((size_t)m->max_context * d * 4);
    mv_pool pool;
    mv_arg args[64];
    pthread_t tid[64];
    int pool_on = 0;
    int rc = 0;
    if (!x || !xn || !proj || !mlp || !q || !k || !v || !attn || !gate || !up || !work || !rl || !rg) {
        rc = -4;
        goto done;
    }
    if (threads > 64) threads = 64;
    if (threads > 1) {
        /* as many workers as start (fewer threads change no result) */
        pthread_mutex_init(&pool.lock, NULL);
        pthread_cond_init(&pool.start, NULL);
        pthread_cond_init(&pool.done_cv, NULL);
        pool.gen = 0;
        pool.workers = 0;
        pool.done = 0;
        pool.quit = 0;
        pool_on = 1;
        for (int t = 1; t < threads; t++) {
            args[t].p = &pool;
            args[t].idx = t;
            if (pthread_create(&tid[t], NULL, mv_worker, &args[t]) != 0) break;
            pool.workers++;
        }
    }
    g3o_rope_precompute(rl, m->max_context, d, m->rope_theta_local);
    g3o_rope_precompute(rg, m->max_context, d, m->rope_theta_global);
    mv_pool *pp = pool_on ? &pool : NULL;
    const float escale = sqrtf((float)H);
    for (int i = 0; i < n && !rc; i++) {
        const int pos = pos0 + i;
        for (int j = 0; j < H; j++) x[j] = g3o_bf16_to_f32(embed[(size_t)tokens[i] * H + j]) * escale;
        for (int l = 0; l < L && !rc; l++) {
            const uint16_t *const *t = layer_w + (size_t)l * 13;
            g3o_rmsnorm_bf16(xn, x, t[0], H, m->rmsnorm_eps);
            pool_matvec(pp, q, t[1], xn, qs, H);
            pool_matvec(pp, k, t[2], xn, ks, H);
            pool_matvec(pp, v, t[3], xn, ks, H);
            rc = g3o_layer_decode(attn, q, k, v, t[5], t[6], kc[l], vc[l],
                                  g3o_is_global_layer(l) ? rg : rl, &cfg, l, pos, work);
            if (rc) break;
            pool_matvec(pp, proj, t[4], attn, H, qs);
            if (t[7]) g3o_rmsnorm_bf16(proj, proj, t[7], H, m->rmsnorm_eps);
            for (int j = 0; j < H; j++) x[j] = x[j] + proj[j];
            if (t[11])
                g3o_rmsnorm_bf16(xn, x, t[11], H, m->rmsnorm_eps);
            else
                memcpy(xn, x, (size_t)H * 4);
            pool_matvec(pp, gate, t[8], xn, I, H);
            pool_matvec(pp, up, t[9], xn, I, H);
            g3o_gelu_tanh(gate, I);
            for (int j = 0; j < I; j++) gate[j] = gate[j] * up[j];
            pool_matvec(pp, mlp, t[10], gate, H, I);
            if (t[12]) g3o_rmsnorm_bf16(mlp, mlp, t[12], H, m->rmsnorm_eps);
            for (int j = 0; j < H; j++) x[j] = x[j] + mlp[j];
        }
        if (rc) break;
        if (i >= n - n_logits) {
            g3o_rmsnorm_bf16(xn, x, norm, H, m->rmsnorm_eps);
            pool_matvec(pp, logits + (size_t)(i - (n - n_logits)) * V, embed, xn, V, H);
        }
    }
    if (!rc && hidden_last) memcpy(hidden_last, x, (size_t)H * 4);
done:
    if (pool_on) {
        pthread_mutex_lock(&pool.lock);
        pool.quit = 1;
        pthread_cond_broadcast(&pool.start);
        pthread_mutex_unlock(&pool.lock);
        for (int t = 1; t <= pool.workers; t++) pthread_join(tid[t], NULL);
        pthread_cond_destroy(&pool.start);
        pthread_cond_destroy(&pool.done_cv);
        pthread_mutex_destroy(&pool.lock);
    }
    free(x); free(xn); free(proj); free(mlp); free(q); free(k); free(v); free(attn);
    free(gate); free(up); free(work); free(rl); free(rg);
    return rc;
}

/* gemma3_transformer.c:396-512 with layer_mlp (:362-391), for a sequence of
 * tokens from an empty cache (positions 0..n-1), on one thread. */
int g3o_forward_seq(float *logits, float *hidden_last, const int *tokens, int n,
                    const uint16_t *embed, const uint16_t *const *layer_w, const uint16_t *norm,
                    const g3o_model *m) {
    const int L = m->num_layers, ks = m->num_kv_heads * m->head_dim;
    float **kc = calloc((size_t)L, sizeof(float *)), **vc = calloc((size_t)L, sizeof(float *));
    int rc = 0;
    if (!kc || !vc) {
        rc = -4;
        goto done;
    }
    for (int l = 0; l < L; l++) {
        const size_t rows = g3o_is_global_layer(l) ? (size_t)m->max_context : (size_t)m->sliding_window;
        kc[l] = calloc(rows * ks, 4);
        vc[l] = calloc(rows * ks, 4);
        if (!kc[l] || !vc[l]) {
            rc = -4;
            goto done;
        }
    }
    rc = g3o_forward_cached(logits, n, hidden_last, tokens, n, 0, embed, layer_w, norm, m, kc, vc, 1);
done:
    if (kc)
        for (int l = 0; l < L; l++) free(kc[l]);
    if (vc)
        for (int l = 0; l < L; l++) free(vc[l]);
    free(kc);
    free(vc);
    return rc;
}
