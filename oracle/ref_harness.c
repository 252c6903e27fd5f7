/*
 * ref_harness.c - drives the REAL reference attention code, compiled in place
 * from /root/reference (never copied), to write golden vectors and to time
 * the reference CPU baseline.  TEST INFRASTRUCTURE; built into oracle/_ref/
 * by oracle/Makefile only where /root/reference exists.
 *
 * gemma3_transformer.c is #included so that its static functions
 * layer_attention (gemma3_transformer.c:258-356) and cache_kv (:236-251) are
 * callable here.  layer_attention begins with the Q/K/V GEMVs and ends with
 * the o_proj GEMV; the harness feeds it one-hot bf16 projection matrices
 * with hidden_size = H_q*d + 2*H_kv*d, so x = [q | k | v] maps to q, k, v
 * exactly (each output is 1.0 * x_j plus exact zeros) and the o_proj output's
 * first H_q*d entries are attn_out exactly.  Everything between the GEMVs is
 * the reference's own code.
 *
 * The reference's batched prefill loop (gemma3_transformer.c:641-692) sits
 * inside a USE_BLAS-only function that cannot compile without cblas.h, so
 * ref_prefill_loop restates only its loop skeleton and calls the
 * reference's own rmsnorm / rope / cache_kv / causal_mask / gqa.
 */
#define _POSIX_C_SOURCE 199309L /* clock_gettime under -std=c11 */
#include "gemma3_transformer.c"

#include <stdint.h>
#include <time.h>

#define RH_D 256

static uint16_t *g_wq, *g_wk, *g_wv, *g_wo;
static int g_hq = -1, g_hkv = -1;

static int ensure_weights(int hq, int hkv) {
    if (g_wq && hq == g_hq && hkv == g_hkv) return 0;
    free(g_wq); free(g_wk); free(g_wv); free(g_wo);
    const int qs = hq * RH_D, ks = hkv * RH_D, hs = qs + 2 * ks;
    g_wq = (uint16_t *)calloc((size_t)qs * hs, 2);
    g_wk = (uint16_t *)calloc((size_t)ks * hs, 2);
    g_wv = (uint16_t *)calloc((size_t)ks * hs, 2);
    g_wo = (uint16_t *)calloc((size_t)hs * qs, 2);
    if (!g_wq || !g_wk || !g_wv || !g_wo) return -4;
    const uint16_t one = 0x3F80; /* bf16 1.0 */
    for (int r = 0; r < qs; r++) g_wq[(size_t)r * hs + r] = one;
    for (int r = 0; r < ks; r++) g_wk[(size_t)r * hs + qs + r] = one;
    for (int r = 0; r < ks; r++) g_wv[(size_t)r * hs + qs + ks + r] = one;
    for (int r = 0; r < qs; r++) g_wo[(size_t)r * qs + r] = one;
    g_hq = hq;
    g_hkv = hkv;
    return 0;
}

static gemma3_config harness_cfg(int hq, int hkv, int max_context, int window) {
    gemma3_config c;
    memset(&c, 0, sizeof c);
    c.vocab_size = GEMMA3_VOCAB_SIZE;
    c.num_layers = GEMMA3_NUM_LAYERS;
    c.num_heads = hq;
    c.num_kv_heads = hkv;
    c.head_dim = RH_D;
    c.hidden_size = hq * RH_D + 2 * hkv * RH_D;
    c.intermediate_size = GEMMA3_INTERMEDIATE_SIZE;
    c.max_context = max_context;
    c.sliding_window = window;
    c.rmsnorm_eps = GEMMA3_RMSNORM_EPS;
    c.rope_theta_local = GEMMA3_ROPE_THETA_LOCAL;
    c.rope_theta_global = GEMMA3_ROPE_THETA_GLOBAL;
    return c;
}

/* Thin exports of the reference kernels on the path. */
void ref_rope_precompute(float *f, int max_pos, int d, float theta) { gemma3_rope_precompute(f, max_pos, d, theta); }
void ref_rope_apply(float *x, const float *f, int d, int pos) { gemma3_rope_apply_precomputed(x, f, d, pos); }
void ref_rmsnorm_bf16(float *y, const float *x, const uint16_t *w, int n, float eps) { gemma3_rmsnorm_bf16(y, x, w, n, eps); }
void ref_softmax(float *x, int n) { gemma3_softmax_inplace(x, n); }
void ref_causal_mask(float *m, int n, int qp) { gemma3_causal_mask(m, n, qp); }
void ref_gqa(float *out, const float *q, const float *k, const float *v, int hq, int hkv,
             int seq_len, int d, float scale, const float *mask, float *scores) {
    gemma3_gqa(out, q, k, v, hq, hkv, seq_len, d, scale, mask, scores);
}
int ref_is_global_layer(int l) { return gemma3_is_global_layer(l); }
void ref_matvec_bf16(float *y, const uint16_t *A, const float *x, int M, int K) {
    gemma3_matvec_bf16(y, A, x, M, K, NULL);
}

/* The whole of layer_attention (gemma3_transformer.c:258-356) for one token
 * with caller-given projection weights: x [hidden] -> out [hidden] through
 * the Q/K/V GEMVs, QK-norm, RoPE, cache_kv, GQA and the o_proj GEMV. */
int ref_layer_attention(float *out, const float *x, const uint16_t *wq, const uint16_t *wk,
                        const uint16_t *wv, const uint16_t *wo, const uint16_t *q_norm,
                        const uint16_t *k_norm, float *k_cache, float *v_cache, const float *rope,
                        int hq, int hkv, int hidden, int layer, int pos, int max_context, int window) {
    gemma3_config cfg = harness_cfg(hq, hkv, max_context, window);
    cfg.hidden_size = hidden;
    const int qs = hq * RH_D, ks = hkv * RH_D;
    const int cap = max_context > window ? max_context : window;
    float *qb = (float *)malloc((size_t)qs * 4), *kb = (float *)malloc((size_t)ks * 4);
    float *vb = (float *)malloc((size_t)ks * 4), *ab = (float *)malloc((size_t)qs * 4);
    float *mask = (float *)malloc((size_t)cap * 4), *scores = (float *)malloc((size_t)cap * 4);
    float *tmp = (float *)malloc((size_t)(hidden > qs ? hidden : qs) * 4);
    int rc = 0;
    if (!qb || !kb || !vb || !ab || !mask || !scores || !tmp) { rc = -4; goto done; }
    layer_kv_cache cache;
    cache.k = k_cache;
    cache.v = v_cache;
    cache.pos = pos;
    layer_attention(out, x, wq, wk, wv, wo, q_norm, k_norm, &cache, qb, kb, vb, ab,
                    mask, scores, tmp, rope, NULL, &cfg, layer, pos);
done:
    free(qb); free(kb); free(vb); free(ab); free(mask); free(scores); free(tmp);
    return rc;
}

/* One decode step through the reference's layer_attention.
 * q/k/v: pre-norm inputs (not modified).  k_cache/v_cache: the layer's cache,
 * [rows][hkv][256] (rows = max_context for global layers, window for local).
 * On return attn_out [hq*256] holds the attention output, q_rot/k_rot (optional)
 * the normed + RoPE'd q and k, and the cache holds the new row. */
int ref_layer_decode(float *attn_out, float *q_rot, float *k_rot,
                     const float *q, const float *k, const float *v,
                     const uint16_t *q_norm, const uint16_t *k_norm,
                     float *k_cache, float *v_cache, const float *rope,
                     int hq, int hkv, int layer, int pos, int max_context, int window) {
    if (ensure_weights(hq, hkv)) return -4;
    gemma3_config cfg = harness_cfg(hq, hkv, max_context, window);
    const int qs = hq * RH_D, ks = hkv * RH_D, hs = cfg.hidden_size;
    const int cap = max_context > window ? max_context : window;
    float *x = (float *)malloc((size_t)hs * 4), *out = (float *)malloc((size_t)hs * 4);
    float *qb = (float *)malloc((size_t)qs * 4), *kb = (float *)malloc((size_t)ks * 4);
    float *vb = (float *)malloc((size_t)ks * 4), *ab = (float *)malloc((size_t)qs * 4);
    float *mask = (float *)malloc((size_t)cap * 4), *scores = (float *)malloc((size_t)cap * 4);
    float *tmp = (float *)malloc((size_t)hs * 4);
    int rc = 0;
    if (!x || !out || !qb || !kb || !vb || !ab || !mask || !scores || !tmp) { rc = -4; goto done; }
    memcpy(x, q, (size_t)qs * 4);
    memcpy(x + qs, k, (size_t)ks * 4);
    memcpy(x + qs + ks, v, (size_t)ks * 4);
    layer_kv_cache cache;
    cache.k = k_cache;
    cache.v = v_cache;
    cache.pos = pos;
    layer_attention(out, x, g_wq, g_wk, g_wv, g_wo, q_norm, k_norm, &cache, qb, kb, vb, ab,
                    mask, scores, tmp, rope, NULL, &cfg, layer, pos);
    memcpy(attn_out, out, (size_t)qs * 4);
    if (q_rot) memcpy(q_rot, qb, (size_t)qs * 4);
    if (k_rot) memcpy(k_rot, kb, (size_t)ks * 4);
done:
    free(x); free(out); free(qb); free(kb); free(vb); free(ab); free(mask); free(scores); free(tmp);
    return rc;
}

/* gemma3_transformer_forward (gemma3_transformer.c:396-512) itself, run for
 * tokens[0..n-1] at positions 0..n-1 from an empty cache, with caller-given
 * bf16 weights (layer_w: num_layers x 13 tensors in the gemma3_weights_t
 * field order) and model shape.  logits [n][vocab] holds every step's
 * logits; hidden_last [hidden] the hidden state after the last step. */
static int cmp_double(const void *a, const void *b);

/* The model config and gemma3_weights_t of caller-given tensors. */
static void harness_model(gemma3_config *cfg, gemma3_weights_t *w, const uint16_t *embed,
                          const uint16_t *const *layer_w, const uint16_t *norm, int vocab, int hidden,
                          int inter, int num_layers, int hq, int hkv, int max_context, int window) {
    *cfg = harness_cfg(hq, hkv, max_context, window);
    cfg->vocab_size = vocab;
    cfg->hidden_size = hidden;
    cfg->intermediate_size = inter;
    cfg->num_layers = num_layers;
    memset(w, 0, sizeof *w);
    w->embed_tokens = embed;
    w->norm = norm;
    for (int l = 0; l < num_layers; l++) {
        const uint16_t *const *t = layer_w + (size_t)l * 13;
        w->layers[l].input_layernorm = t[0];
        w->layers[l].q_proj = t[1];
        w->layers[l].k_proj = t[2];
        w->layers[l].v_proj = t[3];
        w->layers[l].o_proj = t[4];
        w->layers[l].q_norm = t[5];
        w->layers[l].k_norm = t[6];
        w->layers[l].post_attention_layernorm = t[7];
        w->layers[l].gate_proj = t[8];
        w->layers[l].up_proj = t[9];
        w->layers[l].down_proj = t[10];
        w->layers[l].pre_feedforward_layernorm = t[11];
        w->layers[l].post_feedforward_layernorm = t[12];
    }
}

/* CPU baseline of the whole-token forward: seconds per token of
 * gemma3_transformer_forward (one thread, no BLAS) at positions pos ..
 * pos + n_tokens - 1 of a cache whose earlier rows are zero (the attention's
 * cost does not depend on their values); the median after one warm-up token. */
double ref_time_forward(const uint16_t *embed, const uint16_t *const *layer_w, const uint16_t *norm,
                        int vocab, int hidden, int inter, int num_layers, int hq, int hkv,
                        int max_context, int window, int pos, int n_tokens) {
    if (num_layers < 1 || num_layers > GEMMA3_NUM_LAYERS || n_tokens < 1 || pos < 1 ||
        pos + n_tokens > max_context)
        return -1.0;
    gemma3_config cfg;
    gemma3_weights_t w;
    harness_model(&cfg, &w, embed, layer_w, norm, vocab, hidden, inter, num_layers, hq, hkv, max_context,
                  window);
    gemma3_kv_cache *cache = gemma3_kv_cache_alloc(&cfg, max_context);
    activation_buffers *buf = alloc_buffers(&cfg);
    float *rl = (float *)malloc((size_t)max_context * RH_D * 4);
    float *rg = (float *)malloc((size_t)max_context * RH_D * 4);
    float *logits = (float *)malloc((size_t)vocab * 4);
    double *t = (double *)malloc((size_t)n_tokens * sizeof(double));
    double med = -4.0;
    if (cache && buf && rl && rg && logits && t) {
        gemma3_rope_precompute(rl, max_context, RH_D, cfg.rope_theta_local);
        gemma3_rope_precompute(rg, max_context, RH_D, cfg.rope_theta_global);
        int rc = 0;
        for (int r = -1; r < n_tokens && !rc; r++) {
            const int p = r < 0 ? pos - 1 : pos + r;
            struct timespec a, b;
            clock_gettime(CLOCK_MONOTONIC, &a);
            rc = gemma3_transformer_forward(logits, (p * 7919) % vocab, p, &w, cache, buf, &cfg, 1, rl, rg, NULL);
            clock_gettime(CLOCK_MONOTONIC, &b);
            if (r >= 0) t[r] = (b.tv_sec - a.tv_sec) + 1e-9 * (b.tv_nsec - a.tv_nsec);
        }
        if (!rc) {
            qsort(t, (size_t)n_tokens, sizeof(double), cmp_double);
            med = t[n_tokens / 2];
        }
    }
    if (cache) gemma3_kv_cache_free(cache);
    if (buf) free_buffers(buf);
    free(rl); free(rg); free(logits); free(t);
    return med;
}

int ref_forward_seq(float *logits, float *hidden_last, const int *tokens, int n,
                    const uint16_t *embed, const uint16_t *const *layer_w, const uint16_t *norm,
                    int vocab, int hidden, int inter, int num_layers, int hq, int hkv,
                    int max_context, int window) {
    if (num_layers < 1 || num_layers > GEMMA3_NUM_LAYERS) return -1;
    gemma3_config cfg;
    gemma3_weights_t w;
    harness_model(&cfg, &w, embed, layer_w, norm, vocab, hidden, inter, num_layers, hq, hkv, max_context,
                  window);
    gemma3_kv_cache *cache = gemma3_kv_cache_alloc(&cfg, max_context);
    activation_buffers *buf = alloc_buffers(&cfg);
    float *rl = (float *)malloc((size_t)max_context * RH_D * 4);
    float *rg = (float *)malloc((size_t)max_context * RH_D * 4);
    int rc = 0;
    if (!cache || !buf || !rl || !rg) { rc = -4; goto done; }
    gemma3_rope_precompute(rl, max_context, RH_D, cfg.rope_theta_local);
    gemma3_rope_precompute(rg, max_context, RH_D, cfg.rope_theta_global);
    for (int i = 0; i < n && !rc; i++)
        rc = gemma3_transformer_forward(logits + (size_t)i * vocab, tokens[i], i, &w, cache, buf, &cfg, 1,
                                        rl, rg, NULL);
    if (!rc) memcpy(hidden_last, buf->x, (size_t)hidden * 4);
done:
    if (cache) gemma3_kv_cache_free(cache);
    if (buf) free_buffers(buf);
    free(rl);
    free(rg);
    return rc;
}

/* The per-token prefill attention loop of gemma3_transformer.c:641-692, on the
 * reference's own functions.  Q, K are modified in place (normed + RoPE'd). */
int ref_prefill_loop(float *attn_out, float *Q, float *K, const float *V,
                     const uint16_t *q_norm, const uint16_t *k_norm,
                     float *k_cache, float *v_cache, const float *rope,
                     int hq, int hkv, int layer, int start_pos, int n, int max_context, int window) {
    gemma3_config cfg = harness_cfg(hq, hkv, max_context, window);
    const int qs = hq * RH_D, ks = hkv * RH_D, d = RH_D;
    const int cap = max_context > window ? max_context : window;
    float *mask = (float *)malloc((size_t)cap * 4), *scores = (float *)malloc((size_t)cap * 4);
    if (!mask || !scores) { free(mask); free(scores); return -4; }
    layer_kv_cache cache;
    cache.k = k_cache;
    cache.v = v_cache;
    cache.pos = start_pos;
    const int is_global = gemma3_is_global_layer(layer);
    const float scale = 1.0f / sqrtf((float)d);
    for (int i = 0; i < n; i++) {
        const int pos = start_pos + i;
        float *qi = Q + (size_t)i * qs, *ki = K + (size_t)i * ks;
        const float *vi = V + (size_t)i * ks;
        if (q_norm && k_norm) {
            for (int h = 0; h < hq; h++) gemma3_rmsnorm_bf16(qi + h * d, qi + h * d, q_norm, d, cfg.rmsnorm_eps);
            for (int h = 0; h < hkv; h++) gemma3_rmsnorm_bf16(ki + h * d, ki + h * d, k_norm, d, cfg.rmsnorm_eps);
        }
        for (int h = 0; h < hq; h++) gemma3_rope_apply_precomputed(qi + h * d, rope, d, pos);
        for (int h = 0; h < hkv; h++) gemma3_rope_apply_precomputed(ki + h * d, rope, d, pos);
        cache_kv(&cache, ki, vi, ks, is_global, cfg.sliding_window, pos);
        int seq_len;
        if (is_global) {
            seq_len = pos + 1;
            gemma3_causal_mask(mask, seq_len, pos);
        } else {
            seq_len = (pos < cfg.sliding_window) ? pos + 1 : cfg.sliding_window;
            for (int s = 0; s < seq_len; s++) mask[s] = 0.0f;
        }
        gemma3_gqa(attn_out + (size_t)i * qs, qi, k_cache, v_cache, hq, hkv, seq_len, d, scale,
                   mask, scores);
    }
    free(mask);
    free(scores);
    return 0;
}

/* Time `reps` decode steps of the reference attention section (the n = 1 case
 * of ref_prefill_loop: norm, RoPE, cache_kv, mask, gemma3_gqa) at position pos
 * against caller-filled caches; returns the median seconds per step.  q, k are
 * restored from the inputs before every step. */
static int cmp_double(const void *a, const void *b) {
    double x = *(const double *)a, y = *(const double *)b;
    return (x > y) - (x < y);
}
double ref_time_decode(const float *q, const float *k, const float *v, const uint16_t *q_norm,
                       const uint16_t *k_norm, float *k_cache, float *v_cache, const float *rope,
                       int hq, int hkv, int layer, int pos, int max_context, int window,
                       int warmup, int reps) {
    const int qs = hq * RH_D, ks = hkv * RH_D;
    float *qb = (float *)malloc((size_t)qs * 4), *kb = (float *)malloc((size_t)ks * 4);
    float *out = (float *)malloc((size_t)qs * 4);
    double *t = (double *)malloc((size_t)(reps > 0 ? reps : 1) * sizeof(double));
    if (!qb || !kb || !out || !t) return -1.0;
    for (int r = -warmup; r < reps; r++) {
        memcpy(qb, q, (size_t)qs * 4);
        memcpy(kb, k, (size_t)ks * 4);
        struct timespec a, b;
        clock_gettime(CLOCK_MONOTONIC, &a);
        ref_prefill_loop(out, qb, kb, v, q_norm, k_norm, k_cache, v_cache, rope, hq, hkv, layer,
                         pos, 1, max_context, window);
        clock_gettime(CLOCK_MONOTONIC, &b);
        if (r >= 0) t[r] = (b.tv_sec - a.tv_sec) + 1e-9 * (b.tv_nsec - a.tv_nsec);
    }
    qsort(t, (size_t)reps, sizeof(double), cmp_double);
    const double med = reps > 0 ? t[reps / 2] : 0.0;
    free(qb); free(kb); free(out); free(t);
    return med;
}
