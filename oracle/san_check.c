/*
 * san_check.c - a driver for AddressSanitizer / UndefinedBehaviorSanitizer
 * (and, for the oracle's threaded paths, ThreadSanitizer) builds.  TEST
 * INFRASTRUCTURE: oracle/Makefile builds it (targets san / tsan) into
 * oracle/_san/; tests/test_sanitizers.py runs it on the CPU.
 *
 * Part 1 drives the oracle (g3_oracle.c) over small shapes that reach every
 * branch the parity tests use: ring wrap, chunked prefill, masks, absent
 * norms, ragged GEMV widths, a whole tiny model.  Its results are checked
 * against each other (the threaded prefill against the sequential one, token
 * by token decode against the prefill), so the run also fails on a wrong
 * answer, not only on a sanitizer report.
 *
 * Part 2 (not in the TSan build) drives the host side of libg3attn: every
 * entry point's argument checks, with NULL or invalid arguments and, where
 * no GPU is visible, the no-device failure of g3attn_create.  These paths run
 * before any device work, so they need no GPU.
 */
#define _POSIX_C_SOURCE 200112L /* setenv under -std=c11 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "g3_oracle.h"
#ifndef SAN_ORACLE_ONLY
#include "g3attn.h"
#include "g3backend.h"
#endif

static int g_fail;
#define CHECK(cond)                                                              \
    do {                                                                         \
        if (!(cond)) {                                                           \
            fprintf(stderr, "san_check: %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            g_fail = 1;                                                          \
        }                                                                        \
    } while (0)

enum { D = 256 };

static float *fnew(size_t n) { return (float *)calloc(n ? n : 1, sizeof(float)); }

static uint16_t *bf16_weights(size_t n, uint64_t seed, float scale) {
    float *f = fnew(n);
    g3o_gen_normal_bf16(f, n, seed, 0, 1);
    uint16_t *w = (uint16_t *)malloc(n * sizeof(uint16_t));
    for (size_t i = 0; i < n; i++) w[i] = g3o_f32_to_bf16_rne(f[i] * scale);
    free(f);
    return w;
}

/* Prefill of n tokens after `hist` decoded ones on one layer, three ways:
 * token by token through g3o_layer_decode, g3o_prefill, g3o_prefill_mt. */
static void prefill_case(int layer, int hist, int n, int threads, int with_norm) {
    g3o_config cfg;
    g3o_default_config(&cfg);
    cfg.num_layers = 6;
    cfg.max_context = 96;
    cfg.sliding_window = 16;
    const int qs = cfg.num_heads * D, ks = cfg.num_kv_heads * D;
    const int rows = g3o_is_global_layer(layer) ? cfg.max_context : cfg.sliding_window;
    const int total = hist + n;
    float *rope = fnew((size_t)cfg.max_context * D);
    g3o_rope_precompute(rope, cfg.max_context, D, g3o_layer_theta(&cfg, layer));
    uint16_t *qn = with_norm ? bf16_weights(D, 11, 0.125f) : NULL;
    uint16_t *kn = with_norm ? bf16_weights(D, 12, 0.125f) : NULL;
    float *Q = fnew((size_t)total * qs), *K = fnew((size_t)total * ks), *V = fnew((size_t)total * ks);
    g3o_gen_normal_bf16(Q, (size_t)total * qs, 21, 0, 2);
    g3o_gen_normal_bf16(K, (size_t)total * ks, 22, 0, 2);
    g3o_gen_normal_bf16(V, (size_t)total * ks, 23, 0, 2);

    float *kc[3], *vc[3], *out[3];
    for (int w = 0; w < 3; w++) {
        kc[w] = fnew((size_t)rows * ks);
        vc[w] = fnew((size_t)rows * ks);
        out[w] = fnew((size_t)n * qs);
    }
    float *work = fnew(2 * (size_t)(cfg.max_context > cfg.sliding_window ? cfg.max_context : cfg.sliding_window));
    float *q = fnew(qs), *k = fnew(ks), *a = fnew(qs);
    /* history, identical in all three caches */
    for (int t = 0; t < hist; t++)
        for (int w = 0; w < 3; w++) {
            memcpy(q, Q + (size_t)t * qs, qs * 4);
            memcpy(k, K + (size_t)t * ks, ks * 4);
            CHECK(g3o_layer_decode(a, q, k, V + (size_t)t * ks, qn, kn, kc[w], vc[w], rope, &cfg, layer, t, work) == 0);
        }
    /* way 0: token by token */
    for (int t = 0; t < n; t++) {
        memcpy(q, Q + (size_t)(hist + t) * qs, qs * 4);
        memcpy(k, K + (size_t)(hist + t) * ks, ks * 4);
        CHECK(g3o_layer_decode(out[0] + (size_t)t * qs, q, k, V + (size_t)(hist + t) * ks, qn, kn, kc[0], vc[0],
                               rope, &cfg, layer, hist + t, work) == 0);
    }
    /* ways 1, 2: the batch loops (they norm + RoPE Q/K in place: copies) */
    for (int w = 1; w < 3; w++) {
        float *Qb = fnew((size_t)n * qs), *Kb = fnew((size_t)n * ks);
        memcpy(Qb, Q + (size_t)hist * qs, (size_t)n * qs * 4);
        memcpy(Kb, K + (size_t)hist * ks, (size_t)n * ks * 4);
        if (w == 1)
            CHECK(g3o_prefill(out[1], Qb, Kb, V + (size_t)hist * ks, qn, kn, kc[1], vc[1], rope, &cfg, layer, hist, n,
                              work) == 0);
        else
            CHECK(g3o_prefill_mt(out[2], Qb, Kb, V + (size_t)hist * ks, qn, kn, kc[2], vc[2], rope, &cfg, layer, hist,
                                 n, threads) == 0);
        free(Qb);
        free(Kb);
    }
    CHECK(memcmp(out[0], out[1], (size_t)n * qs * 4) == 0);
    CHECK(memcmp(out[1], out[2], (size_t)n * qs * 4) == 0);
    CHECK(memcmp(kc[1], kc[2], (size_t)rows * ks * 4) == 0 && memcmp(vc[0], vc[2], (size_t)rows * ks * 4) == 0);
    /* a subset of rows, threaded */
    {
        int sel[3] = {n - 1, 0, n / 2};
        float *Qb = fnew((size_t)n * qs), *Kb = fnew((size_t)n * ks), *o = fnew(3 * (size_t)qs);
        float *kx = fnew((size_t)rows * ks), *vx = fnew((size_t)rows * ks);
        memcpy(Qb, Q + (size_t)hist * qs, (size_t)n * qs * 4);
        memcpy(Kb, K + (size_t)hist * ks, (size_t)n * ks * 4);
        /* history again, through the batch loop */
        if (hist > 0) {
            float *Qh = fnew((size_t)hist * qs), *Kh = fnew((size_t)hist * ks), *oh = fnew((size_t)hist * qs);
            memcpy(Qh, Q, (size_t)hist * qs * 4);
            memcpy(Kh, K, (size_t)hist * ks * 4);
            CHECK(g3o_prefill(oh, Qh, Kh, V, qn, kn, kx, vx, rope, &cfg, layer, 0, hist, work) == 0);
            free(Qh); free(Kh); free(oh);
        }
        CHECK(g3o_prefill_rows(o, Qb, Kb, V + (size_t)hist * ks, qn, kn, kx, vx, rope, &cfg, layer, hist, n, sel, 3,
                               threads) == 0);
        for (int j = 0; j < 3; j++) CHECK(memcmp(o + (size_t)j * qs, out[0] + (size_t)sel[j] * qs, qs * 4) == 0);
        free(Qb); free(Kb); free(o); free(kx); free(vx);
    }
    /* overflow is refused */
    CHECK(g3o_layer_decode(a, q, k, V, qn, kn, kc[0], vc[0], rope, &cfg, layer, cfg.max_context, work) == -8);
    for (int w = 0; w < 3; w++) {
        free(kc[w]); free(vc[w]); free(out[w]);
    }
    free(work); free(q); free(k); free(a); free(Q); free(K); free(V); free(rope); free(qn); free(kn);
}

static void gqa_case(int n_heads, int n_kv, int seq, int with_mask) {
    const size_t qs = (size_t)n_heads * D, ks = (size_t)n_kv * D;
    float *q = fnew(qs), *k = fnew(seq * ks), *v = fnew(seq * ks), *o1 = fnew(qs), *o2 = fnew(qs);
    float *m = with_mask ? fnew(seq) : NULL, *sc = fnew(seq);
    int *rows = (int *)malloc(seq * sizeof(int));
    g3o_gen_normal_bf16(q, qs, 31, 0, 1);
    g3o_gen_normal_bf16(k, seq * ks, 32, 0, 1);
    g3o_gen_normal_bf16(v, seq * ks, 33, 0, 1);
    if (m) g3o_causal_mask(m, seq, seq / 2);
    for (int i = 0; i < seq; i++) rows[i] = i;
    g3o_gqa(o1, q, k, v, n_heads, n_kv, seq, D, 0.0625f, m, sc);
    g3o_gqa_rows(o2, q, k, v, rows, n_heads, n_kv, seq, D, 0.0625f, m, sc);
    CHECK(memcmp(o1, o2, qs * 4) == 0);
    for (size_t i = 0; i < qs; i++) CHECK(isfinite(o1[i]));
    free(q); free(k); free(v); free(o1); free(o2); free(m); free(sc); free(rows);
}

static void matvec_case(int M, int K) {
    uint16_t *A = bf16_weights((size_t)M * K, 41, 1.0f);
    float *x = fnew(K), *y = fnew(M);
    g3o_gen_normal_bf16(x, K, 42, 0, 1);
    g3o_matvec_bf16(y, A, x, M, K);
    for (int r = 0; r < M; r++) {
        double s = 0;
        for (int c = 0; c < K; c++) s += (double)g3o_bf16_to_f32(A[(size_t)r * K + c]) * x[c];
        CHECK(fabs(s - y[r]) <= 1e-4 * (1 + fabs(s)) + 1e-3);
    }
    free(A); free(x); free(y);
}

static void forward_case(void) {
    g3o_model m = {64, 512, 256, 6, 8, 4, D, 32, 8, 1e-6f, 10000.0f, 1000000.0f};
    const int qs = m.num_heads * D, ks = m.num_kv_heads * D, H = m.hidden_size, I = m.intermediate_size;
    const size_t n13[13] = {H, (size_t)qs * H, (size_t)ks * H, (size_t)ks * H, (size_t)H * qs, D, D, H,
                            (size_t)I * H, (size_t)I * H, (size_t)H * I, H, H};
    uint16_t *embed = bf16_weights((size_t)m.vocab_size * H, 51, 1.0f), *norm = bf16_weights(H, 52, 0.125f);
    const uint16_t **lw = (const uint16_t **)calloc(13 * (size_t)m.num_layers, sizeof(uint16_t *));
    for (int l = 0; l < m.num_layers; l++)
        for (int j = 0; j < 13; j++) {
            const int optional = j == 7 || j == 11 || j == 12 || j == 5 || j == 6;
            if (l == 3 && optional) continue; /* absent norms */
            const float scale = (j == 0 || (j >= 5 && j != 8 && j != 9 && j != 10)) ? 0.125f : 0.05f;
            lw[13 * l + j] = bf16_weights(n13[j], 100 + 13 * l + j, scale);
        }
    const int n = 30; /* wraps the 8-row window */
    int tokens[30];
    for (int i = 0; i < n; i++) tokens[i] = (i * 37 + 5) % m.vocab_size;
    float *logits = fnew((size_t)n * m.vocab_size), *hid = fnew(H);
    CHECK(g3o_forward_seq(logits, hid, tokens, n, embed, lw, norm, &m) == 0);
    for (size_t i = 0; i < (size_t)n * m.vocab_size; i++) CHECK(isfinite(logits[i]));
    for (int i = 0; i < 13 * m.num_layers; i++) free((void *)lw[i]);
    free(lw); free(embed); free(norm); free(logits); free(hid);
}

static void oracle_part(void) {
    /* RoPE table and apply, the whole range of a small table */
    float *t = fnew(64 * D), *x = fnew(D);
    g3o_rope_precompute(t, 64, D, 10000.0f);
    g3o_gen_normal_bf16(x, D, 1, 0, 0);
    for (int p = 0; p < 64; p++) g3o_rope_apply(x, t, D, p);
    free(t); free(x);
    /* generator: odd sizes, offsets, thread counts */
    for (int th = 0; th <= 3; th++) {
        float *g = fnew(1001);
        g3o_gen_normal_bf16(g, 1001, 7, 13, th);
        for (int i = 0; i < 1001; i++) CHECK(isfinite(g[i]) && g3o_bf16_to_f32(g3o_f32_to_bf16_trunc(g[i])) == g[i]);
        free(g);
    }
    for (int layer = 0; layer < 6; layer += 5)
        for (int hist = 0; hist <= 20; hist += 20) {
            prefill_case(layer, hist, 7, 3, 1);
            prefill_case(layer, hist, 19, 4, 0);
        }
    gqa_case(8, 4, 37, 1);
    gqa_case(8, 2, 5, 0);
    gqa_case(4, 4, 1, 1);
    for (int K = 1; K <= 40; K += 13) matvec_case(5, K);
    matvec_case(3, 2560);
    forward_case();
}

#ifndef SAN_ORACLE_ONLY
/* Every entry point with a NULL context or bad arguments: a negative code and
 * a message, no crash, no read of the bad pointers. */
static void host_part(int have_gpu) {
    g3attn_config cfg;
    g3attn_default_config(&cfg);
    CHECK(g3attn_is_global_layer(5) && !g3attn_is_global_layer(4));
    float *t = fnew(64 * D), *o = fnew(64 * D);
    g3attn_rope_precompute(t, 64, D, 10000.0f);
    g3o_rope_precompute(o, 64, D, 10000.0f);
    CHECK(memcmp(t, o, 64 * D * 4) == 0);
    cfg.max_context = 64;
    CHECK(!g3attn_create(NULL, 64, t, t));
    CHECK(!g3attn_create(&cfg, 0, t, t));
    CHECK(!g3attn_create(&cfg, 64, t, NULL));
    g3attn_config bad = cfg;
    bad.head_dim = 128;
    CHECK(!g3attn_create(&bad, 64, t, t));
    bad = cfg;
    bad.num_kv_heads = 3;
    CHECK(!g3attn_create(&bad, 64, t, t));
    bad = cfg;
    bad.sliding_window = 0;
    CHECK(!g3attn_create(&bad, 64, t, t));
    setenv("G3ATTN_FAULT", "upload,create", 1);
    CHECK(!g3attn_create(&cfg, 64, t, t) && strstr(g3attn_last_error(), "injected"));
    unsetenv("G3ATTN_FAULT");
    if (!have_gpu) {
        CHECK(!g3attn_create(&cfg, 64, t, t));
        CHECK(!g3attn_create(&cfg, 64, NULL, NULL));
        CHECK(!gemma3_metal_init(&cfg, 64));
        CHECK(!gemma3_metal_available());
    }
    float buf[8] = {0};
    uint16_t w16[8] = {0};
    int toks[2] = {1, 2};
    CHECK(g3attn_decode(NULL, 0, 0, buf, buf, buf, NULL, NULL, buf) < 0);
    CHECK(g3attn_decode_device(NULL, 0, 0, buf, buf, buf, NULL, NULL, buf) < 0);
    CHECK(g3attn_prefill(NULL, 0, 0, 1, buf, buf, buf, NULL, NULL, buf) < 0);
    CHECK(g3attn_prefill_device(NULL, 0, 0, 1, buf, buf, buf, NULL, NULL, buf) < 0);
    CHECK(g3attn_kv_append(NULL, 0, 0, 1, buf, buf, NULL) < 0);
    CHECK(g3attn_kv_append_device(NULL, 0, 0, 1, buf, buf, NULL) < 0);
    CHECK(g3attn_kv_write(NULL, 0, 0, 1, buf, buf) < 0);
    CHECK(g3attn_kv_read(NULL, 0, 0, 1, buf, buf) < 0);
    CHECK(g3attn_upload_rope(NULL, t, t, 64, D) < 0);
    CHECK(g3attn_upload_weights(NULL, buf) < 0);
    CHECK(g3attn_forward_token(NULL, 0, 0, buf, 1) < 0);
    CHECK(g3attn_forward_token_device(NULL, 0, 0, buf) < 0);
    CHECK(g3attn_prefill_tokens(NULL, toks, 2, 0, buf) < 0);
    CHECK(g3attn_forward_device(NULL, NULL, 0, 0, buf, 1, NULL) < 0);
    CHECK(g3attn_prefill_forward_device(NULL, NULL, toks, 2, 0, buf) < 0);
    CHECK(g3attn_matvec_bf16_device(NULL, buf, w16, buf, 2, 2) < 0);
    CHECK(g3attn_matmul_bf16_device(NULL, buf, w16, buf, 1, 4, 2) < 0);
    CHECK(g3attn_qkv_proj_device(NULL, buf, w16, w16, w16, buf, buf, buf) < 0);
    CHECK(g3attn_layer_attention_device(NULL, 0, 0, buf, w16, w16, w16, w16, NULL, NULL, buf) < 0);
    CHECK(g3attn_synchronize(NULL) < 0);
    CHECK(g3attn_profile_enable(NULL, 1) < 0);
    double ms;
    int cnt;
    CHECK(g3attn_profile_read(NULL, 0, &ms, &cnt) < 0);
    CHECK(g3attn_device_weights(NULL) == NULL);
    g3attn_destroy(NULL);
    g3attn_reset(NULL);
    /* the drop-ins' shape checks come before any device use */
    g3attn_gqa(NULL, buf, buf, buf, 8, 4, 4, D, 0.0625f, NULL, NULL); /* void, as gemma3_gqa */
    CHECK(strlen(g3attn_last_error()) > 0);
    g3attn_gqa(buf, buf, buf, buf, 8, 3, 4, D, 0.0625f, NULL, NULL);
    CHECK(strlen(g3attn_last_error()) > 0);
    g3attn_gqa(buf, buf, buf, buf, 8, 4, 0, D, 0.0625f, NULL, NULL);
    CHECK(g3attn_gqa_noalloc(buf, buf, buf, buf, 8, 4, 4, 128, 0.0625f, NULL, NULL) < 0);
    CHECK(g3attn_gqa_noalloc(buf, buf, buf, buf, 64, 4, 4, D, 0.0625f, NULL, NULL) < 0);
    CHECK(g3attn_gqa_noalloc(NULL, buf, buf, buf, 8, 4, 4, D, 0.0625f, NULL, NULL) < 0);
    g3attn_matvec_bf16(buf, w16, buf, 0, 2, NULL);
    g3attn_matvec_bf16(NULL, w16, buf, 2, 2, NULL);
    CHECK(strlen(g3attn_last_error()) > 0);
    CHECK(gemma3_metal_upload_weights(NULL, buf) < 0);
    CHECK(gemma3_metal_upload_rope(NULL, t, t, 64, D) < 0);
    CHECK(gemma3_metal_forward_token(NULL, 0, 0, buf, 1) < 0);
    CHECK(gemma3_metal_prefill(NULL, toks, 2, 0, buf) < 0);
    gemma3_metal_reset_cache(NULL);
    gemma3_metal_free(NULL);
    free(t);
    free(o);
}
#endif

int main(int argc, char **argv) {
    oracle_part();
#ifndef SAN_ORACLE_ONLY
    host_part(argc > 1 && strcmp(argv[1], "--gpu-present") == 0);
#else
    (void)argc;
    (void)argv;
#endif
    if (g_fail) {
        fprintf(stderr, "san_check: FAILED\n");
        return 1;
    }
    printf("san_check: ok\n");
    return 0;
}
