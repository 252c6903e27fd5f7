/*
 * g3attn.c - C11 host side of libg3attn.so: the entry points of
 * include/g3attn.h.  Argument checking, error codes, the device context (KV
 * cache, RoPE tables, workspaces, stream) and launch shapes live here; the
 * kernels sit behind the thin launcher ABI of csrc/g3k.h.
 *
 * Built with gcc -std=c11 against the HIP runtime's C API.
 */
#include "g3attn.h"

#include <hip/hip_runtime_api.h>
#include <limits.h>
#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../csrc/g3k.h"

#define G3_OK 0
#define G3_ERR_INVALID_ARG (-1)
#define G3_ERR_OUT_OF_MEMORY (-4)
#define G3_ERR_CONTEXT_OVERFLOW (-8)

#define LOG2E 1.4426950408889634f
_Static_assert(G3ATTN_NOALLOC_MAX_HEADS == G3K_NOALLOC_MAX_HEADS, "fixed scratch size");
#define G3_PROF_CAP 256
#define D G3K_HEAD_DIM

/* ------------------------------------------------------------------ errors */

static _Thread_local char g_err[512];

static void set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

const char *g3attn_last_error(void) { return g_err; }

static int hip_fail(hipError_t e, const char *what) {
    set_err("%s: %s", what, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? G3_ERR_OUT_OF_MEMORY : G3_ERR_INVALID_ARG;
}

#define HIP_TRY(call, what)                          \
    do {                                             \
        hipError_t e_ = (call);                      \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

/* ------------------------------------------------------------------ config */

void g3attn_default_config(g3attn_config *c) {
    c->vocab_size = 262208;
    c->hidden_size = 2560;
    c->intermediate_size = 10240;
    c->num_layers = 34;
    c->num_heads = 8;
    c->num_kv_heads = 4;
    c->head_dim = 256;
    c->max_context = 8192;
    c->sliding_window = 1024;
    c->rmsnorm_eps = 1e-6f;
    c->rope_theta_local = 10000.0f;
    c->rope_theta_global = 1000000.0f;
}

int g3attn_is_global_layer(int layer) { return (layer + 1) % 6 == 0; }

static int check_shape(int n_heads, int n_kv, int head_dim) {
    if (head_dim != D) {
        set_err("head_dim %d unsupported (this build: %d)", head_dim, D);
        return 0;
    }
    if (n_heads <= 0 || n_kv <= 0 || n_heads % n_kv) {
        set_err("num_heads %d not a multiple of num_kv_heads %d", n_heads, n_kv);
        return 0;
    }
    const int g = n_heads / n_kv;
    if (g != 1 && g != 2 && g != 4) {
        set_err("GQA group %d unsupported (1, 2 or 4)", g);
        return 0;
    }
    return 1;
}

/* ------------------------------------------------------------------ context */

struct g3attn_ctx {
    g3attn_config cfg;
    int max_context, device, group;
    hipStream_t stream;
    float *rope_local, *rope_global;
    int have_rope;     /* both tables uploaded (at create or by g3attn_upload_rope) */
    float **kc, **vc;
    int *rows;
    float *ws_acc, *ws_ml;
    /* staging of the host-pointer decode: q | k | v | q_norm | k_norm, and out */
    unsigned char *h_in, *d_in;
    float *h_out, *d_out;
    size_t in_bytes;
    /* grow-on-demand device buffers for host-pointer batch calls */
    void *d_big;
    size_t d_big_cap;
    /* grow-on-demand prefill workspace (staged keys and values) */
    void *d_pf;
    size_t d_pf_cap;
    /* layer_attention scratch: q | k | v | attn of one token */
    float *d_la;
    size_t d_la_cap;
    /* token forward activations: x | x_norm | proj | mlp | h (see forward) */
    float *d_fw;
    size_t d_fw_cap;
    /* uploaded model (g3attn_upload_weights): one device arena holding every
     * tensor, the struct of device addresses into it, and the logits of the
     * host-output forward (device, and pinned host staging) */
    void *d_wt;
    g3attn_weights wt;
    int have_wt;
    float *d_logits, *h_logits;
    /* batched prefill activations (see prefill_forward) and token ids */
    void *d_pb;
    size_t d_pb_cap;
    int *d_tok;
    size_t d_tok_cap;
    /* prefill: staging sets *d_vflag = pf_epoch when a value is not exactly
     * bf16 (the attention kernel then adds its V_lo pass) */
    int *d_vflag;
    int pf_epoch;
    /* prefill key splits: per (query block, KV head) arrival counters, zeroed
     * once; each call's S arrivals wrap them back to zero */
    unsigned *d_arrive;
    /* one-launch decode: arrival counters (G3K_XM_COUNTERS), zeroed once and
     * left zero by every launch; xm_ok: the workgroup -> XCD placement probe
     * passed at create; xmerge: G3ATTN_DECODE_XMERGE (0 off, 1 local layers,
     * 2 every layer with few enough splits) */
    unsigned *d_xcount;
    int xm_ok, xmerge;
    /* kernel timing (g3attn_profile_*): event pairs per kind */
    struct {
        int on;
        hipEvent_t ev[2][G3_PROF_CAP][2];
        int used[2];
        double ms[2];
        int count[2];
    } prof;
    int last_splits[3]; /* g3attn_last_splits: decode, prefill, decode heads per one-launch workgroup */
    int split_rows; /* 0 = heuristic */
    int min_rows;   /* smallest heuristic split */
    int prefill_qpw; /* prefill queries per wave: 16 or 32 (G3ATTN_PREFILL_QPW) */
    int prefill_sched; /* prefill phase schedule 0 / 1 (G3ATTN_PREFILL_SCHED) */
    int prefill_ksplit; /* G3ATTN_PREFILL_SPLITS: 1, 2 or 4 key splits for every prefill; 0 = the
                         * makespan model (prefill_splits) */
    int prefill_x8;    /* prefill scores: 1 = fp16 hi + fp8 cross terms (default), 0 = three
                        * fp16 passes (G3ATTN_PREFILL_QK=exact) */
    int target_wgs; /* decode workgroups per call (all KV heads) */
    int n_cu;       /* compute units of the device */
    /* decode: non-temporal cache loads on 1 every layer, 2 global layers
     * only, and every layer inside the token forward (the default), 0 none
     * (G3ATTN_DECODE_NT) */
    int nt_loads;
    /* token forward: residual steps folded into the next GEMV's prologue
     * (bit 0: into the Q/K/V launch, bit 1: into the gate/up launch;
     * G3ATTN_FORWARD_FOLD) */
    int forward_fold;
};

static void prof_destroy(g3attn_ctx *c) {
    for (int k = 0; k < 2; k++)
        for (int i = 0; i < G3_PROF_CAP; i++)
            for (int j = 0; j < 2; j++)
                if (c->prof.ev[k][i][j]) {
                    hipEventDestroy(c->prof.ev[k][i][j]);
                    c->prof.ev[k][i][j] = NULL;
                }
    c->prof.on = 0;
}

static void ctx_free(g3attn_ctx *c) {
    if (!c) return;
    prof_destroy(c);
    if (c->kc)
        for (int l = 0; l < c->cfg.num_layers; l++) hipFree(c->kc[l]);
    if (c->vc)
        for (int l = 0; l < c->cfg.num_layers; l++) hipFree(c->vc[l]);
    free(c->kc);
    free(c->vc);
    free(c->rows);
    hipFree(c->rope_local);
    hipFree(c->rope_global);
    hipFree(c->ws_acc);
    hipFree(c->ws_ml);
    hipFree(c->d_in);
    hipFree(c->d_out);
    hipFree(c->d_big);
    hipFree(c->d_pf);
    hipFree(c->d_vflag);
    hipFree(c->d_arrive);
    hipFree(c->d_xcount);
    hipFree(c->d_la);
    hipFree(c->d_fw);
    hipFree(c->d_wt);
    hipFree(c->d_logits);
    hipFree(c->d_pb);
    hipFree(c->d_tok);

    if (c->h_logits) hipHostFree(c->h_logits);
    if (c->h_in) hipHostFree(c->h_in);
    if (c->h_out) hipHostFree(c->h_out);
    if (c->stream) hipStreamDestroy(c->stream);
    free(c);
}

/* Host-forced failures for testing the caller's fallback paths: G3ATTN_FAULT
 * is a comma-separated list of sites ("create", "upload", "forward").  A
 * listed site fails as its real counterpart would (create returns NULL,
 * upload returns -4, a forward returns -1) before any GPU work is issued. */
static int fault_at(const char *site) {
    const char *f = getenv("G3ATTN_FAULT");
    const size_t n = strlen(site);
    while (f && *f) {
        const char *e = strchr(f, ',');
        const size_t len = e ? (size_t)(e - f) : strlen(f);
        if (len == n && strncmp(f, site, n) == 0) return 1;
        f = e ? e + 1 : NULL;
    }
    return 0;
}

static int alloc_dev(void **p, size_t bytes, const char *what) {
    hipError_t e = hipMalloc(p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        *p = NULL;
        set_err("hipMalloc(%zu) for %s: %s", bytes, what, hipGetErrorString(e));
        return 0;
    }
    return 1;
}

/* Decode combine workspace: split slots [H_kv][G3K_MAX_SPLITS], each
 * group * head_dim floats (+ group * 2 for max and sum). */
static size_t ws_slots(int n_kv) { return (size_t)n_kv * G3K_MAX_SPLITS; }

/* The one-launch decode merges each run's splits in one XCD's L2, so it
 * needs the workgroups whose ids agree mod 8 to run on one XCD (the MI355X
 * dispatcher deals workgroup i to XCD i mod 8).  Checked once per context
 * on a 512-workgroup probe launch; any mismatch, or a failed launch, keeps
 * every decode on the two-launch form. */
static int xcd_placement_ok(g3attn_ctx *c) {
    enum { N = 512 };
    unsigned *d = NULL, h[N];
    int ok = 0;
    if (hipMalloc((void **)&d, sizeof h) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    if (g3k_xcd_probe(d, N, c->stream) == hipSuccess &&
        hipMemcpyAsync(h, d, sizeof h, hipMemcpyDeviceToHost, c->stream) == hipSuccess &&
        hipStreamSynchronize(c->stream) == hipSuccess) {
        ok = 1;
        for (int i = 8; i < N; i++) ok &= h[i] == h[i % 8];
    }
    (void)hipGetLastError();
    hipFree(d);
    return ok;
}

g3attn_ctx *g3attn_create(const g3attn_config *cfg, int max_context,
                          const float *rope_local, const float *rope_global) {
    g_err[0] = 0;
    if (!cfg || !rope_local != !rope_global || max_context <= 0) {
        set_err("g3attn_create: null config, one RoPE table without the other, or max_context <= 0");
        return NULL;
    }
    if (fault_at("create")) {
        set_err("g3attn_create: injected failure (G3ATTN_FAULT=create)");
        return NULL;
    }
    if (!check_shape(cfg->num_heads, cfg->num_kv_heads, cfg->head_dim)) return NULL;
    if (cfg->num_layers <= 0 || cfg->num_layers > 4096 || cfg->sliding_window <= 0) {
        set_err("g3attn_create: num_layers %d / sliding_window %d out of range", cfg->num_layers,
                cfg->sliding_window);
        return NULL;
    }
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess || ndev == 0) {
        set_err("g3attn_create: no HIP device (%s)", hipGetErrorString(e));
        return NULL;
    }
    g3attn_ctx *c = (g3attn_ctx *)calloc(1, sizeof *c);
    if (!c) {
        set_err("g3attn_create: out of host memory");
        return NULL;
    }
    c->cfg = *cfg;
    c->max_context = max_context;
    c->group = cfg->num_heads / cfg->num_kv_heads;
    const char *ov = getenv("G3ATTN_SPLIT_ROWS");
    c->split_rows = ov ? atoi(ov) : 0;
    if (hipGetDevice(&c->device) != hipSuccess) goto fail_rt;
    if (hipDeviceGetAttribute(&c->n_cu, hipDeviceAttributeMultiprocessorCount, c->device) != hipSuccess ||
        c->n_cu < 1)
        c->n_cu = 256;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) goto fail_rt;

    const size_t rope_bytes = (size_t)max_context * D * sizeof(float);
    if (!alloc_dev((void **)&c->rope_local, rope_bytes, "rope table")) goto fail;
    if (!alloc_dev((void **)&c->rope_global, rope_bytes, "rope table")) goto fail;
    if (rope_local) {
        if (hipMemcpy(c->rope_local, rope_local, rope_bytes, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(c->rope_global, rope_global, rope_bytes, hipMemcpyHostToDevice) != hipSuccess)
            goto fail_rt;
        c->have_rope = 1;
    }

    const int L = cfg->num_layers;
    c->kc = (float **)calloc((size_t)L, sizeof(float *));
    c->vc = (float **)calloc((size_t)L, sizeof(float *));
    c->rows = (int *)calloc((size_t)L, sizeof(int));
    if (!c->kc || !c->vc || !c->rows) {
        set_err("g3attn_create: out of host memory");
        goto fail;
    }
    for (int l = 0; l < L; l++) {
        c->rows[l] = g3attn_is_global_layer(l) ? max_context : cfg->sliding_window;
        const size_t bytes = (size_t)cfg->num_kv_heads * c->rows[l] * D * sizeof(float);
        if (!alloc_dev((void **)&c->kc[l], bytes, "K cache")) goto fail;
        if (!alloc_dev((void **)&c->vc[l], bytes, "V cache")) goto fail;
        /* the reference callocs its cache (gemma3_transformer.c:199-200) */
        if (hipMemset(c->kc[l], 0, bytes) != hipSuccess || hipMemset(c->vc[l], 0, bytes) != hipSuccess)
            goto fail_rt;
    }
    const size_t slots = ws_slots(cfg->num_kv_heads) * c->group;
    if (!alloc_dev((void **)&c->ws_acc, slots * D * sizeof(float), "decode workspace")) goto fail;
    if (!alloc_dev((void **)&c->ws_ml, slots * 2 * sizeof(float), "decode workspace")) goto fail;
    if (!alloc_dev((void **)&c->d_vflag, sizeof(int), "prefill flag")) goto fail;
    if (hipMemset(c->d_vflag, 0, sizeof(int)) != hipSuccess) goto fail_rt;
    {
        const size_t nb = (size_t)G3K_PREFILL_ARRIVE(max_context, cfg->num_kv_heads) * sizeof(unsigned);
        if (!alloc_dev((void **)&c->d_arrive, nb, "prefill arrival counters")) goto fail;
        if (hipMemset(c->d_arrive, 0, nb) != hipSuccess) goto fail_rt;
    }
    {
        const size_t nb = G3K_XM_COUNTERS(cfg->num_heads) * sizeof(unsigned);
        if (!alloc_dev((void **)&c->d_xcount, nb, "decode arrival counters")) goto fail;
        if (hipMemset(c->d_xcount, 0, nb) != hipSuccess) goto fail_rt;
        c->xm_ok = xcd_placement_ok(c);
    }
    {
        const char *w = getenv("G3ATTN_DECODE_WGS");
        const char *mr = getenv("G3ATTN_SPLIT_MIN_ROWS");
        int cus = 0;
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, c->device);
        c->target_wgs = w ? atoi(w) : 2 * (cus > 0 ? cus : 256);
        c->min_rows = mr ? atoi(mr) : G3K_SPLIT_GRAIN;
        const char *qpw = getenv("G3ATTN_PREFILL_QPW");
        c->prefill_qpw = (qpw && atoi(qpw) == 32) ? 32 : 16;
        const char *sch = getenv("G3ATTN_PREFILL_SCHED");
        c->prefill_sched = sch ? atoi(sch) : 1;
        const char *qk = getenv("G3ATTN_PREFILL_QK");
        c->prefill_x8 = !(qk && strcmp(qk, "exact") == 0);
        const char *ks = getenv("G3ATTN_PREFILL_SPLITS");
        const int ksv = ks ? atoi(ks) : 0;
        c->prefill_ksplit = (ksv == 1 || ksv == 2 || ksv == 4) ? ksv : 0;
        const char *xm = getenv("G3ATTN_DECODE_XMERGE");
        c->xmerge = xm ? atoi(xm) : 1;
        const char *nt = getenv("G3ATTN_DECODE_NT");
        c->nt_loads = nt ? atoi(nt) : 2;
        const char *ff = getenv("G3ATTN_FORWARD_FOLD");
        c->forward_fold = ff ? atoi(ff) & 3 : 1;
        if (c->min_rows < G3K_SPLIT_GRAIN) c->min_rows = G3K_SPLIT_GRAIN;
    }

    const size_t qs = (size_t)cfg->num_heads * D, ks = (size_t)cfg->num_kv_heads * D;
    c->in_bytes = (qs + 2 * ks) * sizeof(float) + 2 * D * sizeof(uint16_t);
    if (hipHostMalloc((void **)&c->h_in, c->in_bytes, 0) != hipSuccess) goto fail_rt;
    if (hipHostMalloc((void **)&c->h_out, qs * sizeof(float), 0) != hipSuccess) goto fail_rt;
    if (!alloc_dev((void **)&c->d_in, c->in_bytes, "staging")) goto fail;
    if (!alloc_dev((void **)&c->d_out, qs * sizeof(float), "staging")) goto fail;
    if (hipDeviceSynchronize() != hipSuccess) goto fail_rt;
    return c;

fail_rt:
    set_err("g3attn_create: %s", hipGetErrorString(hipGetLastError()));
fail:
    ctx_free(c);
    return NULL;
}

void g3attn_destroy(g3attn_ctx *c) {
    if (!c) return;
    hipSetDevice(c->device);
    hipStreamSynchronize(c->stream);
    ctx_free(c);
}

void g3attn_reset(g3attn_ctx *c) {
    if (!c) return;
    hipSetDevice(c->device);
    hipStreamSynchronize(c->stream);
}

void *g3attn_stream(g3attn_ctx *c) { return c ? (void *)c->stream : NULL; }

int g3attn_synchronize(g3attn_ctx *c) {
    if (!c) {
        set_err("g3attn_synchronize: null context");
        return G3_ERR_INVALID_ARG;
    }
    hipSetDevice(c->device);
    HIP_TRY(hipStreamSynchronize(c->stream), "g3attn_synchronize");
    return G3_OK;
}

static int grow_big(g3attn_ctx *c, size_t bytes) {
    if (bytes <= c->d_big_cap) return G3_OK;
    HIP_TRY(hipStreamSynchronize(c->stream), "grow staging");
    hipFree(c->d_big);
    c->d_big = NULL;
    c->d_big_cap = 0;
    if (!alloc_dev(&c->d_big, bytes, "batch staging")) return G3_ERR_OUT_OF_MEMORY;
    c->d_big_cap = bytes;
    return G3_OK;
}

/* ------------------------------------------------------------------ timing */

/* Folds the recorded pairs of one kind into its running sum. */
static int prof_fold(g3attn_ctx *c, int kind) {
    if (!c->prof.used[kind]) return G3_OK;
    HIP_TRY(hipStreamSynchronize(c->stream), "g3attn_profile");
    for (int i = 0; i < c->prof.used[kind]; i++) {
        float ms = 0.f;
        HIP_TRY(hipEventElapsedTime(&ms, c->prof.ev[kind][i][0], c->prof.ev[kind][i][1]),
                "g3attn_profile");
        c->prof.ms[kind] += ms;
    }
    c->prof.count[kind] += c->prof.used[kind];
    c->prof.used[kind] = 0;
    return G3_OK;
}

/* Event pair for the next launch of `kind` (both NULL when timing is off). */
static int prof_slot(g3attn_ctx *c, int kind, void **ev0, void **ev1) {
    *ev0 = *ev1 = NULL;
    if (!c->prof.on) return G3_OK;
    if (c->prof.used[kind] == G3_PROF_CAP) {
        int rc = prof_fold(c, kind);
        if (rc) return rc;
    }
    const int i = c->prof.used[kind]++;
    *ev0 = c->prof.ev[kind][i][0];
    *ev1 = c->prof.ev[kind][i][1];
    return G3_OK;
}

int g3attn_profile_enable(g3attn_ctx *c, int enable) {
    if (!c) {
        set_err("g3attn_profile_enable: null context");
        return G3_ERR_INVALID_ARG;
    }
    hipSetDevice(c->device);
    HIP_TRY(hipStreamSynchronize(c->stream), "g3attn_profile_enable");
    if (!enable) {
        prof_destroy(c);
        return G3_OK;
    }
    if (c->prof.on) return G3_OK;
    for (int k = 0; k < 2; k++) {
        c->prof.used[k] = c->prof.count[k] = 0;
        c->prof.ms[k] = 0.0;
        for (int i = 0; i < G3_PROF_CAP; i++)
            for (int j = 0; j < 2; j++) {
                hipError_t e = hipEventCreate(&c->prof.ev[k][i][j]);
                if (e != hipSuccess) {
                    prof_destroy(c);
                    return hip_fail(e, "g3attn_profile_enable");
                }
            }
    }
    c->prof.on = 1;
    return G3_OK;
}

int g3attn_profile_read(g3attn_ctx *c, int kind, double *total_ms, int *count) {
    if (!c || kind < 0 || kind > 1 || !total_ms || !count) {
        set_err("g3attn_profile_read: bad arguments");
        return G3_ERR_INVALID_ARG;
    }
    *total_ms = 0.0;
    *count = 0;
    if (!c->prof.on) return G3_OK;
    hipSetDevice(c->device);
    int rc = prof_fold(c, kind);
    if (rc) return rc;
    *total_ms = c->prof.ms[kind];
    *count = c->prof.count[kind];
    c->prof.ms[kind] = 0.0;
    c->prof.count[kind] = 0;
    return G3_OK;
}

int g3attn_last_splits(g3attn_ctx *c, int kind, int *splits) {
    if (!c || kind < 0 || kind > 2 || !splits) {
        set_err("g3attn_last_splits: bad arguments");
        return G3_ERR_INVALID_ARG;
    }
    *splits = c->last_splits[kind];
    return G3_OK;
}

/* ------------------------------------------------------------------ decode */

/* Split-K shape: target_wgs workgroups (default two per compute unit,
 * G3ATTN_DECODE_WGS overrides) spread over the KV heads, rows per split a
 * multiple of G3K_SPLIT_GRAIN and at least min_rows (G3ATTN_SPLIT_MIN_ROWS,
 * default one grain), at most G3K_MAX_SPLITS splits per head.  Mid-size
 * streams take half as many, longer splits, up to SPLIT_LONG_ROWS rows (four
 * 32-row steps): on MI355X at 4 KV heads, 4096 rows went from 14.4 to 13.0 us
 * per call and 8192 rows from 19.3 to 18.2 us, while 16384 rows and more
 * were faster at the full count (fewer partials for combine_kernel against
 * more serial steps per workgroup). */
#define SPLIT_LONG_ROWS 128
static void choose_splits(int n_stream, int n_kv, int target_wgs, int override_rows,
                          int min_rows, g3k_decode_args *a) {
    if (n_stream <= 0) {
        a->rows_per_split = G3K_SPLIT_GRAIN;
        a->n_splits = 1;
        return;
    }
    long per_head = (target_wgs > 0 ? target_wgs : 512) / n_kv;
    if (per_head < 1) per_head = 1;
    long r = override_rows > 0 ? override_rows : (n_stream + per_head - 1) / per_head;
    if (override_rows <= 0) {
        const long half = per_head / 2 > 0 ? per_head / 2 : 1;
        long longer = (n_stream + half - 1) / half;
        if (longer > SPLIT_LONG_ROWS) longer = SPLIT_LONG_ROWS;
        if (r < longer) r = longer;
        if (r < min_rows) r = min_rows;
    }
    r = (r + G3K_SPLIT_GRAIN - 1) / G3K_SPLIT_GRAIN * G3K_SPLIT_GRAIN;
    long s = (n_stream + r - 1) / r;
    if (s > G3K_MAX_SPLITS) {
        r = ((long)n_stream + G3K_MAX_SPLITS - 1) / G3K_MAX_SPLITS;
        r = (r + G3K_SPLIT_GRAIN - 1) / G3K_SPLIT_GRAIN * G3K_SPLIT_GRAIN;
        s = (n_stream + r - 1) / r;
    }
    a->rows_per_split = (int)r;
    a->n_splits = (int)s;
}

static int check_layer(const g3attn_ctx *c, int layer, const char *fn) {
    if (!c) {
        set_err("%s: null context", fn);
        return 0;
    }
    if (layer < 0 || layer >= c->cfg.num_layers) {
        set_err("%s: layer %d out of range [0, %d)", fn, layer, c->cfg.num_layers);
        return 0;
    }
    return 1;
}

static int check_rope(const g3attn_ctx *c, const char *fn) {
    if (!c->have_rope) {
        set_err("%s: RoPE tables not uploaded (g3attn_create without tables needs g3attn_upload_rope)", fn);
        return 0;
    }
    return 1;
}

int g3attn_upload_rope(g3attn_ctx *c, const float *rope_local, const float *rope_global, int max_context,
                       int head_dim) {
    if (!c || !rope_local || !rope_global) {
        set_err("g3attn_upload_rope: null context or table");
        return G3_ERR_INVALID_ARG;
    }
    if (max_context != c->max_context || head_dim != D) {
        set_err("g3attn_upload_rope: tables of %d positions x head_dim %d; the context needs %d x %d",
                max_context, head_dim, c->max_context, D);
        return G3_ERR_INVALID_ARG;
    }
    hipSetDevice(c->device);
    const size_t bytes = (size_t)max_context * D * sizeof(float);
    HIP_TRY(hipStreamSynchronize(c->stream), "g3attn_upload_rope");
    HIP_TRY(hipMemcpy(c->rope_local, rope_local, bytes, hipMemcpyHostToDevice), "g3attn_upload_rope");
    HIP_TRY(hipMemcpy(c->rope_global, rope_global, bytes, hipMemcpyHostToDevice), "g3attn_upload_rope");
    c->have_rope = 1;
    return G3_OK;
}

/* Query heads per workgroup of the one-launch decode, or 0 for the
 * two-launch form.  One launch serves 2..G3K_XM_MAX_SPLITS splits (local
 * layers: at most 32 splits of 32 rows) when the placement probe passed.
 * Its runs of query heads fill all 8 XCDs: the whole group per workgroup
 * where H_kv is a multiple of 8, else one query head per workgroup (H_q a
 * multiple of 8; each KV head's rows are then read once per query head, by
 * workgroups on different XCDs).  On MI355X at 8 query / 4 KV heads the one
 * query head per workgroup took configs[0] from 8.6 to 7.2-7.4 us per call;
 * whole groups on 4 XCDs (the other 4 idle) took 9.9 us.  Global layers
 * (G3ATTN_DECODE_XMERGE=2 admits them) would read their long caches twice. */
static int xm_heads(const g3attn_ctx *c, int n_splits, int is_global) {
    if (!c->xm_ok || !c->xmerge || (is_global && c->xmerge != 2) || n_splits < 2 ||
        n_splits > G3K_XM_MAX_SPLITS)
        return 0;
    const int n_kv = c->cfg.num_kv_heads, g = c->group;
    if (g <= 2 && n_kv % 8 == 0) return g;
    if ((n_kv * g) % 8 == 0) return 1;
    return 0;
}

/* One decode step; in_forward: called by the token forward (cache policy
 * below). */
static int decode_enqueue(g3attn_ctx *c, int layer, int pos, const float *q, const float *k,
                          const float *v, const uint16_t *q_norm, const uint16_t *k_norm,
                          float *attn_out, int in_forward) {
    if (!check_layer(c, layer, "g3attn_decode") || !check_rope(c, "g3attn_decode")) return G3_ERR_INVALID_ARG;
    if (!q || !k || !v || !attn_out || pos < 0) {
        set_err("g3attn_decode: null buffer or pos < 0");
        return G3_ERR_INVALID_ARG;
    }
    if (pos >= c->max_context) {
        set_err("g3attn_decode: pos %d >= max_context %d", pos, c->max_context);
        return G3_ERR_CONTEXT_OVERFLOW;
    }
    const int is_global = g3attn_is_global_layer(layer);
    const int W = c->cfg.sliding_window;
    /* gemma3_transformer.c:318-340: attention range and cache slot */
    const int seq_len = is_global ? pos + 1 : (pos < W ? pos + 1 : W);
    const int slot = is_global ? pos : pos % W;

    g3k_decode_args a;
    memset(&a, 0, sizeof a);
    a.q = q;
    a.k_new = k;
    a.v_new = v;
    a.q_norm = (q_norm && k_norm) ? q_norm : NULL;
    a.k_norm = (q_norm && k_norm) ? k_norm : NULL;
    a.rope_row = (is_global ? c->rope_global : c->rope_local) + (size_t)pos * D;
    a.eps = c->cfg.rmsnorm_eps;
    a.kc = c->kc[layer];
    a.vc = c->vc[layer];
    a.row_stride = D;
    a.head_stride = (long long)c->rows[layer] * D;
    a.n_stream = seq_len - 1;
    a.skip = slot;
    a.new_slot = slot;
    a.mask = NULL;
    a.qscale = (1.0f / sqrtf((float)D)) * LOG2E;
    choose_splits(a.n_stream, c->cfg.num_kv_heads, c->target_wgs, c->split_rows, c->min_rows, &a);
    c->last_splits[0] = a.n_splits;
    a.n_kv_heads = c->cfg.num_kv_heads;
    a.group = c->group;
    a.out = attn_out;
    a.ws_acc = c->ws_acc;
    a.ws_ml = c->ws_ml;
    a.xm_heads = xm_heads(c, a.n_splits, is_global);
    a.xm_count = c->d_xcount;
    c->last_splits[2] = a.xm_heads;
    /* Cache policy of the K/V loads (G3ATTN_DECODE_NT = 2).  A global layer
     * streams its whole cache once per token: non-temporal loads keep it
     * from evicting everything else.  Called for attention alone, a local
     * layer re-reads a window that changes by one row per token, so its rows
     * are loaded normally and the memory-side cache keeps them (29 + 5 stack
     * at 131071: 1089 -> 1079 us per token; configs[0] 9.4 -> 8.9 us).
     * Inside the token forward the 28-29 windows (235 MB) would instead push
     * out the norm rows the residual steps re-read every token (local
     * decode -0.4 us, residual step +0.5 us: 2.10 -> 2.12 ms per token), so
     * there every layer streams non-temporally.  The non-temporal loads
     * address a KV head's rows with 32-bit byte offsets: heads of 4 GiB or
     * more (max_context >= 4M) take plain loads. */
    a.nt_loads = (c->nt_loads == 1 || (c->nt_loads == 2 && (is_global || in_forward))) &&
                 (size_t)c->rows[layer] * D * sizeof(float) < ((size_t)1 << 32);
    hipSetDevice(c->device);
    int rc = prof_slot(c, 0, &a.ev0, &a.ev1);
    if (rc) return rc;
    rc = g3k_decode(&a, 1, c->stream);
    if (rc) return hip_fail((hipError_t)rc, "g3attn_decode launch");
    return G3_OK;
}

int g3attn_decode_device(g3attn_ctx *c, int layer, int pos, const float *q, const float *k,
                         const float *v, const uint16_t *q_norm, const uint16_t *k_norm,
                         float *attn_out) {
    return decode_enqueue(c, layer, pos, q, k, v, q_norm, k_norm, attn_out, 0);
}

int g3attn_decode(g3attn_ctx *c, int layer, int pos, const float *q, const float *k,
                  const float *v, const uint16_t *q_norm, const uint16_t *k_norm, float *attn_out) {
    if (!check_layer(c, layer, "g3attn_decode")) return G3_ERR_INVALID_ARG;
    if (!q || !k || !v || !attn_out) {
        set_err("g3attn_decode: null buffer");
        return G3_ERR_INVALID_ARG;
    }
    const size_t qs = (size_t)c->cfg.num_heads * D, ks = (size_t)c->cfg.num_kv_heads * D;
    hipSetDevice(c->device);
    HIP_TRY(hipStreamSynchronize(c->stream), "g3attn_decode");
    unsigned char *h = c->h_in;
    memcpy(h, q, qs * sizeof(float));
    memcpy(h + qs * 4, k, ks * sizeof(float));
    memcpy(h + (qs + ks) * 4, v, ks * sizeof(float));
    const size_t nb = (qs + 2 * ks) * 4;
    const int norm = q_norm && k_norm;
    if (norm) {
        memcpy(h + nb, q_norm, D * sizeof(uint16_t));
        memcpy(h + nb + D * 2, k_norm, D * sizeof(uint16_t));
    }
    HIP_TRY(hipMemcpyAsync(c->d_in, h, norm ? c->in_bytes : nb, hipMemcpyHostToDevice, c->stream),
            "g3attn_decode upload");
    const float *dq = (const float *)c->d_in;
    int rc = g3attn_decode_device(c, layer, pos, dq, dq + qs, dq + qs + ks,
                                  norm ? (const uint16_t *)(c->d_in + nb) : NULL,
                                  norm ? (const uint16_t *)(c->d_in + nb + D * 2) : NULL, c->d_out);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(c->h_out, c->d_out, qs * sizeof(float), hipMemcpyDeviceToHost, c->stream),
            "g3attn_decode download");
    HIP_TRY(hipStreamSynchronize(c->stream), "g3attn_decode");
    memcpy(attn_out, c->h_out, qs * sizeof(float));
    return G3_OK;
}

/* ------------------------------------------------------------------ KV cache */

int g3attn_kv_append_device(g3attn_ctx *c, int layer, int start_pos, int n, const float *K,
                            const float *V, const uint16_t *k_norm) {
    if (!check_layer(c, layer, "g3attn_kv_append") || !check_rope(c, "g3attn_kv_append")) return G3_ERR_INVALID_ARG;
    if (n < 0 || start_pos < 0 || (n > 0 && (!K || !V))) {
        set_err("g3attn_kv_append: bad arguments");
        return G3_ERR_INVALID_ARG;
    }
    if ((long)start_pos + n > c->max_context) {
        set_err("g3attn_kv_append: positions up to %ld exceed max_context %d", (long)start_pos + n - 1,
                c->max_context);
        return G3_ERR_CONTEXT_OVERFLOW;
    }
    if (n == 0) return G3_OK;
    const int is_global = g3attn_is_global_layer(layer);
    const int W = c->cfg.sliding_window;
    const size_t ks = (size_t)c->cfg.num_kv_heads * D;
    /* On a ring only the last W tokens survive; skip the rest so no two
     * tokens of one launch race for a slot. */
    int skip = (!is_global && n > W) ? n - W : 0;
    g3k_rope_write_args a;
    memset(&a, 0, sizeof a);
    a.K = K + (size_t)skip * ks;
    a.V = V + (size_t)skip * ks;
    a.q_norm = k_norm;
    a.k_norm = k_norm;
    a.rope = is_global ? c->rope_global : c->rope_local;
    a.eps = c->cfg.rmsnorm_eps;
    a.n = n - skip;
    a.start_pos = start_pos + skip;
    a.n_heads = c->cfg.num_heads;
    a.n_kv_heads = c->cfg.num_kv_heads;
    a.k_dst = c->kc[layer];
    a.v_dst = c->vc[layer];
    a.dst_head_stride = (long long)c->rows[layer] * D;
    a.ring = is_global ? 0 : W;
    a.dst_pos0 = 0;
    hipSetDevice(c->device);
    const int rc = g3k_rope_write(&a, c->stream);
    if (rc) return hip_fail((hipError_t)rc, "g3attn_kv_append launch");
    return G3_OK;
}

int g3attn_kv_append(g3attn_ctx *c, int layer, int start_pos, int n, const float *K,
                     const float *V, const uint16_t *k_norm) {
    if (!check_layer(c, layer, "g3attn_kv_append") || !check_rope(c, "g3attn_kv_append")) return G3_ERR_INVALID_ARG;
    if (n <= 0) return n == 0 ? G3_OK : G3_ERR_INVALID_ARG;
    if (!K || !V) {
        set_err("g3attn_kv_append: null buffer");
        return G3_ERR_INVALID_ARG;
    }
    const size_t kb = (size_t)n * c->cfg.num_kv_heads * D * sizeof(float);
    hipSetDevice(c->device);
    int rc = grow_big(c, 2 * kb + 2 * D);
    if (rc) return rc;
    unsigned char *b = (unsigned char *)c->d_big;
    HIP_TRY(hipMemcpyAsync(b, K, kb, hipMemcpyHostToDevice, c->stream), "kv_append upload");
    HIP_TRY(hipMemcpyAsync(b + kb, V, kb, hipMemcpyHostToDevice, c->stream), "kv_append upload");
    if (k_norm)
        HIP_TRY(hipMemcpyAsync(b + 2 * kb, k_norm, D * 2, hipMemcpyHostToDevice, c->stream),
                "kv_append upload");
    rc = g3attn_kv_append_device(c, layer, start_pos, n, (const float *)b, (const float *)(b + kb),
                                 k_norm ? (const uint16_t *)(b + 2 * kb) : NULL);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream), "g3attn_kv_append");
    return G3_OK;
}

/* Host rows in the reference layout [n][H_kv][D] <-> cache slots
 * slot..slot+n-1: one 1-D copy per matrix through the staging buffer, and
 * one kernel between the staging and the head-major cache (instead of a
 * strided 2-D copy per head and matrix). */
static int kv_copy(g3attn_ctx *c, int layer, int slot, int n, float *k_rows, float *v_rows,
                   int to_device, const char *fn) {
    if (!check_layer(c, layer, fn)) return G3_ERR_INVALID_ARG;
    if (slot < 0 || n < 0 || (long)slot + n > c->rows[layer] || (n > 0 && (!k_rows || !v_rows))) {
        set_err("%s: rows [%d, %ld) outside the layer's %d cache rows", fn, slot, (long)slot + n,
                c->rows[layer]);
        return G3_ERR_INVALID_ARG;
    }
    if (n == 0) return G3_OK;
    const int H = c->cfg.num_kv_heads;
    const size_t hs = (size_t)c->rows[layer] * D;
    const size_t mb = (size_t)n * H * D * sizeof(float);
    hipSetDevice(c->device);
    int rc = grow_big(c, 2 * mb);
    if (rc) return rc;
    float *sk = (float *)c->d_big, *sv = (float *)((unsigned char *)c->d_big + mb);
    if (to_device) {
        HIP_TRY(hipMemcpyAsync(sk, k_rows, mb, hipMemcpyHostToDevice, c->stream), fn);
        HIP_TRY(hipMemcpyAsync(sv, v_rows, mb, hipMemcpyHostToDevice, c->stream), fn);
    }
    rc = g3k_kv_scatter(c->kc[layer], c->vc[layer], sk, sv, n, H, (long long)hs, slot, !to_device, c->stream);
    if (rc) return hip_fail((hipError_t)rc, fn);
    if (!to_device) {
        HIP_TRY(hipMemcpyAsync(k_rows, sk, mb, hipMemcpyDeviceToHost, c->stream), fn);
        HIP_TRY(hipMemcpyAsync(v_rows, sv, mb, hipMemcpyDeviceToHost, c->stream), fn);
    }
    HIP_TRY(hipStreamSynchronize(c->stream), fn);
    return G3_OK;
}

int g3attn_kv_write(g3attn_ctx *c, int layer, int slot, int n, const float *k_rows,
                    const float *v_rows) {
    return kv_copy(c, layer, slot, n, (float *)k_rows, (float *)v_rows, 1, "g3attn_kv_write");
}

int g3attn_kv_read(g3attn_ctx *c, int layer, int slot, int n, float *k_rows, float *v_rows) {
    return kv_copy(c, layer, slot, n, k_rows, v_rows, 0, "g3attn_kv_read");
}

/* ------------------------------------------------------------------ prefill */

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

/* Grow-on-demand prefill workspace: kq [H_kv][ldk][2][D] fp16 (hi | lo
 * rows) and vt / vt_lo [H_kv][D][ldk] bf16 (the queries are normed and
 * rotated inside the attention kernel, straight from the caller's Q). */
static int grow_pf(g3attn_ctx *c, size_t bytes) {
    if (bytes <= c->d_pf_cap) return G3_OK;
    HIP_TRY(hipStreamSynchronize(c->stream), "grow prefill workspace");
    hipFree(c->d_pf);
    c->d_pf = NULL;
    c->d_pf_cap = 0;
    if (!alloc_dev(&c->d_pf, bytes, "prefill workspace")) return G3_ERR_OUT_OF_MEMORY;
    c->d_pf_cap = bytes;
    return G3_OK;
}

/* Key splits S (1, 2 or 4) of a prefill call.  A workgroup walks the key
 * tiles of one query block (pb tokens) of one KV head; with S > 1 each
 * block's tiles are dealt to S workgroups, and the last of them to finish
 * merges their parts (inside the kernel).  S minimises a makespan model
 * measured on MI355X:
 * - a tile step costs ~2.2 us, and a workgroup ~12 us more: its prologue
 *   (queries, RoPE rows and the first K / V tiles, read while every CU does
 *   the same) and its output stores;
 * - one workgroup runs per CU (its LDS), and the longest block's part sets a
 *   floor (a 4096-token global prefill unsplit: 128 tiles on one CU while
 *   the average is 65);
 * - the parts and the merge move about (S + 1) n H_q 256 floats at ~5 TB/s.
 * Each split keeps at least 4 tiles. */
static int prefill_splits(int n, int hist, int nk, int window, int pb, int n_kv, int n_q, int n_cu) {
    const int nb = (n + pb - 1) / pb;
    long long total = 0, longest = 0;
    for (int qb = 0; qb < nb; qb++) {
        const long long first = (long long)hist + (long long)qb * pb;
        const long long last = first + pb - 1 < nk - 1 ? first + pb - 1 : nk - 1;
        const long long k0 = first - window + 1 > 0 ? first - window + 1 : 0;
        const long long t = last / 32 - k0 / 32 + 1;
        total += t;
        if (t > longest) longest = t;
    }
    total *= n_kv;
    const double step_us = 2.2, wg_us = 12.0, merge_bytes_per_us = 5.0e6;
    int best = 1;
    double best_us = 0.0;
    for (int S = 1; S <= 4; S *= 2) {
        if (S > 1 && longest < 4LL * S) break;
        const double wgs = (double)nb * n_kv * S;
        const double floor_us = step_us * (double)((longest + S - 1) / S) + wg_us;
        const double spread_us = (step_us * (double)total + wg_us * wgs) / (double)(n_cu > 0 ? n_cu : 256);
        double t = floor_us > spread_us ? floor_us : spread_us;
        if (S > 1) t += 3.0 + (double)(S + 1) * n * n_q * 256 * 4 / merge_bytes_per_us;
        if (S == 1 || t < best_us) {
            best = S;
            best_us = t;
        }
    }
    return best;
}

/* x8: the score policy, 1 = fp16 hi + fp8 cross terms, 0 = three fp16
 * passes (see prefill.hip). */
static int prefill_attention(g3attn_ctx *c, int layer, int start_pos, int n, const float *Q, const float *K,
                             const float *V, const uint16_t *q_norm, const uint16_t *k_norm, float *attn_out,
                             int x8);

int g3attn_prefill_device(g3attn_ctx *c, int layer, int start_pos, int n, const float *Q,
                          const float *K, const float *V, const uint16_t *q_norm,
                          const uint16_t *k_norm, float *attn_out) {
    return prefill_attention(c, layer, start_pos, n, Q, K, V, q_norm, k_norm, attn_out, c ? c->prefill_x8 : 0);
}

static int prefill_attention(g3attn_ctx *c, int layer, int start_pos, int n, const float *Q, const float *K,
                             const float *V, const uint16_t *q_norm, const uint16_t *k_norm, float *attn_out,
                             int x8) {
    if (!check_layer(c, layer, "g3attn_prefill") || !check_rope(c, "g3attn_prefill")) return G3_ERR_INVALID_ARG;
    if (n < 0 || start_pos < 0 || (n > 0 && (!Q || !K || !V || !attn_out))) {
        set_err("g3attn_prefill: null buffer or negative start_pos / n");
        return G3_ERR_INVALID_ARG;
    }
    if ((long)start_pos + n > c->max_context) {
        set_err("g3attn_prefill: positions up to %ld exceed max_context %d",
                (long)start_pos + n - 1, c->max_context);
        return G3_ERR_CONTEXT_OVERFLOW;
    }
    if (n == 0) return G3_OK;
    const int is_global = g3attn_is_global_layer(layer);
    const int W = c->cfg.sliding_window;
    const int Hq = c->cfg.num_heads, Hkv = c->cfg.num_kv_heads;
    /* Keys the batch can see: positions [kstart, start_pos + n), staged in
     * position order (key index kk = pos - kstart); the first hist of them
     * come from the cache, written by earlier calls. */
    const int kstart = is_global ? 0 : (start_pos - W + 1 > 0 ? start_pos - W + 1 : 0);
    const int hist = start_pos - kstart, nk = hist + n;
    const long long ldk = ((long long)nk + 63) / 64 * 64;
    const size_t v_bytes = align256((size_t)Hkv * ldk * D * sizeof(uint16_t));
    const int pb = 16 * ((c->prefill_qpw == 32 ? 2 : 1)) * ((8 / (c->prefill_qpw == 32 ? 2 : 1)) / c->group);
    const int S = c->prefill_ksplit ? c->prefill_ksplit
                                    : prefill_splits(n, hist, nk, is_global ? INT_MAX / 2 : W, pb, Hkv, Hq, c->n_cu);
    const size_t po_bytes = S > 1 ? align256((size_t)S * n * Hq * D * sizeof(float)) : 0;
    const size_t pml_bytes = S > 1 ? align256((size_t)S * n * Hq * 2 * sizeof(float)) : 0;
    /* the fp8 cross policy's key-scale bytes, one per staged key row */
    const size_t ks_bytes = x8 ? align256((size_t)Hkv * ldk) : 0;
    hipSetDevice(c->device);
    int rc = grow_pf(c, 4 * v_bytes + ks_bytes + po_bytes + pml_bytes);
    if (rc) return rc;
    unsigned char *ws = (unsigned char *)c->d_pf;
    uint16_t *kq = (uint16_t *)ws;
    uint16_t *vt = (uint16_t *)(ws + 2 * v_bytes);
    uint16_t *vt_lo = (uint16_t *)(ws + 3 * v_bytes);
    uint8_t *kscale = x8 ? ws + 4 * v_bytes : NULL;
    float *part_o = S > 1 ? (float *)(ws + 4 * v_bytes + ks_bytes) : NULL;
    float *part_ml = S > 1 ? (float *)(ws + 4 * v_bytes + ks_bytes + po_bytes) : NULL;
    /* a fresh epoch per call: a flag left by an earlier call never matches */
    c->pf_epoch = c->pf_epoch >= INT_MAX - 1 ? 1 : c->pf_epoch + 1;
    const int norm = q_norm && k_norm;
    const float *rope = is_global ? c->rope_global : c->rope_local;
    const long long head_stride = (long long)c->rows[layer] * D;

    /* 1. history keys, read from the cache before this batch's ring writes */
    if (hist > 0) {
        g3k_stage_args sa;
        memset(&sa, 0, sizeof sa);
        sa.k_src = c->kc[layer];
        sa.v_src = c->vc[layer];
        sa.head_stride = head_stride;
        sa.row_stride = D;
        sa.ring = is_global ? 0 : W;
        sa.row_pos0 = 0;
        sa.kstart = kstart;
        sa.kk0 = 0;
        sa.cnt = hist;
        sa.nk = nk;
        sa.n_kv_heads = Hkv;
        sa.kq = kq;
        sa.kscale = kscale;
        sa.vt = vt;
        sa.vt_lo = vt_lo;
        sa.ldk = ldk;
        sa.v_lo_flag = c->d_vflag;
        sa.epoch = c->pf_epoch;
        rc = g3k_stage(&sa, c->stream);
        if (rc) return hip_fail((hipError_t)rc, "g3attn_prefill stage");
    }
    /* 2. K-norm + RoPE of the batch, cache_kv, fp16 split keys
     *    (the key half of gemma3_transformer.c:650-671 for every token) */
    g3k_rope_write_args ra;
    memset(&ra, 0, sizeof ra);
    ra.Q = NULL;
    ra.K = K;
    ra.V = V;
    ra.q_norm = norm ? q_norm : NULL;
    ra.k_norm = norm ? k_norm : NULL;
    ra.rope = rope;
    ra.eps = c->cfg.rmsnorm_eps;
    ra.n = n;
    ra.start_pos = start_pos;
    ra.n_heads = Hq;
    ra.n_kv_heads = Hkv;
    ra.q_out = NULL;
    ra.k_dst = c->kc[layer];
    ra.v_dst = c->vc[layer];
    ra.dst_head_stride = head_stride;
    ra.ring = is_global ? 0 : W;
    ra.dst_pos0 = 0;
    ra.kv_skip = (!is_global && n > W) ? n - W : 0;
    ra.kq = kq;
    ra.kscale = kscale;
    ra.ldk = ldk;
    ra.row0 = hist;
    /* 3. the batch's values as bf16 hi / lo V^T, and zeroed padding up to
     *    ldk: read from the batch's own V, so it runs in step 2's launch */
    {
        g3k_stage_args sa;
        memset(&sa, 0, sizeof sa);
        sa.k_src = NULL;
        sa.v_src = V;
        sa.head_stride = D;
        sa.row_stride = (long long)Hkv * D;
        sa.ring = 0;
        sa.row_pos0 = start_pos;
        sa.kstart = kstart;
        sa.kk0 = hist;
        sa.cnt = (int)(ldk - hist);
        sa.nk = nk;
        sa.n_kv_heads = Hkv;
        sa.kq = kq;
        sa.kscale = kscale;
        sa.vt = vt;
        sa.vt_lo = vt_lo;
        sa.ldk = ldk;
        sa.v_lo_flag = c->d_vflag;
        sa.epoch = c->pf_epoch;
        rc = g3k_rope_write_stage(&ra, &sa, c->stream);
        if (rc) return hip_fail((hipError_t)rc, "g3attn_prefill rope / stage");
    }
    /* 4. Q-norm + RoPE and attention (gemma3_transformer.c:650-667 for the
     *    queries, gemma3_gqa for every token, :673-691) */
    g3k_prefill_args pa;
    memset(&pa, 0, sizeof pa);
    pa.q = Q;
    pa.q_norm = norm ? q_norm : NULL;
    pa.rope = rope;
    pa.eps = c->cfg.rmsnorm_eps;
    pa.start_pos = start_pos;
    pa.kq = kq;
    pa.kscale = kscale;
    pa.vt = vt;
    pa.vt_lo = vt_lo;
    pa.v_lo_flag = c->d_vflag;
    pa.epoch = c->pf_epoch;
    pa.out = attn_out;
    pa.ldk = ldk;
    pa.n = n;
    pa.hist = hist;
    pa.nk = nk;
    pa.window = is_global ? INT_MAX / 2 : W;
    pa.n_kv_heads = Hkv;
    pa.group = c->group;
    pa.qscale = (1.0f / sqrtf((float)D)) * LOG2E;
    pa.queries_per_wave = c->prefill_qpw;
    pa.schedule = c->prefill_sched;
    pa.ksplit = S;
    c->last_splits[1] = S;
    pa.part_o = part_o;
    pa.part_ml = part_ml;
    pa.arrive = c->d_arrive;
    rc = prof_slot(c, 1, &pa.ev0, &pa.ev1);
    if (rc) return rc;
    rc = g3k_prefill(&pa, c->stream);
    if (rc) return hip_fail((hipError_t)rc, "g3attn_prefill launch");
    return G3_OK;
}

int g3attn_prefill(g3attn_ctx *c, int layer, int start_pos, int n, const float *Q,
                   const float *K, const float *V, const uint16_t *q_norm,
                   const uint16_t *k_norm, float *attn_out) {
    if (!check_layer(c, layer, "g3attn_prefill") || !check_rope(c, "g3attn_prefill")) return G3_ERR_INVALID_ARG;
    if (n < 0 || (n > 0 && (!Q || !K || !V || !attn_out))) {
        set_err("g3attn_prefill: null buffer or n < 0");
        return G3_ERR_INVALID_ARG;
    }
    if (start_pos < 0) {
        set_err("g3attn_prefill: start_pos < 0");
        return G3_ERR_INVALID_ARG;
    }
    if ((long)start_pos + n > c->max_context) {
        set_err("g3attn_prefill: positions up to %ld exceed max_context %d",
                (long)start_pos + n - 1, c->max_context);
        return G3_ERR_CONTEXT_OVERFLOW;
    }
    if (n == 0) return G3_OK;
    const size_t qb = align256((size_t)n * c->cfg.num_heads * D * sizeof(float));
    const size_t kb = align256((size_t)n * c->cfg.num_kv_heads * D * sizeof(float));
    const int norm = q_norm && k_norm;
    hipSetDevice(c->device);
    int rc = grow_big(c, 2 * qb + 2 * kb + 2 * align256(D * sizeof(uint16_t)));
    if (rc) return rc;
    unsigned char *b = (unsigned char *)c->d_big;
    float *dQ = (float *)b, *dO = (float *)(b + qb);
    float *dK = (float *)(b + 2 * qb), *dV = (float *)(b + 2 * qb + kb);
    uint16_t *dqn = (uint16_t *)(b + 2 * qb + 2 * kb);
    uint16_t *dkn = dqn + D;
    const size_t qs = (size_t)n * c->cfg.num_heads * D * sizeof(float);
    const size_t ks = (size_t)n * c->cfg.num_kv_heads * D * sizeof(float);
    HIP_TRY(hipMemcpyAsync(dQ, Q, qs, hipMemcpyHostToDevice, c->stream), "prefill upload");
    HIP_TRY(hipMemcpyAsync(dK, K, ks, hipMemcpyHostToDevice, c->stream), "prefill upload");
    HIP_TRY(hipMemcpyAsync(dV, V, ks, hipMemcpyHostToDevice, c->stream), "prefill upload");
    if (norm) {
        HIP_TRY(hipMemcpyAsync(dqn, q_norm, D * 2, hipMemcpyHostToDevice, c->stream), "prefill upload");
        HIP_TRY(hipMemcpyAsync(dkn, k_norm, D * 2, hipMemcpyHostToDevice, c->stream), "prefill upload");
    }
    rc = g3attn_prefill_device(c, layer, start_pos, n, dQ, dK, dV, norm ? dqn : NULL,
                               norm ? dkn : NULL, dO);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(attn_out, dO, qs, hipMemcpyDeviceToHost, c->stream), "prefill download");
    HIP_TRY(hipStreamSynchronize(c->stream), "g3attn_prefill");
    return G3_OK;
}

/* ------------------------------------------------------------------ GEMV */

static int grow_la(g3attn_ctx *c, size_t bytes) {
    if (bytes <= c->d_la_cap) return G3_OK;
    HIP_TRY(hipStreamSynchronize(c->stream), "grow layer scratch");
    hipFree(c->d_la);
    c->d_la = NULL;
    c->d_la_cap = 0;
    if (!alloc_dev((void **)&c->d_la, bytes, "layer scratch")) return G3_ERR_OUT_OF_MEMORY;
    c->d_la_cap = bytes;
    return G3_OK;
}

static int matvec_check(int M, int K, const void *y, const void *A, const void *x, const char *who) {
    if (!y || !A || !x || M < 1 || K < 1) {
        set_err("%s: null buffer or M / K < 1", who);
        return G3_ERR_INVALID_ARG;
    }
    return G3_OK;
}

int g3attn_matvec_bf16_device(g3attn_ctx *c, float *y, const uint16_t *A, const float *x, int M, int K) {
    if (!c) {
        set_err("g3attn_matvec_bf16_device: null context");
        return G3_ERR_INVALID_ARG;
    }
    int rc = matvec_check(M, K, y, A, x, "g3attn_matvec_bf16_device");
    if (rc) return rc;
    hipSetDevice(c->device);
    g3k_matvec_args a;
    memset(&a, 0, sizeof a);
    a.x = x;
    a.K = K;
    a.n_mat = 1;
    a.A[0] = A;
    a.y[0] = y;
    a.M[0] = M;
    rc = g3k_matvec(&a, c->stream);
    if (rc) return hip_fail((hipError_t)rc, "g3attn_matvec_bf16_device launch");
    return G3_OK;
}

int g3attn_qkv_proj_device(g3attn_ctx *c, const float *x, const uint16_t *wq, const uint16_t *wk,
                           const uint16_t *wv, float *q, float *k, float *v) {
    if (!c || !x || !wq || !wk || !wv || !q || !k || !v) {
        set_err("g3attn_qkv_proj_device: null context or buffer");
        return G3_ERR_INVALID_ARG;
    }
    const int K = c->cfg.hidden_size;
    int rc = matvec_check(1, K, q, wq, x, "g3attn_qkv_proj_device");
    if (rc) return rc;
    hipSetDevice(c->device);
    g3k_matvec_args a;
    memset(&a, 0, sizeof a);
    a.x = x;
    a.K = K;
    a.n_mat = 3;
    a.A[0] = wq;
    a.y[0] = q;
    a.M[0] = c->cfg.num_heads * D;
    a.A[1] = wk;
    a.y[1] = k;
    a.M[1] = c->cfg.num_kv_heads * D;
    a.A[2] = wv;
    a.y[2] = v;
    a.M[2] = c->cfg.num_kv_heads * D;
    rc = g3k_matvec(&a, c->stream);
    if (rc) return hip_fail((hipError_t)rc, "g3attn_qkv_proj_device launch");
    return G3_OK;
}

/* The whole of layer_attention for one token: Q/K/V GEMVs, the attention
 * section (QK-norm, RoPE, cache write, GQA) and the o_proj GEMV. */
int g3attn_layer_attention_device(g3attn_ctx *c, int layer, int pos, const float *x,
                                  const uint16_t *wq, const uint16_t *wk, const uint16_t *wv,
                                  const uint16_t *wo, const uint16_t *q_norm, const uint16_t *k_norm,
                                  float *out) {
    if (!c || !out) {
        set_err("g3attn_layer_attention_device: null context or buffer");
        return G3_ERR_INVALID_ARG;
    }
    const int qs = c->cfg.num_heads * D, ks = c->cfg.num_kv_heads * D;
    int rc = grow_la(c, (size_t)(2 * qs + 2 * ks) * sizeof(float));
    if (rc) return rc;
    float *q = c->d_la, *k = q + qs, *v = k + ks, *attn = v + ks;
    rc = g3attn_qkv_proj_device(c, x, wq, wk, wv, q, k, v);
    if (rc) return rc;
    rc = g3attn_decode_device(c, layer, pos, q, k, v, q_norm, k_norm, attn);
    if (rc) return rc;
    return g3attn_matvec_bf16_device(c, out, wo, attn, c->cfg.hidden_size, qs);
}

/* ------------------------------------------------------------------ token forward */

static int grow_buf(g3attn_ctx *c, float **p, size_t *cap, size_t bytes, const char *what) {
    if (bytes <= *cap) return G3_OK;
    HIP_TRY(hipStreamSynchronize(c->stream), what);
    hipFree(*p);
    *p = NULL;
    *cap = 0;
    if (!alloc_dev((void **)p, bytes, what)) return G3_ERR_OUT_OF_MEMORY;
    *cap = bytes;
    return G3_OK;
}

static int layer_step(g3attn_ctx *c, int op, float *x, float *t, float *y, const uint16_t *w_post,
                      const uint16_t *w_next, const uint16_t *embed, int token) {
    g3k_layer_args a;
    memset(&a, 0, sizeof a);
    a.op = op;
    a.n = c->cfg.hidden_size;
    a.token = token;
    a.eps = c->cfg.rmsnorm_eps;
    a.embed = embed;
    a.w_post = w_post;
    a.w_next = w_next;
    a.x = x;
    a.t = t;
    a.y = y;
    const int rc = g3k_layer_step(&a, c->stream);
    if (rc) return hip_fail((hipError_t)rc, "g3attn_forward_device step");
    return G3_OK;
}

static int gemv(g3attn_ctx *c, float *y, const uint16_t *A, const float *x, int M, int K) {
    g3k_matvec_args a;
    memset(&a, 0, sizeof a);
    a.x = x;
    a.K = K;
    a.n_mat = 1;
    a.A[0] = A;
    a.y[0] = y;
    a.M[0] = M;
    const int rc = g3k_matvec(&a, c->stream);
    if (rc) return hip_fail((hipError_t)rc, "g3attn_forward_device GEMV");
    return G3_OK;
}

/* Checks shared by the token forward entry points. */
static int forward_check(g3attn_ctx *c, const g3attn_weights *w, int token_id, int pos, const char *who) {
    const g3attn_config *cfg = &c->cfg;
    const int hid = cfg->hidden_size, inter = cfg->intermediate_size, L = cfg->num_layers;
    if (token_id < 0 || token_id >= cfg->vocab_size || L < 1 || L > G3ATTN_MAX_LAYERS || hid < 1 ||
        hid > G3K_LAYER_MAX_HIDDEN || inter < 1) {
        set_err("%s: token %d / vocab %d, layers %d, hidden %d, intermediate %d out of range", who, token_id,
                cfg->vocab_size, L, hid, inter);
        return G3_ERR_INVALID_ARG;
    }
    for (int l = 0; l < L; l++) {
        const g3attn_layer_weights *lw = &w->layers[l];
        if (!lw->input_layernorm || !lw->q_proj || !lw->k_proj || !lw->v_proj || !lw->o_proj ||
            !lw->gate_proj || !lw->up_proj || !lw->down_proj) {
            set_err("%s: layer %d has a null projection or input norm", who, l);
            return G3_ERR_INVALID_ARG;
        }
    }
    if (pos < 0 || pos >= c->max_context) {
        set_err("%s: pos %d outside [0, %d)", who, pos, c->max_context);
        return pos < 0 ? G3_ERR_INVALID_ARG : G3_ERR_CONTEXT_OVERFLOW;
    }
    return G3_OK;
}

/* The activation buffers of the token forward. */
static int forward_buffers(g3attn_ctx *c) {
    const g3attn_config *cfg = &c->cfg;
    const size_t hb = align256((size_t)cfg->hidden_size * 4);
    int rc = grow_buf(c, &c->d_fw, &c->d_fw_cap, 5 * hb + align256((size_t)cfg->intermediate_size * 4),
                      "forward activations");
    if (rc) return rc;
    const int qs = cfg->num_heads * D, ks = cfg->num_kv_heads * D;
    return grow_buf(c, &c->d_la, &c->d_la_cap, (size_t)(2 * qs + 2 * ks) * sizeof(float), "layer scratch");
}

/* A GEMV whose x is formed by the residual prologue (g3k_matvec_args.pre_*):
 * s = *x + rmsnorm(t, w_post) goes to *x_alt, and the two residual buffers
 * swap. */
static void set_pre(g3k_matvec_args *a, const g3attn_config *cfg, float **x, float **x_alt, const float *t,
                    const uint16_t *w_post, const uint16_t *w_next) {
    a->pre_t = t;
    a->pre_r = *x;
    a->pre_r_out = *x_alt;
    a->pre_w_post = w_post;
    a->pre_w_next = w_next;
    a->pre_eps = cfg->rmsnorm_eps;
    float *tmp = *x;
    *x = *x_alt;
    *x_alt = tmp;
}

/* Enqueue one token of gemma3_transformer_forward (:396-512).
 *
 * The residual step between two GEMVs (post-norm, residual add, the next
 * pre-norm) is folded into the prologue of the GEMV that consumes it where
 * c->forward_fold allows and the hidden size fits the prologue: the Q/K/V
 * launch of the next layer, and the gate/up launch.  The residual stream
 * then alternates between two buffers (x, x_alt), since every workgroup of
 * the folded launch reads the old residual while workgroup 0 writes the new
 * one.  Otherwise the one-workgroup residual_kernel runs in between. */
static int forward_enqueue(g3attn_ctx *c, const g3attn_weights *w, int token_id, int pos, float *logits,
                           int compute_logits, float *hidden_out) {
    const g3attn_config *cfg = &c->cfg;
    const int hid = cfg->hidden_size, inter = cfg->intermediate_size, L = cfg->num_layers;
    const size_t hb = align256((size_t)hid * 4);
    const int qs = cfg->num_heads * D, ks = cfg->num_kv_heads * D;
    unsigned char *b = (unsigned char *)c->d_fw;
    float *x = (float *)b, *xn = (float *)(b + hb), *proj = (float *)(b + 2 * hb);
    float *mlp = (float *)(b + 3 * hb), *x_alt = (float *)(b + 4 * hb), *h = (float *)(b + 5 * hb);
    float *q = c->d_la, *k = q + qs, *v = k + ks, *attn = v + ks;
    const int can_fold = hid <= G3K_MATVEC_PRE_MAX && hid % 4 == 0;
    const int fold_qkv = can_fold && (c->forward_fold & 1), fold_mlp = can_fold && (c->forward_fold & 2);
    int rc;
    /* the prologue reads gain rows as 8-byte words: a step whose gains sit at
     * other offsets (weights mapped from a file as is) runs unfolded */
#define AL8(p) (((uintptr_t)(p) & 7) == 0)

    /* embedding * sqrt(hidden) (:415-422), then layer 0's input norm (:444-446) */
    if ((rc = layer_step(c, G3K_OP_EMBED, x, NULL, NULL, NULL, NULL, w->embed_tokens, token_id))) return rc;
    if ((rc = layer_step(c, G3K_OP_NORM, x, NULL, xn, NULL, w->layers[0].input_layernorm, NULL, 0))) return rc;
    for (int l = 0; l < L; l++) {
        const g3attn_layer_weights *lw = &w->layers[l];
        /* layer_attention (:449-460); with fold_qkv (l > 0) the previous
         * layer's post-feedforward norm, residual add and this layer's input
         * norm (:490-496, 444-446) run in the Q/K/V launch's prologue */
        if (fold_qkv && l > 0 && AL8(w->layers[l - 1].post_feedforward_layernorm) &&
            AL8(lw->input_layernorm)) {
            g3k_matvec_args a;
            memset(&a, 0, sizeof a);
            a.K = hid;
            a.n_mat = 3;
            a.A[0] = lw->q_proj;
            a.y[0] = q;
            a.M[0] = qs;
            a.A[1] = lw->k_proj;
            a.y[1] = k;
            a.M[1] = ks;
            a.A[2] = lw->v_proj;
            a.y[2] = v;
            a.M[2] = ks;
            set_pre(&a, cfg, &x, &x_alt, mlp, w->layers[l - 1].post_feedforward_layernorm, lw->input_layernorm);
            if ((rc = g3k_matvec(&a, c->stream))) return hip_fail((hipError_t)rc, "g3attn_forward_device Q/K/V");
        } else if ((rc = g3attn_qkv_proj_device(c, xn, lw->q_proj, lw->k_proj, lw->v_proj, q, k, v))) {
            return rc;
        }
        if ((rc = decode_enqueue(c, l, pos, q, k, v, lw->q_norm, lw->k_norm, attn, 1))) return rc;
        if ((rc = gemv(c, proj, lw->o_proj, attn, hid, qs))) return rc;
        /* layer_mlp (:480-487, 369-388): gate and up GEMVs with gelu(gate) * up,
         * after the post-attention norm, residual add and pre-feedforward
         * norm (:463-477), folded into the launch's prologue with fold_mlp */
        g3k_matvec_args a;
        memset(&a, 0, sizeof a);
        a.K = hid;
        a.n_mat = 2;
        a.mode = G3K_MV_GEGLU;
        a.A[0] = lw->gate_proj;
        a.A[1] = lw->up_proj;
        a.y[0] = h;
        a.M[0] = a.M[1] = inter;
        if (fold_mlp && AL8(lw->post_attention_layernorm) && AL8(lw->pre_feedforward_layernorm)) {
            set_pre(&a, cfg, &x, &x_alt, proj, lw->post_attention_layernorm, lw->pre_feedforward_layernorm);
        } else {
            if ((rc = layer_step(c, G3K_OP_RESIDUAL, x, proj, xn, lw->post_attention_layernorm,
                                 lw->pre_feedforward_layernorm, NULL, 0)))
                return rc;
            a.x = xn;
        }
        if ((rc = g3k_matvec(&a, c->stream))) return hip_fail((hipError_t)rc, "g3attn_forward_device MLP");
        if ((rc = gemv(c, mlp, lw->down_proj, h, hid, inter))) return rc;
        /* post-feedforward norm, residual (:490-496); then the next layer's
         * input norm (folded into its Q/K/V launch with fold_qkv), or the
         * final norm before the logits (:508) */
        const int last = l + 1 == L;
        if (!last && fold_qkv && AL8(lw->post_feedforward_layernorm) && AL8(w->layers[l + 1].input_layernorm))
            continue;
        const uint16_t *w_next = last ? (compute_logits ? w->norm : NULL) : w->layers[l + 1].input_layernorm;
        if ((rc = layer_step(c, G3K_OP_RESIDUAL, x, mlp, (last && !compute_logits) ? NULL : xn,
                             lw->post_feedforward_layernorm, w_next, NULL, 0)))
            return rc;
    }
#undef AL8
    /* tied-embedding logits (:511) */
    if (compute_logits && (rc = gemv(c, logits, w->embed_tokens, xn, cfg->vocab_size, hid))) return rc;
    if (hidden_out)
        HIP_TRY(hipMemcpyAsync(hidden_out, x, (size_t)hid * 4, hipMemcpyDeviceToDevice, c->stream),
                "g3attn_forward_device hidden");
    return G3_OK;
}

int g3attn_forward_device(g3attn_ctx *c, const g3attn_weights *w, int token_id, int pos,
                          float *logits, int compute_logits, float *hidden_out) {
    if (!c || !w || !w->embed_tokens || (compute_logits && (!logits || !w->norm))) {
        set_err("g3attn_forward_device: null context, weights or output");
        return G3_ERR_INVALID_ARG;
    }
    int rc = forward_check(c, w, token_id, pos, "g3attn_forward_device");
    if (rc) return rc;
    hipSetDevice(c->device);
    if ((rc = forward_buffers(c))) return rc;
    return forward_enqueue(c, w, token_id, pos, logits, compute_logits, hidden_out);
}

/* ---------------------------------------------------------- batched GEMM */

int g3attn_matmul_bf16_device(g3attn_ctx *c, float *C, const uint16_t *W, const float *X, int N, int M, int K) {
    if (!c || !C || !W || !X || N < 1 || M < 4 || M % 4 || K < 32 || K % 32) {
        set_err("g3attn_matmul_bf16_device: null buffer, N < 1, M not a positive multiple of 4 or K not a "
                "positive multiple of 32");
        return G3_ERR_INVALID_ARG;
    }
    hipSetDevice(c->device);
    const size_t plane = align256((size_t)N * K * 2);
    int rc = grow_buf(c, (float **)&c->d_big, &c->d_big_cap, 2 * plane, "matmul planes");
    if (rc) return rc;
    uint16_t *xh = (uint16_t *)c->d_big, *xl = (uint16_t *)((unsigned char *)c->d_big + plane);
    g3k_rows_args r;
    memset(&r, 0, sizeof r);
    r.op = G3K_ROWS_SPLIT;
    r.rows = N;
    r.n = K;
    r.t = X;
    r.ldt = K;
    r.y_hi = xh;
    r.y_lo = xl;
    r.ldy = K;
    rc = g3k_rows(&r, c->stream);
    if (rc) return hip_fail((hipError_t)rc, "g3attn_matmul_bf16_device split");
    g3k_gemm_args g;
    memset(&g, 0, sizeof g);
    g.x_hi = xh;
    g.x_lo = xl;
    g.N = N;
    g.K = K;
    g.ldx = K;
    g.n_mat = 1;
    g.ksplit = 1;
    g.W[0] = W;
    g.M[0] = M;
    g.C[0] = C;
    g.ldc[0] = M;
    rc = g3k_gemm(&g, c->stream);
    if (rc) return hip_fail((hipError_t)rc, "g3attn_matmul_bf16_device");
    return G3_OK;
}

/* ---------------------------------------------------------- batched prefill */

/* Tokens per pass through the stack: the activations below take about 100 KiB
 * per token at Gemma3-4B shapes (0.8 GiB at 8192). */
#define PB_CHUNK 8192
#define PB_SPLIT_MAX 4

/* k splits for a GEMM with M output rows over n tokens: the smallest power of
 * two (<= PB_SPLIT_MAX) that gives 512 workgroups of 128 x 128 (two per CU),
 * with K / S a multiple of 32. */
static int pick_ksplit(int n, int M, int K) {
    const long long wgs = (long long)((M + 127) / 128) * ((n + 127) / 128);
    int S = 1;
    while (S < PB_SPLIT_MAX && wgs * S < 512 && K % (32 * 2 * S) == 0) S *= 2;
    return S;
}

typedef struct {
    float *x, *q, *k, *v, *attn, *t, *xn;
    uint16_t *xh, *xl, *ah, *al, *hh, *hl;
} pb_bufs;

static int pb_layout(g3attn_ctx *c, int n, pb_bufs *b) {
    const g3attn_config *cfg = &c->cfg;
    const size_t hid = cfg->hidden_size, inter = cfg->intermediate_size;
    const size_t qs = (size_t)cfg->num_heads * D, ks = (size_t)cfg->num_kv_heads * D, N = n;
    const size_t sz[13] = {N * hid * 4, N * qs * 4, N * ks * 4, N * ks * 4, N * qs * 4, PB_SPLIT_MAX * N * hid * 4, hid * 4,
                           N * hid * 2, N * hid * 2, N * qs * 2, N * qs * 2, N * inter * 2, N * inter * 2};
    size_t total = 0;
    for (int i = 0; i < 13; i++) total += align256(sz[i]);
    int rc = grow_buf(c, (float **)&c->d_pb, &c->d_pb_cap, total, "prefill activations");
    if (rc) return rc;
    unsigned char *p = (unsigned char *)c->d_pb;
    void **dst[13] = {(void **)&b->x, (void **)&b->q, (void **)&b->k, (void **)&b->v, (void **)&b->attn,
                      (void **)&b->t, (void **)&b->xn, (void **)&b->xh, (void **)&b->xl, (void **)&b->ah,
                      (void **)&b->al, (void **)&b->hh, (void **)&b->hl};
    for (int i = 0; i < 13; i++) {
        *dst[i] = p;
        p += align256(sz[i]);
    }
    return G3_OK;
}

static int rows_step(g3attn_ctx *c, const g3k_rows_args *a) {
    const int rc = g3k_rows(a, c->stream);
    return rc ? hip_fail((hipError_t)rc, "g3attn_prefill_forward_device rows") : G3_OK;
}

static int gemm_step(g3attn_ctx *c, const g3k_gemm_args *a) {
    const int rc = g3k_gemm(a, c->stream);
    return rc ? hip_fail((hipError_t)rc, "g3attn_prefill_forward_device GEMM") : G3_OK;
}

/* One chunk of n tokens at positions pos0.. through every layer: the
 * reference's batched prefill (gemma3_transformer.c:585-766) with the
 * projections on MFMA and the attention on the prefill kernel. */
static int prefill_chunk(g3attn_ctx *c, const g3attn_weights *w, int n, int pos0, const pb_bufs *b) {
    const g3attn_config *cfg = &c->cfg;
    const int hid = cfg->hidden_size, inter = cfg->intermediate_size, L = cfg->num_layers;
    const int qs = cfg->num_heads * D, ks = cfg->num_kv_heads * D;
    int rc;
    g3k_rows_args r;
    memset(&r, 0, sizeof r);
    r.rows = n;
    r.n = hid;
    r.eps = cfg->rmsnorm_eps;
    /* embedding * sqrt(hidden) and layer 0's input norm (:585-602) */
    r.op = G3K_ROWS_EMBED;
    r.tokens = c->d_tok;
    r.embed = w->embed_tokens;
    r.w_next = w->layers[0].input_layernorm;
    r.x = b->x;
    r.y_hi = b->xh;
    r.y_lo = b->xl;
    r.ldy = hid;
    if ((rc = rows_step(c, &r))) return rc;
    for (int l = 0; l < L; l++) {
        const g3attn_layer_weights *lw = &w->layers[l];
        g3k_gemm_args g;
        /* Q/K/V projections (:604-639) */
        memset(&g, 0, sizeof g);
        g.x_hi = b->xh;
        g.x_lo = b->xl;
        g.N = n;
        g.K = hid;
        g.ldx = hid;
        g.n_mat = 3;
        g.ksplit = 1;
        g.W[0] = lw->q_proj;
        g.W[1] = lw->k_proj;
        g.W[2] = lw->v_proj;
        g.M[0] = qs;
        g.M[1] = g.M[2] = ks;
        g.C[0] = b->q;
        g.C[1] = b->k;
        g.C[2] = b->v;
        g.ldc[0] = qs;
        g.ldc[1] = g.ldc[2] = ks;
        if ((rc = gemm_step(c, &g))) return rc;
        /* QK-norm, RoPE, cache write, attention (:641-692) */
        /* the whole-model path keeps the exact score policy: its logits are
         * held to the token forward's 1e-4 x RMS, tighter than the
         * attention path's 2e-3 */
        if ((rc = prefill_attention(c, l, pos0, n, b->q, b->k, b->v, lw->q_norm, lw->k_norm, b->attn, 0)))
            return rc;
        /* o_proj (:694-699) */
        memset(&r, 0, sizeof r);
        r.op = G3K_ROWS_SPLIT;
        r.rows = n;
        r.n = qs;
        r.t = b->attn;
        r.ldt = qs;
        r.y_hi = b->ah;
        r.y_lo = b->al;
        r.ldy = qs;
        if ((rc = rows_step(c, &r))) return rc;
        memset(&g, 0, sizeof g);
        g.x_hi = b->ah;
        g.x_lo = b->al;
        g.N = n;
        g.K = qs;
        g.ldx = qs;
        g.n_mat = 1;
        g.ksplit = pick_ksplit(n, hid, qs);
        g.split_stride = (long long)n * hid;
        g.W[0] = lw->o_proj;
        g.M[0] = hid;
        g.C[0] = b->t;
        g.ldc[0] = hid;
        if ((rc = gemm_step(c, &g))) return rc;
        const int o_split = g.ksplit;
        /* post-attention norm + residual, pre-feedforward norm (:701-724) */
        memset(&r, 0, sizeof r);
        r.op = G3K_ROWS_RESIDUAL;
        r.rows = n;
        r.n = hid;
        r.eps = cfg->rmsnorm_eps;
        r.w_post = lw->post_attention_layernorm;
        r.w_next = lw->pre_feedforward_layernorm;
        r.x = b->x;
        r.t = b->t;
        r.ldt = hid;
        r.nsplit = o_split;
        r.split_stride = (long long)n * hid;
        r.y_hi = b->xh;
        r.y_lo = b->xl;
        r.ldy = hid;
        if ((rc = rows_step(c, &r))) return rc;
        /* gate and up projections with gelu(gate) * up (:726-745) */
        memset(&g, 0, sizeof g);
        g.x_hi = b->xh;
        g.x_lo = b->xl;
        g.N = n;
        g.K = hid;
        g.ldx = hid;
        g.n_mat = 2;
        g.ksplit = 1;
        g.mode = G3K_MV_GEGLU;
        g.W[0] = lw->gate_proj;
        g.W[1] = lw->up_proj;
        g.M[0] = g.M[1] = inter;
        g.h_hi = b->hh;
        g.h_lo = b->hl;
        g.ldh = inter;
        if ((rc = gemm_step(c, &g))) return rc;
        /* down projection (:747-751) */
        memset(&g, 0, sizeof g);
        g.x_hi = b->hh;
        g.x_lo = b->hl;
        g.N = n;
        g.K = inter;
        g.ldx = inter;
        g.n_mat = 1;
        g.ksplit = pick_ksplit(n, hid, inter);
        g.split_stride = (long long)n * hid;
        g.W[0] = lw->down_proj;
        g.M[0] = hid;
        g.C[0] = b->t;
        g.ldc[0] = hid;
        if ((rc = gemm_step(c, &g))) return rc;
        const int d_split = g.ksplit;
        /* post-feedforward norm + residual (:753-765), then the next layer's input norm */
        const int last = l + 1 == L;
        memset(&r, 0, sizeof r);
        r.op = G3K_ROWS_RESIDUAL;
        r.rows = n;
        r.n = hid;
        r.eps = cfg->rmsnorm_eps;
        r.w_post = lw->post_feedforward_layernorm;
        r.w_next = last ? NULL : w->layers[l + 1].input_layernorm;
        r.x = b->x;
        r.t = b->t;
        r.ldt = hid;
        r.nsplit = d_split;
        r.split_stride = (long long)n * hid;
        r.y_hi = last ? NULL : b->xh;
        r.y_lo = last ? NULL : b->xl;
        r.ldy = hid;
        if ((rc = rows_step(c, &r))) return rc;
    }
    return G3_OK;
}

int g3attn_prefill_forward_device(g3attn_ctx *c, const g3attn_weights *w, const int *tokens, int num_tokens,
                                  int start_pos, float *logits) {
    if (!c || !w || !tokens || num_tokens < 1 || start_pos < 0 || !w->embed_tokens || (logits && !w->norm)) {
        set_err("g3attn_prefill_forward_device: null context / weights / tokens, num_tokens < 1 or "
                "start_pos < 0");
        return G3_ERR_INVALID_ARG;
    }
    const g3attn_config *cfg = &c->cfg;
    const int hid = cfg->hidden_size, inter = cfg->intermediate_size, L = cfg->num_layers;
    const int qs = cfg->num_heads * D;
    if (L < 1 || L > G3ATTN_MAX_LAYERS || hid < 32 || hid > G3K_LAYER_MAX_HIDDEN || hid % 32 || inter < 32 ||
        inter % 32 || qs > G3K_LAYER_MAX_HIDDEN) {
        set_err("g3attn_prefill_forward_device: layers %d, hidden %d, intermediate %d unsupported (hidden and "
                "intermediate must be multiples of 32, hidden <= %d)", L, hid, inter, G3K_LAYER_MAX_HIDDEN);
        return G3_ERR_INVALID_ARG;
    }
    for (int l = 0; l < L; l++) {
        const g3attn_layer_weights *lw = &w->layers[l];
        if (!lw->input_layernorm || !lw->q_proj || !lw->k_proj || !lw->v_proj || !lw->o_proj ||
            !lw->gate_proj || !lw->up_proj || !lw->down_proj) {
            set_err("g3attn_prefill_forward_device: layer %d has a null projection or input norm", l);
            return G3_ERR_INVALID_ARG;
        }
    }
    if ((long long)start_pos + num_tokens > c->max_context) {
        set_err("g3attn_prefill_forward_device: positions %d..%d exceed max_context %d", start_pos,
                start_pos + num_tokens - 1, c->max_context);
        return G3_ERR_CONTEXT_OVERFLOW;
    }
    for (int i = 0; i < num_tokens; i++)
        if (tokens[i] < 0 || tokens[i] >= cfg->vocab_size) {
            set_err("g3attn_prefill_forward_device: token %d at %d outside the vocabulary (%d)", tokens[i], i,
                    cfg->vocab_size);
            return G3_ERR_INVALID_ARG;
        }
    hipSetDevice(c->device);
    const int chunk = num_tokens < PB_CHUNK ? num_tokens : PB_CHUNK;
    pb_bufs b;
    int rc = pb_layout(c, chunk, &b);
    if (rc) return rc;
    if ((size_t)chunk * sizeof(int) > c->d_tok_cap) {
        HIP_TRY(hipStreamSynchronize(c->stream), "g3attn_prefill_forward_device");
        hipFree(c->d_tok);
        c->d_tok = NULL;
        c->d_tok_cap = 0;
        if (!alloc_dev((void **)&c->d_tok, (size_t)chunk * sizeof(int), "prefill tokens")) return G3_ERR_OUT_OF_MEMORY;
        c->d_tok_cap = (size_t)chunk * sizeof(int);
    }
    int last_n = 0;
    for (int p = 0; p < num_tokens; p += chunk) {
        const int n = num_tokens - p < chunk ? num_tokens - p : chunk;
        /* the previous chunk's kernels may still read the token ids */
        HIP_TRY(hipStreamSynchronize(c->stream), "g3attn_prefill_forward_device");
        HIP_TRY(hipMemcpy(c->d_tok, tokens + p, (size_t)n * sizeof(int), hipMemcpyHostToDevice),
                "g3attn_prefill_forward_device tokens");
        if ((rc = prefill_chunk(c, w, n, start_pos + p, &b))) return rc;
        last_n = n;
    }
    if (logits) {
        /* the last token's final norm and tied logits (:769-773) */
        float *xl = b.x + (size_t)(last_n - 1) * hid;
        if ((rc = layer_step(c, G3K_OP_NORM, xl, NULL, b.xn, NULL, w->norm, NULL, 0))) return rc;
        if ((rc = gemv(c, logits, w->embed_tokens, b.xn, cfg->vocab_size, hid))) return rc;
    }
    return G3_OK;
}

/* ---------------------------------------------------------- uploaded model */

/* Element counts of the 13 per-layer tensors in the g3attn_layer_weights
 * order, the sizes gemma3_metal_upload_weights wraps (gemma3_metal.m:580-594). */
_Static_assert(sizeof(g3attn_layer_weights) == 13 * sizeof(const uint16_t *),
               "g3attn_layer_weights is 13 tensor pointers, in order");
static void layer_tensor_sizes(const g3attn_config *cfg, size_t n[13]) {
    const size_t hs = (size_t)cfg->hidden_size, is = (size_t)cfg->intermediate_size;
    const size_t qs = (size_t)cfg->num_heads * D, ks = (size_t)cfg->num_kv_heads * D;
    const size_t sz[13] = {hs, qs * hs, ks * hs, ks * hs, hs * qs, D, D, hs, is * hs, is * hs, hs * is, hs, hs};
    memcpy(n, sz, sizeof sz);
}

/* Host -> device through two pinned 32 MiB buffers: the CPU copies chunk i+1
 * out of the source (which may be a file mapping) while the DMA engine moves
 * chunk i. */
#define UP_CHUNK ((size_t)32 << 20)
typedef struct {
    unsigned char *stage[2];
    hipEvent_t done[2];
    int next;
} uploader;

static int up_copy(g3attn_ctx *c, uploader *u, void *dst, const void *src, size_t bytes) {
    for (size_t off = 0; off < bytes; off += UP_CHUNK) {
        const size_t n = bytes - off < UP_CHUNK ? bytes - off : UP_CHUNK;
        const int b = u->next;
        u->next ^= 1;
        HIP_TRY(hipEventSynchronize(u->done[b]), "g3attn_upload_weights");
        memcpy(u->stage[b], (const unsigned char *)src + off, n);
        HIP_TRY(hipMemcpyAsync((unsigned char *)dst + off, u->stage[b], n, hipMemcpyHostToDevice, c->stream),
                "g3attn_upload_weights copy");
        HIP_TRY(hipEventRecord(u->done[b], c->stream), "g3attn_upload_weights");
    }
    return G3_OK;
}

int g3attn_upload_weights(g3attn_ctx *c, const void *weights) {
    if (!c || !weights) {
        set_err("g3attn_upload_weights: null context or weights");
        return G3_ERR_INVALID_ARG;
    }
    const g3attn_weights *w = (const g3attn_weights *)weights;
    const g3attn_config *cfg = &c->cfg;
    const int L = cfg->num_layers;
    if (L > G3ATTN_MAX_LAYERS || cfg->vocab_size < 1 || cfg->hidden_size < 1 || cfg->intermediate_size < 1) {
        set_err("g3attn_upload_weights: %d layers (max %d), vocab %d, hidden %d, intermediate %d", L,
                G3ATTN_MAX_LAYERS, cfg->vocab_size, cfg->hidden_size, cfg->intermediate_size);
        return G3_ERR_INVALID_ARG;
    }
    if (!w->embed_tokens || !w->norm) {
        set_err("g3attn_upload_weights: embed_tokens or norm is NULL");
        return G3_ERR_INVALID_ARG;
    }
    if (fault_at("upload")) {
        set_err("g3attn_upload_weights: injected device allocation failure (G3ATTN_FAULT=upload)");
        return G3_ERR_OUT_OF_MEMORY;
    }
    size_t n[13];
    layer_tensor_sizes(cfg, n);
    const size_t embed_n = (size_t)cfg->vocab_size * cfg->hidden_size, norm_n = (size_t)cfg->hidden_size;
    size_t total = align256(embed_n * 2) + align256(norm_n * 2);
    for (int l = 0; l < L; l++) {
        const uint16_t *t[13];
        memcpy(t, &w->layers[l], sizeof t);
        for (int j = 0; j < 13; j++)
            if (t[j]) total += align256(n[j] * 2);
    }
    hipSetDevice(c->device);
    HIP_TRY(hipStreamSynchronize(c->stream), "g3attn_upload_weights");
    hipFree(c->d_wt);
    c->d_wt = NULL;
    c->have_wt = 0;
    memset(&c->wt, 0, sizeof c->wt);
    if (!alloc_dev(&c->d_wt, total, "weights")) return G3_ERR_OUT_OF_MEMORY;

    uploader u;
    memset(&u, 0, sizeof u);
    int rc = G3_OK;
    for (int b = 0; b < 2 && !rc; b++) {
        if (hipHostMalloc((void **)&u.stage[b], UP_CHUNK, 0) != hipSuccess || hipEventCreate(&u.done[b]) != hipSuccess) {
            set_err("g3attn_upload_weights: pinned staging allocation failed");
            rc = G3_ERR_OUT_OF_MEMORY;
        }
    }
    g3attn_weights dw;
    memset(&dw, 0, sizeof dw);
    unsigned char *p = (unsigned char *)c->d_wt;
    if (!rc) {
        dw.embed_tokens = (const uint16_t *)p;
        rc = up_copy(c, &u, p, w->embed_tokens, embed_n * 2);
        p += align256(embed_n * 2);
    }
    if (!rc) {
        dw.norm = (const uint16_t *)p;
        rc = up_copy(c, &u, p, w->norm, norm_n * 2);
        p += align256(norm_n * 2);
    }
    for (int l = 0; l < L && !rc; l++) {
        const uint16_t *src[13], *dst[13] = {NULL};
        memcpy(src, &w->layers[l], sizeof src);
        for (int j = 0; j < 13 && !rc; j++) {
            if (!src[j]) continue;   /* optional norms stay NULL, as on the host */
            dst[j] = (const uint16_t *)p;
            rc = up_copy(c, &u, p, src[j], n[j] * 2);
            p += align256(n[j] * 2);
        }
        memcpy(&dw.layers[l], dst, sizeof dst);
    }
    if (hipStreamSynchronize(c->stream) != hipSuccess && !rc) rc = hip_fail(hipGetLastError(), "g3attn_upload_weights");
    for (int b = 0; b < 2; b++) {
        if (u.stage[b]) hipHostFree(u.stage[b]);
        if (u.done[b]) hipEventDestroy(u.done[b]);
    }
    if (rc) {
        hipFree(c->d_wt);
        c->d_wt = NULL;
        return rc;
    }
    c->wt = dw;
    c->have_wt = 1;
    return G3_OK;
}

const g3attn_weights *g3attn_device_weights(g3attn_ctx *c) { return c && c->have_wt ? &c->wt : NULL; }

/* The device logits of the host-output calls and their pinned staging. */
static int forward_uploaded_logits(g3attn_ctx *c, const char *who) {
    const size_t vb = (size_t)c->cfg.vocab_size * sizeof(float);
    if (!alloc_dev((void **)&c->d_logits, vb, "logits")) return G3_ERR_OUT_OF_MEMORY;
    if (hipHostMalloc((void **)&c->h_logits, vb, 0) != hipSuccess) {
        c->h_logits = NULL;
        hipFree(c->d_logits);
        c->d_logits = NULL;
        set_err("%s: pinned logits allocation failed", who);
        return G3_ERR_OUT_OF_MEMORY;
    }
    return G3_OK;
}

/* Enqueue one token on the uploaded model (checked first); when
 * want_logits, its logits land in c->d_logits.  (Recording the token's
 * launches as a HIP graph and replaying it measured no faster on MI355X: 2.43
 * vs 2.39 ms per token.  The host issues the launches well ahead of the
 * GPU, so nothing waits on their submission.) */
static int forward_uploaded(g3attn_ctx *c, int token_id, int pos, int want_logits, const char *who) {
    if (fault_at("forward")) {
        set_err("%s: injected GPU failure (G3ATTN_FAULT=forward)", who);
        return G3_ERR_INVALID_ARG;
    }
    if (!c->have_wt) {
        set_err("%s: no weights uploaded (g3attn_upload_weights)", who);
        return G3_ERR_INVALID_ARG;
    }
    int rc = forward_check(c, &c->wt, token_id, pos, who);
    if (rc) return rc;
    if ((rc = forward_buffers(c))) return rc;
    if (want_logits && !c->d_logits && (rc = forward_uploaded_logits(c, who))) return rc;
    return forward_enqueue(c, &c->wt, token_id, pos, want_logits ? c->d_logits : NULL, want_logits, NULL);
}

static int logits_to_host(g3attn_ctx *c, float *logits, const char *who) {
    const size_t vb = (size_t)c->cfg.vocab_size * sizeof(float);
    HIP_TRY(hipMemcpyAsync(c->h_logits, c->d_logits, vb, hipMemcpyDeviceToHost, c->stream), who);
    HIP_TRY(hipStreamSynchronize(c->stream), who);
    memcpy(logits, c->h_logits, vb);
    return G3_OK;
}

int g3attn_forward_token_device(g3attn_ctx *c, int token_id, int pos, float *logits) {
    if (!c) {
        set_err("g3attn_forward_token_device: null context");
        return G3_ERR_INVALID_ARG;
    }
    hipSetDevice(c->device);
    int rc = forward_uploaded(c, token_id, pos, logits != NULL, "g3attn_forward_token_device");
    if (rc) return rc;
    if (logits)
        HIP_TRY(hipMemcpyAsync(logits, c->d_logits, (size_t)c->cfg.vocab_size * sizeof(float),
                               hipMemcpyDeviceToDevice, c->stream), "g3attn_forward_token_device");
    return G3_OK;
}

int g3attn_forward_token(g3attn_ctx *c, int token_id, int pos, float *logits, int compute_logits) {
    if (!c) {
        set_err("g3attn_forward_token: null context");
        return G3_ERR_INVALID_ARG;
    }
    hipSetDevice(c->device);
    const int want = compute_logits && logits;
    int rc = forward_uploaded(c, token_id, pos, want, "g3attn_forward_token");
    if (rc) return rc;
    if (want) return logits_to_host(c, logits, "g3attn_forward_token");
    HIP_TRY(hipStreamSynchronize(c->stream), "g3attn_forward_token");
    return G3_OK;
}

int g3attn_prefill_tokens(g3attn_ctx *c, const int *tokens, int num_tokens, int start_pos, float *logits) {
    if (!c || !tokens || num_tokens < 1 || start_pos < 0) {
        set_err("g3attn_prefill_tokens: null context / tokens, num_tokens < 1 or start_pos < 0");
        return G3_ERR_INVALID_ARG;
    }
    if ((long long)start_pos + num_tokens > c->max_context) {
        set_err("g3attn_prefill_tokens: positions %d..%d exceed max_context %d", start_pos,
                start_pos + num_tokens - 1, c->max_context);
        return G3_ERR_CONTEXT_OVERFLOW;
    }
    for (int i = 0; i < num_tokens; i++)
        if (tokens[i] < 0 || tokens[i] >= c->cfg.vocab_size) {
            set_err("g3attn_prefill_tokens: token %d at %d outside the vocabulary (%d)", tokens[i], i,
                    c->cfg.vocab_size);
            return G3_ERR_INVALID_ARG;
        }
    if (fault_at("forward")) {
        set_err("g3attn_prefill_tokens: injected GPU failure (G3ATTN_FAULT=forward)");
        return G3_ERR_INVALID_ARG;
    }
    if (!c->have_wt) {
        set_err("g3attn_prefill_tokens: no weights uploaded (g3attn_upload_weights)");
        return G3_ERR_INVALID_ARG;
    }
    hipSetDevice(c->device);
    int rc = G3_OK;
    if (logits && !c->d_logits && (rc = forward_uploaded_logits(c, "g3attn_prefill_tokens"))) return rc;
    if (num_tokens >= G3ATTN_PREFILL_BATCH_MIN) {
        /* the batched prefill (gemma3_transformer.c:526-787): projections as
         * MFMA GEMMs, attention on the prefill kernel */
        rc = g3attn_prefill_forward_device(c, &c->wt, tokens, num_tokens, start_pos, logits ? c->d_logits : NULL);
    } else {
        /* a short batch: the recorded token forward back to back, logits for
         * the last one only (gemma3_metal.m:977-987) */
        for (int i = 0; i < num_tokens && !rc; i++)
            rc = forward_uploaded(c, tokens[i], start_pos + i, i == num_tokens - 1 && logits,
                                  "g3attn_prefill_tokens");
    }
    if (rc) return rc;
    if (logits) return logits_to_host(c, logits, "g3attn_prefill_tokens");
    HIP_TRY(hipStreamSynchronize(c->stream), "g3attn_prefill_tokens");
    return G3_OK;
}

/* ------------------------------------------------------------------ gemma3_gqa */

/* Process-wide state of the gemma3_gqa-shaped entry point. */
static struct {
    pthread_mutex_t lock;
    int ready, device;
    hipStream_t stream;
    void *buf;
    size_t cap;
    float *ws_acc, *ws_ml;
} g_gqa = {PTHREAD_MUTEX_INITIALIZER, 0, 0, NULL, NULL, 0, NULL, NULL};

#define GQA_MAX_KV 64

static int gqa_init(void) {
    if (g_gqa.ready) return G3_OK;
    HIP_TRY(hipGetDevice(&g_gqa.device), "g3attn_gqa init");
    HIP_TRY(hipStreamCreateWithFlags(&g_gqa.stream, hipStreamNonBlocking), "g3attn_gqa init");
    const size_t slots = ws_slots(GQA_MAX_KV) * 4; /* group <= 4 */
    if (!alloc_dev((void **)&g_gqa.ws_acc, slots * D * sizeof(float), "gqa workspace") ||
        !alloc_dev((void **)&g_gqa.ws_ml, slots * 2 * sizeof(float), "gqa workspace"))
        return G3_ERR_OUT_OF_MEMORY;
    g_gqa.ready = 1;
    return G3_OK;
}

/* The gemma3_gqa call on device buffers: q [n_heads][D], K/V rows
 * [seq_len][n_kv][D] (the reference layout), optional additive mask
 * [seq_len], out [n_heads][D]; split partials in ws_acc / ws_ml. */
static void gqa_args(g3k_decode_args *a, float *dout, const float *dq, const float *dk, const float *dv,
                     const float *dm, int n_heads, int n_kv, int seq_len, float scale, float *ws_acc,
                     float *ws_ml) {
    memset(a, 0, sizeof *a);
    a->q = dq;
    a->kc = (float *)dk;
    a->vc = (float *)dv;
    a->row_stride = (long long)n_kv * D;
    a->head_stride = D;
    a->n_stream = seq_len;
    a->skip = INT_MAX;
    a->new_slot = -1;
    a->mask = dm;
    a->qscale = scale * LOG2E;
    choose_splits(seq_len, n_kv, 512, 0, 64, a);
    a->n_kv_heads = n_kv;
    a->group = n_heads / n_kv;
    a->out = dout;
    a->ws_acc = ws_acc;
    a->ws_ml = ws_ml;
}

/* gemma3_gqa computes any shape whose KV-head index h / (n_heads /
 * n_kv_heads) stays below n_kv_heads, i.e. n_kv_heads divides n_heads (other
 * shapes read past the reference's rows); head_dim up to G3K_GQA_MAX_DIM. */
static int gqa_check(const float *output, const float *q, const float *k_cache, const float *v_cache,
                     int n_heads, int n_kv, int seq_len, int head_dim, const char *who) {
    if (!output || !q || !k_cache || !v_cache || seq_len <= 0) {
        set_err("%s: null buffer or seq_len <= 0", who);
        return G3_ERR_INVALID_ARG;
    }
    if (n_heads <= 0 || n_kv <= 0 || n_heads % n_kv) {
        set_err("%s: num_heads %d not a multiple of num_kv_heads %d", who, n_heads, n_kv);
        return G3_ERR_INVALID_ARG;
    }
    if (head_dim < 1 || head_dim > G3K_GQA_MAX_DIM) {
        set_err("%s: head_dim %d outside 1..%d", who, head_dim, G3K_GQA_MAX_DIM);
        return G3_ERR_INVALID_ARG;
    }
    return G3_OK;
}

/* The split-K decode kernels take head_dim 256 and groups 1, 2, 4 (the
 * model's shapes); every other shape goes to the general kernel. */
static int gqa_fast_shape(int n_heads, int n_kv, int head_dim) {
    const int g = n_heads / n_kv;
    return head_dim == D && (g == 1 || g == 2 || g == 4) && n_kv <= GQA_MAX_KV;
}

/* Split-K shape of the general kernel: about 512 workgroups over the query
 * heads, at least 32 rows per split, and a workspace of at most max_acc
 * partial floats ([n_heads][splits][head_dim]). */
static void gqa_generic_args(g3k_gqa_args *a, float *dout, const float *dq, const float *dk, const float *dv,
                             const float *dm, int n_heads, int n_kv, int seq_len, int head_dim, float scale,
                             float *ws_acc, float *ws_ml, size_t max_acc) {
    memset(a, 0, sizeof *a);
    int S = (512 + n_heads - 1) / n_heads;
    const int by_rows = (seq_len + 31) / 32;
    if (S > by_rows) S = by_rows;
    if (S > G3K_MAX_SPLITS) S = G3K_MAX_SPLITS;
    const size_t fit = max_acc / ((size_t)n_heads * head_dim);
    if ((size_t)S > fit) S = (int)fit;
    if (S < 1) S = 1;
    a->rows_per_split = (seq_len + S - 1) / S;
    a->n_splits = (seq_len + a->rows_per_split - 1) / a->rows_per_split;
    a->q = dq;
    a->k = dk;
    a->v = dv;
    a->mask = dm;
    a->out = dout;
    a->ws_acc = ws_acc;
    a->ws_ml = ws_ml;
    a->n_heads = n_heads;
    a->n_kv_heads = n_kv;
    a->seq_len = seq_len;
    a->head_dim = head_dim;
    a->qscale = scale * LOG2E;
}

static int gqa_run(float *output, const float *q, const float *k_cache, const float *v_cache,
                   int n_heads, int n_kv, int seq_len, int head_dim, float scale, const float *mask) {
    int rc = gqa_check(output, q, k_cache, v_cache, n_heads, n_kv, seq_len, head_dim, "g3attn_gqa");
    if (rc) return rc;
    const int fast = gqa_fast_shape(n_heads, n_kv, head_dim);
    rc = gqa_init();
    if (rc) return rc;
    hipSetDevice(g_gqa.device);
    const size_t qs = (size_t)n_heads * head_dim, kvb = (size_t)seq_len * n_kv * head_dim * sizeof(float);
    /* the general kernel's split partials follow the inputs (at most 256
     * splits, so at most n_heads * 256 * (head_dim + 2) floats) */
    const size_t gen_acc = fast ? 0 : (size_t)n_heads * G3K_MAX_SPLITS * head_dim;
    const size_t gen_ml = fast ? 0 : (size_t)n_heads * G3K_MAX_SPLITS * 2;
    const size_t in_bytes = align256(qs * 4 * 2 + 2 * kvb + (size_t)seq_len * 4);
    const size_t need = in_bytes + (gen_acc + gen_ml) * 4 + 256;
    if (need > g_gqa.cap) {
        hipFree(g_gqa.buf);
        g_gqa.buf = NULL;
        g_gqa.cap = 0;
        if (!alloc_dev(&g_gqa.buf, need, "gqa buffers")) return G3_ERR_OUT_OF_MEMORY;
        g_gqa.cap = need;
    }
    unsigned char *b = (unsigned char *)g_gqa.buf;
    float *dq = (float *)b, *dout = (float *)(b + qs * 4);
    float *dk = (float *)(b + qs * 8), *dv = (float *)(b + qs * 8 + kvb);
    float *dm = mask ? (float *)(b + qs * 8 + 2 * kvb) : NULL;
    hipStream_t s = g_gqa.stream;
    HIP_TRY(hipMemcpyAsync(dq, q, qs * 4, hipMemcpyHostToDevice, s), "g3attn_gqa upload");
    HIP_TRY(hipMemcpyAsync(dk, k_cache, kvb, hipMemcpyHostToDevice, s), "g3attn_gqa upload");
    HIP_TRY(hipMemcpyAsync(dv, v_cache, kvb, hipMemcpyHostToDevice, s), "g3attn_gqa upload");
    if (mask) HIP_TRY(hipMemcpyAsync(dm, mask, (size_t)seq_len * 4, hipMemcpyHostToDevice, s), "g3attn_gqa upload");
    if (fast) {
        g3k_decode_args a;
        gqa_args(&a, dout, dq, dk, dv, dm, n_heads, n_kv, seq_len, scale, g_gqa.ws_acc, g_gqa.ws_ml);
        rc = g3k_decode(&a, 0, s);
    } else {
        g3k_gqa_args a;
        float *acc = (float *)(b + in_bytes);
        gqa_generic_args(&a, dout, dq, dk, dv, dm, n_heads, n_kv, seq_len, head_dim, scale, acc, acc + gen_acc,
                         gen_acc);
        rc = g3k_gqa_generic(&a, s);
    }
    if (rc) return hip_fail((hipError_t)rc, "g3attn_gqa launch");
    HIP_TRY(hipMemcpyAsync(output, dout, qs * 4, hipMemcpyDeviceToHost, s), "g3attn_gqa download");
    HIP_TRY(hipStreamSynchronize(s), "g3attn_gqa");
    return G3_OK;
}

void g3attn_gqa(float *output, const float *q, const float *k_cache, const float *v_cache,
                int n_heads, int n_kv_heads, int seq_len, int head_dim, float scale,
                const float *mask, float *scores_buf) {
    (void)scores_buf;
    g_err[0] = 0;
    pthread_mutex_lock(&g_gqa.lock);
    gqa_run(output, q, k_cache, v_cache, n_heads, n_kv_heads, seq_len, head_dim, scale, mask);
    pthread_mutex_unlock(&g_gqa.lock);
}

/* The same computation on device buffers with no allocation at all: the
 * split partials go to the library's fixed static device scratch (see
 * g3k_noalloc_scratch), looked up once per device.  Same split choice as
 * g3attn_gqa, so the two agree bit for bit. */
int g3attn_gqa_noalloc(float *output, const float *q, const float *k_cache, const float *v_cache,
                       int n_heads, int n_kv_heads, int seq_len, int head_dim, float scale,
                       const float *mask, void *stream) {
    g_err[0] = 0;
    int rc = gqa_check(output, q, k_cache, v_cache, n_heads, n_kv_heads, seq_len, head_dim,
                       "g3attn_gqa_noalloc");
    if (rc) return rc;
    if (n_heads > G3ATTN_NOALLOC_MAX_HEADS) {
        set_err("g3attn_gqa_noalloc: n_heads %d exceeds the fixed scratch's %d heads", n_heads,
                G3ATTN_NOALLOC_MAX_HEADS);
        return G3_ERR_INVALID_ARG;
    }
    float *acc = NULL, *ml = NULL;
    rc = g3k_noalloc_scratch(&acc, &ml);
    if (rc) return hip_fail((hipError_t)rc, "g3attn_gqa_noalloc scratch");
    if (gqa_fast_shape(n_heads, n_kv_heads, head_dim)) {
        g3k_decode_args a;
        gqa_args(&a, output, q, k_cache, v_cache, mask, n_heads, n_kv_heads, seq_len, scale, acc, ml);
        rc = g3k_decode(&a, 0, stream);
    } else {
        /* the same scratch, in the general kernel's layout: its splits are
         * capped so the partials fit (n_heads <= 16 and head_dim <= 512 leave
         * at least 128 splits) */
        g3k_gqa_args a;
        gqa_generic_args(&a, output, q, k_cache, v_cache, mask, n_heads, n_kv_heads, seq_len, head_dim, scale, acc,
                         ml, (size_t)G3K_NOALLOC_MAX_HEADS * G3K_MAX_SPLITS * D);
        rc = g3k_gqa_generic(&a, stream);
    }
    if (rc) return hip_fail((hipError_t)rc, "g3attn_gqa_noalloc launch");
    return G3_OK;
}

/* Host-pointer GEMV through the same process-wide stream; its own grow-on-
 * demand device buffer holds A, x and y. */
static struct {
    void *buf;
    size_t cap;
} g_mv = {NULL, 0};

static int matvec_run(float *y, const uint16_t *A, const float *x, int M, int K) {
    int rc = matvec_check(M, K, y, A, x, "g3attn_matvec_bf16");
    if (rc) return rc;
    rc = gqa_init();
    if (rc) return rc;
    hipSetDevice(g_gqa.device);
    const size_t ab = align256((size_t)M * K * sizeof(uint16_t)), xb = align256((size_t)K * 4);
    const size_t need = ab + xb + (size_t)M * 4;
    if (need > g_mv.cap) {
        hipFree(g_mv.buf);
        g_mv.buf = NULL;
        g_mv.cap = 0;
        if (!alloc_dev(&g_mv.buf, need, "matvec buffers")) return G3_ERR_OUT_OF_MEMORY;
        g_mv.cap = need;
    }
    unsigned char *b = (unsigned char *)g_mv.buf;
    uint16_t *dA = (uint16_t *)b;
    float *dx = (float *)(b + ab), *dy = (float *)(b + ab + xb);
    hipStream_t s = g_gqa.stream;
    HIP_TRY(hipMemcpyAsync(dA, A, (size_t)M * K * sizeof(uint16_t), hipMemcpyHostToDevice, s), "g3attn_matvec_bf16 upload");
    HIP_TRY(hipMemcpyAsync(dx, x, (size_t)K * 4, hipMemcpyHostToDevice, s), "g3attn_matvec_bf16 upload");
    g3k_matvec_args a;
    memset(&a, 0, sizeof a);
    a.x = dx;
    a.K = K;
    a.n_mat = 1;
    a.A[0] = dA;
    a.y[0] = dy;
    a.M[0] = M;
    rc = g3k_matvec(&a, s);
    if (rc) return hip_fail((hipError_t)rc, "g3attn_matvec_bf16 launch");
    HIP_TRY(hipMemcpyAsync(y, dy, (size_t)M * 4, hipMemcpyDeviceToHost, s), "g3attn_matvec_bf16 download");
    HIP_TRY(hipStreamSynchronize(s), "g3attn_matvec_bf16");
    return G3_OK;
}

void g3attn_matvec_bf16(float *y, const uint16_t *A, const float *x, int M, int K, float *scratch) {
    (void)scratch;
    g_err[0] = 0;
    pthread_mutex_lock(&g_gqa.lock);
    matvec_run(y, A, x, M, K);
    pthread_mutex_unlock(&g_gqa.lock);
}
