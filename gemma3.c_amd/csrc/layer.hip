// layer.hip - the small kernels between the GEMVs of one token's forward pass
// (gemma3_transformer_forward, gemma3_transformer.c:396-512): the embedding
// row, the hidden-size RMSNorms with their residual adds.
//
// Each works on one hidden vector (a few thousand floats), so each is one
// workgroup: latency, not bandwidth, is what they cost, and folding the
// norms and adds that sit between two GEMVs into one launch is what matters.
//   embed:     x = bf16(E[token]) * sqrt(hidden)          (:415-422)
//   norm:      y = rmsnorm(x, w)                           (:444-446, 508)
//   residual:  t = rmsnorm(t, w_post)  (if w_post)         (:463-466, 490-493)
//              x = x + t                                   (:469, 496)
//              y = rmsnorm(x, w_next)  (if y; a copy of x if w_next is NULL)
// rmsnorm is gemma3_rmsnorm_bf16 (gemma3_kernels.c:289-304): mean of squares
// + eps, 1 / sqrtf, then x * r * (1 + bf16(w)); the sum of squares is a tree
// here instead of the reference's sequential loop.
#include <hip/hip_runtime.h>

#include "g3k.h"
#include "g3k_device.h"

namespace {

using namespace g3k;

constexpr int NT = 1024;
constexpr int NW = NT / 64;
constexpr int PER = 8;   // values per thread: hidden <= NT * PER

// Sum over the workgroup; every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();   // red may still be read by an earlier call
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < NW; w++) s += red[w];
    return s;
}

// r = 1 / sqrtf(mean(v^2) + eps) over the n values held PER per thread.
__device__ __forceinline__ float rms_scale(const float (&v)[PER], int n, float eps, float *red) {
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < PER; u++) ss += v[u] * v[u];
    ss = block_sum(ss, red);
    return 1.0f / sqrtf(ss / (float)n + eps);
}

__global__ __launch_bounds__(NT) void embed_kernel(g3k_layer_args a) {
    const int n = a.n;
    const float scale = sqrtf((float)n);
    const uint16_t *row = a.embed + (size_t)a.token * n;
    for (int i = threadIdx.x; i < n; i += NT) a.x[i] = bf16f(row[i]) * scale;
}

// The gains (1 + w) of a norm, loaded up front so that their latency overlaps
// the activations' loads instead of following a reduction.
__device__ __forceinline__ void load_gain(float (&g)[PER], const uint16_t *w, int n) {
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = threadIdx.x + NT * u;
        g[u] = (w && i < n) ? 1.0f + bf16f(w[i]) : 0.f;
    }
}

__global__ __launch_bounds__(NT) void norm_kernel(g3k_layer_args a) {
    __shared__ float red[NW];
    const int n = a.n;
    float v[PER], g[PER];
    load_gain(g, a.w_next, n);
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = threadIdx.x + NT * u;
        v[u] = i < n ? a.x[i] : 0.f;
    }
    const float r = rms_scale(v, n, a.eps, red);
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = threadIdx.x + NT * u;
        if (i < n) a.y[i] = v[u] * r * g[u];
    }
}

__global__ __launch_bounds__(NT) void residual_kernel(g3k_layer_args a) {
    __shared__ float red[NW];
    const int n = a.n;
    float t[PER], x[PER], gp[PER], gn[PER];
    load_gain(gp, a.w_post, n);
    load_gain(gn, a.y ? a.w_next : nullptr, n);
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = threadIdx.x + NT * u;
        t[u] = i < n ? a.t[i] : 0.f;
        x[u] = i < n ? a.x[i] : 0.f;
    }
    if (a.w_post) {
        const float r = rms_scale(t, n, a.eps, red);
#pragma unroll
        for (int u = 0; u < PER; u++) t[u] = t[u] * r * gp[u];   // gp is 0 past n
    }
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = threadIdx.x + NT * u;
        x[u] = x[u] + t[u];
        if (i < n) a.x[i] = x[u];
    }
    if (!a.y) return;   // uniform
    if (a.w_next) {
        const float r = rms_scale(x, n, a.eps, red);
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int i = threadIdx.x + NT * u;
            if (i < n) a.y[i] = x[u] * r * gn[u];
        }
    } else {
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int i = threadIdx.x + NT * u;
            if (i < n) a.y[i] = x[u];
        }
    }
}

}  // namespace

extern "C" int g3k_layer_step(const g3k_layer_args *a, void *stream) {
    if (a->n < 1 || a->n > G3K_LAYER_MAX_HIDDEN) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    switch (a->op) {
        case G3K_OP_EMBED:
            if (!a->embed || !a->x || a->token < 0) return (int)hipErrorInvalidValue;
            hipLaunchKernelGGL(embed_kernel, dim3(1), dim3(NT), 0, st, *a);
            break;
        case G3K_OP_NORM:
            if (!a->x || !a->y || !a->w_next) return (int)hipErrorInvalidValue;
            hipLaunchKernelGGL(norm_kernel, dim3(1), dim3(NT), 0, st, *a);
            break;
        case G3K_OP_RESIDUAL:
            if (!a->x || !a->t) return (int)hipErrorInvalidValue;
            hipLaunchKernelGGL(residual_kernel, dim3(1), dim3(NT), 0, st, *a);
            break;
        default:
            return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

// ------------------------------------------------------------ batched rows
// One workgroup of 256 threads per token row (gemma3_transformer.c:585-592,
// 596-602, 702-724, 753-765: the reference's per-token loops of the batched
// prefill).  Values per thread: n <= 256 * RPER.

namespace {

constexpr int RNT = 256;
constexpr int RNW = RNT / 64;
constexpr int RPER = G3K_LAYER_MAX_HIDDEN / RNT;

__device__ __forceinline__ float rblock_sum(float v, float *red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < RNW; w++) s += red[w];
    return s;
}

__device__ __forceinline__ uint32_t rne16(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// y = v * r * gain (gain 1 where w is NULL) as bf16 hi / lo planes
__device__ __forceinline__ void store_split(const g3k_rows_args &a, int row, const float (&v)[RPER], float r,
                                            const uint16_t *w) {
    uint16_t *yh = a.y_hi + (size_t)row * a.ldy, *yl = a.y_lo + (size_t)row * a.ldy;
#pragma unroll
    for (int u = 0; u < RPER; u++) {
        const int i = threadIdx.x + RNT * u;
        if (i < a.n) {
            const float y = w ? v[u] * r * (1.0f + bf16f(w[i])) : v[u];
            const uint32_t hi = rne16(y);
            yh[i] = (uint16_t)hi;
            yl[i] = (uint16_t)rne16(y - __uint_as_float(hi << 16));
        }
    }
}

__global__ __launch_bounds__(RNT) void rows_kernel(g3k_rows_args a) {
    __shared__ float red[RNW];
    const int row = blockIdx.x, n = a.n;
    float v[RPER];
    if (a.op == G3K_ROWS_SPLIT) {   // elementwise: any row length
        const float *t = a.t + (size_t)row * a.ldt;
        uint16_t *yh = a.y_hi + (size_t)row * a.ldy, *yl = a.y_lo + (size_t)row * a.ldy;
        for (int i = threadIdx.x; i < n; i += RNT) {
            const float y = t[i];
            const uint32_t hi = rne16(y);
            yh[i] = (uint16_t)hi;
            yl[i] = (uint16_t)rne16(y - __uint_as_float(hi << 16));
        }
        return;
    }
    float *x = a.x + (size_t)row * n;
    if (a.op == G3K_ROWS_EMBED) {
        const float scale = sqrtf((float)n);
        const uint16_t *e = a.embed + (size_t)a.tokens[row] * n;
#pragma unroll
        for (int u = 0; u < RPER; u++) {
            const int i = threadIdx.x + RNT * u;
            v[u] = i < n ? bf16f(e[i]) * scale : 0.f;
            if (i < n) x[i] = v[u];
        }
    } else {
        const float *t = a.t + (size_t)row * a.ldt;
        float tv[RPER];
#pragma unroll
        for (int u = 0; u < RPER; u++) {
            const int i = threadIdx.x + RNT * u;
            tv[u] = i < n ? t[i] : 0.f;
            v[u] = i < n ? x[i] : 0.f;
        }
        for (int s = 1; s < a.nsplit; s++) {   // the k splits of the producing GEMM, in order
            const float *ts = t + (size_t)s * a.split_stride;
#pragma unroll
            for (int u = 0; u < RPER; u++) {
                const int i = threadIdx.x + RNT * u;
                if (i < n) tv[u] += ts[i];
            }
        }
        if (a.w_post) {
            float ss = 0.f;
#pragma unroll
            for (int u = 0; u < RPER; u++) ss += tv[u] * tv[u];
            const float r = 1.0f / sqrtf(rblock_sum(ss, red) / (float)n + a.eps);
#pragma unroll
            for (int u = 0; u < RPER; u++) {
                const int i = threadIdx.x + RNT * u;
                tv[u] = i < n ? tv[u] * r * (1.0f + bf16f(a.w_post[i])) : 0.f;
            }
        }
#pragma unroll
        for (int u = 0; u < RPER; u++) {
            const int i = threadIdx.x + RNT * u;
            v[u] = v[u] + tv[u];
            if (i < n) x[i] = v[u];
        }
        if (!a.y_hi) return;   // uniform
    }
    float r = 1.f;
    if (a.w_next) {
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < RPER; u++) ss += v[u] * v[u];
        r = 1.0f / sqrtf(rblock_sum(ss, red) / (float)n + a.eps);
    }
    store_split(a, row, v, r, a.w_next);
}

}  // namespace

extern "C" int g3k_rows(const g3k_rows_args *a, void *stream) {
    if (a->rows < 1 || a->n < 1 || (a->op != G3K_ROWS_SPLIT && a->n > G3K_LAYER_MAX_HIDDEN))
        return (int)hipErrorInvalidValue;
    const bool split_out = a->y_hi && a->y_lo && a->ldy >= a->n;
    switch (a->op) {
        case G3K_ROWS_EMBED:
            if (!a->tokens || !a->embed || !a->x || !split_out) return (int)hipErrorInvalidValue;
            break;
        case G3K_ROWS_RESIDUAL:
            if (!a->x || !a->t || a->ldt < a->n || ((a->y_hi || a->y_lo) && !split_out) || a->nsplit < 1 ||
                (a->nsplit > 1 && a->split_stride < (long long)a->rows * a->ldt))
                return (int)hipErrorInvalidValue;
            break;
        case G3K_ROWS_SPLIT:
            if (!a->t || a->ldt < a->n || !split_out) return (int)hipErrorInvalidValue;
            break;
        default:
            return (int)hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(rows_kernel, dim3(a->rows), dim3(RNT), 0, (hipStream_t)stream, *a);
    return (int)hipGetLastError();
}
