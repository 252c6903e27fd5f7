// matvec.hip - bf16-weight GEMV y = A . x on gfx950, for the projections on
// either side of the attention block.
//
// Replaces gemma3_matvec_bf16 (gemma3_kernels.h:217-218, gemma3_kernels.c:
// 188-238): A is [M][K] bf16 row-major, x and y fp32, y[i] = sum_k
// bf16(A[i][k]) * x[k] accumulated in fp32 (the reference's scalar / AVX2
// loops; the summation order differs, which the parity tests bound).
// Callers: layer_attention's Q/K/V projections (gemma3_transformer.c:290-292)
// and its output projection (:355).
//
// At decode batch 1 the GEMV is HBM-bound: 2 bytes of A per multiply-add.
// Workgroup = 4 waves.  Lane l reads the 16-byte chunks l + 64 j of a row
// (8 elements each), so one wave load covers 1 KiB of the row, contiguous;
// CH chunks per lane (a round) are issued, with the x chunks they meet,
// before the FMAs that use them.  Sums reduce over the wave with DPP and
// permlane swaps.  Rows whose length is not a multiple of 8 (or unaligned
// buffers) take a lane-strided scalar path.
//
// Two layouts, picked per shape (measured on the forward's shapes):
//   each wave owns RPW rows of its own (the Q/K/V projections: 1 row, one
//   round of 8 chunks at K = 2560; the tied logits, 262208 rows: 2 rows);
//   or the 4 waves share RPW rows and split each row's chunks in four (KS):
//   the down projection (K = 10240: 5 chunks per lane, one memory round trip
//   instead of five), o_proj (K = 2048) and the GEGLU gate / up pair.
//
// One launch can serve up to three matrices that share x (the Q, K and V
// projections of one token): workgroups are dealt to the matrices in order of
// their row blocks.  The GEGLU mode computes the gate and up rows of the MLP
// together and writes gelu_tanh(gate) * up (gemma3_transformer.c:380-386).
//
// With the residual prologue (pre_t set) the launch also does the step that
// sits between two GEMVs of the token forward: every workgroup forms
// x = rmsnorm(r + rmsnorm(t, w_post), w_next) in LDS while its first round
// of weights is in flight, and workgroup 0 stores the new residual.  That
// takes a one-workgroup launch (a few microseconds of latency) off the
// token's critical path for ~30 KiB of L2 reads per workgroup.
#include <hip/hip_runtime.h>

#include "g3k.h"
#include "g3k_device.h"

namespace {

using namespace g3k;

constexpr int NT = 256;   // 4 waves
constexpr int NW = NT / 64;

__device__ __forceinline__ float dot8(uint4 w, float4 xa, float4 xb) {
    float s = bf16f(w.x & 0xffff) * xa.x;
    s = fmaf(bf16f(w.x >> 16), xa.y, s);
    s = fmaf(bf16f(w.y & 0xffff), xa.z, s);
    s = fmaf(bf16f(w.y >> 16), xa.w, s);
    s = fmaf(bf16f(w.z & 0xffff), xb.x, s);
    s = fmaf(bf16f(w.z >> 16), xb.y, s);
    s = fmaf(bf16f(w.w & 0xffff), xb.z, s);
    s = fmaf(bf16f(w.w >> 16), xb.w, s);
    return s;
}

// Matrix m of the launch and the workgroup's first row in it.
__device__ __forceinline__ int pick(const g3k_matvec_args &a, int rows_per_wg, int &row0) {
    int b = blockIdx.x;
    const int nm = a.mode == G3K_MV_GEGLU ? 1 : a.n_mat;
    for (int m = 0; m < nm; m++) {
        const int nb = (a.M[m] + rows_per_wg - 1) / rows_per_wg;
        if (b < nb) {
            row0 = b * rows_per_wg;
            return m;
        }
        b -= nb;
    }
    row0 = 0;
    return -1;
}

// gelu with the tanh approximation, as gemma3_gelu_tanh_inplace
// (gemma3_kernels.c:348-357): 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
__device__ __forceinline__ float gelu_tanh(float x) {
    const float inner = 0.7978845608028654f * (x + 0.044715f * (x * x * x));
    return 0.5f * x * (1.0f + tanhf(inner));
}

// A streams through a buffer descriptor per matrix with the non-temporal
// cache policy (read once per call, not worth keeping in L2); the byte
// offset of a row chunk fits 32 bits (the launcher checks the matrix size).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t mat_rsrc(const uint16_t *base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(base), (short)0, (int)bytes, 0x00020000);
}

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

// The residual prologue (g3k_matvec_args.pre_*): x = rmsnorm(r + rmsnorm(t,
// w_post), w_next) into xs[0, K), the same operations in the same order as
// the one-workgroup residual step (layer.hip); workgroup 0 stores r +
// rmsnorm(t, w_post) to pre_r_out.  Thread i takes the 4-element groups
// i + NT u (16-byte loads; the launcher checks K % 4 and the alignment of t,
// r, r_out and the gain rows).
constexpr int PRE_P4 = G3K_MATVEC_PRE_MAX / 4 / NT;

// (1 + w) for the 4 gains of group g; 0 past the end or without w.  w is
// 8-byte aligned (the launcher checks).  The load is unconditional (a
// clamped index, or another valid row without w), so no branch forces a
// wait for it before the weights are requested.
__device__ __forceinline__ float4 gain4(const uint16_t *w, const uint16_t *fallback, int g, bool ok) {
    const uint2 p = reinterpret_cast<const uint2 *>(w ? w : fallback)[ok ? g : 0];
    const bool use = w && ok;
    return make_float4(use ? 1.0f + bf16f(p.x & 0xffff) : 0.f, use ? 1.0f + bf16f(p.x >> 16) : 0.f,
                       use ? 1.0f + bf16f(p.y & 0xffff) : 0.f, use ? 1.0f + bf16f(p.y >> 16) : 0.f);
}

__device__ __forceinline__ float sq4(float4 v) { return v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w; }

struct PreVals {
    float4 t[PRE_P4], r[PRE_P4], gp[PRE_P4], gn[PRE_P4];
};

// The prologue's loads; issued before the weights, so that with in-order
// returns its reductions can start while the weights are still in flight.
__device__ __forceinline__ void pre_load(const g3k_matvec_args &a, PreVals &v) {
    const int K4 = a.K >> 2;
    const float4 *t4 = reinterpret_cast<const float4 *>(a.pre_t);
    const float4 *r4 = reinterpret_cast<const float4 *>(a.pre_r);
#pragma unroll
    for (int u = 0; u < PRE_P4; u++) {
        const int g = threadIdx.x + NT * u;
        const bool ok = g < K4;
        const float4 tv = t4[ok ? g : 0], rv = r4[ok ? g : 0];
        v.t[u] = ok ? tv : make_float4(0.f, 0.f, 0.f, 0.f);
        v.r[u] = ok ? rv : make_float4(0.f, 0.f, 0.f, 0.f);
        const uint16_t *any = reinterpret_cast<const uint16_t *>(a.pre_r);
        v.gp[u] = gain4(a.pre_w_post, any, g, ok);
        v.gn[u] = gain4(a.pre_w_next, any, g, ok);
    }
}

__device__ __forceinline__ void pre_finish(const g3k_matvec_args &a, PreVals &v, float4 *xs, float *red) {
    const int K = a.K, K4 = K >> 2;
    if (a.pre_w_post) {   // uniform
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < PRE_P4; u++) ss += sq4(v.t[u]);
        const float rs = 1.0f / sqrtf(block_sum(ss, red) / (float)K + a.pre_eps);
#pragma unroll
        for (int u = 0; u < PRE_P4; u++) {   // gp is 0 past K
            v.t[u].x = v.t[u].x * rs * v.gp[u].x;
            v.t[u].y = v.t[u].y * rs * v.gp[u].y;
            v.t[u].z = v.t[u].z * rs * v.gp[u].z;
            v.t[u].w = v.t[u].w * rs * v.gp[u].w;
        }
    }
#pragma unroll
    for (int u = 0; u < PRE_P4; u++) {
        v.r[u].x = v.r[u].x + v.t[u].x;
        v.r[u].y = v.r[u].y + v.t[u].y;
        v.r[u].z = v.r[u].z + v.t[u].z;
        v.r[u].w = v.r[u].w + v.t[u].w;
    }
    if (blockIdx.x == 0) {
#pragma unroll
        for (int u = 0; u < PRE_P4; u++) {
            const int g = threadIdx.x + NT * u;
            if (g < K4) reinterpret_cast<float4 *>(a.pre_r_out)[g] = v.r[u];
        }
    }
    if (a.pre_w_next) {   // uniform
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < PRE_P4; u++) ss += sq4(v.r[u]);
        const float rs = 1.0f / sqrtf(block_sum(ss, red) / (float)K + a.pre_eps);
#pragma unroll
        for (int u = 0; u < PRE_P4; u++) {
            v.r[u].x = v.r[u].x * rs * v.gn[u].x;
            v.r[u].y = v.r[u].y * rs * v.gn[u].y;
            v.r[u].z = v.r[u].z * rs * v.gn[u].z;
            v.r[u].w = v.r[u].w * rs * v.gn[u].w;
        }
    }
#pragma unroll
    for (int u = 0; u < PRE_P4; u++) {
        const int g = threadIdx.x + NT * u;
        if (g < K4) xs[g] = v.r[u];
    }
    __syncthreads();
}

// NA dot products: RPW consecutive rows of one matrix, or (GEGLU) the same
// rows of the gate and up matrices.  Without KS each wave owns its own RPW
// rows (a workgroup covers 4 RPW rows); with KS the workgroup's 4 waves share
// RPW rows and wave w takes the w-th quarter of every row's chunks (one
// memory round trip for long rows), the four partial sums meeting in LDS.
template <int RPW, int CH, bool VEC, bool KS, bool GEGLU, bool PRE>
__global__ __launch_bounds__(NT) void matvec_kernel(g3k_matvec_args a) {
    constexpr int NA = GEGLU ? 2 * RPW : RPW;
    __shared__ float red[KS ? NW : 1][NA];
    __shared__ float4 xs4[PRE ? G3K_MATVEC_PRE_MAX / 4 : 1];   // x formed by the residual prologue
    __shared__ float pre_red[NW];
    const int K = a.K;
    int row0;
    const int m = pick(a, KS ? RPW : NW * RPW, row0);
    if (m < 0) return;   // uniform over the workgroup
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int M = a.M[m];
    const float *x = a.x;
    const int r0 = KS ? row0 : row0 + wave * RPW;
    const uint16_t *rows[NA];
    unsigned roff[NA];   // byte offset of each row in its matrix
#pragma unroll
    for (int j = 0; j < NA; j++) {
        const int jr = GEGLU ? j % RPW : j;
        const int row = r0 + jr < M ? r0 + jr : M - 1;
        rows[j] = a.A[GEGLU ? j / RPW : m] + (size_t)row * K;
        roff[j] = (unsigned)row * (unsigned)K * 2u;
    }
    float acc[NA];
#pragma unroll
    for (int j = 0; j < NA; j++) acc[j] = 0.f;

    if (VEC) {
        const int nch = K >> 3;
        const int q = KS ? (nch + NW - 1) / NW : nch;
        const int cbeg = KS ? wave * q : 0, cend = KS ? min(cbeg + q, nch) : nch;
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        __amdgpu_buffer_rsrc_t rs[GEGLU ? 2 : 1];
#pragma unroll
        for (int t = 0; t < (GEGLU ? 2 : 1); t++)
            rs[t] = mat_rsrc(a.A[GEGLU ? t : m], (unsigned)((size_t)M * K * 2));
        uint4 w[NA][CH];
        float4 xa[CH], xb[CH];
        // one round: CH chunks per lane of every row (and, without the
        // prologue, the x chunks they meet) requested before any FMA
        auto issue = [&](int base) {
#pragma unroll
            for (int u = 0; u < CH; u++) {
                const int c = base + lane + 64 * u;
                const bool ok = c < cend;
#pragma unroll
                for (int j = 0; j < NA; j++) {
                    const uint4 t = __builtin_bit_cast(
                        uint4, __builtin_amdgcn_raw_buffer_load_b128(rs[GEGLU ? j / RPW : 0], roff[j] + 16u * (ok ? c : 0), 0, 2));
                    w[j][u] = ok ? t : make_uint4(0, 0, 0, 0);
                }
                if (!PRE) {
                    xa[u] = ok ? x4[2 * c] : make_float4(0.f, 0.f, 0.f, 0.f);
                    xb[u] = ok ? x4[2 * c + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
        };
        if (PRE) {
            // the prologue's loads, then the first round's weights, which stay
            // in flight while x is formed
            PreVals pv;
            pre_load(a, pv);
            issue(cbeg);
            pre_finish(a, pv, xs4, pre_red);
        }
        for (int base = cbeg; base < cend; base += 64 * CH) {
            if (!PRE || base != cbeg) issue(base);
            if (PRE) {
#pragma unroll
                for (int u = 0; u < CH; u++) {
                    const int c = base + lane + 64 * u;
                    const bool ok = c < cend;
                    xa[u] = ok ? xs4[2 * c] : make_float4(0.f, 0.f, 0.f, 0.f);
                    xb[u] = ok ? xs4[2 * c + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
#pragma unroll
            for (int u = 0; u < CH; u++)
#pragma unroll
                for (int j = 0; j < NA; j++) acc[j] += dot8(w[j][u], xa[u], xb[u]);
        }
    } else {
        if (PRE) {
            PreVals pv;
            pre_load(a, pv);
            pre_finish(a, pv, xs4, pre_red);
        }
        const int kbeg = KS ? wave * 64 : 0, kstep = KS ? 64 * NW : 64;
        for (int k = kbeg + lane; k < K; k += kstep) {
            const float xv = PRE ? reinterpret_cast<const float *>(xs4)[k] : x[k];
#pragma unroll
            for (int j = 0; j < NA; j++) acc[j] = fmaf(bf16f(rows[j][k]), xv, acc[j]);
        }
    }
    float tot[NA];
#pragma unroll
    for (int j = 0; j < NA; j++) tot[j] = wave_sum(acc[j]);
    if (KS) {
        if (lane == 0) {
#pragma unroll
            for (int j = 0; j < NA; j++) red[wave][j] = tot[j];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int j = 0; j < NA; j++) {
            float t = red[0][j];
#pragma unroll
            for (int w = 1; w < NW; w++) t += red[w][j];
            tot[j] = t;
        }
    }
    if (lane != 0) return;
#pragma unroll
    for (int j = 0; j < RPW; j++) {
        if (r0 + j >= M) break;
        a.y[GEGLU ? 0 : m][r0 + j] = GEGLU ? gelu_tanh(tot[j]) * tot[RPW + j] : tot[j];
    }
}

template <int RPW, int CH, bool VEC, bool KS = false, bool GEGLU = false>
hipError_t launch(const g3k_matvec_args *a, hipStream_t st) {
    int blocks = 0;
    const int nm = GEGLU ? 1 : a->n_mat;
    const int rows_per_wg = KS ? RPW : NW * RPW;
    for (int m = 0; m < nm; m++) blocks += (a->M[m] + rows_per_wg - 1) / rows_per_wg;
    if (a->pre_t)
        hipLaunchKernelGGL((matvec_kernel<RPW, CH, VEC, KS, GEGLU, true>), dim3(blocks), dim3(NT), 0, st, *a);
    else
        hipLaunchKernelGGL((matvec_kernel<RPW, CH, VEC, KS, GEGLU, false>), dim3(blocks), dim3(NT), 0, st, *a);
    return hipGetLastError();
}

}  // namespace

extern "C" int g3k_matvec(const g3k_matvec_args *a, void *stream) {
    const bool pre = a->pre_t != nullptr;
    if (a->n_mat < 1 || a->n_mat > G3K_MATVEC_MAX || a->K < 1 || (!pre && !a->x))
        return (int)hipErrorInvalidValue;
    if (pre && (!a->pre_r || !a->pre_r_out || a->K > G3K_MATVEC_PRE_MAX || a->K % 4 ||
                (((uintptr_t)a->pre_t | (uintptr_t)a->pre_r | (uintptr_t)a->pre_r_out) & 15) ||
                (((uintptr_t)a->pre_w_post | (uintptr_t)a->pre_w_next) & 7) ||
                ((uintptr_t)a->pre_r_out < (uintptr_t)(a->pre_r + a->K) &&
                 (uintptr_t)a->pre_r < (uintptr_t)(a->pre_r_out + a->K))))
        return (int)hipErrorInvalidValue;
    // with the prologue x comes from LDS, 16-byte aligned
    bool vec = a->K % 8 == 0 && (pre || ((uintptr_t)a->x & 15) == 0);
    long long rows = 0;
    for (int m = 0; m < a->n_mat; m++) {
        // GEGLU writes one output (y[0]) from the two matrices
        if (a->M[m] < 1 || !a->A[m] || (!a->y[m] && (a->mode != G3K_MV_GEGLU || m == 0)))
            return (int)hipErrorInvalidValue;
        vec = vec && ((uintptr_t)a->A[m] & 15) == 0;
        rows += a->M[m];
    }
    if (rows > (1LL << 30)) return (int)hipErrorInvalidValue;
    // the vector path addresses each matrix through a 32-bit byte offset
    for (int m = 0; m < a->n_mat; m++) vec = vec && (long long)a->M[m] * a->K * 2 < (1LL << 32);
    hipStream_t st = (hipStream_t)stream;
    if (a->mode == G3K_MV_GEGLU) {
        if (a->n_mat != 2 || a->M[0] != a->M[1]) return (int)hipErrorInvalidValue;
        return (int)(vec ? launch<2, 2, true, true, true>(a, st) : launch<2, 1, false, true, true>(a, st));
    }
    if (a->mode != 0) return (int)hipErrorInvalidValue;
    if (!vec) return (int)(rows >= 16384 ? launch<2, 1, false>(a, st) : launch<1, 1, false>(a, st));
    // two rows per wave once there are enough rows to fill the chip with them
    if (rows >= 16384) return (int)launch<2, 8, true>(a, st);
    // long rows: the row's chunks split over the workgroup's waves (5 per lane at K = 10240)
    if (a->K >= 8192) return (int)launch<2, 5, true, true>(a, st);
    if (a->K <= 2048) return (int)launch<2, 2, true, true>(a, st);
    return (int)launch<1, 8, true>(a, st);
}
