// decode.hip - split-K flash-decoding GQA attention over the fp32 KV cache.
//
// Replaces, for one token and one layer, the attention section of
// layer_attention (gemma3_transformer.c:294-352): QK-RMSNorm
// (gemma3_kernels.c:289-304), RoPE from the precomputed table (:470-484),
// cache_kv (gemma3_transformer.c:236-251) and gemma3_gqa (gemma3_kernels.c:527-597).
// The same kernel without the fused front end serves the gemma3_gqa-shaped
// entry point (q already final, cache given, optional additive mask).
//
// Work decomposition (one launch):
//   grid (n_splits, n_kv_heads), 256 threads = 4 wave64.  A workgroup owns one
//   KV head and one contiguous run of rows_per_split attention indices, and
//   serves all `group` query heads of that KV head, so every K/V byte is read
//   from HBM once per call (the reference reads each row once per query head).
//   Lane layout inside a wave: 4 lane-groups of 16 lanes; a lane-group holds
//   one cache row per sub-step, lane c covering dims c*4 + 64*j + e (j, e < 4),
//   so one load instruction moves 4 rows x 256 contiguous bytes (dwordx4), and
//   the RoPE partner dim i+128 (j+2) lives in the same lane.
//   Per step a wave streams 16 consecutive rows (16 KiB of K + 16 KiB of V).
//   Dot products reduce over 16 lanes with four DPP adds; the running max is
//   kept per query head and wave-uniform (two cross-group shuffles per step).
//   Softmax runs in the exp2 domain: q is pre-scaled by scale*log2(e).
//   Waves merge through LDS; workgroups write (m, l, acc) partials and the
//   last workgroup of each KV head (atomic counter, self-resetting) combines.
#include <hip/hip_runtime.h>

#include "g3k.h"
#include "g3k_device.h"

namespace {

using namespace g3k;

constexpr int D = G3K_HEAD_DIM;
constexpr int NT = 256;               // threads per workgroup
constexpr int NW = NT / 64;           // waves per workgroup
constexpr int ROWS_PER_WAVE_STEP = 16;
constexpr float NEG_BIG = -1.0e30f;   // "no row seen yet": finite so exp2 never sees inf - inf

// x: this lane's 16 dims of one 256-vector (lane c: dims c*4 + 64j + e).
// RMSNorm with (1 + w) gain (gemma3_kernels.c:289-304), then the NeoX
// half-split rotation from the table row (gemma3_kernels.c:470-484).
__device__ __forceinline__ void norm_rope16(float (&x)[4][4], const uint16_t *w, float eps,
                                            const float (&cs)[2][4], const float (&sn)[2][4], int c) {
    if (w) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) ss += x[j][e] * x[j][e];
        ss = row16_sum(ss);
        const float r = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint2 wb = *reinterpret_cast<const uint2 *>(w + c * 4 + 64 * j);
            const float g0 = 1.0f + bf16f(wb.x & 0xffff), g1 = 1.0f + bf16f(wb.x >> 16);
            const float g2 = 1.0f + bf16f(wb.y & 0xffff), g3 = 1.0f + bf16f(wb.y >> 16);
            x[j][0] = x[j][0] * r * g0;
            x[j][1] = x[j][1] * r * g1;
            x[j][2] = x[j][2] * r * g2;
            x[j][3] = x[j][3] * r * g3;
        }
    }
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float a = x[j][e], b = x[j + 2][e];
            x[j][e] = a * cs[j][e] - b * sn[j][e];
            x[j + 2][e] = a * sn[j][e] + b * cs[j][e];
        }
}

__device__ __forceinline__ void load16(float (&x)[4][4], const float *src, int c) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float4 t = *reinterpret_cast<const float4 *>(src + c * 4 + 64 * j);
        x[j][0] = t.x; x[j][1] = t.y; x[j][2] = t.z; x[j][3] = t.w;
    }
}

__device__ __forceinline__ void store16(float *dst, const float (&x)[4][4], int c) {
#pragma unroll
    for (int j = 0; j < 4; j++)
        *reinterpret_cast<float4 *>(dst + c * 4 + 64 * j) = make_float4(x[j][0], x[j][1], x[j][2], x[j][3]);
}

template <int G, bool FUSED>
__global__ __launch_bounds__(NT, 2) void decode_kernel(g3k_decode_args p) {
    const int split = blockIdx.x, kvh = blockIdx.y;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, grp = lane >> 4, c = lane & 15;

    __shared__ float s_acc[NW][G][D];
    __shared__ float s_m[NW][G], s_l[NW][G];
    __shared__ float s_ml[G3K_MAX_SPLITS * G * 2];
    __shared__ unsigned s_last;

    // ---- query: this lane's 16 dims of each of the G query heads ----
    float qv[G][4][4];
    float cs[2][4], sn[2][4];
    if (FUSED) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const float4 a = *reinterpret_cast<const float4 *>(p.rope_row + 2 * (c * 4 + 64 * j));
            const float4 b = *reinterpret_cast<const float4 *>(p.rope_row + 2 * (c * 4 + 64 * j) + 4);
            cs[j][0] = a.x; sn[j][0] = a.y; cs[j][1] = a.z; sn[j][1] = a.w;
            cs[j][2] = b.x; sn[j][2] = b.y; cs[j][3] = b.z; sn[j][3] = b.w;
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
        load16(qv[g], p.q + (size_t)(kvh * G + g) * D, c);
        if (FUSED) norm_rope16(qv[g], p.k_norm ? p.q_norm : nullptr, p.eps, cs, sn, c);
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) qv[g][j][e] *= p.qscale;
    }

    float m[G], l[G], acc[G][4][4];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = NEG_BIG;
        l[g] = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[g][j][e] = 0.f;
    }

    float *kbase = p.kc + (size_t)kvh * p.head_stride;
    float *vbase = p.vc + (size_t)kvh * p.head_stride;

    // ---- the new token (fused decode): split 0, wave 0 seeds its state with it ----
    if (FUSED && split == 0 && wave == 0) {
        float kn[4][4], vn[4][4];
        load16(kn, p.k_new + (size_t)kvh * D, c);
        load16(vn, p.v_new + (size_t)kvh * D, c);
        norm_rope16(kn, p.q_norm ? p.k_norm : nullptr, p.eps, cs, sn, c);
        if (grp == 0) {
            store16(kbase + (size_t)p.new_slot * p.row_stride, kn, c);
            store16(vbase + (size_t)p.new_slot * p.row_stride, vn, c);
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int e = 0; e < 4; e++) s += qv[g][j][e] * kn[j][e];
            m[g] = row16_sum(s);
            if (grp == 0) {
                l[g] = 1.f;
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[g][j][e] = vn[j][e];
            }
        }
    }

    // ---- stream this split's rows ----
    const int c0 = split * p.rows_per_split;
    const int c1 = min(c0 + p.rows_per_split, p.n_stream);
    for (int base = c0 + wave * ROWS_PER_WAVE_STEP; base < c1; base += NW * ROWS_PER_WAVE_STEP) {
        const int base_row = base + (base >= p.skip);
        float kk[4][4][4], vv[4][4][4];
        bool valid[4];
        int idx[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            idx[r] = base + grp * 4 + r;
            valid[r] = idx[r] < c1;
            const int row = valid[r] ? idx[r] + (idx[r] >= p.skip) : base_row;
            load16(kk[r], kbase + (size_t)row * p.row_stride, c);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = valid[r] ? idx[r] + (idx[r] >= p.skip) : base_row;
            load16(vv[r], vbase + (size_t)row * p.row_stride, c);
        }
        float s[G][4];
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float d = 0.f;
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int e = 0; e < 4; e++) d += qv[g][j][e] * kk[r][j][e];
                s[g][r] = row16_sum(d);
            }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float add = 0.f;
            if (!FUSED && p.mask && valid[r]) add = p.mask[idx[r]] * 1.4426950408889634f;
#pragma unroll
            for (int g = 0; g < G; g++) s[g][r] = valid[r] ? s[g][r] + add : -INFINITY;
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            float mx = fmaxf(fmaxf(s[g][0], s[g][1]), fmaxf(s[g][2], s[g][3]));
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float mn = fmaxf(m[g], mx);
            const float alpha = fast_exp2(m[g] - mn);
            m[g] = mn;
            float pr[4];
#pragma unroll
            for (int r = 0; r < 4; r++) pr[r] = fast_exp2(s[g][r] - mn);
            l[g] = l[g] * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float a = acc[g][j][e] * alpha;
#pragma unroll
                    for (int r = 0; r < 4; r++) a += pr[r] * vv[r][j][e];
                    acc[g][j][e] = a;
                }
        }
    }

    // ---- merge the four lane-groups of each wave (they share m) ----
#pragma unroll
    for (int g = 0; g < G; g++) {
        l[g] += __shfl_xor(l[g], 16);
        l[g] += __shfl_xor(l[g], 32);
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float a = acc[g][j][e];
                a += __shfl_xor(a, 16);
                a += __shfl_xor(a, 32);
                acc[g][j][e] = a;
            }
    }
    if (grp == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) store16(&s_acc[wave][g][0], acc[g], c);
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            s_m[wave][g] = m[g];
            s_l[wave][g] = l[g];
        }
    }
    __syncthreads();

    // ---- merge the waves: this workgroup's (m, l, acc) per query head ----
    const bool single = p.n_splits == 1;
    for (int e = tid; e < G * D; e += NT) {
        const int g = e / D, d = e % D;
        float M = s_m[0][g];
#pragma unroll
        for (int w = 1; w < NW; w++) M = fmaxf(M, s_m[w][g]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = fast_exp2(s_m[w][g] - M);
            L += s_l[w][g] * f;
            A += s_acc[w][g][d] * f;
        }
        if (single) {
            p.out[(size_t)(kvh * G + g) * D + d] = A / L;
        } else {
            const size_t slot = ((size_t)kvh * p.n_splits + split) * G + g;
            p.ws_acc[slot * D + d] = A;
            if (d == 0) {
                p.ws_ml[slot * 2] = M;
                p.ws_ml[slot * 2 + 1] = L;
            }
        }
    }
    if (single) return;

    // ---- last workgroup of this KV head combines all splits ----
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(&p.counters[kvh], 1u) == (unsigned)(p.n_splits - 1);
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const int S = p.n_splits;
    const float *ml = p.ws_ml + (size_t)kvh * S * G * 2;
    for (int i = tid; i < S * G * 2; i += NT) s_ml[i] = __builtin_nontemporal_load(ml + i);
    __syncthreads();
    for (int e = tid; e < G * D; e += NT) {
        const int g = e / D, d = e % D;
        float M = NEG_BIG;
        for (int s = 0; s < S; s++) M = fmaxf(M, s_ml[(s * G + g) * 2]);
        float L = 0.f, A = 0.f;
        const float *src = p.ws_acc + ((size_t)kvh * S * G + g) * D + d;
#pragma unroll 8
        for (int s = 0; s < S; s++) {
            const float f = fast_exp2(s_ml[(s * G + g) * 2] - M);
            L += s_ml[(s * G + g) * 2 + 1] * f;
            A += __builtin_nontemporal_load(src + (size_t)s * G * D) * f;
        }
        p.out[(size_t)(kvh * G + g) * D + d] = A / L;
    }
    if (tid == 0) atomicExch(&p.counters[kvh], 0u);
}

template <int G, bool FUSED>
hipError_t launch(const g3k_decode_args *a, hipStream_t st) {
    dim3 grid(a->n_splits, a->n_kv_heads);
    hipLaunchKernelGGL((decode_kernel<G, FUSED>), grid, dim3(NT), 0, st, *a);
    return hipGetLastError();
}

}  // namespace

extern "C" int g3k_decode(const g3k_decode_args *a, int fused, void *stream) {
    hipStream_t st = (hipStream_t)stream;
    if (a->n_splits < 1 || a->n_splits > G3K_MAX_SPLITS || a->rows_per_split % 64) return (int)hipErrorInvalidValue;
    switch (a->group) {
        case 1: return (int)(fused ? launch<1, true>(a, st) : launch<1, false>(a, st));
        case 2: return (int)(fused ? launch<2, true>(a, st) : launch<2, false>(a, st));
        case 4: return (int)(fused ? launch<4, true>(a, st) : launch<4, false>(a, st));
        default: return (int)hipErrorInvalidValue;
    }
}
