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
//   Per step a wave streams 4*R consecutive rows (R rows per lane-group).
//   Dot products reduce over 16 lanes with four DPP adds; the running max is
//   kept per query head and wave-uniform (two cross-group shuffles per step).
//   Softmax runs in the exp2 domain: q is pre-scaled by scale*log2(e).
//   Waves merge through LDS; with more than one split each workgroup writes
//   an (m, l, acc) partial and a second small launch (combine_kernel)
//   merges them.
//
// One-launch form (XM, local layers: <= 32 splits): the grid is ordered so
// that all splits of one run of query heads have workgroup ids equal mod 8,
// which the MI355X dispatcher places on one XCD (the host checks this with
// a probe launch per context).  Each split's partial then lands in that
// XCD's L2, the last workgroup to count itself in the run's L2 counter
// merges the run's partials from there, and no combine launch follows.  With
// 4 KV heads the 8 runs are the 8 query heads (one head per workgroup), so
// every XCD takes part and each KV head's window is read twice.  A merge at
// the device's point of coherence instead (agent-scope stores, counter and
// loads, any placement) was measured slower than the second launch.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <pthread.h>
#include <type_traits>

#include "g3k.h"
#include "g3k_device.h"

namespace {

using namespace g3k;

constexpr int D = G3K_HEAD_DIM;
constexpr int NT = 256;               // threads per workgroup
constexpr int NW = NT / 64;           // waves per workgroup
// Rows per lane-group per step (a wave step covers 4*R rows); G = 4 keeps
// one row so its larger q / acc arrays fit without spills.  Only the R
// values below are built for the GPU.  The source is generic in R: its host
// build (tests/hostemu) matches the oracle at R = 1..4.  gfx950 builds at
// R = 3 and R = 4 return wrong outputs from -O2 up; bisecting the device
// passes puts the change at si-form-memory-clauses, and with
// -mllvm -amdgpu-max-memory-clause=1 both are correct, but no faster than
// R = 2 (measured), so they are not built.
#ifdef G3K_DECODE_ROWS
// Host-emulation builds of this file (tests/hostemu) set one R for every
// group, to run the other R values on the CPU; GPU builds never define it.
template <int G> constexpr int rows_for() { return G3K_DECODE_ROWS; }
#else
template <int G> constexpr int rows_for() { return G >= 4 ? 1 : 2; }
#endif
#ifndef G3K_DECODE_DB
#define G3K_DECODE_DB 1   // double-buffered row steps at group <= 2 (see the row loop); 0: single set
#endif
constexpr float NEG_BIG = -1.0e30f;  // "no row seen yet": finite so exp2 never sees inf - inf
// Measured on MI355X: two workgroups per CU (<= 256 VGPRs), one 8-row step
// in flight per wave, one contiguous row range per split.  Double-buffered
// steps, three workgroups per CU and block-cyclic row assignment were each
// slower or no faster at both 8K and 128K.

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


// One cache row's 16 dims of this lane.
__device__ __forceinline__ void load16_stream(float (&x)[4][4], const float *src, int c) { load16(x, src, c); }

// The same through a buffer descriptor with the non-temporal cache policy
// (the context-owned cache: streamed once per call, not worth keeping in
// L2).  rs covers one KV head's rows; voff = the row's byte offset + 16 c.
__device__ __forceinline__ void load16_nt(float (&x)[4][4], __amdgpu_buffer_rsrc_t rs, unsigned voff) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float4 t = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 256 * j, 0, 2));
        x[j][0] = t.x; x[j][1] = t.y; x[j][2] = t.z; x[j][3] = t.w;
    }
}

// Buffer descriptor over one KV head's cache rows (bytes < 2^32).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_rsrc(const float *base, long long head_stride) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, (int)(head_stride * 4), 0x00020000);
}

template <int R, bool NTL>
__device__ __forceinline__ void load_step(float (&kk)[R][4][4], float (&vv)[R][4][4],
                                          const float *kbase, const float *vbase, long long rs,
                                          long long head_stride, int base, int c1, int skip, int grp, int c) {
    const int base_row = base + (base >= skip);
    int rows[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int idx = base + grp * R + r;
        rows[r] = idx < c1 ? idx + (idx >= skip) : base_row;
    }
    if (NTL) {
        const __amdgpu_buffer_rsrc_t kr = head_rsrc(kbase, head_stride), vr = head_rsrc(vbase, head_stride);
#pragma unroll
        for (int r = 0; r < R; r++) load16_nt(kk[r], kr, (unsigned)(rows[r] * rs * 4) + 16 * c);
#pragma unroll
        for (int r = 0; r < R; r++) load16_nt(vv[r], vr, (unsigned)(rows[r] * rs * 4) + 16 * c);
    } else {
#pragma unroll
        for (int r = 0; r < R; r++) load16_stream(kk[r], kbase + (size_t)rows[r] * rs, c);
#pragma unroll
        for (int r = 0; r < R; r++) load16_stream(vv[r], vbase + (size_t)rows[r] * rs, c);
    }
}

// One step: scores of this lane-group's R rows for the G query heads (16-lane
// DPP reduction), online-softmax update with a wave-uniform running max, and
// the P.V accumulation.
template <int G, int R, bool FUSED>
__device__ __forceinline__ void step_compute(const float (&kk)[R][4][4], const float (&vv)[R][4][4],
                                             const float (&qv)[G][4][4], float (&m)[G], float (&l)[G],
                                             float (&acc)[G][4][4], int base, int c1, int grp,
                                             const float *mask) {
    bool valid[R];
    int idx[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        idx[r] = base + grp * R + r;
        valid[r] = idx[r] < c1;
    }
    float s[G][R];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int r = 0; r < R; r++) {
            float d = 0.f;
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int e = 0; e < 4; e++) d += qv[g][j][e] * kk[r][j][e];
            s[g][r] = row16_sum(d);
        }
#pragma unroll
    for (int r = 0; r < R; r++) {
        float add = 0.f;
        if (!FUSED && mask && valid[r]) add = mask[idx[r]] * 1.4426950408889634f;
#pragma unroll
        for (int g = 0; g < G; g++) s[g][r] = valid[r] ? s[g][r] + add : -INFINITY;
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
        float mx = s[g][0];
#pragma unroll
        for (int r = 1; r < R; r++) mx = fmaxf(mx, s[g][r]);
        mx = col4_max(mx);
        const float mn = fmaxf(m[g], mx);
        const float alpha = fast_exp2(m[g] - mn);
        m[g] = mn;
        float pr[R], psum = 0.f;
#pragma unroll
        for (int r = 0; r < R; r++) {
            pr[r] = fast_exp2(s[g][r] - mn);
            psum += pr[r];
        }
        l[g] = l[g] * alpha + psum;
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float a = acc[g][j][e] * alpha;
#pragma unroll
                for (int r = 0; r < R; r++) a += pr[r] * vv[r][j][e];
                acc[g][j][e] = a;
            }
    }
}

// (M, L, A) <- merge of two online-softmax partials
__device__ __forceinline__ void merge_ml(float &M, float &L, float4 &A, float m2, float l2, float4 a2) {
    const float Mn = fmaxf(M, m2);
    const float f1 = fast_exp2(M - Mn), f2 = fast_exp2(m2 - Mn);
    L = L * f1 + l2 * f2;
    A.x = A.x * f1 + a2.x * f2;
    A.y = A.y * f1 + a2.y * f2;
    A.z = A.z * f1 + a2.z * f2;
    A.w = A.w * f1 + a2.w * f2;
    M = Mn;
}

// (M, L, A) <- the merge of the partials of lanes l and l ^ X (X = 16 or 32),
// lower lane first, through v_permlane{16,32}_swap.
template <int X>
__device__ __forceinline__ void swap_merge(float &M, float &L, float4 &A) {
    auto sw = [](float v) {
        const auto r = X == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false)
                               : __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
    };
    const float2 m = sw(M), l = sw(L), ax = sw(A.x), ay = sw(A.y), az = sw(A.z), aw = sw(A.w);
    M = m.x;
    L = l.x;
    A = make_float4(ax.x, ay.x, az.x, aw.x);
    merge_ml(M, L, A, m.y, l.y, make_float4(ax.y, ay.y, az.y, aw.y));
}

// The one-launch form's merge of a run's n_splits (<= G3K_XM_MAX_SPLITS)
// partials, in split order: out = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M)
// l_s.  Thread t owns dim t of each of the G heads (NT == D); all of a
// head's partial loads are issued at once (one L2 round trip).  Splits past
// n_splits read the last split's partial and weigh it 0.
template <int G>
__device__ __forceinline__ void xm_merge(const g3k_decode_args &p, int kvh, int gq0, int GF, int tid) {
    static_assert(NT == D, "one thread per dim");
    const int S = p.n_splits;
    constexpr int CP_SC0 = 1;   // cache policy: bypass the L1
#pragma unroll
    for (int g = 0; g < G; g++) {
        const int h = gq0 + g;
        // run h's partial of split s: ws_acc[((kvh * MAX + s) * GF + h) * D + d]
        const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
            p.ws_acc + ((size_t)kvh * G3K_MAX_SPLITS * GF + h) * D, (short)0, S * GF * D * 4, 0x00020000);
        const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
            p.ws_ml + ((size_t)kvh * G3K_MAX_SPLITS * GF + h) * 2, (short)0, S * GF * 2 * 4, 0x00020000);
        uint32_t a[G3K_XM_MAX_SPLITS], ml[G3K_XM_MAX_SPLITS][2];
#pragma unroll
        for (int s = 0; s < G3K_XM_MAX_SPLITS; s++) {
            const int sc = s < S ? s : S - 1;
            a[s] = __builtin_amdgcn_raw_buffer_load_b32(ra, (unsigned)((sc * GF * D + tid) * 4), 0, CP_SC0);
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(rm, (unsigned)(sc * GF * 2 * 4), 0, CP_SC0);
            ml[s][0] = v[0];
            ml[s][1] = v[1];
        }
        // every load above is issued before the first use below
        __builtin_amdgcn_sched_barrier(0);
        float ms[G3K_XM_MAX_SPLITS];
#pragma unroll
        for (int s = 0; s < G3K_XM_MAX_SPLITS; s++) ms[s] = s < S ? __uint_as_float(ml[s][0]) : NEG_BIG;
        float M = ms[0];
#pragma unroll
        for (int s = 1; s < G3K_XM_MAX_SPLITS; s++) M = fmaxf(M, ms[s]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int s = 0; s < G3K_XM_MAX_SPLITS; s++) {
            const float f = fast_exp2(ms[s] - M);
            L += __uint_as_float(ml[s][1]) * f;
            A += __uint_as_float(a[s]) * f;
        }
        p.out[(size_t)(kvh * GF + h) * D + tid] = A / L;
    }
}

template <int G, bool FUSED, bool NTL, bool XM>
__global__ __launch_bounds__(NT, 2) void decode_kernel(g3k_decode_args p) {
    constexpr int R = rows_for<G>();
    constexpr int ROWS_PER_WAVE_STEP = 4 * R;
    // Two-launch form: grid (n_splits, H_kv), the workgroup serves all G query
    // heads of its KV head.  One-launch form (XM): a 1-D grid of PP * n_splits
    // workgroups for P = H_kv * GF / G runs of G query heads (the group GF
    // split into runs), PP = P rounded up to a multiple of 8; run pg of split
    // s is workgroup s * PP + pg, so every split of a run has the same id
    // mod 8.  Workgroups pg >= P have no run and end at once.
    const int GF = XM ? p.group : G;
    int split, kvh, gq0, pg = 0;
    if constexpr (XM) {
        const int runs = GF / G, P = p.n_kv_heads * runs, PP = (P + 7) & ~7;
        pg = (int)blockIdx.x % PP;
        if (pg >= P) return;
        split = (int)blockIdx.x / PP;
        kvh = pg / runs;
        gq0 = (pg % runs) * G;
    } else {
        split = blockIdx.x;
        kvh = blockIdx.y;
        gq0 = 0;
    }
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, grp = lane >> 4, c = lane & 15;

    // the partials of every lane-group (four per wave) for the merge
    __shared__ float s_acc[4 * NW][G * D];
    __shared__ float s_m[NW][G], s_l[4 * NW][G];

    const float *kbase = p.kc + (size_t)kvh * p.head_stride;
    const float *vbase = p.vc + (size_t)kvh * p.head_stride;
    const int c0 = split * p.rows_per_split;
    const int c1 = min(c0 + p.rows_per_split, p.n_stream);
    const int stride = NW * ROWS_PER_WAVE_STEP;

    // ---- first step's K/V loads go out before the query prologue ----
    float kk[R][4][4], vv[R][4][4];
    int base = c0 + wave * ROWS_PER_WAVE_STEP;
    if (base < c1) load_step<R, NTL>(kk, vv, kbase, vbase, p.row_stride, p.head_stride, base, c1, p.skip, grp, c);
    // the new token's k / v (split 0, wave 0) are in flight during the prologue too
    const bool seeds = FUSED && split == 0 && wave == 0;
    float kn[4][4], vn[4][4];
    if (seeds) {
        load16(kn, p.k_new + (size_t)kvh * D, c);
        load16(vn, p.v_new + (size_t)kvh * D, c);
    }

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
        load16(qv[g], p.q + (size_t)(kvh * GF + gq0 + g) * D, c);
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

    // ---- the new token (fused decode): split 0, wave 0 seeds its state with it ----
    if (seeds) {
        norm_rope16(kn, p.q_norm ? p.k_norm : nullptr, p.eps, cs, sn, c);
        if (grp == 0 && gq0 == 0) {   // one writer per KV head
            store16(p.kc + (size_t)kvh * p.head_stride + (size_t)p.new_slot * p.row_stride, kn, c);
            store16(p.vc + (size_t)kvh * p.head_stride + (size_t)p.new_slot * p.row_stride, vn, c);
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
    // Double-buffered row steps where the registers allow them (group <= 2;
    // at group 4 the second set spilled to scratch)
    constexpr bool DB = G3K_DECODE_DB && G <= 2;
    if constexpr (DB) {
    // Two register sets: the next step's loads are issued before the current
    // step is reduced, so each wave keeps a step in flight while it computes.
    // The last step is peeled, so every load in the loop body is
    // unconditional and the waits before each reduction count exactly the
    // next step's loads.
    if (base < c1) {
        float kk2[R][4][4], vv2[R][4][4];
        for (;;) {
            int nb = base + stride;
            if (nb >= c1) {
                step_compute<G, R, FUSED>(kk, vv, qv, m, l, acc, base, c1, grp, p.mask);
                break;
            }
            load_step<R, NTL>(kk2, vv2, kbase, vbase, p.row_stride, p.head_stride, nb, c1, p.skip, grp, c);
            __builtin_amdgcn_sched_barrier(0);   // the loads go out before the reduction
            step_compute<G, R, FUSED>(kk, vv, qv, m, l, acc, base, c1, grp, p.mask);
            base = nb;
            nb = base + stride;
            if (nb >= c1) {
                step_compute<G, R, FUSED>(kk2, vv2, qv, m, l, acc, base, c1, grp, p.mask);
                break;
            }
            load_step<R, NTL>(kk, vv, kbase, vbase, p.row_stride, p.head_stride, nb, c1, p.skip, grp, c);
            __builtin_amdgcn_sched_barrier(0);
            step_compute<G, R, FUSED>(kk2, vv2, qv, m, l, acc, base, c1, grp, p.mask);
            base = nb;
        }
    }
    } else {
    // reduce the loaded step, then load the next
    while (base < c1) {
        step_compute<G, R, FUSED>(kk, vv, qv, m, l, acc, base, c1, grp, p.mask);
        base += stride;
        if (base < c1) load_step<R, NTL>(kk, vv, kbase, vbase, p.row_stride, p.head_stride, base, c1, p.skip, grp, c);
    }
    }

    // ---- every lane-group's (l, acc) to LDS as it is (the four groups of a
    // wave share m, so the merge below only adds them; adding them across lanes
    // first, with permlane swaps, was 0.9-1 us slower per 8K decode step) ----
#pragma unroll
    for (int g = 0; g < G; g++) store16(&s_acc[4 * wave + grp][g * D], acc[g], c);
    if (c == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) s_l[4 * wave + grp][g] = l[g];
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) s_m[wave][g] = m[g];
    }
    __syncthreads();

    // ---- merge the waves: this workgroup's (m, l, acc) per query head, stored
    // straight from the merging thread (every thread of a head computes the
    // same M and L): the normalised output with one split, else this split's
    // partial ----
    float *out = p.out + (size_t)(kvh * GF + gq0) * D;
    const size_t slot = (size_t)kvh * G3K_MAX_SPLITS + split;
    for (int e = tid; e < G * D; e += NT) {
        const int g = e / D;
        float M = s_m[0][g];
#pragma unroll
        for (int w = 1; w < NW; w++) M = fmaxf(M, s_m[w][g]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = fast_exp2(s_m[w][g] - M);
            const float lw = (s_l[4 * w][g] + s_l[4 * w + 1][g]) + (s_l[4 * w + 2][g] + s_l[4 * w + 3][g]);
            const float aw = (s_acc[4 * w][e] + s_acc[4 * w + 1][e]) + (s_acc[4 * w + 2][e] + s_acc[4 * w + 3][e]);
            L += lw * f;
            A += aw * f;
        }
        if (p.n_splits == 1) {   // uniform
            out[e] = A / L;
        } else {
            p.ws_acc[(slot * GF + gq0) * D + e] = A;
            if (e % D == 0) {
                p.ws_ml[(slot * GF + gq0 + g) * 2] = M;
                p.ws_ml[(slot * GF + gq0 + g) * 2 + 1] = L;
            }
        }
    }
    if constexpr (XM) {
        if (p.n_splits == 1) return;
        // Last-arrival merge on this XCD.  Every split of this run stores its
        // partial with plain stores, which land in the XCD's L2 (the vector L1
        // writes through); the wait below (vmcnt counts stores on this family)
        // and the barrier put all of this workgroup's stores there before it
        // counts itself.  The counter is a workgroup-scope atomic, performed
        // in that same L2: the runs never span XCDs (the host checks the
        // workgroup -> XCD placement first), so the L2 orders the arrivals and
        // holds every partial, with no write-back to memory and no cache
        // invalidation.  The last to arrive resets the counter for the next
        // launch and reads the partials past its L1 (sc0 loads).
        G3K_WAIT_VMEM();
        __syncthreads();
        __shared__ int s_last;
        if (tid == 0) {
            unsigned *cnt = p.xm_count + (size_t)pg * G3K_XM_COUNTER_STRIDE;
            const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            s_last = old == (unsigned)(p.n_splits - 1);
            if (s_last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        __syncthreads();
        if (s_last) xm_merge<G>(p, kvh, gq0, GF, tid);
    }
}

// Cross-split combine, one launch after decode_kernel (kernel order makes
// the partials visible; no fences or atomics).  Each wave owns 4 dims of one
// query head and merges every split across its 64 lanes: lane l loads the
// partials of splits l, l + 64, ... at once (one memory round trip) and
// merges them in registers; the lanes then meet pairwise, l ^ 1 and l ^ 2
// (DPP quad_perm), the quads and the half-rows of a 16-lane row (DPP
// row_half_mirror, row_mirror), and the rows (v_permlane16/32_swap), all VALU:
// no LDS and no barrier.  grid (D / 16, group, H_kv), 4 waves per
// workgroup.  (A workgroup-wide form, 8 split lanes per wave and the 4 waves
// merged through LDS, took 0.55 us more per 8K decode step.)
template <int G>
__global__ __launch_bounds__(NT) void combine_kernel(g3k_decode_args p) {
    const int g = blockIdx.y, kvh = blockIdx.z;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int d = 4 * (blockIdx.x * NW + wave);
    const int S = p.n_splits;
    const size_t slot0 = (size_t)kvh * G3K_MAX_SPLITS;
    constexpr int U = G3K_MAX_SPLITS / 64;   // splits per lane, at most
    float2 mlq[U];
    float4 aq[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int s = lane + 64 * u;
        if (s < S) {
            const size_t sg = (slot0 + s) * G + g;
            mlq[u] = *reinterpret_cast<const float2 *>(p.ws_ml + sg * 2);
            aq[u] = *reinterpret_cast<const float4 *>(p.ws_acc + sg * D + d);
        } else {
            mlq[u] = make_float2(NEG_BIG, 0.f);
            aq[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    float M = NEG_BIG, L = 0.f;
    float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < U; u++) merge_ml(M, L, A, mlq[u].x, mlq[u].y, aq[u]);
    auto dpp_merge = [&](auto ctrl) {
        constexpr int C = decltype(ctrl)::value;
        float4 a2;
        const float m2 = dpp<C>(M), l2 = dpp<C>(L);
        a2.x = dpp<C>(A.x);
        a2.y = dpp<C>(A.y);
        a2.z = dpp<C>(A.z);
        a2.w = dpp<C>(A.w);
        merge_ml(M, L, A, m2, l2, a2);
    };
    dpp_merge(std::integral_constant<int, 0xB1>{});    // quad_perm [1,0,3,2]
    dpp_merge(std::integral_constant<int, 0x4E>{});    // quad_perm [2,3,0,1]
    dpp_merge(std::integral_constant<int, 0x141>{});   // row_half_mirror
    dpp_merge(std::integral_constant<int, 0x140>{});   // row_mirror
    swap_merge<16>(M, L, A);
    swap_merge<32>(M, L, A);
    // a division, as the single-split path's store: one split gives the same bits either way
    if (lane == 0)
        *reinterpret_cast<float4 *>(p.out + ((size_t)kvh * G + g) * D + d) =
            make_float4(A.x / L, A.y / L, A.z / L, A.w / L);
}

template <int G, bool FUSED, bool NTL>
hipError_t launch(const g3k_decode_args *a, hipStream_t st) {
    dim3 grid(a->n_splits, a->n_kv_heads);
    // With timing events the dispatch itself records them (kernel begin / end).
    hipExtLaunchKernelGGL((decode_kernel<G, FUSED, NTL, false>), grid, dim3(NT), 0, st, (hipEvent_t)a->ev0,
                          (hipEvent_t)a->ev1, 0, *a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a->n_splits == 1) return e;
    hipLaunchKernelGGL((combine_kernel<G>), dim3(D / (4 * NW), G, a->n_kv_heads), dim3(NT), 0, st, *a);
    return hipGetLastError();
}

// One-launch form: runs of GW query heads (GW divides the group), P = H_kv *
// group / GW runs, padded to PP, a multiple of 8.
template <int GW, bool NTL>
hipError_t launch_xm(const g3k_decode_args *a, hipStream_t st) {
    const int PP = (a->n_kv_heads * (a->group / GW) + 7) & ~7;
    hipExtLaunchKernelGGL((decode_kernel<GW, true, NTL, true>), dim3(PP * a->n_splits), dim3(NT), 0, st,
                          (hipEvent_t)a->ev0, (hipEvent_t)a->ev1, 0, *a);
    return hipGetLastError();
}

template <int G>
hipError_t launch_g(const g3k_decode_args *a, int fused, hipStream_t st) {
    if (!fused) return launch<G, false, false>(a, st);
    return a->nt_loads ? launch<G, true, true>(a, st) : launch<G, true, false>(a, st);
}

__global__ __launch_bounds__(64) void xcd_probe_kernel(unsigned *xcc, int n) {
    unsigned v = G3K_XCC_ID();
    if (threadIdx.x == 0 && (int)blockIdx.x < n) xcc[blockIdx.x] = v & 0xf;
}

template <int G, bool FUSED>
int capacity() {
    int per_cu = 0, cus = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_kernel<G, FUSED, FUSED, false>, NT, 0) != hipSuccess)
        return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return per_cu * cus;
}

}  // namespace

extern "C" int g3k_decode(const g3k_decode_args *a, int fused, void *stream) {
    hipStream_t st = (hipStream_t)stream;
    if (a->n_splits < 1 || a->n_splits > G3K_MAX_SPLITS || a->rows_per_split % G3K_SPLIT_GRAIN)
        return (int)hipErrorInvalidValue;
    if (a->xm_heads) {
        // the one-launch form: fused decode, 2..G3K_XM_MAX_SPLITS splits, runs
        // of 1 or 2 query heads dividing the group
        const int gw = a->xm_heads;
        if (!fused || !a->xm_count || a->n_splits < 2 || a->n_splits > G3K_XM_MAX_SPLITS ||
            (gw != 1 && gw != 2) || a->group % gw)
            return (int)hipErrorInvalidValue;
        if (gw == 1) return (int)(a->nt_loads ? launch_xm<1, true>(a, st) : launch_xm<1, false>(a, st));
        return (int)(a->nt_loads ? launch_xm<2, true>(a, st) : launch_xm<2, false>(a, st));
    }
    switch (a->group) {
        case 1: return (int)launch_g<1>(a, fused, st);
        case 2: return (int)launch_g<2>(a, fused, st);
        case 4: return (int)launch_g<4>(a, fused, st);
        default: return (int)hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------------------
// Fixed scratch of the allocation-free gemma3_gqa entry point: the split
// partials of up to G3K_NOALLOC_MAX_HEADS query heads x G3K_MAX_SPLITS splits
// (acc [.][D], then (max, sum) [.][2]), 4.03 MiB per device, held until the
// process ends.  Host code never passes `scratch` itself to a kernel: that
// name is a host-side stand-in, not a device address.  Each device's address
// comes from hipGetSymbolAddress, once per device with that device current.
// ---------------------------------------------------------------------------
namespace {
constexpr size_t NOALLOC_ACC = (size_t)G3K_NOALLOC_MAX_HEADS * G3K_MAX_SPLITS * D;
constexpr size_t NOALLOC_ML = (size_t)G3K_NOALLOC_MAX_HEADS * G3K_MAX_SPLITS * 2;
constexpr int NOALLOC_MAX_DEVICES = 64;
float *g_scratch_ptr[NOALLOC_MAX_DEVICES];
pthread_mutex_t g_scratch_lock = PTHREAD_MUTEX_INITIALIZER;
}  // namespace

static __device__ __align__(256) float scratch[NOALLOC_ACC + NOALLOC_ML];

extern "C" int g3k_noalloc_scratch(float **acc, float **ml) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return (int)hipErrorInvalidDevice;
    pthread_mutex_lock(&g_scratch_lock);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e == hipSuccess) g_scratch_ptr[dev] = static_cast<float *>(p);
    }
    float *base = g_scratch_ptr[dev];
    pthread_mutex_unlock(&g_scratch_lock);
    if (!base) return (int)(e != hipSuccess ? e : hipErrorInvalidSymbol);
    *acc = base;
    *ml = base + NOALLOC_ACC;
    return 0;
}

// ---------------------------------------------------------------------------
// gemma3_gqa of any shape (the fast kernels above take head_dim 256 and
// groups 1, 2, 4).  One workgroup per (split, query head), 256 threads: each
// 16-lane group takes one key row per step (lane c holds dims c + 16 j), so
// a wave scores four rows at once and reduces each dot product with four DPP
// adds; every lane group keeps its own online softmax over its rows.  The
// 16 lane groups of the workgroup then merge through LDS, per dim.
// ---------------------------------------------------------------------------
namespace {

constexpr int GEN_J = G3K_GQA_MAX_DIM / 16;   // dims per lane, at most

__global__ __launch_bounds__(NT) void gqa_generic_kernel(g3k_gqa_args a) {
    __shared__ float s_acc[16][G3K_GQA_MAX_DIM];
    __shared__ float s_m[16], s_l[16];
    const int split = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x, grp = tid >> 4, c = tid & 15;   // 16 lane groups of the workgroup
    const int hd = a.head_dim;
    const int kvh = h / (a.n_heads / a.n_kv_heads);
    const long long rs = (long long)a.n_kv_heads * hd;
    float qv[GEN_J], acc[GEN_J];
#pragma unroll
    for (int j = 0; j < GEN_J; j++) {
        const int d = c + 16 * j;
        qv[j] = d < hd ? a.q[(size_t)h * hd + d] * a.qscale : 0.f;
        acc[j] = 0.f;
    }
    float m = NEG_BIG, l = 0.f;
    const int c0 = split * a.rows_per_split, c1 = min(c0 + a.rows_per_split, a.seq_len);
    // wave-uniform trip count (the DPP reduction needs every lane of the
    // wave); a lane group past the split's end scores -inf and adds nothing
    for (int base = c0; base < c1; base += 16) {
        const int row = base + grp;
        const bool valid = row < c1;
        const int r = valid ? row : c0;
        const float *kr = a.k + (size_t)r * rs + (size_t)kvh * hd;
        const float *vr = a.v + (size_t)r * rs + (size_t)kvh * hd;
        float dot = 0.f;
#pragma unroll
        for (int j = 0; j < GEN_J; j++) {
            const int d = c + 16 * j;
            if (d < hd) dot += qv[j] * kr[d];
        }
        float sc = row16_sum(dot);
        if (a.mask) sc += a.mask[r] * 1.4426950408889634f;
        sc = valid ? sc : -INFINITY;
        const float mn = fmaxf(m, sc);
        const float alpha = fast_exp2(m - mn), pr = fast_exp2(sc - mn);
        m = mn;
        l = l * alpha + pr;
#pragma unroll
        for (int j = 0; j < GEN_J; j++) {
            const int d = c + 16 * j;
            acc[j] = acc[j] * alpha + (d < hd ? pr * vr[d] : 0.f);
        }
    }
    // lane groups whose rows were all masked to -inf keep m = -inf: their
    // weight below is exp2(-inf - M) = 0 (M is finite when any row is)
#pragma unroll
    for (int j = 0; j < GEN_J; j++) {
        const int d = c + 16 * j;
        if (d < hd) s_acc[grp][d] = acc[j];
    }
    if (c == 0) {
        s_m[grp] = m;
        s_l[grp] = l;
    }
    __syncthreads();
    float M = s_m[0];
    for (int g = 1; g < 16; g++) M = fmaxf(M, s_m[g]);
    float L = 0.f;
    for (int g = 0; g < 16; g++) L += s_l[g] * fast_exp2(s_m[g] - M);
    const size_t slot = (size_t)h * a.n_splits + split;
    for (int d = tid; d < hd; d += NT) {
        float A = 0.f;
        for (int g = 0; g < 16; g++) A += s_acc[g][d] * fast_exp2(s_m[g] - M);
        if (a.n_splits == 1)
            a.out[(size_t)h * hd + d] = A / L;
        else
            a.ws_acc[slot * hd + d] = A;
    }
    if (a.n_splits > 1 && tid == 0) {
        a.ws_ml[slot * 2] = M;
        a.ws_ml[slot * 2 + 1] = L;
    }
}

// The splits' partials of one query head, merged in split order per dim.
__global__ __launch_bounds__(NT) void gqa_generic_combine_kernel(g3k_gqa_args a) {
    const int h = blockIdx.x, hd = a.head_dim, S = a.n_splits;
    const size_t s0 = (size_t)h * S;
    float M = NEG_BIG;
    for (int s = 0; s < S; s++) M = fmaxf(M, a.ws_ml[(s0 + s) * 2]);
    float L = 0.f;
    for (int s = 0; s < S; s++) L += a.ws_ml[(s0 + s) * 2 + 1] * fast_exp2(a.ws_ml[(s0 + s) * 2] - M);
    for (int d = threadIdx.x; d < hd; d += NT) {
        float A = 0.f;
        for (int s = 0; s < S; s++) A += a.ws_acc[(s0 + s) * hd + d] * fast_exp2(a.ws_ml[(s0 + s) * 2] - M);
        a.out[(size_t)h * hd + d] = A / L;
    }
}

}  // namespace

extern "C" int g3k_gqa_generic(const g3k_gqa_args *a, void *stream) {
    if (a->n_heads < 1 || a->n_kv_heads < 1 || a->n_heads % a->n_kv_heads || a->seq_len < 1 ||
        a->head_dim < 1 || a->head_dim > G3K_GQA_MAX_DIM || a->n_splits < 1 || a->rows_per_split < 1 ||
        (long long)a->n_splits * a->rows_per_split < a->seq_len || (a->n_splits > 1 && (!a->ws_acc || !a->ws_ml)))
        return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(gqa_generic_kernel, dim3(a->n_splits, a->n_heads), dim3(NT), 0, st, *a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a->n_splits == 1) return (int)e;
    hipLaunchKernelGGL(gqa_generic_combine_kernel, dim3(a->n_heads), dim3(NT), 0, st, *a);
    return (int)hipGetLastError();
}

extern "C" int g3k_xcd_probe(unsigned *xcc, int n, void *stream) {
    if (n < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(xcd_probe_kernel, dim3(n), dim3(64), 0, (hipStream_t)stream, xcc, n);
    return (int)hipGetLastError();
}

extern "C" int g3k_decode_capacity(int group, int fused) {
    switch (group) {
        case 1: return fused ? capacity<1, true>() : capacity<1, false>();
        case 2: return fused ? capacity<2, true>() : capacity<2, false>();
        case 4: return fused ? capacity<4, true>() : capacity<4, false>();
        default: return 0;
    }
}
