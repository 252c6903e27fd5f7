// prefill.hip - causal / sliding-window prefill attention on MFMA (gfx950).
//
// Replaces the per-token attention loop of the reference prefill
// (gemma3_transformer.c:641-692; gemma3_gqa at :689-691): every token i of the
// batch attends the keys of positions [pos - window + 1, pos] (local layer)
// or [0, pos] (global layer), pos = start_pos + i, with the reference's
// softmax (gemma3_kernels.c:396-415) and scale 1/sqrt(head_dim).
//
// Precision policy.  Post-RoPE q and k are fp32 and not representable in
// any MFMA input format, and the path is held to max-abs error <= 2e-3 x
// output RMS.  A single bf16 or fp16 pass misses that bar by 5-60x on the
// early causal rows, so:
//   S = q.k   as three fp16 MFMA passes  q_hi.k_hi + q_lo.k_hi + q_hi.k_lo,
//             x_hi = fp16(x), x_lo = fp16(x - x_hi)  (about 22 bits);
//   O = P.V   as two bf16 MFMA passes    P_hi.V + P_lo.V  (16 bits of P),
//             V in bf16, exact for the bf16-valued inputs the path is
//             specified on; fp32 accumulation throughout.
// That is 2.5x the algorithmic MFMA work.
//
// Data flow.  One workgroup = 8 wave64 = one KV head x 32*4/G query
// positions of each of its G query heads.  Waves work in pairs on 32 queries
// of one head; wave 2p+e owns the head-dim half e (128 dims) of them:
//   partial S^T[key][query] = K[:, half] . Q[:, half]^T with
//     v_mfma_f32_32x32x16_f16: A = K tile rows from LDS, B = the wave's Q^T
//     fragments in registers (hi / lo: 64 VGPRs);
//   the pair adds its two partial S^T tiles through LDS (4 KiB per wave), both
//     waves run the same softmax;
//   O^T[dim in half][query] += V^T . P^T with v_mfma_f32_32x32x16_bf16: A = V^T
//     tile rows from LDS, B = P straight from the S^T registers (O^T: 64 regs).
// Splitting the head dim keeps each wave near 200 registers (two waves per
// SIMD) while every K / V byte staged in LDS still serves 32 queries per MFMA.
// In the 32x32 accumulator layout lane l holds column (query) l % 32, so the
// softmax row statistics of a query live in one lane pair (l, l ^ 32) and the
// O^T rescale is lane-local.  K rows are fed to the MFMA in the order
// key(m) = m with bits 2 and 3 swapped; then accumulator register r of lane
// half h holds key 16*(r/8) + 8*h + r%8, which is exactly the B-operand
// order of the P.V MFMA (no shuffles between the two products).
// Key tiles of 32 are double-buffered in LDS and fetched one tile ahead with
// gfx950's direct global->LDS loads (global_load_lds_dwordx4: no staging
// registers; each wave instruction fills 1 KiB of LDS in lane order):
// K_hi, K_lo [32][256] fp16 and V^T [256][32] bf16, unpadded, with the 16-byte
// chunks of each row XOR-swizzled so that the MFMA fragment reads
// (ds_read_b128) hit distinct bank groups.  Two barriers per tile (partial-S
// exchange, stage hand-over).
// Softmax runs in the exp2 domain (q pre-scaled by scale*log2(e)) with a
// lazy running max: O and l are rescaled only when a tile's max exceeds the
// reference max by more than 2^8.
#include <hip/hip_runtime.h>

#include "g3k.h"
#include "g3k_device.h"

namespace {

using namespace g3k;

constexpr int D = G3K_HEAD_DIM;
constexpr int NT = 256;                      // staging kernel
constexpr int NTA = 512;                     // attention kernel: 8 waves
constexpr int BK = 32;                       // keys per tile
constexpr int KTILE = BK * D;                // halves in one K_hi or K_lo tile (16 KiB)
constexpr int VTILE = D * BK;                // halves in one V^T tile (16 KiB)
constexpr int STAGE = 2 * KTILE + VTILE;     // halves per pipeline stage (48 KiB)
constexpr int XCH = 8 * 16 * 64;             // floats of the partial-S exchange (32 KiB)
constexpr float NEG_BIG = -1.0e30f;
constexpr float LAZY = 8.0f;                 // log2 headroom of the lazy max

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint16_t f16_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }

// ---------------------------------------------------------------------------
// Staging: fp32 K rows -> fp16 hi / lo rows, fp32 V rows -> bf16 V^T columns.
// Workgroup = 64 keys x 64 dims of one head (grid: key blocks, D/64, H_kv).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(NT) void stage_kernel(g3k_stage_args a) {
    __shared__ uint16_t s_t[64][64 + 8];
    const int kb = blockIdx.x, dx = blockIdx.y, h = blockIdx.z;
    const int tid = threadIdx.x;
    const int kkbase = a.kk0 + kb * 64;
    const int kend = a.kk0 + a.cnt;
    // four float4 per thread: key row r = c / 16, float4 column c % 16
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int c = tid + NT * u;
        const int r = c >> 4, col = (c & 15) * 4;
        const int kk = kkbase + r;
        if (kk >= kend) continue;
        float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
        if (kk < a.nk) {
            const int pos = a.kstart + kk;
            const long long row = a.ring > 0 ? pos % a.ring : pos - a.row_pos0;
            const size_t off = (size_t)h * a.head_stride + (size_t)row * a.row_stride + dx * 64 + col;
            vv = *reinterpret_cast<const float4 *>(a.v_src + off);
            if (a.k_src) kv = *reinterpret_cast<const float4 *>(a.k_src + off);
        }
        if (a.k_src || kk >= a.nk) {
            const float x[4] = {kv.x, kv.y, kv.z, kv.w};
            uint16_t hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const _Float16 xh = (_Float16)x[e];
                hi[e] = f16_bits(xh);
                lo[e] = f16_bits((_Float16)(x[e] - (float)xh));
            }
            const size_t o = ((size_t)h * a.ldk + kk) * D + dx * 64 + col;
            *reinterpret_cast<uint2 *>(a.k_hi + o) =
                make_uint2(hi[0] | (uint32_t)hi[1] << 16, hi[2] | (uint32_t)hi[3] << 16);
            *reinterpret_cast<uint2 *>(a.k_lo + o) =
                make_uint2(lo[0] | (uint32_t)lo[1] << 16, lo[2] | (uint32_t)lo[3] << 16);
        }
        s_t[col + 0][r] = __builtin_bit_cast(uint16_t, (__bf16)vv.x);
        s_t[col + 1][r] = __builtin_bit_cast(uint16_t, (__bf16)vv.y);
        s_t[col + 2][r] = __builtin_bit_cast(uint16_t, (__bf16)vv.z);
        s_t[col + 3][r] = __builtin_bit_cast(uint16_t, (__bf16)vv.w);
    }
    __syncthreads();
    // V^T: dim row d (64 of them) x 64 keys = 128 B; 8 threads per row, 16 B each
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int c = tid + NT * u;
        const int d = c >> 3, part = c & 7;
        const int kk = kkbase + part * 8;
        if (kk >= kend) continue;
        const uint16_t *s = &s_t[d][part * 8];
        uint4 w;
        w.x = s[0] | (uint32_t)s[1] << 16;
        w.y = s[2] | (uint32_t)s[3] << 16;
        w.z = s[4] | (uint32_t)s[5] << 16;
        w.w = s[6] | (uint32_t)s[7] << 16;
        uint16_t *dst = a.vt + ((size_t)h * D + dx * 64 + d) * a.ldk + kk;
        if (kk + 8 <= kend) {
            *reinterpret_cast<uint4 *>(dst) = w;
        } else {
            for (int e = 0; kk + e < kend; e++) dst[e] = s[e];
        }
    }
}

// ---------------------------------------------------------------------------
// Attention.
// ---------------------------------------------------------------------------

// Row of the K tile fed to MFMA row m: bits 2 and 3 of m swapped.
__device__ __forceinline__ int key_of_row(int m) {
    return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1);
}

// Swizzles of the 16-byte chunks inside an LDS row.  K rows hold 32 chunks
// (512 B); a fragment read takes chunk 2t + h of rows key_of_row(l % 32):
// kswz is a bijection on row % 16 with kswz >> 1 distinct over each 8 rows
// that lanes 0-7 / 8-15 read, so 16 lanes of one chunk, or 8 lanes of each
// of two adjacent chunks, always fall in 16 different bank groups.  V^T rows
// hold 4 chunks (64 B); vswz spreads the 4 rows of one bank residue
// (d, d+4, d+8, d+12) over the 4 chunk positions, in pairs for two chunks.
__device__ __forceinline__ int kswz(int r) { return 2 * (r & 3) + 8 * ((r >> 3) & 1) + ((r >> 2) & 1); }
__device__ __forceinline__ int vswz(int d) { return 2 * ((d >> 2) & 1) + ((d >> 3) & 1); }

typedef __attribute__((address_space(3))) void *lds_ptr;
typedef const __attribute__((address_space(1))) void *gbl_ptr;

// Direct global -> LDS fetch of key tile kt into stage `st`: 48 one-KiB
// blocks (16 K_hi, 16 K_lo, 16 V^T), six per wave.
__device__ __forceinline__ void tile_fetch(uint16_t *st, const g3k_prefill_args &p, int kvh, int kt,
                                           int wave, int lane) {
    const uint16_t *kh = p.k_hi + ((size_t)kvh * p.ldk + (size_t)kt * BK) * D;
    const uint16_t *kl = p.k_lo + ((size_t)kvh * p.ldk + (size_t)kt * BK) * D;
    const uint16_t *vt = p.vt + (size_t)kvh * D * p.ldk + (size_t)kt * BK;
#pragma unroll
    for (int u = 0; u < 6; u++) {
        const int j = wave * 6 + u;
        if (j < 32) {
            const int b = j & 15;                   // rows 2b, 2b+1 of a K tile
            const int r = 2 * b + (lane >> 5);
            const int c = (lane & 31) ^ kswz(r);
            const uint16_t *src = (j < 16 ? kh : kl) + (size_t)r * D + c * 8;
            __builtin_amdgcn_global_load_lds((gbl_ptr)src, (lds_ptr)(st + (j >> 4) * KTILE + b * 512),
                                             16, 0, 0);
        } else {
            const int b = j - 32;                   // V^T rows 16b .. 16b+15
            const int d = 16 * b + (lane >> 2);
            const int c = (lane & 3) ^ vswz(d);
            __builtin_amdgcn_global_load_lds((gbl_ptr)(vt + (size_t)d * p.ldk + c * 8),
                                             (lds_ptr)(st + 2 * KTILE + b * 512), 16, 0, 0);
        }
    }
}

__device__ __forceinline__ void wait_fetch() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Workgroup barrier that orders LDS traffic only (ds_write before, ds_read
// after).  __syncthreads() would also wait for every outstanding global load,
// including the next tile's global->LDS fetch that is meant to overlap.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int G>
__global__ __launch_bounds__(NTA, 1) void prefill_kernel(g3k_prefill_args p) {
    __shared__ __attribute__((aligned(16))) uint16_t smem[2 * STAGE];
    __shared__ __attribute__((aligned(16))) float xch[XCH];
    constexpr int PPG = 4 / G;        // wave pairs per query head
    constexpr int PB = 32 * PPG;      // query positions per workgroup
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int h = lane >> 5, ln = lane & 31;
    const int pair = wave >> 1, e = wave & 1;     // e: head-dim half of this wave
    const int kvh = blockIdx.y;
    const int qb = gridDim.x - 1 - blockIdx.x;  // longest (latest) query blocks first
    const int g = pair / PPG;
    const int qhead = kvh * G + g;
    const int tok0 = qb * PB + (pair % PPG) * 32;
    const int tok = tok0 + ln;
    const bool wave_live = tok0 < p.n;
    const int q_kk = p.hist + tok;    // key index of this lane's query

    // key index range of the workgroup and of this wave pair (inclusive)
    const int wg_first = p.hist + qb * PB;
    const int wg_last = min(p.hist + min(qb * PB + PB, p.n) - 1, p.nk - 1);
    const int kt0 = max(0, wg_first - p.window + 1) / BK;
    const int kt1 = wg_last / BK;
    const int w_first = p.hist + tok0;
    const int w_last = min(w_first + 31, p.hist + p.n - 1);
    const int wkt0 = max(0, w_first - p.window + 1) / BK;
    const int wkt1 = w_last / BK;

    // ---- first tile in flight, then this wave's Q^T fragments (hi / lo) ----
    tile_fetch(smem, p, kvh, kt0, wave, lane);

    half8 qh[8], ql[8];
    {
        const float *qrow = p.q + ((size_t)qhead * p.n + (tok < p.n ? tok : 0)) * D + 128 * e;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const float4 a = *reinterpret_cast<const float4 *>(qrow + 16 * t + 8 * h);
            const float4 b = *reinterpret_cast<const float4 *>(qrow + 16 * t + 8 * h + 4);
            const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float v = tok < p.n ? x[u] * p.qscale : 0.f;
                const _Float16 hi = (_Float16)v;
                qh[t][u] = hi;
                ql[t][u] = (_Float16)(v - (float)hi);
            }
        }
    }

    f32x16 o[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[mt][r] = 0.f;
    float m_ref = NEG_BIG, l_sum = 0.f;
    const int krow = key_of_row(ln);
    const int ksw = kswz(krow), vsw = vswz(ln);  // (32*mt + ln) has the same vswz as ln
    float *x_mine = xch + wave * 1024 + lane * 4;         // [wave][r/4][lane][4]
    const float *x_other = xch + (wave ^ 1) * 1024 + lane * 4;

    wait_fetch();
    __syncthreads();

    for (int kt = kt0; kt <= kt1; kt++) {
        const int cur = (kt - kt0) & 1;
        if (kt < kt1) tile_fetch(smem + (cur ^ 1) * STAGE, p, kvh, kt + 1, wave, lane);
        const uint16_t *st = smem + cur * STAGE;
        const bool live = wave_live && kt >= wkt0 && kt <= wkt1;

        // ---- partial S^T over this wave's head-dim half, three fp16 passes ----
        f32x16 s;
        if (live) {
#pragma unroll
            for (int r = 0; r < 16; r++) s[r] = 0.f;
            const uint16_t *kh = st + krow * D;
            const uint16_t *kl = kh + KTILE;
            // fragments of d-step t + 1 are read while step t's MFMAs run
            half8 ah = *reinterpret_cast<const half8 *>(kh + ((16 * e + h) ^ ksw) * 8);
            half8 al = *reinterpret_cast<const half8 *>(kl + ((16 * e + h) ^ ksw) * 8);
#pragma unroll
            for (int t = 0; t < 8; t++) {
                half8 ah_n = ah, al_n = al;
                if (t < 7) {
                    const int cofs = ((16 * e + 2 * t + 2 + h) ^ ksw) * 8;
                    ah_n = *reinterpret_cast<const half8 *>(kh + cofs);
                    al_n = *reinterpret_cast<const half8 *>(kl + cofs);
                }
                s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, qh[t], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, ql[t], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, qh[t], s, 0, 0, 0);
                ah = ah_n;
                al = al_n;
            }
#pragma unroll
            for (int j = 0; j < 4; j++)
                *reinterpret_cast<float4 *>(x_mine + j * 256) =
                    make_float4(s[4 * j], s[4 * j + 1], s[4 * j + 2], s[4 * j + 3]);
        }
        lds_barrier();

        if (live) {
            // ---- full S^T = half 0 + half 1 (same order in both waves) ----
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 y = *reinterpret_cast<const float4 *>(x_other + j * 256);
                const float yy[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
                for (int i = 0; i < 4; i++)
                    s[4 * j + i] = e == 0 ? s[4 * j + i] + yy[i] : yy[i] + s[4 * j + i];
            }
            // ---- mask (diagonal, window edge, ragged end) ----
            const int kbase = kt * BK + 8 * h;
            const bool edge = (kt * BK + BK - 1 > w_first) || (kt * BK <= w_last - p.window) ||
                              (kt * BK + BK > p.nk);
            if (edge) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int kk = kbase + 16 * (r >> 3) + (r & 7);
                    const bool ok = kk <= q_kk && kk > q_kk - p.window && kk < p.nk;
                    s[r] = ok ? s[r] : -INFINITY;
                }
            }
            // ---- online softmax with a lazy reference max ----
            float mx = s[0];
#pragma unroll
            for (int r = 1; r < 16; r++) mx = fmaxf(mx, s[r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const bool bump = mx > m_ref + LAZY;
            if (__builtin_amdgcn_ballot_w64(bump)) {
                const float m_new = bump ? mx : m_ref;
                const float alpha = fast_exp2(m_ref - m_new);
                m_ref = m_new;
                l_sum *= alpha;
#pragma unroll
                for (int mt = 0; mt < 4; mt++)
#pragma unroll
                    for (int r = 0; r < 16; r++) o[mt][r] *= alpha;
            }
            float psum = 0.f;
            bf16x8 ph[2], pl[2];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float pr = s[r] == -INFINITY ? 0.f : fast_exp2(s[r] - m_ref);
                psum += pr;
                const __bf16 hi = (__bf16)pr;
                ph[r >> 3][r & 7] = hi;
                pl[r >> 3][r & 7] = (__bf16)(pr - (float)hi);
            }
            psum += __shfl_xor(psum, 32);
            l_sum += psum;
            // ---- O^T[half] += V^T . P^T, two bf16 passes ----
            const uint16_t *vt = st + 2 * KTILE + (128 * e + ln) * BK;
            bf16x8 av = *reinterpret_cast<const bf16x8 *>(vt + ((h ^ vsw) * 8));
#pragma unroll
            for (int f = 0; f < 8; f++) {          // f = 2 * mt + t2
                const int mt = f >> 1, t2 = f & 1;
                bf16x8 av_n = av;
                if (f < 7) {
                    const int cofs = ((2 * ((f + 1) & 1) + h) ^ vsw) * 8;
                    av_n = *reinterpret_cast<const bf16x8 *>(vt + ((f + 1) >> 1) * 32 * BK + cofs);
                }
                o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, ph[t2], o[mt], 0, 0, 0);
                o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pl[t2], o[mt], 0, 0, 0);
                av = av_n;
            }
        }

        wait_fetch();
        __syncthreads();
    }

    // ---- normalise and write attn_out[token][qhead][dim] ----
    if (!wave_live || tok >= p.n) return;
    const float inv = 1.0f / l_sum;
    float *orow = p.out + ((size_t)tok * p.n_kv_heads * G + qhead) * D + 128 * e + 4 * h;
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            *reinterpret_cast<float4 *>(orow + mt * 32 + 8 * j) =
                make_float4(o[mt][4 * j] * inv, o[mt][4 * j + 1] * inv, o[mt][4 * j + 2] * inv,
                            o[mt][4 * j + 3] * inv);
}

template <int G>
hipError_t launch_prefill(const g3k_prefill_args *a, hipStream_t st) {
    constexpr int PB = 32 * (4 / G);
    const int nqb = (a->n + PB - 1) / PB;
    if (a->ev0 && hipEventRecord((hipEvent_t)a->ev0, st) != hipSuccess) return hipErrorInvalidValue;
    hipLaunchKernelGGL(prefill_kernel<G>, dim3(nqb, a->n_kv_heads), dim3(NTA), 0, st, *a);
    const hipError_t e = hipGetLastError();
    if (a->ev1 && hipEventRecord((hipEvent_t)a->ev1, st) != hipSuccess) return hipErrorInvalidValue;
    return e;
}

}  // namespace

extern "C" int g3k_stage(const g3k_stage_args *a, void *stream) {
    if (a->cnt <= 0) return 0;
    if (a->ldk % 64 || a->kk0 + a->cnt > a->ldk) return (int)hipErrorInvalidValue;
    dim3 grid((a->cnt + 63) / 64, D / 64, a->n_kv_heads);
    hipLaunchKernelGGL(stage_kernel, grid, dim3(NT), 0, (hipStream_t)stream, *a);
    return (int)hipGetLastError();
}

extern "C" int g3k_prefill(const g3k_prefill_args *a, void *stream) {
    if (a->n <= 0) return 0;
    if (a->ldk % 64 || a->nk > a->ldk || a->hist + a->n != a->nk || a->window < 1)
        return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    switch (a->group) {
        case 1: return (int)launch_prefill<1>(a, st);
        case 2: return (int)launch_prefill<2>(a, st);
        case 4: return (int)launch_prefill<4>(a, st);
        default: return (int)hipErrorInvalidValue;
    }
}
