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
// Data flow.  One workgroup = 8 wave64 = one KV head x 16*8/G query
// positions of each of its G query heads; each wave owns 16 queries of one
// head over the full head dim (Q^T hi / lo: 64 VGPRs, O^T: 64):
//   S^T[key][query] = K . Q^T   with v_mfma_f32_16x16x32_f16: A = K tile rows
//     from LDS, B = the wave's Q^T fragments in registers;
//   O^T[dim][query] += V^T . P^T with v_mfma_f32_16x16x32_bf16: A = V^T tile
//     rows from LDS, B = P straight from the S^T registers.
// In the 16x16 accumulator layout lane l holds column (query) l % 16, so a
// query's softmax statistics live in the four lanes l % 16 + 16 g and the
// O^T rescale is lane-local.  The K rows fed to S^T sub-tile j (keys
// 16 j .. of a 32-key tile) are permuted, row m -> key 8 (m / 4) + 4 j + m % 4,
// so lane group g = l / 16 ends up holding keys 8 g .. 8 g + 7 in its eight
// S^T registers: exactly the B operand of the P.V MFMA (no shuffles).
// Key tiles of 32 are triple-buffered in LDS and fetched two tiles ahead with
// gfx950's direct global->LDS loads (global_load_lds_dwordx4: no staging
// registers; one wave instruction moves 1 KiB in lane order):
//   K: one LDS row per key, fp16 hi (512 B) | lo (512 B), rows padded to
//      1040 B, so 16 lanes reading 16 rows at one chunk hit 16 bank groups and
//      every fragment address is a per-lane base + an immediate offset;
//   V^T: [256][32] bf16, the four 16-byte chunks of a row XOR-swizzled by
//      row bits 2-3 (conflict-free fragment reads, also base + immediate).
// One barrier per tile (stage hand-over).  Softmax runs in the exp2 domain
// (q pre-scaled by scale * log2(e)) with a lazy running max: O and l are
// rescaled only when a tile's max exceeds the reference max by more than 2^8.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "g3k.h"
#include "g3k_device.h"

namespace {

using namespace g3k;

constexpr int D = G3K_HEAD_DIM;
constexpr int NT = 256;                      // staging kernel
constexpr int NTA = 512;                     // attention kernel: 8 waves
constexpr int BK = 32;                       // keys per tile
constexpr int KROWB = 1040;                  // bytes per K row in LDS: hi | lo | pad
constexpr int KTILEB = BK * KROWB;           // bytes of the K tile (33280)
constexpr int VTILEB = D * BK * 2;           // bytes of the V^T tile (16 KiB)
constexpr int STAGEB = KTILEB + VTILEB;      // bytes per pipeline stage
constexpr int NSTAGE = 3;                    // tiles in flight: compute kt, fetch kt+1, kt+2
constexpr int FETCH_OPS = 6;                 // global->LDS instructions per wave per tile
constexpr float NEG_BIG = -1.0e30f;
constexpr float LAZY = 8.0f;                 // log2 headroom of the lazy max

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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

typedef __attribute__((address_space(3))) void *lds_ptr;
typedef const __attribute__((address_space(1))) void *gbl_ptr;

// XOR swizzle of the four 16-byte chunks of a V^T row: rows d, d+4, d+8,
// d+12 (one bank residue) take the four chunk positions.
__device__ __forceinline__ int vswz(int d) { return (d >> 2) & 3; }

// Direct global -> LDS fetch of key tile kt into the stage at byte offset
// `st`: 32 K rows (lanes 0-31 the hi half, 32-63 the lo half) and 16 V^T
// blocks of 16 rows; six one-KiB instructions per wave.
__device__ __forceinline__ void tile_fetch(unsigned char *st, const g3k_prefill_args &p, int kvh,
                                           int kt, int wave, int lane) {
    const size_t krow0 = (size_t)kvh * p.ldk + (size_t)kt * BK;
    const uint16_t *vt = p.vt + (size_t)kvh * D * p.ldk + (size_t)kt * BK;
#pragma unroll
    for (int u = 0; u < 6; u++) {
        const int j = wave * 6 + u;
        if (j < 32) {
            const uint16_t *src = (lane < 32 ? p.k_hi : p.k_lo) + (krow0 + j) * D + (lane & 31) * 8;
            __builtin_amdgcn_global_load_lds((gbl_ptr)src, (lds_ptr)(st + j * KROWB), 16, 0, 0);
        } else {
            const int b = j - 32;                   // V^T rows 16b .. 16b+15
            const int d = 16 * b + (lane >> 2);
            const int c = (lane & 3) ^ vswz(d);
            __builtin_amdgcn_global_load_lds((gbl_ptr)(vt + (size_t)d * p.ldk + c * 8),
                                             (lds_ptr)(st + KTILEB + b * 1024), 16, 0, 0);
        }
    }
}

// Wait until this wave's fetches of all but the newest tile have landed
// (vmcnt counts the global->LDS loads; nothing else is outstanding in the loop).
__device__ __forceinline__ void wait_fetch_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void wait_fetch_but_one() {
    static_assert(FETCH_OPS == 6, "vmcnt below assumes six fetch instructions per tile");
    asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
}

template <int G>
__global__ __launch_bounds__(NTA, 1) void prefill_kernel(g3k_prefill_args p) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[NSTAGE * STAGEB];
    constexpr int WPH = 8 / G;        // waves per query head
    constexpr int PB = 16 * WPH;      // query positions per workgroup
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, ln = lane & 15;     // lane group, query column
    // 1-D grid, longest (latest) query blocks first across all heads: with
    // workgroups dealt round-robin to the 8 XCDs, block id -> (qb, id % H_kv)
    // also keeps each XCD on one KV head (its L2 streams one head's K / V).
    const int kvh = blockIdx.x % p.n_kv_heads;
    const int qb = (int)(gridDim.x / p.n_kv_heads) - 1 - (int)(blockIdx.x / p.n_kv_heads);
    const int qhead = kvh * G + wave / WPH;
    const int tok0 = qb * PB + (wave % WPH) * 16;
    const int tok = tok0 + ln;
    const bool wave_live = tok0 < p.n;
    const int q_kk = p.hist + tok;    // key index of this lane's query

    // key index range of the workgroup and of this wave (inclusive)
    const int wg_first = p.hist + qb * PB;
    const int wg_last = min(p.hist + min(qb * PB + PB, p.n) - 1, p.nk - 1);
    const int kt0 = max(0, wg_first - p.window + 1) / BK;
    const int kt1 = wg_last / BK;
    const int w_first = p.hist + tok0;
    const int w_last = min(w_first + 15, p.hist + p.n - 1);
    const int wkt0 = max(0, w_first - p.window + 1) / BK;
    const int wkt1 = w_last / BK;

    // ---- first two tiles in flight, then this wave's Q^T fragments (hi / lo) ----
    tile_fetch(smem, p, kvh, kt0, wave, lane);
    if (kt0 + 1 <= kt1) tile_fetch(smem + STAGEB, p, kvh, kt0 + 1, wave, lane);

    half8 qh[8], ql[8];
    {
        const float *qrow = p.q + ((size_t)qhead * p.n + (tok < p.n ? tok : 0)) * D + 8 * g;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const float4 a = *reinterpret_cast<const float4 *>(qrow + 32 * t);
            const float4 b = *reinterpret_cast<const float4 *>(qrow + 32 * t + 4);
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

    f32x4 o[16];
#pragma unroll
    for (int mt = 0; mt < 16; mt++) o[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_ref = NEG_BIG, l_sum = 0.f;
    // per-lane LDS byte offsets inside a stage: K rows of the two S^T
    // sub-tiles (row m -> key 8 (m / 4) + 4 j + m % 4) at chunk g, and the
    // V^T row ln of each 16-dim block at its swizzled chunk g
    const int krow = 8 * (ln >> 2) + (ln & 3);
    const int koff0 = krow * KROWB + 16 * g;
    const int koff1 = (krow + 4) * KROWB + 16 * g;
    const int voff = KTILEB + ln * 64 + 16 * (g ^ vswz(ln));

    if (kt0 + 1 <= kt1) wait_fetch_but_one(); else wait_fetch_all();
    __syncthreads();

    int cur = 0;                      // stage holding tile kt
    for (int kt = kt0; kt <= kt1; kt++) {
        const int nxt2 = cur == 0 ? 2 : cur - 1;    // stage of tile kt + 2 (= kt - 1's)
        if (kt + 2 <= kt1) tile_fetch(smem + nxt2 * STAGEB, p, kvh, kt + 2, wave, lane);
        const unsigned char *st = smem + cur * STAGEB;

        if (wave_live && kt >= wkt0 && kt <= wkt1) {
            // ---- S^T = K . Q^T for keys 0-15 (s0) and 16-31 (s1), three fp16 passes ----
            f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const half8 ah0 = *reinterpret_cast<const half8 *>(st + koff0 + 64 * t);
                const half8 al0 = *reinterpret_cast<const half8 *>(st + koff0 + 512 + 64 * t);
                const half8 ah1 = *reinterpret_cast<const half8 *>(st + koff1 + 64 * t);
                const half8 al1 = *reinterpret_cast<const half8 *>(st + koff1 + 512 + 64 * t);
                s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah0, qh[t], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah1, qh[t], s1, 0, 0, 0);
                s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah0, ql[t], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah1, ql[t], s1, 0, 0, 0);
                s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(al0, qh[t], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(al1, qh[t], s1, 0, 0, 0);
            }
            // register u of this lane: key kt*32 + 8 g + u (u < 4: s0[u], else s1[u-4])
            float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
            // ---- mask (diagonal, window edge, ragged end) ----
            const bool edge = (kt * BK + BK - 1 > w_first) || (kt * BK <= w_last - p.window) ||
                              (kt * BK + BK > p.nk);
            if (edge) {
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int kk = kt * BK + 8 * g + u;
                    const bool ok = kk <= q_kk && kk > q_kk - p.window && kk < p.nk;
                    sv[u] = ok ? sv[u] : -INFINITY;
                }
            }
            // ---- online softmax with a lazy reference max ----
            float mx = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                             fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const bool bump = mx > m_ref + LAZY;
            if (__builtin_amdgcn_ballot_w64(bump)) {
                const float m_new = bump ? mx : m_ref;
                const float alpha = fast_exp2(m_ref - m_new);
                m_ref = m_new;
                l_sum *= alpha;
#pragma unroll
                for (int mt = 0; mt < 16; mt++) o[mt] *= alpha;
            }
            float psum = 0.f;
            bf16x8 ph, pl;
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float pr = fast_exp2(sv[u] - m_ref);   // exp2(-inf) = 0 for masked keys
                psum += pr;
                const __bf16 hi = (__bf16)pr;
                ph[u] = hi;
                pl[u] = (__bf16)(pr - (float)hi);
            }
            psum += __shfl_xor(psum, 16);
            psum += __shfl_xor(psum, 32);
            l_sum += psum;
            // ---- O^T += V^T . P^T, two bf16 passes, 16 dim blocks ----
#pragma unroll
            for (int mt = 0; mt < 16; mt++) {
                const bf16x8 av = *reinterpret_cast<const bf16x8 *>(st + voff + 1024 * mt);
                o[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, ph, o[mt], 0, 0, 0);
                o[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pl, o[mt], 0, 0, 0);
            }
        }

        // tile kt + 1 must have landed before the barrier; kt + 2 may still fly
        if (kt + 2 <= kt1) wait_fetch_but_one(); else wait_fetch_all();
        __syncthreads();
        cur = cur == 2 ? 0 : cur + 1;
    }

    // ---- normalise and write attn_out[token][qhead][dim] ----
    if (!wave_live || tok >= p.n) return;
    const float inv = 1.0f / l_sum;
    float *orow = p.out + ((size_t)tok * p.n_kv_heads * G + qhead) * D + 4 * g;
#pragma unroll
    for (int mt = 0; mt < 16; mt++)
        *reinterpret_cast<float4 *>(orow + 16 * mt) =
            make_float4(o[mt][0] * inv, o[mt][1] * inv, o[mt][2] * inv, o[mt][3] * inv);
}

template <int G>
hipError_t launch_prefill(const g3k_prefill_args *a, hipStream_t st) {
    constexpr int PB = 16 * (8 / G);
    const int nqb = (a->n + PB - 1) / PB;
    // With timing events the dispatch itself records them (kernel begin / end).
    hipExtLaunchKernelGGL(prefill_kernel<G>, dim3(nqb * a->n_kv_heads), dim3(NTA), 0, st,
                          (hipEvent_t)a->ev0, (hipEvent_t)a->ev1, 0, *a);
    return hipGetLastError();
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
