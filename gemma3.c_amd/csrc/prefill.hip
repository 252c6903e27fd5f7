// prefill.hip - causal / sliding-window prefill attention on MFMA (gfx950).
//
// Replaces the per-token attention loop of the reference prefill
// (gemma3_transformer.c:641-692; gemma3_gqa at :689-691): every token i of the
// batch attends the keys of positions [pos - window + 1, pos] (local layer)
// or [0, pos] (global layer), pos = start_pos + i, with the reference's
// softmax (gemma3_kernels.c:396-415) and scale 1/sqrt(head_dim).
//
// Precision policy.  Post-RoPE q and k, P and V are fp32 and not
// representable in any MFMA input format, and the path is held to max-abs
// error <= 2e-3 x output RMS.  A single bf16 or fp16 pass misses that bar by
// 5-60x on the early causal rows, so every operand is split, x = x_hi + x_lo
// (x_hi = fp16(x) for q and k, bf16(x) for P and V):
//   S = q.k   q_hi.k_hi + q_lo.k_hi + q_hi.k_lo, by default one fp16 MFMA pass
//             for q_hi.k_hi and the two cross terms as one scaled fp8 MFMA dot
//             with per-key and per-query power-of-two scales (tile_scores);
//             with the exact policy three fp16 passes (x_lo = fp16(x - x_hi));
//   O = P.V   bf16 MFMA passes        P_hi.V_hi + P_lo.V_hi (+ P_hi.V_lo)
//             (16 bits of P and V).  The staging pass records whether any
//             V_lo is nonzero; when every staged value is exactly bf16 (the
//             bf16-valued inputs the path is specified on) V_lo is zero and
//             its pass is skipped, which changes no bit of the result.
// fp32 accumulation throughout: 2.5x (3x with V_lo) the algorithmic MFMA
// FLOPs; in MFMA-pipe time 2x under the fp8 cross policy (its fp8 MFMAs run
// at twice the fp16 rate).
//
// Data flow.  One workgroup = 8 / NQB waves = one KV head x the queries of
// its G query heads; each wave owns NQB blocks of 16 queries of one head over
// the full head dim (per block Q^T hi / lo or hi / fp8 cross operand: 64
// VGPRs, O^T: 64):
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
// Key tiles of 32 live in two LDS rings, K tiles two deep and V^T tiles two
// deep, filled by gfx950's direct buffer -> LDS loads (buffer_load_dwordx4
// ... lds: no staging registers; one wave instruction moves 1 KiB in lane
// order; the addresses are a scalar buffer descriptor + one per-lane offset):
//   K: one 1 KiB LDS row per key, fp16 hi (512 B) | lo (512 B) or | the fp8
//      cross operand bytes (512 B, G3K_KROW_X8 in g3k.h), its 16-byte
//      chunks XOR-swizzled by key bits (kswz), so the 16 rows one fragment
//      read touches hit 16 bank groups; every fragment address is one of
//      four per-lane bases + an immediate offset;
//   V^T: [256][32] bf16 (then the lo part), the four 16-byte chunks of a row
//      XOR-swizzled by row bits 2-3 (conflict-free fragment reads).
// Iteration kt computes the scores of tile kt + 1 and the P.V of tile kt,
// while K of tile kt + 2 and V of tile kt + 1 stream in; one barrier per
// tile.  Softmax runs in the exp2 domain (q pre-scaled by scale * log2(e))
// with a lazy running max: O and l are rescaled only when a tile's max
// exceeds the reference max by more than 2^8.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "g3k.h"
#include "g3k_device.h"
#include "rope_write_body.h"

namespace {

using namespace g3k;

constexpr int D = G3K_HEAD_DIM;
constexpr int NT = 256;                      // staging kernel
constexpr int BK = 32;                       // keys per tile
constexpr int KROWB = 1024;                  // bytes per K row in LDS: hi | lo
constexpr int KTILEB = BK * KROWB;           // bytes of a K tile (32768)
constexpr int VTILEB = D * BK * 2;           // bytes of a V^T tile, one part (16 KiB)
constexpr int LDS_V0 = 2 * KTILEB;           // V ring after the K ring
constexpr int LDS_BYTES = LDS_V0 + 2 * 2 * VTILEB;   // 131072
constexpr int LDS_KS0 = LDS_BYTES;           // fp8 cross policy: key-scale ring after the V ring
constexpr int KS_SLOT = 256;                 // one tile's 32 scale bytes (a 256-byte fetch)
constexpr int LDS_BYTES_X8 = LDS_KS0 + 2 * KS_SLOT;
constexpr float NEG_BIG = -1.0e30f;
constexpr float LAZY = 8.0f;                 // log2 headroom of the lazy max
#ifndef G3K_KPF
#define G3K_KPF 1                            // K fragment prefetch depth (d-steps)
#endif
#ifndef G3K_VPF
#define G3K_VPF 2                            // V^T fragment prefetch depth (16-dim blocks)
#endif

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }
// 32 fp8 bytes of an MFMA operand from two 16-byte pieces (bytes 0-15, 16-31)
__device__ __forceinline__ i32x8 cat8(u32x4 a, u32x4 b) {
    return __builtin_bit_cast(i32x8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Cache-policy bits of a buffer access: sc1, agent-coherent (written through
// to / read from the point of coherence shared by every XCD).
constexpr int CP_SC1 = 16;

__device__ __forceinline__ uint16_t bf16_bits(__bf16 h) { return __builtin_bit_cast(uint16_t, h); }

// Two floats -> bf16 (round to nearest even), a in the low half
// (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, b2));
}

// ---------------------------------------------------------------------------
// Staging: fp32 V rows -> bf16 hi and lo V^T columns (workgroups of 64 keys
// x 64 dims of one head); fp32 K rows -> key rows in the policy's format
// (write_krow: one wave per key row, which holds the whole row for the fp8
// format's per-row scale).
// ---------------------------------------------------------------------------
// vc != nullptr (the prefill front launch, staging the batch's own V): the
// staged V values are also written to the cache rows vc describes
// (rope_write_vec's destination rules), so the batch's V is read once.
__device__ __forceinline__ void stage_block(const g3k_stage_args &a, int kb, int dx, int h,
                                            const g3k_rope_write_args *vc = nullptr) {
    __shared__ uint16_t s_t[2][64][64 + 8];
    const int tid = threadIdx.x;
    const int kkbase = a.kk0 + kb * 64;
    const int kend = a.kk0 + a.cnt;
    int any_lo = 0;
    // four float4 per thread: key row r = c / 16, float4 column c % 16
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int c = tid + NT * u;
        const int r = c >> 4, col = (c & 15) * 4;
        const int kk = kkbase + r;
        if (kk >= kend) continue;
        float4 vv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (kk < a.nk) {
            const int pos = a.kstart + kk;
            const long long row = a.ring > 0 ? pos % a.ring : pos - a.row_pos0;
            const size_t off = (size_t)h * a.head_stride + (size_t)row * a.row_stride + dx * 64 + col;
            vv = *reinterpret_cast<const float4 *>(a.v_src + off);
            if (vc && pos - vc->start_pos >= vc->kv_skip && pos - vc->start_pos < vc->n) {
                const int slot = vc->ring > 0 ? pos % vc->ring : pos - vc->dst_pos0;
                *reinterpret_cast<float4 *>(vc->v_dst + (size_t)h * vc->dst_head_stride + (size_t)slot * D + dx * 64 +
                                            col) = vv;
            }
        }
        const float y[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const __bf16 yh = (__bf16)y[e];
            const uint16_t lo = bf16_bits((__bf16)(y[e] - (float)yh));
            s_t[0][col + e][r] = bf16_bits(yh);
            s_t[1][col + e][r] = lo;
            any_lo |= lo & 0x7fff;
        }
    }
    if (__syncthreads_or(any_lo) && tid == 0) *a.v_lo_flag = a.epoch;
    // V^T: dim row d (64 of them) x 64 keys = 128 B per part; 8 threads per
    // row, 16 B each
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int c = tid + NT * u;
        const int part = c >> 9;                 // 0: hi, 1: lo
        const int d = (c >> 3) & 63, seg = c & 7;
        const int kk = kkbase + seg * 8;
        if (kk >= kend) continue;
        const uint16_t *s = &s_t[part][d][seg * 8];
        uint4 w;
        w.x = s[0] | (uint32_t)s[1] << 16;
        w.y = s[2] | (uint32_t)s[3] << 16;
        w.z = s[4] | (uint32_t)s[5] << 16;
        w.w = s[6] | (uint32_t)s[7] << 16;
        uint16_t *dst = (part ? a.vt_lo : a.vt) + ((size_t)h * D + dx * 64 + d) * a.ldk + kk;
        if (kk + 8 <= kend) {
            *reinterpret_cast<uint4 *>(dst) = w;
        } else {
            for (int e = 0; kk + e < kend; e++) dst[e] = s[e];
        }
    }
}

// Key rows of the staging (one wave each): the first key index whose row
// this launch writes, and how many (times the KV heads).  With k_src every
// row of [kk0, kk0 + cnt) (from the cache below nk, zeros above); without it
// (the batch's own keys come from rope_write_vec) only the zero padding rows
// from nk on.
__device__ __host__ __forceinline__ int krow_first(const g3k_stage_args &a) {
    return a.k_src ? a.kk0 : (a.nk > a.kk0 ? a.nk : a.kk0);
}
__device__ __host__ __forceinline__ long long krow_count(const g3k_stage_args &a) {
    const int n = a.kk0 + a.cnt - krow_first(a);
    return n > 0 ? (long long)n * a.n_kv_heads : 0;
}

// Key row w (of krow_count) of the staging: key index kk = krow_first + w /
// H_kv, head w % H_kv.
__device__ __forceinline__ void stage_krow(const g3k_stage_args &a, long long w, int lane) {
    if (w >= krow_count(a)) return;
    const int kk = krow_first(a) + (int)(w / a.n_kv_heads), h = (int)(w % a.n_kv_heads);
    float2 lo = make_float2(0.f, 0.f), hi = lo;
    if (a.k_src && kk < a.nk) {
        const int pos = a.kstart + kk;
        const long long row = a.ring > 0 ? pos % a.ring : pos - a.row_pos0;
        const float *src = a.k_src + (size_t)h * a.head_stride + (size_t)row * a.row_stride;
        lo = *reinterpret_cast<const float2 *>(src + 2 * lane);
        hi = *reinterpret_cast<const float2 *>(src + 128 + 2 * lane);
    }
    const size_t r = (size_t)h * a.ldk + kk;
    write_krow(a.kq + r * (2 * D), a.kscale ? a.kscale + r : nullptr, lo.x, lo.y, hi.x, hi.y, lane);
}

// History staging in one launch: the V^T blocks (key blocks x D / 64 x H_kv,
// first) and the key-row waves (four per workgroup).
__global__ __launch_bounds__(NT) void stage_kernel(g3k_stage_args a, unsigned vblocks, unsigned kblocks) {
    const unsigned b = blockIdx.x;
    if (b < vblocks) {
        const unsigned per_head = kblocks * (D / 64);
        stage_block(a, (int)(b % kblocks), (int)((b % per_head) / kblocks), (int)(b / per_head));
        return;
    }
    stage_krow(a, ((long long)(b - vblocks) * NT + threadIdx.x) >> 6, threadIdx.x & 63);
}

// The batch's front end in one launch: the V^T staging blocks of `sa` (first:
// fewer and heavier), which also write the batch's V rows to the cache, the
// K waves of rope_write_vec over `ra` (K-norm, RoPE, cache write, staged key
// rows), then the zero key rows of the padding.  The parts read disjoint
// inputs (V / K) and write disjoint buffers, so their order does not matter.
__global__ __launch_bounds__(NT) void front_kernel(g3k_rope_write_args ra, g3k_stage_args sa, unsigned stage_blocks,
                                                   unsigned kblocks, unsigned rw_blocks) {
    const unsigned b = blockIdx.x;
    if (b < stage_blocks) {
        const unsigned per_head = kblocks * (D / 64);
        // the cache rows are written only for a batch that has tokens
        stage_block(sa, (int)(b % kblocks), (int)((b % per_head) / kblocks), (int)(b / per_head),
                    ra.n > 0 ? &ra : nullptr);
        return;
    }
    if (b >= stage_blocks + rw_blocks) {
        stage_krow(sa, ((long long)(b - stage_blocks - rw_blocks) * NT + threadIdx.x) >> 6, threadIdx.x & 63);
        return;
    }
    // K wave kw = token i x H_kv + head h is rope_write_vec's vector i x
    // (2 H_kv) + h (no queries: K heads first, then V heads)
    const long long kw = ((long long)(b - stage_blocks) * NT + threadIdx.x) >> 6;
    const long long i = kw / ra.n_kv_heads, h = kw % ra.n_kv_heads;
    rope_write_vec(ra, i < ra.n ? i * (2 * ra.n_kv_heads) + h : (long long)ra.n * 2 * ra.n_kv_heads, threadIdx.x & 63);
}

// ---------------------------------------------------------------------------
// Attention.
// ---------------------------------------------------------------------------

typedef __attribute__((address_space(3))) void *lds_ptr;

// XOR swizzle of the four 16-byte chunks of a V^T row: rows d, d+4, d+8,
// d+12 (one bank residue) take the four chunk positions.
__device__ __forceinline__ int vswz(int d) { return (d >> 2) & 3; }

// Chunk swizzle of key row r of a tile: logical 16-byte chunk c of the row
// sits at chunk c ^ kswz(r).  A K fragment read touches the rows {0-3, 8-11,
// 16-19, 24-27} (or that set + 4) at one logical chunk; with 1 KiB rows the
// bank group of a chunk is its index % 16, and kswz maps each read set onto
// all 16 values.  It replaced 1040-byte padded rows: the kernel's LDS
// bank-conflict cycles fell from 4.0 to 1.33 per LDS instruction and
// configs[3] from 588.6 to 578.6 us on one box.
__device__ __forceinline__ int kswz(int r) { return ((r >> 3) << 2) | (r & 3); }

// Raw buffer descriptor over [base, base + bytes): stride 0, the gfx9
// family's dword-3 format word for untyped access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// K tile kt -> LDS ring slot `dst`: 32 rows of 1 KiB (hi | lo); lane l moves
// the row's logical chunk l ^ kswz(row) to LDS chunk l; 32 / NW rows per
// wave.
template <int NW>
__device__ __forceinline__ void fetch_k(unsigned char *dst, __amdgpu_buffer_rsrc_t kr, int kt, int wave,
                                        int lane) {
#pragma unroll
    for (int u = 0; u < 32 / NW; u++) {
        const int j = wave * (32 / NW) + u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (lds_ptr)(dst + j * KROWB), 16, (lane ^ kswz(j)) * 16,
                                                 (kt * BK + j) * (4 * D), 0, 0);
    }
}

// One part (hi or lo) of V^T tile kt -> LDS: 16 blocks of 16 rows x 64 B;
// lane l moves row 16 b + l / 4, chunk (l % 4) ^ vswz(row) (voff), so LDS
// position c of a row holds global chunk c ^ vswz(row).  16 / NW blocks per
// wave.
template <int NW>
__device__ __forceinline__ void fetch_v(unsigned char *dst, __amdgpu_buffer_rsrc_t vr, int kt, int wave,
                                        unsigned voff, int ldk) {
#pragma unroll
    for (int u = 0; u < 16 / NW; u++) {
        const int b = wave * (16 / NW) + u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (lds_ptr)(dst + b * 1024), 16, voff,
                                                 (16 * b * ldk + kt * BK) * 2, 0, 0);
    }
}

// Wait until this wave's buffer->LDS fetches have landed (vmcnt counts them;
// nothing else is outstanding in the loop).
__device__ __forceinline__ void wait_fetch_all() { G3K_WAIT_VMEM(); }

// Keeps the compiler's scheduler from moving instructions across this point:
// used to hold fragment reads one step ahead of the MFMAs that consume them.
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// S^T of one key tile for this wave's NQB blocks of 16 queries: keys 0-15
// (s[b][0]) and 16-31 (s[b][1]) of the tile.  Every K fragment read from LDS
// feeds all NQB query blocks; the fragments of step t + 1 are read while
// step t's MFMAs run.
//   Exact policy (X8 = false): three fp16 passes per 32-dim step (k_hi q_hi,
//     k_hi q_lo, k_lo q_hi); qlo holds fp16 q_lo.
//   Fp8 cross policy (X8): one fp16 pass k_hi q_hi over the 8 dim steps, and
//     the cross terms k_hi q_lo + k_lo q_hi as four scaled fp8 MFMAs
//     (v_mfma_scale_f32_16x16x128_f8f6f4, OCP e4m3) over the rows' fp8 half:
//     MFMA j (part p = j / 2: k_hi with q_lo, then k_lo with q_hi) takes the
//     row's 16-byte chunks 8 + 2 j and 9 + 2 j and the query's fp8 bytes
//     qlo[b][2 j], qlo[b][2 j + 1].  The E8M0 scales (key row: sa, query:
//     sb[b]) undo the per-row and per-query exponents and the 2^11 of the
//     low parts, so the cross terms land in the same fp32 accumulator as
//     the fp16 pass.  Eight steps of four fragment reads each: the fp16
//     passes two dim steps at a time, alternating with the fp8 MFMAs.
template <int NQB, bool X8>
__device__ __forceinline__ void tile_scores(f32x4 (&s)[NQB][2], const unsigned char *st, const int (&ka)[4],
                                            const int (&kb)[4], const half8 (&qh)[NQB][8],
                                            const u32x4 (&qlo)[NQB][8], const unsigned char *ks, int krow,
                                            const int (&sb)[NQB]) {
    constexpr int PF = G3K_KPF;       // steps of K fragments in flight
#pragma unroll
    for (int b = 0; b < NQB; b++) s[b][0] = s[b][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 f[PF + 1][4];
    // chunk t (16 bytes of lane group g) of the sub-tile 0 / 1 rows
    auto c0 = [&](int t) { return *reinterpret_cast<const u32x4 *>(st + ka[t & 3] + 256 * (t >> 2)); };
    auto c1 = [&](int t) { return *reinterpret_cast<const u32x4 *>(st + kb[t & 3] + 256 * (t >> 2)); };
    auto load = [&](u32x4 (&r)[4], int t) {
        if (!X8) {   // d-step t: hi and lo chunks of both sub-tiles
            r[0] = c0(t); r[1] = c0(t + 8); r[2] = c1(t); r[3] = c1(t + 8);
        } else if ((t & 1) == 0) {   // d-steps t, t + 1 of the fp16 hi pass
            r[0] = c0(t); r[1] = c1(t); r[2] = c0(t + 1); r[3] = c1(t + 1);
        } else {     // fp8 MFMA j = t / 2: chunks 8 + 2 j, 9 + 2 j
            const int j = t >> 1;
            r[0] = c0(8 + 2 * j); r[1] = c0(9 + 2 * j); r[2] = c1(8 + 2 * j); r[3] = c1(9 + 2 * j);
        }
    };
    // this lane's key rows' scale bytes (sub-tile 0: krow, 1: krow + 4)
    int sa0 = 0, sa1 = 0;
    if (X8) {
        sa0 = ks[krow];
        sa1 = ks[krow + 4];
    }
#pragma unroll
    for (int t = 0; t < PF; t++) load(f[t], t);
    // issue priority for the score MFMAs over the other wave of the SIMD
    // (its softmax and P.V): configs[3] 580.5 -> 570.8 us, configs[2]
    // 52.7 -> 51.9 us; the same around the P.V MFMAs gained nothing
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int t = 0; t < 8; t++) {
        const int c = t % (PF + 1);
        if (t + PF < 8) load(f[(t + PF) % (PF + 1)], t + PF);
        sched_fence();
#pragma unroll
        for (int b = 0; b < NQB; b++) {
            if (!X8) {
                const half8 kh0 = as_half8(f[c][0]), kl0 = as_half8(f[c][1]);
                const half8 kh1 = as_half8(f[c][2]), kl1 = as_half8(f[c][3]);
                const half8 ql = as_half8(qlo[b][t]);
                s[b][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh0, qh[b][t], s[b][0], 0, 0, 0);
                s[b][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh1, qh[b][t], s[b][1], 0, 0, 0);
                s[b][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh0, ql, s[b][0], 0, 0, 0);
                s[b][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh1, ql, s[b][1], 0, 0, 0);
                s[b][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl0, qh[b][t], s[b][0], 0, 0, 0);
                s[b][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl1, qh[b][t], s[b][1], 0, 0, 0);
            } else if ((t & 1) == 0) {
                s[b][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(f[c][0]), qh[b][t], s[b][0], 0, 0, 0);
                s[b][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(f[c][1]), qh[b][t], s[b][1], 0, 0, 0);
                s[b][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(f[c][2]), qh[b][t + 1], s[b][0], 0, 0, 0);
                s[b][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_half8(f[c][3]), qh[b][t + 1], s[b][1], 0, 0, 0);
            } else {
                const int j = t >> 1;
                const i32x8 qx = cat8(qlo[b][2 * j], qlo[b][2 * j + 1]);
                s[b][0] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(cat8(f[c][0], f[c][1]), qx, s[b][0], 0, 0,
                                                                           0, sa0, 0, sb[b]);
                s[b][1] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(cat8(f[c][2], f[c][3]), qx, s[b][1], 0, 0,
                                                                           0, sa1, 0, sb[b]);
            }
        }
        sched_fence();
    }
    __builtin_amdgcn_s_setprio(0);
}

// Loads, QK-norms and rotates (gemma3_kernels.c:289-304, 470-484) one block of
// 16 queries into the B-operand layout and splits it: qh = fp16(v), and in
// qlo either fp16(v - qh) (exact policy) or, for the fp8 cross policy, the
// query's fp8 operand bytes of the four cross MFMAs: MFMA j = 2 p + jj takes
// part p (0: (v - qh) 2^11 / 2^E, 1: qh / 2^E) of dims 32 t + 8 g + u,
// t = 4 jj .. 4 jj + 3, at byte 8 (t - 4 jj) + u of qlo[2 j] | qlo[2 j + 1]
// (the key rows' fp8 bytes are in the same order), with E the query's
// exponent (x8_exponent of its largest |v|) and sb the E8M0 code 127 + E -
// 11 of the product scale.
// Lane (ln, g) holds dims 32 t + 8 g + u; dim d < 128 and its RoPE partner
// d + 128 are t and t + 4 of the same lane.
template <bool X8>
__device__ __forceinline__ void load_queries(half8 (&qh)[8], u32x4 (&qlo)[8], int &sb, const g3k_prefill_args &p,
                                             int tok, int qhead, int n_heads, int g) {
    // Arithmetic exactly as written (explicit fmaf where fused): how the
    // compiler would otherwise fuse multiplies into adds can differ between
    // the kernel forms this is inlined into, and the forms must agree bit for
    // bit.
#pragma clang fp contract(off)
    const bool qv = tok < p.n;
    const float *qrow = p.q + ((size_t)(qv ? tok : 0) * n_heads + qhead) * D + 8 * g;
    const float *rrow = p.rope + (size_t)(p.start_pos + (qv ? tok : 0)) * D + 2 * 8 * g;
    // Every load of the prologue is issued before the first use: the query
    // row, the norm gains and the RoPE table row come back in one memory
    // round trip.  (Without q_norm the gain load reads a valid row of the
    // table and its values are not used: no branch between the loads.)
    float x[8][8];
    uint4 wv[8];
    float4 cs[4][4];
#pragma unroll
    for (int t = 0; t < 8; t++) {
        const float4 a = *reinterpret_cast<const float4 *>(qrow + 32 * t);
        const float4 b = *reinterpret_cast<const float4 *>(qrow + 32 * t + 4);
        x[t][0] = a.x; x[t][1] = a.y; x[t][2] = a.z; x[t][3] = a.w;
        x[t][4] = b.x; x[t][5] = b.y; x[t][6] = b.z; x[t][7] = b.w;
    }
    const uint16_t *wrow = p.q_norm ? p.q_norm : reinterpret_cast<const uint16_t *>(p.rope);
#pragma unroll
    for (int t = 0; t < 8; t++) wv[t] = *reinterpret_cast<const uint4 *>(wrow + 32 * t + 8 * g);
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int h = 0; h < 4; h++) cs[t][h] = *reinterpret_cast<const float4 *>(rrow + 64 * t + 4 * h);
    // keep the scheduler from sinking the gain and table loads below the
    // query row's waits (which would make them further round trips)
    __builtin_amdgcn_sched_barrier(0);
    if (p.q_norm) {
        float ss = 0.f;
#pragma unroll
        for (int t = 0; t < 8; t++)
#pragma unroll
            for (int u = 0; u < 8; u++) ss = fmaf(x[t][u], x[t][u], ss);
        ss = col4_sum(ss);
        // x r (1 + w) with the softmax scale folded into r (RoPE is linear),
        // and zero for a query column past the batch
        const float rq = qv ? (1.0f / sqrtf(ss / (float)D + p.eps)) * p.qscale : 0.f;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const uint32_t w[4] = {wv[t].x, wv[t].y, wv[t].z, wv[t].w};
#pragma unroll
            for (int u = 0; u < 8; u++)
                x[t][u] = x[t][u] * fmaf(rq, bf16f((w[u >> 1] >> (16 * (u & 1))) & 0xffff), rq);
        }
    }
#pragma unroll
    for (int t = 0; t < 4; t++) {
#pragma unroll
        for (int h = 0; h < 4; h++) {
            const float c[2] = {cs[t][h].x, cs[t][h].z}, sn[2] = {cs[t][h].y, cs[t][h].w};
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int u = 2 * h + e;
                const float a = x[t][u], b = x[t + 4][u];
                x[t][u] = fmaf(a, c[e], -(b * sn[e]));
                x[t + 4][u] = fmaf(a, sn[e], b * c[e]);
            }
        }
    }
    // without QK-norm the scale (and the zero past the batch) comes here
    const float qsc = p.q_norm ? 1.f : (qv ? p.qscale : 0.f);
    float mloc = 0.f;
#pragma unroll
    for (int t = 0; t < 8; t++)
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float v = p.q_norm ? x[t][u] : x[t][u] * qsc;
            const _Float16 hi = (_Float16)v;
            qh[t][u] = hi;
            x[t][u] = v - (float)hi;      // the low part, exact in fp32
            mloc = fmaxf(mloc, fabsf(v));
        }
    if (!X8) {
#pragma unroll
        for (int t = 0; t < 8; t++) {
            half8 l;
#pragma unroll
            for (int u = 0; u < 8; u++) l[u] = (_Float16)x[t][u];
            qlo[t] = __builtin_bit_cast(u32x4, l);
        }
        sb = 0;
        return;
    }
    // the query's exponent: its 256 dims are in the four lanes ln + 16 g;
    // at least -115 so that the product scale's code 127 + E - 11 stays >= 1
    int E = x8_exponent(col4_max(mloc));
    E = E < -115 ? -115 : E;
    sb = 127 + E - 11;
    const float inv = __builtin_amdgcn_ldexpf(1.0f, -E), inv_lo = __builtin_amdgcn_ldexpf(1.0f, 11 - E);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int part = j >> 1, jj = j & 1;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            u32x4 w;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                // bytes 16 h + 4 k .. + 3: t = 4 jj + 2 h + k / 2, u = 4 (k % 2) .. + 3
                const int t = 4 * jj + 2 * h + (k >> 1), u0 = 4 * (k & 1);
                float y[4];
#pragma unroll
                for (int e = 0; e < 4; e++)
                    y[e] = part == 0 ? x[t][u0 + e] * inv_lo : (float)qh[t][u0 + e] * inv;
                w[k] = e4m3_pair(y[2], y[3], e4m3_pair(y[0], y[1]), true);
            }
            qlo[2 * j + h] = w;
        }
    }
}

// One workgroup's attention: 8 / NQB waves, each owning NQB blocks of 16
// queries of one head over the full head dim.  VLO adds the P_hi.V_lo pass;
// X8 selects the fp8 cross policy of the scores (staged key rows in that
// format, with a ring of the tiles' key-scale bytes after the V ring).
template <int G, int NQB, bool VLO, bool X8>
__device__ __forceinline__ void attend(const g3k_prefill_args &p, unsigned char *smem) {
    constexpr int NW = 8 / NQB;       // waves per workgroup
    constexpr int WPH = NW / G;       // waves per query head
    constexpr int QW = 16 * NQB;      // queries per wave
    constexpr int PB = QW * WPH;      // query positions per workgroup
    constexpr int VST = VTILEB * (VLO ? 2 : 1);   // V ring slot: hi (| lo)
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // The wave index is uniform per wave; saying so for the fetches keeps
    // their offsets and LDS addresses in SGPRs (no per-lane loop around each).
    const int fwave = __builtin_amdgcn_readfirstlane(wave);
    const int g = lane >> 4, ln = lane & 15;     // lane group, query column
    // 1-D grid, longest (latest) query blocks first across all heads: with
    // workgroups dealt round-robin to the 8 XCDs, block id -> (qb, id % H_kv)
    // also keeps each XCD on one KV head (its L2 streams one head's K / V).
    // With key splits, block id -> (qb, split, kvh), kvh fastest; when H_kv
    // divides 8 and the blocks fill whole groups of Q = 8 / H_kv, the splits
    // of one (qb, kvh) are 8 ids apart instead (ids sg * 8 S + split * 8 +
    // (qb % Q) * H_kv + kvh), so they share an XCD and its L2 serves the
    // block's query rows and RoPE rows once for all of them.
    const int S = p.ksplit;
    const int nbq = (int)(gridDim.x / (p.n_kv_heads * S));   // query blocks
    int kvh, split, qbi;
    if (S > 1 && 8 % p.n_kv_heads == 0 && nbq % (8 / p.n_kv_heads) == 0) {
        const int Q = 8 / p.n_kv_heads;
        const int id = (int)blockIdx.x, sg = id / (8 * S), r = id % (8 * S);
        split = r / 8;
        kvh = (r % 8) % p.n_kv_heads;
        qbi = sg * Q + (r % 8) / p.n_kv_heads;
    } else {
        kvh = blockIdx.x % p.n_kv_heads;
        const int pair = (int)(blockIdx.x / p.n_kv_heads);
        split = pair % S;
        qbi = pair / S;
    }
    const int qb = nbq - 1 - qbi;
    const int qhead = kvh * G + wave / WPH;
    // uniform, so the wave's query range and tile bounds below stay in
    // SGPRs (the head and the phase order stay per lane: as uniform values
    // they made the compiler move the O^T accumulators at every phase join)
    const int tok0 = qb * PB + (fwave % WPH) * QW;
    const bool wave_live = tok0 < p.n;
    // waves w and w + 4 share a SIMD; with schedule 1 the upper four run each
    // tile's softmax + P.V before the next tile's scores
    const bool late = NW == 8 && ((p.schedule == 1 && (wave >> 2) == 1) || (p.schedule == 2 && (wave & 1)));

    // key index range of the workgroup and of this wave (inclusive)
    const int wg_first = p.hist + qb * PB;
    const int wg_last = min(p.hist + min(qb * PB + PB, p.n) - 1, p.nk - 1);
    int kt0 = max(0, wg_first - p.window + 1) / BK;
    int kt1 = wg_last / BK;
    if (S > 1) {   // this split's consecutive part of the tiles (may be empty)
        const int per = (kt1 - kt0 + S) / S;
        kt0 += split * per;
        kt1 = min(kt1, kt0 + per - 1);
    }
    const int w_first = p.hist + tok0;
    const int w_last = min(w_first + QW - 1, p.hist + p.n - 1);
    const int wkt0 = max(0, w_first - p.window + 1) / BK;
    const int wkt1 = w_last / BK;

    // this KV head's staged keys and values as buffer descriptors
    const int ldk = (int)p.ldk;
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(p.kq + (size_t)kvh * ldk * (2 * D), (unsigned)ldk * (4 * D));
    const __amdgpu_buffer_rsrc_t vr = make_rsrc(p.vt + (size_t)kvh * D * ldk, (unsigned)ldk * (2 * D));
    const __amdgpu_buffer_rsrc_t vlr = make_rsrc(p.vt_lo + (size_t)kvh * D * ldk, (unsigned)ldk * (2 * D));
    const unsigned voff_v = (unsigned)((lane >> 2) * ldk * 2 + ((lane & 3) ^ ((lane >> 4) & 3)) * 16);
    auto kbuf = [&](int kt) { return smem + (kt & 1) * KTILEB; };
    auto vbuf = [&](int kt) { return smem + LDS_V0 + (kt & 1) * VST; };
    auto fetch_vt = [&](int kt) {
        fetch_v<NW>(vbuf(kt), vr, kt, fwave, voff_v, ldk);
        if (VLO) fetch_v<NW>(vbuf(kt) + VTILEB, vlr, kt, fwave, voff_v, ldk);
    };
    // fp8 cross policy: tile kt's 32 key-scale bytes -> its scale slot, one
    // 4-byte buffer -> LDS fetch per lane of wave 0 (the 256 bytes past the
    // tile's 32 are unused; past the head's ldk bytes they read as zero)
    const __amdgpu_buffer_rsrc_t ksr = make_rsrc(X8 ? (const void *)(p.kscale + (size_t)kvh * ldk) : (const void *)p.kq, (unsigned)ldk);
    auto ksbuf = [&](int kt) { return smem + LDS_KS0 + (kt & 1) * KS_SLOT; };
    auto fetch_kt = [&](int kt) {
        fetch_k<NW>(kbuf(kt), kr, kt, fwave, lane);
        if (X8 && fwave == 0)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ksr, (lds_ptr)ksbuf(kt), 4, lane * 4, kt * BK, 0, 0);
    };

    // ---- K of the first two tiles and V of the first in flight, then this
    // wave's queries ----
    fetch_kt(kt0);
    if (kt0 + 1 <= kt1) fetch_kt(kt0 + 1);
    fetch_vt(kt0);

    half8 qh[NQB][8];
    u32x4 qlo[NQB][8];
    int sb[NQB];
#pragma unroll
    for (int b = 0; b < NQB; b++)
        load_queries<X8>(qh[b], qlo[b], sb[b], p, tok0 + 16 * b + ln, qhead, p.n_kv_heads * G, g);

    f32x4 o[NQB][16];
    float m_ref[NQB], l_sum[NQB];
#pragma unroll
    for (int b = 0; b < NQB; b++) {
        m_ref[b] = NEG_BIG;
        l_sum[b] = 0.f;
#pragma unroll
        for (int mt = 0; mt < 16; mt++) o[b][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // per-lane LDS byte offsets: K rows of the two S^T sub-tiles (row m ->
    // key 8 (m / 4) + 4 j + m % 4) at chunk g, and the V^T row ln of each
    // 16-dim block at its swizzled chunk g
    const int krow = 8 * (ln >> 2) + (ln & 3);
    // logical chunk g + 4 t of row r sits at chunk (g ^ fl) + 4 (t ^ fh), with
    // fl = kswz(r) & 3 and fh = kswz(r) >> 2: four bases per row for t % 4,
    // t / 4 as an immediate (kswz(krow + 4) == kswz(krow))
    int koff0[4], koff1[4];
    {
        const int f = kswz(krow), fl = f & 3, fh = f >> 2;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            koff0[u] = krow * KROWB + 16 * (g ^ fl) + 64 * (u ^ fh);
            koff1[u] = (krow + 4) * KROWB + 16 * (g ^ fl) + 64 * (u ^ fh);
        }
    }
    const int voff = ln * 64 + 16 * (g ^ vswz(ln));

    wait_fetch_all();
    __syncthreads();

    // Software pipeline: iteration kt issues tile kt+1's S^T MFMAs and tile
    // kt's softmax + P.V (in either order, see `late`).
    // Two score sets, used in turn (the loop is unrolled by two), so no
    // iteration copies one into the other.  A set is read only for a tile
    // the wave scored into it (the same liveness test on both sides).
    f32x4 sc0[NQB][2], sc1[NQB][2];
#pragma unroll
    for (int b = 0; b < NQB; b++) sc1[b][0] = sc1[b][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (wave_live && kt0 >= wkt0 && kt0 <= wkt1)
        tile_scores<NQB, X8>(sc0, kbuf(kt0), koff0, koff1, qh, qlo, ksbuf(kt0), krow, sb);
    // the first iteration refills K tile kt0's slot: every wave must be done
    // reading it
    __syncthreads();

    // iteration kt: s holds tile kt's scores, sn receives tile kt + 1's
    auto step = [&](int kt, f32x4 (&s)[NQB][2], f32x4 (&sn)[NQB][2]) {
        // K of tile kt + 2 replaces K of tile kt (scored last iteration), V
        // of tile kt + 1 replaces V of tile kt - 1
        if (kt + 2 <= kt1) fetch_kt(kt + 2);
        if (kt + 1 <= kt1) fetch_vt(kt + 1);
        const unsigned char *vs = vbuf(kt);

        auto scores_next = [&]() {
            if (wave_live && kt + 1 >= wkt0 && kt + 1 <= wkt1)
                tile_scores<NQB, X8>(sn, kbuf(kt + 1), koff0, koff1, qh, qlo, ksbuf(kt + 1), krow, sb);
        };
        auto softmax_pv = [&]() {
          if (wave_live && kt >= wkt0 && kt <= wkt1) {
            // the first V^T fragments load while the softmax runs
            constexpr int VPF = G3K_VPF;
            bf16x8 vf[VPF + 1], vl[VPF + 1];
#pragma unroll
            for (int i = 0; i < VPF; i++) {
                vf[i] = *reinterpret_cast<const bf16x8 *>(vs + voff + 1024 * i);
                if (VLO) vl[i] = *reinterpret_cast<const bf16x8 *>(vs + VTILEB + voff + 1024 * i);
            }
            const bool edge = (kt * BK + BK - 1 > w_first) || (kt * BK <= w_last - p.window) ||
                              (kt * BK + BK > p.nk);
            bf16x8 ph[NQB], pl[NQB];
#pragma unroll
            for (int b = 0; b < NQB; b++) {
                // register u of this lane: key kt*32 + 8 g + u (u < 4: s[b][0][u], else s[b][1][u-4])
                // ---- mask (diagonal, window edge, ragged end), in place ----
                if (edge) {
                    // the query at key index q_kk sees keys q_kk - window + 1
                    // .. min(q_kk, nk - 1): here u = lo .. hi
                    const int q_kk = p.hist + tok0 + 16 * b + ln;
                    const int base = kt * BK + 8 * g;
                    const int lo = q_kk - p.window + 1 - base, hi = min(q_kk, p.nk - 1) - base;
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        const bool ok = u >= lo && u <= hi;
                        s[b][u >> 2][u & 3] = ok ? s[b][u >> 2][u & 3] : -INFINITY;
                    }
                }
                float sv[8] = {s[b][0][0], s[b][0][1], s[b][0][2], s[b][0][3],
                               s[b][1][0], s[b][1][1], s[b][1][2], s[b][1][3]};
                // ---- online softmax with a lazy reference max ----
                // The lane's own eight keys first: the max over the query's
                // four lanes is needed only when one of them passes the lazy
                // bound, which the ballot shows as well.
                float mx = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                                 fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
                if (__builtin_amdgcn_ballot_w64(mx > m_ref[b] + LAZY)) {
                    mx = col4_max(mx);
                    const bool bump = mx > m_ref[b] + LAZY;
                    const float m_new = bump ? mx : m_ref[b];
                    const float alpha = fast_exp2(m_ref[b] - m_new);
                    m_ref[b] = m_new;
                    l_sum[b] *= alpha;
#pragma unroll
                    for (int mt = 0; mt < 16; mt++) o[b][mt] *= alpha;
                }
                float pr[8];
#pragma unroll
                for (int u = 0; u < 8; u++) pr[u] = fast_exp2(sv[u] - m_ref[b]);   // exp2(-inf) = 0 for masked keys
                // this lane's keys (the four lanes add up at the end), as a tree
                l_sum[b] += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
                // P = hi + lo, two bf16 (round to nearest even) per word: each
                // pair is converted once, and its hi values come back as floats
                // by a shift and a mask
                u32x4 hw, lw;
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const uint32_t h = bf16_pair(pr[2 * u], pr[2 * u + 1]);
                    hw[u] = h;
                    lw[u] = bf16_pair(pr[2 * u] - __uint_as_float(h << 16), pr[2 * u + 1] - __uint_as_float(h & 0xffff0000u));
                }
                ph[b] = __builtin_bit_cast(bf16x8, hw);
                pl[b] = __builtin_bit_cast(bf16x8, lw);
            }
            // ---- O^T += V^T . P^T over 16 dim blocks; the V^T fragments of
            // block mt + VPF are read while block mt's MFMAs run ----
#pragma unroll
            for (int mt = 0; mt < 16; mt++) {
                if (mt + VPF < 16) {
                    vf[(mt + VPF) % (VPF + 1)] = *reinterpret_cast<const bf16x8 *>(vs + voff + 1024 * (mt + VPF));
                    if (VLO)
                        vl[(mt + VPF) % (VPF + 1)] =
                            *reinterpret_cast<const bf16x8 *>(vs + VTILEB + voff + 1024 * (mt + VPF));
                }
                sched_fence();
#pragma unroll
                for (int b = 0; b < NQB; b++) {
                    const bf16x8 v = vf[mt % (VPF + 1)];
                    o[b][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v, ph[b], o[b][mt], 0, 0, 0);
                    o[b][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v, pl[b], o[b][mt], 0, 0, 0);
                    if (VLO)
                        o[b][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl[mt % (VPF + 1)], ph[b], o[b][mt], 0,
                                                                          0, 0);
                }
                sched_fence();
            }
          }
        };
        // The two waves of a SIMD run the phases in opposite order, so one's
        // softmax (VALU) overlaps the other's matrix work.
        if (late) {
            softmax_pv();
            scores_next();
        } else {
            scores_next();
            softmax_pv();
        }

        // K of tile kt + 2 and V of tile kt + 1 must have landed before the
        // barrier (next iteration's scores and P.V)
        wait_fetch_all();
        __syncthreads();
    };
    for (int kt = kt0; kt <= kt1; kt += 2) {
        step(kt, sc0, sc1);
        if (kt + 1 <= kt1) step(kt + 1, sc1, sc0);
    }

    // ---- normalise and write attn_out[token][qhead][dim]; with key splits,
    // publish this split's unnormalised part and let the last split of the
    // block to arrive merge them ----
    if (S > 1) {
        const int hq = p.n_kv_heads * G;
        // Parts are written and read with agent-coherent (sc1) accesses,
        // which go to and come from the point of coherence shared by all
        // XCDs, so no cache-wide writeback or invalidate is needed.  (An
        // agent-scope __threadfence does both to the XCD's whole L2; with
        // one per workgroup configs[2] took 188 us instead of 53.)  The
        // parts of split s of this block are one run of PB * H_q rows: one
        // descriptor per split, offsets relative to the block's first token.
        auto part_rsrc = [&](int sp) {
            return make_rsrc(p.part_o + ((size_t)sp * p.n + (size_t)qb * PB) * hq * D, (unsigned)(PB * hq * D * 4));
        };
        float lt[NQB];
#pragma unroll
        for (int b = 0; b < NQB; b++) {
            lt[b] = col4_sum(l_sum[b]);   // all lanes active here
            const int tok = tok0 + 16 * b + ln;
            if (!wave_live || tok >= p.n) continue;
            const __amdgpu_buffer_rsrc_t pr = part_rsrc(split);
            const unsigned voff = (unsigned)((((tok - qb * PB) * hq + qhead) * D + 4 * g) * 4);
#pragma unroll
            for (int mt = 0; mt < 16; mt++)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[b][mt]), pr, voff + 64 * mt, 0, CP_SC1);
            if (g == 0) {
                float *ml = p.part_ml + (((size_t)split * p.n + tok) * hq + qhead) * 2;
                __hip_atomic_store(ml, m_ref[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(ml + 1, lt[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        // Every part store of the wave has completed (vmcnt counts stores on
        // this family) before the block's arrival is counted; the counter
        // wraps to 0 on the S-th arrival, ready for the next call.  The
        // loop's last barrier has retired every LDS access, so the flag
        // reuses smem.
        G3K_WAIT_VMEM();
        __syncthreads();
        int *last = reinterpret_cast<int *>(smem);
        if (tid == 0) *last = atomicInc(p.arrive + (size_t)qb * p.n_kv_heads + kvh, (unsigned)(S - 1)) == (unsigned)(S - 1);
        __syncthreads();
        if (!*last || !wave_live) return;
        // merge in split order, as out = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s;
        // this split's part is still in registers
#pragma unroll
        for (int b = 0; b < NQB; b++) {
            const int tok = tok0 + 16 * b + ln;
            if (tok >= p.n) continue;
            const unsigned voff = (unsigned)((((tok - qb * PB) * hq + qhead) * D + 4 * g) * 4);
            // S <= 4: fixed trip counts keep ms / ls in registers
            float ms[4], ls[4];
            float M = NEG_BIG;
#pragma unroll
            for (int sp = 0; sp < 4; sp++) {
                if (sp >= S) break;
                if (sp == split) {
                    ms[sp] = m_ref[b];
                    ls[sp] = lt[b];
                } else {
                    const float *ml = p.part_ml + (((size_t)sp * p.n + tok) * hq + qhead) * 2;
                    ms[sp] = __hip_atomic_load(ml, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ls[sp] = __hip_atomic_load(ml + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                M = fmaxf(M, ms[sp]);
            }
            float L = 0.f;
            f32x4 A[16];
#pragma unroll
            for (int mt = 0; mt < 16; mt++) A[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int sp = 0; sp < 4; sp++) {
                if (sp >= S) break;
                const float f = fast_exp2(ms[sp] - M);
                L += ls[sp] * f;
                if (sp == split) {
#pragma unroll
                    for (int mt = 0; mt < 16; mt++) A[mt] += o[b][mt] * f;
                } else {
                    const __amdgpu_buffer_rsrc_t pr = part_rsrc(sp);
#pragma unroll
                    for (int mt = 0; mt < 16; mt++)
                        A[mt] += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(pr, voff + 64 * mt, 0, CP_SC1)) * f;
                }
            }
            const float inv = 1.0f / L;
            float *orow = p.out + ((size_t)tok * hq + qhead) * D + 4 * g;
#pragma unroll
            for (int mt = 0; mt < 16; mt++)
                *reinterpret_cast<float4 *>(orow + 16 * mt) =
                    make_float4(A[mt][0] * inv, A[mt][1] * inv, A[mt][2] * inv, A[mt][3] * inv);
        }
        return;
    }
    if (!wave_live) return;
#pragma unroll
    for (int b = 0; b < NQB; b++) {
        const float inv = 1.0f / col4_sum(l_sum[b]);   // all lanes active here
        const int tok = tok0 + 16 * b + ln;
        if (tok >= p.n) continue;
        float *orow = p.out + ((size_t)tok * p.n_kv_heads * G + qhead) * D + 4 * g;
#pragma unroll
        for (int mt = 0; mt < 16; mt++)
            *reinterpret_cast<float4 *>(orow + 16 * mt) =
                make_float4(o[b][mt][0] * inv, o[b][mt][1] * inv, o[b][mt][2] * inv, o[b][mt][3] * inv);
    }
}

// The V_lo pass is taken when this call's staging found a V that is not
// exactly bf16 (flag == epoch); the branch is uniform over the grid.
template <int G, int NQB, bool X8>
__global__ __launch_bounds__(512 / NQB, 1) void prefill_kernel(g3k_prefill_args p) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[X8 ? LDS_BYTES_X8 : LDS_BYTES];
    if (*p.v_lo_flag == p.epoch)
        attend<G, NQB, true, X8>(p, smem);
    else
        attend<G, NQB, false, X8>(p, smem);
}

template <int G, int NQB>
hipError_t launch_prefill(const g3k_prefill_args *a, hipStream_t st) {
    constexpr int PB = 16 * NQB * ((8 / NQB) / G);
    const int nqb = (a->n + PB - 1) / PB;
    const dim3 grid(nqb * a->n_kv_heads * a->ksplit);
    // With timing events the dispatch itself records them (kernel begin / end).
    if (a->kscale)
        hipExtLaunchKernelGGL((prefill_kernel<G, NQB, true>), grid, dim3(512 / NQB), 0, st, (hipEvent_t)a->ev0,
                              (hipEvent_t)a->ev1, 0, *a);
    else
        hipExtLaunchKernelGGL((prefill_kernel<G, NQB, false>), grid, dim3(512 / NQB), 0, st, (hipEvent_t)a->ev0,
                              (hipEvent_t)a->ev1, 0, *a);
    return hipGetLastError();
}

}  // namespace

extern "C" int g3k_stage(const g3k_stage_args *a, void *stream) {
    if (a->cnt <= 0) return 0;
    if (a->ldk % 64 || a->kk0 + a->cnt > a->ldk || !a->v_lo_flag) return (int)hipErrorInvalidValue;
    const long long kblocks = (a->cnt + 63) / 64;
    const long long vblocks = kblocks * (D / 64) * a->n_kv_heads;
    const long long kr_blocks = (krow_count(*a) + 3) / 4;
    if (vblocks + kr_blocks > 0x7fffffffLL) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(stage_kernel, dim3((unsigned)(vblocks + kr_blocks)), dim3(NT), 0, (hipStream_t)stream, *a,
                       (unsigned)vblocks, (unsigned)kblocks);
    return (int)hipGetLastError();
}

extern "C" int g3k_rope_write_stage(const g3k_rope_write_args *ra, const g3k_stage_args *sa, void *stream) {
    if (ra->n <= 0 && sa->cnt <= 0) return 0;
    if (sa->cnt > 0 && (sa->ldk % 64 || sa->kk0 + sa->cnt > sa->ldk || !sa->v_lo_flag)) return (int)hipErrorInvalidValue;
    if (ra->n > 0 && ra->Q) return (int)hipErrorInvalidValue;   // the prefill front end stages no queries
    const long long kblocks = sa->cnt > 0 ? (sa->cnt + 63) / 64 : 0;
    const long long stage_blocks = kblocks * (D / 64) * sa->n_kv_heads;
    // the staging blocks write the batch's V rows to the cache: they must
    // cover every token of ra (key indices kk0 .. kk0 + n - 1, positions
    // start_pos ..) and read V from the batch's own rows
    if (ra->n > 0 && (sa->cnt < ra->n || sa->nk != sa->kk0 + ra->n || sa->k_src || sa->ring ||
                      sa->row_pos0 != ra->start_pos ||
                      sa->kstart + sa->kk0 != ra->start_pos || sa->v_src != ra->V || sa->n_kv_heads != ra->n_kv_heads ||
                      ra->kq != sa->kq || ra->kscale != sa->kscale || ra->row0 != sa->kk0 || ra->ldk != sa->ldk))
        return (int)hipErrorInvalidValue;
    const long long rw_blocks = ra->n > 0 ? ((long long)ra->n * ra->n_kv_heads + 3) / 4 : 0;
    const long long pad_blocks = sa->cnt > 0 ? (krow_count(*sa) + 3) / 4 : 0;
    if (stage_blocks + rw_blocks + pad_blocks > 0x7fffffffLL) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(front_kernel, dim3((unsigned)(stage_blocks + rw_blocks + pad_blocks)), dim3(NT), 0,
                       (hipStream_t)stream, *ra, *sa, (unsigned)stage_blocks, (unsigned)kblocks, (unsigned)rw_blocks);
    return (int)hipGetLastError();
}

extern "C" int g3k_prefill(const g3k_prefill_args *a, void *stream) {
    if (a->n <= 0) return 0;
    // buffer descriptors address one head's staging: ldk * 1 KiB must fit
    // the 32-bit record count and the fetch offsets
    if (a->ldk % 64 || a->ldk > (1LL << 20) || a->nk > a->ldk || a->hist + a->n != a->nk ||
        a->window < 1 || !a->v_lo_flag)
        return (int)hipErrorInvalidValue;
    if ((a->ksplit != 1 && a->ksplit != 2 && a->ksplit != 4) ||
        (a->ksplit > 1 && (!a->part_o || !a->part_ml || !a->arrive)))
        return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    const bool wide = a->queries_per_wave == 32;
    switch (a->group) {
        case 1: return (int)(wide ? launch_prefill<1, 2>(a, st) : launch_prefill<1, 1>(a, st));
        case 2: return (int)(wide ? launch_prefill<2, 2>(a, st) : launch_prefill<2, 1>(a, st));
        case 4: return (int)(wide ? launch_prefill<4, 2>(a, st) : launch_prefill<4, 1>(a, st));
        default: return (int)hipErrorInvalidValue;
    }
}
