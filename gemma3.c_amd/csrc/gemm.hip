// gemm.hip - the batched-prefill projections on MFMA (gfx950).
//
// Replaces the bf16 -> fp32 weight conversion + cblas_sgemm pairs of the
// reference's batched prefill (gemma3_transformer.c:614-639 Q/K/V, 694-699
// o_proj, 726-751 gate / up / down): C[n][m] = sum_k X[n][k] W[m][k], X the
// fp32 activations of N tokens [N][K], W a bf16 weight matrix [M][K].
//
// Precision.  W is exact in bf16.  X is fp32; it arrives split into two bf16
// planes, x = x_hi + x_lo (x_hi = bf16(x), x_lo = bf16(x - x_hi): 16
// significant bits, relative error <= 2^-17), written by the kernel that
// produces X.  Each product is W.x_hi + W.x_lo on v_mfma_f32_16x16x32_bf16
// with fp32 accumulation: twice the algorithmic MFMA work, within a few
// 2^-17 of the reference's fp32 sgemm.
//
// Tiling.  Workgroup = 4 waves = a 128 (weight rows) x 128 (tokens) tile of
// C; wave (wm, wn) owns 64 x 64 of it, 4 x 4 MFMA tiles of 16 x 16 (64
// accumulator registers).  K advances 32 at a time: per stage the W tile and
// the x_hi / x_lo tiles (128 rows x 32 k each, 8 KiB) move from global memory
// straight into LDS with buffer -> LDS loads (buffer_load_dwordx4 ... lds, one
// wave instruction = 1 KiB = 16 rows).  Rows beyond M or N read zero (the
// buffer descriptor's range check), so ragged tiles need no masking until the
// stores.  LDS rows are 64 B; within each 16-row group the four 16-byte
// chunks of row r sit at slot 4 r + (c ^ (r / 4 % 4)), so a fragment read (16
// rows, one chunk) touches all 64 banks once.  MFMA operands: A = W rows (lane
// l: row l % 16, k 8 (l / 16) .. + 7), B = X rows in the same pattern; the
// accumulator of lane l holds C rows m = 4 (l / 16) + i for token l % 16.
//
// Modes.  PLAIN: up to three weight matrices that share X in one launch (the
// Q, K and V projections), each written as fp32 C [N][ldc].  GEGLU: the gate
// and up matrices together; the epilogue computes gelu_tanh(gate) * up
// (gemma3_transformer.c:741-745) and writes it as the bf16 hi / lo planes
// that the down projection reads.
#include <hip/hip_runtime.h>

#include "g3k.h"
#include "g3k_device.h"

namespace {

using namespace g3k;

constexpr int BN = 128, BK = 32, NT = 256;
constexpr int TILE_B = 128 * BK * 2;   // one operand tile in LDS: 8 KiB

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void *lds_ptr;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// Byte offset, inside a tile, of chunk c (8 k values) of row r.
__device__ __forceinline__ int tile_off(int r, int c) {
    return ((r >> 4) * 64 + (r & 15) * 4 + (c ^ ((r >> 2) & 3))) * 16;
}

// Copy rows row0 .. row0 + 127, k0 .. k0 + 31 of a [rows][ld] bf16 matrix
// into an LDS tile.  Wave w moves the 16-row groups w and w + 4; lane i of
// a group instruction lands at byte 16 i of the group, which is slot i =
// 4 r + c' with c' = c ^ (r / 4 % 4).
__device__ __forceinline__ void fetch_tile(__amdgpu_buffer_rsrc_t rs, char *tile, int row0, int ld, int k0,
                                           int wave, int lane) {
    const int r = lane >> 2, cp = lane & 3;
    const int c = cp ^ ((r >> 2) & 3);
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int g = wave + 4 * h;
        const int row = row0 + g * 16 + r;
        const uint32_t voff = (uint32_t)row * (uint32_t)ld * 2u + (uint32_t)(k0 + c * 8) * 2u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(tile + g * 1024), 16, voff, 0, 0, 0);
    }
}

__device__ __forceinline__ bf16x8 frag(const char *tile, int r, int c) {
    return *reinterpret_cast<const bf16x8 *>(tile + tile_off(r, c));
}

__device__ __forceinline__ float gelu_tanh(float x) {
    const float inner = 0.7978845608028654f * (x + 0.044715f * (x * x * x));
    return 0.5f * x * (1.0f + tanhf(inner));
}

// bf16 round-to-nearest-even of a finite float, as bits.
__device__ __forceinline__ uint32_t bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// MT: 16-row MFMA tiles per wave along the weight rows (4 or 8).  The
// workgroup's 4 waves sit 2 (rows) x 2 (tokens); the W region of a stage
// holds 32 MT rows (GEGLU, MT = 8: 128 gate rows, then the same 128 up rows).
// Wave (wm, wn) owns rows wm * 16 MT .. of the region (GEGLU: 64 gate rows and
// the same 64 up rows) and tokens wn * 64 .. + 63.  Per 32-wide k step a wave
// reads MT W fragments and 8 x fragments (4 hi, 4 lo) for 8 MT MFMAs.
// blockIdx.z = k split: split s sums k in [s K / S, (s + 1) K / S) and writes
// C + s * split_stride (the consumer adds the S partial products).
template <bool GEGLU, int MT>
__global__ __launch_bounds__(NT, 2) void gemm_kernel(g3k_gemm_args a) {
    static_assert(!GEGLU || MT == 8, "GEGLU tiles pair 4 gate and 4 up tiles per wave");
    constexpr int RW = 32 * MT;                          // W rows per stage
    constexpr int W_B = RW * BK * 2;
    constexpr int STAGE_B = W_B + 2 * TILE_B;
    __shared__ __attribute__((aligned(1024))) char smem[2 * STAGE_B];

    // this workgroup's weight matrix and row block
    constexpr int BMW = GEGLU ? RW / 2 : RW;             // matrix rows per workgroup
    int bx = blockIdx.x, m_idx = 0;
    if (!GEGLU) {
        while (m_idx + 1 < a.n_mat && bx >= (a.M[m_idx] + BMW - 1) / BMW) {
            bx -= (a.M[m_idx] + BMW - 1) / BMW;
            m_idx++;
        }
    }
    const int M = a.M[m_idx], K = a.K, N = a.N;
    const int m0 = bx * BMW, n0 = blockIdx.y * BN;
    const int kc = K / a.ksplit, kbeg = blockIdx.z * kc;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;

    const uint32_t wbytes = (uint32_t)((size_t)M * K * 2);
    const __amdgpu_buffer_rsrc_t rw0 = rsrc(a.W[GEGLU ? 0 : m_idx], wbytes);
    const __amdgpu_buffer_rsrc_t rw1 = rsrc(a.W[GEGLU ? 1 : m_idx], wbytes);
    const uint32_t xbytes = (uint32_t)((size_t)N * a.ldx * 2);
    const __amdgpu_buffer_rsrc_t rxh = rsrc(a.x_hi, xbytes), rxl = rsrc(a.x_lo, xbytes);

    f32x4 acc[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < 4; nt++) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto fetch = [&](int s, int k0) {
        char *st = smem + s * STAGE_B;
        if (GEGLU) {
            fetch_tile(rw0, st, m0, K, k0, wave, lane);
            fetch_tile(rw1, st + TILE_B, m0, K, k0, wave, lane);
        } else {
#pragma unroll
            for (int h = 0; h < RW / 128; h++) fetch_tile(rw0, st + h * TILE_B, m0 + 128 * h, K, k0, wave, lane);
        }
        fetch_tile(rxh, st + W_B, n0, a.ldx, k0, wave, lane);
        fetch_tile(rxl, st + W_B + TILE_B, n0, a.ldx, k0, wave, lane);
    };
    // W region row of the wave's tile mt
    auto wrow = [&](int mt) {
        if (GEGLU) return (mt >> 2) * 128 + wm * 64 + (mt & 3) * 16;
        return wm * 16 * MT + mt * 16;
    };

    const int nk = kc / BK;
    const int fr = lane & 15, fc = lane >> 4;
    fetch(0, kbeg);
    for (int kt = 0; kt < nk; kt++) {
        __syncthreads();   // stage kt has landed; stage kt + 1's slot is free
        if (kt + 1 < nk) fetch((kt + 1) & 1, kbeg + (kt + 1) * BK);
        const char *st = smem + (kt & 1) * STAGE_B;
        bf16x8 bh[4], bl[4];
#pragma unroll
        for (int nt = 0; nt < 4; nt++) {
            bh[nt] = frag(st + W_B, wn * 64 + nt * 16 + fr, fc);
            bl[nt] = frag(st + W_B + TILE_B, wn * 64 + nt * 16 + fr, fc);
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const bf16x8 w = frag(st, wrow(mt) + fr, fc);
#pragma unroll
            for (int nt = 0; nt < 4; nt++) {
                acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w, bh[nt], acc[mt][nt], 0, 0, 0);
                acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w, bl[nt], acc[mt][nt], 0, 0, 0);
            }
        }
    }

    // epilogue: lane holds C rows m = base + 4 (l / 16) + i, i = 0..3, of token l % 16
    constexpr int MO = GEGLU ? MT / 2 : MT;   // output tiles per wave along m
#pragma unroll
    for (int mt = 0; mt < MO; mt++)
#pragma unroll
        for (int nt = 0; nt < 4; nt++) {
            const int m = m0 + (GEGLU ? wm * 64 : wm * 16 * MT) + mt * 16 + 4 * fc;
            const int n = n0 + wn * 64 + nt * 16 + fr;
            if (n >= N || m >= M) continue;   // M is a multiple of 4 (checked on the host)
            if (GEGLU) {
                const f32x4 g = acc[mt][nt], u = acc[mt + 4][nt];
                uint32_t hi[4], lo[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float h = gelu_tanh(g[i]) * u[i];
                    hi[i] = bf16_rne(h);
                    lo[i] = bf16_rne(h - __uint_as_float(hi[i] << 16));
                }
                const size_t o = (size_t)n * a.ldh + m;
                *reinterpret_cast<uint2 *>(a.h_hi + o) = make_uint2(hi[0] | (hi[1] << 16), hi[2] | (hi[3] << 16));
                *reinterpret_cast<uint2 *>(a.h_lo + o) = make_uint2(lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16));
            } else {
                const f32x4 c = acc[mt][nt];
                float *dst = a.C[m_idx] + (size_t)blockIdx.z * a.split_stride + (size_t)n * a.ldc[m_idx] + m;
                *reinterpret_cast<float4 *>(dst) = make_float4(c[0], c[1], c[2], c[3]);
            }
        }
}

template <bool GEGLU, int MT>
int launch(const g3k_gemm_args *a, hipStream_t st) {
    constexpr int BMW = GEGLU ? 16 * MT : 32 * MT;
    int tiles = 0;
    const int nm = GEGLU ? 1 : a->n_mat;
    for (int m = 0; m < nm; m++) tiles += (a->M[m] + BMW - 1) / BMW;
    const dim3 grid(tiles, (a->N + BN - 1) / BN, a->ksplit);
    hipLaunchKernelGGL((gemm_kernel<GEGLU, MT>), grid, dim3(NT), 0, st, *a);
    return (int)hipGetLastError();
}

}  // namespace

extern "C" int g3k_gemm(const g3k_gemm_args *a, void *stream) {
    const bool geglu = a->mode == G3K_MV_GEGLU;
    const int S = a->ksplit;
    if (a->N < 1 || a->K < BK || a->ldx < a->K || a->ldx % 8 || !a->x_hi || !a->x_lo)
        return (int)hipErrorInvalidValue;
    if (S < 1 || S > 16 || a->K % (BK * S) || (geglu && S != 1)) return (int)hipErrorInvalidValue;
    if (a->n_mat < 1 || a->n_mat > G3K_MATVEC_MAX || (geglu && a->n_mat != 2) || (a->mode != 0 && !geglu))
        return (int)hipErrorInvalidValue;
    // 32-bit buffer offsets, including the rows of a last partial tile
    if ((size_t)(a->N + BN) * a->ldx * 2 >= (1ull << 32)) return (int)hipErrorInvalidValue;
    long long tiles128 = 0;
    for (int m = 0; m < a->n_mat; m++) {
        if (a->M[m] < 4 || a->M[m] % 4 || !a->W[m] || (size_t)(a->M[m] + 256) * a->K * 2 >= (1ull << 32))
            return (int)hipErrorInvalidValue;
        if (geglu) continue;
        if (!a->C[m] || a->ldc[m] < a->M[m] || a->ldc[m] % 4) return (int)hipErrorInvalidValue;
        if (S > 1 && a->split_stride < (long long)a->N * a->ldc[m]) return (int)hipErrorInvalidValue;
        tiles128 += (a->M[m] + 127) / 128;
    }
    hipStream_t st = (hipStream_t)stream;
    if (geglu) {
        if (a->M[0] != a->M[1] || !a->h_hi || !a->h_lo || a->ldh < a->M[0] || a->ldh % 4)
            return (int)hipErrorInvalidValue;
        return launch<true, 8>(a, st);
    }
    // 256-row tiles once they give two workgroups per CU; 128-row tiles below
    const long long wgs256 = (tiles128 + 1) / 2 * ((a->N + BN - 1) / BN) * S;
    return wgs256 >= 512 ? launch<false, 8>(a, st) : launch<false, 4>(a, st);
}
