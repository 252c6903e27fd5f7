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
// Workgroup = 4 waves; each wave owns RPW consecutive rows.  Lane l reads the
// 16-byte chunks l + 64 j of each row (8 elements each), so one wave load
// covers 1 KiB of a row, contiguous; CH chunks per lane (a round) are issued,
// with the x chunks they meet, before the FMAs that use them.  Row sums
// reduce over the wave with DPP and
// permlane swaps.  Rows whose length is not a multiple of 8 (or unaligned
// buffers) take a lane-strided scalar path.
//
// Shapes pick the variant (measured on the forward's shapes): long rows
// (K >= 8192, the MLP's down projection) stage x in LDS once per workgroup
// instead of once per wave; rows of at most 2048 elements take 4 chunks per
// round (one round); very tall matrices (the tied logits) take 2 rows per wave.
//
// One launch can serve up to three matrices that share x (the Q, K and V
// projections of one token): workgroups are dealt to the matrices in order of
// their row blocks.  The GEGLU mode computes the gate and up rows of the MLP
// together and writes gelu_tanh(gate) * up (gemma3_transformer.c:380-386).
#include <hip/hip_runtime.h>

#include "g3k.h"
#include "g3k_device.h"

namespace {

using namespace g3k;

constexpr int NT = 256;   // 4 waves
constexpr int NW = NT / 64;
constexpr int G3K_MATVEC_LDS_MAX_K = 16384;

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

// 16 bytes of A.  Plain loads: non-temporal ones stream faster, but the
// decode kernel's measurements showed them returning stale values for memory
// that a host -> device copy rewrote after kernels had touched it, and A may
// be re-uploaded in place (g3attn_upload_weights, a caller's own buffers).
__device__ __forceinline__ uint4 load_a(const uint16_t *p) { return *reinterpret_cast<const uint4 *>(p); }

// NA dot products per wave: RPW consecutive rows of one matrix, or (GEGLU)
// the same row of the gate and up matrices.  XLDS: x is copied to LDS by the
// workgroup (dynamic shared memory of K floats) after the first round's A
// loads are issued.
template <int RPW, int CH, bool VEC, bool XLDS, bool GEGLU>
__global__ __launch_bounds__(NT) void matvec_kernel(g3k_matvec_args a) {
    extern __shared__ float4 xs4[];
    constexpr int NA = GEGLU ? 2 : RPW;
    const int K = a.K;
    int row0;
    const int m = pick(a, NW * RPW, row0);
    if (m < 0) return;   // uniform over the workgroup
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int M = a.M[m];
    const float *x = a.x;
    const int r0 = row0 + wave * RPW;
    const uint16_t *rows[NA];
#pragma unroll
    for (int j = 0; j < NA; j++) {
        const int row = GEGLU ? (r0 < M ? r0 : M - 1) : (r0 + j < M ? r0 + j : M - 1);
        rows[j] = a.A[GEGLU ? j : m] + (size_t)row * K;
    }
    float acc[NA];
#pragma unroll
    for (int j = 0; j < NA; j++) acc[j] = 0.f;

    if (VEC) {
        const int nch = K >> 3;
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        // rounds are uniform over the workgroup (the LDS copy has a barrier)
        for (int base = 0; base < nch; base += 64 * CH) {
            uint4 w[NA][CH];
            float4 xa[CH], xb[CH];
#pragma unroll
            for (int u = 0; u < CH; u++) {
                const int c = base + lane + 64 * u;
                const bool ok = c < nch;
#pragma unroll
                for (int j = 0; j < NA; j++) w[j][u] = ok ? load_a(rows[j] + 8 * c) : make_uint4(0, 0, 0, 0);
                if (!XLDS) {
                    xa[u] = ok ? x4[2 * c] : make_float4(0.f, 0.f, 0.f, 0.f);
                    xb[u] = ok ? x4[2 * c + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
            if (XLDS && base == 0) {
                for (int i = threadIdx.x; i < 2 * nch; i += NT) xs4[i] = x4[i];
                __syncthreads();
            }
#pragma unroll
            for (int u = 0; u < CH; u++) {
                if (XLDS) {
                    const int c = base + lane + 64 * u;
                    const bool ok = c < nch;
                    xa[u] = ok ? xs4[2 * c] : make_float4(0.f, 0.f, 0.f, 0.f);
                    xb[u] = ok ? xs4[2 * c + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
                }
#pragma unroll
                for (int j = 0; j < NA; j++) acc[j] += dot8(w[j][u], xa[u], xb[u]);
            }
        }
    } else {
        for (int k = lane; k < K; k += 64) {
            const float xv = x[k];
#pragma unroll
            for (int j = 0; j < NA; j++) acc[j] = fmaf(bf16f(rows[j][k]), xv, acc[j]);
        }
    }
    if (GEGLU) {
        const float g = wave_sum(acc[0]), u = wave_sum(acc[1]);
        if (lane == 0 && r0 < M) a.y[0][r0] = gelu_tanh(g) * u;
    } else {
#pragma unroll
        for (int j = 0; j < NA; j++) {
            const float s = wave_sum(acc[j]);
            if (lane == 0 && r0 + j < M) a.y[m][r0 + j] = s;
        }
    }
}

template <int RPW, int CH, bool VEC, bool XLDS = false, bool GEGLU = false>
hipError_t launch(const g3k_matvec_args *a, hipStream_t st) {
    int blocks = 0;
    const int nm = GEGLU ? 1 : a->n_mat;
    for (int m = 0; m < nm; m++) blocks += (a->M[m] + NW * RPW - 1) / (NW * RPW);
    const size_t lds = XLDS ? (size_t)a->K * sizeof(float) : 0;
    hipLaunchKernelGGL((matvec_kernel<RPW, CH, VEC, XLDS, GEGLU>), dim3(blocks), dim3(NT), lds, st, *a);
    return hipGetLastError();
}

}  // namespace

extern "C" int g3k_matvec(const g3k_matvec_args *a, void *stream) {
    if (a->n_mat < 1 || a->n_mat > G3K_MATVEC_MAX || a->K < 1 || !a->x)
        return (int)hipErrorInvalidValue;
    bool vec = a->K % 8 == 0 && ((uintptr_t)a->x & 15) == 0;
    long long rows = 0;
    for (int m = 0; m < a->n_mat; m++) {
        // GEGLU writes one output (y[0]) from the two matrices
        if (a->M[m] < 1 || !a->A[m] || (!a->y[m] && (a->mode != G3K_MV_GEGLU || m == 0)))
            return (int)hipErrorInvalidValue;
        vec = vec && ((uintptr_t)a->A[m] & 15) == 0;
        rows += a->M[m];
    }
    if (rows > (1LL << 30)) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    if (a->mode == G3K_MV_GEGLU) {
        if (a->n_mat != 2 || a->M[0] != a->M[1]) return (int)hipErrorInvalidValue;
        return (int)(vec ? launch<1, 4, true, false, true>(a, st) : launch<1, 1, false, false, true>(a, st));
    }
    if (a->mode != 0) return (int)hipErrorInvalidValue;
    if (!vec) return (int)(rows >= 16384 ? launch<2, 1, false>(a, st) : launch<1, 1, false>(a, st));
    // two rows per wave once there are enough rows to fill the chip with them
    if (rows >= 16384) return (int)launch<2, 8, true>(a, st);
    // long rows: x in LDS (K floats, at most 64 KiB of the workgroup's LDS)
    if (a->K >= 8192 && a->K <= G3K_MATVEC_LDS_MAX_K) return (int)launch<1, 4, true, true>(a, st);
    if (a->K <= 2048) return (int)launch<1, 4, true>(a, st);
    return (int)launch<1, 8, true>(a, st);
}
