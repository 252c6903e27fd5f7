// rope_write.hip - batched QK-RMSNorm + RoPE + KV-cache write for n tokens.
//
// The per-token front end of the prefill loop (gemma3_transformer.c:650-671):
// per-head RMSNorm with (1 + w) gain (gemma3_kernels.c:289-304), RoPE from the
// precomputed table (gemma3_kernels.c:470-484) and cache_kv
// (gemma3_transformer.c:236-251), for every token of a batch in one launch.
// Q heads go to a head-major [H_q][n][D] buffer for the prefill attention
// kernel; K (normed + RoPE'd) and V rows go to the cache (or to a staging
// buffer), head-major [H_kv][rows][D].  For prefill the rotated keys are also
// written as fp16 hi / lo parts to the attention kernel's staging rows, and
// tokens whose ring slot a later token of the same batch overwrites
// (kv_skip) are not written to the cache.
//
// One wave per 256-float head vector.  Lane l holds dims {2l, 2l+1} and their
// RoPE partners {2l+128, 2l+129}: two 512-byte coalesced float2 loads, the
// rotation stays inside the lane and the table row is one float4 per lane.
#include <hip/hip_runtime.h>

#include "g3k.h"
#include "g3k_device.h"

namespace {

using namespace g3k;
constexpr int D = G3K_HEAD_DIM;

__device__ __forceinline__ uint32_t pack_f16(_Float16 a, _Float16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | (uint32_t)__builtin_bit_cast(uint16_t, b) << 16;
}

__global__ __launch_bounds__(256) void rope_write_kernel(g3k_rope_write_args a) {
    const int nq = a.Q ? a.n_heads : 0;
    const int nvec = nq + 2 * a.n_kv_heads;
    const long long wid = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (wid >= (long long)a.n * nvec) return;
    const int i = (int)(wid / nvec), v = (int)(wid % nvec);
    const int lane = threadIdx.x & 63;
    const int pos = a.start_pos + i;

    const float *src;
    const uint16_t *w = nullptr;
    int h;
    int kind;  // 0 = q, 1 = k, 2 = v
    if (v < nq) {
        kind = 0; h = v;
        src = a.Q + ((size_t)i * a.n_heads + h) * D;
        if (a.q_norm && a.k_norm) w = a.q_norm;
    } else if (v < nq + a.n_kv_heads) {
        kind = 1; h = v - nq;
        src = a.K + ((size_t)i * a.n_kv_heads + h) * D;
        if (a.q_norm && a.k_norm) w = a.k_norm;
    } else {
        kind = 2; h = v - nq - a.n_kv_heads;
        src = a.V + ((size_t)i * a.n_kv_heads + h) * D;
    }
    float2 lo = *reinterpret_cast<const float2 *>(src + 2 * lane);
    float2 hi = *reinterpret_cast<const float2 *>(src + 128 + 2 * lane);

    if (kind != 2) {
        if (w) {
            const float ss = wave_sum(lo.x * lo.x + lo.y * lo.y + hi.x * hi.x + hi.y * hi.y);
            const float r = 1.0f / sqrtf(ss / (float)D + a.eps);
            const uint32_t wl = *reinterpret_cast<const uint32_t *>(w + 2 * lane);
            const uint32_t wh = *reinterpret_cast<const uint32_t *>(w + 128 + 2 * lane);
            lo.x = lo.x * r * (1.0f + bf16f(wl & 0xffff));
            lo.y = lo.y * r * (1.0f + bf16f(wl >> 16));
            hi.x = hi.x * r * (1.0f + bf16f(wh & 0xffff));
            hi.y = hi.y * r * (1.0f + bf16f(wh >> 16));
        }
        const float4 t = *reinterpret_cast<const float4 *>(a.rope + (size_t)pos * D + 4 * lane);
        const float a0 = lo.x, b0 = hi.x, a1 = lo.y, b1 = hi.y;
        lo.x = a0 * t.x - b0 * t.y;
        hi.x = a0 * t.y + b0 * t.x;
        lo.y = a1 * t.z - b1 * t.w;
        hi.y = a1 * t.w + b1 * t.z;
    }

    if (kind == 1 && a.kq) {
        // prefill staging: fp16 hi | lo row of the rotated key
        const _Float16 h0 = (_Float16)lo.x, h1 = (_Float16)lo.y, h2 = (_Float16)hi.x, h3 = (_Float16)hi.y;
        const _Float16 l0 = (_Float16)(lo.x - (float)h0), l1 = (_Float16)(lo.y - (float)h1);
        const _Float16 l2 = (_Float16)(hi.x - (float)h2), l3 = (_Float16)(hi.y - (float)h3);
        uint16_t *row = a.kq + ((size_t)h * a.ldk + a.row0 + i) * (2 * D);
        *reinterpret_cast<uint32_t *>(row + 2 * lane) = pack_f16(h0, h1);
        *reinterpret_cast<uint32_t *>(row + 128 + 2 * lane) = pack_f16(h2, h3);
        *reinterpret_cast<uint32_t *>(row + D + 2 * lane) = pack_f16(l0, l1);
        *reinterpret_cast<uint32_t *>(row + D + 128 + 2 * lane) = pack_f16(l2, l3);
    }
    if (kind != 0 && i < a.kv_skip) return;

    float *dst;
    if (kind == 0) {
        dst = a.q_out + ((size_t)h * a.n + i) * D;
    } else {
        const int slot = a.ring > 0 ? pos % a.ring : pos - a.dst_pos0;
        dst = (kind == 1 ? a.k_dst : a.v_dst) + (size_t)h * a.dst_head_stride + (size_t)slot * D;
    }
    *reinterpret_cast<float2 *>(dst + 2 * lane) = lo;
    *reinterpret_cast<float2 *>(dst + 128 + 2 * lane) = hi;
}

}  // namespace

extern "C" int g3k_rope_write(const g3k_rope_write_args *a, void *stream) {
    if (a->n <= 0) return 0;
    const int nvec = (a->Q ? a->n_heads : 0) + 2 * a->n_kv_heads;
    const long long waves = (long long)a->n * nvec;
    const long long blocks = (waves + 3) / 4;
    if (blocks > 0x7fffffffLL) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(rope_write_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, *a);
    return (int)hipGetLastError();
}

namespace {

// Rows in the reference layout [n][H_kv][D] <-> the head-major cache: one
// thread per float4, consecutive threads along a row (coalesced on both
// sides: a cache row is contiguous, and so is a reference-layout head row).
__global__ __launch_bounds__(256) void kv_scatter_kernel(float *ck, float *cv, float *rk, float *rv, int n,
                                                         int n_kv, long long head_stride, int slot,
                                                         int to_rows) {
    const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long per_mat = (long long)n * n_kv * (D / 4);
    if (t >= 2 * per_mat) return;
    const int mat = (int)(t / per_mat);
    const long long r = t % per_mat;
    const int c4 = (int)(r % (D / 4));
    const long long hr = r / (D / 4);
    const int h = (int)(hr % n_kv), i = (int)(hr / n_kv);
    float4 *rows = reinterpret_cast<float4 *>(mat ? rv : rk) + ((size_t)i * n_kv + h) * (D / 4) + c4;
    float4 *cache = reinterpret_cast<float4 *>((mat ? cv : ck) + (size_t)h * head_stride + (size_t)(slot + i) * D) + c4;
    if (to_rows)
        *rows = *cache;
    else
        *cache = *rows;
}

}  // namespace

extern "C" int g3k_kv_scatter(float *dst_k, float *dst_v, float *rows_k, float *rows_v, int n, int n_kv_heads,
                              long long head_stride, int slot, int to_rows, void *stream) {
    if (n <= 0) return 0;
    const long long threads = 2LL * n * n_kv_heads * (D / 4);
    const long long blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffffLL) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(kv_scatter_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, dst_k, dst_v,
                       rows_k, rows_v, n, n_kv_heads, head_stride, slot, to_rows);
    return (int)hipGetLastError();
}
