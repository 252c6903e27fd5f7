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
#include "rope_write_body.h"

namespace {

using namespace g3k;
constexpr int D = G3K_HEAD_DIM;

__global__ __launch_bounds__(256) void rope_write_kernel(g3k_rope_write_args a) {
    rope_write_vec(a, ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 6, threadIdx.x & 63);
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
