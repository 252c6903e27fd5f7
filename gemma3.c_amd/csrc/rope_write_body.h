// rope_write_body.h - one wave's share of the batched QK-RMSNorm + RoPE +
// KV-cache write (the per-token front end of the prefill loop,
// gemma3_transformer.c:650-671): one 256-float head vector of one token.
// Shared by rope_write_kernel (rope_write.hip) and the prefill front launch
// (prefill.hip), which runs it beside the batch's V^T staging.
#ifndef G3K_ROPE_WRITE_BODY_H
#define G3K_ROPE_WRITE_BODY_H

#include "g3k.h"
#include "g3k_device.h"

namespace g3k {

__device__ __forceinline__ uint32_t pack_f16(_Float16 a, _Float16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | (uint32_t)__builtin_bit_cast(uint16_t, b) << 16;
}

// Wave wid of the batch (token wid / nvec, vector wid % nvec: the Q heads,
// then K, then V); lane l holds dims {2l, 2l+1} and their RoPE partners
// {2l+128, 2l+129}.
__device__ __forceinline__ void rope_write_vec(const g3k_rope_write_args &a, long long wid, int lane) {
    constexpr int D = G3K_HEAD_DIM;
    const int nq = a.Q ? a.n_heads : 0;
    const int nvec = nq + 2 * a.n_kv_heads;
    if (wid >= (long long)a.n * nvec) return;
    const int i = (int)(wid / nvec), v = (int)(wid % nvec);
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


}  // namespace g3k

#endif
