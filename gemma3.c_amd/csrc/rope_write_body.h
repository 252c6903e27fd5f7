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

// One staged key row (1 KiB: row points at its fp16 hi half) from this
// lane's four dims {2l, 2l+1} (x0, x1) and {2l+128, 2l+129} (x2, x3); the
// wave holds the whole 256-float row.  scale == nullptr: the exact format,
// fp16 hi | fp16 lo.  Otherwise the fp8 cross format of G3K_KROW_X8 (fp16 hi
// | e4m3 of hi / 2^E and of lo * 2^11 / 2^E) and the row's E8M0 scale byte
// 127 + E, written by lane 0.
__device__ __forceinline__ void write_krow(uint16_t *row, uint8_t *scale, float x0, float x1, float x2, float x3,
                                           int lane) {
    constexpr int D = G3K_HEAD_DIM;
    const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1, h2 = (_Float16)x2, h3 = (_Float16)x3;
    const float l0 = x0 - (float)h0, l1 = x1 - (float)h1, l2 = x2 - (float)h2, l3 = x3 - (float)h3;
    *reinterpret_cast<uint32_t *>(row + 2 * lane) = pack_f16(h0, h1);
    *reinterpret_cast<uint32_t *>(row + 128 + 2 * lane) = pack_f16(h2, h3);
    if (!scale) {
        *reinterpret_cast<uint32_t *>(row + D + 2 * lane) = pack_f16((_Float16)l0, (_Float16)l1);
        *reinterpret_cast<uint32_t *>(row + D + 128 + 2 * lane) = pack_f16((_Float16)l2, (_Float16)l3);
        return;
    }
    const float m = wave_max(fmaxf(fmaxf(fabsf(x0), fabsf(x1)), fmaxf(fabsf(x2), fabsf(x3))));
    const int E = x8_exponent(m);
    const float inv = __builtin_amdgcn_ldexpf(1.0f, -E), inv_lo = __builtin_amdgcn_ldexpf(1.0f, 11 - E);
    unsigned char *x8 = reinterpret_cast<unsigned char *>(row);
    // dims 2l, 2l+1 and 2l+128, 2l+129 are adjacent bytes of one 8-byte run
    // (u even, u + 1), so each pair is one 16-bit store per part
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int d = 2 * lane + 128 * k;
        const int t = d >> 5, g = (d >> 3) & 3, u = d & 7;
        const int off = 512 + 64 * (t >> 1) + 16 * g + 8 * (t & 1) + u;
        const float ha = (float)(k ? h2 : h0), hb = (float)(k ? h3 : h1);
        const float la = k ? l2 : l0, lb = k ? l3 : l1;
        *reinterpret_cast<uint16_t *>(x8 + off) = (uint16_t)e4m3_pair(ha * inv, hb * inv);
        *reinterpret_cast<uint16_t *>(x8 + off + 256) = (uint16_t)e4m3_pair(la * inv_lo, lb * inv_lo);
    }
    if (lane == 0) *scale = (uint8_t)(127 + E);
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
        // prefill staging: the rotated key's row in the staging format
        const size_t r = (size_t)h * a.ldk + a.row0 + i;
        write_krow(a.kq + r * (2 * D), a.kscale ? a.kscale + r : nullptr, lo.x, lo.y, hi.x, hi.y, lane);
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
