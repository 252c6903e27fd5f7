// g3k_device.h - small device helpers shared by the HIP kernels (gfx950, wave64).
#ifndef G3K_DEVICE_H
#define G3K_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

// Waits until every vector-memory operation this wave issued has completed,
// buffer -> LDS fetches included.  An asm statement with a memory clobber,
// so it also keeps the compiler from moving memory accesses across it.  The
// host-emulation build (tests/hostemu), whose loads complete when issued,
// defines it away before this header.
#ifndef G3K_WAIT_VMEM
#define G3K_WAIT_VMEM() asm volatile("s_waitcnt vmcnt(0)" ::: "memory")
#endif

// The XCD this wave runs on: the hardware register XCC_ID (gfx940 and
// later), whose low 4 bits number the XCDs.  The host-emulation build
// defines it as the workgroup id mod 8.
#ifndef G3K_XCC_ID
#define G3K_XCC_ID() g3k::xcc_id()
namespace g3k {
__device__ __forceinline__ unsigned xcc_id() {
    unsigned v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v;
}
}  // namespace g3k
#endif

namespace g3k {

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the total.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror: quad q <-> quad 1-q within 8 lanes
    v += dpp<0x140>(v);  // row_mirror: half h <-> half 1-h within 16 lanes
    return v;
}

// gfx950 v_permlane32_swap / v_permlane16_swap with both operands = v: the
// two results hold v of lanes {l, l ^ 32} (resp. {l, l ^ 16}) in some order,
// so their sum / max is the pair's.  VALU only, no LDS round trip.
__device__ __forceinline__ float pair32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum / max over the four lanes l % 16 + 16 g (g = 0..3); every lane gets it.
__device__ __forceinline__ float col4_sum(float v) { return pair16_sum(pair32_sum(v)); }
__device__ __forceinline__ float col4_max(float v) { return pair16_max(pair32_max(v)); }

// Sum over all 64 lanes; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) { return col4_sum(row16_sum(v)); }

// Max over the 16 lanes of a DPP row, then over all 64 lanes.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return v;
}
__device__ __forceinline__ float wave_max(float v) { return col4_max(row16_max(v)); }

// Power-of-two scale of a block of values whose largest magnitude is m: the
// exponent E = floor(log2 m) - 7, so every value / 2^E lies within +-256
// (OCP e4m3 holds +-448), clamped to [-126, 127]; E = 0 for m = 0.
__device__ __forceinline__ int x8_exponent(float m) {
    if (!(m > 0.f)) return 0;
    const int e = __builtin_amdgcn_frexp_expf(m) - 8;   // m = f 2^k, f in [0.5, 1): floor(log2 m) = k - 1
    return e < -126 ? -126 : (e > 127 ? 127 : e);
}

// Two floats -> two OCP e4m3 codes (round to nearest even) in the low 16
// bits, or, with hi, in the high 16 bits of `old` (v_cvt_pk_fp8_f32).
__device__ __forceinline__ uint32_t e4m3_pair(float a, float b, uint32_t old = 0, bool hi = false) {
    return hi ? (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)old, true)
              : (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)old, false);
}

// v_exp_f32: 2^x, flushes to 0 for very negative x.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// bf16 -> f32 is a 16-bit left shift (gemma3_kernels.h:268-275).
__device__ __forceinline__ float bf16f(uint32_t b) { return __uint_as_float(b << 16); }

}  // namespace g3k

#endif
