// hip/hip_runtime.h for the host-emulation builds of the library's kernels.
//
// TEST INFRASTRUCTURE.  tests/hostemu/Makefile compiles
// gemma3.c_amd/csrc/*.hip as plain C++ for x86-64 (ROCm's clang,
// -fsanitize=address,undefined) with this directory first on the include
// path, so the kernels' own source runs on the CPU under the sanitizers.
// This header supplies the subset of the HIP device language those kernels
// use, emulated on the host (the runtime API is hip_runtime_api.h):
//
//   - A launch runs every workgroup of the grid in turn (first to last, or
//     last to first with HOSTEMU_WG_ORDER=reverse) on one team of blockDim
//     fibers (one stack per GPU thread, all on the calling OS
//     thread), so 64 consecutive fibers form one wave64.  __shared__ becomes
//     a function-local static: one copy, used by one workgroup at a time.
//   - __syncthreads is a barrier over the team; every cross-lane operation
//     (DPP, v_permlane16/32_swap, __shfl_xor, readfirstlane, ballot, MFMA)
//     is an exchange through a double-buffered per-wave buffer with one
//     barrier over the wave's 64 fibers.  A barrier or cross-lane operation that not every
//     lane reaches leaves no fiber runnable, and the launch aborts (on the
//     GPU it would be undefined).  A fiber runs until it reaches one, so the
//     waves of a workgroup interleave at every cross-lane step.
//   - Loads complete when issued: a buffer -> LDS fetch writes LDS at once,
//     so one that overwrites data another wave still reads (a missing
//     barrier) shows in the results.
//   - Buffer loads into registers check their offset against the
//     descriptor's num_records and abort on an out-of-range load instead of
//     returning zero: the kernels clamp every row index, so none may go out
//     of range.  Buffer -> LDS loads return zero there, as the hardware
//     does: the prefill and GEMM kernels rely on it for ragged tiles.
//   - MFMA 16x16x32 (f16 / bf16) computes the exact products and sums them
//     in double: any operand placed in the wrong lane changes the result.
//   - DPP controls and load forms other than the ones the kernels use abort.
//
// Cross-lane semantics follow AMD's CDNA4 ISA descriptions of
// DPP quad_perm / row_mirror / row_half_mirror, V_PERMLANE16_SWAP_B32 and
// V_PERMLANE32_SWAP_B32, and ds_bpermute-based __shfl_xor.
#ifndef G3_HOSTEMU_HIP_RUNTIME_H
#define G3_HOSTEMU_HIP_RUNTIME_H

#include <array>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <math.h>
#include <functional>
#include <vector>
#if defined(__SANITIZE_ADDRESS__)
#include <sanitizer/common_interface_defs.h>
#endif

// ---- language keywords ------------------------------------------------------
#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __shared__ static
#define __launch_bounds__(...)
#define __align__(n) __attribute__((aligned(n)))

// ---- vector types -------------------------------------------------------------
struct dim3 {
    unsigned x, y, z;
    constexpr dim3(unsigned x_ = 1, unsigned y_ = 1, unsigned z_ = 1) : x(x_), y(y_), z(z_) {}
};
struct alignas(16) float4 { float x, y, z, w; };
struct alignas(8) float2 { float x, y; };
struct alignas(8) uint2 { unsigned x, y; };
struct alignas(16) uint4 { unsigned x, y, z, w; };
inline uint4 make_uint4(unsigned x, unsigned y, unsigned z, unsigned w) { return uint4{x, y, z, w}; }
inline float4 make_float4(float x, float y, float z, float w) { return float4{x, y, z, w}; }
inline float2 make_float2(float x, float y) { return float2{x, y}; }
inline uint2 make_uint2(unsigned x, unsigned y) { return uint2{x, y}; }

inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }

inline unsigned __float_as_uint(float f) { unsigned u; std::memcpy(&u, &f, 4); return u; }
inline int __float_as_int(float f) { int u; std::memcpy(&u, &f, 4); return u; }
inline float __uint_as_float(unsigned u) { float f; std::memcpy(&f, &u, 4); return f; }
inline float __int_as_float(int u) { float f; std::memcpy(&f, &u, 4); return f; }

// ---- runtime API (hip_runtime_api.h, implemented in ../hostrt.cpp) ----------
#include "hip_runtime_api.h"
#define HIP_SYMBOL(x) (&(x))
template <typename K>
hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int *n, K, int, size_t) { *n = 2; return hipSuccess; }

// Loads complete when issued here, so the library's explicit wait for them
// is empty.
#define G3K_WAIT_VMEM() ((void)0)
// The emulated machine deals workgroup i to XCD i mod 8, as the MI355X
// dispatcher does.
#define G3K_XCC_ID() (blockIdx.x % 8u)

// ---- the emulated machine ------------------------------------------------------
// One fiber per thread of the workgroup, all on the calling OS thread: a
// barrier parks the fiber and the scheduler resumes the next runnable one in
// order.  Deterministic, and no OS-thread contention.
//
// hostemu_switch(from, to) is the x86-64 SysV stack switch: it pushes the
// callee-saved registers and the SSE / x87 control words, stores the stack
// pointer in *from, loads `to` and pops the same from there.  (glibc's
// swapcontext also saves the signal mask with a system call each time.)
// Defined in ../hostrt.cpp.
extern "C" void hostemu_switch(void **from, void *to);


namespace hostemu {

[[noreturn]] inline void fail(const char *what) {
    std::fprintf(stderr, "hostemu: %s\n", what);
    std::fflush(stderr);
    std::abort();
}

struct Fiber {
    void *sp = nullptr;       // saved stack pointer while switched out
    char *stack = nullptr;
    size_t stack_size = 0;
    void *fake_stack = nullptr;
    dim3 tid;
    int lane = 0, wave = 0;
    bool blocked = false, done = false;
};

// A barrier over n fibers: the last to arrive releases the others.
struct Barrier {
    int n = 0;
    std::vector<Fiber *> waiting;
    void wait();
};

// Per-wave exchange buffers, two of each: exchange k of a wave uses set
// k % 2, so one barrier per exchange suffices.  A lane can write set k % 2
// again only at exchange k + 2, after passing exchange k + 1's barrier, which
// every lane reaches only after reading exchange k.
struct Wave {
    Barrier bar;
    uint32_t a[2][64], b[2][64];
    uint32_t op[2][64][18];  // MFMA A and B operands (16 or 32 bytes each per lane), then the fp8 scales
    unsigned gen[64] = {};   // exchanges each lane has started
};

struct Machine {
    std::vector<Fiber> fibers;
    Barrier block;
    std::vector<Wave> waves;
    std::vector<int> slot;   // one int per thread (__syncthreads_or)
    Fiber *current = nullptr;
    void *sched_sp = nullptr;
    void *sched_fake = nullptr;
    const void *sched_bottom = nullptr;
    size_t sched_size = 0;
    std::function<void()> body;
};

inline Machine *&machine() { static Machine *m = nullptr; return m; }
inline int t_lane = 0, t_wave = 0, t_flat = 0;

// Switches from the running fiber back to the scheduler.
inline void yield_to_scheduler(bool dying) {
    Machine &m = *machine();
    Fiber *f = m.current;
#if defined(__SANITIZE_ADDRESS__)
    __sanitizer_start_switch_fiber(dying ? nullptr : &f->fake_stack, m.sched_bottom, m.sched_size);
#else
    (void)dying;
#endif
    hostemu_switch(&f->sp, m.sched_sp);
#if defined(__SANITIZE_ADDRESS__)
    __sanitizer_finish_switch_fiber(f->fake_stack, nullptr, nullptr);
#endif
}

inline void Barrier::wait() {
    Machine &m = *machine();
    if ((int)waiting.size() + 1 == n) {
        for (Fiber *f : waiting) f->blocked = false;
        waiting.clear();
        return;
    }
    m.current->blocked = true;
    waiting.push_back(m.current);
    yield_to_scheduler(false);
}

// Every lane publishes (x, y); each returns the pair published by lane src.
inline void exchange(uint32_t x, uint32_t y, int src, uint32_t *rx, uint32_t *ry) {
    Wave &w = machine()->waves[t_wave];
    const int k = w.gen[t_lane]++ & 1;
    w.a[k][t_lane] = x;
    w.b[k][t_lane] = y;
    w.bar.wait();
    if (src < 0 || src >= 64) fail("cross-lane source lane out of range");
    *rx = w.a[k][src];
    *ry = w.b[k][src];
}

}  // namespace hostemu

inline dim3 threadIdx, blockIdx, gridDim, blockDim;
inline void __syncthreads() { hostemu::machine()->block.wait(); }
// Barrier that also returns whether any thread of the workgroup passed nonzero.
inline int __syncthreads_or(int p) {
    hostemu::Machine &m = *hostemu::machine();
    m.slot[hostemu::t_flat] = p != 0;
    m.block.wait();
    int r = 0;
    for (int v : m.slot) r |= v;
    m.block.wait();   // every thread has read the slots before any rewrites them
    return r;
}
// Workgroups run one after another, so a fence has nothing to order and an
// atomic is a plain read-modify-write.  atomicInc wraps as the hardware's
// atomic_inc does: old >= v ? 0 : old + 1.
inline void __threadfence() {}
// (__hip_atomic_load / __hip_atomic_store are clang builtins on the host
// too; only their scope names are HIP-mode macros.)
#ifndef __HIP_MEMORY_SCOPE_AGENT
#define __HIP_MEMORY_SCOPE_AGENT 4
#endif
#ifndef __HIP_MEMORY_SCOPE_WORKGROUP
#define __HIP_MEMORY_SCOPE_WORKGROUP 3
#endif
inline unsigned atomicInc(unsigned *p, unsigned v) {
    const unsigned old = *p;
    *p = old >= v ? 0u : old + 1u;
    return old;
}

// ---- cross-lane builtins ---------------------------------------------------------
// DPP (row = 16 lanes): quad_perm 0x00-0xff, row_ror:8 0x128 (lane i reads
// lane i ^ 8 of its row), row_mirror 0x140, row_half_mirror 0x141.
inline int hostemu_update_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
    const int l = hostemu::t_lane;
    int from;
    if (ctrl >= 0 && ctrl <= 0xff) from = (l & ~3) + ((ctrl >> (2 * (l & 3))) & 3);
    else if (ctrl == 0x128) from = l ^ 8;
    else if (ctrl == 0x140) from = (l & ~15) + (15 - (l & 15));
    else if (ctrl == 0x141) from = (l & ~7) + (7 - (l & 7));
    else hostemu::fail("DPP control not emulated");
    (void)bound_ctrl;
    uint32_t r, unused;
    hostemu::exchange((uint32_t)src, 0, from, &r, &unused);
    const bool enabled = ((row_mask >> (l >> 4)) & 1) && ((bank_mask >> ((l >> 2) & 3)) & 1);
    return enabled ? (int)r : old;
}
#define __builtin_amdgcn_update_dpp hostemu_update_dpp

// V_PERMLANE32_SWAP_B32 vdst, vsrc: lanes 32-63 of vdst swap with lanes 0-31
// of vsrc.  Returns {new vdst, new vsrc}.
inline std::array<uint32_t, 2> hostemu_permlane32_swap(uint32_t vdst, uint32_t vsrc, bool, bool) {
    const int l = hostemu::t_lane;
    uint32_t d, s;
    if (l < 32) {
        uint32_t hi_d, unused;
        hostemu::exchange(vdst, vsrc, l + 32, &hi_d, &unused);  // vsrc_new[l] = vdst[l + 32]
        d = vdst;
        s = hi_d;
    } else {
        uint32_t unused, lo_s;
        hostemu::exchange(vdst, vsrc, l - 32, &unused, &lo_s);  // vdst_new[l] = vsrc[l - 32]
        d = lo_s;
        s = vsrc;
    }
    return {d, s};
}
// V_PERMLANE16_SWAP_B32 vdst, vsrc: odd rows of vdst swap with even rows of
// vsrc (row = 16 lanes).
inline std::array<uint32_t, 2> hostemu_permlane16_swap(uint32_t vdst, uint32_t vsrc, bool, bool) {
    const int l = hostemu::t_lane;
    uint32_t d, s;
    if (((l >> 4) & 1) == 0) {
        uint32_t odd_d, unused;
        hostemu::exchange(vdst, vsrc, l + 16, &odd_d, &unused);  // vsrc_new[l] = vdst[l + 16]
        d = vdst;
        s = odd_d;
    } else {
        uint32_t unused, even_s;
        hostemu::exchange(vdst, vsrc, l - 16, &unused, &even_s);  // vdst_new[l] = vsrc[l - 16]
        d = even_s;
        s = vsrc;
    }
    return {d, s};
}
#define __builtin_amdgcn_permlane32_swap hostemu_permlane32_swap
#define __builtin_amdgcn_permlane16_swap hostemu_permlane16_swap

inline float __shfl_xor(float v, int mask, int width = 64) {
    if (width != 64) hostemu::fail("__shfl_xor width other than 64 not emulated");
    uint32_t r, unused;
    hostemu::exchange(__float_as_uint(v), 0, hostemu::t_lane ^ mask, &r, &unused);
    return __uint_as_float(r);
}

inline float hostemu_exp2f(float x) { return exp2f(x); }
#define __builtin_amdgcn_exp2f hostemu_exp2f

// ---- buffer resources ------------------------------------------------------------
struct __amdgpu_buffer_rsrc_t {
    const char *base;
    uint32_t num_records;
};
inline __amdgpu_buffer_rsrc_t hostemu_make_buffer_rsrc(void *base, short stride, int num_records, int flags) {
    if (stride != 0) hostemu::fail("strided buffer descriptor not emulated");
    (void)flags;
    return __amdgpu_buffer_rsrc_t{static_cast<const char *>(base), (uint32_t)num_records};
}
inline std::array<uint32_t, 4> hostemu_raw_buffer_load_b128(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff,
                                                           int aux) {
    (void)aux;
    const uint64_t off = (uint64_t)voff + soff;
    if (off + 16 > r.num_records) hostemu::fail("buffer load beyond num_records");
    std::array<uint32_t, 4> v;
    std::memcpy(v.data(), r.base + off, 16);
    return v;
}
// 16-byte buffer store; out of range aborts (the hardware would drop it).
template <typename T>
inline void hostemu_raw_buffer_store_b128(T v, __amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff, int aux) {
    static_assert(sizeof(T) == 16, "b128 store");
    (void)aux;
    const uint64_t off = (uint64_t)voff + soff;
    if (off + 16 > r.num_records) hostemu::fail("buffer store beyond num_records");
    std::memcpy(const_cast<char *>(r.base) + off, &v, 16);
}
// 4- and 8-byte buffer loads into registers, range-checked like the b128 form.
inline uint32_t hostemu_raw_buffer_load_b32(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff, int aux) {
    (void)aux;
    const uint64_t off = (uint64_t)voff + soff;
    if (off + 4 > r.num_records) hostemu::fail("buffer load beyond num_records");
    uint32_t v;
    std::memcpy(&v, r.base + off, 4);
    return v;
}
inline std::array<uint32_t, 2> hostemu_raw_buffer_load_b64(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff,
                                                          int aux) {
    (void)aux;
    const uint64_t off = (uint64_t)voff + soff;
    if (off + 8 > r.num_records) hostemu::fail("buffer load beyond num_records");
    std::array<uint32_t, 2> v;
    std::memcpy(v.data(), r.base + off, 8);
    return v;
}
#define __builtin_amdgcn_make_buffer_rsrc hostemu_make_buffer_rsrc
#define __builtin_amdgcn_raw_buffer_load_b128 hostemu_raw_buffer_load_b128
#define __builtin_amdgcn_raw_buffer_load_b32 hostemu_raw_buffer_load_b32
#define __builtin_amdgcn_raw_buffer_load_b64 hostemu_raw_buffer_load_b64
#define __builtin_amdgcn_raw_buffer_store_b128 hostemu_raw_buffer_store_b128

// Buffer -> LDS load (gfx950 buffer_load_dword{,x4} ... lds), 4 or 16 bytes
// per lane: lane l's bytes go to LDS at the given base + size l.  A dword whose
// offset + 4 exceeds num_records reads zero, as the hardware's range check
// for a raw (stride 0) buffer gives; the kernels rely on this for ragged
// tiles.  Other sizes and a nonzero instruction offset abort.
template <typename P>
inline void hostemu_buffer_load_lds(__amdgpu_buffer_rsrc_t r, P lds, int size, unsigned voff, unsigned soff,
                                    int offset, int aux) {
    (void)aux;
    if ((size != 16 && size != 4) || offset != 0) hostemu::fail("buffer->LDS load form not emulated");
    char *dst = (char *)lds + size * hostemu::t_lane;
    for (int i = 0; i < size / 4; i++) {
        const uint64_t o = (uint64_t)voff + soff + 4 * i;
        uint32_t v = 0;
        if (o + 4 <= r.num_records) std::memcpy(&v, r.base + o, 4);
        std::memcpy(dst + 4 * i, &v, 4);
    }
}
#define __builtin_amdgcn_raw_ptr_buffer_load_lds hostemu_buffer_load_lds

// ---- wave-level builtins ------------------------------------------------------------
inline int hostemu_readfirstlane(int v) {
    uint32_t r, unused;
    hostemu::exchange((uint32_t)v, 0, 0, &r, &unused);
    return (int)r;
}
#define __builtin_amdgcn_readfirstlane hostemu_readfirstlane

inline uint64_t hostemu_ballot_w64(bool p) {
    hostemu::Wave &w = hostemu::machine()->waves[hostemu::t_wave];
    const int k = w.gen[hostemu::t_lane]++ & 1;
    w.a[k][hostemu::t_lane] = p;
    w.bar.wait();
    uint64_t mask = 0;
    for (int i = 0; i < 64; i++) mask |= (uint64_t)(w.a[k][i] != 0) << i;
    return mask;
}
#define __builtin_amdgcn_ballot_w64 hostemu_ballot_w64

// Scheduling hints have no effect here.
#define __builtin_amdgcn_s_setprio(x) ((void)(x))
#define __builtin_amdgcn_sched_barrier(x) ((void)(x))

// V_MFMA_F32_16X16X32_{F16,BF16}: D = A B + C for a 16 x 32 A, a 32 x 16 B
// and 16 x 16 C / D, one wave.  Operand layout (the one the kernels are
// written to): lane l holds A[l % 16][8 (l / 16) + j] and
// B[8 (l / 16) + j][l % 16] as element j of its 8-element operands, and
// D[4 (l / 16) + r][l % 16] as element r of its 4 accumulators.  The
// products are summed in double and rounded once (the hardware's fp32
// summation order is not modelled).  Broadcast controls abort.
template <typename V8, typename F4>
inline F4 hostemu_mfma_16x16x32(V8 a, V8 b, F4 c, int cbsz, int abid, int blgp) {
    static_assert(sizeof(V8) == 16, "8 x 16-bit operands");
    if (cbsz || abid || blgp) hostemu::fail("MFMA broadcast controls not emulated");
    hostemu::Wave &w = hostemu::machine()->waves[hostemu::t_wave];
    const int l = hostemu::t_lane;
    const int k = w.gen[l]++ & 1;
    std::memcpy(&w.op[k][l][0], &a, 16);
    std::memcpy(&w.op[k][l][4], &b, 16);
    w.bar.wait();
    const int n = l & 15, g = l >> 4;
    float bcol[32];
    for (int q = 0; q < 4; q++) {
        V8 bv;
        std::memcpy(&bv, &w.op[k][n + 16 * q][4], 16);
        for (int j = 0; j < 8; j++) bcol[8 * q + j] = (float)bv[j];
    }
    F4 d;
    for (int r = 0; r < 4; r++) {
        const int m = 4 * g + r;
        double acc = (double)c[r];
        for (int q = 0; q < 4; q++) {
            V8 av;
            std::memcpy(&av, &w.op[k][m + 16 * q][0], 16);
            for (int j = 0; j < 8; j++) acc += (double)(float)av[j] * (double)bcol[8 * q + j];
        }
        d[r] = (float)acc;
    }
    return d;
}
#define __builtin_amdgcn_mfma_f32_16x16x32_f16 hostemu_mfma_16x16x32
#define __builtin_amdgcn_mfma_f32_16x16x32_bf16 hostemu_mfma_16x16x32

// OCP fp8 e4m3 (FN: bias 7, no infinities, 0x7f / 0xff NaN, largest 448).
inline float hostemu_e4m3_value(uint8_t b) {
    const int e = (b >> 3) & 15, m = b & 7;
    if ((b & 0x7f) == 0x7f) return NAN;
    const float v = e == 0 ? ldexpf((float)m, -9) : ldexpf(8.0f + (float)m, e - 10);
    return (b & 0x80) ? -v : v;
}
// float -> e4m3 code, round to nearest even; magnitudes from 464 on (and
// NaN) give NaN, as gfx950's v_cvt_pk_fp8_f32 was measured to.
inline uint8_t hostemu_e4m3_code(float x) {
    const uint8_t sign = std::signbit(x) ? 0x80 : 0;
    const float a = fabsf(x);
    if (!(a < 464.0f)) return sign | 0x7f;
    uint8_t best = 0;
    float bd = INFINITY;
    for (int c = 0; c < 0x7f; c++) {   // finite magnitudes, increasing
        const float d = fabsf(hostemu_e4m3_value((uint8_t)c) - a);
        if (d < bd || (d == bd && (c & 1) == 0 && (best & 1))) {
            bd = d;
            best = (uint8_t)c;
        }
    }
    return sign | best;
}
// V_CVT_PK_FP8_F32: two codes into the low (word_sel false) or high 16 bits
// of old.
inline int hostemu_cvt_pk_fp8_f32(float a, float b, int old, bool word_sel) {
    const uint32_t pair = (uint32_t)hostemu_e4m3_code(a) | (uint32_t)hostemu_e4m3_code(b) << 8;
    const uint32_t o = (uint32_t)old;
    return (int)(word_sel ? (o & 0xffffu) | pair << 16 : (o & 0xffff0000u) | pair);
}
#define __builtin_amdgcn_cvt_pk_fp8_f32 hostemu_cvt_pk_fp8_f32

inline int hostemu_frexp_expf(float x) {
    int e = 0;
    (void)frexpf(x, &e);
    return e;
}
#define __builtin_amdgcn_frexp_expf hostemu_frexp_expf
#define __builtin_amdgcn_ldexpf ldexpf

// V_MFMA_SCALE_F32_16X16X128_F8F6F4 with e4m3 A and B (cbsz = blgp = 0):
// D = A B + C over K = 128, with E8M0 scales (2^(code - 127)).  Operand
// layout (the kernels' and CK's): lane l holds A[l % 16][32 (l / 16) + j]
// and B[32 (l / 16) + j][l % 16] as byte j of its 32-byte operands.  Scales
// as measured on gfx950: the scale byte (opsel 0) of lane m + 16 s applies
// to row m's bytes 16 (s / 2) .. + 15 of the lanes m + 16 g with g in
// {2 (s % 2), 2 (s % 2) + 1}; likewise for B's columns.  Summed in double.
template <typename V8I, typename F4>
inline F4 hostemu_mfma_scale_16x16x128_f8(V8I a, V8I b, F4 c, int cbsz, int blgp, int opsel_a, int scale_a,
                                           int opsel_b, int scale_b) {
    static_assert(sizeof(V8I) == 32, "32-byte fp8 operands");
    if (cbsz || blgp || opsel_a || opsel_b) hostemu::fail("fp8 MFMA format / opsel not emulated");
    hostemu::Wave &w = hostemu::machine()->waves[hostemu::t_wave];
    const int l = hostemu::t_lane;
    const int k = w.gen[l]++ & 1;
    std::memcpy(&w.op[k][l][0], &a, 32);
    std::memcpy(&w.op[k][l][8], &b, 32);
    w.op[k][l][16] = (uint32_t)scale_a & 0xff;
    w.op[k][l][17] = (uint32_t)scale_b & 0xff;
    w.bar.wait();
    const int n = l & 15, g = l >> 4;
    F4 d;
    for (int r = 0; r < 4; r++) {
        const int m = 4 * g + r;
        double acc = (double)c[r];
        for (int q = 0; q < 4; q++) {          // lane group of the data
            const uint8_t *ab = reinterpret_cast<const uint8_t *>(&w.op[k][m + 16 * q][0]);
            const uint8_t *bb = reinterpret_cast<const uint8_t *>(&w.op[k][n + 16 * q][8]);
            for (int j = 0; j < 32; j++) {
                const int sl = (q >> 1) + 2 * (j >> 4);   // the scale lane group of (q, byte j)
                const double sa = ldexp(1.0, (int)w.op[k][m + 16 * sl][16] - 127);
                const double sb = ldexp(1.0, (int)w.op[k][n + 16 * sl][17] - 127);
                acc += (double)hostemu_e4m3_value(ab[j]) * (double)hostemu_e4m3_value(bb[j]) * sa * sb;
            }
        }
        d[r] = (float)acc;
    }
    return d;
}
#define __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4 hostemu_mfma_scale_16x16x128_f8

// ---- launches ------------------------------------------------------------------------
namespace hostemu {

inline void fiber_entry() {
    Machine &m = *machine();
#if defined(__SANITIZE_ADDRESS__)
    __sanitizer_finish_switch_fiber(nullptr, &m.sched_bottom, &m.sched_size);
#endif
    m.body();
    m.current->done = true;
    yield_to_scheduler(true);
    fail("finished fiber resumed");
}

inline unsigned workgroups(dim3 g) { return g.x * g.y * g.z; }

// Fiber stacks, allocated once per thread index and reused by every launch.
// The pool is never destroyed, so the stacks stay reachable at exit (no
// leak report).
inline char *stack_pool(int i, size_t bytes) {
    static std::vector<char *> *pool = new std::vector<char *>;
    while ((int)pool->size() <= i) {
        pool->push_back(static_cast<char *>(std::malloc(bytes)));
        if (!pool->back()) fail("fiber stack allocation");
    }
    return (*pool)[i];
}

// Runs every workgroup of `grid` in order on one team of blockDim fibers.
template <typename K, typename... A>
void launch(K kernel, dim3 grid, dim3 block, A... args) {
    const int nt = (int)(block.x * block.y * block.z);
    if (nt % 64) fail("workgroup size not a multiple of 64");
    Machine m;
    machine() = &m;
    gridDim = grid;
    blockDim = block;
    m.fibers = std::vector<Fiber>(nt);
    m.block.n = nt;
    m.waves = std::vector<Wave>(nt / 64);
    m.slot = std::vector<int>(nt);
    for (auto &w : m.waves) w.bar.n = 64;
    // HOSTEMU_WG_ORDER=reverse runs the workgroups last to first, so a
    // result that depends on which workgroup of a group arrives last (the
    // prefill key-split merge) is checked in both orders.
    const char *order = std::getenv("HOSTEMU_WG_ORDER");
    const bool reverse = order && !std::strcmp(order, "reverse");
    m.body = [&] {
        const unsigned nwg = grid.x * grid.y * grid.z;
        for (unsigned i = 0; i < nwg; i++) {
            const unsigned w = reverse ? nwg - 1 - i : i;
            blockIdx = dim3(w % grid.x, (w / grid.x) % grid.y, w / (grid.x * grid.y));
            kernel(args...);
            __syncthreads();  // the workgroup has ended before the next one starts
        }
    };
    const size_t stack_size = (size_t)1 << 17;
    for (int i = 0; i < nt; i++) {
        Fiber &f = m.fibers[i];
        f.tid = dim3(i % block.x, (i / block.x) % block.y, i / (block.x * block.y));
        f.lane = i & 63;
        f.wave = i >> 6;
        f.stack = stack_pool(i, stack_size);
        f.stack_size = stack_size;
        if (!f.stack) fail("fiber setup");
        // the frame hostemu_switch pops on the first switch in: control
        // words, six zeroed registers, then fiber_entry as the return
        // address, entered with the stack aligned as after a call
        uint64_t *top = reinterpret_cast<uint64_t *>(f.stack + stack_size) - 2;   // 16-byte aligned
        top[1] = 0;   // fiber_entry's own (never used) return address
        top[0] = reinterpret_cast<uint64_t>(&fiber_entry);
        uint64_t *sp = top - 7;
        for (int r = 1; r < 7; r++) sp[r] = 0;
        const uint32_t mxcsr = 0x1F80, fcw = 0x037F;   // power-on defaults
        sp[0] = mxcsr | (uint64_t)fcw << 32;
        f.sp = sp;
    }
    for (int left = nt; left > 0;) {
        bool ran = false;
        for (auto &f : m.fibers) {
            if (f.done || f.blocked) continue;
            ran = true;
            m.current = &f;
            threadIdx = f.tid;
            t_lane = f.lane;
            t_wave = f.wave;
            t_flat = (int)(&f - m.fibers.data());
#if defined(__SANITIZE_ADDRESS__)
            __sanitizer_start_switch_fiber(&m.sched_fake, f.stack, f.stack_size);
#endif
            hostemu_switch(&m.sched_sp, f.sp);
#if defined(__SANITIZE_ADDRESS__)
            __sanitizer_finish_switch_fiber(m.sched_fake, nullptr, nullptr);
#endif
            if (f.done) left--;
        }
        if (!ran && left > 0) fail("deadlock: a barrier or cross-lane operation not reached by every lane");
    }
    machine() = nullptr;
}

// launch, recorded in the launch log under `name`
template <typename K, typename... A>
void launch_named(const char *name, K kernel, dim3 grid, dim3 block, A... args) {
    const double t0 = hostemu_now_ms();
    launch(kernel, grid, block, args...);
    hostemu_count_launch(name, workgroups(grid), block.x * block.y * block.z, hostemu_now_ms() - t0);
}

}  // namespace hostemu

#define hipLaunchKernelGGL(kernel, grid, block, shmem, stream, ...) \
    ((void)(stream), hostemu::launch_named(#kernel, kernel, dim3(grid), dim3(block), __VA_ARGS__))

#endif
