// hostrt.cpp - the HIP runtime API subset of hip/hip_runtime_api.h for the
// host-emulation builds (TEST INFRASTRUCTURE).  Device memory is host heap
// memory, every call is synchronous.
#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>

struct hostemu_stream {
    unsigned flags;
};
struct hostemu_event {
    double ms;
    bool recorded;
};

// The fibers' stack switch (declared in hip/hip_runtime.h): pushes the
// callee-saved registers and the SSE / x87 control words, stores the stack
// pointer in *from, loads `to` and pops the same from there.
asm(R"(
    .text
    .globl hostemu_switch
    .type hostemu_switch, @function
hostemu_switch:
    pushq %rbp
    pushq %rbx
    pushq %r12
    pushq %r13
    pushq %r14
    pushq %r15
    subq $8, %rsp
    stmxcsr (%rsp)
    fnstcw 4(%rsp)
    movq %rsp, (%rdi)
    movq %rsi, %rsp
    ldmxcsr (%rsp)
    fldcw 4(%rsp)
    addq $8, %rsp
    popq %r15
    popq %r14
    popq %r13
    popq %r12
    popq %rbx
    popq %rbp
    ret
    .size hostemu_switch, .-hostemu_switch
)");

namespace {

struct LaunchCount {
    int launches = 0;
    unsigned long long workgroups = 0;
    double ms = 0.0;
    unsigned threads = 0;   // threads per workgroup of the last launch
};
std::map<std::string, LaunchCount> &launches() {
    static std::map<std::string, LaunchCount> m;
    return m;
}

double now_ms() {
    using namespace std::chrono;
    return duration<double, std::milli>(steady_clock::now().time_since_epoch()).count();
}

unsigned long long g_alloc_calls = 0;   // hipMalloc / hipFree / hipHostMalloc / hipHostFree

void *aligned(size_t bytes) {
    // 256-byte alignment, as hipMalloc gives, and exactly the requested size
    // (at least one byte), so AddressSanitizer flags any access past it even
    // where the GPU allocator's granularity would have hidden it
    void *p = nullptr;
    return posix_memalign(&p, 256, bytes ? bytes : 1) == 0 ? p : nullptr;
}

}  // namespace

extern "C" {

hipError_t hipGetLastError(void) { return hipSuccess; }

const char *hipGetErrorString(hipError_t e) {
    switch (e) {
        case hipSuccess: return "hipSuccess";
        case hipErrorInvalidValue: return "hipErrorInvalidValue";
        case hipErrorOutOfMemory: return "hipErrorOutOfMemory";
        case hipErrorInvalidSymbol: return "hipErrorInvalidSymbol";
        case hipErrorInvalidDevice: return "hipErrorInvalidDevice";
    }
    return "hipErrorUnknown";
}

hipError_t hipGetDeviceCount(int *n) {
    *n = 1;
    return hipSuccess;
}
hipError_t hipGetDevice(int *d) {
    *d = 0;
    return hipSuccess;
}
hipError_t hipSetDevice(int d) { return d == 0 ? hipSuccess : hipErrorInvalidDevice; }

hipError_t hipDeviceGetAttribute(int *v, hipDeviceAttribute_t attr, int device) {
    if (device != 0) return hipErrorInvalidDevice;
    if (attr != hipDeviceAttributeMultiprocessorCount) return hipErrorInvalidValue;
    const char *e = std::getenv("HOSTEMU_CUS");
    *v = e && std::atoi(e) > 0 ? std::atoi(e) : 256;
    return hipSuccess;
}
hipError_t hipDeviceSynchronize(void) { return hipSuccess; }

hipError_t hipMalloc(void **p, size_t bytes) {
    g_alloc_calls++;
    *p = aligned(bytes);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipFree(void *p) {
    g_alloc_calls++;
    std::free(p);
    return hipSuccess;
}
hipError_t hipHostMalloc(void **p, size_t bytes, unsigned) {
    g_alloc_calls++;
    *p = aligned(bytes);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipHostFree(void *p) {
    g_alloc_calls++;
    std::free(p);
    return hipSuccess;
}
unsigned long long hostemu_alloc_calls(void) { return g_alloc_calls; }
hipError_t hipMemcpy(void *dst, const void *src, size_t bytes, hipMemcpyKind) {
    if (bytes) std::memcpy(dst, src, bytes);
    return hipSuccess;
}
hipError_t hipMemcpyAsync(void *dst, const void *src, size_t bytes, hipMemcpyKind kind, hipStream_t) {
    return hipMemcpy(dst, src, bytes, kind);
}
hipError_t hipMemset(void *p, int value, size_t bytes) {
    if (bytes) std::memset(p, value, bytes);
    return hipSuccess;
}

hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned flags) {
    *s = new hostemu_stream{flags};
    return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t s) {
    delete s;
    return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }

hipError_t hipEventCreate(hipEvent_t *e) {
    *e = new hostemu_event{0.0, false};
    return hipSuccess;
}
hipError_t hipEventDestroy(hipEvent_t e) {
    delete e;
    return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t e, hipStream_t) {
    if (!e) return hipErrorInvalidValue;
    e->ms = now_ms();
    e->recorded = true;
    return hipSuccess;
}
hipError_t hipEventSynchronize(hipEvent_t e) { return e ? hipSuccess : hipErrorInvalidValue; }
hipError_t hipEventElapsedTime(float *ms, hipEvent_t start, hipEvent_t stop) {
    if (!start || !stop || !start->recorded || !stop->recorded) return hipErrorInvalidValue;
    *ms = (float)(stop->ms - start->ms);
    return hipSuccess;
}

hipError_t hipGetSymbolAddress(void **p, const void *symbol) {
    if (!symbol) return hipErrorInvalidSymbol;
    *p = const_cast<void *>(symbol);
    return hipSuccess;
}

void hostemu_count_launch(const char *name, unsigned workgroups, unsigned threads, double ms) {
    LaunchCount &c = launches()[name];
    c.launches++;
    c.workgroups += workgroups;
    c.threads = threads;
    c.ms += ms;
}

double hostemu_now_ms(void) { return now_ms(); }

void hostemu_print_launches(void) {
    for (const auto &kv : launches())
        std::printf("launch %s %d %llu %u %.1f\n", kv.first.c_str(), kv.second.launches, kv.second.workgroups,
                    kv.second.threads, kv.second.ms);
}

}  // extern "C"
