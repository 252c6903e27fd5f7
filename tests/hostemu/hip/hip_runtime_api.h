/* hip/hip_runtime_api.h for the host-emulation builds (TEST INFRASTRUCTURE).
 *
 * The subset of the HIP runtime API that the library's host code
 * (gemma3.c_amd/host/g3attn.c, C11) and the kernels' launchers call, for a
 * GPU emulated on the host (hip_runtime.h here).  C and C++.  Implemented in
 * ../hostrt.cpp:
 *   - "device" memory is host heap memory (hipMalloc is an aligned malloc), so
 *     AddressSanitizer sees every access the kernels and copies make;
 *   - everything is synchronous: a launch runs to completion before it
 *     returns, streams only order, events record the host clock;
 *   - hipDeviceGetAttribute(hipDeviceAttributeMultiprocessorCount) returns
 *     the environment variable HOSTEMU_CUS if set, else 256.
 */
#ifndef G3_HOSTEMU_HIP_RUNTIME_API_H
#define G3_HOSTEMU_HIP_RUNTIME_API_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum hipError_t {
    hipSuccess = 0,
    hipErrorInvalidValue = 1,
    hipErrorOutOfMemory = 2,
    hipErrorInvalidSymbol = 13,
    hipErrorInvalidDevice = 101,
} hipError_t;

typedef enum hipMemcpyKind {
    hipMemcpyHostToHost = 0,
    hipMemcpyHostToDevice = 1,
    hipMemcpyDeviceToHost = 2,
    hipMemcpyDeviceToDevice = 3,
    hipMemcpyDefault = 4,
} hipMemcpyKind;

typedef enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 0 } hipDeviceAttribute_t;

typedef struct hostemu_stream *hipStream_t;
typedef struct hostemu_event *hipEvent_t;

#define hipStreamNonBlocking 0x01

hipError_t hipGetLastError(void);
const char *hipGetErrorString(hipError_t e);
hipError_t hipGetDeviceCount(int *n);
hipError_t hipGetDevice(int *d);
hipError_t hipSetDevice(int d);
hipError_t hipDeviceGetAttribute(int *v, hipDeviceAttribute_t attr, int device);
hipError_t hipDeviceSynchronize(void);

hipError_t hipMalloc(void **p, size_t bytes);
hipError_t hipFree(void *p);
hipError_t hipHostMalloc(void **p, size_t bytes, unsigned flags);
hipError_t hipHostFree(void *p);
hipError_t hipMemcpy(void *dst, const void *src, size_t bytes, hipMemcpyKind kind);
hipError_t hipMemcpyAsync(void *dst, const void *src, size_t bytes, hipMemcpyKind kind, hipStream_t s);
hipError_t hipMemset(void *p, int value, size_t bytes);

hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned flags);
hipError_t hipStreamDestroy(hipStream_t s);
hipError_t hipStreamSynchronize(hipStream_t s);

hipError_t hipEventCreate(hipEvent_t *e);
hipError_t hipEventDestroy(hipEvent_t e);
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s);
hipError_t hipEventSynchronize(hipEvent_t e);
hipError_t hipEventElapsedTime(float *ms, hipEvent_t start, hipEvent_t stop);

hipError_t hipGetSymbolAddress(void **p, const void *symbol);

/* Emulator bookkeeping: counts launches, their workgroups and the host
 * milliseconds they took by kernel name, with the last launch's threads per
 * workgroup (hip_runtime.h's launch macros call it after each launch);
 * hostemu_print_launches writes
 * "launch <name> <launches> <workgroups> <threads> <ms>" lines to stdout. */
void hostemu_count_launch(const char *name, unsigned workgroups, unsigned threads, double ms);
/* Calls of the allocating and freeing entry points above (hipMalloc,
 * hipFree, hipHostMalloc, hipHostFree) since the process started. */
unsigned long long hostemu_alloc_calls(void);
double hostemu_now_ms(void);
void hostemu_print_launches(void);

#ifdef __cplusplus
}
#endif

#endif
