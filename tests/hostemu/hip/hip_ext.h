// hip/hip_ext.h for the host-emulation build (see hip_runtime.h here).
// hipExtLaunchKernelGGL's timing events are ignored.
#ifndef G3_HOSTEMU_HIP_EXT_H
#define G3_HOSTEMU_HIP_EXT_H

#include "hip_runtime.h"

#define hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, ev0, ev1, flags, ...) \
    hostemu::launch(kernel, dim3(grid), dim3(block), __VA_ARGS__)

#endif
