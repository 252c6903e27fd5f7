// hip/hip_ext.h for the host-emulation builds (see hip_runtime.h here).
// hipExtLaunchKernelGGL records its start / stop events (when given) around
// the launch, on the host clock.
#ifndef G3_HOSTEMU_HIP_EXT_H
#define G3_HOSTEMU_HIP_EXT_H

#include "hip_runtime.h"

#define hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, ev0, ev1, flags, ...)      \
    do {                                                                                    \
        hipEvent_t hostemu_e0 = (ev0), hostemu_e1 = (ev1);                                  \
        if (hostemu_e0) hipEventRecord(hostemu_e0, (stream));                                \
        hostemu::launch_named(#kernel, kernel, dim3(grid), dim3(block), __VA_ARGS__);       \
        if (hostemu_e1) hipEventRecord(hostemu_e1, (stream));                                \
    } while (0)

#endif
