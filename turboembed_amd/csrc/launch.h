// The one way the kernel sources enqueue a kernel: through the launch hook
// (LaunchTiming), so a timed run's events are bound to the kernels' own
// dispatch packets.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "kernels.h"

namespace rocm {

template <typename... Formals, typename... Actuals>
inline void enqueue(void (*k)(Formals...), dim3 grid, dim3 block, uint32_t lds, hipStream_t s, Actuals... a) {
    LaunchTiming &t = launch_timing();
    hipExtLaunchKernelGGL(k, grid, block, lds, s, t.start, t.stop, 0u, a...);
    if (t.stop) {
        t.start = nullptr;
        t.bound = true;
    }
}

}  // namespace rocm
