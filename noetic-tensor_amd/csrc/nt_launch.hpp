// One launch of a kernel instance along the library's kernel path: the ahead-of-time code object
// (hipLaunchKernelGGL), or the instance compiled by hiprtc and launched with
// hipModuleLaunchKernel (rtc.cpp). Included by the .hip sources whose kernels take both paths.
#pragma once

#include <hip/hip_runtime.h>

#include "nt_rtc.hpp"

namespace nt {

// `aot` is the kernel's ahead-of-time instance, `name` the same instance's name expression in the
// embedded source, `p` its one by-value argument. An entry that pins the ahead-of-time path
// (AotPin) launches `aot` whatever the library's path. A failure on the run-time path is kept in
// rtc_status() (the first one of an entry's launches; later launches of that entry are skipped);
// the ahead-of-time path's launch errors are hipGetLastError's.
template <class P>
void launch_path(void (*aot)(P), const char *name, dim3 grid, dim3 block, size_t shm, hipStream_t s, const P &p) {
    if (kernel_path() == NT_KERNELS_RTC && !aot_pinned()) {
        if (rtc_status() == 0) rtc_status() = rtc_launch(name, grid, block, shm, s, &p);
        return;
    }
    hipLaunchKernelGGL(aot, grid, block, shm, s, p);
}

}  // namespace nt
