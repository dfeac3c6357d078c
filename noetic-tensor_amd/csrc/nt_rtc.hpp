// The row kernels' run-time path (the samplers, the scorer and its backward): compiled by hiprtc
// at first use from the device source embedded in the library (rl_sample_kernels.hpp,
// rl_score_kernels.hpp and the headers they include), loaded with
// hipModuleLoadData and launched with hipModuleLaunchKernel, one function per template instance.
// The ahead-of-time code objects (hipcc, the library's default) run the same source.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <string>

#include "../../include/noetic_hip.h"

namespace nt {

// NT_KERNELS_AOT or NT_KERNELS_RTC: from nt_hip_set_kernel_path, else NOETIC_HIP_KERNELS
// ("aot" or "rtc"), else NT_KERNELS_AOT.
int kernel_path();

// Launch `name` (a name expression of the embedded source, such as
// "nt::k_sample_rr<1, 1, 16, false, 8, 1>") on `s`: compiled, loaded and cached on first use on
// the current device. `arg` is the kernel's one by-value argument. Call with the context lock
// held; a compile failure is returned as NT_E_RTC with hiprtc's log, a load failure as HIP's.
int rtc_launch(const std::string &name, dim3 grid, dim3 block, size_t shm, hipStream_t s, const void *arg);

// The status of the run-time path's launches since an entry point last cleared it (0: none
// failed). Entry points clear it before their launches and return it if set; they are serialised
// by the context lock.
int &rtc_status();

// The key's middle for the run-time path: "hiprtc<version>-kernels-<sha16 of the embedded source>".
std::string rtc_key_part();

// Set while an entry point must launch the ahead-of-time code objects whatever kernel_path()
// says: the allocation-free entry (compiling and loading a run-time code object allocates device
// memory). Entry points are serialised by the context lock; the flag is per thread all the same.
bool &aot_pinned();
struct AotPin {
    bool prev;
    AotPin() : prev(aot_pinned()) { aot_pinned() = true; }
    ~AotPin() { aot_pinned() = prev; }
};

// "true" / "false" for a name expression.
inline const char *rtc_bool(bool b) { return b ? "true" : "false"; }

}  // namespace nt
