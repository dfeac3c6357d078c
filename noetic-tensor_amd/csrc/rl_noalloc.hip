// nt_hip_rl_sample_noalloc: nt_hip_rl_sample for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It has
// the same arguments, kernels and results; the one difference is where the segmented sampler's
// workspace lives: a fixed device array, `scratch`, instead of the library's allocation. The
// call makes no hipMalloc, hipFree or other allocating call, and it always launches the
// library's ahead-of-time code objects: on the run-time kernel path (hiprtc) a kernel instance's
// first launch compiles it and loads its code object, which allocates device memory, so this
// entry does not take that path (both paths compute the same bytes).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/noetic_hip.h"
#include "nt_internal.hpp"
#include "nt_rtc.hpp"

namespace nt {
namespace {

// The workspace: the segmented sampler's arrival counters (kSegCounterBytes, zero between
// launches) and its wave records, kNoallocScratchBytes in all, one copy per GPU, held until the
// process ends. Static storage starts at zero; the counters are cleared once more when a device
// first uses the array. Every call on a GPU shares that GPU's copy and leaves it holding the last
// call's records (the counters back at zero). Calls are ordered by the library's one stream;
// calls that overlap on one GPU race (for example a captured graph of this call replayed on
// another stream while the library's stream runs one). Another process has its own copy.
constexpr size_t kNoallocScratchBytes = size_t(2) << 20;
static_assert(kNoallocScratchBytes > kSegCounterBytes, "scratch holds the counters and the records");
__device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
// This device's address of `scratch`, once looked up (the host-side name is only a stand-in).
uint8_t *g_scratch_ptr[kMaxDevices] = {};

int scratch_workspace(size_t need, uint8_t **out) {
    if (need > kNoallocScratchBytes)
        return fail(NT_E_ARG, "nt_hip_rl_sample_noalloc: the launch needs " + std::to_string(need) +
                                  " bytes of workspace, more than the allocation-free maximum of " +
                                  std::to_string(kNoallocScratchBytes) + " bytes");
    const int dev = ctx().device;
    if (dev < 0 || dev >= kMaxDevices) return fail(NT_E_ARG, "nt_hip_rl_sample_noalloc: device index");
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        if (int rc = hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress")) return rc;
        if (int rc = zero_words(static_cast<uint32_t *>(ptr), kSegCounterBytes / sizeof(uint32_t))) return rc;
        g_scratch_ptr[dev] = static_cast<uint8_t *>(ptr);
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace
}  // namespace nt

extern "C" int nt_hip_rl_sample_noalloc(const NtRlSampleArgs *a) {
    const nt::AotPin pin;  // the ahead-of-time code objects whatever the library's kernel path
    return nt::sample_entry(a, nt::scratch_workspace, true, "nt_hip_rl_sample_noalloc");
}
