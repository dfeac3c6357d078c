// Internal declarations shared by the translation units of libnoetic_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <string>

#include "../../include/noetic_hip.h"

namespace nt {

// The process-wide device context: one claimed device, one non-blocking stream at the default
// priority, one mutex serialising every device entry point, a launch counter.
struct Ctx {
    int device = -1;
    hipStream_t stream = nullptr;
    bool pools = false;  // stream-ordered allocation (hipMallocAsync / hipFreeAsync) on the device
    std::mutex mu;
    uint64_t launches = 0;
};

Ctx &ctx();

// Record the failure text for nt_hip_last_error() and return `code`.
int fail(int code, const std::string &msg);
// hipSuccess -> 0, else fail(err, "<what>: <name> (<code>): <desc>").
int hip_check(hipError_t err, const char *what);
// Check a kernel launch just issued on the library stream and count it.
int launched(const char *what);

// Lock the context, require a claimed device, make it current and free (stream-ordered) what
// nt_hip_free recorded since; on success `*out` holds the lock.
int enter(std::unique_lock<std::mutex> *out);
// enter() without the deferred frees: for entry points that must call no allocator routine.
int enter_nofree(std::unique_lock<std::mutex> *out);

// Device scratch for work queued on the library stream, with the context lock held: from the
// stream-ordered pool when the device has one. scratch_release orders the free after the work
// queued so far (hipFreeAsync), or, without a pool, records it for the next entry to free.
int scratch_alloc(size_t bytes, void **out);
int scratch_release(void *ptr);

// Clear n u32 words of device memory with a kernel on the library stream (a kernel, so that a
// caller capturing the stream into a graph records no memset node).
int zero_words(uint32_t *p, size_t n);

// The segmented sampler's workspace: kSegCounterBytes of u32 arrival counters, one per row, zero
// between launches, then the launch's wave records.
constexpr size_t kSegCounterBytes = size_t(1) << 18;
using WorkspaceFn = int (*)(size_t need, uint8_t **out);
// nt_hip_rl_sample's argument checks and dispatch with the workspace from `workspace`.
int sample_entry(const NtRlSampleArgs *a, WorkspaceFn workspace, bool nofree, const char *who);

}  // namespace nt
