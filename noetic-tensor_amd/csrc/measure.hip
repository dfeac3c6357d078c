// Platform figures for the benchmark's roofline (include/noetic_measure.h): the device's
// streaming-read rate and the period of dependent launches of an empty kernel.
#include <hip/hip_runtime.h>

#include <string>

#include "../../include/noetic_measure.h"
#include "nt_internal.hpp"

namespace nt {
namespace {

// Each block reads its own contiguous share of the buffer, every thread eight 16-byte words at a
// time (all eight in flight), with non-temporal loads; each block writes one word, so the reads
// cannot be dropped. Of the plain read kernels tried on MI355X (grid-stride over the whole buffer,
// contiguous shares of 256- to 1024-thread blocks, 4 or 8 words in flight, default or
// non-temporal loads) this one read fastest: 6.97 TB/s over 2 GiB, against 6.75 with default
// loads and 5.57 for a grid-stride loop.
typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));
constexpr int kReadThreads = 256;
constexpr int kReadInFlight = 8;
constexpr int kReadBlocks = 4096;
__global__ __launch_bounds__(kReadThreads) void k_stream_read(const v4u32 *p, size_t per_block, uint32_t *sink) {
    const v4u32 *q = p + per_block * blockIdx.x;
    uint32_t acc = 0;
    for (size_t i = threadIdx.x; i < per_block; i += size_t(kReadInFlight) * kReadThreads) {
        v4u32 v[kReadInFlight];
#pragma unroll
        for (int u = 0; u < kReadInFlight; u++) v[u] = __builtin_nontemporal_load(q + i + size_t(u) * kReadThreads);
#pragma unroll
        for (int u = 0; u < kReadInFlight; u++) acc ^= v[u].x ^ v[u].w;
    }
    if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

__global__ void k_nothing(uint32_t *never) {
    if (never && threadIdx.x == 0 && blockIdx.x == 0x7fffffff) never[0] = 1;
}

// HIP-event time (ms) of `run` queued on the library stream.
template <class F>
int event_ms(F run, float *ms) {
    hipEvent_t e0, e1;
    if (int rc = hip_check(hipEventCreate(&e0), "hipEventCreate")) return rc;
    if (int rc = hip_check(hipEventCreate(&e1), "hipEventCreate")) {
        (void)hipEventDestroy(e0);
        return rc;
    }
    int rc = hip_check(hipEventRecord(e0, ctx().stream), "hipEventRecord");
    if (!rc) rc = run();
    if (!rc) rc = hip_check(hipEventRecord(e1, ctx().stream), "hipEventRecord");
    if (!rc) rc = hip_check(hipEventSynchronize(e1), "hipEventSynchronize");
    if (!rc) rc = hip_check(hipEventElapsedTime(ms, e0, e1), "hipEventElapsedTime");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" {

int nt_measure_read(size_t bytes, int32_t reps, double *gbs) {
    constexpr size_t kUnit = size_t(kReadBlocks) * kReadThreads * kReadInFlight * 16;  // 128 MiB
    if (!gbs || reps < 1 || bytes < kUnit || bytes % kUnit != 0)
        return fail(NT_E_ARG, "nt_measure_read: bytes a positive multiple of 128 MiB, reps >= 1");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    constexpr int kBlocks = kReadBlocks;
    void *buf = nullptr, *sink = nullptr;
    if (int rc = hip_check(hipMalloc(&buf, bytes), "hipMalloc")) return rc;
    int rc = hip_check(hipMalloc(&sink, kBlocks * sizeof(uint32_t)), "hipMalloc");
    if (!rc) rc = zero_words(static_cast<uint32_t *>(buf), bytes / 4);
    auto once = [&]() {
        hipLaunchKernelGGL(k_stream_read, dim3(kBlocks), dim3(kReadThreads), 0, ctx().stream,
                           static_cast<const v4u32 *>(buf), bytes / 16 / kBlocks, static_cast<uint32_t *>(sink));
        return launched("nt_measure_read");
    };
    if (!rc) rc = once();  // first touch
    float ms = 0.0f;
    if (!rc)
        rc = event_ms([&]() {
            for (int i = 0; i < reps; i++)
                if (int r = once()) return r;
            return 0;
        }, &ms);
    if (!rc) *gbs = double(bytes) * reps / (double(ms) * 1e-3) / 1e9;
    (void)hipStreamSynchronize(ctx().stream);
    (void)hipFree(sink);
    (void)hipFree(buf);
    return rc;
}

int nt_measure_launch_period(int32_t blocks, int32_t threads, int32_t launches, double *us) {
    if (!us || blocks < 1 || threads < 1 || threads > 1024 || launches < 1)
        return fail(NT_E_ARG, "nt_measure_launch_period: blocks >= 1, threads in 1..1024, launches >= 1");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    auto run = [&]() {
        for (int i = 0; i < launches; i++) {
            hipLaunchKernelGGL(k_nothing, dim3(blocks), dim3(threads), 0, ctx().stream, nullptr);
            if (int r = launched("nt_measure_launch_period")) return r;
        }
        return 0;
    };
    if (int rc = run()) return rc;  // warm the launch path
    float ms = 0.0f;
    if (int rc = event_ms(run, &ms)) return rc;
    *us = double(ms) * 1e3 / launches;
    return 0;
}

}  // extern "C"
