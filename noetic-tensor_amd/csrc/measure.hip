// Platform figures for the benchmark's roofline (include/noetic_measure.h): the device's
// streaming-read rate and the period of dependent launches of an empty kernel.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <string>
#include <vector>

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

// Shader clock against the 100 MHz real-time counter over a dependent chain of fused
// multiply-adds on every lane (each block's first wave records both deltas).
__global__ __launch_bounds__(256) void k_clock(uint64_t *out, int iters) {
    const uint64_t c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    float a = float(threadIdx.x), b = 0.5f;
    for (int i = 0; i < iters; i++) {
        a = fmaf(a, 0.99993f, b);
        b = fmaf(b, 0.99991f, 0.25f);
    }
    const uint64_t c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        out[2 * blockIdx.x] = c1 - c0;
        out[2 * blockIdx.x + 1] = r1 - r0;
    }
    if (a == 1234.5f && b == 6.5f) out[0] = 0;  // keeps the chain
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

int nt_measure_shader_clock(int32_t seconds_ms, double *mhz) {
    if (!mhz || seconds_ms < 1 || seconds_ms > 10000)
        return fail(NT_E_ARG, "nt_measure_shader_clock: 1 to 10000 ms of load");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    constexpr int kBlocks = 256 * 8;   // eight 256-thread blocks per compute unit: every SIMD busy
    constexpr int kIters = 1 << 16;    // about 0.25 ms per launch
    void *out = nullptr;
    if (int rc = hip_check(hipMalloc(&out, 2 * kBlocks * sizeof(uint64_t)), "hipMalloc")) return rc;
    std::vector<uint64_t> h(2 * kBlocks);
    int rc = 0;
    const auto t0 = std::chrono::steady_clock::now();
    while (!rc) {  // the load, for the clock to settle; the last launch is the one read
        hipLaunchKernelGGL(k_clock, dim3(kBlocks), dim3(256), 0, ctx().stream, static_cast<uint64_t *>(out), kIters);
        rc = launched("nt_measure_shader_clock");
        if (!rc) rc = hip_check(hipStreamSynchronize(ctx().stream), "hipStreamSynchronize");
        if (std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(seconds_ms)) break;
    }
    if (!rc) rc = hip_check(hipMemcpy(h.data(), out, h.size() * sizeof(uint64_t), hipMemcpyDeviceToHost), "hipMemcpy");
    (void)hipFree(out);
    if (rc) return rc;
    std::vector<double> r;
    for (int b = 0; b < kBlocks; b++)
        if (h[2 * b + 1] > 0) r.push_back(double(h[2 * b]) / double(h[2 * b + 1]) * 100.0);
    if (r.empty()) return fail(NT_E_ARG, "nt_measure_shader_clock: no sample");
    std::nth_element(r.begin(), r.begin() + r.size() / 2, r.end());
    *mhz = r[r.size() / 2];
    return 0;
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
