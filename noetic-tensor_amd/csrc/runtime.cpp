// Host runtime of libnoetic_hip.so: device claim, the library stream, memory and copies,
// errors, the provenance key. It replaces the device/context/memory part of the reference's
// GpuBackend (src/tensor/gpu/mod.rs:137-207) and CUDA context handling
// (src/tensor/cuda/backend.rs:104-264) for a `Device::Hip(i)`.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/noetic_hip.h"
#include "nt_internal.hpp"
#include "nt_rtc.hpp"

#ifndef NT_KERNELS_SHA
#define NT_KERNELS_SHA "unknown"
#endif

namespace nt {

Ctx &ctx() {
    static Ctx c;
    return c;
}

static thread_local std::string g_last_error;

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

int hip_check(hipError_t err, const char *what) {
    if (err == hipSuccess) return 0;
    char buf[512];
    std::snprintf(buf, sizeof buf, "HIP %s: %s (%d): %s", what, hipGetErrorName(err), (int)err,
                  hipGetErrorString(err));
    return fail((int)err, buf);
}

int launched(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_check(e, what);
    ctx().launches++;
    return 0;
}

// Pointers released by nt_hip_free since the last entry, freed on the stream by the next one
// (the reference's PENDING_FREE, src/tensor/cuda/backend.rs:35-45 and 222-243: a release only
// records the pointer, so it never waits for the device or for the context's lock).
static std::mutex g_pending_mu;
static std::vector<void *> g_pending;

int enter_nofree(std::unique_lock<std::mutex> *out) {
    Ctx &c = ctx();
    std::unique_lock<std::mutex> lk(c.mu);
    if (c.device < 0) return fail(NT_E_UNCLAIMED, "no HIP device claimed in this process (nt_hip_claim)");
    hipError_t e = hipSetDevice(c.device);
    if (e != hipSuccess) return hip_check(e, "hipSetDevice");
    *out = std::move(lk);
    return 0;
}

int enter(std::unique_lock<std::mutex> *out) {
    Ctx &c = ctx();
    std::unique_lock<std::mutex> lk(c.mu);
    if (c.device < 0) return fail(NT_E_UNCLAIMED, "no HIP device claimed in this process (nt_hip_claim)");
    hipError_t e = hipSetDevice(c.device);
    if (e != hipSuccess) return hip_check(e, "hipSetDevice");
    std::vector<void *> freed;
    {
        std::lock_guard<std::mutex> pl(g_pending_mu);
        freed.swap(g_pending);
    }
    for (size_t i = 0; i < freed.size(); ++i) {
        // the work queued before the release still runs first: the free is ordered after it
        void *p = freed[i];
        int rc = 0;
        if (c.pools) {
            rc = hip_check(hipFreeAsync(p, c.stream), "hipFreeAsync");
        } else {
            rc = hip_check(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
            if (!rc) rc = hip_check(hipFree(p), "hipFree");
        }
        if (rc) {
            // keep what is not freed yet for the next entry
            std::lock_guard<std::mutex> pl(g_pending_mu);
            g_pending.insert(g_pending.end(), freed.begin() + (ptrdiff_t)i + 1, freed.end());
            return rc;
        }
    }
    *out = std::move(lk);
    return 0;
}

int scratch_alloc(size_t bytes, void **out) {
    *out = nullptr;
    if (bytes == 0) return 0;
    if (ctx().pools) return hip_check(hipMallocAsync(out, bytes, ctx().stream), "hipMallocAsync");
    return hip_check(hipMalloc(out, bytes), "hipMalloc");
}

int scratch_release(void *ptr) {
    if (!ptr) return 0;
    if (ctx().pools) return hip_check(hipFreeAsync(ptr, ctx().stream), "hipFreeAsync");
    std::lock_guard<std::mutex> pl(g_pending_mu);
    g_pending.push_back(ptr);
    return 0;
}

}  // namespace nt

using namespace nt;

extern "C" {

int nt_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

int nt_hip_claim(int device) {
    Ctx &c = ctx();
    std::lock_guard<std::mutex> lk(c.mu);
    if (c.device == device) return 0;
    if (c.device >= 0) {
        char buf[160];
        std::snprintf(buf, sizeof buf, "Hip(%d): this process already uses Hip(%d) (one device per process)",
                      device, c.device);
        return fail(NT_E_CLAIMED, buf);
    }
    int n = 0;
    if (int rc = hip_check(hipGetDeviceCount(&n), "hipGetDeviceCount")) return rc;
    if (device < 0 || device >= n) {
        char buf[120];
        std::snprintf(buf, sizeof buf, "Hip(%d): %d HIP device(s) visible", device, n);
        return fail(NT_E_ARG, buf);
    }
    if (int rc = hip_check(hipSetDevice(device), "hipSetDevice")) return rc;
    int pools = 0;
    if (hipDeviceGetAttribute(&pools, hipDeviceAttributeMemoryPoolsSupported, device) != hipSuccess) {
        (void)hipGetLastError();
        pools = 0;
    }
    if (pools) {
        // Keep freed memory in the pool across synchronisations instead of returning it to the
        // driver, as the reference does (src/tensor/cuda/backend.rs:207-213): otherwise the first
        // allocation after every sync maps its memory again.
        hipMemPool_t pool = nullptr;
        if (int rc = hip_check(hipDeviceGetDefaultMemPool(&pool, device), "hipDeviceGetDefaultMemPool")) return rc;
        uint64_t threshold = UINT64_MAX;
        if (int rc = hip_check(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &threshold),
                               "hipMemPoolSetAttribute"))
            return rc;
    }
    hipStream_t s = nullptr;
    // Default priority only: streams of other priorities are not used by this library.
    if (int rc = hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags"))
        return rc;
    c.device = device;
    c.stream = s;
    c.pools = pools != 0;
    return 0;
}

const char *nt_hip_last_error(void) { return g_last_error.c_str(); }

int nt_hip_key(char *buf, size_t cap) {
    if (!buf || cap == 0) return fail(NT_E_ARG, "nt_hip_key: empty buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    hipDeviceProp_t prop;
    if (int rc = hip_check(hipGetDeviceProperties(&prop, ctx().device), "hipGetDeviceProperties")) return rc;
    int rt = 0;
    (void)hipRuntimeGetVersion(&rt);
    std::string arch(prop.gcnArchName);
    for (char &ch : arch)
        if (ch == ':') ch = '_';
    std::string sha(NT_KERNELS_SHA);
    std::string key = "hip-" + arch + "-hiprt" + std::to_string(rt) + "-kernels-" + sha.substr(0, 16);
    // the sampler kernels compiled at run time add hiprtc's version and the embedded source's hash
    // (the CUDA backend's key names NVRTC and its sources, cuda/backend.rs:962-966)
    if (kernel_path() == NT_KERNELS_RTC) key += "-" + rtc_key_part();
    std::snprintf(buf, cap, "%s", key.c_str());
    return 0;
}

int nt_hip_platform_details(char *buf, size_t cap) {
    if (!buf || cap == 0) return fail(NT_E_ARG, "nt_hip_platform_details: empty buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    int drv = 0;
    if (int rc = hip_check(hipDriverGetVersion(&drv), "hipDriverGetVersion")) return rc;
    // The kernel driver's release, when the amdgpu module reports one (a packaged driver does;
    // the one built into the kernel does not).
    std::string kmd = "inbox";
    if (std::FILE *f = std::fopen("/sys/module/amdgpu/version", "r")) {
        char v[64] = {0};
        if (std::fgets(v, sizeof v, f)) {
            std::string t(v);
            while (!t.empty() && (t.back() == '\n' || t.back() == ' ')) t.pop_back();
            if (!t.empty()) kmd = t;
        }
        std::fclose(f);
    }
    // The compiler that built the code objects: its version and release tag, without the
    // repository URL and commit.
    std::string cc;
    {
        std::string word;
        const std::string text = std::string(__clang_version__) + " ";
        for (char ch : text) {
            if (ch != ' ' && ch != '(' && ch != ')') {
                word += ch;
                continue;
            }
            bool url = word.rfind("http", 0) == 0;
            bool commit = word.size() >= 32 && word.find_first_not_of("0123456789abcdef") == std::string::npos;
            if (!word.empty() && !url && !commit) cc += (cc.empty() ? "" : "-") + word;
            word.clear();
        }
    }
    std::string d = "hipdriver" + std::to_string(drv) + "-amdgpu-" + kmd + "-clang-" + cc;
    for (char &ch : d)
        if (ch == ' ' || ch == ':') ch = '_';
    if (d.size() + 1 > cap) return fail(NT_E_ARG, "nt_hip_platform_details: buffer too small");
    std::snprintf(buf, cap, "%s", d.c_str());
    return 0;
}

int nt_hip_alloc(size_t bytes, void **out) {
    if (!out) return fail(NT_E_ARG, "nt_hip_alloc: null out");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    *out = nullptr;
    if (bytes == 0) return 0;
    // From the device's stream-ordered pool when it has one (cuMemAllocAsync in the reference,
    // src/tensor/cuda/backend.rs:245-264): usable by work queued on the library stream after it.
    if (ctx().pools) return hip_check(hipMallocAsync(out, bytes, ctx().stream), "hipMallocAsync");
    return hip_check(hipMalloc(out, bytes), "hipMalloc");
}

int nt_hip_free(void *ptr) {
    if (!ptr) return 0;
    std::lock_guard<std::mutex> pl(g_pending_mu);
    g_pending.push_back(ptr);
    return 0;
}

int nt_hip_upload(void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return 0;
    if (!dst || !src) return fail(NT_E_ARG, "nt_hip_upload: null pointer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (int rc = hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx().stream), "upload"))
        return rc;
    return hip_check(hipStreamSynchronize(ctx().stream), "hipStreamSynchronize");
}

int nt_hip_download(void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return 0;
    if (!dst || !src) return fail(NT_E_ARG, "nt_hip_download: null pointer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (int rc = hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx().stream), "download"))
        return rc;
    return hip_check(hipStreamSynchronize(ctx().stream), "hipStreamSynchronize");
}

int nt_hip_memset(void *dst, int value, size_t bytes) {
    if (bytes == 0) return 0;
    if (!dst) return fail(NT_E_ARG, "nt_hip_memset: null pointer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    return hip_check(hipMemsetAsync(dst, value, bytes, ctx().stream), "hipMemsetAsync");
}

int nt_hip_sync(void) {
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    return hip_check(hipStreamSynchronize(ctx().stream), "hipStreamSynchronize");
}

int nt_hip_stream(void **out) {
    if (!out) return fail(NT_E_ARG, "nt_hip_stream: null out");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    *out = (void *)ctx().stream;
    return 0;
}

uint64_t nt_hip_launches(void) {
    std::lock_guard<std::mutex> lk(ctx().mu);
    return ctx().launches;
}

}  // extern "C"
