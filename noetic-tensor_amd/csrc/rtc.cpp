// The row kernels' run-time path (nt_rtc.hpp: the samplers, the scorer and its backward): hiprtc
// compiles one template instance per program from the embedded device source, with the options
// the ahead-of-time build uses, so the two paths run the same code. Functions are cached per device and instance for the process, and
// code objects on disk (NOETIC_HIP_CACHE_DIR, else $HOME/.cache/noetic-hip) under a name that
// carries the source's SHA-256, the hiprtc version, the options and the instance, so a later
// process loads instead of compiling. The reference compiles its CUDA kernels with NVRTC at first
// use and caches the functions (src/tensor/cuda/mod.rs:169-218, cuda/backend.rs:281-293,
// 322-358).
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <sys/stat.h>
#include <unistd.h>
#include <utility>
#include <vector>

#include "../../include/noetic_hip.h"
#include "nt_internal.hpp"
#include "nt_rtc.hpp"
#include "rtc_sources.inc"

namespace nt {
namespace {

// The ahead-of-time build's device options (Makefile: DEVFLAGS, CXXFLAGS' -O3, -std=c++17 and
// -ffp-contract=off).
const char *const kOptions[] = {"--offload-arch=gfx950", "-O3",    "-std=c++17",      "-ffp-contract=off",
                                "-Xclang",              "-target-feature", "-Xclang", "-packed-fp32-ops"};
constexpr int kNumOptions = sizeof(kOptions) / sizeof(kOptions[0]);

std::mutex g_path_mu;
int g_path = -1;  // -1: not chosen yet

std::mutex g_mu;                                          // the cache (the context lock is held too)
std::map<std::pair<int, std::string>, hipFunction_t> g_fn;  // (device, name) -> function

int hiprtc_version() {
    int major = 0, minor = 0;
    if (hiprtcVersion(&major, &minor) != HIPRTC_SUCCESS) return 0;
    return major * 100 + minor;
}

uint64_t fnv1a(const std::string &s) {
    uint64_t h = 1469598103934665603ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 1099511628211ull;
    }
    return h;
}

// The on-disk code object's path for `name` (empty when no cache directory is usable).
std::string cache_path(const std::string &name) {
    std::string dir;
    if (const char *d = std::getenv("NOETIC_HIP_CACHE_DIR")) dir = d;
    else if (const char *h = std::getenv("HOME")) dir = std::string(h) + "/.cache/noetic-hip";
    if (dir.empty()) return std::string();
    std::string opts;
    for (int i = 0; i < kNumOptions; i++) opts += std::string(kOptions[i]) + " ";
    char tag[64];
    std::snprintf(tag, sizeof tag, "%016llx", (unsigned long long)fnv1a(opts + "|" + name));
    return dir + "/" + std::string(kRtcSha).substr(0, 16) + "-hiprtc" + std::to_string(hiprtc_version()) + "-" +
           tag + ".co";
}

// A cached entry: the lowered name, a newline, then the code object.
bool cache_read(const std::string &path, std::string *lowered, std::vector<char> *code) {
    if (path.empty()) return false;
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    std::stringstream ss;
    ss << f.rdbuf();
    const std::string all = ss.str();
    const size_t nl = all.find('\n');
    if (nl == std::string::npos || nl + 1 >= all.size()) return false;
    *lowered = all.substr(0, nl);
    code->assign(all.begin() + nl + 1, all.end());
    return true;
}

void cache_write(const std::string &path, const std::string &lowered, const std::vector<char> &code) {
    if (path.empty()) return;
    const size_t slash = path.rfind('/');
    const std::string dir = path.substr(0, slash);
    // make the directory chain (a missing parent is made first)
    for (size_t i = 1; i <= dir.size(); i++)
        if (i == dir.size() || dir[i] == '/') mkdir(dir.substr(0, i).c_str(), 0755);
    const std::string tmp = path + ".tmp" + std::to_string(getpid());
    {
        std::ofstream f(tmp, std::ios::binary);
        if (!f) return;
        f << lowered << '\n';
        f.write(code.data(), std::streamsize(code.size()));
        if (!f) return;
    }
    std::rename(tmp.c_str(), path.c_str());  // whole files only: a reader sees the old or the new
}

int compile(const std::string &name, std::string *lowered, std::vector<char> *code) {
    hiprtcProgram prog;
    const char *src =
        "#include \"rl_sample_kernels.hpp\"\n#include \"rl_score_kernels.hpp\"\n#include \"rl_gumbel_kernels.hpp\"\n";
    if (hiprtcCreateProgram(&prog, src, "nt_rtc.hip", kRtcFiles, kRtcTexts, kRtcNames) != HIPRTC_SUCCESS)
        return fail(NT_E_RTC, "hiprtcCreateProgram failed");
    hiprtcResult r = hiprtcAddNameExpression(prog, name.c_str());
    if (r == HIPRTC_SUCCESS) r = hiprtcCompileProgram(prog, kNumOptions, kOptions);
    if (r != HIPRTC_SUCCESS) {
        size_t n = 0;
        std::string log;
        if (hiprtcGetProgramLogSize(prog, &n) == HIPRTC_SUCCESS && n > 1) {
            log.resize(n);
            hiprtcGetProgramLog(prog, &log[0]);
        }
        hiprtcDestroyProgram(&prog);
        return fail(NT_E_RTC, "hiprtc: " + name + ": " + hiprtcGetErrorString(r) + "\n" + log.substr(0, 4000));
    }
    const char *ln = nullptr;
    size_t size = 0;
    if (hiprtcGetLoweredName(prog, name.c_str(), &ln) != HIPRTC_SUCCESS || !ln ||
        hiprtcGetCodeSize(prog, &size) != HIPRTC_SUCCESS || size == 0) {
        hiprtcDestroyProgram(&prog);
        return fail(NT_E_RTC, "hiprtc: no code or lowered name for " + name);
    }
    *lowered = ln;
    code->resize(size);
    r = hiprtcGetCode(prog, code->data());
    hiprtcDestroyProgram(&prog);
    if (r != HIPRTC_SUCCESS) return fail(NT_E_RTC, "hiprtcGetCode failed for " + name);
    return 0;
}

int function_for(const std::string &name, hipFunction_t *out) {
    std::lock_guard<std::mutex> lk(g_mu);
    const auto key = std::make_pair(ctx().device, name);
    auto it = g_fn.find(key);
    if (it != g_fn.end()) {
        *out = it->second;
        return 0;
    }
    std::string lowered;
    std::vector<char> code;
    const std::string path = cache_path(name);
    hipModule_t mod;
    bool loaded = false;
    if (cache_read(path, &lowered, &code)) {
        loaded = hipModuleLoadData(&mod, code.data()) == hipSuccess;  // a damaged file is compiled again
        if (!loaded) (void)hipGetLastError();
    }
    if (!loaded) {
        if (int rc = compile(name, &lowered, &code)) return rc;
        if (int rc = hip_check(hipModuleLoadData(&mod, code.data()), "hipModuleLoadData")) return rc;
        cache_write(path, lowered, code);
    }
    hipFunction_t fn;
    if (int rc = hip_check(hipModuleGetFunction(&fn, mod, lowered.c_str()), "hipModuleGetFunction")) return rc;
    g_fn.emplace(key, fn);  // the module stays loaded for the process, as the function needs it
    *out = fn;
    return 0;
}

}  // namespace

bool &aot_pinned() {
    thread_local bool pinned = false;
    return pinned;
}

int kernel_path() {
    std::lock_guard<std::mutex> lk(g_path_mu);
    if (g_path < 0) {
        const char *e = std::getenv("NOETIC_HIP_KERNELS");
        g_path = (e && std::strcmp(e, "rtc") == 0) ? NT_KERNELS_RTC : NT_KERNELS_AOT;
    }
    return g_path;
}

int rtc_launch(const std::string &name, dim3 grid, dim3 block, size_t shm, hipStream_t s, const void *arg) {
    hipFunction_t fn;
    if (int rc = function_for(name, &fn)) return rc;
    void *params[] = {const_cast<void *>(arg)};
    return hip_check(hipModuleLaunchKernel(fn, grid.x, grid.y, grid.z, block.x, block.y, block.z, unsigned(shm), s,
                                           params, nullptr),
                     "hipModuleLaunchKernel");
}

int &rtc_status() {
    static int rc = 0;
    return rc;
}

std::string rtc_key_part() {
    return "hiprtc" + std::to_string(hiprtc_version()) + "-kernels-" + std::string(kRtcSha).substr(0, 16);
}

}  // namespace nt

using namespace nt;

extern "C" int nt_hip_set_kernel_path(int path) {
    if (path != NT_KERNELS_AOT && path != NT_KERNELS_RTC)
        return fail(NT_E_ARG, "nt_hip_set_kernel_path: NT_KERNELS_AOT or NT_KERNELS_RTC");
    const int prev = kernel_path();
    std::lock_guard<std::mutex> lk(g_path_mu);
    g_path = path;
    return prev;
}

extern "C" int nt_hip_kernel_path(void) { return kernel_path(); }
