// Synthetic workload generators (no reference counterpart): seeded inputs of the benchmark
// configurations, generated on the device from counter-addressed ChaCha20 blocks.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/noetic_hip.h"
#include "../../include/noetic_rng.h"
#include "../../include/noetic_synth.h"
#include "nt_chacha.hpp"
#include "nt_internal.hpp"

namespace nt {
namespace {

using Key = ChachaKey;

__device__ __forceinline__ uint64_t u64_at(const uint32_t w[16], int j) {
    return uint64_t(w[2 * j]) | (uint64_t(w[2 * j + 1]) << 32);
}

// bf16 round-to-nearest-even of an f32 (src/tensor/half.rs:16-23).
__device__ __forceinline__ uint16_t to_bf16(float x) {
    uint32_t b = __float_as_uint(x);
    if (x != x) return uint16_t((b >> 16) | 0x0040u);
    return uint16_t((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ double box_muller(uint64_t k1, uint64_t k2) {
    double u1 = double(k1 >> 11) * 0x1p-53;
    if (u1 < 1e-300) u1 = 1e-300;
    const double u2 = double(k2 >> 11) * 0x1p-53;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925 * u2);
}

struct NormalP {
    void *out;
    const void *base;
    int dtype;
    int64_t n, V;
    Key key;
    double mean, std, zipf;
    const int64_t *rot;
};

__global__ void k_normal(NormalP p) {
    const int64_t nblk = (p.n + 3) / 4;
    for (int64_t b = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; b < nblk; b += int64_t(gridDim.x) * blockDim.x) {
        uint32_t w[16];
        chacha_block_dev(p.key, uint64_t(b), w);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int64_t i = 4 * b + j;
            if (i >= p.n) break;
            double v = p.mean + p.std * box_muller(u64_at(w, 2 * j), u64_at(w, 2 * j + 1));
            if (p.zipf > 0.0) {
                const int64_t r = i / p.V, col = i % p.V;
                const int64_t rank = (col + p.rot[r]) % p.V;
                v += -p.zipf * log(1.0 + double(rank));
            }
            if (p.base) {
                if (p.dtype == NT_F32) v += double(static_cast<const float *>(p.base)[i]);
                else v += double(__uint_as_float(uint32_t(static_cast<const uint16_t *>(p.base)[i]) << 16));
            }
            const float f = float(v);
            if (p.dtype == NT_F32) static_cast<float *>(p.out)[i] = f;
            else static_cast<uint16_t *>(p.out)[i] = to_bf16(f);
        }
    }
}

// Draw r of a stream: u64 r mod m, written for r < n.
__global__ void k_u64_mod(Key key, int64_t n, int64_t m, int64_t *out64, int32_t *out32) {
    const int64_t nblk = (n + 7) / 8;
    for (int64_t b = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; b < nblk; b += int64_t(gridDim.x) * blockDim.x) {
        uint32_t w[16];
        chacha_block_dev(key, uint64_t(b), w);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int64_t i = 8 * b + j;
            if (i >= n) break;
            const int64_t v = int64_t(u64_at(w, j) % uint64_t(m));
            if (out64) out64[i] = v;
            if (out32) out32[i] = int32_t(v);
        }
    }
}

__global__ void k_spikes(void *x, int dtype, int64_t rows, int64_t V, int k, const int64_t *base, double value) {
    const int64_t r = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
    if (r >= rows) return;
    const int64_t step = V / k;
    for (int j = 0; j < k; j++) {
        const int64_t i = r * V + (base[r] + j * step) % V;
        if (dtype == NT_F32) {
            float *p = static_cast<float *>(x) + i;
            *p = float(double(*p) + value);
        } else {
            uint16_t *p = static_cast<uint16_t *>(x) + i;
            *p = to_bf16(float(double(__uint_as_float(uint32_t(*p) << 16)) + value));
        }
    }
}

__global__ void k_bernoulli(uint8_t *out, int64_t n, Key key, uint32_t thresh, int full) {
    const int64_t nblk = (n + 15) / 16;
    for (int64_t b = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; b < nblk; b += int64_t(gridDim.x) * blockDim.x) {
        uint32_t w[16];
        chacha_block_dev(key, uint64_t(b), w);
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int64_t i = 16 * b + j;
            if (i >= n) break;
            out[i] = (full || w[j] < thresh) ? 1 : 0;
        }
    }
}

__global__ void k_keep_tokens(uint8_t *mask, int64_t rows, int64_t ld, const int32_t *tokens) {
    const int64_t r = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
    if (r < rows) mask[r * ld + tokens[r]] = 1;
}

int grid_for(int64_t work, int threads) {
    int64_t g = (work + threads - 1) / threads;
    if (g > 1 << 20) g = 1 << 20;
    return int(g < 1 ? 1 : g);
}

Key to_key(const uint32_t k[8]) {
    Key r;
    for (int i = 0; i < 8; i++) r.k[i] = k[i];
    return r;
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" {

int nt_synth_normal(const NtSynthNormal *a) {
    if (!a || !a->out || a->rows < 0 || a->vocab < 1 || (a->dtype != NT_F32 && a->dtype != NT_BF16))
        return fail(NT_E_ARG, "nt_synth_normal: invalid arguments");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    const int64_t n = a->rows * a->vocab;
    if (n == 0) return 0;
    hipStream_t s = ctx().stream;
    int64_t *rot = nullptr;
    if (a->zipf_s > 0.0) {
        if (int rc = hip_check(hipMalloc(&rot, size_t(a->rows) * sizeof(int64_t)), "hipMalloc")) return rc;
        hipLaunchKernelGGL(k_u64_mod, dim3(grid_for((a->rows + 7) / 8, 256)), dim3(256), 0, s, to_key(a->rot_key),
                           a->rows, a->vocab, rot, (int32_t *)nullptr);
        if (int rc = launched("synth rotations")) return rc;
    }
    NormalP p{a->out, a->base, a->dtype, n, a->vocab, to_key(a->key), a->mean, a->std, a->zipf_s, rot};
    hipLaunchKernelGGL(k_normal, dim3(grid_for((n + 3) / 4, 256)), dim3(256), 0, s, p);
    int rc = launched("nt_synth_normal");
    if (rot) {
        int rc2 = hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        (void)hipFree(rot);
        if (!rc) rc = rc2;
    }
    return rc;
}

int nt_synth_spikes(void *x, int32_t dtype, int64_t rows, int64_t vocab, int32_t k, const uint32_t key[8],
                    double value) {
    if (!x || !key || rows < 0 || vocab < 1 || k < 1 || k > vocab || (dtype != NT_F32 && dtype != NT_BF16))
        return fail(NT_E_ARG, "nt_synth_spikes: invalid arguments");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (rows == 0) return 0;
    hipStream_t s = ctx().stream;
    int64_t *base = nullptr;
    if (int rc = hip_check(hipMalloc(&base, size_t(rows) * sizeof(int64_t)), "hipMalloc")) return rc;
    hipLaunchKernelGGL(k_u64_mod, dim3(grid_for((rows + 7) / 8, 256)), dim3(256), 0, s, to_key(key), rows, vocab, base,
                       (int32_t *)nullptr);
    int rc = launched("synth spike bases");
    if (!rc) {
        hipLaunchKernelGGL(k_spikes, dim3(grid_for(rows, 64)), dim3(64), 0, s, x, int(dtype), rows, vocab, int(k), base,
                           value);
        rc = launched("nt_synth_spikes");
    }
    int rc2 = hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    (void)hipFree(base);
    return rc ? rc : rc2;
}

int nt_synth_bernoulli_mask(uint8_t *out, int64_t n, const uint32_t key[8], double p) {
    if (!out || !key || n < 0 || !(p >= 0.0 && p <= 1.0)) return fail(NT_E_ARG, "nt_synth_bernoulli_mask: invalid arguments");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (n == 0) return 0;
    const double t = p * 4294967296.0;
    const uint32_t thresh = t >= 4294967295.0 ? 0xffffffffu : uint32_t(t);
    hipLaunchKernelGGL(k_bernoulli, dim3(grid_for((n + 15) / 16, 256)), dim3(256), 0, ctx().stream, out, n, to_key(key),
                       thresh, p >= 1.0 ? 1 : 0);
    return launched("nt_synth_bernoulli_mask");
}

int nt_synth_tokens(int32_t *out, int64_t n, const uint32_t key[8], int64_t vocab) {
    if (!out || !key || n < 0 || vocab < 1 || vocab > 0x7fffffffLL) return fail(NT_E_ARG, "nt_synth_tokens: invalid arguments");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_u64_mod, dim3(grid_for((n + 7) / 8, 256)), dim3(256), 0, ctx().stream, to_key(key), n, vocab,
                       (int64_t *)nullptr, out);
    return launched("nt_synth_tokens");
}

int nt_synth_keep_tokens(uint8_t *mask, int64_t rows, int64_t mask_ld, const int32_t *tokens) {
    if (!mask || !tokens || rows < 0 || mask_ld < 1) return fail(NT_E_ARG, "nt_synth_keep_tokens: invalid arguments");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (rows == 0) return 0;
    hipLaunchKernelGGL(k_keep_tokens, dim3(grid_for(rows, 256)), dim3(256), 0, ctx().stream, mask, rows, mask_ld, tokens);
    return launched("nt_synth_keep_tokens");
}

int nt_synth_runs_mask_host(uint8_t *out, int64_t rows, int64_t vocab, uint64_t root, const char *label,
                            size_t label_len, int32_t mean_kept, int32_t mean_gap) {
    if (!out || rows < 0 || vocab < 1 || mean_kept < 1 || mean_gap < 1)
        return fail(NT_E_ARG, "nt_synth_runs_mask_host: invalid arguments");
    NtRng r;
    if (nt_rng_derive(&r, root, label, label_len) != 0) return fail(NT_E_ARG, "nt_synth_runs_mask_host: bad label");
    for (int64_t row = 0; row < rows; row++) {
        uint8_t *m = out + row * vocab;
        // A gap of random phase first, then alternating kept / excluded runs.
        int64_t v = -int64_t(nt_rng_next_u64(&r) % uint64_t(2 * mean_gap - 1));
        bool kept = false;
        int64_t nkept = 0;
        while (v < vocab) {
            const int32_t mean = kept ? mean_kept : mean_gap;
            int64_t len = 1 + int64_t(nt_rng_next_u64(&r) % uint64_t(2 * mean - 1));
            if (v < 0) len = (len + v > 0) ? len : 1 - v;  // the initial phase ends at or after 0
            for (int64_t k = (v < 0 ? 0 : v); k < v + len && k < vocab; k++) {
                m[k] = kept ? 1 : 0;
                nkept += kept ? 1 : 0;
            }
            v += len;
            kept = !kept;
        }
        if (nkept == 0) m[nt_rng_next_u64(&r) % uint64_t(vocab)] = 1;
    }
    return 0;
}

}  // extern "C"
