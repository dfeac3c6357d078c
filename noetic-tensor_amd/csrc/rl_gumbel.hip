// The reference's Gumbel-max sampler on the device: sample_categorical (src/nn/rl.rs:488-529)
// for a Hip tensor, with the reference's contract kept whole: one u64 of the caller's ChaCha20
// stream per logit in row-major order, the draw u = ((k >> 11) + 0.5) / 2^53, the f64 noise
// -ln(-ln u) rounded once to f32, the f32 sum z + g and the first maximum of each row.
//
// The reference draws the noise on the host and uploads it (rows x V f64 values turned into
// f32, then an add kernel and an argmax kernel). Here the noise is generated where it is used:
// ChaCha20 is a counter-mode stream, so word w of the keystream is word w % 16 of block w / 16
// and every element's u64 is computed from the stream's key and starting word position alone.
// One workgroup takes one row; each thread takes whole keystream blocks (8 u64 = 8 elements
// when the stream's position is even) in index order, keeps its first maximum, and the
// workgroup combines the (value, index) pairs with "greater value, else smaller index", which
// is associative, so the result is the sequential first maximum whatever the timing.
//
// A block whose eight logits are all excluded (-inf) is skipped without generating it: such an
// element can never be the maximum of an accepted row (a row with no other candidate is
// refused), so skipping changes no token.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <string>

#include "../../include/noetic_hip.h"
#include "nt_chacha.hpp"
#include "nt_internal.hpp"

namespace nt {
namespace {

constexpr int kGumbelMaxThreads = 512;

struct GumbelP {
    const void *logits;
    const void *mask;
    int64_t V, ld, mask_ld;
    float tau;
    int tau_one;
    ChachaKey key;
    uint64_t h;  // pair index of the stream's u64 0: its low word is keystream word 2 h + ODD
    int32_t *ids;
    uint8_t *status;
};

// z_v = tempered_logits (rl.rs:475-486) in f32: x / tau (skipped at tau == 1), then the
// additive f32 mask, or -inf at a token a u8 keep-mask excludes.
template <int DT, int MK>
__device__ __forceinline__ float tempered_at(const GumbelP &p, int64_t row, int64_t v) {
    float x;
    if constexpr (DT == NT_F32) {
        x = static_cast<const float *>(p.logits)[row * p.ld + v];
    } else {
        x = __uint_as_float(uint32_t(static_cast<const uint16_t *>(p.logits)[row * p.ld + v]) << 16);
    }
    if (!p.tau_one) x = x / p.tau;
    if constexpr (MK == NT_MASK_U8) {
        if (static_cast<const uint8_t *>(p.mask)[row * p.mask_ld + v] == 0) x = -INFINITY;
    } else if constexpr (MK == NT_MASK_F32) {
        x = x + static_cast<const float *>(p.mask)[row * p.mask_ld + v];
    }
    return x;
}

// f32(-ln(-ln u)) of one u64 of the stream, u = ((k >> 11) + 0.5) / 2^53 (rl.rs:490-498): the
// f64 add rounds to nearest even as the host's does, the scale by 2^-53 is exact.
__device__ __forceinline__ float gumbel_f32(uint32_t lo, uint32_t hi) {
    const uint64_t k = ((uint64_t(hi) << 32) | lo) >> 11;
    const double u = (double(k) + 0.5) * 0x1p-53;
    return float(-log(-log(u)));
}

// (value, index) pair order of the first maximum: b replaces a when greater, or equal with a
// smaller index. Candidates are never NaN (a NaN refuses the row).
__device__ __forceinline__ void best_merge(float &a, int &ia, float b, int ib) {
    if (b > a || (b == a && ib < ia)) {
        a = b;
        ia = ib;
    }
}

template <int DT, int MK, bool ODD, bool GREEDY>
__global__ __launch_bounds__(kGumbelMaxThreads) void k_sample_gumbel(GumbelP p) {
    __shared__ float sbest[kGumbelMaxThreads / 64];
    __shared__ int sidx[kGumbelMaxThreads / 64];
    __shared__ int sflags[kGumbelMaxThreads / 64];
    const int64_t row = blockIdx.x;
    const int64_t V = p.V;
    // Pair q = h + row V + v holds element v's u64; block q >> 3, pair q & 7 of it.
    const uint64_t q0 = p.h + uint64_t(row) * uint64_t(V);
    const uint64_t b0 = q0 >> 3, b1 = (q0 + uint64_t(V) - 1) >> 3;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    int flags = 0;  // bit 0: a candidate (z > -inf); bit 1: a NaN
    for (uint64_t b = b0 + threadIdx.x; b <= b1; b += blockDim.x) {
        const int64_t v0 = int64_t(8 * b - q0);  // element of pair 0 of block b (may be < 0)
        float z[8];
        bool any = false;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int64_t v = v0 + j;
            z[j] = (v >= 0 && v < V) ? tempered_at<DT, MK>(p, row, v) : -INFINITY;
            if (z[j] != z[j]) flags |= 2;
            any |= z[j] > -INFINITY;
        }
        if (!any) continue;
        flags |= 1;
        if constexpr (GREEDY) {
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (z[j] > best) {  // strictly greater: the first maximum of this thread's elements
                    best = z[j];
                    bidx = int(v0 + j);
                }
        } else {
            uint32_t w[16];
            chacha_block_dev(p.key, b, w);
            uint32_t next0 = 0;  // word 0 of block b + 1: the high word of pair 7 when ODD
            if constexpr (ODD) {
                if (z[7] > -INFINITY) {
                    uint32_t w2[16];
                    chacha_block_dev(p.key, b + 1, w2);
                    next0 = w2[0];
                }
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                if (z[j] > -INFINITY) {
                    const uint32_t lo = ODD ? w[2 * j + 1] : w[2 * j];
                    const uint32_t hi = ODD ? (j == 7 ? next0 : w[2 * j + 2]) : w[2 * j + 1];
                    const float s = z[j] + gumbel_f32(lo, hi);
                    if (s > best) {
                        best = s;
                        bidx = int(v0 + j);
                    }
                }
            }
        }
    }
    // The workgroup's first maximum: a fixed butterfly inside each wave, then the waves in order.
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ob = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bidx, o, 64);
        best_merge(best, bidx, ob, oi);
        flags |= __shfl_xor(flags, o, 64);
    }
    const int wave = threadIdx.x / 64, nw = blockDim.x / 64;
    if ((threadIdx.x & 63) == 0) {
        sbest[wave] = best;
        sidx[wave] = bidx;
        sflags[wave] = flags;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    float rb = sbest[0];
    int ri = sidx[0], rf = sflags[0];
    for (int i = 1; i < nw; i++) {
        best_merge(rb, ri, sbest[i], sidx[i]);
        rf |= sflags[i];
    }
    // The reference refuses a row whose maximum is NaN (any NaN: max_dim propagates it) or -inf
    // (rl.rs:515-519).
    if (rf & 2) {
        p.ids[row] = -1;
        p.status[row] = NT_ROW_NAN;
    } else if (!(rf & 1)) {
        p.ids[row] = -1;
        p.status[row] = NT_ROW_NO_TOKEN;
    } else {
        p.ids[row] = ri;
        p.status[row] = NT_ROW_OK;
    }
}

template <int DT, int MK, bool ODD, bool GREEDY>
void launch_gumbel(const GumbelP &p, int64_t rows, int threads, hipStream_t s) {
    hipLaunchKernelGGL((k_sample_gumbel<DT, MK, ODD, GREEDY>), dim3(unsigned(rows)), dim3(threads), 0, s, p);
}

template <int DT, int MK>
void pick_gumbel(bool odd, bool greedy, const GumbelP &p, int64_t rows, int threads, hipStream_t s) {
    if (greedy) launch_gumbel<DT, MK, false, true>(p, rows, threads, s);
    else if (odd) launch_gumbel<DT, MK, true, false>(p, rows, threads, s);
    else launch_gumbel<DT, MK, false, false>(p, rows, threads, s);
}

template <int DT>
void pick_gumbel_mk(int mk, bool odd, bool greedy, const GumbelP &p, int64_t rows, int threads, hipStream_t s) {
    if (mk == NT_MASK_U8) pick_gumbel<DT, NT_MASK_U8>(odd, greedy, p, rows, threads, s);
    else if (mk == NT_MASK_F32) pick_gumbel<DT, NT_MASK_F32>(odd, greedy, p, rows, threads, s);
    else pick_gumbel<DT, NT_MASK_NONE>(odd, greedy, p, rows, threads, s);
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" int nt_hip_rl_sample_gumbel(const NtRlGumbelArgs *a) {
    if (!a) return fail(NT_E_ARG, "nt_hip_rl_sample_gumbel: null args");
    const int64_t rows = a->rows, V = a->vocab;
    if (rows < 0 || V < 1 || a->ld < V || (a->dtype != NT_F32 && a->dtype != NT_BF16) ||
        a->mask_kind < NT_MASK_NONE || a->mask_kind > NT_MASK_F32 ||
        ((a->mask_kind == NT_MASK_NONE) != (a->mask == nullptr)) || (a->mask_ld != 0 && a->mask_ld < V) ||
        rows > 0x7fffffffLL || V > 0x7fffffffLL || a->word < 0 || a->word > 15)
        return fail(NT_E_ARG, "nt_hip_rl_sample_gumbel: invalid rows " + std::to_string(rows) + ", V " +
                                  std::to_string(V) + ", ld " + std::to_string(a->ld) + ", dtype, mask or word " +
                                  std::to_string(a->word));
    if (!(a->temperature >= 0.0) || !std::isfinite(a->temperature))
        return fail(NT_E_ARG, "sample_categorical: temperature " + std::to_string(a->temperature) + " (must be ≥ 0)");
    if (!a->logits || !a->ids || !a->status)
        return fail(NT_E_ARG, "nt_hip_rl_sample_gumbel: null logits, ids or status");
    // The stream's block counter is 64-bit: the draws of this call must not wrap it.
    const uint64_t words = 2 * uint64_t(rows) * uint64_t(V);
    if (a->block > (~uint64_t(0) >> 5) || words > (uint64_t(1) << 62))
        return fail(NT_E_ARG, "nt_hip_rl_sample_gumbel: stream position or draw count out of range");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (rows == 0) return 0;
    const bool greedy = a->temperature == 0.0;
    GumbelP p;
    p.logits = a->logits;
    p.mask = a->mask;
    p.V = V;
    p.ld = a->ld;
    p.mask_ld = a->mask_ld;
    const double T = greedy ? 1.0 : a->temperature;
    p.tau = float(T);  // the reference divides by `temperature as f32` (float.rs:494-499)
    p.tau_one = T == 1.0;
    for (int i = 0; i < 8; i++) p.key.k[i] = a->key[i];
    const uint64_t w0 = 16 * a->block + uint64_t(a->word);
    p.h = w0 >> 1;
    const bool odd = (w0 & 1) != 0;
    p.ids = a->ids;
    p.status = a->status;
    // Threads per row: one per keystream block of the row, in whole waves, at most 512.
    const int64_t nblk = V / 8 + 2;
    int threads = int(((nblk + 63) / 64) * 64);
    threads = threads > kGumbelMaxThreads ? kGumbelMaxThreads : threads;
    hipStream_t s = ctx().stream;
    if (a->dtype == NT_F32) pick_gumbel_mk<NT_F32>(a->mask_kind, odd, greedy, p, rows, threads, s);
    else pick_gumbel_mk<NT_BF16>(a->mask_kind, odd, greedy, p, rows, threads, s);
    return launched("nt_hip_rl_sample_gumbel");
}
