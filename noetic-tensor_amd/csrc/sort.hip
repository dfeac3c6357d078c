// Descending sort along the middle of a contiguous f32 [outer, n, inner] of a Device::Hip tensor
// (GpuBackend::sort_desc, src/tensor/gpu/mod.rs:186-191): the values and their I32 source
// positions, in CpuRef's order (src/tensor/kernels.rs:374-413, `sort_order`): every NaN above
// +inf and equal to every other NaN, otherwise total_cmp (+0 above -0), stable (ties keep
// ascending source position). The CUDA backend sorts lanes of up to 4096 on the device and sends
// longer ones through the host (cuda/backend.rs:919-937); here every lane length stays on the
// device.
//
// Each element becomes one 64-bit key, (order key << 32) | ~position, so that a plain descending
// comparison of keys is CpuRef's order with ties broken by position, and no two keys are equal.
// A lane of up to kSortCap elements is sorted by one workgroup (bitonic, the keys in registers,
// LDS only for exchanges between waves). A longer lane is
// cut into kSortCap-long runs, each sorted that way into a scratch buffer, and the runs are
// merged pairwise (merge path: each workgroup stages the two input windows that feed its tile of
// outputs into LDS and merges them there) until one run remains. The last step writes each position's value, decoded from its key (a NaN is read back
// from its source to keep the payload), and its index.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <string>

#include "../../include/noetic_hip.h"
#include "../../include/noetic_ops.h"
#include "nt_internal.hpp"

namespace nt {
namespace {

constexpr int kSortThreads = 1024;
constexpr int kSortCap = 8192;   // elements one workgroup sorts in LDS (64 KB of keys)
constexpr int kMergeThreads = 256;
constexpr int kMergeItems = 8;   // outputs per thread of a merge pass
constexpr int kMergeTile = kMergeThreads * kMergeItems;  // outputs per workgroup (divides 2 kSortCap)
constexpr int kWaveSize = 64;

__device__ __forceinline__ uint64_t sort_key(float v, uint32_t pos) {
    uint32_t k;
    if (v != v) {
        k = 0xffffffffu;  // every NaN, whatever its sign and payload, above +inf
    } else {
        const uint32_t b = __float_as_uint(v);
        k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);  // total_cmp's order as an unsigned key
    }
    return (uint64_t(k) << 32) | uint64_t(~pos);
}

__device__ __forceinline__ uint32_t key_pos(uint64_t c) { return ~uint32_t(c); }

// The element a key came from: the order key is a bijection of the value's bits except for NaN
// (every NaN has one key), so only a NaN is read back from x to keep its payload.
__device__ __forceinline__ float key_value(uint64_t c, const float *x, int64_t at_src) {
    const uint32_t k = uint32_t(c >> 32);
    if (k == 0xffffffffu) return x[at_src];
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

struct SortP {
    const float *x;
    float *vals;
    int32_t *idx;
    uint64_t *runs;   // [lanes][n] sorted runs (multi-run lanes)
    int64_t outer, n, inner;
    int32_t chunks;   // runs per lane
    int32_t pw;       // power of two >= the longest run (<= kSortCap)
};

// Sort run `chunk` of lane `lane`; a lane of one run is written out directly. Thread tid holds
// positions tid + 1024 q (q < 8) in registers through the whole bitonic network, so a stage's
// partner t ^ j is in the same thread when j >= 1024 (a register swap), in the same wave when
// j < 64 (a lane shuffle), and only for 64 <= j < 1024 in another wave (an exchange through LDS
// between two barriers): 22 of the 91 stages of 8192 keys touch LDS.
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int j) {
    const uint32_t lo = uint32_t(v), hi = uint32_t(v >> 32);
    return (uint64_t(uint32_t(__shfl_xor(int(hi), j))) << 32) | uint32_t(__shfl_xor(int(lo), j));
}

// The value position t keeps at stage (k, j) given its partner's: the lower position of a pair
// takes the larger key in a descending block ((t & k) == 0), the smaller in an ascending one.
__device__ __forceinline__ uint64_t cmp_keep(uint64_t mine, uint64_t other, int t, int j, int k) {
    const bool lower = (t & j) == 0;
    const bool desc = (t & k) == 0;
    const bool take_max = lower == desc;
    const bool mine_bigger = mine > other;
    return (take_max == mine_bigger) ? mine : other;
}

__global__ __launch_bounds__(kSortThreads) void k_sort_runs(SortP p) {
    __shared__ uint64_t s[kSortCap];
    constexpr int Q = kSortCap / kSortThreads;  // keys per thread
    const int64_t lane = blockIdx.x / p.chunks;
    const int chunk = int(blockIdx.x - lane * p.chunks);
    const int64_t o = lane / p.inner, i = lane - o * p.inner;
    const int64_t beg = int64_t(chunk) * kSortCap;
    const int len = int(std::min<int64_t>(kSortCap, p.n - beg));
    const int P = p.pw;
    const int tid = threadIdx.x;
    uint64_t v[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int t = tid + kSortThreads * q;
        uint64_t c = 0;  // padding: below every real key (the smallest real order key is 0x007fffff)
        if (t < len) c = sort_key(p.x[(o * p.n + beg + t) * p.inner + i], uint32_t(beg + t));
        v[q] = c;
    }
    // Positions at or past P only meet each other (t ^ j >= P for t >= P, j < P): zeros stay there.
    for (int k = 2; k <= P; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            if (j >= kSortThreads) {
                const int jq = j / kSortThreads;
#pragma unroll
                for (int q = 0; q < Q; q++) {
                    if (q & jq) continue;
                    const int t = tid + kSortThreads * q;
                    const uint64_t a = v[q], b = v[q | jq];
                    v[q] = cmp_keep(a, b, t, j, k);
                    v[q | jq] = cmp_keep(b, a, t + j, j, k);
                }
            } else if (j >= kWaveSize) {
#pragma unroll
                for (int q = 0; q < Q; q++) s[tid + kSortThreads * q] = v[q];
                __syncthreads();
#pragma unroll
                for (int q = 0; q < Q; q++) {
                    const int t = tid + kSortThreads * q;
                    v[q] = cmp_keep(v[q], s[t ^ j], t, j, k);
                }
                __syncthreads();
            } else {
#pragma unroll
                for (int q = 0; q < Q; q++) {
                    const int t = tid + kSortThreads * q;
                    v[q] = cmp_keep(v[q], shfl_xor_u64(v[q], j), t, j, k);
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int t = tid + kSortThreads * q;
        if (t >= len) continue;
        const uint64_t c = v[q];
        if (p.chunks == 1) {
            const uint32_t src = key_pos(c);
            const int64_t at = (o * p.n + t) * p.inner + i;
            p.vals[at] = key_value(c, p.x, (o * p.n + src) * p.inner + i);
            p.idx[at] = int32_t(src);
        } else {
            p.runs[lane * p.n + beg + t] = c;
        }
    }
}

// How many of the first d outputs of merging descending runs A (la keys) and B (lb keys) come
// from A (the merge path's co-rank; keys are distinct, so there are no ties).
__device__ __forceinline__ int64_t co_rank(const uint64_t *A, int64_t la, const uint64_t *B, int64_t lb, int64_t d) {
    int64_t lo = std::max<int64_t>(0, d - lb), hi = std::min<int64_t>(d, la);
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (A[mid] > B[d - mid - 1]) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// One merge pass: in every lane, runs [base, base + w) and [base + w, base + 2w) (clipped to n)
// into one run of `dst`. A workgroup makes kMergeTile consecutive outputs (kMergeTile divides 2w,
// so they come from one pair of runs): two co-ranks in global memory bound the A and B windows
// that feed them, both windows are staged into LDS with coalesced loads, each thread merges its
// kMergeItems outputs from LDS (its own co-rank by a search in LDS), and the tile is written back
// coalesced. If LAST, the outputs are the values and positions instead of keys.
template <bool LAST>
__global__ __launch_bounds__(kMergeThreads) void k_merge(SortP p, const uint64_t *src, uint64_t *dst, int64_t w,
                                                         int64_t tiles_per_lane) {
    __shared__ uint64_t sa[kMergeTile], sb[kMergeTile], so[kMergeTile];
    __shared__ int64_t cr[2];
    const int tid = threadIdx.x;
    const int64_t lane = blockIdx.x / tiles_per_lane;
    const int64_t n = p.n;
    const int64_t o0 = (blockIdx.x - lane * tiles_per_lane) * kMergeTile;
    const int64_t o1 = std::min<int64_t>(n, o0 + kMergeTile);
    const int64_t base = o0 / (2 * w) * (2 * w);
    const int64_t la = std::min<int64_t>(w, n - base);
    const int64_t lb = std::max<int64_t>(0, std::min<int64_t>(w, n - base - la));
    const uint64_t *A = src + lane * n + base;
    const uint64_t *B = A + la;
    const int64_t d0 = o0 - base, d1 = o1 - base;
    if (tid < 2) cr[tid] = co_rank(A, la, B, lb, tid == 0 ? d0 : d1);
    __syncthreads();
    const int64_t a0 = cr[0], b0 = d0 - cr[0];
    const int na = int(cr[1] - cr[0]), nb = int((d1 - cr[1]) - b0);
    for (int e = tid; e < na; e += kMergeThreads) sa[e] = A[a0 + e];
    for (int e = tid; e < nb; e += kMergeThreads) sb[e] = B[b0 + e];
    __syncthreads();
    const int dl = tid * kMergeItems;
    const int total = na + nb;
    if (dl < total) {
        int lo = std::max(0, dl - nb), hi = std::min(dl, na);
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (sa[mid] > sb[dl - mid - 1]) lo = mid + 1;
            else hi = mid;
        }
        int ia = lo, ib = dl - lo;
        const int end = std::min(kMergeItems, total - dl);
        for (int q = 0; q < end; q++) {
            const bool from_a = ib >= nb || (ia < na && sa[ia] > sb[ib]);
            so[dl + q] = from_a ? sa[ia++] : sb[ib++];
        }
    }
    __syncthreads();
    const int64_t o = lane / p.inner, i = lane - o * p.inner;
    for (int e = tid; e < total; e += kMergeThreads) {
        const uint64_t c = so[e];
        if constexpr (LAST) {
            const uint32_t s = key_pos(c);
            const int64_t at = (o * n + o0 + e) * p.inner + i;
            p.vals[at] = key_value(c, p.x, (o * n + s) * p.inner + i);
            p.idx[at] = int32_t(s);
        } else {
            dst[lane * n + o0 + e] = c;
        }
    }
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" {

int nt_hip_sort_desc(const float *x, int64_t outer, int64_t n, int64_t inner, float *vals, int32_t *idx) {
    if (outer < 0 || n < 0 || inner < 0) return fail(NT_E_ARG, "sort_desc: negative lanes");
    if (n > int64_t(0x7fffffff)) return fail(NT_E_ARG, "sort_desc: a lane longer than 2^31 - 1 (I32 positions)");
    const int64_t lanes = outer * inner;
    if (lanes == 0 || n == 0) return 0;
    if (!x || !vals || !idx) return fail(NT_E_ARG, "sort_desc: null buffer");
    SortP p{};
    p.x = x;
    p.vals = vals;
    p.idx = idx;
    p.outer = outer;
    p.n = n;
    p.inner = inner;
    const int64_t chunks = (n + kSortCap - 1) / kSortCap;
    if (lanes * chunks > int64_t(0x7fffffff)) return fail(NT_E_ARG, "sort_desc: too many lanes");
    p.chunks = int32_t(chunks);
    int pw = 1;
    while (pw < std::min<int64_t>(n, kSortCap)) pw <<= 1;
    p.pw = pw;
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    hipStream_t st = ctx().stream;
    if (chunks == 1) {
        hipLaunchKernelGGL(k_sort_runs, dim3(unsigned(lanes)), dim3(kSortThreads), 0, st, p);
        return launched("k_sort_runs");
    }
    void *buf[2] = {nullptr, nullptr};
    const size_t bytes = size_t(lanes) * size_t(n) * sizeof(uint64_t);
    if (int rc = scratch_alloc(bytes, &buf[0])) return rc;
    if (int rc = scratch_alloc(bytes, &buf[1])) {
        scratch_release(buf[0]);
        return rc;
    }
    p.runs = static_cast<uint64_t *>(buf[0]);
    hipLaunchKernelGGL(k_sort_runs, dim3(unsigned(lanes * chunks)), dim3(kSortThreads), 0, st, p);
    int rc = launched("k_sort_runs");
    const int64_t tiles = (n + kMergeTile - 1) / kMergeTile;
    const int64_t blocks = lanes * tiles;
    if (blocks > int64_t(0x7fffffff)) {
        scratch_release(buf[0]);
        scratch_release(buf[1]);
        return fail(NT_E_ARG, "sort_desc: too many merge tiles");
    }
    int cur = 0;
    for (int64_t w = kSortCap; !rc && w < n; w *= 2) {
        const uint64_t *src = static_cast<const uint64_t *>(buf[cur]);
        uint64_t *dst = static_cast<uint64_t *>(buf[cur ^ 1]);
        if (2 * w >= n) {
            hipLaunchKernelGGL((k_merge<true>), dim3(unsigned(blocks)), dim3(kMergeThreads), 0, st, p, src, dst, w,
                               tiles);
        } else {
            hipLaunchKernelGGL((k_merge<false>), dim3(unsigned(blocks)), dim3(kMergeThreads), 0, st, p, src, dst, w,
                               tiles);
        }
        rc = launched("k_merge");
        cur ^= 1;
    }
    const int r0 = scratch_release(buf[0]);
    const int r1 = scratch_release(buf[1]);
    return rc ? rc : (r0 ? r0 : r1);
}

}  // extern "C"
