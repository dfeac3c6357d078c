// General device ops of a Device::Hip tensor: the GpuBackend methods the nn::rl chain uses around
// the fused entry points (src/tensor/gpu/mod.rs:137-207). Every op is HBM-bound integer or
// float work with no reuse, so the kernels are grid-stride loops over the output with the
// views' index arithmetic in registers; the only ordering that matters is the reference's
// (CpuRef's sum order, the first maximum), which the reductions keep exactly.
//
// Views are simplified on the host before launch: dimensions of size 1 are dropped and
// neighbouring dimensions that form one stride run in every operand are merged, so a contiguous
// view is rank 1 and a row broadcast ([rows, V] against [1, V]) is rank 2. The kernels are
// instantiated per merged rank, so the coordinate loop unrolls.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <string>

#include "../../include/noetic_hip.h"
#include "../../include/noetic_ops.h"
#include "nt_internal.hpp"

namespace nt {
namespace {

constexpr int kWave = 64;  // CDNA wavefront
constexpr int kOpsThreads = 256;
constexpr int64_t kMaxBlocks = 16384;  // grid-stride beyond this (64 blocks per CU)

// A view after simplification: R dimensions, element strides per operand.
struct View {
    int64_t shape[NT_MAX_RANK];
    int64_t st[NT_MAX_RANK];
    int64_t off;
};

template <int R>
__device__ __forceinline__ int64_t at(int64_t i, const View &v) {
    int64_t o = v.off;
    if constexpr (R == 1) {
        o += i * v.st[0];
    } else if (i <= int64_t(0xffffffff)) {
        // coordinates by 32-bit division (a third of the 64-bit sequence's instructions)
        uint32_t u = uint32_t(i);
#pragma unroll
        for (int d = R - 1; d >= 1; d--) {
            const uint32_t s = uint32_t(v.shape[d]);
            const uint32_t q = u / s;
            o += int64_t(u - q * s) * v.st[d];
            u = q;
        }
        o += int64_t(u) * v.st[0];
    } else {
#pragma unroll
        for (int d = R - 1; d >= 1; d--) {
            const int64_t s = v.shape[d];
            const int64_t q = i / s;
            o += (i - q * s) * v.st[d];
            i = q;
        }
        o += i * v.st[0];
    }
    return o;
}

// Host: simplify up to three views of one shape together (size-1 dimensions dropped, mergeable
// neighbours merged). Returns the merged rank (at least 1).
int simplify(const NtLayout *const *ls, int nl, View *out) {
    const int rank = ls[0]->rank;
    int64_t shape[NT_MAX_RANK];
    int64_t st[3][NT_MAX_RANK];
    int r = 0;
    for (int d = 0; d < rank; d++) {
        if (ls[0]->shape[d] == 1) continue;
        shape[r] = ls[0]->shape[d];
        for (int k = 0; k < nl; k++) st[k][r] = ls[k]->strides[d];
        r++;
    }
    if (r == 0) {  // one element
        shape[0] = 1;
        for (int k = 0; k < nl; k++) st[k][0] = 0;
        r = 1;
    }
    // merge d into d - 1 when, in every operand, stride[d - 1] == stride[d] * shape[d]
    int m = 0;
    for (int d = 1; d < r; d++) {
        bool ok = true;
        for (int k = 0; k < nl; k++) ok = ok && st[k][m] == st[k][d] * shape[d];
        if (ok) {
            shape[m] *= shape[d];
            for (int k = 0; k < nl; k++) st[k][m] = st[k][d];
        } else {
            m++;
            shape[m] = shape[d];
            for (int k = 0; k < nl; k++) st[k][m] = st[k][d];
        }
    }
    const int R = m + 1;
    for (int k = 0; k < nl; k++) {
        for (int d = 0; d < R; d++) {
            out[k].shape[d] = shape[d];
            out[k].st[d] = st[k][d];
        }
        out[k].off = ls[k]->offset;
    }
    return R;
}

int64_t numel_of(const NtLayout *l) {
    int64_t n = 1;
    for (int d = 0; d < l->rank; d++) n *= l->shape[d];
    return n;
}

int check_layout(const NtLayout *l, const char *what) {
    if (!l) return fail(NT_E_ARG, std::string(what) + ": null layout");
    if (l->rank < 0 || l->rank > NT_MAX_RANK)
        return fail(NT_E_ARG, std::string(what) + ": rank " + std::to_string(l->rank) + " (at most 8)");
    if (l->offset < 0) return fail(NT_E_ARG, std::string(what) + ": negative offset");
    for (int d = 0; d < l->rank; d++)
        if (l->shape[d] < 0 || l->strides[d] < 0)
            return fail(NT_E_ARG, std::string(what) + ": negative shape or stride");
    return 0;
}

bool same_shape(const NtLayout *a, const NtLayout *b) {
    if (a->rank != b->rank) return false;
    for (int d = 0; d < a->rank; d++)
        if (a->shape[d] != b->shape[d]) return false;
    return true;
}

unsigned blocks_for(int64_t n) {
    const int64_t b = (n + kOpsThreads - 1) / kOpsThreads;
    return unsigned(b < 1 ? 1 : (b > kMaxBlocks ? kMaxBlocks : b));
}

#define GRID_STRIDE(i, n) \
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < (n); i += int64_t(gridDim.x) * blockDim.x)

// Dispatch a kernel template on the merged rank R (1..8).
#define RANK_SWITCH(R, CALL)            \
    switch (R) {                        \
        case 1: { constexpr int RR = 1; CALL; } break; \
        case 2: { constexpr int RR = 2; CALL; } break; \
        case 3: { constexpr int RR = 3; CALL; } break; \
        case 4: { constexpr int RR = 4; CALL; } break; \
        case 5: { constexpr int RR = 5; CALL; } break; \
        case 6: { constexpr int RR = 6; CALL; } break; \
        case 7: { constexpr int RR = 7; CALL; } break; \
        default: { constexpr int RR = 8; CALL; } break; \
    }

// ------------------------------------------------------------------ copies and writes

template <typename T, int R>
__global__ __launch_bounds__(kOpsThreads) void k_copy(const T *__restrict__ x, View xv, T *__restrict__ y, View yv,
                                                      int64_t n) {
    GRID_STRIDE(i, n) { y[at<R>(i, yv)] = x[at<R>(i, xv)]; }
}

// A transposed view into a contiguous output, out[a, b] = x[off + a + b ld]: 64 x 64 tiles
// through LDS, read along a and written along b, so both sides are coalesced (the element loop
// above would read with stride ld).
template <typename T>
__global__ __launch_bounds__(kOpsThreads) void k_transpose(const T *__restrict__ x, int64_t off, int64_t ld,
                                                           T *__restrict__ y, int64_t A, int64_t B) {
    __shared__ T tile[64][65];
    const int64_t ta_n = (A + 63) / 64, tiles = ta_n * ((B + 63) / 64);
    const int c = threadIdx.x & 63, r0 = threadIdx.x >> 6;
    for (int64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
        const int64_t a0 = (t % ta_n) * 64, b0 = (t / ta_n) * 64;
        for (int k = r0; k < 64; k += kOpsThreads / 64)
            if (a0 + c < A && b0 + k < B) tile[k][c] = x[off + (b0 + k) * ld + a0 + c];
        __syncthreads();
        for (int k = r0; k < 64; k += kOpsThreads / 64)
            if (a0 + k < A && b0 + c < B) y[(a0 + k) * B + b0 + c] = tile[c][k];
        __syncthreads();
    }
}

template <typename T>
int launch_copy(const void *x, const NtLayout *xl, void *y, const NtLayout *yl) {
    const NtLayout *ls[2] = {xl, yl};
    View v[2];
    const int R = simplify(ls, 2, v);
    const int64_t n = numel_of(xl);
    if (n == 0) return 0;
    hipStream_t s = ctx().stream;
    if (R == 2 && v[1].off == 0 && v[1].st[1] == 1 && v[1].st[0] == v[1].shape[1] && v[0].st[0] == 1 &&
        v[0].st[1] > 1) {
        const int64_t A = v[0].shape[0], B = v[0].shape[1];
        const int64_t tiles = ((A + 63) / 64) * ((B + 63) / 64);
        hipLaunchKernelGGL((k_transpose<T>), dim3(unsigned(tiles < kMaxBlocks ? tiles : kMaxBlocks)), dim3(kOpsThreads),
                           0, s, static_cast<const T *>(x), v[0].off, v[0].st[1], static_cast<T *>(y), A, B);
        return launched("copy (transpose)");
    }
    RANK_SWITCH(R, hipLaunchKernelGGL((k_copy<T, RR>), dim3(blocks_for(n)), dim3(kOpsThreads), 0, s,
                                      static_cast<const T *>(x), v[0], static_cast<T *>(y), v[1], n));
    return launched("copy");
}

int copy_any(const void *x, const NtLayout *xl, void *y, const NtLayout *yl, int eb) {
    switch (eb) {
        case 1: return launch_copy<uint8_t>(x, xl, y, yl);
        case 2: return launch_copy<uint16_t>(x, xl, y, yl);
        case 4: return launch_copy<uint32_t>(x, xl, y, yl);
        case 8: return launch_copy<uint64_t>(x, xl, y, yl);
        default: return fail(NT_E_ARG, "copy: element size " + std::to_string(eb) + " (1, 2, 4 or 8)");
    }
}

NtLayout contiguous_like(const NtLayout *l) {
    NtLayout c{};
    c.rank = l->rank;
    c.offset = 0;
    int64_t s = 1;
    for (int d = l->rank - 1; d >= 0; d--) {
        c.shape[d] = l->shape[d];
        c.strides[d] = s;
        s *= l->shape[d];
    }
    return c;
}

// ------------------------------------------------------------------ casts

// f32 -> bf16 bits, round to nearest even; a NaN stays a quiet NaN (half.rs:14-22).
__device__ __forceinline__ uint16_t to_bf16(float x) {
    const uint32_t b = __float_as_uint(x);
    if (x != x) return uint16_t((b >> 16) | 0x0040u);
    return uint16_t((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float from_bf16(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// f32 -> IEEE binary16 bits, round to nearest even, subnormals, overflow to inf, NaN kept quiet
// with its top payload bits (half.rs:30-60), written from the format's definition.
__device__ __forceinline__ uint16_t to_f16(float x) {
    const uint32_t b = __float_as_uint(x);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const int ex = int((b >> 23) & 0xffu);
    const uint32_t man = b & 0x7fffffu;
    if (ex == 0xff) return uint16_t(sign | 0x7c00u | (man ? (0x0200u | (man >> 13)) : 0u));
    const int e = ex - 112;  // rebias 127 -> 15
    if (e >= 31) return uint16_t(sign | 0x7c00u);
    uint32_t q, rem, half;
    if (e <= 0) {
        if (e < -10) return uint16_t(sign);
        const uint32_t m = man | 0x800000u;  // the implicit bit
        const uint32_t sh = uint32_t(14 - e);  // 14 .. 24
        q = m >> sh;
        rem = m & ((1u << sh) - 1u);
        half = 1u << (sh - 1);
    } else {
        q = (uint32_t(e) << 10) | (man >> 13);
        rem = man & 0x1fffu;
        half = 0x1000u;
    }
    q += (rem > half || (rem == half && (q & 1u))) ? 1u : 0u;  // a carry rounds into the exponent
    return uint16_t(sign | q);
}
__device__ __forceinline__ float from_f16(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1f) return __uint_as_float(sign | 0x7f800000u | (m << 13));
    if (e != 0) return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
    // zero or subnormal: m 2^-24 exactly
    const float v = float(m) * 5.9604644775390625e-08f;
    return sign ? -v : v;
}

template <int FROM, int TO, int R>
__global__ __launch_bounds__(kOpsThreads) void k_cast(const void *__restrict__ xv_, View xv, void *__restrict__ y_,
                                                      int64_t n) {
    GRID_STRIDE(i, n) {
        const int64_t o = at<R>(i, xv);
        float f;
        if constexpr (FROM == NT_DT_F32) f = static_cast<const float *>(xv_)[o];
        else if constexpr (FROM == NT_DT_BF16) f = from_bf16(static_cast<const uint16_t *>(xv_)[o]);
        else if constexpr (FROM == NT_DT_F16) f = from_f16(static_cast<const uint16_t *>(xv_)[o]);
        else f = static_cast<const uint8_t *>(xv_)[o] != 0 ? 1.0f : 0.0f;  // bool
        if constexpr (TO == NT_DT_F32) static_cast<float *>(y_)[i] = f;
        else if constexpr (TO == NT_DT_BF16) static_cast<uint16_t *>(y_)[i] = to_bf16(f);
        else static_cast<uint16_t *>(y_)[i] = to_f16(f);
    }
}

template <int FROM, int TO>
int launch_cast(const void *x, const NtLayout *xl, void *y) {
    const NtLayout *ls[1] = {xl};
    View v[1];
    const int R = simplify(ls, 1, v);
    const int64_t n = numel_of(xl);
    if (n == 0) return 0;
    hipStream_t s = ctx().stream;
    RANK_SWITCH(R, hipLaunchKernelGGL((k_cast<FROM, TO, RR>), dim3(blocks_for(n)), dim3(kOpsThreads), 0, s, x, v[0],
                                      y, n));
    return launched("cast");
}

// ------------------------------------------------------------------ elementwise float ops

// exp, ln and pow rounded to f32 from the f64 library functions: the f64 result is within an
// f64 ulp or so of the exact value, so its rounding to f32 is the nearest f32 unless the exact
// value lies within about 2^-29 f32 ulp of a midpoint.
__device__ __forceinline__ float exp_f(float a) { return float(exp(double(a))); }
__device__ __forceinline__ float log_f(float a) { return float(log(double(a))); }
__device__ __forceinline__ float pow_f(float a, float s) { return float(pow(double(a), double(s))); }
// The correctly rounded f32 quotient and square root: the division operator and sqrtf compile to
// the IEEE sequences (v_div_scale / v_div_fmas / v_div_fixup; v_sqrt_f32 with its residual
// correction). __fsqrt_rn is not used: on this target it is v_sqrt_f32 alone, 1 ulp.
__device__ __forceinline__ float div_f(float a, float b) { return a / b; }
__device__ __forceinline__ float sqrt_f(float a) { return sqrtf(a); }

__device__ __forceinline__ float unary_op(int op, float a, float s) {
    switch (op) {
        case NT_UN_NEG: return -a;
        case NT_UN_EXP: return exp_f(a);
        case NT_UN_LOG: return log_f(a);
        case NT_UN_SQRT: return sqrt_f(a);
        case NT_UN_RECIP: return div_f(1.0f, a);
        case NT_UN_ABS: return fabsf(a);
        // 0 for +-0, 1 for a positive sign bit, -1 otherwise (a NaN by its sign bit): float.rs:537-541
        case NT_UN_SIGN: return a == 0.0f ? 0.0f : (signbit(a) ? -1.0f : 1.0f);
        case NT_UN_SIGMOID: {
            if (a >= 0.0f) return div_f(1.0f, 1.0f + exp_f(-a));
            const float e = exp_f(a);
            return div_f(e, 1.0f + e);
        }
        case NT_UN_ADD_SCALAR: return a + s;
        case NT_UN_SUB_SCALAR: return a - s;
        case NT_UN_MUL_SCALAR: return a * s;
        case NT_UN_DIV_SCALAR: return div_f(a, s);
        default: return pow_f(a, s);
    }
}

template <int R>
__global__ __launch_bounds__(kOpsThreads) void k_unary(int op, float s, const float *__restrict__ x, View xv,
                                                       float *__restrict__ y, int64_t n) {
    GRID_STRIDE(i, n) { y[i] = unary_op(op, x[at<R>(i, xv)], s); }
}

// The contiguous case, 16-byte aligned: four elements per thread through one 16-byte load and
// store (the element loop moves 4 bytes per instruction).
__global__ __launch_bounds__(kOpsThreads) void k_unary_vec(int op, float s, const float *__restrict__ x,
                                                           float *__restrict__ y, int64_t n) {
    const int64_t n4 = n / 4;
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    float4 *y4 = reinterpret_cast<float4 *>(y);
    GRID_STRIDE(i, n4) {
        float4 a = x4[i];
        a.x = unary_op(op, a.x, s);
        a.y = unary_op(op, a.y, s);
        a.z = unary_op(op, a.z, s);
        a.w = unary_op(op, a.w, s);
        y4[i] = a;
    }
    GRID_STRIDE(i, n - 4 * n4) { y[4 * n4 + i] = unary_op(op, x[4 * n4 + i], s); }
}

template <int R>
__global__ __launch_bounds__(kOpsThreads) void k_compare(int op, float s, const float *__restrict__ x, View xv,
                                                         uint8_t *__restrict__ y, int64_t n) {
    GRID_STRIDE(i, n) {
        const float a = x[at<R>(i, xv)];
        bool r;
        switch (op) {
            case NT_CMP_GT: r = a > s; break;
            case NT_CMP_GE: r = a >= s; break;
            case NT_CMP_LT: r = a < s; break;
            case NT_CMP_LE: r = a <= s; break;
            default: r = a == s; break;
        }
        y[i] = r ? 1 : 0;
    }
}

template <int R>
__global__ __launch_bounds__(kOpsThreads) void k_binary(int op, const float *__restrict__ a, View av,
                                                        const float *__restrict__ b, View bv, float *__restrict__ y,
                                                        int64_t n) {
    GRID_STRIDE(i, n) {
        const float p = a[at<R>(i, av)], q = b[at<R>(i, bv)];
        float r;
        switch (op) {
            case NT_BIN_ADD: r = p + q; break;
            case NT_BIN_SUB: r = p - q; break;
            case NT_BIN_MUL: r = p * q; break;
            default: r = div_f(p, q); break;
        }
        y[i] = r;
    }
}

template <int R>
__global__ __launch_bounds__(kOpsThreads) void k_mask_fill(const float *__restrict__ x, View xv,
                                                           const uint8_t *__restrict__ m, View mv, float value,
                                                           float *__restrict__ y, int64_t n) {
    GRID_STRIDE(i, n) { y[i] = m[at<R>(i, mv)] != 0 ? value : x[at<R>(i, xv)]; }
}

// ------------------------------------------------------------------ reductions

// CpuRef's sum of one lane of n contiguous elements (ndarray's unrolled_fold, kernels.rs:120-150):
// eight partial sums p0..p7 over the whole blocks of eight, each folded in order from zero, then
// acc = 0 + (p0 + p4), + (p1 + p5), + (p2 + p6), + (p3 + p7), then the tail in order. Eight
// lanes of a wave take one row, lane p folding p_p (an 8-lane group reads 32 contiguous bytes
// per step); lane 0 of the group combines. Eight rows per wave.
__global__ __launch_bounds__(kOpsThreads) void k_sum_last(const float *__restrict__ x, int64_t outer, int64_t n,
                                                          float *__restrict__ y) {
    const int g = threadIdx.x & 7;
    const int64_t groups = int64_t(gridDim.x) * (blockDim.x / 8);
    for (int64_t row = int64_t(blockIdx.x) * (blockDim.x / 8) + threadIdx.x / 8; row < outer; row += groups) {
        const float *r = x + row * n;
        const int64_t n8 = n - n % 8;
        float p = 0.0f;
        // The fold is one dependent chain per lane, so its loads go out 64 at a time ahead of
        // the adds (the order of the adds is unchanged).
        constexpr int kB = 64;
        int64_t j = g;
        for (; j + 8 * (kB - 1) < n8; j += 8 * kB) {
            float v[kB];
#pragma unroll
            for (int t = 0; t < kB; t++) v[t] = r[j + 8 * t];
#pragma unroll
            for (int t = 0; t < kB; t++) p = p + v[t];
        }
        for (; j < n8; j += 8) p = p + r[j];
        // the group's partials to its lane 0 (widths of 8)
        const float p0 = __shfl(p, 0, 8), p1 = __shfl(p, 1, 8), p2 = __shfl(p, 2, 8), p3 = __shfl(p, 3, 8);
        const float p4 = __shfl(p, 4, 8), p5 = __shfl(p, 5, 8), p6 = __shfl(p, 6, 8), p7 = __shfl(p, 7, 8);
        if (g == 0) {
            float acc = 0.0f;
            acc = acc + (p0 + p4);
            acc = acc + (p1 + p5);
            acc = acc + (p2 + p6);
            acc = acc + (p3 + p7);
            for (int64_t j = n8; j < n; j++) acc = acc + r[j];
            y[row] = acc;
        }
    }
}

// Along any other axis: the n slices added in order from zero (kernels.rs:163-171); one thread
// per output, neighbouring threads on neighbouring inner positions.
__global__ __launch_bounds__(kOpsThreads) void k_sum_mid(const float *__restrict__ x, int64_t outer, int64_t n,
                                                         int64_t inner, float *__restrict__ y) {
    GRID_STRIDE(t, outer * inner) {
        const int64_t o = t / inner, i = t - o * inner;
        const float *p = x + o * n * inner + i;
        float acc = 0.0f;
        for (int64_t k = 0; k < n; k++) acc = acc + p[k * inner];
        y[t] = acc;
    }
}

// The first maximum, NaN-propagating (kernels.rs:184-209): a NaN beats any number and the
// earlier of two NaNs wins; otherwise the larger value wins and the earlier index breaks ties.
// This choice is associative, so any grouping gives the sequential fold's (value, index).
struct Best {
    float v;
    int64_t k;
};
__device__ __forceinline__ Best pick(Best a, Best b) {
    const bool an = a.v != a.v, bn = b.v != b.v;
    if (an || bn) {
        if (an && bn) return a.k <= b.k ? a : b;
        return an ? a : b;
    }
    if (a.v > b.v) return a;
    if (b.v > a.v) return b;
    return a.k <= b.k ? a : b;
}
__device__ __forceinline__ Best shfl_best(Best b, int src_lane_delta) {
    Best o;
    o.v = __shfl_down(b.v, src_lane_delta, kWave);
    o.k = __shfl_down(b.k, src_lane_delta, kWave);
    return o;
}

// One 1024-thread block per lane of the last axis (or per lane of everything, outer = 1): each
// thread picks over its strided subsequence, then the block combines.
constexpr int kBestThreads = 1024;
__global__ __launch_bounds__(kBestThreads) void k_best_last(const float *__restrict__ x, int64_t outer, int64_t n,
                                                            float *__restrict__ val, int32_t *__restrict__ idx) {
    __shared__ Best wb[kBestThreads / kWave];
    for (int64_t row = blockIdx.x; row < outer; row += gridDim.x) {
        const float *r = x + row * n;
        Best b{r[0], 0};
        if (n <= int64_t(0x7fffffff)) {
            // 32-bit positions in the loop (the pick compares indices only on ties)
            float bv = r[0];
            int32_t bk = 0;
            for (int32_t k = int32_t(threadIdx.x); k < int32_t(n); k += kBestThreads) {
                const float e = r[k];
                const bool en = e != e, bn = bv != bv;
                // k > bk always here, so the earlier index wins ties: take e only if it is a NaN
                // over a number, or a larger number
                if (!bn && (en || e > bv)) {
                    bv = e;
                    bk = k;
                }
            }
            b = Best{bv, bk};
        } else {
            for (int64_t k = threadIdx.x; k < n; k += kBestThreads) b = pick(b, Best{r[k], k});
        }
        for (int o = kWave / 2; o > 0; o >>= 1) {
            const Best other = shfl_best(b, o);
            b = pick(b, other);
        }
        if ((threadIdx.x & (kWave - 1)) == 0) wb[threadIdx.x / kWave] = b;
        __syncthreads();
        if (threadIdx.x == 0) {
            Best t = wb[0];
            for (int w = 1; w < kBestThreads / kWave; w++) t = pick(t, wb[w]);
            if (val) val[row] = t.v;
            if (idx) idx[row] = int32_t(t.k);
        }
        __syncthreads();
    }
}

// Along any other axis: one thread per output, the sequential fold.
__global__ __launch_bounds__(kOpsThreads) void k_best_mid(const float *__restrict__ x, int64_t outer, int64_t n,
                                                          int64_t inner, float *__restrict__ val,
                                                          int32_t *__restrict__ idx) {
    GRID_STRIDE(t, outer * inner) {
        const int64_t o = t / inner, i = t - o * inner;
        const float *p = x + o * n * inner + i;
        Best b{p[0], 0};
        for (int64_t k = 0; k < n; k++) b = pick(b, Best{p[k * inner], k});
        if (val) val[t] = b.v;
        if (idx) idx[t] = int32_t(b.k);
    }
}

// ------------------------------------------------------------------ indexing

__global__ __launch_bounds__(kOpsThreads) void k_gather(const float *__restrict__ x, int64_t outer, int64_t n,
                                                        int64_t inner, const int32_t *__restrict__ idx, int64_t m,
                                                        float *__restrict__ y) {
    GRID_STRIDE(t, outer * m * inner) {
        const int64_t i = t % inner, o = t / (m * inner);
        const int32_t j = idx[t];
        y[t] = (j >= 0 && j < n) ? x[(o * n + j) * inner + i] : __builtin_nanf("");
    }
}

__global__ __launch_bounds__(kOpsThreads) void k_index_select(const float *__restrict__ x, int64_t outer, int64_t n,
                                                              int64_t inner, const int32_t *__restrict__ idx,
                                                              int64_t m, float *__restrict__ y) {
    GRID_STRIDE(t, outer * m * inner) {
        const int64_t i = t % inner, r = t / inner, k = r % m, o = r / m;
        const int32_t j = idx[k];
        y[t] = (j >= 0 && j < n) ? x[(o * n + j) * inner + i] : __builtin_nanf("");
    }
}

__global__ __launch_bounds__(kOpsThreads) void k_one_hot(const int32_t *__restrict__ idx, int64_t count, int64_t n,
                                                         float *__restrict__ y) {
    GRID_STRIDE(t, count * n) { y[t] = int64_t(idx[t / n]) == t % n ? 1.0f : 0.0f; }
}

// One thread per target, the contributions in ascending source order (no atomics).
__global__ __launch_bounds__(kOpsThreads) void k_scatter_add(const int32_t *__restrict__ idx,
                                                             const float *__restrict__ v, int64_t outer, int64_t n,
                                                             int64_t inner, int64_t m, float *__restrict__ y) {
    GRID_STRIDE(t, outer * n * inner) {
        const int64_t i = t % inner, r = t / inner, j = r % n, o = r / n;
        float acc = 0.0f;
        for (int64_t k = 0; k < m; k++) {
            const int64_t q = (o * m + k) * inner + i;
            if (int64_t(idx[q]) == j) acc = acc + v[q];
        }
        y[t] = acc;
    }
}

__global__ __launch_bounds__(kOpsThreads) void k_index_add(const int32_t *__restrict__ idx,
                                                           const float *__restrict__ v, int64_t outer, int64_t n,
                                                           int64_t inner, int64_t m, float *__restrict__ y) {
    GRID_STRIDE(t, outer * n * inner) {
        const int64_t i = t % inner, r = t / inner, j = r % n, o = r / n;
        float acc = 0.0f;
        for (int64_t k = 0; k < m; k++)
            if (int64_t(idx[k]) == j) acc = acc + v[(o * m + k) * inner + i];
        y[t] = acc;
    }
}

__global__ __launch_bounds__(kOpsThreads) void k_fill(float *__restrict__ y, int64_t n, float value) {
    GRID_STRIDE(i, n) { y[i] = value; }
}

int check_lanes(int64_t outer, int64_t n, int64_t inner, int64_t m, const char *what) {
    if (outer < 0 || n < 0 || inner < 0 || m < 0) return fail(NT_E_ARG, std::string(what) + ": negative size");
    return 0;
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" {

int nt_hip_copy(const void *x, const NtLayout *xl, int32_t elem_bytes, void *out) {
    if (int rc = check_layout(xl, "copy")) return rc;
    if (!x || !out) return numel_of(xl) == 0 ? 0 : fail(NT_E_ARG, "copy: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    const NtLayout yl = contiguous_like(xl);
    return copy_any(x, xl, out, &yl, elem_bytes);
}

int nt_hip_write(void *dst, const NtLayout *dl, const void *src, const NtLayout *sl, int32_t elem_bytes) {
    if (int rc = check_layout(dl, "write")) return rc;
    if (int rc = check_layout(sl, "write")) return rc;
    if (!same_shape(dl, sl)) return fail(NT_E_ARG, "write: the views' shapes differ");
    if (!dst || !src) return numel_of(sl) == 0 ? 0 : fail(NT_E_ARG, "write: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    return copy_any(src, sl, dst, dl, elem_bytes);
}

int nt_hip_cast(const void *x, const NtLayout *xl, int32_t from, int32_t to, void *out) {
    if (int rc = check_layout(xl, "cast")) return rc;
    if (!x || !out) return numel_of(xl) == 0 ? 0 : fail(NT_E_ARG, "cast: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (from == to) {
        const NtLayout yl = contiguous_like(xl);
        const int eb = (from == NT_DT_BF16 || from == NT_DT_F16) ? 2
                       : (from == NT_DT_BOOL || from == NT_DT_U8) ? 1
                       : from == NT_DT_I64                          ? 8
                                                                    : 4;
        return copy_any(x, xl, out, &yl, eb);
    }
    if (to == NT_DT_F32) {
        if (from == NT_DT_BF16) return launch_cast<NT_DT_BF16, NT_DT_F32>(x, xl, out);
        if (from == NT_DT_F16) return launch_cast<NT_DT_F16, NT_DT_F32>(x, xl, out);
        if (from == NT_DT_BOOL) return launch_cast<NT_DT_BOOL, NT_DT_F32>(x, xl, out);
    } else if (to == NT_DT_BF16) {
        if (from == NT_DT_F32) return launch_cast<NT_DT_F32, NT_DT_BF16>(x, xl, out);
        if (from == NT_DT_F16) return launch_cast<NT_DT_F16, NT_DT_BF16>(x, xl, out);
    } else if (to == NT_DT_F16) {
        if (from == NT_DT_F32) return launch_cast<NT_DT_F32, NT_DT_F16>(x, xl, out);
        if (from == NT_DT_BF16) return launch_cast<NT_DT_BF16, NT_DT_F16>(x, xl, out);
    }
    return fail(NT_E_UNSUPPORTED, "cast " + std::to_string(from) + " -> " + std::to_string(to));
}

int nt_hip_unary(int32_t op, float scalar, const float *x, const NtLayout *xl, float *out) {
    if (int rc = check_layout(xl, "unary")) return rc;
    if (op < NT_UN_NEG || op > NT_UN_POW_SCALAR) return fail(NT_E_ARG, "unary: op " + std::to_string(op));
    const int64_t n = numel_of(xl);
    if (n == 0) return 0;
    if (!x || !out) return fail(NT_E_ARG, "unary: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    const NtLayout *ls[1] = {xl};
    View v[1];
    const int R = simplify(ls, 1, v);
    hipStream_t s = ctx().stream;
    if (R == 1 && v[0].st[0] == 1 && reinterpret_cast<uintptr_t>(x + v[0].off) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(out) % 16 == 0) {
        hipLaunchKernelGGL(k_unary_vec, dim3(blocks_for((n + 3) / 4)), dim3(kOpsThreads), 0, s, int(op), scalar,
                           x + v[0].off, out, n);
        return launched("unary");
    }
    RANK_SWITCH(R, hipLaunchKernelGGL((k_unary<RR>), dim3(blocks_for(n)), dim3(kOpsThreads), 0, s, int(op), scalar, x,
                                      v[0], out, n));
    return launched("unary");
}

int nt_hip_compare(int32_t op, float scalar, const float *x, const NtLayout *xl, uint8_t *out) {
    if (int rc = check_layout(xl, "compare")) return rc;
    if (op < NT_CMP_GT || op > NT_CMP_EQ) return fail(NT_E_ARG, "compare: op " + std::to_string(op));
    const int64_t n = numel_of(xl);
    if (n == 0) return 0;
    if (!x || !out) return fail(NT_E_ARG, "compare: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    const NtLayout *ls[1] = {xl};
    View v[1];
    const int R = simplify(ls, 1, v);
    hipStream_t s = ctx().stream;
    RANK_SWITCH(R, hipLaunchKernelGGL((k_compare<RR>), dim3(blocks_for(n)), dim3(kOpsThreads), 0, s, int(op), scalar,
                                      x, v[0], out, n));
    return launched("compare");
}

int nt_hip_binary(int32_t op, const float *a, const NtLayout *al, const float *b, const NtLayout *bl, float *out) {
    if (int rc = check_layout(al, "binary")) return rc;
    if (int rc = check_layout(bl, "binary")) return rc;
    if (op < NT_BIN_ADD || op > NT_BIN_DIV) return fail(NT_E_ARG, "binary: op " + std::to_string(op));
    if (!same_shape(al, bl)) return fail(NT_E_ARG, "binary: the operands are not broadcast to one shape");
    const int64_t n = numel_of(al);
    if (n == 0) return 0;
    if (!a || !b || !out) return fail(NT_E_ARG, "binary: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    const NtLayout *ls[2] = {al, bl};
    View v[2];
    const int R = simplify(ls, 2, v);
    hipStream_t s = ctx().stream;
    RANK_SWITCH(R, hipLaunchKernelGGL((k_binary<RR>), dim3(blocks_for(n)), dim3(kOpsThreads), 0, s, int(op), a, v[0],
                                      b, v[1], out, n));
    return launched("binary");
}

int nt_hip_mask_fill(const float *x, const NtLayout *xl, const uint8_t *mask, const NtLayout *ml, float value,
                     float *out) {
    if (int rc = check_layout(xl, "mask_fill")) return rc;
    if (int rc = check_layout(ml, "mask_fill")) return rc;
    if (!same_shape(xl, ml)) return fail(NT_E_ARG, "mask_fill: the mask is not broadcast to the input's shape");
    const int64_t n = numel_of(xl);
    if (n == 0) return 0;
    if (!x || !mask || !out) return fail(NT_E_ARG, "mask_fill: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    const NtLayout *ls[2] = {xl, ml};
    View v[2];
    const int R = simplify(ls, 2, v);
    hipStream_t s = ctx().stream;
    RANK_SWITCH(R, hipLaunchKernelGGL((k_mask_fill<RR>), dim3(blocks_for(n)), dim3(kOpsThreads), 0, s, x, v[0], mask,
                                      v[1], value, out, n));
    return launched("mask_fill");
}

int nt_hip_reduce_dim(int32_t op, const float *x, int64_t outer, int64_t n, int64_t inner, int32_t last_axis,
                      void *out) {
    if (int rc = check_lanes(outer, n, inner, 0, "reduce_dim")) return rc;
    if (op < NT_RED_SUM || op > NT_RED_ARGMAX) return fail(NT_E_ARG, "reduce_dim: op " + std::to_string(op));
    if (op != NT_RED_SUM && n == 0) return fail(NT_E_ARG, "max or argmax along an empty dimension");
    if (last_axis && inner != 1) return fail(NT_E_ARG, "reduce_dim: the last axis has inner size 1");
    const int64_t lanes = outer * inner;
    if (lanes == 0) return 0;
    if (!out || (!x && n > 0)) return fail(NT_E_ARG, "reduce_dim: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    hipStream_t s = ctx().stream;
    float *val = op == NT_RED_ARGMAX ? nullptr : static_cast<float *>(out);
    int32_t *idx = op == NT_RED_ARGMAX ? static_cast<int32_t *>(out) : nullptr;
    if (op == NT_RED_SUM) {
        if (last_axis) {
            const int64_t per_block = kOpsThreads / 8;
            int64_t b = (outer + per_block - 1) / per_block;
            b = b > kMaxBlocks ? kMaxBlocks : b;
            hipLaunchKernelGGL(k_sum_last, dim3(unsigned(b)), dim3(kOpsThreads), 0, s, x, outer, n, val);
        } else {
            hipLaunchKernelGGL(k_sum_mid, dim3(blocks_for(lanes)), dim3(kOpsThreads), 0, s, x, outer, n, inner, val);
        }
        return launched("reduce_dim sum");
    }
    if (inner == 1) {
        const int64_t b = outer > kMaxBlocks ? kMaxBlocks : outer;
        hipLaunchKernelGGL(k_best_last, dim3(unsigned(b)), dim3(kBestThreads), 0, s, x, outer, n, val, idx);
    } else {
        hipLaunchKernelGGL(k_best_mid, dim3(blocks_for(lanes)), dim3(kOpsThreads), 0, s, x, outer, n, inner, val, idx);
    }
    return launched("reduce_dim max");
}

int nt_hip_reduce_all(int32_t op, const float *x, int64_t n, float *out) {
    if (n < 0) return fail(NT_E_ARG, "reduce_all: negative size");
    if (op == NT_RED_ARGMAX) return fail(NT_E_UNSUPPORTED, "argmax over all elements");
    if (op != NT_RED_SUM && op != NT_RED_MAX) return fail(NT_E_ARG, "reduce_all: op " + std::to_string(op));
    if (op == NT_RED_MAX && n == 0) return fail(NT_E_ARG, "max of an empty tensor");
    if (!out || (!x && n > 0)) return fail(NT_E_ARG, "reduce_all: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    hipStream_t s = ctx().stream;
    if (op == NT_RED_SUM) hipLaunchKernelGGL(k_sum_last, dim3(1), dim3(kOpsThreads), 0, s, x, int64_t(1), n, out);
    else hipLaunchKernelGGL(k_best_last, dim3(1), dim3(kBestThreads), 0, s, x, int64_t(1), n, out, (int32_t *)nullptr);
    return launched("reduce_all");
}

int nt_hip_gather(const float *x, int64_t outer, int64_t n, int64_t inner, const int32_t *idx, int64_t m, float *out) {
    if (int rc = check_lanes(outer, n, inner, m, "gather")) return rc;
    const int64_t t = outer * m * inner;
    if (t == 0) return 0;
    if (!x || !idx || !out) return fail(NT_E_ARG, "gather: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    hipLaunchKernelGGL(k_gather, dim3(blocks_for(t)), dim3(kOpsThreads), 0, ctx().stream, x, outer, n, inner, idx, m,
                       out);
    return launched("gather");
}

int nt_hip_index_select(const float *x, int64_t outer, int64_t n, int64_t inner, const int32_t *idx, int64_t m,
                        float *out) {
    if (int rc = check_lanes(outer, n, inner, m, "index_select")) return rc;
    const int64_t t = outer * m * inner;
    if (t == 0) return 0;
    if (!x || !idx || !out) return fail(NT_E_ARG, "index_select: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    hipLaunchKernelGGL(k_index_select, dim3(blocks_for(t)), dim3(kOpsThreads), 0, ctx().stream, x, outer, n, inner,
                       idx, m, out);
    return launched("index_select");
}

int nt_hip_one_hot(const int32_t *idx, int64_t count, int64_t n, float *out) {
    if (count < 0 || n < 0) return fail(NT_E_ARG, "one_hot: negative size");
    if (count * n == 0) return 0;
    if (!idx || !out) return fail(NT_E_ARG, "one_hot: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    hipLaunchKernelGGL(k_one_hot, dim3(blocks_for(count * n)), dim3(kOpsThreads), 0, ctx().stream, idx, count, n, out);
    return launched("one_hot");
}

int nt_hip_scatter_add(const int32_t *idx, const float *v, int64_t outer, int64_t n, int64_t inner, int64_t m,
                       float *out) {
    if (int rc = check_lanes(outer, n, inner, m, "scatter_add")) return rc;
    const int64_t t = outer * n * inner;
    if (t == 0) return 0;
    if (!out || (m > 0 && (!idx || !v))) return fail(NT_E_ARG, "scatter_add: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    hipLaunchKernelGGL(k_scatter_add, dim3(blocks_for(t)), dim3(kOpsThreads), 0, ctx().stream, idx, v, outer, n, inner,
                       m, out);
    return launched("scatter_add");
}

int nt_hip_index_add(const int32_t *idx, const float *v, int64_t outer, int64_t n, int64_t inner, int64_t m,
                     float *out) {
    if (int rc = check_lanes(outer, n, inner, m, "index_add")) return rc;
    const int64_t t = outer * n * inner;
    if (t == 0) return 0;
    if (!out || (m > 0 && (!idx || !v))) return fail(NT_E_ARG, "index_add: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    hipLaunchKernelGGL(k_index_add, dim3(blocks_for(t)), dim3(kOpsThreads), 0, ctx().stream, idx, v, outer, n, inner,
                       m, out);
    return launched("index_add");
}

int nt_hip_fill(float *out, int64_t n, float value) {
    if (n < 0) return fail(NT_E_ARG, "fill: negative size");
    if (n == 0) return 0;
    if (!out) return fail(NT_E_ARG, "fill: null buffer");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    hipLaunchKernelGGL(k_fill, dim3(blocks_for(n)), dim3(kOpsThreads), 0, ctx().stream, out, n, value);
    return launched("fill");
}

}  // extern "C"
