// Device helpers shared by the nn::rl row kernels (rl_sample.hip, rl_kernels.hip): element
// access and decoding of f32/bf16 logit rows and their masks, the hardware exp2/log and the
// fixed-order DPP reductions and scans, and the host-side argument checks of the row entry points.
#pragma once

#ifdef __HIPCC_RTC__
// compiled at run time by hiprtc (rtc.cpp): the device part only, the C header under its own name
#include <stdint.h>
#include <type_traits>

#include "noetic_hip.h"
// <cmath>'s and <cfloat>'s constants, as the compiler defines them there
#define INFINITY __builtin_inff()
#define NAN __builtin_nanf("")
#define FLT_MAX __FLT_MAX__
#else
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <type_traits>

#include "../../include/noetic_hip.h"
#include "nt_internal.hpp"
#endif

namespace nt {
namespace {

constexpr int kWave = 64;
constexpr int kEpl = 8;                  // elements per lane per chunk
constexpr int kChunk = kWave * kEpl;     // 512 elements per chunk
constexpr int kBatch = 4;                // chunks per wave with loads in flight together
constexpr int kMaskStage = 2;            // streaming sampler, f32 mask on 16-bit rows: chunks per wave staged in LDS
// The most a lane's 8 weights of one chunk may sum to before its exponent reference moves to the
// chunk's maximum, where a finishing difference of two log-sums must stay small (entropy, KL):
// the reference then trails the maximum by at most log2 32 = 5 (log2 units).
constexpr float kChunkSumCap = 32.0f;
constexpr float kLog2e = 1.44269504088896340736f;
constexpr double kLn2 = 0.69314718055994530942;
constexpr int kRowBadToken = NT_ROW_BAD_TOKEN;

// ------------------------------------------------------------------ element access

template <int DT>
struct Elem;
template <>
struct Elem<NT_F32> {
    static constexpr int kWords = 8;     // 8 f32 per lane per chunk
    static constexpr uint32_t kNegInf = 0xff800000u;
    static constexpr int kBytes = 4;
};
template <>
struct Elem<NT_BF16> {
    static constexpr int kWords = 4;     // 8 bf16 packed two per word
    static constexpr uint32_t kNegInf = 0xff80ff80u;
    static constexpr int kBytes = 2;
};
template <>
struct Elem<NT_F16> {
    static constexpr int kWords = 4;     // 8 f16 packed two per word
    static constexpr uint32_t kNegInf = 0xfc00fc00u;
    static constexpr int kBytes = 2;
};

// A 16-bit logit (the low half of h) as f32, exactly: bf16 is f32's top half; f16 converts
// with v_cvt_f32_f16, exact for every f16 value (subnormals, infinities and NaNs included).
template <int DT>
__device__ __forceinline__ float widen16(uint32_t h) {
    if constexpr (DT == NT_BF16) return __uint_as_float(h << 16);
    else return float(__builtin_bit_cast(_Float16, uint16_t(h)));
}

// The mask row a logits row reads (NtMaskRows): row = (s B + b) T + t reads the mask row at
// element s ld_s + b ld_b + t ld. The host sets T = rows and B = 1 for rows of stride ld.
struct MaskMap {
    int64_t ld, ld_b, ld_s;
    uint32_t T, B;
};
__device__ __forceinline__ int64_t mask_row_at(const MaskMap &m, int64_t row) {
    const uint32_t r = uint32_t(row);
    const uint32_t q = r / m.T, t = r - q * m.T;
    const uint32_t s = q / m.B, b = q - s * m.B;
    return int64_t(s) * m.ld_s + int64_t(b) * m.ld_b + int64_t(t) * m.ld;
}

template <int MK>
struct MaskWords {
    static constexpr int kWords = MK == NT_MASK_U8 ? 2 : (MK == NT_MASK_F32 ? 8 : 0);
    static constexpr int kBytes = MK == NT_MASK_U8 ? 1 : (MK == NT_MASK_F32 ? 4 : 0);
};

// The raw bits of one lane's 8 elements of one chunk (logits and mask).
template <int DT, int MK>
struct Raw {
    uint32_t x[Elem<DT>::kWords];
    uint32_t m[MaskWords<MK>::kWords > 0 ? MaskWords<MK>::kWords : 1];
};

// Load the 8 elements at e0 of a row. AL: the row and mask are 16-/8-byte aligned and V % 8
// == 0, so a lane's 8 elements are all inside the row or all outside it. Elements outside
// the row read as -inf logits.
template <int DT, int MK, bool AL>
__device__ __forceinline__ void load_raw(Raw<DT, MK> &r, const void *xrow, const void *mrow, int64_t e0,
                                         int64_t V) {
    if constexpr (MK == NT_MASK_NONE) r.m[0] = 0;
    if constexpr (AL) {
        if (e0 < V) {
            if constexpr (DT == NT_F32) {
                const uint4 *q = reinterpret_cast<const uint4 *>(static_cast<const float *>(xrow) + e0);
                uint4 a = q[0], b = q[1];
                r.x[0] = a.x; r.x[1] = a.y; r.x[2] = a.z; r.x[3] = a.w;
                r.x[4] = b.x; r.x[5] = b.y; r.x[6] = b.z; r.x[7] = b.w;
            } else {
                uint4 a = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(xrow) + e0);
                r.x[0] = a.x; r.x[1] = a.y; r.x[2] = a.z; r.x[3] = a.w;
            }
            if constexpr (MK == NT_MASK_U8) {
                uint2 k = *reinterpret_cast<const uint2 *>(static_cast<const uint8_t *>(mrow) + e0);
                r.m[0] = k.x; r.m[1] = k.y;
            } else if constexpr (MK == NT_MASK_F32) {
                const uint4 *q = reinterpret_cast<const uint4 *>(static_cast<const float *>(mrow) + e0);
                uint4 a = q[0], b = q[1];
                r.m[0] = a.x; r.m[1] = a.y; r.m[2] = a.z; r.m[3] = a.w;
                r.m[4] = b.x; r.m[5] = b.y; r.m[6] = b.z; r.m[7] = b.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < Elem<DT>::kWords; i++) r.x[i] = Elem<DT>::kNegInf;
#pragma unroll
            for (int i = 0; i < (MaskWords<MK>::kWords > 0 ? MaskWords<MK>::kWords : 1); i++) r.m[i] = 0;
        }
    } else {
#pragma unroll
        for (int j = 0; j < kEpl; j++) {
            const int64_t e = e0 + j;
            const bool in = e < V;
            if constexpr (DT == NT_F32) {
                r.x[j] = in ? __float_as_uint(static_cast<const float *>(xrow)[e]) : Elem<DT>::kNegInf;
            } else {
                uint32_t h = in ? uint32_t(static_cast<const uint16_t *>(xrow)[e]) : (Elem<DT>::kNegInf & 0xffffu);
                if (j % 2 == 0) r.x[j / 2] = h;
                else r.x[j / 2] |= h << 16;
            }
            if constexpr (MK == NT_MASK_U8) {
                uint32_t k = in ? uint32_t(static_cast<const uint8_t *>(mrow)[e]) : 0u;
                if (j % 4 == 0) r.m[j / 4] = k;
                else r.m[j / 4] |= k << (8 * (j % 4));
            } else if constexpr (MK == NT_MASK_F32) {
                r.m[j] = in ? __float_as_uint(static_cast<const float *>(mrow)[e]) : 0u;
            }
        }
    }
}

// Aligned load of the 8 elements at e0 with no bounds test (the caller passes an in-bounds
// e0), so that a run of these loads is straight-line code the compiler can wait on one by one.
template <int DT, int MK>
__device__ __forceinline__ void load_raw_inbounds(Raw<DT, MK> &r, const void *xrow, const void *mrow, int64_t e0) {
    if constexpr (DT == NT_F32) {
        const uint4 *q = reinterpret_cast<const uint4 *>(static_cast<const float *>(xrow) + e0);
        uint4 a = q[0], b = q[1];
        r.x[0] = a.x; r.x[1] = a.y; r.x[2] = a.z; r.x[3] = a.w;
        r.x[4] = b.x; r.x[5] = b.y; r.x[6] = b.z; r.x[7] = b.w;
    } else {
        uint4 a = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(xrow) + e0);
        r.x[0] = a.x; r.x[1] = a.y; r.x[2] = a.z; r.x[3] = a.w;
    }
    if constexpr (MK == NT_MASK_U8) {
        uint2 k = *reinterpret_cast<const uint2 *>(static_cast<const uint8_t *>(mrow) + e0);
        r.m[0] = k.x; r.m[1] = k.y;
    } else if constexpr (MK == NT_MASK_F32) {
        const uint4 *q = reinterpret_cast<const uint4 *>(static_cast<const float *>(mrow) + e0);
        uint4 a = q[0], b = q[1];
        r.m[0] = a.x; r.m[1] = a.y; r.m[2] = a.z; r.m[3] = a.w;
        r.m[4] = b.x; r.m[5] = b.y; r.m[6] = b.z; r.m[7] = b.w;
    } else {
        r.m[0] = 0;
    }
}

// Logit j of a lane's chunk as f32 (bf16 and f16 widened exactly).
template <int DT>
__device__ __forceinline__ float logit(const uint32_t *x, int j) {
    if constexpr (DT == NT_F32) return __uint_as_float(x[j]);
    else if constexpr (DT == NT_BF16) return __uint_as_float((j % 2 == 0) ? (x[j / 2] << 16) : (x[j / 2] & 0xffff0000u));
    else return widen16<DT>((j % 2 == 0) ? (x[j / 2] & 0xffffu) : (x[j / 2] >> 16));
}

// z[j] / tau in place for tau > 0, each quotient the correctly rounded f32 of the division. The
// f64 product of z with rt = 1 / tau (rounded to f64) lies within 2^-52 relative of the exact
// quotient. An exact quotient of two f32 values of magnitude at least 2^-126 lies at least 2^-49
// relative from every boundary where f32 rounding changes (the midpoints M 2^e between
// neighbours, M odd with 2^24 <= M < 2^25, and the overflow threshold, which is one of them:
// reaching one would take a numerator of more than 24 significant bits). So the product rounded
// to f32 is the division's result, zeros, infinities and NaN included. Below 2^-126 the midpoints
// are evenly spaced and a quotient can be one exactly; a wave holding such a nonzero element
// divides those. (The f32 division is a ten-instruction sequence; this is three, and a lane's
// test for such elements is one minimum over its N quotients. A NaN can hide a small quotient
// from that minimum; its row is refused, NaN, whatever the other values.)
template <int N>
__device__ __forceinline__ void div_tau(float *z, float tau) {
    const double rt = 1.0 / double(tau);
    float q[N];
#pragma unroll
    for (int j = 0; j < N; j++) q[j] = float(double(z[j]) * rt);
    // one test per lane: the smallest magnitude of its quotients (v_min3 with |.| modifiers; a
    // zero quotient, exact, sends the wave down the test per element as well)
    float m = fabsf(q[0]);
#pragma unroll
    for (int j = 1; j < N; j += 2) {
        float r;
        asm volatile("v_min3_f32 %0, |%1|, |%2|, |%3|" : "=v"(r) : "v"(m), "v"(q[j]), "v"(q[j + 1 < N ? j + 1 : j]));
        m = r;
    }
    if (__builtin_amdgcn_ballot_w64(m < 0x1p-126f)) {
#pragma unroll
        for (int j = 0; j < N; j++)
            if (fabsf(q[j]) < 0x1p-126f && z[j] != 0.0f) q[j] = z[j] / tau;
    }
#pragma unroll
    for (int j = 0; j < N; j++) z[j] = q[j];
}

// The "value" of an element, the quantity the kernels take maxima and exponentials of.
//  - no mask / u8 mask: v = x (an excluded token -> -inf); the temperature is applied through
//    the exponent scale c = log2(e)/T, and m_z = max(x)/T is exact because correctly rounded
//    division by T > 0 is monotonic.
//  - additive f32 mask: v = z = x / T + mask exactly as tempered_logits computes it
//    (rl.rs:477-484, float.rs:494-499); c = log2(e).
template <int DT, int MK>
__device__ __forceinline__ void decode_words(const uint32_t *xw, const uint32_t *mw, float v[kEpl], float tau,
                                             bool tau_one) {
    if constexpr (MK == NT_MASK_F32) {
        float z[kEpl];
#pragma unroll
        for (int j = 0; j < kEpl; j++) z[j] = logit<DT>(xw, j);
        if (!tau_one) div_tau<kEpl>(z, tau);
#pragma unroll
        for (int j = 0; j < kEpl; j++) v[j] = z[j] + __uint_as_float(mw[j]);
        return;
    }
#pragma unroll
    for (int j = 0; j < kEpl; j++) {
        float x = logit<DT>(xw, j);
        if constexpr (MK == NT_MASK_U8) {
            const uint32_t keep = (mw[j / 4] >> (8 * (j % 4))) & 0xffu;
            v[j] = keep ? x : -INFINITY;
        } else if constexpr (MK == NT_MASK_F32) {
            const float z = tau_one ? x : x / tau;
            v[j] = z + __uint_as_float(mw[j]);
        } else {
            v[j] = x;
        }
    }
}

template <int DT, int MK>
__device__ __forceinline__ void decode(const Raw<DT, MK> &r, float v[kEpl], float tau, bool tau_one) {
    decode_words<DT, MK>(r.x, r.m, v, tau, tau_one);
}

template <int MK>
__device__ __forceinline__ void load_mask_inbounds(uint32_t *m, const void *mrow, int64_t e0) {
    if constexpr (MK == NT_MASK_U8) {
        uint2 k = *reinterpret_cast<const uint2 *>(static_cast<const uint8_t *>(mrow) + e0);
        m[0] = k.x; m[1] = k.y;
    } else if constexpr (MK == NT_MASK_F32) {
        const uint4 *q = reinterpret_cast<const uint4 *>(static_cast<const float *>(mrow) + e0);
        uint4 a = q[0], b = q[1];
        m[0] = a.x; m[1] = a.y; m[2] = a.z; m[3] = a.w;
        m[4] = b.x; m[5] = b.y; m[6] = b.z; m[7] = b.w;
    }
}

// Write decoded values back into the logit words (exact: each value is the widened logit or
// -inf, both representable in the storage type), so the mask is no longer needed.
template <int DT>
__device__ __forceinline__ void fold_values(uint32_t *x, const float v[kEpl]) {
#pragma unroll
    for (int j = 0; j < kEpl; j++) {
        if constexpr (DT == NT_F32) {
            x[j] = __float_as_uint(v[j]);
        } else if constexpr (DT == NT_BF16) {
            if (j % 2 == 1) x[j / 2] = (__float_as_uint(v[j]) & 0xffff0000u) | (__float_as_uint(v[j - 1]) >> 16);
        } else if (j % 2 == 1) {
            // f16: each value is a widened f16 or -inf, so the narrowing is exact in any rounding
            x[j / 2] = uint32_t(__builtin_bit_cast(uint16_t, _Float16(v[j - 1]))) |
                       (uint32_t(__builtin_bit_cast(uint16_t, _Float16(v[j]))) << 16);
        }
    }
}

// Decode words that were folded (the mask already applied) or, for an f32 mask, not.
template <int DT, int MK, bool FOLDED>
__device__ __forceinline__ void decode_folded(const Raw<DT, MK> &r, float v[kEpl], float tau, bool tau_one) {
    if constexpr (FOLDED) decode_words<DT, NT_MASK_NONE>(r.x, r.m, v, tau, tau_one);
    else decode_words<DT, MK>(r.x, r.m, v, tau, tau_one);
}

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// ln x for a finite x >= 2^-1021 in f64, within about 1e-7 absolute: the binary exponent exactly,
// plus v_log_f32 of the mantissa in [0.5, 1) rounded to f32 (2^-24 relative, then the
// instruction's 1 ulp). A dozen instructions where the f64 library log takes about a hundred
// on the row's critical path.
__device__ __forceinline__ double ln_fast(double x) {
    const uint64_t b = uint64_t(__double_as_longlong(x));
    const int e = int((b >> 52) & 0x7ff) - 1022;
    const double m = __longlong_as_double(int64_t((b & 0x000fffffffffffffull) | (1022ull << 52)));
    return (double(e) + double(__builtin_amdgcn_logf(float(m)))) * 0.69314718055994530942;
}

__device__ __forceinline__ float max8(const float v[kEpl]) {
    return fmaxf(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])), fmaxf(fmaxf(v[4], v[5]), fmaxf(v[6], v[7])));
}

__device__ __forceinline__ float tree8(const float w[kEpl]) {
    return ((w[0] + w[1]) + (w[2] + w[3])) + ((w[4] + w[5]) + (w[6] + w[7]));
}

// Butterfly reductions over the 64 lanes: every lane ends with the same bits (the operations
// are commutative), the order is fixed.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
// Inclusive prefix sum over lanes (Hillis-Steele, fixed order).
__device__ __forceinline__ double wave_scan_d(double v, int lane) {
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        double n = __shfl_up(v, o, kWave);
        if (lane >= o) v += n;
    }
    return v;
}
__device__ __forceinline__ int first_lane(uint64_t ballot) { return ballot ? __builtin_ctzll(ballot) : -1; }
__device__ __forceinline__ int last_lane(uint64_t ballot) { return ballot ? 63 - __builtin_clzll(ballot) : -1; }

typedef __attribute__((address_space(3))) void *lds_ptr_t;
// Word 3 of a gfx9-family buffer resource: 32-bit data format, no swizzle; with stride 0 every
// access is range-checked against the byte count in word 2.
constexpr int kBufferWord3 = 0x00020000;
// Four dwords as the buffer load/store builtins take them.
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
// Buffer access cache policy for data read or written once: non-temporal.
constexpr int kCachePolicyNT = 2;
typedef __attribute__((address_space(1))) void *glb_ptr_t;

template <int B, int E, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// s_waitcnt with only the vector-memory counter constrained (expcnt and lgkmcnt at their
// maxima): gfx9 encoding, vmcnt bits [3:0] and [15:14].
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// An LDS read the compiler does not track (it would otherwise wait for every outstanding load
// because the data came from an LDS DMA); the caller has waited for that DMA.
__device__ __forceinline__ uint2 lds_read_b64(uint32_t addr) {
    uint2 r;
    asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(addr) : "memory");
    return r;
}
template <int OFF>
__device__ __forceinline__ uint2 lds_read_b64_off(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
    uint2 r;
    asm volatile("ds_read_b64 %0, %1 offset:%2\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
    return r;
}
// Four such reads at immediate offsets from one address, then one wait. The results are
// early-clobber: the reads are still in flight while the address register is read again.
template <int O0, int O1, int O2, int O3>
__device__ __forceinline__ void lds_read4_b64(uint32_t addr, uint2 &r0, uint2 &r1, uint2 &r2, uint2 &r3) {
    static_assert(O0 >= 0 && O3 < 65536 && O1 < 65536 && O2 < 65536, "ds offset field");
    asm volatile(
        "ds_read_b64 %0, %4 offset:%5\n\tds_read_b64 %1, %4 offset:%6\n\t"
        "ds_read_b64 %2, %4 offset:%7\n\tds_read_b64 %3, %4 offset:%8\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
        : "v"(addr), "i"(O0), "i"(O1), "i"(O2), "i"(O3)
        : "memory");
}
__device__ __forceinline__ uint4 lds_read_b128(uint32_t addr) {
    uint4 r;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(addr) : "memory");
    return r;
}

// v_max3_f32 without the canonicalising moves the compiler puts in front of fmaxf: the inputs
// are widened logits or -inf, and a NaN among them reaches the row's sum through exp2 anyway.
__device__ __forceinline__ float max3_hw(float a, float b, float c) {
    float r;
    asm volatile("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ float max8_hw(const float v[kEpl]) {
    const float t0 = max3_hw(v[0], v[1], v[2]);
    const float t1 = max3_hw(v[3], v[4], v[5]);
    return max3_hw(t0, t1, max3_hw(v[6], v[7], v[7]));
}

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    const uint64_t b = uint64_t(__double_as_longlong(v));
    const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b)), l));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b >> 32)), l));
    return __longlong_as_double(int64_t((uint64_t(hi) << 32) | lo));
}
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
// Maximum over the 64 lanes: xor-1 and xor-2 quad permutes, the 8- and 16-lane mirrors, then
// the four rows in a fixed order, each step a v_max3_f32 (no canonicalising moves; the inputs
// are maxima of widened logits or -inf). The result is uniform and independent of timing.
// Maximum inside each 16-lane row (the first four steps of wave_max3_dpp): every lane of a row
// holds its row's maximum.
__device__ __forceinline__ float row_max3_dpp(float v) {
    v = max3_hw(v, dpp_mov<0xB1>(v), dpp_mov<0xB1>(v));
    v = max3_hw(v, dpp_mov<0x4E>(v), dpp_mov<0x4E>(v));
    v = max3_hw(v, dpp_mov<0x141>(v), dpp_mov<0x141>(v));
    return max3_hw(v, dpp_mov<0x140>(v), dpp_mov<0x140>(v));
}
__device__ __forceinline__ float wave_max3_dpp(float v) {
    v = row_max3_dpp(v);
    return max3_hw(max3_hw(readlane_f(v, 0), readlane_f(v, 16), readlane_f(v, 32)), readlane_f(v, 48),
                   readlane_f(v, 48));
}
// One DPP step on an f64: both 32-bit halves move with the same control; lanes with no
// source (or in rows the row mask leaves out) read 0, the identity of the sum.
template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, int(uint32_t(b)), CTRL, ROWS, 0xf, true);
    const int hi = __builtin_amdgcn_update_dpp(0, int(uint32_t(b >> 32)), CTRL, ROWS, 0xf, true);
    return __longlong_as_double(int64_t((uint64_t(uint32_t(hi)) << 32) | uint32_t(lo)));
}
// Inclusive prefix sum over the 64 lanes in f64, in a fixed order: shifts by 1, 2, 4 and 8
// inside each 16-lane row, then the row broadcasts of lanes 15 and 31 (the gfx9 DPP scan).
// Inclusive prefix sum inside each 16-lane row in f64 (the first four steps of wave_scan_dpp).
__device__ __forceinline__ double row_scan_dpp(double v) {
    v += dpp_f64<0x111, 0xf>(v);  // row_shr:1
    v += dpp_f64<0x112, 0xf>(v);  // row_shr:2
    v += dpp_f64<0x114, 0xf>(v);  // row_shr:4
    v += dpp_f64<0x118, 0xf>(v);  // row_shr:8
    return v;
}
__device__ __forceinline__ double wave_scan_dpp(double v) {
    v = row_scan_dpp(v);
    v += dpp_f64<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_f64<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

// Sum over each 16-lane row in four DPP steps (the two quad permutes, then the 8- and 16-lane
// mirrors); every lane of a row holds its row's sum.
__device__ __forceinline__ float row_sum_dpp(float v) {
    v = v + dpp_mov<0xB1>(v);
    v = v + dpp_mov<0x4E>(v);
    v = v + dpp_mov<0x141>(v);
    v = v + dpp_mov<0x140>(v);
    return v;
}
__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, kWave));
    return v;
}

// Per-lane data of one chunk of the register-resident sampler: EPL elements (8 or 16), read
// as 16-byte pieces (8 bf16 or 4 f32 each).
template <int DT, int EPL>
struct RRX {
    static constexpr int kWords = DT == NT_F32 ? EPL : EPL / 2;
    static constexpr int kPieces = kWords / 4;
    uint32_t x[kWords];
};

// Mask bytes per chunk in LDS and the LDS DMA instructions that bring one chunk's mask: lane l
// of DMA instruction d writes B bytes at slot + d * 64 B + l B (B = 16 when the chunk's mask is
// a whole number of 1 KiB, else 4).
template <int MK, int EPL>
struct RRMask {
    static constexpr int kBytes = MK == NT_MASK_U8 ? kWave * EPL : (MK == NT_MASK_F32 ? 4 * kWave * EPL : 0);
    static constexpr int kDmaBytes = kBytes % (16 * kWave) == 0 ? 16 : 4;
    static constexpr int kDma = kBytes / (kDmaBytes * kWave);
    static constexpr int kWords = MK == NT_MASK_U8 ? EPL / 4 : (MK == NT_MASK_F32 ? EPL : 1);  // per lane
};

// x if byte B (0, 1 or 2) of a mask word is nonzero, else -inf: one SDWA compare against the
// inline 0 (the compiler masks bytes 1 and 2 with a separate AND and keeps a zero register for
// byte 0; byte 3 it compares in one instruction).
template <int B>
__device__ __forceinline__ float keep_byte(uint32_t mw, float x, float ninf) {
    float r;
    if constexpr (B == 0)
        asm("v_cmp_ne_u32_sdwa vcc, %1, 0 src0_sel:BYTE_0 src1_sel:DWORD\n\tv_cndmask_b32 %0, %2, %3, vcc"
            : "=v"(r) : "v"(mw), "v"(ninf), "v"(x) : "vcc");
    else if constexpr (B == 1)
        asm("v_cmp_ne_u32_sdwa vcc, %1, 0 src0_sel:BYTE_1 src1_sel:DWORD\n\tv_cndmask_b32 %0, %2, %3, vcc"
            : "=v"(r) : "v"(mw), "v"(ninf), "v"(x) : "vcc");
    else
        asm("v_cmp_ne_u32_sdwa vcc, %1, 0 src0_sel:BYTE_2 src1_sel:DWORD\n\tv_cndmask_b32 %0, %2, %3, vcc"
            : "=v"(r) : "v"(mw), "v"(ninf), "v"(x) : "vcc");
    return r;
}

// Decode EPL elements (logit words + mask words) into the kernel's value space.
template <int DT, int MK, int EPL>
__device__ __forceinline__ void decode_e(const uint32_t *xw, const uint32_t *mw, float *v, float tau, bool tau_one) {
    if constexpr (MK == NT_MASK_F32) {
        float z[EPL];
#pragma unroll
        for (int j = 0; j < EPL; j++) z[j] = logit<DT>(xw, j);
        if (!tau_one) div_tau<EPL>(z, tau);
#pragma unroll
        for (int j = 0; j < EPL; j++) v[j] = z[j] + __uint_as_float(mw[j]);
        return;
    }
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const float x = logit<DT>(xw, j);
        if constexpr (MK == NT_MASK_U8) {
            if (j % 4 == 0) {
                v[j] = keep_byte<0>(mw[j / 4], x, -INFINITY);
            } else if (j % 4 == 1) {
                v[j] = keep_byte<1>(mw[j / 4], x, -INFINITY);
            } else if (j % 4 == 2) {
                v[j] = keep_byte<2>(mw[j / 4], x, -INFINITY);
            } else {
                const uint32_t keep = (mw[j / 4] >> (8 * (j % 4))) & 0xffu;
                v[j] = keep ? x : -INFINITY;
            }
        } else if constexpr (MK == NT_MASK_F32) {
            const float z = tau_one ? x : x / tau;
            v[j] = z + __uint_as_float(mw[j]);
        } else {
            v[j] = x;
        }
    }
}

// The lane's mask words of one chunk, from its LDS slot (the caller has waited for the DMA).
template <int MK, int EPL>
__device__ __forceinline__ void lds_mask_words(uint32_t a, uint32_t *mw) {
    if constexpr (MK == NT_MASK_U8 && EPL == 8) {
        const uint2 m2 = lds_read_b64(a);
        mw[0] = m2.x;
        mw[1] = m2.y;
    } else if constexpr (MK != NT_MASK_NONE) {
#pragma unroll
        for (int q = 0; q < RRMask<MK, EPL>::kWords / 4; q++) {
            const uint4 m4 = lds_read_b128(a + 16 * q);
            mw[4 * q] = m4.x;
            mw[4 * q + 1] = m4.y;
            mw[4 * q + 2] = m4.z;
            mw[4 * q + 3] = m4.w;
        }
    } else {
        mw[0] = 0;
    }
}

template <int N>
__device__ __forceinline__ float max_hw(const float *v) {
    if constexpr (N == 8) {
        return max8_hw(v);
    } else {
        const float a = max8_hw(v), b = max8_hw(v + 8);
        return max3_hw(a, b, b);
    }
}

template <int N>
__device__ __forceinline__ float tree_sum(const float *w) {
    if constexpr (N == 8) return tree8(w);
    else return tree8(w) + tree8(w + 8);
}

// ------------------------------------------------------------------ sampler arguments

struct SampleP {
    const void *logits;
    const void *mask;
    int64_t V, ld;
    MaskMap mm;       // the mask row of each logits row
    float c;          // exponent scale: log2(e)/T (no/u8 mask) or log2(e) (f32 mask)
    float tau;        // (float)T, the reference's divisor (float.rs:494-499)
    int tau_one;      // T == 1 (or greedy): no divide
    int greedy;
    int nc;           // chunks per row
    const double *u;
    int32_t *ids;
    float *logp;
    float *ent;
    uint8_t *status;
    // The largest f32 M whose tempered maximum M / tau rounds to -inf (-inf when tau >= 1): a
    // row whose maximum is at most this has no token (set by the host, neg_overflow_bound).
    float m_ovf;
};

// ------------------------------------------------------------------ host-side checks

#ifndef __HIPCC_RTC__
inline int check_rows(int64_t rows, int64_t V, int64_t ld, int32_t dtype, int32_t mk, const void *mask, int64_t mask_ld,
               const char *who) {
    char buf[256];
    if (rows < 0 || V < 1 || ld < V || (dtype != NT_F32 && dtype != NT_BF16 && dtype != NT_F16) || mk < NT_MASK_NONE ||
        mk > NT_MASK_F32 || ((mk == NT_MASK_NONE) != (mask == nullptr)) || (mask_ld != 0 && mask_ld < V) ||
        rows > 0x7fffffffLL) {
        std::snprintf(buf, sizeof buf,
                      "%s: invalid rows %lld, V %lld, ld %lld, dtype %d, mask kind %d (mask %s), mask_ld %lld", who,
                      (long long)rows, (long long)V, (long long)ld, dtype, mk, mask ? "set" : "null",
                      (long long)mask_ld);
        return fail(NT_E_ARG, buf);
    }
    return 0;
}

// The largest f32 m with m / tau == -inf in f32 (correctly rounded division, as the kernels'), or
// -inf when no finite m overflows (tau >= 1): a search over the f32 magnitudes, on which the
// quotient is monotonic. It lets a kernel refuse a row by one comparison instead of a division on
// its critical path.
inline float neg_overflow_bound(float tau) {
    const auto over = [&](uint32_t bits) {
        float m;
        std::memcpy(&m, &bits, 4);
        volatile float q = -m / tau;  // (computed at run time, in f32)
        return q == -INFINITY;
    };
    uint32_t lo = 0, hi = 0x7f7fffffu;  // magnitudes 0 .. FLT_MAX as their bit patterns
    if (!(tau > 0.0f) || !over(hi)) return -INFINITY;
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (over(mid)) hi = mid;
        else lo = mid + 1;
    }
    float m;
    std::memcpy(&m, &lo, 4);
    return -m;
}

// The mask map of a call (NtMaskRows, validated): all zero is T = rows, B = 1 (rows of mask_ld).
inline int mask_map(const NtMaskRows &mr, int64_t rows, int64_t V, int32_t mk, int64_t mask_ld, const char *who,
                    MaskMap *out) {
    MaskMap m{mask_ld, 0, 0, uint32_t(rows > 0 ? rows : 1), 1u};
    const bool dflt = mr.t_rows == 0 && mr.b_rows == 0 && mr.ld_b == 0 && mr.ld_s == 0;
    if (mk != NT_MASK_NONE && !dflt) {
        const int64_t T = mr.t_rows, B = mr.b_rows;
        const bool ok = T >= 1 && B >= 1 && T <= 0x7fffffffLL && B <= 0x7fffffffLL &&
                        (rows == 0 || rows % (T * B) == 0) && (mr.ld_b == 0 || mr.ld_b >= V) &&
                        (mr.ld_s == 0 || mr.ld_s >= V);
        if (!ok) {
            char buf[256];
            std::snprintf(buf, sizeof buf,
                          "%s: mask rows T %lld, B %lld, ld_b %lld, ld_s %lld for %lld rows of %lld (rows a multiple "
                          "of T B; strides 0 or at least vocab)",
                          who, (long long)T, (long long)B, (long long)mr.ld_b, (long long)mr.ld_s, (long long)rows,
                          (long long)V);
            return fail(NT_E_ARG, buf);
        }
        m = MaskMap{mask_ld, mr.ld_b, mr.ld_s, uint32_t(T), uint32_t(B)};
    }
    *out = m;
    return 0;
}

inline bool aligned_rows(const void *x, int64_t V, int64_t ld, int32_t dtype, int32_t mk, const void *mask,
                         const MaskMap &mm) {
    if (V % kEpl != 0 || ld % kEpl != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0) return false;
    (void)dtype;
    const auto strides = [&](int64_t u) { return mm.ld % u == 0 && mm.ld_b % u == 0 && mm.ld_s % u == 0; };
    if (mk == NT_MASK_U8) return strides(8) && reinterpret_cast<uintptr_t>(mask) % 8 == 0;
    if (mk == NT_MASK_F32) return strides(4) && reinterpret_cast<uintptr_t>(mask) % 16 == 0;
    return true;
}
#endif

}  // namespace
}  // namespace nt
