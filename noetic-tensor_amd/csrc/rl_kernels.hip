// Fused nn::rl vocabulary-row kernels for gfx950 (MI355X), and their C-ABI entry points.
//
// A row is one (s, b, t) position of logits [S, B, T, V] (src/nn/rl.rs:8-14). The reference
// runs every nn::rl function as a chain of generic tensor kernels (log_softmax = max_dim x2,
// sub, exp, sum_dim, log, sub; src/tensor/activation.rs:30-42), materialising [rows, V] about
// ten times per call. Here one workgroup streams one row once:
//
//  * Data layout: a row is cut into chunks of 512 elements (one wavefront x 8 elements per
//    lane, 16-byte loads for bf16, 2 x 16-byte loads for f32, 8-byte loads of the u8 mask).
//    Chunk c of a row is processed by wave c % nwaves, so every wave-wide load is a contiguous
//    1 KiB (bf16) / 2 KiB (f32) read and each wave keeps several chunks in flight.
//  * Arithmetic: f32 per element; bf16 is widened exactly by a shift. Exponentials are
//    exp2 of (v - shift) * c on the hardware v_exp_f32, where c = log2(e) / temperature folds
//    the temperature divide into the exponent (no per-element divide).
//  * Determinism: no atomics; every reduction (per lane, across a wave, across waves) has a
//    fixed order independent of timing, so reruns are bit-identical (the contract of
//    src/nn/tests/gpu/rl.rs:125-128).
//
// Sampler (nt_hip_rl_sample): each chunk's (max, sum of exp) goes to LDS; wave 0 then merges
// the chunk sums in index order in f64, finds the chunk holding u*S, re-reads only that chunk
// (512 elements, an L2 hit in practice) and scans it in f64. HBM traffic is one pass over the
// row plus one chunk.
//
// Scorer (nt_hip_rl_score): every lane keeps running (max, sum exp, sum exp*d, sum exp*(z-r))
// for the policy and (max, sum exp) for the reference, rescaled when its max grows (online
// log-sum-exp); waves and then the workgroup merge them in a fixed order; per-row scalars are
// finished in f64.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <string>
#include <type_traits>

#include "../../include/noetic_hip.h"
#include "nt_internal.hpp"

namespace nt {
namespace {

constexpr int kWave = 64;
constexpr int kEpl = 8;                  // elements per lane per chunk
constexpr int kChunk = kWave * kEpl;     // 512 elements per chunk
constexpr int kBatch = 4;                // chunks per wave with loads in flight together
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
                uint32_t h = in ? uint32_t(static_cast<const uint16_t *>(xrow)[e]) : 0xff80u;
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

// Logit j of a lane's chunk as f32 (bf16 widened exactly).
template <int DT>
__device__ __forceinline__ float logit(const uint32_t *x, int j) {
    if constexpr (DT == NT_F32) return __uint_as_float(x[j]);
    else return __uint_as_float((j % 2 == 0) ? (x[j / 2] << 16) : (x[j / 2] & 0xffff0000u));
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
        } else if (j % 2 == 1) {
            x[j / 2] = (__float_as_uint(v[j]) & 0xffff0000u) | (__float_as_uint(v[j - 1]) >> 16);
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

// ------------------------------------------------------------------ sampler

struct SampleP {
    const void *logits;
    const void *mask;
    int64_t V, ld, mask_ld;
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
};

template <int DT, int MK, bool ENT, bool AL>
__global__ __launch_bounds__(1024) void k_sample(SampleP p) {
    extern __shared__ float smem[];
    float *cmax = smem;                 // [nc] chunk max (value space)
    float *csum = smem + p.nc;          // [nc] chunk sum of exp2((v - cmax) c)
    float *cent = smem + 2 * p.nc;      // [nc] chunk sum of w * (v - cmax) c   (ENT only)
    const int64_t row = blockIdx.x;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int nw = blockDim.x / kWave;
    const bool tau_one = p.tau_one != 0;
    const void *xrow = static_cast<const char *>(p.logits) + row * p.ld * Elem<DT>::kBytes;
    const void *mrow = nullptr;
    if constexpr (MK != NT_MASK_NONE) mrow = static_cast<const char *>(p.mask) + row * p.mask_ld * MaskWords<MK>::kBytes;

    // ---- phase 1: stream the row once, per-chunk (max, sum exp[, sum exp * d]) into LDS.
    for (int c0 = wave; c0 < p.nc; c0 += nw * kBatch) {
        Raw<DT, MK> raw[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; b++) {
            const int c = c0 + b * nw;
            const int64_t e0 = int64_t(c < p.nc ? c : 0) * kChunk + lane * kEpl;
            load_raw<DT, MK, AL>(raw[b], xrow, mrow, c < p.nc ? e0 : p.V, p.V);
        }
#pragma unroll
        for (int b = 0; b < kBatch; b++) {
            const int c = c0 + b * nw;
            if (c < p.nc) {
            float v[kEpl];
            decode<DT, MK>(raw[b], v, p.tau, tau_one);
            const float cm = wave_max(max8(v));
            const float sh = (cm == -INFINITY) ? 0.0f : cm;
            float w[kEpl], h[kEpl];
#pragma unroll
            for (int j = 0; j < kEpl; j++) {
                const float d = (v[j] - sh) * p.c;
                w[j] = exp2_hw(d);
                if constexpr (ENT) h[j] = w[j] * fmaxf(d, -FLT_MAX);
            }
            const float cs = wave_sum(tree8(w));
            float ce = 0.0f;
            if constexpr (ENT) ce = wave_sum(tree8(h));
            if (lane == 0) {
                cmax[c] = cm;
                csum[c] = cs;
                if constexpr (ENT) cent[c] = ce;
            }
            }
        }
    }
    __syncthreads();
    if (wave != 0) return;

    // ---- phase 2 (wave 0): merge the chunks in index order, in f64.
    const int nc = p.nc;
    const int q = (nc + kWave - 1) / kWave;
    const int cb = min(lane * q, nc), ce_ = min(cb + q, nc);
    float lm = -INFINITY;
    for (int c = cb; c < ce_; c++) lm = fmaxf(lm, cmax[c]);
    const float a = wave_max(lm);
    auto refuse = [&](uint8_t st) {
        if (lane == 0) {
            p.ids[row] = -1;
            if (p.logp) p.logp[row] = NAN;
            if (p.ent) p.ent[row] = NAN;
            p.status[row] = st;
        }
    };
    if (a == -INFINITY) {
        refuse(NT_ROW_NO_TOKEN);
        return;
    }
    double lsum = 0.0, lh = 0.0;
    for (int c = cb; c < ce_; c++) {
        const float f = exp2_hw((cmax[c] - a) * p.c);
        lsum += double(f) * double(csum[c]);
        if constexpr (ENT) {
            if (csum[c] > 0.0f) lh += double(f) * (double(cent[c]) + double((cmax[c] - a) * p.c) * double(csum[c]));
        }
    }
    const double incl = wave_scan_d(lsum, lane);
    const double S = __shfl(incl, kWave - 1, kWave);
    double H2 = 0.0;
    if constexpr (ENT) H2 = wave_sum_d(lh);
    if (!(S == S)) {
        refuse(NT_ROW_NAN);
        return;
    }
    int cstar = -1;
    double tloc = 0.0;  // target inside chunk cstar, in the chunk's own scale
    if (p.greedy) {
        int mine = -1;
        for (int c = cb; c < ce_; c++)
            if (cmax[c] == a) { mine = c; break; }
        const int l = first_lane(__ballot(mine >= 0));
        cstar = l >= 0 ? __shfl(mine, l, kWave) : -1;
    } else {
        const double t = p.u[row] * S;
        // Every lane runs the shuffle: a disabled source lane would read as 0.
        const double prev = __shfl_up(incl, 1, kWave);
        const double excl = (lane == 0) ? 0.0 : prev;
        // Only a lane that holds weight can contain the crossing (a zero-weight lane's
        // inclusive sum may round above its neighbour's in the scan tree).
        int l = first_lane(__ballot(incl > t && lsum > 0.0));
        int mine = -1;
        double mt = INFINITY;
        if (l >= 0) {
            if (lane == l) {
                double C = excl;
                int lastpos = -1;
                for (int c = cb; c < ce_; c++) {
                    const float f = exp2_hw((cmax[c] - a) * p.c);
                    const double wt = double(f) * double(csum[c]);
                    if (wt > 0.0) lastpos = c;
                    if (C + wt > t) {
                        mine = c;
                        mt = (t - C) / double(f);
                        break;
                    }
                    C += wt;
                }
                if (mine < 0) mine = lastpos;  // rounding: no crossing inside the lane
            }
        } else {
            // u*S rounded up to S: the last chunk with weight.
            int lastpos = -1;
            for (int c = cb; c < ce_; c++)
                if (csum[c] > 0.0f && cmax[c] != -INFINITY) lastpos = c;
            l = last_lane(__ballot(lastpos >= 0));
            if (lane == l) mine = lastpos;
        }
        cstar = l >= 0 ? __shfl(mine, l, kWave) : -1;
        tloc = l >= 0 ? __shfl(mt, l, kWave) : INFINITY;
    }
    if (cstar < 0 || cstar >= nc) {
        // Unreachable with S > 0 (some chunk holds weight); kept so that no path re-reads
        // outside the row: take the first chunk holding the maximum.
        int mine = -1;
        for (int c = cb; c < ce_; c++)
            if (cmax[c] == a) { mine = c; break; }
        const int l = first_lane(__ballot(mine >= 0));
        cstar = l >= 0 ? __shfl(mine, l, kWave) : 0;
        tloc = INFINITY;
    }

    // ---- phase 3 (wave 0): re-read chunk cstar, find the token inside it.
    Raw<DT, MK> raw;
    const int64_t e0 = int64_t(cstar) * kChunk + lane * kEpl;
    load_raw<DT, MK, AL>(raw, xrow, mrow, e0, p.V);
    float v[kEpl];
    decode<DT, MK>(raw, v, p.tau, tau_one);
    int jsel = -1, lsel = -1;
    if (p.greedy) {
        int mine = -1;
#pragma unroll
        for (int j = kEpl - 1; j >= 0; j--)
            if (v[j] == a) mine = j;
        lsel = first_lane(__ballot(mine >= 0));
        jsel = lsel >= 0 ? __shfl(mine, lsel, kWave) : -1;
    } else {
        const float cm = cmax[cstar];
        const float sh = (cm == -INFINITY) ? 0.0f : cm;
        float w[kEpl];
        double ls = 0.0;
#pragma unroll
        for (int j = 0; j < kEpl; j++) {
            w[j] = exp2_hw((v[j] - sh) * p.c);
            ls += double(w[j]);
        }
        const double incl2 = wave_scan_d(ls, lane);
        const double prev2 = __shfl_up(incl2, 1, kWave);
        const double excl2 = (lane == 0) ? 0.0 : prev2;
        int mine = -1;
        int lastj = -1;
#pragma unroll
        for (int j = 0; j < kEpl; j++)
            if (w[j] > 0.0f) lastj = j;
        lsel = first_lane(__ballot(incl2 > tloc && ls > 0.0));
        if (lsel >= 0) {
            if (lane == lsel) {
                double C = excl2;
                for (int j = 0; j < kEpl; j++) {
                    C += double(w[j]);
                    if (C > tloc) { mine = j; break; }
                }
                if (mine < 0) mine = lastj;
            }
        } else {
            lsel = last_lane(__ballot(lastj >= 0));
            if (lane == lsel) mine = lastj;
        }
        jsel = lsel >= 0 ? __shfl(mine, lsel, kWave) : -1;
    }
    if (lsel < 0 || jsel < 0) {
        // Unreachable (chunk cstar holds weight, or the maximum when greedy); the first
        // element equal to the chunk's maximum keeps the result a valid token.
        int mine = -1;
#pragma unroll
        for (int j = kEpl - 1; j >= 0; j--)
            if (v[j] == cmax[cstar]) mine = j;
        lsel = first_lane(__ballot(mine >= 0));
        jsel = lsel >= 0 ? __shfl(mine, lsel, kWave) : 0;
        if (lsel < 0) lsel = 0;
    }
    if (lane == lsel) {
        // jsel indexes this lane's registers: select it without a dynamic register index.
        float vz = v[0];
#pragma unroll
        for (int j = 1; j < kEpl; j++)
            if (j == jsel) vz = v[j];
        const int64_t id = int64_t(cstar) * kChunk + lane * kEpl + jsel;
        // logp = (z_id - m) - ln S, with z_id - m the reference's f32 subtraction
        // (activation.rs:32-35).
        float zid = vz, mz = a;
        if constexpr (MK != NT_MASK_F32) {
            if (!tau_one) {
                zid = vz / p.tau;
                mz = a / p.tau;
            }
        }
        const double lnS = log(S);
        p.ids[row] = int32_t(id);
        if (p.logp) p.logp[row] = float((double(zid) - double(mz)) - lnS);
        if (p.ent) p.ent[row] = float(lnS - kLn2 * H2 / S);
        p.status[row] = NT_ROW_OK;
    }
}

// ------------------------------------------------------------------ register-resident sampler
//
// For rows of at most 16*K chunks (V <= 131072 for bf16 at K = 16) one 1024-thread workgroup
// keeps the whole row on chip: each wave's logit words stay in VGPRs (64 registers at K = 16)
// and the u8 mask is copied by the load unit straight into LDS (buffer_load ... lds, 128 KiB at
// K = 16), so nothing is read twice. Each wave issues chunk k + 1 while it processes chunk k,
// after decoding it (kRRWindow = 1): phase 1 is VALU-bound, and on MI355X that measured faster
// than two or three chunks ahead (17.40 against 17.57 and 18.27 us at c4, before the issue point
// moved into the chunk).
//
// Wave w owns the K consecutive chunks [w K, w K + K) of the row, so the index order of the
// row is the order of the waves, then of each wave's chunks.
// Phase 1 (all waves): as each chunk lands, w = 2^(v c - s) with s the wave's exponent
// reference (the maximum of its first chunk holding an allowed value; moved only when a chunk's
// weights overflow), so no exponential waits on a reduction. The chunk's sum of weights is a
// fixed-order DPP reduction written to LDS as four 16-lane partials. Each wave then takes the
// f64 prefix over its own chunks (kept in registers) and publishes its total.
// Phase 2 (every wave, after the one barrier): f64 scan over the 16 wave totals in index order,
// the wave whose chunks hold u*S. That wave alone goes on (no second barrier).
// Phase 3 (that wave): the crossing chunk from its prefix, then a scan of that chunk's registers.
// Measured at c4 against one 256-chunk scan by wave 0 and a second barrier: 20.2 against 20.6 us
// HBM-cold, 17.0-17.2 against 17.2-17.4 us cache-warm.

constexpr int kRRWaves = 16;
constexpr int kRRThreads = kRRWaves * kWave;
constexpr int kRRWindow = 1;  // chunks in flight ahead of the one being consumed

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

template <int DT, int MK, int K, bool ENT, int EPL>
__global__ __launch_bounds__(kRRThreads) void k_sample_rr(SampleP p) {
    constexpr int CH = kWave * EPL;                // elements per chunk
    constexpr int NCH = K * kRRWaves;
    constexpr int LX = RRX<DT, EPL>::kPieces;      // logit load instructions per chunk
    constexpr int LD = RRMask<MK, EPL>::kDma;      // mask DMA instructions per chunk
    constexpr int MB = RRMask<MK, EPL>::kBytes;    // mask bytes per chunk
    constexpr int DB = RRMask<MK, EPL>::kDmaBytes;
    constexpr int L = LX + LD;
    __shared__ __attribute__((aligned(16))) uint8_t mlds[MK == NT_MASK_NONE ? 16 : NCH * MB];
    __shared__ __attribute__((aligned(16))) float csum4[NCH * 4];  // per chunk and 16-lane row: sum of 2^(v c - wref)
    __shared__ __attribute__((aligned(16))) float cent4[ENT ? NCH * 4 : 4];  // per chunk and row: sum of w (v c - wref)
    __shared__ float wref[kRRWaves];    // per wave: its final exponent reference
    __shared__ float wmax[kRRWaves];    // per wave: its maximum (greedy) or its reference's source
    __shared__ double wtot[kRRWaves];   // per wave: its sum of weights, relative to its reference
    __shared__ double went[ENT ? kRRWaves : 1];  // per wave: its sum of w (v c - wref)
    __shared__ int wpick[kRRWaves];

    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int nc = p.nc;
    const float c = p.c;
    const bool tau_one = p.tau_one != 0;
    const void *xrow = static_cast<const char *>(p.logits) + row * p.ld * Elem<DT>::kBytes;
    const uint8_t *mrow = nullptr;
    if constexpr (MK != NT_MASK_NONE)
        mrow = static_cast<const uint8_t *>(p.mask) + row * p.mask_ld * MaskWords<MK>::kBytes;
    const uint32_t mbase = uint32_t((uintptr_t)(lds_ptr_t)(mlds));
    // The row's uniform, read now so that its latency hides under the row's loads.
    const double u_row = p.greedy ? 0.0 : p.u[row];

    // ---- loads: the first W chunks now, chunk k + W while chunk k is consumed.
    constexpr int W = K < kRRWindow ? K : kRRWindow;
    RRX<DT, EPL> raw[K];
    // Buffer resources over the row's logits and mask bytes: a read at or past the end returns
    // zeros (mask 0 = excluded), so chunks past the row need no address clamping. All of the
    // offset goes in the per-lane register, which the hardware range-checks.
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(xrow), short(0), int(p.V * Elem<DT>::kBytes), kBufferWord3);
    __amdgpu_buffer_rsrc_t mres;
    if constexpr (MK != NT_MASK_NONE)
        mres = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(mrow), short(0),
                                                 int(p.V * MaskWords<MK>::kBytes), kBufferWord3);
    auto issue = [&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const int ch = wave * K + k;
        const int xo = (ch * CH + lane * EPL) * Elem<DT>::kBytes;
#pragma unroll
        for (int q = 0; q < LX; q++) {
            // default cache policy: non-temporal loads leave the Infinity Cache unfilled, which
            // measured slower when a row is read again (19.4 against 17.1 us at c4) and no faster
            // HBM-cold
            const auto a = __builtin_amdgcn_raw_buffer_load_b128(xres, xo + 16 * q, 0, 0);
            raw[k].x[4 * q] = a[0];
            raw[k].x[4 * q + 1] = a[1];
            raw[k].x[4 * q + 2] = a[2];
            raw[k].x[4 * q + 3] = a[3];
        }
        if constexpr (MK != NT_MASK_NONE) {
            // The chunk's mask bytes, DB bytes per lane per instruction, into the chunk's slot
            // of mlds (lane l writes slot + DB l).
#pragma unroll
            for (int d = 0; d < LD; d++) {
                if constexpr (DB == 16)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(mres, (lds_ptr_t)(mlds + ch * MB + d * DB * kWave), 16,
                                                             ch * MB + d * DB * kWave + DB * lane, 0, 0, 0);
                else
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(mres, (lds_ptr_t)(mlds + ch * MB + d * DB * kWave), 4,
                                                             ch * MB + d * DB * kWave + DB * lane, 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    static_for<0, W>(issue);

    // ---- phase 1: each chunk as it lands. The wave's exponent reference is set from its first
    // chunk holding an allowed value (its exact maximum) and moves only when a chunk's weights
    // overflow (a weight or a lane sum of at least 2^128), to that chunk's maximum; the partials
    // already written are then rescaled. No maximum is taken per chunk otherwise.
    // Each chunk's row partial goes to csum4[4 ch + lane / 16]: a per-lane base, plus 256 bytes
    // per k (an immediate offset).
    float *const cpart = csum4 + 4 * K * wave + lane / 16;
    float *const epart = ENT ? cent4 + 4 * K * wave + lane / 16 : nullptr;
    const bool row_leader = (lane & 15) == 0;
    const int Vi = int(p.V);  // < 2^31 (at most 16 K chunks of CH)
    // This lane's mask bytes of the wave's chunk k: mlw + k MB.
    const uint32_t mlw = mbase + wave * K * MB + lane * EPL * MaskWords<MK>::kBytes;
    bool have_ref = false;     // sref set (uniform)
    float lmax = -INFINITY;    // the exact maximum, kept when greedy only
    float sref = -INFINITY;    // RN(sref_v c), uniform
    float sref_v = -INFINITY;  // the wave maximum the reference was taken from
    static_for<0, K>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const int ch = wave * K + k;
        if (ch < nc) {
            const int64_t e0 = int64_t(ch) * CH + lane * EPL;
            uint32_t mw[RRMask<MK, EPL>::kWords];
            if constexpr (MK != NT_MASK_NONE) {
                // Chunks k+1 .. min(K, k+W)-1 may still be in flight.
                wait_vmcnt<L * ((K < k + W ? K : k + W) - 1 - k)>();
                constexpr int kOff = k * MB;
                if constexpr (MK == NT_MASK_U8 && EPL == 8 && kOff < 65536) {
                    const uint2 m2 = lds_read_b64_off<kOff < 65536 ? kOff : 0>(mlw);
                    mw[0] = m2.x;
                    mw[1] = m2.y;
                } else {
                    lds_mask_words<MK, EPL>(mlw + kOff, mw);
                }
            } else {
                mw[0] = 0;
            }
            float v[EPL];
            decode_e<DT, MK, EPL>(raw[k].x, mw, v, p.tau, tau_one);
            if ((ch + 1) * CH > Vi) {  // only the row's last chunk can be partial
#pragma unroll
                for (int j = 0; j < EPL; j++)
                    if (e0 + j >= p.V) v[j] = -INFINITY;
            }
            // The next chunk's loads go out once this chunk's data is in registers: between one
            // and two chunks in flight per wave (measured faster than issuing after the chunk,
            // 17.11 against 17.38 us at c4, and than two whole chunks ahead).
            if constexpr (k + W < K) issue(std::integral_constant<int, k + W>{});
            if (p.greedy) {
                const float m8 = max_hw<EPL>(v);
                lmax = max3_hw(lmax, m8, m8);
            }
            if (!have_ref) {
                const float wm = wave_max3_dpp(max_hw<EPL>(v));
                if (wm != -INFINITY) {
                    have_ref = true;
                    sref_v = wm;
                    sref = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(wm * c)));
                }
            }
            float gs = 0.0f, gh = 0.0f;
            auto weigh = [&]() {
                float w[EPL], h[EPL];
#pragma unroll
                for (int j = 0; j < EPL; j++) {
                    const float d = fmaf(v[j], c, -sref);
                    w[j] = exp2_hw(d);
                    if constexpr (ENT) h[j] = w[j] * fmaxf(d, -FLT_MAX);
                }
                gs = tree_sum<EPL>(w);
                if constexpr (ENT) gh = tree_sum<EPL>(h);
            };
            if (have_ref) {
                weigh();
                // An overflow (or a NaN, which compares false below and stays in the sums) moves
                // the wave's reference to the chunk's maximum. With the entropy wanted, so does a
                // lane's 8 weights summing to more than kChunkSumCap: the entropy is ln S - ln2 H / S,
                // and a reference far below the maximum would make both terms large and cancelling.
                bool move = !(gs < INFINITY);
                if constexpr (ENT) move = !(gs <= kChunkSumCap);
                if (__ballot(move) != 0) {
                    const float wm = wave_max3_dpp(max_hw<EPL>(v));
                    const float nref = wm * c;
                    if (nref > sref) {
                        const float dk = sref - nref, f = exp2_hw(dk);
                        if ((lane & 15) == 0) {
                            // this wave's earlier partials, owned by lanes 0, 16, 32, 48
                            static_for<0, k>([&](auto jc) {
                                constexpr int kk = decltype(jc)::value;
                                const int idx = (wave * K + kk) * 4 + lane / 16;
                                const float o = csum4[idx];
                                csum4[idx] = f * o;
                                if constexpr (ENT) cent4[idx] = f * (cent4[idx] + dk * o);
                            });
                        }
                        sref = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(nref)));
                        sref_v = wm;
                        weigh();
                    }
                }
            }
            // The chunk's four 16-lane row sums (phase 2 adds them in a fixed order).
            const float cs = row_sum_dpp(gs);
            float ce = 0.0f;
            if constexpr (ENT) ce = row_sum_dpp(gh);
            if (row_leader) {
                cpart[4 * k] = cs;
                if constexpr (ENT) epart[4 * k] = ce;
            }
        }
        if constexpr (k + W < K) {
            if (!(ch < nc)) issue(std::integral_constant<int, k + W>{});  // (no chunk here to process)
        }
    });
    // ---- end of phase 1 (each wave on its own, while the others still stream): lane k < K
    // takes chunk k's sum (its four 16-lane partials, in a fixed order) in f64, in the wave's
    // scale; the f64 prefix over the wave's chunks stays in registers and the wave's totals go
    // to LDS.
    double wcs = 0.0, wce = 0.0;
    {
        const int ch = wave * K + lane;
        if (lane < K && ch < nc) {
            const float4 q = *reinterpret_cast<const float4 *>(csum4 + 4 * ch);
            wcs = double((q.x + q.y) + (q.z + q.w));
            if constexpr (ENT) {
                const float4 e = *reinterpret_cast<const float4 *>(cent4 + 4 * ch);
                wce = double((e.x + e.y) + (e.z + e.w));
            }
        }
    }
    const double wincl = row_scan_dpp(wcs);  // lane k < 16: the wave's sum through its chunk k
    {
        // the wave's maximum when greedy; otherwise the value its reference came from (a lower
        // bound of its maximum: every sum is taken relative to RN(value c))
        const float wm = p.greedy ? wave_max3_dpp(lmax) : sref_v;
        double wh = 0.0;
        if constexpr (ENT) wh = row_scan_dpp(wce);
        if (lane == kRRWaves - 1) {
            wtot[wave] = wincl;
            if constexpr (ENT) went[wave] = wh;
        }
        if (lane == 0) {
            wmax[wave] = wm;
            wref[wave] = sref;
        }
    }
    __syncthreads();

    // ---- phase 2 (every wave, to the same bits): lane w of each 16-lane row takes wave w's
    // totals. The row's reference value M (the largest wave reference; the exact maximum when
    // greedy), the row's sums relative to A = M c by an f64 scan over the waves in index order,
    // and the wave whose chunks hold u S. No second barrier: that wave goes on alone.
    const int lw = lane & (kRRWaves - 1);
    const float rw = wref[lw];
    const double tw = wtot[lw];
    double hw = 0.0;
    if constexpr (ENT) hw = went[lw];
    const float M = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(row_max3_dpp(wmax[lw]))));
    auto refuse = [&](uint8_t st, bool leader) {
        if (leader) {
            p.ids[row] = -1;
            if (p.logp) p.logp[row] = NAN;
            if (p.ent) p.ent[row] = NAN;
            p.status[row] = st;
        }
    };
    if (M == -INFINITY) {
        refuse(NT_ROW_NO_TOKEN, tid == 0);
        return;
    }
    const float A = M * c;  // >= every wave reference (rounding is monotonic)
    const bool wlive = rw != -INFINITY;
    const float wf = wlive ? exp2_hw(rw - A) : 0.0f;
    const double wt = wlive ? double(wf) * tw : 0.0;
    const double incl = row_scan_dpp(wt);
    const double S = readlane_d(incl, kRRWaves - 1);
    if (!(S == S)) {
        refuse(NT_ROW_NAN, tid == 0);
        return;
    }
    // The entropy sum relative to A, taken only by the wave that writes the row (every wave
    // works this phase on the same values, four to a SIMD, so it holds no more than it needs).
    auto entropy_sum = [&]() -> double {
        if constexpr (!ENT) return 0.0;
        const double lh = (wlive && tw > 0.0) ? double(wf) * (hw + double(rw - A) * tw) : 0.0;
        return readlane_d(row_scan_dpp(lh), kRRWaves - 1);
    };
    // ln sum exp(z - m) and the entropy, from the sums relative to A = M c (computed by the
    // one lane that writes the row).
    auto write_row = [&](int64_t id, float vz, double H) {
        const double shiftA = double(A) - double(M) * double(c);
        const double lnS = ln_fast(S) + shiftA * kLn2;
        const bool zv = MK == NT_MASK_F32 || tau_one;
        const float zid = zv ? vz : vz / p.tau;
        const float mz = zv ? M : M / p.tau;  // the maximum in z units
        p.ids[row] = int32_t(id);
        if (p.logp) p.logp[row] = float((double(zid) - double(mz)) - lnS);
        if (p.ent) p.ent[row] = float(lnS - kLn2 * (H / S + shiftA));
        p.status[row] = NT_ROW_OK;
    };
    // Decode chunk k of this wave again (the mask from LDS; every DMA has completed).
    auto chunk_values = [&](const RRX<DT, EPL> &r, int ch, float *v) {
        uint32_t mw[RRMask<MK, EPL>::kWords];
        lds_mask_words<MK, EPL>(mbase + ch * MB + lane * EPL * MaskWords<MK>::kBytes, mw);
        decode_e<DT, MK, EPL>(r.x, mw, v, p.tau, tau_one);
        if (int64_t(ch + 1) * CH > p.V) {
            const int64_t e0 = int64_t(ch) * CH + lane * EPL;
#pragma unroll
            for (int j = 0; j < EPL; j++)
                if (e0 + j >= p.V) v[j] = -INFINITY;
        }
    };

    if (p.greedy) {
        // The first element equal to the maximum, in index order.
        int first = 0x7fffffff;
        static_for<0, K>([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            const int ch = wave * K + k;
            if (ch < nc) {
                float v[EPL];
                chunk_values(raw[k], ch, v);
#pragma unroll
                for (int j = EPL - 1; j >= 0; j--)
                    if (v[j] == M) first = min(first, ch * CH + lane * EPL + j);
            }
        });
        first = wave_min_i(first);
        if (lane == 0) wpick[wave] = first;
        __syncthreads();
        int best = 0x7fffffff;
        for (int i = 0; i < kRRWaves; i++) best = min(best, wpick[i]);
        const double H = entropy_sum();
        if (tid == 0) write_row(best, M, H);
        return;
    }

    // The wave whose chunks hold t = u S: the first with its inclusive sum past t.
    const double t = u_row * S;
    const bool wl = lane < kRRWaves;
    int wsel = first_lane(__ballot(wl && incl > t && wt > 0.0));
    if (wsel < 0) wsel = last_lane(__ballot(wl && wt > 0.0));  // u S rounded up to S
    if (wsel < 0) {  // unreachable: M's wave has weight; never leave stale outputs
        refuse(NT_ROW_NAN, tid == 0);
        return;
    }
    if (wave != wsel) return;
    // ---- phase 3 (that wave alone): the target in its own scale (the part of t past the waves
    // before it, divided by 2^(s - A)), the crossing chunk from the prefix held since phase 1,
    // then that chunk's registers.
    const double tl = readlane_d((t - (incl - wt)) * double(exp2_hw(A - rw)), wsel);
    const bool lk = lane < K;
    int kstar = first_lane(__ballot(lk && wincl > tl && wcs > 0.0));
    if (kstar < 0) kstar = last_lane(__ballot(lk && wcs > 0.0));  // rounding between the two scans
    if (kstar < 0) {  // unreachable: the wave has weight
        refuse(NT_ROW_NAN, lane == 0);
        return;
    }
    const double tloc = readlane_d(tl - (wincl - wcs), kstar);
    const int cstar = wave * K + kstar;
    const double H = entropy_sum();
    RRX<DT, EPL> r = raw[0];
    static_for<1, K>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        if (k == kstar) r = raw[k];
    });
    float v[EPL];
    chunk_values(r, cstar, v);
    const float sr = sref;
    float w[EPL];
    int jlast = -1;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        w[j] = exp2_hw(fmaf(v[j], c, -sr));
        if (w[j] > 0.0f) jlast = j;
    }
    const double ls = double(tree_sum<EPL>(w));
    const double cincl = wave_scan_dpp(ls);
    int lsel = first_lane(__ballot(cincl > tloc && ls > 0.0));
    const bool none = lsel < 0;
    if (none) lsel = last_lane(__ballot(jlast >= 0));  // rounding: the last lane with weight
    if (lsel < 0) {  // unreachable: the chunk holds weight
        refuse(NT_ROW_NAN, lane == 0);
        return;
    }
    // The crossing lane walks its elements from the prefix before them (f32 partial sums
    // inside the lane, compared against the f64 target).
    int jsel = -1;
    {
        const double t0 = tloc - (cincl - ls);
        float C = 0.0f;
#pragma unroll
        for (int j = 0; j < EPL; j++) {
            C += w[j];
            if (jsel < 0 && !none && double(C) > t0) jsel = j;
        }
        if (jsel < 0) jsel = jlast;
    }
    if (lane == lsel) {
        if (jsel < 0) jsel = 0;
        float vz = v[0];
#pragma unroll
        for (int j = 1; j < EPL; j++)
            if (j == jsel) vz = v[j];
        write_row(int64_t(cstar) * CH + lane * EPL + jsel, vz, H);
    }
}

// ------------------------------------------------------------------ scorer

struct ScoreP {
    const void *logits;
    const void *ref;
    const void *mask;
    int64_t V, ld, mask_ld;
    float c;
    float tau;
    int tau_one;
    int nc;
    const int32_t *tokens;
    float *logp, *ref_logp, *kl, *ent;
    uint8_t *status;
    float *lse_base, *lse_rest, *ref_lse_base, *ref_lse_rest;
};

// Running state of one lane (value space, exponent scale c). Every sum is relative to the
// lane's running maxima, so no term cancels against another of size |logit|:
//   S  = sum w,                 w = exp2((v - a) c)
//   H  = sum w (v - a) c                                  (entropy)
//   B  = sum w ((v - a) - (v_ref - a_ref)) c              (exact KL)
//   Sr = sum exp2((v_ref - a_ref) c)                      (reference normaliser)
struct RowState {
    float a, S, H, B;
    float ar, Sr;
};

__device__ __forceinline__ float shift_of(float a) { return a == -INFINITY ? 0.0f : a; }

// The B update when the maxima move by d = (a_old - a_new) c and e = (a_ref_old - a_ref_new) c:
// B' = f (B + (d - e) S). A state with S == 0 holds no policy term.
__device__ __forceinline__ float b_rescaled(float B, float S, float f, float d, float e) {
    return S > 0.0f ? f * (B + (d - e) * S) : 0.0f;
}

// Merge state o into s (the same arithmetic whichever side is s).
template <bool REF, bool KL, bool ENT>
__device__ __forceinline__ void state_merge(RowState &s, const RowState &o, float c) {
    const float an = fmaxf(s.a, o.a), sh = shift_of(an);
    const float d1 = (s.a - sh) * c, d2 = (o.a - sh) * c;
    const float f1 = exp2_hw(d1), f2 = exp2_hw(d2);
    float e1 = 0.0f, e2 = 0.0f;
    if constexpr (REF) {
        const float anr = fmaxf(s.ar, o.ar), shr = shift_of(anr);
        e1 = (s.ar - shr) * c;
        e2 = (o.ar - shr) * c;
        s.Sr = exp2_hw(e1) * s.Sr + exp2_hw(e2) * o.Sr;
        s.ar = anr;
    }
    if constexpr (ENT) s.H = f1 * (s.H + fmaxf(d1, -FLT_MAX) * s.S) + f2 * (o.H + fmaxf(d2, -FLT_MAX) * o.S);
    if constexpr (KL) s.B = b_rescaled(s.B, s.S, f1, d1, e1) + b_rescaled(o.B, o.S, f2, d2, e2);
    s.S = f1 * s.S + f2 * o.S;
    s.a = an;
}

__device__ __forceinline__ RowState shfl_down_state(const RowState &s, int o) {
    RowState r;
    r.a = __shfl_down(s.a, o, kWave);
    r.S = __shfl_down(s.S, o, kWave);
    r.H = __shfl_down(s.H, o, kWave);
    r.B = __shfl_down(s.B, o, kWave);
    r.ar = __shfl_down(s.ar, o, kWave);
    r.Sr = __shfl_down(s.Sr, o, kWave);
    return r;
}

constexpr int kScoreThreads = 256;
constexpr int kScoreWaves = kScoreThreads / kWave;

// load_raw for aligned rows through per-row buffer resources (row bytes below 2^31), no bounds
// branch, 32-bit offsets, non-temporal (every input is read once). Past the row's end the
// hardware range check returns zeros (the caller excludes those lanes). A lane's elements in a
// 512-element chunk at c: bf16 c + 8l .. c + 8l + 7 (one 16-byte load per input); f32 two groups,
// c + 4l .. c + 4l + 3 and c + 256 + 4l .. c + 256 + 4l + 3, so that each 16-byte load
// instruction reads one contiguous kilobyte rather than every other 16 bytes of two (measured
// faster with non-temporal loads). e0 is the lane's first element; each group lies wholly inside
// the row or wholly past its end (V % 8 == 0).
template <int DT>
__device__ __forceinline__ int buf_lane_first(int chunk, int lane) {
    return chunk * kChunk + lane * (DT == NT_F32 ? 4 : kEpl);
}

template <int DT, int MK>
__device__ __forceinline__ void load_raw_buf(Raw<DT, MK> &r, __amdgpu_buffer_rsrc_t xres,
                                             __amdgpu_buffer_rsrc_t mres, int e0) {
    constexpr int kHalf = kChunk / 2;
    if constexpr (DT == NT_F32) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const auto a = __builtin_amdgcn_raw_buffer_load_b128(xres, (e0 + q * kHalf) * 4, 0, kCachePolicyNT);
            for (int i = 0; i < 4; i++) r.x[4 * q + i] = a[i];
        }
        if constexpr (MK == NT_MASK_U8) {
            r.m[0] = __builtin_amdgcn_raw_buffer_load_b32(mres, e0, 0, kCachePolicyNT);
            r.m[1] = __builtin_amdgcn_raw_buffer_load_b32(mres, e0 + kHalf, 0, kCachePolicyNT);
        } else if constexpr (MK == NT_MASK_F32) {
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const auto a = __builtin_amdgcn_raw_buffer_load_b128(mres, (e0 + q * kHalf) * 4, 0, kCachePolicyNT);
                for (int i = 0; i < 4; i++) r.m[4 * q + i] = a[i];
            }
        } else {
            r.m[0] = 0;
        }
    } else {
        const auto a = __builtin_amdgcn_raw_buffer_load_b128(xres, e0 * 2, 0, kCachePolicyNT);
        for (int i = 0; i < 4; i++) r.x[i] = a[i];
        if constexpr (MK == NT_MASK_U8) {
            const auto k = __builtin_amdgcn_raw_buffer_load_b64(mres, e0, 0, kCachePolicyNT);
            r.m[0] = k[0];
            r.m[1] = k[1];
        } else if constexpr (MK == NT_MASK_F32) {
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const auto a = __builtin_amdgcn_raw_buffer_load_b128(mres, e0 * 4 + 16 * q, 0, kCachePolicyNT);
                for (int i = 0; i < 4; i++) r.m[4 * q + i] = a[i];
            }
        } else {
            r.m[0] = 0;
        }
    }
}


template <int DT, int MK, bool REF, bool KL, bool ENT, bool AL>
__global__ __launch_bounds__(kScoreThreads) void k_score(ScoreP p) {
    __shared__ RowState ws[kScoreWaves];
    const int64_t row = blockIdx.x;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int nw = blockDim.x / kWave;
    const bool tau_one = p.tau_one != 0;
    const float c = p.c;
    const void *xrow = static_cast<const char *>(p.logits) + row * p.ld * Elem<DT>::kBytes;
    const void *yrow = nullptr;
    if constexpr (REF) yrow = static_cast<const char *>(p.ref) + row * p.ld * Elem<DT>::kBytes;
    const void *mrow = nullptr;
    if constexpr (MK != NT_MASK_NONE) mrow = static_cast<const char *>(p.mask) + row * p.mask_ld * MaskWords<MK>::kBytes;

    // (used by the aligned path only, whose rows are below 2^31 bytes)
    const int Vb = AL ? int(p.V) : 0;
    const __amdgpu_buffer_rsrc_t xres =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(xrow), short(0), Vb * Elem<DT>::kBytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t yres =
        REF ? __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(yrow), short(0), Vb * Elem<DT>::kBytes, kBufferWord3)
            : xres;
    const __amdgpu_buffer_rsrc_t mres =
        MK != NT_MASK_NONE ? __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(mrow), short(0),
                                                               Vb * MaskWords<MK>::kBytes, kBufferWord3)
                           : xres;

    RowState st{-INFINITY, 0.0f, 0.0f, 0.0f, -INFINITY, 0.0f};
    for (int c0 = wave; c0 < p.nc; c0 += nw * kBatch) {
        Raw<DT, MK> rx[kBatch];
        Raw<DT, NT_MASK_NONE> ry[REF ? kBatch : 1];
#pragma unroll
        for (int b = 0; b < kBatch; b++) {
            const int ch = c0 + b * nw;
            if constexpr (AL) {
                const int e0 = ch < p.nc ? buf_lane_first<DT>(ch, lane) : int(p.V);
                load_raw_buf<DT, MK>(rx[b], xres, mres, e0);
                if constexpr (REF) load_raw_buf<DT, NT_MASK_NONE>(ry[b], yres, mres, e0);
            } else {
                const int64_t e0 = ch < p.nc ? int64_t(ch) * kChunk + lane * kEpl : p.V;
                load_raw<DT, MK, AL>(rx[b], xrow, mrow, e0, p.V);
                if constexpr (REF) load_raw<DT, NT_MASK_NONE, AL>(ry[b], yrow, nullptr, e0, p.V);
            }
        }
#pragma unroll
        for (int b = 0; b < kBatch; b++) {
            const int ch = c0 + b * nw;
            if (ch < p.nc) {
                float v[kEpl], vr[kEpl];
                decode<DT, MK>(rx[b], v, p.tau, tau_one);
                // The reference logits take the same temperature and vocabulary mask
                // (reference_kl, rl.rs:347-351).
                if constexpr (REF) decode_words<DT, MK>(ry[b].x, rx[b].m, vr, p.tau, tau_one);
                if constexpr (AL) {
                    // buffer loads past the row's end read zeros: only the last chunk can hold such
                    // element groups, which take no part in the sums
                    if (ch == p.nc - 1) {
                        const int e0 = buf_lane_first<DT>(ch, lane);
#pragma unroll
                        for (int j = 0; j < kEpl; j++) {
                            const int e = DT == NT_F32 ? e0 + (j < 4 ? j : kChunk / 2 + j - 4) : e0 + j;
                            if (e >= int(p.V)) {
                                v[j] = -INFINITY;
                                vr[j] = -INFINITY;
                            }
                        }
                    }
                }
                // The chunk's weights against the lane's current references. A reference is set
                // at the first chunk with a finite value and moves (the sums are rescaled and
                // the chunk weighed again) to the chunk's maximum whenever the lane's 8 weights
                // of one chunk sum to more than kChunkSumCap: then no weight exceeds kChunkSumCap,
                // so the reference trails the lane's maximum by at most log2 kChunkSumCap, the
                // sums cannot overflow, and the finishing differences (ln S - ln2 H / S for the
                // entropy, ln S - ln S_ref for the KL) stay small: no two terms of the size of the
                // logits cancel. (A NaN fails the test too, and stays in the sums.)
                auto rescale = [&](bool pol, bool rf, float an, float anr) {
                    float dold = 0.0f, eold = 0.0f, f = 1.0f;
                    if (pol) {
                        an = fmaxf(an, st.a);
                        dold = (st.a - shift_of(an)) * c;
                        f = exp2_hw(dold);
                        st.a = an;
                    }
                    if constexpr (REF) {
                        if (rf) {
                            anr = fmaxf(anr, st.ar);
                            eold = (st.ar - shift_of(anr)) * c;
                            st.Sr = exp2_hw(eold) * st.Sr;
                            st.ar = anr;
                        }
                    }
                    if constexpr (ENT) st.H = f * (st.H + fmaxf(dold, -FLT_MAX) * st.S);
                    if constexpr (KL) st.B = b_rescaled(st.B, st.S, f, dold, eold);
                    st.S = f * st.S;
                };
                float S, H, Bk, Sr;
                auto accumulate = [&]() {
                    const float sh = shift_of(st.a);
                    float shr = 0.0f;
                    if constexpr (REF) shr = shift_of(st.ar);
                    S = st.S, H = st.H, Bk = st.B, Sr = st.Sr;
#pragma unroll
                    for (int j = 0; j < kEpl; j++) {
                        const float d = (v[j] - sh) * c;
                        const float w = exp2_hw(d);
                        S += w;
                        if constexpr (ENT) H = fmaf(w, fmaxf(d, -FLT_MAX), H);
                        if constexpr (REF) {
                            const float e = (vr[j] - shr) * c;
                            Sr += exp2_hw(e);
                            if constexpr (KL) Bk = fmaf(w, fmaxf(d - e, -FLT_MAX), Bk);
                        }
                    }
                };
                // A lane's first reference is the maximum of the wave's whole chunk (512 values),
                // which makes later moves rare. (A wave-uniform branch: every lane takes part in
                // the DPP maxima.)
                if (__ballot(st.a == -INFINITY || (REF && st.ar == -INFINITY)) != 0) {
                    const float wm = wave_max3_dpp(max8_hw(v));
                    float wmr = -INFINITY;
                    if constexpr (REF) wmr = wave_max3_dpp(max8_hw(vr));
                    const bool pol = st.a == -INFINITY, rf = REF && st.ar == -INFINITY;
                    if (pol || rf) rescale(pol, rf, wm, wmr);
                }
                accumulate();
                {
                    // the chunk's weight sums (to within rounding, enough for the test)
                    const bool pol = !(S - st.S <= kChunkSumCap), rf = REF && !(Sr - st.Sr <= kChunkSumCap);
                    if (pol || rf) {
                        rescale(pol, rf, max8_hw(v), REF ? max8_hw(vr) : -INFINITY);
                        accumulate();
                    }
                }
                st.S = S;
                if constexpr (ENT) st.H = H;
                if constexpr (KL) st.B = Bk;
                if constexpr (REF) st.Sr = Sr;
            }
        }
    }
    // Wave tree (lane i takes lane i + o), then the waves in order.
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
        const RowState t = shfl_down_state(st, o);
        if (lane < o) state_merge<REF, KL, ENT>(st, t, c);
    }
    if (lane == 0) ws[wave] = st;
    __syncthreads();
    if (threadIdx.x != 0) return;

    // Finish the row in f64.
    float af = -INFINITY, arf = -INFINITY;
    for (int i = 0; i < nw; i++) {
        af = fmaxf(af, ws[i].a);
        arf = fmaxf(arf, ws[i].ar);
    }
    double S = 0.0, H = 0.0, B = 0.0, Sr = 0.0;
    for (int i = 0; i < nw; i++) {
        if (ws[i].S > 0.0f) {
            const double d = double(ws[i].a - af) * double(c);
            const double f = exp2(d);
            S += f * double(ws[i].S);
            if (ENT) H += f * (double(ws[i].H) + d * double(ws[i].S));
            if (KL) {
                const double e = ws[i].ar == -INFINITY ? -INFINITY : double(ws[i].ar - arf) * double(c);
                B += f * (double(ws[i].B) + (d - e) * double(ws[i].S));
            }
        } else if (!(ws[i].S == ws[i].S)) {
            S = NAN;
        }
        if (REF && ws[i].ar != -INFINITY) Sr += exp2(double(ws[i].ar - arf) * double(c)) * double(ws[i].Sr);
    }
    int stt = NT_ROW_OK;
    if (af == -INFINITY) stt = NT_ROW_NO_TOKEN;
    else if (!(S == S)) stt = NT_ROW_NAN;
    const double lnS = log(S);
    // The value-space max as the reference's f32 max of the tempered logits.
    auto zmax = [&](float a) -> float {
        if constexpr (MK != NT_MASK_F32) return tau_one ? a : a / p.tau;
        else return a;
    };
    // The tempered logit of one token, with the reference's f32 arithmetic.
    auto ztok = [&](const void *rowp, int64_t tok) -> float {
        float x;
        if constexpr (DT == NT_F32) x = static_cast<const float *>(rowp)[tok];
        else x = __uint_as_float(uint32_t(static_cast<const uint16_t *>(rowp)[tok]) << 16);
        float z = tau_one ? x : x / p.tau;
        if constexpr (MK == NT_MASK_U8) {
            if (static_cast<const uint8_t *>(mrow)[tok] == 0) z = -INFINITY;
        } else if constexpr (MK == NT_MASK_F32) {
            z = z + static_cast<const float *>(mrow)[tok];
        }
        return z;
    };
    int64_t tok = -1;
    if (p.tokens) {
        tok = p.tokens[row];
        if ((tok < 0 || tok >= p.V) && stt == NT_ROW_OK) stt = kRowBadToken;
    }
    const bool rowok = stt == NT_ROW_OK || stt == kRowBadToken;
    if (p.logp) p.logp[row] = stt == NT_ROW_OK ? float((double(ztok(xrow, tok)) - double(zmax(af))) - lnS) : NAN;
    if (p.ent) p.ent[row] = rowok ? float(lnS - kLn2 * H / S) : NAN;
    // The log-sum-exp as base + rest (z units): the base is the tempered value of the row's
    // final reference, the rest ln of the sum relative to it.
    if (p.lse_base) p.lse_base[row] = rowok ? zmax(af) : NAN;
    if (p.lse_rest) p.lse_rest[row] = rowok ? float(lnS) : NAN;
    if constexpr (REF) {
        const bool rok = arf != -INFINITY && Sr == Sr;
        if (p.ref_lse_base) p.ref_lse_base[row] = rok ? zmax(arf) : NAN;
        if (p.ref_lse_rest) p.ref_lse_rest[row] = rok ? float(log(Sr)) : NAN;
        if (p.ref_logp)
            p.ref_logp[row] = (rok && tok >= 0 && tok < p.V) ? float((double(ztok(yrow, tok)) - double(zmax(arf))) - log(Sr)) : NAN;
        if constexpr (KL) {
            // KL = sum p ((z - m) - (z_ref - m_ref)) - ln S + ln S_ref; the first sum is
            // ln2 * B / S because c ln2 is the value-to-logit scale (1/T, or 1 with an f32 mask).
            if (p.kl) p.kl[row] = (rowok && rok) ? float(kLn2 * B / S - log(S / Sr)) : NAN;
        }
    }
    if (p.status) p.status[row] = uint8_t(stt);
}

// ------------------------------------------------------------------ fused backward
//
// dL/dz_v = [v == token] g_logp - pi_v (A + B log pi_v + C log pi_ref,v) with A = g_logp +
// g_kl KL + g_H H, B = g_H - g_kl, C = g_kl (the sum of the three row gradients), and
// dL/dx_v = dL/dz_v / T. The kernel works in base 2: with l_v = log2 pi_v and r_v = log2 pi_ref,v,
// dL/dx_v = [v == token] g_logp / T - pi_v (A' + B' l_v + C' r_v), where A' = A / T,
// B' = B ln2 / T and C' = C ln2 / T are per-row constants. l_v is clamped at -256: an excluded
// (-inf) logit then has pi_v = 0 and a finite sum, so its gradient is exactly zero without a
// select. A refused row (NaN statistics) sets A' to NaN, which makes the whole row NaN, as the
// op sequence's log_softmax does. One block per row; each lane streams 8 elements per step,
// two steps in flight.

struct GradP {
    const void *logits, *ref, *mask;
    int64_t V, ld, mask_ld, gld;
    float tau;
    int tau_one;
    const int32_t *tokens;
    const float *lb, *lr, *rlb, *rlr, *kl, *ent, *glp, *gkl, *gh;
    void *grad;
};

constexpr int kGradThreads = 256;
constexpr int kGradStep = kGradThreads * kEpl;  // elements a block covers per step

// f32 pair -> packed bf16 pair, round to nearest even (lo from a, hi from b).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    uint32_t r;
    asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// The per-row constants of the backward (see above).
struct GradRow {
    float lb, l2, rlb, r2, A, B, C, gtok;
    int64_t tok;
};

template <bool KL>
__device__ __forceinline__ GradRow grad_row(const GradP &p, int64_t row) {
    GradRow g;
    const float inv_tau = p.tau_one ? 1.0f : 1.0f / p.tau;
    const float glp = p.glp ? p.glp[row] : 0.0f;
    const float gh = p.gh ? p.gh[row] : 0.0f;
    const float hv = p.gh ? p.ent[row] : 0.0f;
    float gkl = 0.0f, klv = 0.0f;
    g.lb = p.lb[row];
    const float lr = p.lr[row];
    g.l2 = lr * kLog2e;
    g.rlb = 0.0f;
    g.r2 = 0.0f;
    bool refused = !(g.lb == g.lb) || !(lr == lr);
    if constexpr (KL) {
        gkl = p.gkl[row];
        klv = p.kl[row];
        g.rlb = p.rlb[row];
        const float rlr = p.rlr[row];
        g.r2 = rlr * kLog2e;
        refused = refused || !(g.rlb == g.rlb) || !(rlr == rlr);
    }
    const float A = glp + (KL ? gkl * klv : 0.0f) + (p.gh ? gh * hv : 0.0f);
    g.A = refused ? __builtin_nanf("") : A * inv_tau;
    g.B = (gh - gkl) * float(kLn2) * inv_tau;
    g.C = gkl * float(kLn2) * inv_tau;
    g.gtok = glp * inv_tau;
    g.tok = p.glp ? int64_t(p.tokens[row]) : -1;
    return g;
}

// One element's gradient from its tempered logit z (and reference zr).
template <bool KL>
__device__ __forceinline__ float grad_elem(const GradRow &g, float z, float zr) {
    const float l = fmaxf(fmaf(z - g.lb, kLog2e, -g.l2), -256.0f);
    const float pi = exp2_hw(l);
    float t = fmaf(g.B, l, g.A);
    if constexpr (KL) {
        const float r = fmaxf(fmaf(zr - g.rlb, kLog2e, -g.r2), -256.0f);
        t = fmaf(g.C, r, t);
    }
    return fmaf(-pi, t, 0.0f);
}

// The tempered logit as tempered_logits computes it: x / T (an f32 divide), then the mask.
template <int MK, bool TAU1>
__device__ __forceinline__ float grad_tempered(float x, float tau, uint32_t mword, int j) {
    float z = TAU1 ? x : x / tau;
    if constexpr (MK == NT_MASK_U8) {
        if (((mword >> (8 * (j % 4))) & 0xffu) == 0) z = -INFINITY;
    } else if constexpr (MK == NT_MASK_F32) {
        z = z + __uint_as_float(mword);
    }
    return z;
}

// The token's own term, in the one lane (of one step) that holds it. A lane's 8 elements are
// e0 + j, or with SPLIT two groups of 4: e0 + j (j < 4) and e1 + j - 4 (j >= 4).
template <bool SPLIT>
__device__ __forceinline__ void add_token_term(const GradRow &g, int64_t e0, int64_t e1, float *out) {
    const int64_t d = g.tok - e0;
    if (static_cast<uint64_t>(d) < uint64_t(SPLIT ? 4 : kEpl)) {
#pragma unroll
        for (int j = 0; j < (SPLIT ? 4 : kEpl); j++) out[j] += (j == int(d)) ? g.gtok : 0.0f;
    }
    if constexpr (SPLIT) {
        const int64_t d1 = g.tok - e1;
        if (static_cast<uint64_t>(d1) < 4u) {
#pragma unroll
            for (int j = 0; j < 4; j++) out[4 + j] += (j == int(d1)) ? g.gtok : 0.0f;
        }
    }
}

template <int DT, int MK, bool KL, bool TAU1, bool SPLIT = false>
__device__ __forceinline__ void grad_step(const GradRow &g, float tau, const Raw<DT, MK> &rx,
                                          const Raw<DT, NT_MASK_NONE> &ry, int64_t e0, int64_t e1, float *out) {
#pragma unroll
    for (int j = 0; j < kEpl; j++) {
        const uint32_t mword = MK == NT_MASK_U8 ? rx.m[j / 4] : (MK == NT_MASK_F32 ? rx.m[j] : 0u);
        const float z = grad_tempered<MK, TAU1>(logit<DT>(rx.x, j), tau, mword, j);
        const float zr = KL ? grad_tempered<MK, TAU1>(logit<DT>(ry.x, j), tau, mword, j) : 0.0f;
        out[j] = grad_elem<KL>(g, z, zr);
    }
    add_token_term<SPLIT>(g, e0, e1, out);
}

// Aligned rows (V % 8 == 0, 16-byte rows, row bytes below 2^31): every access goes through a
// per-row buffer resource. Past the end of the row loads return zeros and stores are dropped by
// the hardware range check, so the loop needs no bounds tests: every lane runs the same number
// of steps. A step covers 2048 elements. With a bf16 gradient lane t owns elements 8t..8t+7 (one
// 16-byte load per input, one 16-byte store). With an f32 gradient (32 bytes per lane) it owns
// 4t..4t+3 and 1024+4t..1024+4t+3 instead, so that each store instruction writes one contiguous
// stretch of whole cache lines rather than every other 16 bytes of them. Either way a group of
// a lane's elements lies wholly inside the row or wholly past it (V % 8 == 0). Every input is
// read once and the gradient written once, so all of them are accessed non-temporally.
template <int DT, int MK, bool KL, int GDT, bool TAU1>
__device__ __forceinline__ void grad_row_aligned(const GradP &p, const GradRow &g, int64_t row) {
    constexpr int XB = Elem<DT>::kBytes, MB = MaskWords<MK>::kBytes, GB = GDT == NT_F32 ? 4 : 2;
    constexpr bool SPLIT = GDT == NT_F32;
    constexpr int kHalf = kGradStep / 2;
    const int V = int(p.V);
    const auto xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char *>(static_cast<const char *>(p.logits) + row * p.ld * XB), short(0), V * XB, kBufferWord3);
    __amdgpu_buffer_rsrc_t yres = xres, mres = xres;
    if constexpr (KL)
        yres = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<char *>(static_cast<const char *>(p.ref) + row * p.ld * XB), short(0), V * XB, kBufferWord3);
    if constexpr (MK != NT_MASK_NONE)
        mres = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<char *>(static_cast<const char *>(p.mask) + row * p.mask_ld * MB), short(0), V * MB,
            kBufferWord3);
    const auto gres = __builtin_amdgcn_make_buffer_rsrc(static_cast<char *>(p.grad) + row * p.gld * GB, short(0),
                                                        V * GB, kBufferWord3);
    // 4 elements of one input at element e into words w0.. of dst (f32: 4 words, bf16: 2)
    auto load4 = [&](uint32_t *dst, __amdgpu_buffer_rsrc_t rs, int e) {
        if constexpr (DT == NT_F32) {
            const auto a = __builtin_amdgcn_raw_buffer_load_b128(rs, e * 4, 0, kCachePolicyNT);
            for (int i = 0; i < 4; i++) dst[i] = a[i];
        } else {
            const auto a = __builtin_amdgcn_raw_buffer_load_b64(rs, e * 2, 0, kCachePolicyNT);
            dst[0] = a[0];
            dst[1] = a[1];
        }
    };
    auto load = [&](auto &rx, auto &ry, int e0, int e1) {
        if constexpr (SPLIT) {
            constexpr int H = Elem<DT>::kWords / 2;
            load4(rx.x, xres, e0);
            load4(rx.x + H, xres, e1);
            if constexpr (KL) {
                load4(ry.x, yres, e0);
                load4(ry.x + H, yres, e1);
            }
            if constexpr (MK == NT_MASK_U8) {
                rx.m[0] = __builtin_amdgcn_raw_buffer_load_b32(mres, e0, 0, kCachePolicyNT);
                rx.m[1] = __builtin_amdgcn_raw_buffer_load_b32(mres, e1, 0, kCachePolicyNT);
            } else if constexpr (MK == NT_MASK_F32) {
                const auto a = __builtin_amdgcn_raw_buffer_load_b128(mres, e0 * 4, 0, kCachePolicyNT);
                const auto b = __builtin_amdgcn_raw_buffer_load_b128(mres, e1 * 4, 0, kCachePolicyNT);
                for (int i = 0; i < 4; i++) {
                    rx.m[i] = a[i];
                    rx.m[4 + i] = b[i];
                }
            }
        } else {
            if constexpr (DT == NT_F32) {
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const auto a = __builtin_amdgcn_raw_buffer_load_b128(xres, e0 * 4 + 16 * q, 0, kCachePolicyNT);
                    for (int i = 0; i < 4; i++) rx.x[4 * q + i] = a[i];
                    if constexpr (KL) {
                        const auto b = __builtin_amdgcn_raw_buffer_load_b128(yres, e0 * 4 + 16 * q, 0, kCachePolicyNT);
                        for (int i = 0; i < 4; i++) ry.x[4 * q + i] = b[i];
                    }
                }
            } else {
                const auto a = __builtin_amdgcn_raw_buffer_load_b128(xres, e0 * 2, 0, kCachePolicyNT);
                for (int i = 0; i < 4; i++) rx.x[i] = a[i];
                if constexpr (KL) {
                    const auto b = __builtin_amdgcn_raw_buffer_load_b128(yres, e0 * 2, 0, kCachePolicyNT);
                    for (int i = 0; i < 4; i++) ry.x[i] = b[i];
                }
            }
            if constexpr (MK == NT_MASK_U8) {
                const auto k = __builtin_amdgcn_raw_buffer_load_b64(mres, e0, 0, kCachePolicyNT);
                rx.m[0] = k[0];
                rx.m[1] = k[1];
            } else if constexpr (MK == NT_MASK_F32) {
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const auto a = __builtin_amdgcn_raw_buffer_load_b128(mres, e0 * 4 + 16 * q, 0, kCachePolicyNT);
                    for (int i = 0; i < 4; i++) rx.m[4 * q + i] = a[i];
                }
            }
        }
    };
    auto store = [&](int e0, int e1, const float *o) {
        if constexpr (GDT == NT_F32) {
            const v4u a = {__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]), __float_as_uint(o[3])};
            const v4u b = {__float_as_uint(o[4]), __float_as_uint(o[5]), __float_as_uint(o[6]), __float_as_uint(o[7])};
            __builtin_amdgcn_raw_buffer_store_b128(a, gres, e0 * 4, 0, kCachePolicyNT);
            __builtin_amdgcn_raw_buffer_store_b128(b, gres, e1 * 4, 0, kCachePolicyNT);
        } else {
            const v4u w = {pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3]), pack_bf16(o[4], o[5]), pack_bf16(o[6], o[7])};
            __builtin_amdgcn_raw_buffer_store_b128(w, gres, e0 * 2, 0, kCachePolicyNT);
        }
    };
    const int t = int(threadIdx.x);
    const int first = SPLIT ? 4 * t : kEpl * t;  // the lane's first element in step 0
    for (int s0 = 0; s0 < V; s0 += 2 * kGradStep) {
        Raw<DT, MK> x0, x1;
        Raw<DT, NT_MASK_NONE> y0, y1;
        const int a0 = s0 + first, a1 = a0 + kGradStep;
        load(x0, y0, a0, a0 + kHalf);
        load(x1, y1, a1, a1 + kHalf);
        float o[kEpl];
        grad_step<DT, MK, KL, TAU1, SPLIT>(g, p.tau, x0, y0, a0, a0 + kHalf, o);
        store(a0, a0 + kHalf, o);
        grad_step<DT, MK, KL, TAU1, SPLIT>(g, p.tau, x1, y1, a1, a1 + kHalf, o);
        store(a1, a1 + kHalf, o);
    }
}

// Any other row layout: element-wise bounds and plain stores.
template <int DT, int MK, bool KL, int GDT, bool TAU1>
__device__ __forceinline__ void grad_row_general(const GradP &p, const GradRow &g, int64_t row) {
    const char *xrow = static_cast<const char *>(p.logits) + row * p.ld * Elem<DT>::kBytes;
    const char *yrow = KL ? static_cast<const char *>(p.ref) + row * p.ld * Elem<DT>::kBytes : nullptr;
    const char *mrow = MK != NT_MASK_NONE ? static_cast<const char *>(p.mask) + row * p.mask_ld * MaskWords<MK>::kBytes
                                          : nullptr;
    char *grow = static_cast<char *>(p.grad) + row * p.gld * (GDT == NT_F32 ? 4 : 2);
    for (int64_t e0 = int64_t(threadIdx.x) * kEpl; e0 < p.V; e0 += kGradStep) {
        Raw<DT, MK> rx;
        Raw<DT, NT_MASK_NONE> ry;
        load_raw<DT, MK, false>(rx, xrow, mrow, e0, p.V);
        if constexpr (KL) load_raw<DT, NT_MASK_NONE, false>(ry, yrow, nullptr, e0, p.V);
        float o[kEpl];
        grad_step<DT, MK, KL, TAU1>(g, p.tau, rx, ry, e0, 0, o);
        for (int j = 0; j < kEpl; j += 2) {
            if constexpr (GDT == NT_F32) {
                if (e0 + j < p.V) reinterpret_cast<float *>(grow)[e0 + j] = o[j];
                if (e0 + j + 1 < p.V) reinterpret_cast<float *>(grow)[e0 + j + 1] = o[j + 1];
            } else {
                const uint32_t w = pack_bf16(o[j], o[j + 1]);
                if (e0 + j < p.V) reinterpret_cast<uint16_t *>(grow)[e0 + j] = uint16_t(w);
                if (e0 + j + 1 < p.V) reinterpret_cast<uint16_t *>(grow)[e0 + j + 1] = uint16_t(w >> 16);
            }
        }
    }
}

template <int DT, int MK, bool KL, int GDT, bool AL>
__global__ __launch_bounds__(kGradThreads) void k_score_grad(GradP p) {
    const int64_t row = blockIdx.x;
    const GradRow g = grad_row<KL>(p, row);
    if (p.tau_one) {
        if constexpr (AL) grad_row_aligned<DT, MK, KL, GDT, true>(p, g, row);
        else grad_row_general<DT, MK, KL, GDT, true>(p, g, row);
    } else {
        if constexpr (AL) grad_row_aligned<DT, MK, KL, GDT, false>(p, g, row);
        else grad_row_general<DT, MK, KL, GDT, false>(p, g, row);
    }
}

// ------------------------------------------------------------------ per-token kernels

__global__ void k_kl_estimate(const float *lp, const float *lr, const float *mask, int64_t n, int est,
                              float clamp, int clamped, float *out) {
    for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        const bool scored = mask ? (mask[i] != 0.0f) : true;
        // zero_masked is a select (rl.rs:100-102); then the optional clamp (rl.rs:389-392).
        float d = scored ? (lr[i] - lp[i]) : 0.0f;
        if (clamped) d = fminf(fmaxf(d, -clamp), clamp);
        float k;
        if (est == 1) k = -d;
        else if (est == 2) k = (d * d) / 2.0f;
        else k = expm1f(d) - d;  // = exp(d) - d - 1 without the cancellation near d = 0
        out[i] = scored ? k : 0.0f;
    }
}

__global__ void k_zero_masked(const float *x, const float *mask, int64_t n, float *out) {
    for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
        out[i] = mask[i] != 0.0f ? x[i] : 0.0f;
}

__global__ void k_reduce_tokens(const float *per, const float *mask, int64_t S, int64_t B, int64_t T, int red,
                                float *out) {
    const int64_t nout = red == 3 ? S * B : S;
    const int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
    if (i >= nout) return;
    if (red == 3) {
        double v = 0.0, m = 0.0;
        for (int64_t t = 0; t < T; t++) {
            v += double(per[i * T + t]);
            m += mask ? double(mask[i * T + t]) : 1.0;
        }
        out[i] = float(v / (m > 1.0 ? m : 1.0));
        return;
    }
    double tot = 0.0, cnt = 0.0, seq = 0.0, nonempty = 0.0;
    for (int64_t b = 0; b < B; b++) {
        double v = 0.0, m = 0.0;
        for (int64_t t = 0; t < T; t++) {
            const int64_t k = (i * B + b) * T + t;
            v += double(per[k]);
            m += mask ? double(mask[k]) : 1.0;
        }
        tot += v;
        cnt += m;
        seq += v / (m > 1.0 ? m : 1.0);
        nonempty += (m > 1.0 ? 1.0 : m);
    }
    if (red == 1) out[i] = float(tot);
    else if (red == 2) out[i] = float(tot / (cnt > 1.0 ? cnt : 1.0));
    else out[i] = float(seq / (nonempty > 1.0 ? nonempty : 1.0));
}

// ------------------------------------------------------------------ reductions per seed
//
// One 1024-thread block per seed s: wave w sums sequences w, w+16, ... over T (lane-strided, f64,
// then a fixed DPP tree), keeping each sequence's value sum and mask sum in LDS; thread 0 folds
// them in sequence order. The forward writes reduce_tokens' outputs (rl.rs:69-92); the backward
// writes each position's share of the reduced outputs' upstream gradient.

constexpr int kSeedThreads = 1024;
constexpr int64_t kSeedMaxB = 4096;  // sequences per seed the LDS of one block holds (2 x f64 each)

template <bool BWD>
__global__ __launch_bounds__(kSeedThreads) void k_reduce_seed(const float *per, const float *mask, int64_t B,
                                                               int64_t T, int red, float *out, const float *up,
                                                               float scale, const float *local) {
    extern __shared__ double seqs[];  // [B] value sums, then [B] mask sums
    __shared__ double seed[4];        // total, scored count, sum of sequence means, non-empty sequences
    double *sv = seqs, *sm = seqs + B;
    const int64_t s = blockIdx.x;
    const int tid = int(threadIdx.x), wave = tid / kWave, lane = tid % kWave;
    const int64_t base = s * B * T;
    for (int64_t b = wave; b < B; b += kSeedThreads / kWave) {
        double v = 0.0, m = 0.0;
        for (int64_t t = lane; t < T; t += kWave) {
            const int64_t k = base + b * T + t;
            if constexpr (!BWD) v += double(per[k]);
            m += mask ? double(mask[k]) : 1.0;
        }
        if constexpr (!BWD) v = readlane_d(wave_scan_dpp(v), kWave - 1);
        m = readlane_d(wave_scan_dpp(m), kWave - 1);
        if (lane == 0) {
            sv[b] = v;
            sm[b] = m;
        }
    }
    __syncthreads();
    if (tid == 0) {
        double tot = 0.0, cnt = 0.0, seq = 0.0, nonempty = 0.0;
        for (int64_t b = 0; b < B; b++) {
            tot += sv[b];
            cnt += sm[b];
            seq += sv[b] / (sm[b] > 1.0 ? sm[b] : 1.0);
            nonempty += sm[b] > 1.0 ? 1.0 : sm[b];  // clamp_max(1) of the sequence's count
        }
        seed[0] = tot;
        seed[1] = cnt > 1.0 ? cnt : 1.0;
        seed[2] = seq;
        seed[3] = nonempty > 1.0 ? nonempty : 1.0;
    }
    __syncthreads();
    if constexpr (!BWD) {
        if (red == 3) {
            for (int64_t b = tid; b < B; b += kSeedThreads) out[s * B + b] = float(sv[b] / (sm[b] > 1.0 ? sm[b] : 1.0));
        } else if (tid == 0) {
            out[s] = float(red == 1 ? seed[0] : (red == 2 ? seed[0] / seed[1] : seed[2] / seed[3]));
        }
    } else {
        const double gs = red == 0 || red == 3 ? 0.0 : (up ? double(up[s]) : 1.0);
        for (int64_t j = tid; j < B * T; j += kSeedThreads) {
            const int64_t k = base + j, b = j / T;
            const float m = mask ? mask[k] : 1.0f;
            double g;
            if (red == 0) g = up ? double(up[k]) : 1.0;
            else if (red == 1) g = gs;
            else if (red == 2) g = gs / seed[1];
            else if (red == 3) g = (up ? double(up[s * B + b]) : 1.0) / (sm[b] > 1.0 ? sm[b] : 1.0);
            else g = gs / (seed[3] * (sm[b] > 1.0 ? sm[b] : 1.0));
            const float gl = float(double(scale) * g);
            out[k] = m != 0.0f ? (local ? gl * local[k] : gl) : 0.0f;
        }
    }
}

// ------------------------------------------------------------------ policy losses per token

struct LossP {
    const float *lp, *old, *w, *mask;
    int64_t n, T;
    int kind, per_seq;
    float lo, hi;          // 1 - low, 1 + high (f32, as the op sequence's scalar clamp)
    float neg_c, c;        // -c, c (dual clip)
    float b;               // the log-ratio clamp
    int dual, clamped;
    float *loss, *dloss, *hit;
};

__global__ void k_policy_loss(LossP p) {
    for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < p.n; i += int64_t(gridDim.x) * blockDim.x) {
        const float m = p.mask ? p.mask[i] : 1.0f;
        const bool scored = m != 0.0f;
        const float a = p.per_seq ? p.w[i / p.T] : p.w[i];
        float per, dper, hit = 0.0f;
        if (p.kind == NT_LOSS_PG) {
            per = -(p.lp[i] * a);
            dper = -a;
        } else {
            // log_ratio (rl.rs:237-245): zero_masked, then the clamp (its gradient passes inside)
            const float d = scored ? p.lp[i] - p.old[i] : 0.0f;
            const float dc = p.clamped ? fminf(fmaxf(d, -p.b), p.b) : d;
            const float gate = p.clamped ? ((d >= -p.b && d <= p.b) ? 1.0f : 0.0f) : 1.0f;
            const float r = expf(dc);
            const float un = -(r * a);
            const float rc = fminf(fmaxf(r, p.lo), p.hi);
            const float cl = -(rc * a);
            // select_max(unclipped, clipped) (rl.rs:124-129): the unclipped branch wins only on a
            // positive difference; the gradient goes to the selected branch (the clipped one's is
            // zero outside [1 - low, 1 + high])
            const bool un_wins = (un - cl) > 0.0f;
            float v = un_wins ? un : cl;
            float gr = (un_wins || (r >= p.lo && r <= p.hi)) ? -a : 0.0f;
            if (p.dual && a < 0.0f) {
                // min(v, -c A) as -select_max(-v, -cap) with cap = A (-c)
                const float cap = a * p.neg_c;
                const bool keep = ((-v) - (-cap)) > 0.0f;
                v = keep ? v : cap;
                gr = keep ? gr : 0.0f;
            }
            per = v;
            dper = (gr * r) * gate;  // exp's derivative is r (0 * inf = NaN, as the op sequence)
            // clip_fraction (rl.rs:293-317) uses the unclamped ratio
            const float r0 = expf(d);
            float h = ((a > 0.0f && r0 > p.hi) ? 1.0f : 0.0f) + ((a < 0.0f && r0 < p.lo) ? 1.0f : 0.0f);
            if (p.dual) h += (r0 > p.c && a < 0.0f) ? 1.0f : 0.0f;
            if (p.clamped) h += fabsf(d) > p.b ? 1.0f : 0.0f;
            hit = fminf(h, 1.0f) * m;
        }
        if (p.loss) p.loss[i] = scored ? per : 0.0f;
        if (p.dloss) p.dloss[i] = scored ? dper : 0.0f;
        if (p.hit) p.hit[i] = scored ? hit : 0.0f;
    }
}

// group_advantages (rl.rs:436-463): one thread per group, f64, sums left to right.
__global__ void k_group_advantages(const float *r, int64_t groups, int64_t n, int std_norm, double eps, int unbiased,
                                   float *out) {
    const int64_t g = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
    if (g >= groups) return;
    const float *x = r + g * n;
    float *y = out + g * n;
    double lo = INFINITY, hi = -INFINITY, sum = 0.0;
    for (int64_t i = 0; i < n; i++) {
        const double v = double(x[i]);
        lo = v < lo ? v : lo;
        hi = v > hi ? v : hi;
    }
    if (lo == hi) {
        for (int64_t i = 0; i < n; i++) y[i] = 0.0f;
        return;
    }
    for (int64_t i = 0; i < n; i++) sum += double(x[i]);
    const double mean = sum / double(n);
    double scale = 1.0;
    if (std_norm) {
        double ss = 0.0;
        for (int64_t i = 0; i < n; i++) {
            const double d = double(x[i]) - mean;
            ss += d * d;
        }
        scale = sqrt(ss / (unbiased ? double(n - 1) : double(n))) + eps;
    }
    for (int64_t i = 0; i < n; i++) y[i] = float((double(x[i]) - mean) / scale);
}

__global__ void k_kl_estimate_grad(const float *lp, const float *lr, const float *mask, int64_t n, int est,
                                   float clamp, int clamped, float *out) {
    for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
        const bool scored = mask ? (mask[i] != 0.0f) : true;
        const float d = scored ? (lr[i] - lp[i]) : 0.0f;
        const bool active = clamped && !(d >= -clamp && d <= clamp);
        const float dc = clamped ? fminf(fmaxf(d, -clamp), clamp) : d;
        // dk/dlogp = -dk/d(delta)
        float g;
        if (est == 1) g = 1.0f;
        else if (est == 2) g = -dc;
        else g = -expm1f(dc);
        out[i] = (scored && !active) ? g : 0.0f;
    }
}

// ------------------------------------------------------------------ dispatch helpers

int check_rows(int64_t rows, int64_t V, int64_t ld, int32_t dtype, int32_t mk, const void *mask, int64_t mask_ld,
               const char *who) {
    char buf[256];
    if (rows < 0 || V < 1 || ld < V || (dtype != NT_F32 && dtype != NT_BF16) || mk < NT_MASK_NONE ||
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

bool aligned_rows(const void *x, int64_t V, int64_t ld, int32_t dtype, int32_t mk, const void *mask, int64_t mask_ld) {
    if (V % kEpl != 0 || ld % kEpl != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0) return false;
    (void)dtype;
    if (mk == NT_MASK_U8) return mask_ld % 8 == 0 && reinterpret_cast<uintptr_t>(mask) % 8 == 0;
    if (mk == NT_MASK_F32) return mask_ld % 4 == 0 && reinterpret_cast<uintptr_t>(mask) % 16 == 0;
    return true;
}

template <int DT, int MK, bool ENT, bool AL>
void launch_sample(const SampleP &p, int64_t rows, int threads, size_t shm, hipStream_t s) {
    hipLaunchKernelGGL((k_sample<DT, MK, ENT, AL>), dim3(unsigned(rows)), dim3(threads), shm, s, p);
}

template <int DT, int MK, bool ENT>
void pick_al_sample(bool al, const SampleP &p, int64_t rows, int threads, size_t shm, hipStream_t s) {
    if (al) launch_sample<DT, MK, ENT, true>(p, rows, threads, shm, s);
    else launch_sample<DT, MK, ENT, false>(p, rows, threads, shm, s);
}

template <int DT, int MK>
void pick_ent_sample(bool ent, bool al, const SampleP &p, int64_t rows, int threads, size_t shm, hipStream_t s) {
    if (ent) pick_al_sample<DT, MK, true>(al, p, rows, threads, shm, s);
    else pick_al_sample<DT, MK, false>(al, p, rows, threads, shm, s);
}

template <int DT>
void pick_mk_sample(int mk, bool ent, bool al, const SampleP &p, int64_t rows, int threads, size_t shm,
                    hipStream_t s) {
    if (mk == NT_MASK_U8) pick_ent_sample<DT, NT_MASK_U8>(ent, al, p, rows, threads, shm, s);
    else if (mk == NT_MASK_F32) pick_ent_sample<DT, NT_MASK_F32>(ent, al, p, rows, threads, shm, s);
    else pick_ent_sample<DT, NT_MASK_NONE>(ent, al, p, rows, threads, shm, s);
}

// Largest chunks-per-wave of the register-resident sampler at EPL elements per lane: K chunks
// of logit words live in VGPRs (64 registers: bf16 EPL/2 words per chunk, f32 EPL) and the mask
// of every chunk in LDS (u8 64 EPL bytes, f32 256 EPL bytes; at most 128 KiB).
int rr_kmax(int dtype, int mk, int epl) {
    int k = (dtype == NT_BF16 ? 128 : 64) / epl;
    if (mk == NT_MASK_F32) k = k < 32 / epl ? k : 32 / epl;  // 16 waves * K * 256 EPL bytes <= 128 KiB
    return k;
}

template <int DT, int MK, int K, int EPL>
void launch_rr_k(bool ent, const SampleP &p, int64_t rows, hipStream_t s) {
    if (ent) hipLaunchKernelGGL((k_sample_rr<DT, MK, K, true, EPL>), dim3(unsigned(rows)), dim3(kRRThreads), 0, s, p);
    else hipLaunchKernelGGL((k_sample_rr<DT, MK, K, false, EPL>), dim3(unsigned(rows)), dim3(kRRThreads), 0, s, p);
}

// K is a power of two up to rr_kmax(DT, MK, EPL); the instantiations are exactly those.
template <int DT, int MK, int EPL>
void launch_rr_mk(int K, bool ent, const SampleP &p, int64_t rows, hipStream_t s) {
    constexpr int KREG = (DT == NT_BF16 ? 128 : 64) / EPL;
    constexpr int KMAX = MK == NT_MASK_F32 && 32 / EPL < KREG ? 32 / EPL : KREG;
    switch (K) {
        case 1: launch_rr_k<DT, MK, 1, EPL>(ent, p, rows, s); break;
        case 2: launch_rr_k<DT, MK, 2, EPL>(ent, p, rows, s); break;
        case 4: if constexpr (KMAX >= 4) launch_rr_k<DT, MK, 4, EPL>(ent, p, rows, s); break;
        case 8: if constexpr (KMAX >= 8) launch_rr_k<DT, MK, 8, EPL>(ent, p, rows, s); break;
        case 16: if constexpr (KMAX >= 16) launch_rr_k<DT, MK, 16, EPL>(ent, p, rows, s); break;
        default: break;
    }
}

template <int EPL>
void launch_rr(int dtype, int mk, int K, bool ent, const SampleP &p, int64_t rows, hipStream_t s) {
    if (dtype == NT_F32) {
        if (mk == NT_MASK_U8) launch_rr_mk<NT_F32, NT_MASK_U8, EPL>(K, ent, p, rows, s);
        else if (mk == NT_MASK_F32) launch_rr_mk<NT_F32, NT_MASK_F32, EPL>(K, ent, p, rows, s);
        else launch_rr_mk<NT_F32, NT_MASK_NONE, EPL>(K, ent, p, rows, s);
    } else {
        if (mk == NT_MASK_U8) launch_rr_mk<NT_BF16, NT_MASK_U8, EPL>(K, ent, p, rows, s);
        else if (mk == NT_MASK_F32) launch_rr_mk<NT_BF16, NT_MASK_F32, EPL>(K, ent, p, rows, s);
        else launch_rr_mk<NT_BF16, NT_MASK_NONE, EPL>(K, ent, p, rows, s);
    }
}

template <int DT, int MK, bool REF, bool KL, bool ENT>
void pick_al_score(bool al, const ScoreP &p, int64_t rows, hipStream_t s) {
    if (al) hipLaunchKernelGGL((k_score<DT, MK, REF, KL, ENT, true>), dim3(unsigned(rows)), dim3(kScoreThreads), 0, s, p);
    else hipLaunchKernelGGL((k_score<DT, MK, REF, KL, ENT, false>), dim3(unsigned(rows)), dim3(kScoreThreads), 0, s, p);
}

template <int DT, int MK>
void pick_flags_score(bool ref, bool kl, bool ent, bool al, const ScoreP &p, int64_t rows, hipStream_t s) {
    if (ref && kl) {
        if (ent) pick_al_score<DT, MK, true, true, true>(al, p, rows, s);
        else pick_al_score<DT, MK, true, true, false>(al, p, rows, s);
    } else if (ref) {
        if (ent) pick_al_score<DT, MK, true, false, true>(al, p, rows, s);
        else pick_al_score<DT, MK, true, false, false>(al, p, rows, s);
    } else {
        if (ent) pick_al_score<DT, MK, false, false, true>(al, p, rows, s);
        else pick_al_score<DT, MK, false, false, false>(al, p, rows, s);
    }
}

template <int DT>
void pick_mk_score(int mk, bool ref, bool kl, bool ent, bool al, const ScoreP &p, int64_t rows, hipStream_t s) {
    if (mk == NT_MASK_U8) pick_flags_score<DT, NT_MASK_U8>(ref, kl, ent, al, p, rows, s);
    else if (mk == NT_MASK_F32) pick_flags_score<DT, NT_MASK_F32>(ref, kl, ent, al, p, rows, s);
    else pick_flags_score<DT, NT_MASK_NONE>(ref, kl, ent, al, p, rows, s);
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" {

int nt_hip_rl_sample(const NtRlSampleArgs *a) {
    if (!a) return fail(NT_E_ARG, "nt_hip_rl_sample: null args");
    if (int rc = check_rows(a->rows, a->vocab, a->ld, a->dtype, a->mask_kind, a->mask, a->mask_ld, "nt_hip_rl_sample"))
        return rc;
    if (!(a->temperature >= 0.0) || !std::isfinite(a->temperature))
        return fail(NT_E_ARG, "sample_categorical: temperature " + std::to_string(a->temperature) + " (must be ≥ 0)");
    const bool greedy = a->temperature == 0.0;
    if (!a->logits || !a->ids || !a->status || (!greedy && !a->uniforms))
        return fail(NT_E_ARG, "nt_hip_rl_sample: null logits, ids, status or uniforms");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (a->rows == 0) return 0;
    const int64_t nc = (a->vocab + kChunk - 1) / kChunk;
    const bool ent = a->entropy != nullptr;
    const size_t shm = size_t(nc) * sizeof(float) * (ent ? 3 : 2);
    if (shm > 64 * 1024) return fail(NT_E_UNSUPPORTED, "nt_hip_rl_sample: V " + std::to_string(a->vocab) + " too large");
    SampleP p;
    p.logits = a->logits;
    p.mask = a->mask;
    p.V = a->vocab;
    p.ld = a->ld;
    p.mask_ld = a->mask_ld;
    const double T = greedy ? 1.0 : a->temperature;
    p.tau = float(T);
    p.tau_one = (T == 1.0);
    p.c = (a->mask_kind == NT_MASK_F32 || T == 1.0) ? kLog2e : float(double(kLog2e) / double(p.tau));
    p.greedy = greedy;
    p.nc = int(nc);
    p.u = a->uniforms;
    p.ids = a->ids;
    p.logp = a->logp;
    p.ent = a->entropy;
    p.status = a->status;
    // Waves per row: about four chunks per wave, at most 16; many rows get smaller groups.
    int nw = int(nc / 4);
    nw = nw < 1 ? 1 : (nw > 16 ? 16 : nw);
    if (a->rows >= 2048 && nw > 4) nw = 4;
    const bool al = aligned_rows(a->logits, a->vocab, a->ld, a->dtype, a->mask_kind, a->mask, a->mask_ld);
    hipStream_t s = ctx().stream;
    // Rows that fit the register-resident kernel take it (chunks per wave K = 1..16); the
    // streaming kernel takes everything else (unaligned rows, larger V).
    if (al) {
        // 8 elements per lane (512-element chunks): 16 per lane measured slower on MI355X at c4
        // (19.37 us, or 18.81 with a one-chunk window, against 18.24-18.52 us at 8).
        constexpr int epl = 8;
        const int64_t nch = (a->vocab + kWave * epl - 1) / (kWave * epl);
        const int kmax = rr_kmax(a->dtype, a->mask_kind, epl);
        if (nch <= int64_t(kRRWaves) * kmax) {
            int K = 1;
            while (int64_t(kRRWaves) * K < nch) K *= 2;
            p.nc = int(nch);
            launch_rr<8>(a->dtype, a->mask_kind, K, ent, p, a->rows, s);
            return launched("nt_hip_rl_sample");
        }
    }
    if (a->dtype == NT_F32) pick_mk_sample<NT_F32>(a->mask_kind, ent, al, p, a->rows, nw * kWave, shm, s);
    else pick_mk_sample<NT_BF16>(a->mask_kind, ent, al, p, a->rows, nw * kWave, shm, s);
    return launched("nt_hip_rl_sample");
}

int nt_hip_rl_score(const NtRlScoreArgs *a) {
    if (!a) return fail(NT_E_ARG, "nt_hip_rl_score: null args");
    if (int rc = check_rows(a->rows, a->vocab, a->ld, a->dtype, a->mask_kind, a->mask, a->mask_ld, "nt_hip_rl_score"))
        return rc;
    if (!(a->temperature > 0.0) || !std::isfinite(a->temperature))
        return fail(NT_E_ARG, "tempered_logits: temperature " + std::to_string(a->temperature) + " (must be positive)");
    if (!a->logits) return fail(NT_E_ARG, "nt_hip_rl_score: null logits");
    if ((a->logp || a->ref_logp) && !a->tokens) return fail(NT_E_ARG, "nt_hip_rl_score: log-probabilities need tokens");
    if ((a->ref_logp || a->kl) && !a->ref_logits) return fail(NT_E_ARG, "nt_hip_rl_score: ref_logp/kl need ref_logits");
    if ((a->ref_lse_base || a->ref_lse_rest) && !a->ref_logits)
        return fail(NT_E_ARG, "nt_hip_rl_score: reference statistics need ref_logits");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (a->rows == 0) return 0;
    ScoreP p;
    p.logits = a->logits;
    p.ref = a->ref_logits;
    p.mask = a->mask;
    p.V = a->vocab;
    p.ld = a->ld;
    p.mask_ld = a->mask_ld;
    p.tau = float(a->temperature);
    p.tau_one = (a->temperature == 1.0);
    p.c = (a->mask_kind == NT_MASK_F32 || p.tau_one) ? kLog2e : float(double(kLog2e) / double(p.tau));
    p.nc = int((a->vocab + kChunk - 1) / kChunk);
    p.tokens = a->tokens;
    p.logp = a->logp;
    p.ref_logp = a->ref_logp;
    p.kl = a->kl;
    p.ent = a->entropy;
    p.status = a->status;
    p.lse_base = a->lse_base;
    p.lse_rest = a->lse_rest;
    p.ref_lse_base = a->ref_lse_base;
    p.ref_lse_rest = a->ref_lse_rest;
    const bool ref = a->ref_logits != nullptr && (a->ref_logp || a->kl || a->ref_lse_base || a->ref_lse_rest);
    const bool kl = a->kl != nullptr;
    const bool ent = a->entropy != nullptr;
    // the aligned path addresses a row's bytes with 32-bit buffer offsets
    bool al = aligned_rows(a->logits, a->vocab, a->ld, a->dtype, a->mask_kind, a->mask, a->mask_ld) &&
              a->vocab * 4 <= int64_t(0x7fffffff);
    if (ref) al = al && reinterpret_cast<uintptr_t>(a->ref_logits) % 16 == 0;
    hipStream_t s = ctx().stream;
    if (a->dtype == NT_F32) pick_mk_score<NT_F32>(a->mask_kind, ref, kl, ent, al, p, a->rows, s);
    else pick_mk_score<NT_BF16>(a->mask_kind, ref, kl, ent, al, p, a->rows, s);
    return launched("nt_hip_rl_score");
}

int nt_hip_rl_score_backward(const NtRlScoreGradArgs *a) {
    if (!a) return fail(NT_E_ARG, "nt_hip_rl_score_backward: null args");
    if (int rc = check_rows(a->rows, a->vocab, a->ld, a->dtype, a->mask_kind, a->mask, a->mask_ld,
                            "nt_hip_rl_score_backward"))
        return rc;
    if (!(a->temperature > 0.0) || !std::isfinite(a->temperature))
        return fail(NT_E_ARG, "tempered_logits: temperature " + std::to_string(a->temperature) + " (must be positive)");
    if (!a->logits || !a->grad || !a->lse_base || !a->lse_rest)
        return fail(NT_E_ARG, "nt_hip_rl_score_backward: null logits, grad or log-sum-exp statistics");
    if (a->grad_dtype != NT_F32 && a->grad_dtype != NT_BF16)
        return fail(NT_E_ARG, "nt_hip_rl_score_backward: grad dtype " + std::to_string(a->grad_dtype));
    if (a->grad_ld < a->vocab) return fail(NT_E_ARG, "nt_hip_rl_score_backward: grad_ld < vocab");
    if (a->g_logp && !a->tokens) return fail(NT_E_ARG, "nt_hip_rl_score_backward: g_logp needs tokens");
    if (a->g_kl && (!a->ref_logits || !a->ref_lse_base || !a->ref_lse_rest || !a->kl))
        return fail(NT_E_ARG, "nt_hip_rl_score_backward: g_kl needs ref_logits, the reference statistics and kl");
    if (a->g_entropy && !a->entropy) return fail(NT_E_ARG, "nt_hip_rl_score_backward: g_entropy needs entropy");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (a->rows == 0) return 0;
    GradP p;
    p.logits = a->logits;
    p.ref = a->ref_logits;
    p.mask = a->mask;
    p.V = a->vocab;
    p.ld = a->ld;
    p.mask_ld = a->mask_ld;
    p.gld = a->grad_ld;
    p.tau = float(a->temperature);
    p.tau_one = a->temperature == 1.0;
    p.tokens = a->tokens;
    p.lb = a->lse_base;
    p.lr = a->lse_rest;
    p.rlb = a->ref_lse_base;
    p.rlr = a->ref_lse_rest;
    p.kl = a->kl;
    p.ent = a->entropy;
    p.glp = a->g_logp;
    p.gkl = a->g_kl;
    p.gh = a->g_entropy;
    p.grad = a->grad;
    const bool kl = a->g_kl != nullptr;
    // the buffer-resource path addresses a row's bytes with 32-bit offsets
    bool al = aligned_rows(a->logits, a->vocab, a->ld, a->dtype, a->mask_kind, a->mask, a->mask_ld) &&
              reinterpret_cast<uintptr_t>(a->grad) % 16 == 0 && a->grad_ld % kEpl == 0 &&
              a->vocab * 4 <= int64_t(0x7fffffff);
    if (kl) al = al && reinterpret_cast<uintptr_t>(a->ref_logits) % 16 == 0;
    hipStream_t s = ctx().stream;
    auto go = [&](auto dt, auto mk) {
        constexpr int DT = decltype(dt)::value, MK = decltype(mk)::value;
        auto launch = [&](auto klc, auto gdt, auto alc) {
            hipLaunchKernelGGL((k_score_grad<DT, MK, decltype(klc)::value, decltype(gdt)::value, decltype(alc)::value>),
                               dim3(unsigned(a->rows)), dim3(kGradThreads), 0, s, p);
        };
        auto by_al = [&](auto klc, auto gdt) {
            if (al) launch(klc, gdt, std::true_type{});
            else launch(klc, gdt, std::false_type{});
        };
        auto by_gdt = [&](auto klc) {
            if (a->grad_dtype == NT_F32) by_al(klc, std::integral_constant<int, NT_F32>{});
            else by_al(klc, std::integral_constant<int, NT_BF16>{});
        };
        if (kl) by_gdt(std::true_type{});
        else by_gdt(std::false_type{});
    };
    auto by_mk = [&](auto dt) {
        if (a->mask_kind == NT_MASK_U8) go(dt, std::integral_constant<int, NT_MASK_U8>{});
        else if (a->mask_kind == NT_MASK_F32) go(dt, std::integral_constant<int, NT_MASK_F32>{});
        else go(dt, std::integral_constant<int, NT_MASK_NONE>{});
    };
    if (a->dtype == NT_F32) by_mk(std::integral_constant<int, NT_F32>{});
    else by_mk(std::integral_constant<int, NT_BF16>{});
    return launched("nt_hip_rl_score_backward");
}

int nt_hip_rl_kl_estimate(const float *logp, const float *ref_logp, const float *mask, int64_t n, int32_t estimator,
                          double clamp, float *out) {
    if (n < 0 || !logp || !ref_logp || !out || estimator < 1 || estimator > 3)
        return fail(NT_E_ARG, "nt_hip_rl_kl_estimate: invalid arguments");
    if (clamp < 0.0) return fail(NT_E_ARG, "kl_estimate: δ clamp " + std::to_string(clamp) + " (need b > 0)");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (n == 0) return 0;
    const int threads = 256;
    int64_t blocks = (n + threads - 1) / threads;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_kl_estimate, dim3(unsigned(blocks)), dim3(threads), 0, ctx().stream, logp, ref_logp, mask, n,
                       int(estimator), float(clamp), clamp > 0.0 ? 1 : 0, out);
    return launched("nt_hip_rl_kl_estimate");
}

int nt_hip_rl_zero_masked(const float *x, const float *mask, int64_t n, float *out) {
    if (n < 0 || !x || !mask || !out) return fail(NT_E_ARG, "nt_hip_rl_zero_masked: invalid arguments");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (n == 0) return 0;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_zero_masked, dim3(unsigned(blocks)), dim3(256), 0, ctx().stream, x, mask, n, out);
    return launched("nt_hip_rl_zero_masked");
}

int nt_hip_rl_reduce_tokens(const float *per, const float *mask, int64_t S, int64_t B, int64_t T, int32_t reduction,
                            float *out) {
    if (!per || !out || S < 0 || B < 0 || T < 0 || reduction < 1 || reduction > 4)
        return fail(NT_E_ARG, "nt_hip_rl_reduce_tokens: invalid arguments");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    const int64_t nout = reduction == 3 ? S * B : S;
    if (nout == 0) return 0;
    if (B <= kSeedMaxB && S <= 0x7fffffffLL) {
        hipLaunchKernelGGL(k_reduce_seed<false>, dim3(unsigned(S)), dim3(kSeedThreads), size_t(2 * B) * sizeof(double),
                           ctx().stream, per, mask, B, T, int(reduction), out, nullptr, 1.0f, nullptr);
    } else {
        const int threads = 64;
        hipLaunchKernelGGL(k_reduce_tokens, dim3(unsigned((nout + threads - 1) / threads)), dim3(threads), 0,
                           ctx().stream, per, mask, S, B, T, int(reduction), out);
    }
    return launched("nt_hip_rl_reduce_tokens");
}

int nt_hip_rl_reduce_tokens_backward(const float *mask, int64_t S, int64_t B, int64_t T, int32_t reduction,
                                     const float *upstream, double scale, const float *local, float *out) {
    if (!out || S < 0 || B < 0 || T < 0 || reduction < 0 || reduction > 4 || !std::isfinite(scale))
        return fail(NT_E_ARG, "nt_hip_rl_reduce_tokens_backward: invalid arguments");
    if (B > kSeedMaxB || S > 0x7fffffffLL)
        return fail(NT_E_UNSUPPORTED, "nt_hip_rl_reduce_tokens_backward: more than 4096 sequences per seed");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (S == 0 || B == 0 || T == 0) return 0;
    hipLaunchKernelGGL(k_reduce_seed<true>, dim3(unsigned(S)), dim3(kSeedThreads), size_t(2 * B) * sizeof(double),
                       ctx().stream, nullptr, mask, B, T, int(reduction), out, upstream, float(scale), local);
    return launched("nt_hip_rl_reduce_tokens_backward");
}

int nt_hip_rl_kl_estimate_backward(const float *logp, const float *ref_logp, const float *mask, int64_t n,
                                   int32_t estimator, double clamp, float *out) {
    if (n < 0 || !logp || !ref_logp || !out || estimator < 1 || estimator > 3)
        return fail(NT_E_ARG, "nt_hip_rl_kl_estimate_backward: invalid arguments");
    if (clamp < 0.0) return fail(NT_E_ARG, "kl_estimate: δ clamp " + std::to_string(clamp) + " (need b > 0)");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (n == 0) return 0;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_kl_estimate_grad, dim3(unsigned(blocks)), dim3(256), 0, ctx().stream, logp, ref_logp, mask, n,
                       int(estimator), float(clamp), clamp > 0.0 ? 1 : 0, out);
    return launched("nt_hip_rl_kl_estimate_backward");
}

int nt_hip_rl_group_advantages(const float *rewards, int64_t groups, int64_t n, int32_t norm, double eps,
                               int32_t unbiased, float *out) {
    if (!rewards || !out || groups < 0 || (norm != 0 && norm != 1))
        return fail(NT_E_ARG, "nt_hip_rl_group_advantages: invalid arguments");
    if (n < 1) return fail(NT_E_ARG, "group_advantages: rewards in groups of " + std::to_string(n));
    if (norm == 1 && !(eps >= 0.0)) return fail(NT_E_ARG, "group_advantages: ε " + std::to_string(eps) + " < 0");
    if (norm == 1 && unbiased && n < 2)
        return fail(NT_E_ARG, "group_advantages: the sample standard deviation needs groups of at least 2");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (groups == 0) return 0;
    const int threads = 64;
    hipLaunchKernelGGL(k_group_advantages, dim3(unsigned((groups + threads - 1) / threads)), dim3(threads), 0,
                       ctx().stream, rewards, groups, n, int(norm), eps, int(unbiased != 0), out);
    return launched("nt_hip_rl_group_advantages");
}

int nt_hip_rl_policy_loss(const NtRlPolicyLossArgs *a) {
    if (!a) return fail(NT_E_ARG, "nt_hip_rl_policy_loss: null args");
    if (!a->logp || !a->weights || a->S < 0 || a->B < 0 || a->T < 0 ||
        (a->kind != NT_LOSS_PG && a->kind != NT_LOSS_PPO) || (a->kind == NT_LOSS_PPO && !a->old_logp))
        return fail(NT_E_ARG, "nt_hip_rl_policy_loss: invalid arguments");
    if (a->kind == NT_LOSS_PPO) {
        char buf[200];
        // Clip::check (rl.rs:189-200)
        if (!(a->clip_low >= 0.0 && a->clip_low < 1.0 && a->clip_high >= 0.0 && std::isfinite(a->clip_low) &&
              std::isfinite(a->clip_high))) {
            std::snprintf(buf, sizeof buf, "clip range [1 − %g, 1 + %g] (need 0 ≤ low < 1, 0 ≤ high)", a->clip_low,
                          a->clip_high);
            return fail(NT_E_ARG, buf);
        }
        if (a->dual != 0.0 && !(a->dual > 1.0 && std::isfinite(a->dual))) {
            std::snprintf(buf, sizeof buf, "dual clip %g (need c > 1)", a->dual);
            return fail(NT_E_ARG, buf);
        }
        if (!(a->log_ratio_clamp >= 0.0)) {
            std::snprintf(buf, sizeof buf, "log-ratio clamp %g (need b > 0)", a->log_ratio_clamp);
            return fail(NT_E_ARG, buf);
        }
    }
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    const int64_t n = a->S * a->B * a->T;
    if (n == 0) return 0;
    LossP p;
    p.lp = a->logp;
    p.old = a->old_logp;
    p.w = a->weights;
    p.mask = a->mask;
    p.n = n;
    p.T = a->T;
    p.kind = a->kind;
    p.per_seq = a->weights_per_sequence != 0;
    p.lo = float(1.0 - a->clip_low);
    p.hi = float(1.0 + a->clip_high);
    p.neg_c = float(-a->dual);
    p.c = float(a->dual);
    p.b = float(a->log_ratio_clamp);
    p.dual = a->dual != 0.0;
    p.clamped = a->log_ratio_clamp > 0.0;
    p.loss = a->loss;
    p.dloss = a->dloss;
    p.hit = a->hit;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_policy_loss, dim3(unsigned(blocks)), dim3(256), 0, ctx().stream, p);
    return launched("nt_hip_rl_policy_loss");
}

}  // extern "C"
