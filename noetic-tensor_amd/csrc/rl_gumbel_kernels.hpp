// The reference's Gumbel-max sampler's device code for gfx950 (MI355X), sample_categorical
// (src/nn/rl.rs:488-529) on a Hip tensor. One source for both ways the library builds it:
// compiled ahead of time into libnoetic_hip.so (rl_gumbel.hip includes this file), and compiled
// at run time by hiprtc from the text embedded in the library (rtc.cpp). The algorithm and its
// contract are described in rl_gumbel.hip.
#pragma once

#include "nt_chacha.hpp"
#include "nt_rows.hpp"

namespace nt {
namespace {

constexpr int kGumbelMaxThreads = 1024;

struct GumbelP {
    const void *logits;
    const void *mask;
    int64_t V, ld;
    MaskMap mm;  // the mask row of each logits row
    float tau;
    int tau_one;
    ChachaKey key;
    uint64_t h;  // pair index of the stream's u64 0: its low word is keystream word 2 h + ODD
    int vec;     // rows (and mask rows) aligned for one vector load per 8 elements
    int32_t *ids;
    uint8_t *status;
};

// z_v = tempered_logits (rl.rs:475-486) in f32: x / tau (skipped at tau == 1), then the
// additive f32 mask, or -inf at a token a u8 keep-mask excludes. Without DIV the division is
// left to the caller (with a u8 mask or none it commutes with the exclusion: -inf / tau = -inf).
// moff: the row's mask row (mask_row_at).
template <int DT, int MK, bool DIV = true>
__device__ __forceinline__ float tempered_at(const GumbelP &p, int64_t row, int64_t moff, int64_t v) {
    float x;
    if constexpr (DT == NT_F32) {
        x = static_cast<const float *>(p.logits)[row * p.ld + v];
    } else {
        x = widen16<DT>(uint32_t(static_cast<const uint16_t *>(p.logits)[row * p.ld + v]));
    }
    if (DIV && !p.tau_one) x = x / p.tau;
    if constexpr (MK == NT_MASK_U8) {
        if (static_cast<const uint8_t *>(p.mask)[moff + v] == 0) x = -INFINITY;
    } else if constexpr (MK == NT_MASK_F32) {
        x = x + static_cast<const float *>(p.mask)[moff + v];
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

// A block's 8 logits and mask entries, loaded together (the aligned path).
template <int DT, int MK>
struct GumbelRaw {
    uint32_t x[DT == NT_F32 ? 8 : 4];
    uint32_t m[MK == NT_MASK_F32 ? 8 : (MK == NT_MASK_U8 ? 2 : 1)];
};

template <int DT, int MK>
__device__ __forceinline__ void gumbel_load(GumbelRaw<DT, MK> &r, __amdgpu_buffer_rsrc_t xres,
                                            __amdgpu_buffer_rsrc_t mres, int v0) {
    if constexpr (DT == NT_F32) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const auto a = __builtin_amdgcn_raw_buffer_load_b128(xres, (v0 + 4 * q) * 4, 0, 0);
            for (int i = 0; i < 4; i++) r.x[4 * q + i] = a[i];
        }
    } else {
        const auto a = __builtin_amdgcn_raw_buffer_load_b128(xres, v0 * 2, 0, 0);
        for (int i = 0; i < 4; i++) r.x[i] = a[i];
    }
    if constexpr (MK == NT_MASK_U8) {
        const auto k = __builtin_amdgcn_raw_buffer_load_b64(mres, v0, 0, 0);
        r.m[0] = k[0];
        r.m[1] = k[1];
    } else if constexpr (MK == NT_MASK_F32) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const auto a = __builtin_amdgcn_raw_buffer_load_b128(mres, (v0 + 4 * q) * 4, 0, 0);
            for (int i = 0; i < 4; i++) r.m[4 * q + i] = a[i];
        }
    }
}

// tempered_at's values from a loaded block (elements v0 .. v0 + 7; those at or past V are -inf).
template <int DT, int MK, bool DIV = true>
__device__ __forceinline__ void gumbel_values(const GumbelRaw<DT, MK> &r, const GumbelP &p, int v0, float (&z)[8]) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float x;
        x = logit<DT>(r.x, j);
        if (DIV && !p.tau_one) x = x / p.tau;
        if constexpr (MK == NT_MASK_U8) {
            if (((r.m[j / 4] >> (8 * (j % 4))) & 0xffu) == 0) x = -INFINITY;
        } else if constexpr (MK == NT_MASK_F32) {
            x = x + __uint_as_float(r.m[j]);
        }
        z[j] = v0 + j < p.V ? x : -INFINITY;
    }
}

// The screen (a draw's value in f32 from hardware logarithms): within 1e-5 of gumbel_f32's
// value, and infinite exactly where it is, with no branch and no division. k = (hi:lo) >> 11 and
// u = (k + 0.5) / 2^53. Below u = 1 - 2^-4, t = -ln u from u in f32 (hi's and k's low 21 bits
// converted apart); t >= 0.06 there, so the logarithm's rounding stays a small relative error.
// Above it, t = -ln(1 - d) = d (1 + d/2 + ... + d^5/6) (the next term is below 2^-24 of t) with
// d = 1 - u taken from the integer: 2^53 d = (2^32 - hi) 2^21 - (k mod 2^21) - (k & 1), the f64
// sum k + 0.5 rounding to even from 2^52 on, in one fused multiply-add. d = 0 (k = 2^53 - 1, u
// rounds to 1) gives t = 0 and g = +inf, as the exact value is.
__device__ __forceinline__ float gumbel_screen(uint32_t lo, uint32_t hi) {
    constexpr float kLn2f = 0.69314718055994530942f;
    const uint32_t kl = lo >> 11;  // k's low 21 bits (its high 32 are hi)
    const float u = fmaf(float(hi), 0x1p-32f, fmaf(float(kl), 0x1p-53f, 0x1p-54f));
    const float tl = __builtin_amdgcn_logf(u) * -kLn2f;
    const float d = fmaf(float(kl + (kl & 1u)), -0x1p-53f, float(0u - hi) * 0x1p-32f);
    float ser = fmaf(d, 1.0f / 6.0f, 1.0f / 5.0f);
    ser = fmaf(ser, d, 1.0f / 4.0f);
    ser = fmaf(ser, d, 1.0f / 3.0f);
    ser = fmaf(ser, d, 0.5f);
    ser = fmaf(ser, d, 1.0f);
    const float t = hi >= 0xf0000000u ? d * ser : tl;
    return __builtin_amdgcn_logf(t) * -kLn2f;
}

constexpr int kGumbelCand = 4;         // screened candidates a thread keeps
constexpr int kGumbelQueue = 128;      // a wave's queue of blocks with an allowed element (LDS)
// The queue's dynamic LDS for a launch of `threads` threads: per wave kGumbelQueue block indices
// and their 8 values each (36 KiB at 16 waves, 2.25 KiB for a one-wave row).
constexpr size_t gumbel_queue_bytes(int threads, bool greedy) {
    return greedy ? 0 : size_t(threads / 64) * kGumbelQueue * 9 * sizeof(float);
}
constexpr float kGumbelScreen = 1e-3f;  // the screen's margin, at least: 250 times its error bound

// The lowest screened value kept as a candidate beside a largest screened value x: x less the
// larger of kGumbelScreen and |x| rel. The value compared is z + g rounded to f32, so a screened
// and an exact sum differ by the screen's error and up to an ulp of the sum; with rel = 2^-21
// (four ulps of x) the margin exceeds two such differences at every magnitude, so an element
// below it cannot reach or pass the element at x exactly. A thread keeps its own candidates
// with rel = 2^-20, a superset of the row's. (x = +inf: the candidates are the infinite values.)
__device__ __forceinline__ float screen_floor(float x, float rel) {
    return x == INFINITY ? x : x - fmaxf(kGumbelScreen, fabsf(x) * rel);
}

// The row's first maximum of z + g. Past temperature 0 it runs in two steps: every allowed
// element's value is screened in f32 (the keystream is generated, the logarithms are the
// hardware's), and only the elements whose screened value lies within the margin of the row's
// largest (screen_floor) are evaluated exactly (gumbel_f32, their keystream block generated
// again). The exact maximum is among them, since the margin covers the screen's error and the
// rounding of z + g on both sides; so a row with a single candidate has its answer without the
// exact evaluation. A thread whose candidates within the margin of its own largest outnumber its
// slots makes the row take the exact evaluation of every element instead.
template <int DT, int MK, bool ODD, bool GREEDY>
__global__ __launch_bounds__(kGumbelMaxThreads) void k_sample_gumbel(GumbelP p) {
    __shared__ float sbest[kGumbelMaxThreads / 64];
    __shared__ int sidx[kGumbelMaxThreads / 64];
    __shared__ int sflags[kGumbelMaxThreads / 64];
    __shared__ int scount[kGumbelMaxThreads / 64];
    // per wave, the queue of blocks to draw: their index and their 8 values ([8][kGumbelQueue]),
    // in dynamic LDS sized by the launch for its waves (gumbel_queue_bytes; none when greedy)
    extern __shared__ __attribute__((aligned(16))) int gdyn[];
    int *const gqb = gdyn;
    float *const gqz = reinterpret_cast<float *>(gdyn + (blockDim.x / 64) * kGumbelQueue);
    const int64_t row = blockIdx.x;
    const int64_t moff = MK != NT_MASK_NONE ? mask_row_at(p.mm, row) : 0;  // the row's mask row
    const int64_t V = p.V;
    // Pair q = h + row V + v holds element v's u64; block q >> 3, pair q & 7 of it.
    const uint64_t q0 = p.h + uint64_t(row) * uint64_t(V);
    const uint64_t b0 = q0 >> 3, b1 = (q0 + uint64_t(V) - 1) >> 3;
    const int wave = threadIdx.x / 64, nw = blockDim.x / 64, lane = threadIdx.x & 63;
    int flags = 0;  // bit 0: a candidate (z > -inf); bit 1: a NaN; bit 2: a thread's slots overflowed
    int count = 0;  // summed by the reductions
    // Every block holding an allowed element: fn(b, v0, z), z the block's 8 tempered values
    // (elements v0 .. v0 + 7; -inf outside the row). Without COMPACT each thread takes its own
    // blocks in index order. With COMPACT a wave's blocks that hold an allowed element go through
    // its queue, and each call takes whichever queued block falls to the lane, so that the
    // keystream is generated by full waves (the order does not matter to the caller:
    // its merges break ties by index).
    auto walk = [&](auto compact_c, auto &&fn) {
        constexpr bool COMPACT = decltype(compact_c)::value && !GREEDY;
        // COMPACT without an additive mask: the blocks are queued before the division by tau,
        // which is done for the queued blocks only. The NaN test gives the same answer before it
        // (tau > 0: NaN stays NaN); the candidate test does not for a finite logit below
        // -FLT_MAX tau, which the division takes to -inf, so a row's candidate flag is then set
        // from the divided values (a row whose allowed logits all lie there has no candidate and
        // is refused, as the reference's max_dim of -inf is, rl.rs:515-519).
        constexpr bool DEFER = COMPACT && MK != NT_MASK_F32;
        const int n = blockDim.x;
        // COMPACT: the row's blocks i = 0 .. nbk - 1 (keystream block b0 + i, elements
        // 8 i - r .. 8 i - r + 7), a wave's 64 consecutive ones per step, n apart. z_of(i, z) fills
        // block i's values (every lane calls it once per step, in order; -inf past the row).
        // Blocks holding an allowed element are queued with their values; each time 64 are
        // queued every lane takes one, and the rest are taken at the end.
        auto queued = [&](int nbk, int r, auto &&z_of) {
            int *qb = gqb + wave * kGumbelQueue;
            float *qz = gqz + wave * 8 * kGumbelQueue;
            int head = 0, count = 0;  // the queue's first entry and its length (uniform)
            auto pop = [&](bool have) {
                // (every lane's queue writes are in LDS before any lane reads)
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                __builtin_amdgcn_wave_barrier();
                if (have) {
                    const int e = (head + lane) % kGumbelQueue;
                    const int ie = qb[e];
                    float ze[8];
                    bool cand = false;
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        ze[j] = qz[j * kGumbelQueue + e];
                        if (DEFER && !p.tau_one) ze[j] = ze[j] / p.tau;
                        cand |= ze[j] > -INFINITY;
                    }
                    if (DEFER && !p.tau_one && cand) flags |= 1;
                    fn(b0 + uint64_t(ie), 8 * int64_t(ie) - r, ze);
                }
                // (the reads are done before a later write reuses their slots)
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                __builtin_amdgcn_wave_barrier();
            };
            // (two steps per pass: z_of keeps a set of loads in flight per step parity)
            auto step = [&](int base, auto par_c) {
                const int i = base + lane;
                float z[8];
                z_of(i, z, par_c);
                bool any = false;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    if (z[j] != z[j]) flags |= 2;
                    any |= z[j] > -INFINITY;
                }
                const uint64_t bal = __ballot(any);
                if (any) {
                    if (!DEFER || p.tau_one) flags |= 1;  // (deferred: from the divided values, in pop)
                    const int pos = (head + count + int(__builtin_amdgcn_mbcnt_hi(
                                                           uint32_t(bal >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(bal), 0u)))) %
                                    kGumbelQueue;
                    qb[pos] = i;
#pragma unroll
                    for (int j = 0; j < 8; j++) qz[j * kGumbelQueue + pos] = z[j];
                }
                count += __builtin_popcountll(bal);
                if (count >= 64) {
                    pop(true);
                    head = (head + 64) % kGumbelQueue;
                    count -= 64;
                }
            };
            for (int base = 64 * wave; base < nbk; base += 2 * n) {
                step(base, std::integral_constant<int, 0>{});
                if (base + n < nbk) step(base + n, std::integral_constant<int, 1>{});
            }
            if (count > 0) pop(lane < count);
        };
        if (!ODD && p.vec && (q0 & 7) == 0) {
            // The aligned path: keystream block b0 + i holds elements 8 i .. 8 i + 7 exactly, read
            // with one or two 16-byte loads (with the queue, issued two steps ahead of their use).
            // Loads past the row read zeros (the buffer's range) and those elements are -inf.
            const int nb = int((V + 7) / 8);
            const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<char *>(static_cast<const char *>(p.logits) + row * p.ld * (DT == NT_F32 ? 4 : 2)),
                short(0), int(V * (DT == NT_F32 ? 4 : 2)), kBufferWord3);
            __amdgpu_buffer_rsrc_t mres = xres;
            if constexpr (MK != NT_MASK_NONE)
                mres = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<char *>(static_cast<const char *>(p.mask) + moff * (MK == NT_MASK_F32 ? 4 : 1)),
                    short(0), int(V * (MK == NT_MASK_F32 ? 4 : 1)), kBufferWord3);
            GumbelRaw<DT, MK> cur, nxt;
            if constexpr (COMPACT) {
                // two steps of loads in flight: the set of a step's parity is used, then loaded
                // again for the step two ahead
                const int i0 = 64 * wave + lane;
                if (i0 < nb) gumbel_load<DT, MK>(cur, xres, mres, 8 * i0);
                if (i0 + n < nb) gumbel_load<DT, MK>(nxt, xres, mres, 8 * (i0 + n));
                queued(nb, 0, [&](int i, float (&z)[8], auto par_c) {
                    GumbelRaw<DT, MK> &rr = decltype(par_c)::value ? nxt : cur;
                    if (i < nb) {
                        gumbel_values<DT, MK, !DEFER>(rr, p, 8 * i, z);
                    } else {
#pragma unroll
                        for (int j = 0; j < 8; j++) z[j] = -INFINITY;
                    }
                    if (i + 2 * n < nb) gumbel_load<DT, MK>(rr, xres, mres, 8 * (i + 2 * n));
                });
            } else {
                int i = threadIdx.x;
                if (i < nb) gumbel_load<DT, MK>(cur, xres, mres, 8 * i);
                for (; i < nb; i += n) {
                    if (i + n < nb) gumbel_load<DT, MK>(nxt, xres, mres, 8 * (i + n));
                    float z[8];
                    gumbel_values<DT, MK>(cur, p, 8 * i, z);
                    bool any = false;
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        if (z[j] != z[j]) flags |= 2;
                        any |= z[j] > -INFINITY;
                    }
                    if (any) {
                        flags |= 1;
                        fn(b0 + uint64_t(i), 8 * int64_t(i), z);
                    }
                    cur = nxt;
                }
            }
        } else if constexpr (COMPACT) {
            // element by element: block b0 + i holds elements 8 i - r .. 8 i - r + 7
            const int r = int(q0 & 7);
            queued(int(b1 - b0 + 1), r, [&](int i, float (&z)[8], auto) {
                const int64_t v0 = 8 * int64_t(i) - r;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int64_t v = v0 + j;
                    z[j] = (v >= 0 && v < V) ? tempered_at<DT, MK, !DEFER>(p, row, moff, v) : -INFINITY;
                }
            });
        } else {
            for (uint64_t b = b0 + threadIdx.x; b <= b1; b += blockDim.x) {
                const int64_t v0 = int64_t(8 * b - q0);  // element of pair 0 of block b (may be < 0)
                float z[8];
                bool any = false;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int64_t v = v0 + j;
                    z[j] = (v >= 0 && v < V) ? tempered_at<DT, MK>(p, row, moff, v) : -INFINITY;
                    if (z[j] != z[j]) flags |= 2;
                    any |= z[j] > -INFINITY;
                }
                if (any) {
                    flags |= 1;
                    fn(b, v0, z);
                }
            }
        }
    };
    // Each allowed element of a block with its stream words: fn(v, z, lo, hi).
    auto draws = [&](uint64_t b, int64_t v0, const float (&z)[8], auto &&fn) {
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
                fn(v0 + j, z[j], lo, hi);
            }
        }
    };
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    // the exact evaluation of one element, into this thread's first maximum
    auto exact = [&](int64_t v, float zj, uint32_t lo, uint32_t hi) {
        best_merge(best, bidx, zj + gumbel_f32(lo, hi), int(v));
    };
    // the workgroup's (best, bidx) first maximum, OR of the flags and sum of the counts: a fixed
    // butterfly inside each wave, then the waves in order (the result in every thread)
    auto reduce_best = [&]() {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ob = __shfl_xor(best, o, 64);
            const int oi = __shfl_xor(bidx, o, 64);
            best_merge(best, bidx, ob, oi);
            flags |= __shfl_xor(flags, o, 64);
            count += __shfl_xor(count, o, 64);
        }
        if (lane == 0) {
            sbest[wave] = best;
            sidx[wave] = bidx;
            sflags[wave] = flags;
            scount[wave] = count;
        }
        __syncthreads();
        float rb = sbest[0];
        int ri = sidx[0], rf = sflags[0], rc = scount[0];
        for (int i = 1; i < nw; i++) {
            best_merge(rb, ri, sbest[i], sidx[i]);
            rf |= sflags[i];
            rc += scount[i];
        }
        __syncthreads();  // (the arrays are written again by a later reduction)
        best = rb;
        bidx = ri;
        flags = rf;
        count = rc;
    };
    if constexpr (GREEDY) {
        walk(std::false_type{}, [&](uint64_t, int64_t v0, const float (&z)[8]) {
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (z[j] > best) {  // strictly greater: the first maximum of this thread's elements
                    best = z[j];
                    bidx = int(v0 + j);
                }
        });
        reduce_best();
    } else {
        // ---- the screen: the thread's largest screened value and its candidates within the margin
        // (four slots as separate values: an array here would be indexed through memory)
        static_assert(kGumbelCand == 4, "the four slots below");
        float amax = -INFINITY;
        float ca0 = -INFINITY, ca1 = -INFINITY, ca2 = -INFINITY, ca3 = -INFINITY;  // screened values
        float cz0 = 0.0f, cz1 = 0.0f, cz2 = 0.0f, cz3 = 0.0f;                       // tempered logits
        int cv0 = 0, cv1 = 0, cv2 = 0, cv3 = 0;                                     // elements
        walk(std::true_type{}, [&](uint64_t b, int64_t v0, const float (&z)[8]) {
            draws(b, v0, z, [&](int64_t v, float zj, uint32_t lo, uint32_t hi) {
                const float a = zj + gumbel_screen(lo, hi);
                if (a > amax) amax = a;
                const float lo_keep = screen_floor(amax, 0x1p-20f);
                if (a >= lo_keep) {
                    // into the first slot that holds nothing within the margin (slots are reused)
                    bool placed = false;
                    auto slot = [&](float &ca, float &cz, int &cv) {
                        if (!placed && !(ca >= lo_keep)) {
                            ca = a;
                            cz = zj;
                            cv = int(v);
                            placed = true;
                        }
                    };
                    slot(ca0, cz0, cv0);
                    slot(ca1, cz1, cv1);
                    slot(ca2, cz2, cv2);
                    slot(ca3, cz3, cv3);
                    if (!placed) flags |= 4;
                }
            });
        });
        // the row's largest screened value and the flags
        best = amax;
        bidx = 0;
        reduce_best();
        const float amx = best, lo_row = screen_floor(amx, 0x1p-21f);
        // the candidates within the row's margin: when there is one, it is the row's exact first
        // maximum (every other element lies below it exactly), and its index is the answer
        best = -INFINITY;
        bidx = 0x7fffffff;
        count = 0;
        auto offer = [&](float ca, int cv) {
            if (ca >= lo_row) {
                best_merge(best, bidx, ca, cv);
                count++;
            }
        };
        offer(ca0, cv0);
        offer(ca1, cv1);
        offer(ca2, cv2);
        offer(ca3, cv3);
        reduce_best();
        if ((flags & 2) || !(flags & 1) || (count == 1 && !(flags & 4))) {
            // a refused row (a NaN, or nothing allowed), or bidx is the one candidate's (with no
            // thread's slots overflowed: an element left out of them could lie within the margin)
        } else if (flags & 4) {
            best = -INFINITY;
            bidx = 0x7fffffff;
            // a thread ran out of slots: every element exactly
            walk(std::true_type{}, [&](uint64_t b, int64_t v0, const float (&z)[8]) { draws(b, v0, z, exact); });
            reduce_best();
        } else {
            // the candidates within the margin of the row's largest, exactly (their blocks again)
            best = -INFINITY;
            bidx = 0x7fffffff;
            auto resolve = [&](float ca, float cz, int cv) {
                const bool take = ca >= lo_row;
                if (__ballot(take) == 0) return;
                if (take) {
                    const uint64_t w0 = 2 * (q0 + uint64_t(cv)) + (ODD ? 1 : 0);  // its low word
                    uint32_t w[16];
                    chacha_block_dev(p.key, w0 >> 4, w);
                    uint32_t lo = w[0], hi = w[0];
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        if (e == int(w0 & 15)) lo = w[e];
                        if (e == int((w0 + 1) & 15)) hi = w[e];
                    }
                    if ((w0 & 15) == 15) {  // the high word opens the next block
                        uint32_t w2[16];
                        chacha_block_dev(p.key, (w0 >> 4) + 1, w2);
                        hi = w2[0];
                    }
                    exact(cv, cz, lo, hi);
                }
            };
            resolve(ca0, cz0, cv0);
            resolve(ca1, cz1, cv1);
            resolve(ca2, cz2, cv2);
            resolve(ca3, cz3, cv3);
            reduce_best();
        }
    }
    if (threadIdx.x != 0) return;
    // The reference refuses a row whose maximum is NaN (any NaN: max_dim propagates it) or -inf
    // (rl.rs:515-519).
    if (flags & 2) {
        p.ids[row] = -1;
        p.status[row] = NT_ROW_NAN;
    } else if (!(flags & 1)) {
        p.ids[row] = -1;
        p.status[row] = NT_ROW_NO_TOKEN;
    } else {
        p.ids[row] = bidx;
        p.status[row] = NT_ROW_OK;
    }
}

}  // namespace
}  // namespace nt
