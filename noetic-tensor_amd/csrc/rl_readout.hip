// The readout-fused sampler: one decode step's readout product and its masked inverse-CDF
// sample + log-probability, without writing the logits.
//
// The reference computes the logits as the decoder's readout `x · W` (src/nn/decoder.rs:272,286;
// a Linear is one matmul, src/nn/linear.rs:1-3) into a [rows, V] tensor and then runs nn::rl on
// it (tempered_logits, the sampler, token_log_probs: rl.rs:134-141, 475-529). Here:
//
//  Pass 1 (k_readout_tiles): logits = h · W on the matrix cores, bf16 operands and f32
//  accumulation (v_mfma_f32_32x32x16_bf16, as the reference's half-precision product,
//  src/tensor/gpu/half_gemm.rs:1-10). One 512-thread workgroup owns 256 vocabulary columns for
//  every row (up to 256 rows); each wave a 128 x 64 part as 4 x 2 MFMA tiles. Both operands are
//  in fragment order (the weight packed once by nt_hip_rl_readout_pack_weight, h per call), so
//  one k-step's operands for 32 rows or columns are 1 KiB contiguous, which the load unit copies
//  straight into LDS (buffer_load ... lds), nine 16 KiB stages deep, eight in flight. The
//  epilogue turns the tile into the sampler's per-row records instead of writing it: the tile's
//  maximum and exponent reference, and the sum of the weights 2^(x c - ref) of each 32-column
//  block (f32). A debug pointer also writes the logits.
//
//  Pass 2 (k_readout_resolve): one workgroup per row merges the records in index order in f64,
//  finds the block holding u S, recomputes that block's 32 logits with the same MFMA chain (the
//  same instruction over the same k order from zero, so the values equal pass 1's bit for bit)
//  and resolves the draw inside it, as the fused sampler's phase 3 does.
//
// HBM traffic: the weight once (V d 2 bytes), the mask once, h from the L2 (2 MB, shared by all
// tiles), the records (12 bytes per row per 32 columns, written and read once) and, per row, the
// crossing block's 32 weight rows again (32 d 2 bytes).
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <string>

#include "../../include/noetic_hip.h"
#include "nt_internal.hpp"

namespace nt {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void *lds_ptr_t;

constexpr int kRoThreads = 512;       // 8 waves: two per SIMD, so one wave's LDS reads overlap the other's MFMAs
constexpr int kRoCols = 256;          // vocabulary columns per workgroup (tile)
constexpr int kRoRows = 256;          // rows per launch at most
constexpr int64_t kRoMaxVocab = 262144;  // the resolve's per-thread block and tile arrays
constexpr int kRoBlock = 32;          // columns per record block
constexpr int kRoDepth = 8;           // k-steps of 16 in flight
constexpr int kRoStages = kRoDepth + 1;
constexpr int kRoStageBytes = 16384;  // 8 A fragments + 8 B fragments of 1 KiB
constexpr int kBufferWord3 = 0x00020000;
constexpr float kLog2e = 1.44269504088896340736f;
constexpr double kLn2 = 0.69314718055994530942;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Wait until at most n (an even number up to 16) vector memory operations of this wave are
// outstanding.
__device__ __forceinline__ void wait_vmcnt_upto16(int n) {
    switch (n) {
        case 0: wait_vmcnt<0>(); break;
        case 2: wait_vmcnt<2>(); break;
        case 4: wait_vmcnt<4>(); break;
        case 6: wait_vmcnt<6>(); break;
        case 8: wait_vmcnt<8>(); break;
        case 10: wait_vmcnt<10>(); break;
        case 12: wait_vmcnt<12>(); break;
        case 14: wait_vmcnt<14>(); break;
        default: wait_vmcnt<16>(); break;
    }
}

// Wait until at most 2 n vector memory operations of this wave are outstanding (n in 0..7): the
// DMAs of the n k-steps issued after the one awaited.
__device__ __forceinline__ void wait_vmcnt_steps(int n) {
    switch (n) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<2>(); break;
        case 2: wait_vmcnt<4>(); break;
        case 3: wait_vmcnt<6>(); break;
        case 4: wait_vmcnt<8>(); break;
        case 5: wait_vmcnt<10>(); break;
        case 6: wait_vmcnt<12>(); break;
        default: wait_vmcnt<14>(); break;
    }
}

// Fragment order: the MFMA operands of 32 rows (or vocabulary columns) g 32 .. g 32 + 31 for
// k-step s (k 16 s .. 16 s + 15) are 1 KiB at ((g S + s) 64 + l) 16 bytes, lane l holding row
// g 32 + l % 32 at k 16 s + 8 (l / 32) .. + 7: a DMA of one fragment reads 1 KiB contiguous.
struct ReadoutP {
    const uint8_t *hp;   // h in fragment order, ceil(rows / 32) row groups
    const uint8_t *wp;   // the weight in fragment order, ceil(V / 32) column groups
    int rows, V, K;
    int ntile, nblk;     // tiles of 256 columns, blocks of 32 columns
    const uint8_t *mask; // u8 keep-mask [rows, mask_ld] or null
    int64_t mask_ld;
    int mask_vec;        // mask rows 16-byte aligned: 16-byte loads
    float c;             // log2(e) / T
    float *tref;         // [rows][ntile] the tile's exponent reference RN(max c) (-inf: nothing allowed)
    float *tmax;         // [rows][ntile] the tile's maximum of the allowed logits
    int *tfirst;         // [rows][ntile] the first column holding it
    float *bsum;         // [rows][nblk] the block's sum of 2^(x c - tref)
    float *logits;       // [rows][V] debug copy or null
};

// Six 16-byte LDS reads (four A fragments 1 KiB apart, two B fragments) and the wait for them,
// in one statement: the data came from LDS DMA, which the compiler's own wait insertion would
// treat as outstanding vector memory (a wait for every load in flight).
__device__ __forceinline__ void lds_read_frags(uint32_t a, uint32_t b, v4u (&fa)[4], v4u (&fb)[2]) {
    asm volatile(
        "ds_read_b128 %0, %6\n\t"
        "ds_read_b128 %1, %6 offset:1024\n\t"
        "ds_read_b128 %2, %6 offset:2048\n\t"
        "ds_read_b128 %3, %6 offset:3072\n\t"
        "ds_read_b128 %4, %7\n\t"
        "ds_read_b128 %5, %7 offset:1024\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(fa[0]), "=&v"(fa[1]), "=&v"(fa[2]), "=&v"(fa[3]), "=&v"(fb[0]), "=&v"(fb[1])
        : "v"(a), "v"(b)
        : "memory");
}

template <bool MASK, bool DBG>
__global__ __launch_bounds__(kRoThreads) void k_readout_tiles(ReadoutP p) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[kRoStages * kRoStageBytes];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rh = wave >> 2, cq = wave & 3;  // this wave's 128 rows and 64 columns
    const int tile = blockIdx.x;
    const int n0 = tile * kRoCols;
    const int ncols = min(kRoCols, p.V - n0);
    const int S = p.K / 16;
    // Buffer resources over the packed operands: reads past the row groups (or past the
    // vocabulary's column groups) return zeros.
    const int hgroups = (p.rows + 31) / 32, wgroups = (ncols + 31) / 32;
    const __amdgpu_buffer_rsrc_t hres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(p.hp), short(0), hgroups * S * 1024, kBufferWord3);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(p.wp + int64_t(n0 / 32) * S * 1024), short(0), wgroups * S * 1024, kBufferWord3);
    const uint32_t lbase = uint32_t((uintptr_t)(lds_ptr_t)(lds));
    // This wave's DMA share of a k-step: A fragment `wave` (row group) and B fragment `wave`
    // (column group of the tile), 1 KiB contiguous each in fragment order; lane l's 16 bytes land
    // at 16 l of the fragment's LDS slot, the MFMA operand of that lane.
    const int fr = lane & 31;
    const int frag = wave * S * 1024 + lane * 16;
    auto issue = [&](int s) {
        uint8_t *st = lds + (s % kRoStages) * kRoStageBytes;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(hres, (lds_ptr_t)(st + wave * 1024), 16, frag + s * 1024, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wres, (lds_ptr_t)(st + 8192 + wave * 1024), 16, frag + s * 1024, 0, 0, 0);
    };
    f32x16_t acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;
    const int pre = S < kRoDepth ? S : kRoDepth;
    for (int s = 0; s < pre; s++) issue(s);
    for (int s = 0; s < S; s++) {
        // step s's fragments (this wave's DMAs) have landed once at most 2 (steps in flight after
        // it) remain; the barrier makes every wave's visible and retires step s - 1's reads
        const int after = min(S - 1 - s, kRoDepth - 1);
        if (after == kRoDepth - 1) wait_vmcnt<2 * (kRoDepth - 1)>();
        else wait_vmcnt_steps(after);
        // a bare barrier: each wave has waited for its own DMAs above, and LDS is coherent within
        // the workgroup (__syncthreads' fence would wait for every DMA in flight)
        asm volatile("s_barrier" ::: "memory");
        if (s + kRoDepth < S) issue(s + kRoDepth);
        const uint32_t sb = lbase + (s % kRoStages) * kRoStageBytes + lane * 16;
        v4u fa[4], fb[2];
        lds_read_frags(sb + rh * 4096, sb + 8192 + cq * 2048, fa, fb);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, fa[i]),
                                                                    __builtin_bit_cast(bf16x8_t, fb[j]), acc[i][j], 0, 0, 0);
    }
    __syncthreads();

    // ---- epilogue: eight passes of 32 rows x 256 columns through LDS ([32][256 + 4] f32). In pass
    // q the four waves holding rows 32 q .. 32 q + 31 store them; then thread t < 256 takes row
    // t / 8 and the 32 columns 32 (t % 8) .. + 31 of it.
    float *T = reinterpret_cast<float *>(lds);
    constexpr int TLD = kRoCols + 4;
    const int prow = tid >> 3, part = tid & 7;
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const int qh = q >> 2, qi = q & 3;  // row half and row tile within it (constants once unrolled)
        if (rh == qh) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int r = 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
                    T[r * TLD + cq * 64 + j * 32 + fr] = acc[qi][j][v];
                }
        }
        __syncthreads();
        if (tid >= 256) {  // 256 threads take the 32 rows x 256 columns
            __syncthreads();
            continue;
        }
        const int row = 32 * q + prow;
        const int col0 = n0 + 32 * part;
        float x[32];
#pragma unroll
        for (int e = 0; e < 32; e += 4) {
            const float4 f = *reinterpret_cast<const float4 *>(&T[prow * TLD + 32 * part + e]);
            x[e] = f.x;
            x[e + 1] = f.y;
            x[e + 2] = f.z;
            x[e + 3] = f.w;
        }
        const bool live = row < p.rows;
        if constexpr (DBG) {
            if (live)
#pragma unroll
                for (int e = 0; e < 32; e++)
                    if (col0 + e < p.V) p.logits[int64_t(row) * p.V + col0 + e] = x[e];
        }
        // the sampler's values: an excluded column or one past the vocabulary is -inf
        uint32_t mw[8];
        if constexpr (MASK) {
            const uint8_t *mrow = p.mask + (live ? int64_t(row) * p.mask_ld : 0) + col0;
#pragma unroll
            for (int e = 0; e < 8; e++) mw[e] = 0;
            if (live && col0 + 32 <= p.V && p.mask_vec) {
                const uint4 m0 = *reinterpret_cast<const uint4 *>(mrow);
                const uint4 m1 = *reinterpret_cast<const uint4 *>(mrow + 16);
                mw[0] = m0.x; mw[1] = m0.y; mw[2] = m0.z; mw[3] = m0.w;
                mw[4] = m1.x; mw[5] = m1.y; mw[6] = m1.z; mw[7] = m1.w;
            } else if (live) {
                for (int e = 0; e < 32 && col0 + e < p.V; e++) mw[e / 4] |= uint32_t(mrow[e]) << (8 * (e % 4));
            }
        }
        float m = -INFINITY;
        int first = 0x7fffffff;
#pragma unroll
        for (int e = 0; e < 32; e++) {
            bool keep = live && col0 + e < p.V;
            if constexpr (MASK) keep = keep && ((mw[e / 4] >> (8 * (e % 4))) & 0xffu) != 0;
            x[e] = keep ? x[e] : -INFINITY;
            if (x[e] > m) {
                m = x[e];
                first = col0 + e;
            }
        }
        // the tile's maximum over the row's eight threads (consecutive lanes), the first column
        // holding it
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) {
            const float om = __shfl_xor(m, o, 64);
            const int of = __shfl_xor(first, o, 64);
            if (om > m || (om == m && of < first)) {
                m = om;
                first = of;
            }
        }
        const float ref = m * p.c;  // RN(max c); -inf when nothing is allowed
        float w[32];
#pragma unroll
        for (int e = 0; e < 32; e++) w[e] = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(fmaf(x[e], p.c, -ref));
        // the block's sum in a fixed tree
#pragma unroll
        for (int span = 1; span < 32; span <<= 1)
#pragma unroll
            for (int e = 0; e < 32; e += 2 * span) w[e] = w[e] + w[e + span];
        const int blk = tile * (kRoCols / kRoBlock) + part;
        if (live && blk < p.nblk) p.bsum[int64_t(row) * p.nblk + blk] = w[0];
        if (live && part == 0) {
            p.tref[int64_t(row) * p.ntile + tile] = ref;
            p.tmax[int64_t(row) * p.ntile + tile] = m;
            p.tfirst[int64_t(row) * p.ntile + tile] = first;
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------ pass 2: resolve

struct ResolveP {
    const uint16_t *h;   // [rows, ldh] bf16, row-major
    const uint8_t *wp;   // the weight in fragment order
    int rows, V, K, ldh, ntile, nblk;
    const uint8_t *mask;
    int64_t mask_ld;
    float c, tau;
    int tau_one, greedy;
    const float *tref, *tmax;
    const int *tfirst;
    const float *bsum;
    const double *u;
    int32_t *ids;
    float *logp;
    uint8_t *status;
    float *dbg_block;  // [rows][32] the recomputed logits of the crossing block, or null
    int *dbg_index;    // [rows] that block's index, or null
};

constexpr int kResThreads = 256;
constexpr int kResMaxBlocks = 32;  // blocks of 32 columns per thread: V <= 262144
constexpr int kResMaxTiles = 4;    // tiles of 256 columns per thread
constexpr int kResPhase = 16;     // k-steps per phase of the recomputation's ring
constexpr int kResSlots = 4;      // phases in the ring (three in flight)

// Sixteen 16-byte LDS reads: the A and B fragments of eight consecutive k-steps (2 KiB apart,
// B 1 KiB after A), and the wait for them (see lds_read_frags).
__device__ __forceinline__ void lds_read_8x2(uint32_t a, v4u (&fa)[8], v4u (&fb)[8]) {
    asm volatile(
        "ds_read_b128 %0, %16\n\t"
        "ds_read_b128 %1, %16 offset:2048\n\t"
        "ds_read_b128 %2, %16 offset:4096\n\t"
        "ds_read_b128 %3, %16 offset:6144\n\t"
        "ds_read_b128 %4, %16 offset:8192\n\t"
        "ds_read_b128 %5, %16 offset:10240\n\t"
        "ds_read_b128 %6, %16 offset:12288\n\t"
        "ds_read_b128 %7, %16 offset:14336\n\t"
        "ds_read_b128 %8, %16 offset:1024\n\t"
        "ds_read_b128 %9, %16 offset:3072\n\t"
        "ds_read_b128 %10, %16 offset:5120\n\t"
        "ds_read_b128 %11, %16 offset:7168\n\t"
        "ds_read_b128 %12, %16 offset:9216\n\t"
        "ds_read_b128 %13, %16 offset:11264\n\t"
        "ds_read_b128 %14, %16 offset:13312\n\t"
        "ds_read_b128 %15, %16 offset:15360\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(fa[0]), "=&v"(fa[1]), "=&v"(fa[2]), "=&v"(fa[3]), "=&v"(fa[4]), "=&v"(fa[5]), "=&v"(fa[6]), "=&v"(fa[7]),
          "=&v"(fb[0]), "=&v"(fb[1]), "=&v"(fb[2]), "=&v"(fb[3]), "=&v"(fb[4]), "=&v"(fb[5]), "=&v"(fb[6]), "=&v"(fb[7])
        : "v"(a)
        : "memory");
}

// Inclusive prefix sum over the 64 lanes in f64 by a fixed sequence of shuffles.
__device__ __forceinline__ double wave_incl_scan(double v, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
    }
    return v;
}

__global__ __launch_bounds__(kResThreads) void k_readout_resolve(ResolveP p) {
    __shared__ double wsum[kResThreads / 64];
    __shared__ float wmax[kResThreads / 64];
    __shared__ int wsel[kResThreads / 64];
    __shared__ int s_blk;
    __shared__ double s_tl;
    __shared__ __attribute__((aligned(16))) uint8_t ring[kResSlots * kResPhase * 2048];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *tref = p.tref + int64_t(row) * p.ntile;
    const float *tmax = p.tmax + int64_t(row) * p.ntile;
    const int *tfirst = p.tfirst + int64_t(row) * p.ntile;
    const float *bsum = p.bsum + int64_t(row) * p.nblk;
    auto refuse = [&](uint8_t st) {
        if (tid == 0) {
            p.ids[row] = -1;
            if (p.logp) p.logp[row] = NAN;
            p.status[row] = st;
        }
    };
    // ---- the row's maximum over the tiles (exact; the order does not matter for a maximum)
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < kResMaxTiles; i++) {
        const int t = tid + i * kResThreads;
        if (t < p.ntile) m = fmaxf(m, tmax[t]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (lane == 0) wmax[wave] = m;
    __syncthreads();
    const float M = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    if (M == -INFINITY) {
        refuse(NT_ROW_NO_TOKEN);
        return;
    }
    const float A = M * p.c;
    // ---- block weights relative to A, each thread a contiguous run of blocks, f64 in index order
    const int per = (p.nblk + kResThreads - 1) / kResThreads;  // at most kResMaxBlocks
    const int b0 = tid * per, b1 = min(p.nblk, b0 + per);
    // every load of the thread's blocks first (one wait), then the f64 sums in order
    float bs[kResMaxBlocks], br[kResMaxBlocks];
#pragma unroll
    for (int i = 0; i < kResMaxBlocks; i++) {
        const int b = b0 + i;
        const bool in = i < per && b < b1;
        bs[i] = in ? bsum[b] : 0.0f;
        br[i] = in ? tref[b / (kRoCols / kRoBlock)] : -INFINITY;
    }
    double wbk[kResMaxBlocks];
    double run = 0.0;
#pragma unroll
    for (int i = 0; i < kResMaxBlocks; i++) {
        const double f = br[i] == -INFINITY ? 0.0 : double(__builtin_amdgcn_exp2f(br[i] - A));
        wbk[i] = f * double(bs[i]);
        run += wbk[i];
    }
    const double incl_w = wave_incl_scan(run, lane);
    if (lane == 63) wsum[wave] = incl_w;
    __syncthreads();
    double before = 0.0;
    for (int w2 = 0; w2 < wave; w2++) before += wsum[w2];
    const double incl = before + incl_w, excl = incl - run;
    // the row's sum: the last thread's inclusive prefix (the same additions in the same order)
    __shared__ double s_tot;
    if (tid == kResThreads - 1) s_tot = incl;
    __syncthreads();
    const double Sall = s_tot;
    if (!(Sall == Sall)) {
        refuse(NT_ROW_NAN);
        return;
    }
    const double shiftA = double(A) - double(M) * double(p.c);
    const double lnS = log(Sall) + shiftA * kLn2;
    if (p.greedy) {
        // the first column holding the maximum: the first tile whose maximum it is
        int best = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < kResMaxTiles; i++) {
            const int t = tid + i * kResThreads;
            if (t < p.ntile && tmax[t] == M) best = min(best, tfirst[t]);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) best = min(best, __shfl_xor(best, o, 64));
        if (lane == 0) wsel[wave] = best;
        __syncthreads();
        if (tid == 0) {
            const int id = min(min(wsel[0], wsel[1]), min(wsel[2], wsel[3]));
            p.ids[row] = id;
            if (p.logp) p.logp[row] = float(-lnS);  // z_id - m = 0 exactly
            p.status[row] = NT_ROW_OK;
        }
        return;
    }
    // ---- the block holding t = u S: the first thread whose inclusive prefix passes t (with
    // weight), then its blocks in order; rounding that leaves no crossing takes the last weight
    const double t = p.u[row] * Sall;
    {
        const uint64_t cross = __ballot(incl > t && run > 0.0);
        const uint64_t any = __ballot(run > 0.0);
        if (lane == 0) wsel[wave] = cross ? wave * 64 + __builtin_ctzll(cross) : -1;
        __shared__ int wlast[kResThreads / 64];
        if (lane == 0) wlast[wave] = any ? wave * 64 + 63 - __builtin_clzll(any) : -1;
        __syncthreads();
        int sel = -1;
        for (int w2 = 0; w2 < 4 && sel < 0; w2++) sel = wsel[w2];
        if (sel < 0)
            for (int w2 = 3; w2 >= 0 && sel < 0; w2--) sel = wlast[w2];
        if (tid == 0) s_blk = -1;
        __syncthreads();
        if (tid == sel) {
            double acc = excl;
            int bstar = -1, blast = -1;
            double bexcl = 0.0, lexcl = 0.0;
#pragma unroll
            for (int i = 0; i < kResMaxBlocks; i++) {
                const double wb = wbk[i];
                if (wb > 0.0) {
                    blast = b0 + i;
                    lexcl = acc;
                }
                if (bstar < 0 && wb > 0.0 && acc + wb > t) {
                    bstar = b0 + i;
                    bexcl = acc;
                }
                acc += wb;
            }
            if (bstar < 0) {
                bstar = blast;
                bexcl = lexcl;
            }
            const float r = tref[bstar / (kRoCols / kRoBlock)];
            s_blk = bstar;
            // the target inside the block, in the scale of its tile's reference
            s_tl = (t - bexcl) * double(__builtin_amdgcn_exp2f(A - r));
        }
        __syncthreads();
    }
    const int bstar = s_blk;
    if (bstar < 0) {
        refuse(NT_ROW_NAN);
        return;
    }
    const double tl = s_tl;
    // ---- recompute the block's 32 logits: the same MFMA over the same k order from zero. Every
    // lane's A row is this row (so every output row holds it); lane l's B column is 32 b + l % 32.
    // The four waves copy the operand fragments into an LDS ring by DMA, three phases of 16
    // k-steps ahead; wave 0 runs the MFMA chain from LDS.
    const int fr = lane & 31, fk = 8 * (lane >> 5);
    const int col = bstar * kRoBlock + fr;
    const bool colok = col < p.V;
    const int S2 = p.K / 16;
    const int NP = (S2 + kResPhase - 1) / kResPhase;
    // the row of h (every lane's A operand: k 16 s + 8 (l / 32) .. + 7 of it) and the block's
    // column group of the packed weight (1 KiB per k-step, the B operands in lane order)
    const __amdgpu_buffer_rsrc_t hres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(p.h + int64_t(row) * p.ldh), short(0), p.K * 2, kBufferWord3);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(p.wp + int64_t(bstar) * S2 * 1024), short(0), S2 * 1024, kBufferWord3);
    const int hoff = fk * 2, woff = lane * 16;
    const uint32_t rbase = uint32_t((uintptr_t)(lds_ptr_t)(ring));
    // phase q: step q 16 + i is issued by wave i % 4 (two DMAs: its A and B fragments), into
    // slot (q % 4) of the ring: 16 steps x 2 KiB
    auto issue_phase = [&](int q) {
        for (int i = wave; i < kResPhase; i += 4) {
            const int st = q * kResPhase + i;
            if (st < S2) {
                uint8_t *d = ring + ((q % kResSlots) * kResPhase + i) * 2048;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(hres, (lds_ptr_t)(d), 16, hoff + st * 32, 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wres, (lds_ptr_t)(d + 1024), 16, woff + st * 1024, 0, 0, 0);
            }
        }
    };
    // the DMAs this wave issues for phase q: two per step i = wave, wave + 4, ... below S2
    auto own_dmas = [&](int q) {
        int n = 0;
        for (int i = wave; i < kResPhase; i += 4) n += q * kResPhase + i < S2 ? 2 : 0;
        return n;
    };
    const int pre = NP < kResSlots - 1 ? NP : kResSlots - 1;
    for (int q = 0; q < pre; q++) issue_phase(q);
    f32x16_t acc;
#pragma unroll
    for (int v = 0; v < 16; v++) acc[v] = 0.0f;
    for (int q = 0; q < NP; q++) {
        // this wave's DMAs of phase q have landed when at most those it issued for the (up to
        // two) phases after it remain
        int later = 0;
        for (int q2 = q + 1; q2 < NP && q2 < q + kResSlots - 1; q2++) later += own_dmas(q2);
        wait_vmcnt_upto16(later);
        asm volatile("s_barrier" ::: "memory");
        if (q + kResSlots - 1 < NP) issue_phase(q + kResSlots - 1);
        if (wave == 0) {
            const uint32_t pb = rbase + (q % kResSlots) * kResPhase * 2048 + lane * 16;
            const int n = min(kResPhase, S2 - q * kResPhase);
            for (int i0 = 0; i0 < n; i0 += 8) {
                v4u fa[8], fb[8];
                lds_read_8x2(pb + i0 * 2048, fa, fb);
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (i0 + i < n)
                        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, fa[i]),
                                                                      __builtin_bit_cast(bf16x8_t, fb[i]), acc, 0, 0, 0);
            }
        }
    }
    if (wave != 0) return;
    // lane l (< 32) holds column 32 b + l (output row 0, every row being this row)
    float x = acc[0];
    if (p.dbg_block && lane < 32) p.dbg_block[int64_t(row) * 32 + lane] = x;
    if (p.dbg_index && lane == 0) p.dbg_index[row] = bstar;
    bool keep = lane < 32 && colok;
    if (keep && p.mask) keep = p.mask[int64_t(row) * p.mask_ld + col] != 0;
    x = keep ? x : -INFINITY;
    const float r = p.tref[int64_t(row) * p.ntile + bstar / (kRoCols / kRoBlock)];
    const float w = keep ? __builtin_amdgcn_exp2f(fmaf(x, p.c, -r)) : 0.0f;
    const double cw = wave_incl_scan(double(w), lane);
    int lsel = -1;
    {
        const uint64_t c1 = __ballot(cw > tl && w > 0.0f);
        if (c1) lsel = __builtin_ctzll(c1);
        else {
            const uint64_t c2 = __ballot(w > 0.0f);
            lsel = c2 ? 63 - __builtin_clzll(c2) : -1;
        }
    }
    if (lsel < 0) {
        refuse(NT_ROW_NAN);
        return;
    }
    if (lane == lsel) {
        const float zid = p.tau_one ? x : x / p.tau;
        const float mz = p.tau_one ? M : M / p.tau;
        p.ids[row] = bstar * kRoBlock + lane;
        if (p.logp) p.logp[row] = float((double(zid) - double(mz)) - lnS);
        p.status[row] = NT_ROW_OK;
    }
}

// ------------------------------------------------------------------ packing

// Fragment order (see ReadoutP) of a [R, K] bf16 matrix: k contiguous (row r at src + r ld) or,
// K_MAJOR, the transpose of a [K, R] one (row r is column r of src, k at src + k ld + r). Rows
// from R up to the next multiple of 32 are zeros. One thread writes one lane's 16 bytes.
template <bool K_MAJOR>
__global__ void k_pack_frags(const uint16_t *src, int R, int K, int64_t ld, v4u *out, int64_t total) {
    const int S = K / 16;
    for (int64_t idx = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; idx < total;
         idx += int64_t(gridDim.x) * blockDim.x) {
        const int l = int(idx % 64);
        const int64_t gs = idx / 64;
        const int s = int(gs % S);
        const int64_t g = gs / S;
        const int64_t r = g * 32 + (l & 31);
        const int k0 = 16 * s + 8 * (l >> 5);
        v4u v = {0, 0, 0, 0};
        if (r < R) {
            if constexpr (!K_MAJOR) {
                v = *reinterpret_cast<const v4u *>(src + r * ld + k0);
            } else {
                uint32_t w4[4];
#pragma unroll
                for (int j = 0; j < 4; j++)
                    w4[j] = uint32_t(src[int64_t(k0 + 2 * j) * ld + r]) |
                            (uint32_t(src[int64_t(k0 + 2 * j + 1) * ld + r]) << 16);
                v = v4u{w4[0], w4[1], w4[2], w4[3]};
            }
        }
        out[idx] = v;
    }
}

int launch_pack(const void *src, int R, int K, int64_t ld, bool k_major, void *out) {
    const int64_t total = int64_t((R + 31) / 32) * (K / 16) * 64;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    const dim3 g{unsigned(blocks), 1, 1}, b{256, 1, 1};
    if (k_major)
        hipLaunchKernelGGL(k_pack_frags<true>, g, b, 0, ctx().stream, static_cast<const uint16_t *>(src), R, K, ld,
                           static_cast<v4u *>(out), total);
    else
        hipLaunchKernelGGL(k_pack_frags<false>, g, b, 0, ctx().stream, static_cast<const uint16_t *>(src), R, K, ld,
                           static_cast<v4u *>(out), total);
    return launched("readout pack");
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" int64_t nt_hip_rl_readout_packed_bytes(int64_t vocab, int64_t dim) {
    if (vocab < 1 || dim < 16 || dim % 16 != 0) return -1;
    return (vocab + 31) / 32 * 32 * dim * 2;
}

extern "C" int nt_hip_rl_readout_pack_weight(const void *weight, int32_t layout, int64_t vocab, int64_t dim,
                                             int64_t ld, void *packed) {
    const char *who = "nt_hip_rl_readout_pack_weight";
    const bool dv = layout == NT_READOUT_W_DV;
    if ((layout != NT_READOUT_W_VD && !dv) || vocab < 1 || vocab > kRoMaxVocab || dim < 16 || dim % 16 != 0 ||
        !weight || !packed || ld < (dv ? vocab : dim) || (!dv && (ld % 8 != 0 || reinterpret_cast<uintptr_t>(weight) % 16)) ||
        reinterpret_cast<uintptr_t>(packed) % 16 || (vocab + 31) / 32 * (dim / 16) * 1024 >= (int64_t(1) << 31))
        return fail(NT_E_ARG, std::string(who) + ": layout " + std::to_string(layout) + ", vocab " +
                                  std::to_string(vocab) + " (at most 262144), dim " + std::to_string(dim) +
                                  " (a multiple of 16), ld " + std::to_string(ld) +
                                  " (at least the row; [V, d] rows a multiple of 8 and 16-byte aligned)");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    return launch_pack(weight, int(vocab), int(dim), ld, dv, packed);
}

extern "C" int nt_hip_rl_readout_sample(const NtRlReadoutSampleArgs *a) {
    const char *who = "nt_hip_rl_readout_sample";
    if (!a) return fail(NT_E_ARG, std::string(who) + ": null args");
    const int64_t rows = a->rows, V = a->vocab, K = a->dim;
    if (rows < 0 || rows > kRoRows || V < 1 || V > kRoMaxVocab || K < 16 || K % 16 != 0 || a->ldh < K ||
        a->ldh % 8 != 0 || rows * a->ldh * 2 >= (int64_t(1) << 31) ||
        (V + 31) / 32 * (K / 16) * 1024 >= (int64_t(1) << 31))
        return fail(NT_E_ARG, std::string(who) + ": rows " + std::to_string(rows) + " (at most 256), vocab " +
                                  std::to_string(V) + " (at most 262144), dim " + std::to_string(K) +
                                  " (a multiple of 16), ldh (>= dim, a multiple of 8)");
    if (a->mask_kind != NT_MASK_NONE && a->mask_kind != NT_MASK_U8)
        return fail(NT_E_UNSUPPORTED, std::string(who) + ": only no mask or a u8 keep-mask");
    if ((a->mask_kind == NT_MASK_U8) != (a->mask != nullptr))
        return fail(NT_E_ARG, std::string(who) + ": mask kind and mask pointer disagree");
    if (a->mask && a->mask_ld < V)
        return fail(NT_E_ARG, std::string(who) + ": mask_ld " + std::to_string(a->mask_ld) +
                                  " (one mask row of at least vocab bytes per logits row)");
    if (!a->hidden || !a->weight_packed || !a->ids || !a->status || reinterpret_cast<uintptr_t>(a->hidden) % 16 ||
        reinterpret_cast<uintptr_t>(a->weight_packed) % 16)
        return fail(NT_E_ARG, std::string(who) + ": null or unaligned hidden, packed weight, ids or status");
    if (!(a->temperature >= 0.0) || !std::isfinite(a->temperature))
        return fail(NT_E_ARG, "sample_categorical: temperature " + std::to_string(a->temperature) + " (must be ≥ 0)");
    const bool greedy = a->temperature == 0.0;
    if (!greedy && !a->uniforms) return fail(NT_E_ARG, std::string(who) + ": null uniforms");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (rows == 0) return 0;
    const int ntile = int((V + kRoCols - 1) / kRoCols), nblk = int((V + kRoBlock - 1) / kRoBlock);
    const size_t rec = size_t(rows) * size_t(ntile) * 4;
    const size_t hpack = size_t((rows + 31) / 32) * size_t(K / 16) * 1024;
    const size_t need = hpack + 3 * rec + size_t(rows) * size_t(nblk) * 4;
    void *ws = nullptr;
    if (int rc = scratch_alloc(need, &ws)) return rc;
    uint8_t *wb = static_cast<uint8_t *>(ws);
    // h into fragment order (2 MB at 256 rows of 4096)
    if (int rc = launch_pack(a->hidden, int(rows), int(K), a->ldh, false, wb)) return rc;
    const double T = greedy ? 1.0 : a->temperature;
    ReadoutP p;
    p.hp = wb;
    p.wp = static_cast<const uint8_t *>(a->weight_packed);
    p.rows = int(rows);
    p.V = int(V);
    p.K = int(K);
    p.ntile = ntile;
    p.nblk = nblk;
    p.mask = static_cast<const uint8_t *>(a->mask);
    p.mask_ld = a->mask_ld;
    p.mask_vec = a->mask && a->mask_ld % 16 == 0 && reinterpret_cast<uintptr_t>(a->mask) % 16 == 0;
    p.c = T == 1.0 ? kLog2e : float(double(kLog2e) / double(float(T)));
    p.tref = reinterpret_cast<float *>(wb + hpack);
    p.tmax = reinterpret_cast<float *>(wb + hpack + rec);
    p.tfirst = reinterpret_cast<int *>(wb + hpack + 2 * rec);
    p.bsum = reinterpret_cast<float *>(wb + hpack + 3 * rec);
    p.logits = a->logits;
    hipStream_t st = ctx().stream;
    const dim3 g1{unsigned(ntile), 1, 1}, b1{unsigned(kRoThreads), 1, 1};
    if (a->logits) {
        if (p.mask) hipLaunchKernelGGL((k_readout_tiles<true, true>), g1, b1, 0, st, p);
        else hipLaunchKernelGGL((k_readout_tiles<false, true>), g1, b1, 0, st, p);
    } else {
        if (p.mask) hipLaunchKernelGGL((k_readout_tiles<true, false>), g1, b1, 0, st, p);
        else hipLaunchKernelGGL((k_readout_tiles<false, false>), g1, b1, 0, st, p);
    }
    if (int rc = launched(who)) return rc;
    ResolveP q;
    q.h = static_cast<const uint16_t *>(a->hidden);
    q.wp = p.wp;
    q.rows = p.rows;
    q.V = p.V;
    q.K = p.K;
    q.ldh = int(a->ldh);
    q.ntile = ntile;
    q.nblk = nblk;
    q.mask = p.mask;
    q.mask_ld = p.mask_ld;
    q.c = p.c;
    q.tau = float(T);
    q.tau_one = T == 1.0;
    q.greedy = greedy;
    q.tref = p.tref;
    q.tmax = p.tmax;
    q.tfirst = p.tfirst;
    q.bsum = p.bsum;
    q.u = a->uniforms;
    q.ids = a->ids;
    q.logp = a->logp;
    q.status = a->status;
    q.dbg_block = a->debug_block;
    q.dbg_index = a->debug_block_index;
    hipLaunchKernelGGL(k_readout_resolve, dim3(unsigned(rows)), dim3(kResThreads), 0, st, q);
    if (int rc = launched(who)) return rc;
    return scratch_release(ws);
}
