// The readout-fused sampler: one decode step's readout product and its masked inverse-CDF
// sample + log-probability, without writing the logits.
//
// The reference computes the logits as the decoder's readout `x · W` (src/nn/decoder.rs:272,286;
// a Linear is one matmul, src/nn/linear.rs:1-3) into a [rows, V] tensor and then runs nn::rl on
// it (tempered_logits, the sampler, token_log_probs: rl.rs:134-141, 475-529). Here:
//
//  Pass 1 (k_readout_tiles): logits = h · W on the matrix cores, bf16 operands and f32
//  accumulation (v_mfma_f32_32x32x16_bf16, as the reference's half-precision product,
//  src/tensor/gpu/half_gemm.rs:1-10). One 256-thread workgroup (a wave per SIMD) owns 256
//  vocabulary columns for every row (up to 256 rows); each wave a 256 x 64 part as 8 x 2 MFMA
//  tiles in its AGPRs. Both operands are in fragment order (the weight packed once by
//  nt_hip_rl_readout_pack_weight, h per call), so one k-step's operands for 32 rows or columns
//  are 1 KiB contiguous: h, shared by the waves, is copied by the load unit straight into LDS
//  (buffer_load ... lds) through 14 stages of 8 KiB; each wave loads its own weight columns into
//  a register ring 12 k-steps deep. The epilogue turns the tile into the sampler's per-row
//  records instead of writing it: the tile's maximum and exponent reference, and the sum of the
//  weights 2^(x c - ref) of each 32-column block (f32). A debug pointer also writes the logits.
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
#include <type_traits>

#include "../../include/noetic_hip.h"
#include "nt_internal.hpp"
#include "nt_mfma_pipe.hpp"

namespace nt {
namespace {

using namespace pipe;

constexpr int kRoThreads = 256;       // 4 waves, one per SIMD: each holds 16 MFMA tiles in its AGPRs
constexpr int kRoCols = 256;          // vocabulary columns per workgroup (tile)
constexpr int kRoRows = 256;          // rows per launch at most
constexpr int64_t kRoMaxVocab = 262144;  // the resolve's per-thread block and tile arrays
constexpr int kRoBlock = 32;          // columns per record block
constexpr int kRoStages = kPipeStages;  // h's LDS stages (one k-step each)
constexpr int kRoStageBytes = kPipeStageBytes;
constexpr float kLog2e = 1.44269504088896340736f;
constexpr double kLn2 = 0.69314718055994530942;

// Fragment order: the MFMA operands of 32 rows (or vocabulary columns) g 32 .. g 32 + 31 for
// k-step s (k 16 s .. 16 s + 15) are one 1 KiB fragment, lane l's 16 bytes at 16 l holding row
// g 32 + l % 32 at k 16 s + 8 (l / 32) .. + 7, so a DMA of one fragment reads 1 KiB contiguous.
// h: row group g's fragment of step s at (g S + s) KiB. The weight, tile-major: column group g
// (tile t = g / 8, gi = g % 8) at ((t S + s) 8 + gi) KiB, a tile's eight fragments of one step
// 8 KiB contiguous, the vocabulary padded with zero columns to whole tiles of 256.
struct ReadoutP {
    const uint8_t *hp;   // h in fragment order, ceil(rows / 32) row groups
    const uint8_t *wp;   // the weight in fragment order, tile-major, ntile tiles
    int rows, V, K;
    int ntile, nblk;     // tiles of 256 columns, blocks of 32 columns
    const uint8_t *mask; // u8 keep-mask [rows, mask_ld] (mask_ld 0: one row shared) or null
    int64_t mask_ld;
    int mask_vec;        // mask rows 16-byte aligned: 16-byte loads
    float c;             // log2(e) / T
    float *tref;         // [rows][ntile] the tile's exponent reference RN(max c) (-inf: nothing allowed)
    float *tmax;         // [rows][ntile] the tile's maximum of the allowed logits
    int *tfirst;         // [rows][ntile] the first column holding it
    float *bsum;         // [rows][nblk] the block's sum of 2^(x c - tref)
    float *ebsum;        // [rows][nblk] the block's sum of 2^(x c - tref) (x c - tref) (ENT)
    const int32_t *tokens;  // [rows] the tokens being scored (TOKX)
    float *xtok;         // [rows] their logits, -inf where the mask excludes them (TOKX)
    float *logits;       // [rows][V] debug copy or null
};

// FIRST: the tile records carry each row's first column of the maximum (the greedy draw's
// answer); the sampler otherwise needs only the maximum. ENT: each block also records the sum
// of w y over its columns (w = 2^y, y = x c - tref), the entropy's term. TOKX: the lane holding
// a row's token column writes that logit (-inf if excluded) for the scorer.
template <bool MASK, bool DBG, bool FIRST, bool ENT, bool TOKX>
__global__ __launch_bounds__(kRoThreads) void k_readout_tiles(ReadoutP p) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[kRoStages * kRoStageBytes];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // this wave's columns 64 wave .. + 63
    const int tile = blockIdx.x;
    const int n0 = tile * kRoCols;
    const int S = p.K / 16;
    // Buffer resources over the packed operands. Loads past a range return zeros and touch no
    // memory: the loop below issues the copies of steps past the last (never used) instead of
    // branching around them. h's row groups past the rows are such zeros too.
    const int hgroups = (p.rows + 31) / 32;
    const __amdgpu_buffer_rsrc_t hres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(p.hp), short(0), hgroups * S * 1024, kBufferWord3);
    // Step t's operands. h (shared by the waves) through LDS: this wave copies row groups
    // 2 wave, 2 wave + 1 of it by DMA into stage t % kRoStages (lane l's 16 bytes at 16 l of the
    // fragment's slot). The weight (this wave's own two column groups) straight into registers.
    const int hoff = 2 * wave * S * 1024 + lane * 16, woff = 2 * wave * 1024 + lane * 16;
    // the weight's resource as four scalar words for the loads below (base, stride 0, size, flags)
    const uint64_t wbase = reinterpret_cast<uint64_t>(p.wp + int64_t(tile) * S * 8192);
    const v4u wrs = {uint32_t(wbase), uint32_t(wbase >> 32), uint32_t(S * 8192), uint32_t(kBufferWord3)};
    // the product over the k-steps (the weight as the A operand: see the epilogue)
    f32x16_t acc[8][2];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;
    MfmaPipe<true> pp;
    pp.run(lds, hres, hoff, wrs, woff, S, wave, lane, acc);
    // ---- epilogue, in the MFMA output's own layout. The product is the transposed block, so lane
    // l of wave w holds in acc[i][j][4 a + b] row r = 32 i + l % 32 at tile column
    // 64 w + 32 j + 8 a + 4 (l / 32) + b (j < 2, a < 4, b < 4): 32 of the row's 64 columns of this
    // wave, the partner lane l ^ 32 the other 32. Per row group i each lane takes its row's
    // maximum and first column over its 32 (in column order) and the partner's; the four waves'
    // go through LDS (one barrier), then each lane weighs its 32 against the tile's reference and
    // sums each 32-column block with the partner's half.
    // (the lane index again, from the exec mask's count below this lane: keeping the thread id
    // live through the loop would take a register the loop needs)
    const int el = int(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
    const int rw = el & 31, hh = el >> 5;
    const int cw0 = n0 + 64 * wave + 4 * hh;  // column of acc[i][0][0]; + 32 j + 8 a + b
    // The tile's mask (256 rows x 256 bytes) comes into LDS by coalesced 1 KiB copies, four rows
    // each, over the stages (every wave is past its last read of them after the barrier). Row r's
    // sixteen 16-byte chunks sit rotated by r (chunk k at position (k + r) % 16), so that the 32
    // lanes of a half, reading one column of 32 consecutive rows, spread over the banks. Rows past
    // the last and bytes past the mask read as zeros (the buffer's range); columns past the
    // vocabulary are excluded below. Rows that are not 16-byte aligned take byte loads instead.
    // The last odd step's MFMAs run while the copies are in flight.
    uint8_t *const lmask = lds;                                           // [256 rows][256 bytes]
    float *const Sm = reinterpret_cast<float *>(lds + kRoRows * kRoCols);  // [4 waves][256 rows] maxima
    int *const Sf = reinterpret_cast<int *>(Sm + 4 * kRoRows);            // [4 waves][256 rows] first columns
    static_assert(kRoRows * kRoCols + 8 * kRoRows * 4 <= kRoStages * kRoStageBytes, "the mask and the exchange fit");
    const bool mdma = MASK && p.mask_vec;
    asm volatile("s_barrier" ::: "memory");
    if (mdma) {
        const __amdgpu_buffer_rsrc_t mres = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(p.mask), short(0), int((int64_t(p.rows) - 1) * p.mask_ld + p.V), kBufferWord3);
#pragma unroll
        for (int qq = 0; qq < kRoRows / 16; qq++) {
            const int q = 4 * qq + wave;  // four rows per copy, copy q by wave q % 4
            const int r = 4 * q + (el >> 4), pos = el & 15, k = (pos - r) & 15;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(mres, (lds_ptr_t)(lmask + q * 1024), 16,
                                                     int(int64_t(r) * p.mask_ld) + n0 + 16 * k, 0, 0, 0);
        }
    }
    pp.last_odd_step(S, acc);  // (S odd) while the copies are in flight

    if (mdma) {
        wait_vmcnt<0>();
        asm volatile("s_barrier" ::: "memory");  // every wave's copies of the mask have landed
    }
    // the scored token of each of this lane's rows, relative to its first column (loaded once the
    // weight ring's registers are free; with the debug copy of the logits, one row at a time)
    int tkd[8];
    if constexpr (TOKX && !DBG) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int r = 32 * i + rw;
            tkd[i] = p.tokens[r < p.rows ? r : 0] - cw0;
        }
    }
    // per (i, j, a) the row's four bytes at column cw0 + 32 j + 8 a (all ones without a mask);
    // zero for a row past the last, so that the byte test below also excludes it
    uint32_t mk[8][2][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int a4 = 0; a4 < 4; a4++) mk[i][j][a4] = 32 * i + rw < p.rows ? 0xffffffffu : 0u;
    if constexpr (MASK) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int r = 32 * i + rw;
            if (r >= p.rows) continue;
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int c2 = 0; c2 < 2; c2++) {
                    if (mdma) {
                        const int k = 4 * wave + 2 * j + c2;
                        const uint32_t *w32 =
                            reinterpret_cast<const uint32_t *>(lmask + r * kRoCols + ((k + r) & 15) * 16 + 4 * hh);
                        mk[i][j][2 * c2] = w32[0];
                        mk[i][j][2 * c2 + 1] = w32[2];
                    } else {
                        const uint8_t *mrow = p.mask + int64_t(r < p.rows ? r : 0) * p.mask_ld;
#pragma unroll
                        for (int a2 = 0; a2 < 2; a2++) {
                            const int c0 = cw0 + 32 * j + 8 * (2 * c2 + a2);
                            uint32_t wd = 0;
                            for (int e = 0; e < 4 && c0 + e < p.V; e++) wd |= uint32_t(mrow[c0 + e]) << (8 * e);
                            mk[i][j][2 * c2 + a2] = wd;
                        }
                    }
                }
        }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = 32 * i + rw;
        const bool live = r < p.rows;
        if constexpr (DBG) {
            if (live)
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int col = cw0 + 32 * j + 8 * (v / 4) + (v % 4);
                        if (col < p.V) p.logits[int64_t(r) * p.V + col] = acc[i][j][v];
                    }
        }
        // the sampler's values: an excluded column or one past the vocabulary is -inf (the
        // column bound only in the tile that crosses the vocabulary's end)
        float m = -INFINITY;
        int first = 0x7fffffff;
        auto maxima = [&](auto full_c) {
            constexpr bool FULL = decltype(full_c)::value;
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int off = 32 * j + 8 * (v / 4) + (v % 4);  // column cw0 + off
                    bool keep = ((mk[i][j][v / 4] >> (8 * (v % 4))) & 0xffu) != 0;
                    if constexpr (!FULL) keep = keep && cw0 + off < p.V;
                    const float x = keep ? acc[i][j][v] : -INFINITY;
                    acc[i][j][v] = x;
                    if constexpr (FIRST) {
                        if (x > m) {
                            m = x;
                            first = off;
                        }
                    } else {
                        m = fmaxf(m, x);
                    }
                }
        };
        if (n0 + kRoCols <= p.V) maxima(std::true_type{});
        else maxima(std::false_type{});
        if constexpr (TOKX) {
            // the token's logit, if it is one of this lane's columns 32 j + 8 a + b (a, b < 4)
            // (excluded: -inf, as the maxima left it)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int d = (DBG ? p.tokens[live ? r : 0] - cw0 : tkd[i]) - 32 * j;
                if (live && d >= 0 && d < 32 && (d & 4) == 0) {
                    const int v = 4 * (d >> 3) + (d & 3);
                    float x = acc[i][j][0];
#pragma unroll
                    for (int vv = 1; vv < 16; vv++)
                        if (vv == v) x = acc[i][j][vv];
                    p.xtok[r] = x;
                }
            }
        }
        const float om = __shfl_xor(m, 32, 64);
        if constexpr (FIRST) {
            first = first == 0x7fffffff ? first : cw0 + first;
            const int of = __shfl_xor(first, 32, 64);
            if (om > m || (om == m && of < first)) {
                m = om;
                first = of;
            }
        } else {
            m = fmaxf(m, om);
        }
        if (hh == 0) {
            Sm[wave * kRoRows + r] = m;
            if constexpr (FIRST) Sf[wave * kRoRows + r] = first;
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // every wave's maxima in LDS
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = 32 * i + rw;
        const bool live = r < p.rows;
        // the tile's maximum and first column (the waves in column order; a tie keeps the earlier)
        float M = Sm[r];
        int F = 0x7fffffff;
        if constexpr (FIRST) F = Sf[r];
#pragma unroll
        for (int w2 = 1; w2 < 4; w2++) {
            const float m2 = Sm[w2 * kRoRows + r];
            if (m2 > M) {
                M = m2;
                if constexpr (FIRST) F = Sf[w2 * kRoRows + r];
            }
        }
        const float ref = M * p.c;  // RN(max c); -inf when nothing is allowed
        // (with nothing allowed every value is -inf: a finite reference weighs them all 0)
        const float wref = M == -INFINITY ? 0.0f : ref;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            float w[16], wy[16];
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const float y = fmaf(acc[i][j][v], p.c, -wref);
                w[v] = __builtin_amdgcn_exp2f(y);
                // (an excluded column: y = -inf, w = 0, a term of 0)
                if constexpr (ENT) wy[v] = w[v] * fmaxf(y, -FLT_MAX);
            }
            // this half's 16 in a fixed tree, then the two halves (column 4 (l / 32) of each 8)
#pragma unroll
            for (int span = 1; span < 16; span <<= 1)
#pragma unroll
                for (int e = 0; e < 16; e += 2 * span) {
                    w[e] = w[e] + w[e + span];
                    if constexpr (ENT) wy[e] = wy[e] + wy[e + span];
                }
            const float other = __shfl_xor(w[0], 32, 64);
            const int blk = tile * (kRoCols / kRoBlock) + 2 * wave + j;
            if (hh == 0 && live && blk < p.nblk) p.bsum[int64_t(r) * p.nblk + blk] = w[0] + other;
            if constexpr (ENT) {
                const float eo = __shfl_xor(wy[0], 32, 64);
                if (hh == 0 && live && blk < p.nblk) p.ebsum[int64_t(r) * p.nblk + blk] = wy[0] + eo;
            }
        }
        if (wave == 0 && hh == 0 && live) {
            p.tref[int64_t(r) * p.ntile + tile] = ref;
            p.tmax[int64_t(r) * p.ntile + tile] = M;
            if constexpr (FIRST) p.tfirst[int64_t(r) * p.ntile + tile] = F;
        }
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
    const float *ebsum;  // [rows][nblk] the entropy's block terms (scoring with entropy) or null
    const double *u;
    const int32_t *tokens;  // [rows] scoring: the token whose log-probability is asked for, or null
    const float *xtok;   // [rows] scoring: that token's logit from pass 1
    int32_t *ids;        // sampling: the draw
    float *logp;
    float *ent;          // scoring: the entropy, or null
    uint8_t *status;
    float *dbg_block;  // [rows][32] the recomputed logits of the crossing block, or null
    int *dbg_index;    // [rows] that block's index, or null
};

constexpr int kResThreads = 256;
constexpr int kResMaxBlocks = 32;  // blocks of 32 columns per thread: V <= 262144 (16: V <= 131072)
constexpr int kResMaxTiles = 4;    // tiles of 256 columns per thread
constexpr int kResMaxK = 16384;    // dim at most: the row of h is held in LDS (32 KiB)
constexpr int kResRing = 48;       // the block's weight fragments in flight in wave 0's registers
constexpr int kResAGroup = 4;      // k-steps of h read from LDS per statement
// (an even number of groups per pass of the ring: the two read buffers alternate across passes)
static_assert(kResRing % (2 * kResAGroup) == 0 && kResRing < 64, "the ring's passes and waits");

// One k-step's weight fragment (16 bytes of lane l at `off`) into `d`, issued only: `d` is in
// flight until the wait that takes it as an in-out operand.
__device__ __forceinline__ void load_frag(v4u &d, uint32_t off, const v4u &rs) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=&v"(d) : "v"(off), "s"(rs) : "memory");
}

// The A operands of kResAGroup consecutive k-steps (this row of h, 32 bytes a step apart in
// LDS), issued only; lds_wait_group waits for them.
__device__ __forceinline__ void lds_issue_group(uint32_t a, v4u (&fa)[kResAGroup]) {
    static_assert(kResAGroup == 4, "four reads");
    asm volatile(
        "ds_read_b128 %0, %4\n\t"
        "ds_read_b128 %1, %4 offset:32\n\t"
        "ds_read_b128 %2, %4 offset:64\n\t"
        "ds_read_b128 %3, %4 offset:96"
        : "=&v"(fa[0]), "=&v"(fa[1]), "=&v"(fa[2]), "=&v"(fa[3])
        : "v"(a)
        : "memory");
}

__device__ __forceinline__ void lds_wait_group(v4u (&fa)[kResAGroup]) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]) : : "memory");
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

// Pass 2, one workgroup per row:
//  - the row's records come in by coalesced loads (thread t takes elements t, t + 256, ...) and
//    through LDS to each thread's run of consecutive blocks; the row of h is copied into LDS and
//    the row's uniform loaded at the start, so that their latency hides under the records';
//  - the maximum over the tiles, the blocks' weights relative to it in f64 in index order (each
//    thread its run, a wave scan, the waves in order), the block holding u S (four barriers);
//  - wave 0 alone recomputes that block's 32 logits: the same MFMA over the same k order from
//    zero, so that they equal pass 1's bit for bit. The block's weight fragments (1 KiB a k-step,
//    256 KiB at C4's dim) stream into a ring of kResRing registers, loaded kResRing steps ahead of
//    their MFMA, and h's steps come from LDS four at a time, the next four in flight. Each MFMA
//    waits for the one before it (a dependent chain of K/16), so nothing else waits: no barrier
//    stands between the copies and the chain.
// Block b's sum sits at s_bs[b + b / 16] in LDS: a thread's run of 16 (or 32) consecutive blocks
// then starts 17 (34) words after the previous thread's, so a wave's reads of it spread over the
// banks.
__device__ __forceinline__ int bs_slot(int b) { return b + (b >> 4); }

// SCORE: the row's token logit comes from pass 1 (no block is recomputed), and the entropy from
// the records.
template <int MAXB, bool SCORE>
__global__ __launch_bounds__(kResThreads) void k_readout_resolve(ResolveP p) {
    __shared__ double wsum[kResThreads / 64];
    __shared__ double hsum[kResThreads / 64];
    __shared__ float wmax[kResThreads / 64];
    __shared__ int wsel[kResThreads / 64];
    __shared__ int wlast[kResThreads / 64];
    __shared__ int s_blk;
    __shared__ float s_ref;
    __shared__ double s_tl;
    __shared__ __attribute__((aligned(16))) float s_bs[MAXB * kResThreads * 17 / 16];  // the row's block sums
    __shared__ float s_tr[kResMaxTiles * kResThreads];                                 // its tile references
    // (scoring recomputes no block: no row of h)
    __shared__ __attribute__((aligned(16))) uint8_t hrow[SCORE ? 16 : kResMaxK * 2];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *tref = p.tref + int64_t(row) * p.ntile;
    const float *tmax = p.tmax + int64_t(row) * p.ntile;
    const int *tfirst = p.tfirst + int64_t(row) * p.ntile;
    const float *bsum = p.bsum + int64_t(row) * p.nblk;
    // The row of h into LDS (1 KiB pieces, piece c by wave c % 4): whichever block the records
    // pick, the recomputation needs it.
    if constexpr (!SCORE) {
        const __amdgpu_buffer_rsrc_t hres = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t *>(p.h + int64_t(row) * p.ldh), short(0), p.K * 2, kBufferWord3);
        for (int c = wave; c * 1024 < p.K * 2; c += 4)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(hres, (lds_ptr_t)(hrow + c * 1024), 16, c * 1024 + lane * 16, 0,
                                                     0, 0);
    }
    const double u_row = (SCORE || p.greedy) ? 0.0 : p.u[row];
    const int tok = SCORE && p.tokens ? p.tokens[row] : -1;
    // The records, coalesced. (Every load reads a valid index and the unused ones are masked
    // after: a load under a condition becomes a branch of its own, with its wait before the next.)
    float tm[kResMaxTiles], tr[kResMaxTiles], bv[MAXB], ev[MAXB];
#pragma unroll
    for (int i = 0; i < kResMaxTiles; i++) {
        const int t = tid + i * kResThreads, tc = min(t, p.ntile - 1);
        const float vm = tmax[tc], vr = tref[tc];
        tm[i] = t < p.ntile ? vm : -INFINITY;
        tr[i] = vr;
    }
    const int nb_rounds = (p.nblk + kResThreads - 1) / kResThreads;  // at most MAXB
#pragma unroll
    for (int i = 0; i < MAXB; i++) {
        if (i < nb_rounds) bv[i] = bsum[min(tid + i * kResThreads, p.nblk - 1)];
    }
    if (SCORE && p.ebsum) {
        // every slot loaded (a clamped index), so that the loads issue together
        const float *eb = p.ebsum + int64_t(row) * p.nblk;
#pragma unroll
        for (int i = 0; i < MAXB; i++) ev[i] = eb[min(tid + i * kResThreads, p.nblk - 1)];
    }
#pragma unroll
    for (int i = 0; i < kResMaxTiles; i++) s_tr[tid + i * kResThreads] = tr[i];
#pragma unroll
    for (int i = 0; i < MAXB; i++)
        if (i < nb_rounds) s_bs[bs_slot(tid + i * kResThreads)] = bv[i];
    // (a wave that leaves early first lets its copies into LDS land: the LDS is the workgroup's
    // until its last wave ends; the loads above were issued after them and have landed, so they
    // have too)
    auto refuse = [&](uint8_t st) {
        wait_vmcnt<0>();
        if (tid == 0) {
            if (p.ids) p.ids[row] = -1;
            if (p.logp) p.logp[row] = NAN;
            if (p.ent) p.ent[row] = NAN;
            p.status[row] = st;
        }
    };
    // ---- the row's maximum over the tiles (exact; the order does not matter for a maximum)
    static_assert(kResMaxTiles == 4, "the maximum over the thread's tiles");
    float m = fmaxf(fmaxf(tm[0], tm[1]), fmaxf(tm[2], tm[3]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (lane == 0) wmax[wave] = m;
    __syncthreads();  // (1) the maximum's parts, the block sums and references in LDS
    const float M = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    // (nothing allowed, or every allowed logit below -FLT_MAX T, whose tempered value is -inf)
    if (M == -INFINITY || (!p.tau_one && M / p.tau == -INFINITY)) {
        refuse(NT_ROW_NO_TOKEN);
        return;
    }
    const float A = M * p.c;
    // ---- block weights relative to A, f64 in index order: this thread's run b0 .. b1 - 1
    const int per = nb_rounds;
    const int b0 = tid * per, b1 = min(p.nblk, b0 + per);
    // (a run of at most 32 blocks spans at most five tiles of 8: their factors 2^(ref - A) once each)
    double wbk[MAXB];
    double run = 0.0;
    const int t0 = b0 / (kRoCols / kRoBlock);
    double tf[MAXB / 8 + 1];
#pragma unroll
    for (int j = 0; j <= MAXB / 8; j++) {
        const float r = s_tr[min(t0 + j, kResMaxTiles * kResThreads - 1)];
        tf[j] = r == -INFINITY ? 0.0 : double(__builtin_amdgcn_exp2f(r - A));
    }
#pragma unroll
    for (int i = 0; i < MAXB; i++) {
        const int b = b0 + i;
        double wb = 0.0;
        if (i < per && b < b1) {
            double f = tf[0];
#pragma unroll
            for (int j = 1; j <= MAXB / 8; j++)
                if (b / (kRoCols / kRoBlock) - t0 == j) f = tf[j];
            wb = f * double(s_bs[bs_slot(b)]);
        }
        wbk[i] = wb;
        run += wb;
    }
    const double incl_w = wave_incl_scan(run, lane);
    if (lane == 63) wsum[wave] = incl_w;
    if constexpr (SCORE) {
        // the entropy's sum relative to A, sum_v 2^(x c - A) (x c - A): per block
        // 2^(ref - A) (E + (ref - A) B) from its records, over this thread's blocks in order
        double hp = 0.0;
        if (p.ebsum) {
#pragma unroll
            for (int i = 0; i < MAXB; i++) {
                const int b = tid + i * kResThreads;
                if (i < nb_rounds && b < p.nblk) {
                    const float r = s_tr[b / (kRoCols / kRoBlock)];
                    if (r != -INFINITY) {
                        const double d = double(r) - double(A);
                        hp += double(__builtin_amdgcn_exp2f(r - A)) * (double(ev[i]) + d * double(bv[i]));
                    }
                }
            }
        }
        const double incl_h = wave_incl_scan(hp, lane);
        if (lane == 63) hsum[wave] = incl_h;
    }
    __syncthreads();  // (2) the waves' totals
    double before = 0.0;
    for (int w2 = 0; w2 < wave; w2++) before += wsum[w2];
    const double incl = before + incl_w, excl = incl - run;
    // the row's sum: the last thread's inclusive prefix (the same additions in the same order)
    const double Sall = (((0.0 + wsum[0]) + wsum[1]) + wsum[2]) + wsum[3];
    if (!(Sall == Sall)) {
        refuse(NT_ROW_NAN);
        return;
    }
    const double shiftA = double(A) - double(M) * double(p.c);
    if constexpr (SCORE) {
        // H = ln S - ln2 (sum 2^(x c - A) (x c - A)) / S, both sums relative to A
        const double Hall = (((0.0 + hsum[0]) + hsum[1]) + hsum[2]) + hsum[3];
        const bool tok_ok = tok >= 0 && tok < p.V;
        if (!p.logp || !tok_ok) {
            wait_vmcnt<0>();
            if (tid == 0) {
                if (p.ent) p.ent[row] = float(log(Sall) - kLn2 * Hall / Sall);
                if (p.logp) p.logp[row] = NAN;
                p.status[row] = (p.tokens && !tok_ok) ? NT_ROW_BAD_TOKEN : NT_ROW_OK;
            }
            return;
        }
        // the token's logit comes from pass 1 (the same value a recomputation gives)
        wait_vmcnt<0>();
        if (tid == 0) {
            if (p.ent) p.ent[row] = float(log(Sall) - kLn2 * Hall / Sall);
            const float x = p.xtok[row];
            const double lnS = log(Sall) + shiftA * kLn2;
            const float zt = p.tau_one ? x : x / p.tau;
            const float mz = p.tau_one ? M : M / p.tau;
            p.logp[row] = float((double(zt) - double(mz)) - lnS);
            p.status[row] = NT_ROW_OK;
        }
        return;
    } else if (p.greedy) {
        wait_vmcnt<0>();
        const double lnS = log(Sall) + shiftA * kLn2;
        // the first column holding the maximum: the first tile whose maximum it is
        int best = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < kResMaxTiles; i++) {
            const int t = tid + i * kResThreads;
            if (t < p.ntile && tm[i] == M) best = min(best, tfirst[t]);
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
    const double t = u_row * Sall;
    if constexpr (!SCORE) {
        const uint64_t cross = __ballot(incl > t && run > 0.0);
        const uint64_t any = __ballot(run > 0.0);
        if (lane == 0) wsel[wave] = cross ? wave * 64 + __builtin_ctzll(cross) : -1;
        if (lane == 0) wlast[wave] = any ? wave * 64 + 63 - __builtin_clzll(any) : -1;
        __syncthreads();  // (3) the waves' crossings
        int sel = -1;
        for (int w2 = 0; w2 < 4 && sel < 0; w2++) sel = wsel[w2];
        if (sel < 0)
            for (int w2 = 3; w2 >= 0 && sel < 0; w2--) sel = wlast[w2];
        if (tid == 0) s_blk = -1;
        if (tid == sel) {
            double acc = excl;
            int bstar = -1, blast = -1;
            double bexcl = 0.0, lexcl = 0.0;
#pragma unroll
            for (int i = 0; i < MAXB; i++) {
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
            const float r = s_tr[bstar / (kRoCols / kRoBlock)];
            s_blk = bstar;
            s_ref = r;
            // the target inside the block, in the scale of its tile's reference
            s_tl = (t - bexcl) * double(__builtin_amdgcn_exp2f(A - r));
        }
        __syncthreads();  // (4) the block
    } else {
        return;  // (the scoring path has ended above)
    }
    const int bstar = s_blk;
    if (bstar < 0) {
        refuse(NT_ROW_NAN);
        return;
    }
    if (wave != 0) return;  // (their copies of h landed before barrier 1)
    const double tl = s_tl;
    const float r = s_ref;
    // ---- wave 0: recompute the block's 32 logits. Every lane's A row is this row (so every
    // output row holds it); lane l's B column is 32 b + l % 32.
    const int fr = lane & 31;
    const int col = bstar * kRoBlock + fr;
    const bool colok = col < p.V;
    const int S2 = p.K / 16;
    const int bt = bstar / 8, bg = bstar % 8;  // the block's tile and column group within it
    // the mask byte of this lane's column, loaded before the ring (so that it has landed whenever
    // the ring's oldest load has)
    bool keep = lane < 32 && colok;
    if (keep && p.mask) keep = p.mask[int64_t(row) * p.mask_ld + col] != 0;
    // the block's fragments: step s at (s 8 + 0) KiB from the block's first (tile-major order)
    const uint64_t wbase = reinterpret_cast<uint64_t>(p.wp + (int64_t(bt) * S2 * 8 + bg) * 1024);
    const v4u wrs = {uint32_t(wbase), uint32_t(wbase >> 32), uint32_t((S2 - 1) * 8192 + 1024), uint32_t(kBufferWord3)};
    const uint32_t woff = uint32_t(lane) * 16;
    v4u ring[kResRing];
#pragma unroll
    for (int j = 0; j < kResRing; j++) load_frag(ring[j], woff + uint32_t(j) * 8192, wrs);  // past the block: zeros
    // ln S (for the log-probability at the end), while the first loads are in flight
    const double lnS = log(Sall) + shiftA * kLn2;
    f32x16_t acc;
#pragma unroll
    for (int v = 0; v < 16; v++) acc[v] = 0.0f;
    const uint32_t hbase = uint32_t((uintptr_t)(lds_ptr_t)(hrow)) + (lane >> 5) * 16;
    const uint32_t hlim = uint32_t((uintptr_t)(lds_ptr_t)(hrow)) + kResMaxK * 2;  // reads stay in hrow
    v4u fa0[kResAGroup], fa1[kResAGroup];
#pragma unroll
    for (int j = 0; j < kResAGroup; j++) fa0[j] = fa1[j] = v4u{0, 0, 0, 0};
    auto issue_a = [&](int s0, v4u(&fa)[kResAGroup]) {
        const uint32_t a = hbase + uint32_t(s0) * 32;
        if (s0 < S2 && a + kResAGroup * 32 <= hlim) lds_issue_group(a, fa);
    };
    // one pass of the ring from step `base`; PARTIAL: the last, with steps past S2 (their MFMAs
    // skipped, their waits and loads kept so that every slot's load is waited for)
    auto pass = [&](int base, auto partial_c) {
        constexpr bool PARTIAL = decltype(partial_c)::value;
#pragma unroll
        for (int g = 0; g < kResRing / kResAGroup; g++) {
            v4u(&cur)[kResAGroup] = (g & 1) ? fa1 : fa0;
            v4u(&nxt)[kResAGroup] = (g & 1) ? fa0 : fa1;
            lds_wait_group(cur);
            issue_a(base + (g + 1) * kResAGroup, nxt);
#pragma unroll
            for (int j = 0; j < kResAGroup; j++) {
                const int k = g * kResAGroup + j, st = base + k;
                // the ring's oldest load (step st) has landed when kResRing - 1 remain
                asm volatile("s_waitcnt vmcnt(47)" : "+v"(ring[k]) : : "memory");
                static_assert(kResRing - 1 == 47, "the wait above");
                if (!PARTIAL || st < S2)  // (the weight as A, h as B: pass 1's order)
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, ring[k]),
                                                                  __builtin_bit_cast(bf16x8_t, cur[j]), acc, 0, 0, 0);
                load_frag(ring[k], woff + uint32_t(st + kResRing) * 8192, wrs);
            }
        }
    };
    issue_a(0, fa0);
    int base = 0;
    for (; base + kResRing <= S2; base += kResRing) pass(base, std::false_type{});
    if (base < S2) pass(base, std::true_type{});
    // every load lands before its register is given to anything else (the ring's last loads are
    // never read): the wait, then each register taken as an in-out operand after it
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(ring[0]) : : "memory");
#pragma unroll
    for (int j = 1; j < kResRing; j++) asm volatile("" : "+v"(ring[j]) : : "memory");
    lds_wait_group(fa0);
    lds_wait_group(fa1);
    // Block column c (lane c < 32) is acc[4 (c / 8) + c % 4] of a lane in half (c / 4) % 2, as in
    // pass 1's layout (this row is each of B's 32 columns): this lane's half at that index, or its
    // partner's (lane c ^ 32, the same index).
    float x;
    {
        const int c = lane & 31, v = 4 * (c / 8) + (c % 4);
        float own = acc[0];
#pragma unroll
        for (int vv = 1; vv < 16; vv++)
            if (vv == v) own = acc[vv];
        const float other = __shfl_xor(own, 32, 64);
        x = (lane >> 5) == ((c / 4) & 1) ? own : other;
    }
    if (p.dbg_block && lane < 32) p.dbg_block[int64_t(row) * 32 + lane] = x;
    if (p.dbg_index && lane == 0) p.dbg_index[row] = bstar;
    x = keep ? x : -INFINITY;
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

// Two f32 values rounded to bf16 (to nearest, ties to even; a NaN stays a quiet NaN), `lo` in
// the low half: the reduced-precision product's rounding of f32 operands as they are loaded
// (src/tensor/precision.rs:4-8, half.rs:16-23).
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
    uint32_t r;
    asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
    return r;
}

// One f32 or f16 element of an operand as f32 (an f16 widens exactly).
template <int SRC>
__device__ __forceinline__ float operand_f32(const void *src, int64_t i) {
    if constexpr (SRC == NT_F32) return static_cast<const float *>(src)[i];
    else return float(__builtin_bit_cast(_Float16, static_cast<const uint16_t *>(src)[i]));
}

// Fragment order (see ReadoutP) of a [R, K] matrix, bf16, or f32 or f16 (SRC) rounded to bf16 as
// it is packed (an f16 widened to f32 exactly first, so one rounding): k contiguous (row r at src + r ld) or, K_MAJOR, the transpose of a [K, R] one (row r is
// column r of src, k at src + k ld + r); TILED, the weight's tile-major order over `groups`
// column groups (a multiple of 8), else h's group-major order. Rows from R up to the groups' end
// are zeros. One thread writes one lane's 16 bytes.
template <bool K_MAJOR, bool TILED, int SRC>
__global__ void k_pack_frags(const void *srcv, int R, int K, int64_t ld, v4u *out, int64_t total) {
    const uint16_t *src = static_cast<const uint16_t *>(srcv);
    const int S = K / 16;
    for (int64_t idx = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; idx < total;
         idx += int64_t(gridDim.x) * blockDim.x) {
        const int l = int(idx % 64);
        const int64_t q = idx / 64;
        int s;
        int64_t g;
        if constexpr (TILED) {
            const int64_t ts = q / 8;  // tile t, step s: t S + s
            s = int(ts % S);
            g = ts / S * 8 + q % 8;
        } else {
            s = int(q % S);
            g = q / S;
        }
        const int64_t r = g * 32 + (l & 31);
        const int k0 = 16 * s + 8 * (l >> 5);
        v4u v = {0, 0, 0, 0};
        if (r < R) {
            if constexpr (SRC != NT_BF16) {
                uint32_t w4[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int64_t a0 = K_MAJOR ? int64_t(k0 + 2 * j) * ld + r : r * ld + k0 + 2 * j;
                    const int64_t a1 = K_MAJOR ? int64_t(k0 + 2 * j + 1) * ld + r : r * ld + k0 + 2 * j + 1;
                    w4[j] = bf16_pair(operand_f32<SRC>(srcv, a0), operand_f32<SRC>(srcv, a1));
                }
                v = v4u{w4[0], w4[1], w4[2], w4[3]};
            } else if constexpr (!K_MAJOR) {
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

// f32 or f16 (SRC) rows [R, K] (row stride ld) rounded to bf16, row-major with stride K: such a
// readout input as the bf16 operand both the product and the resolve read.
template <int SRC>
__global__ void k_round_rows_bf16(const void *src, int R, int K, int64_t ld, uint32_t *dst) {
    const int64_t pairs = int64_t(R) * (K / 2);
    for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < pairs; i += int64_t(gridDim.x) * blockDim.x) {
        const int64_t r = i / (K / 2), k = 2 * (i % (K / 2));
        dst[i] = bf16_pair(operand_f32<SRC>(src, r * ld + k), operand_f32<SRC>(src, r * ld + k + 1));
    }
}

// h (group-major, ceil(R / 32) groups) or the weight (tile-major, whole tiles of 256 columns),
// from bf16, or f32 or f16 (SRC) rounded to bf16.
template <bool K_MAJOR, bool TILED, int SRC = NT_BF16>
int launch_pack_t(const void *src, int R, int K, int64_t ld, void *out) {
    const int64_t groups = TILED ? int64_t((R + kRoCols - 1) / kRoCols) * 8 : (R + 31) / 32;
    const int64_t total = groups * (K / 16) * 64;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    const dim3 g{unsigned(blocks), 1, 1}, b{256, 1, 1};
    hipLaunchKernelGGL((k_pack_frags<K_MAJOR, TILED, SRC>), g, b, 0, ctx().stream, src, R, K, ld,
                       static_cast<v4u *>(out), total);
    return launched("readout pack");
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" int64_t nt_hip_rl_readout_packed_bytes(int64_t vocab, int64_t dim) {
    if (vocab < 1 || dim < 16 || dim % 16 != 0) return -1;
    return (vocab + kRoCols - 1) / kRoCols * kRoCols * dim * 2;
}

extern "C" int nt_hip_rl_readout_pack_weight(const void *weight, int32_t dtype, int32_t layout, int64_t vocab,
                                             int64_t dim, int64_t ld, void *packed) {
    const char *who = "nt_hip_rl_readout_pack_weight";
    const bool dv = layout == NT_READOUT_W_DV, bf16 = dtype == NT_BF16;
    if ((dtype != NT_F32 && dtype != NT_BF16 && dtype != NT_F16) || (layout != NT_READOUT_W_VD && !dv) || vocab < 1 ||
        vocab > kRoMaxVocab || dim < 16 || dim % 16 != 0 || !weight || !packed || ld < (dv ? vocab : dim) ||
        (!dv && bf16 && (ld % 8 != 0 || reinterpret_cast<uintptr_t>(weight) % 16)) ||
        reinterpret_cast<uintptr_t>(weight) % (dtype == NT_F32 ? 4 : 2) ||
        reinterpret_cast<uintptr_t>(packed) % 16 || (vocab + kRoCols - 1) / kRoCols * (dim / 16) * 8192 >= (int64_t(1) << 31))
        return fail(NT_E_ARG, std::string(who) + ": dtype " + std::to_string(dtype) + ", layout " + std::to_string(layout) +
                                  ", vocab " + std::to_string(vocab) + " (at most 262144), dim " + std::to_string(dim) +
                                  " (a multiple of 16), ld " + std::to_string(ld) +
                                  " (at least the row; bf16 [V, d] rows a multiple of 8 and 16-byte aligned)");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (dtype == NT_F32)
        return dv ? launch_pack_t<true, true, NT_F32>(weight, int(vocab), int(dim), ld, packed)
                  : launch_pack_t<false, true, NT_F32>(weight, int(vocab), int(dim), ld, packed);
    if (dtype == NT_F16)
        return dv ? launch_pack_t<true, true, NT_F16>(weight, int(vocab), int(dim), ld, packed)
                  : launch_pack_t<false, true, NT_F16>(weight, int(vocab), int(dim), ld, packed);
    return dv ? launch_pack_t<true, true>(weight, int(vocab), int(dim), ld, packed)
              : launch_pack_t<false, true>(weight, int(vocab), int(dim), ld, packed);
}

namespace nt {
namespace {

// One readout call of either entry point: the checks they share, h into fragment order, pass 1
// and the resolve, on the library stream.
struct ReadoutCall {
    const char *who;
    const void *hidden, *weight_packed, *mask;
    int64_t rows, V, K, ldh, mask_ld;
    int32_t mask_kind;
    int32_t hidden_dtype;      // NT_BF16, or NT_F32 / NT_F16 (rounded to bf16 once, first)
    double T;                  // > 0 (1 when greedy)
    bool greedy, score;
    const double *u;           // sampling
    const int32_t *tokens;     // scoring
    int32_t *ids;              // sampling
    float *logp, *ent;         // ent: scoring
    uint8_t *status;
    float *logits, *dbg_block;
    int32_t *dbg_index;
};

int readout_run(const ReadoutCall &c) {
    const char *who = c.who;
    const int64_t rows = c.rows, V = c.V, K = c.K;
    if (c.hidden_dtype != NT_BF16 && c.hidden_dtype != NT_F32 && c.hidden_dtype != NT_F16)
        return fail(NT_E_ARG, std::string(who) + ": hidden_dtype " + std::to_string(c.hidden_dtype) +
                                  " (NT_BF16, NT_F32 or NT_F16)");
    const bool hf32 = c.hidden_dtype != NT_BF16;  // (f32 or f16: rounded first)
    // A bf16 h is read in place (16-byte loads, 32-bit offsets); an f32 or f16 one is first
    // rounded into a packed bf16 copy, so only its row stride has to cover the row.
    if (rows < 0 || rows > kRoRows || V < 1 || V > kRoMaxVocab || K < 16 || K % 16 != 0 || K > kResMaxK || c.ldh < K ||
        (!hf32 && (c.ldh % 8 != 0 || rows * c.ldh * 2 >= (int64_t(1) << 31))) ||
        (V + kRoCols - 1) / kRoCols * (K / 16) * 8192 >= (int64_t(1) << 31))
        return fail(NT_E_ARG, std::string(who) + ": rows " + std::to_string(rows) + " (at most 256), vocab " +
                                  std::to_string(V) + " (at most 262144), dim " + std::to_string(K) +
                                  " (a multiple of 16, at most 16384), ldh (>= dim; bf16: a multiple of 8)");
    if (c.mask_kind != NT_MASK_NONE && c.mask_kind != NT_MASK_U8)
        return fail(NT_E_UNSUPPORTED, std::string(who) + ": only no mask or a u8 keep-mask");
    if ((c.mask_kind == NT_MASK_U8) != (c.mask != nullptr))
        return fail(NT_E_ARG, std::string(who) + ": mask kind and mask pointer disagree");
    if (c.mask && c.mask_ld != 0 && c.mask_ld < V)
        return fail(NT_E_ARG, std::string(who) + ": mask_ld " + std::to_string(c.mask_ld) +
                                  " (one mask row of at least vocab bytes per logits row)");
    if (!c.hidden || !c.weight_packed || !c.status ||
        reinterpret_cast<uintptr_t>(c.hidden) % (c.hidden_dtype == NT_F32 ? 4 : (hf32 ? 2 : 16)) ||
        reinterpret_cast<uintptr_t>(c.weight_packed) % 16)
        return fail(NT_E_ARG, std::string(who) + ": null or unaligned hidden or packed weight, or null status");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (rows == 0) return 0;
    const bool ent = c.score && c.ent;
    const int ntile = int((V + kRoCols - 1) / kRoCols), nblk = int((V + kRoBlock - 1) / kRoBlock);
    const size_t rec = size_t(rows) * size_t(ntile) * 4, brec = size_t(rows) * size_t(nblk) * 4;
    const size_t hpack = size_t((rows + 31) / 32) * size_t(K / 16) * 1024;
    const bool tokx = c.score && c.tokens && c.logp;  // the scored tokens' logits from pass 1
    const size_t hround = hf32 ? size_t(rows) * size_t(K) * 2 : 0;  // an f32 / f16 h in bf16, 256-byte aligned
    const size_t hoff = (hpack + 3 * rec + (ent ? 2 : 1) * brec + (tokx ? size_t(rows) * 4 : 0) + 255) & ~size_t(255);
    const size_t need = hoff + hround;
    void *ws = nullptr;
    if (int rc = scratch_alloc(need, &ws)) return rc;
    uint8_t *wb = static_cast<uint8_t *>(ws);
    // An f32 or f16 h is rounded to bf16 once (row-major, stride K), the operand the product
    // and the resolve both read.
    const void *hidden = c.hidden;
    int64_t ldh = c.ldh;
    if (hround) {
        uint16_t *hb = reinterpret_cast<uint16_t *>(wb + hoff);
        const int64_t blocks = std::min<int64_t>((rows * K / 2 + 255) / 256, 4096);
        if (c.hidden_dtype == NT_F32)
            hipLaunchKernelGGL(k_round_rows_bf16<NT_F32>, dim3(unsigned(blocks)), dim3(256), 0, ctx().stream,
                               c.hidden, int(rows), int(K), c.ldh, reinterpret_cast<uint32_t *>(hb));
        else
            hipLaunchKernelGGL(k_round_rows_bf16<NT_F16>, dim3(unsigned(blocks)), dim3(256), 0, ctx().stream,
                               c.hidden, int(rows), int(K), c.ldh, reinterpret_cast<uint32_t *>(hb));
        if (int rc = launched(who)) {
            scratch_release(ws);
            return rc;
        }
        hidden = hb;
        ldh = K;
    }
    // h into fragment order (2 MB at 256 rows of 4096)
    if (int rc = launch_pack_t<false, false>(hidden, int(rows), int(K), ldh, wb)) {
        scratch_release(ws);
        return rc;
    }
    ReadoutP p;
    p.hp = wb;
    p.wp = static_cast<const uint8_t *>(c.weight_packed);
    p.rows = int(rows);
    p.V = int(V);
    p.K = int(K);
    p.ntile = ntile;
    p.nblk = nblk;
    p.mask = static_cast<const uint8_t *>(c.mask);
    p.mask_ld = c.mask_ld;
    p.mask_vec = c.mask && c.mask_ld % 16 == 0 && reinterpret_cast<uintptr_t>(c.mask) % 16 == 0;
    p.c = c.T == 1.0 ? kLog2e : float(double(kLog2e) / double(float(c.T)));
    p.tref = reinterpret_cast<float *>(wb + hpack);
    p.tmax = reinterpret_cast<float *>(wb + hpack + rec);
    p.tfirst = reinterpret_cast<int *>(wb + hpack + 2 * rec);
    p.bsum = reinterpret_cast<float *>(wb + hpack + 3 * rec);
    p.ebsum = ent ? reinterpret_cast<float *>(wb + hpack + 3 * rec + brec) : nullptr;
    p.tokens = c.tokens;
    p.xtok = tokx ? reinterpret_cast<float *>(wb + hpack + 3 * rec + (ent ? 2 : 1) * brec) : nullptr;
    p.logits = c.logits;
    hipStream_t st = ctx().stream;
    const dim3 g1{unsigned(ntile), 1, 1}, b1{unsigned(kRoThreads), 1, 1};
    auto launch1 = [&](auto mask_c, auto dbg_c) {
        constexpr bool MK = decltype(mask_c)::value, DB = decltype(dbg_c)::value;
        if (c.greedy) hipLaunchKernelGGL((k_readout_tiles<MK, DB, true, false, false>), g1, b1, 0, st, p);
        else if (ent && tokx) hipLaunchKernelGGL((k_readout_tiles<MK, DB, false, true, true>), g1, b1, 0, st, p);
        else if (ent) hipLaunchKernelGGL((k_readout_tiles<MK, DB, false, true, false>), g1, b1, 0, st, p);
        else if (tokx) hipLaunchKernelGGL((k_readout_tiles<MK, DB, false, false, true>), g1, b1, 0, st, p);
        else hipLaunchKernelGGL((k_readout_tiles<MK, DB, false, false, false>), g1, b1, 0, st, p);
    };
    if (c.logits) {
        if (p.mask) launch1(std::true_type{}, std::true_type{});
        else launch1(std::false_type{}, std::true_type{});
    } else {
        if (p.mask) launch1(std::true_type{}, std::false_type{});
        else launch1(std::false_type{}, std::false_type{});
    }
    if (int rc = launched(who)) {
        scratch_release(ws);
        return rc;
    }
    ResolveP q;
    q.h = static_cast<const uint16_t *>(hidden);
    q.wp = p.wp;
    q.rows = p.rows;
    q.V = p.V;
    q.K = p.K;
    q.ldh = int(ldh);
    q.ntile = ntile;
    q.nblk = nblk;
    q.mask = p.mask;
    q.mask_ld = p.mask_ld;
    q.c = p.c;
    q.tau = float(c.T);
    q.tau_one = c.T == 1.0;
    q.greedy = c.greedy;
    q.tref = p.tref;
    q.tmax = p.tmax;
    q.tfirst = p.tfirst;
    q.bsum = p.bsum;
    q.ebsum = p.ebsum;
    q.u = c.u;
    q.tokens = c.tokens;
    q.xtok = p.xtok;
    q.ids = c.ids;
    q.logp = c.logp;
    q.ent = c.ent;
    q.status = c.status;
    q.dbg_block = c.dbg_block;
    q.dbg_index = c.dbg_index;
    const dim3 g2{unsigned(rows), 1, 1}, b2{unsigned(kResThreads), 1, 1};
    const bool small = nblk <= 16 * kResThreads;
    if (c.score) {
        if (small) hipLaunchKernelGGL((k_readout_resolve<16, true>), g2, b2, 0, st, q);
        else hipLaunchKernelGGL((k_readout_resolve<kResMaxBlocks, true>), g2, b2, 0, st, q);
    } else {
        if (small) hipLaunchKernelGGL((k_readout_resolve<16, false>), g2, b2, 0, st, q);
        else hipLaunchKernelGGL((k_readout_resolve<kResMaxBlocks, false>), g2, b2, 0, st, q);
    }
    const int rc = launched(who);
    const int rf = scratch_release(ws);
    return rc ? rc : rf;
}

}  // namespace
}  // namespace nt

extern "C" int nt_hip_rl_readout_sample(const NtRlReadoutSampleArgs *a) {
    const char *who = "nt_hip_rl_readout_sample";
    if (!a) return fail(NT_E_ARG, std::string(who) + ": null args");
    if (!(a->temperature >= 0.0) || !std::isfinite(a->temperature))
        return fail(NT_E_ARG, "sample_categorical: temperature " + std::to_string(a->temperature) + " (must be ≥ 0)");
    const bool greedy = a->temperature == 0.0;
    if (!greedy && !a->uniforms) return fail(NT_E_ARG, std::string(who) + ": null uniforms");
    if (!a->ids) return fail(NT_E_ARG, std::string(who) + ": null ids");
    ReadoutCall c{};
    c.who = who;
    c.hidden = a->hidden;
    c.hidden_dtype = a->hidden_dtype;
    c.weight_packed = a->weight_packed;
    c.mask = a->mask;
    c.rows = a->rows;
    c.V = a->vocab;
    c.K = a->dim;
    c.ldh = a->ldh;
    c.mask_ld = a->mask_ld;
    c.mask_kind = a->mask_kind;
    c.T = greedy ? 1.0 : a->temperature;
    c.greedy = greedy;
    c.score = false;
    c.u = a->uniforms;
    c.ids = a->ids;
    c.logp = a->logp;
    c.status = a->status;
    c.logits = a->logits;
    c.dbg_block = a->debug_block;
    c.dbg_index = a->debug_block_index;
    return readout_run(c);
}

extern "C" int nt_hip_rl_readout_score(const NtRlReadoutScoreArgs *a) {
    const char *who = "nt_hip_rl_readout_score";
    if (!a) return fail(NT_E_ARG, std::string(who) + ": null args");
    if (!(a->temperature > 0.0) || !std::isfinite(a->temperature))
        return fail(NT_E_ARG, "tempered_logits: temperature " + std::to_string(a->temperature) + " (must be positive)");
    if (a->logp && !a->tokens) return fail(NT_E_ARG, std::string(who) + ": log-probabilities need tokens");
    if (!a->logp && !a->entropy) return fail(NT_E_ARG, std::string(who) + ": neither logp nor entropy asked for");
    ReadoutCall c{};
    c.who = who;
    c.hidden = a->hidden;
    c.hidden_dtype = a->hidden_dtype;
    c.weight_packed = a->weight_packed;
    c.mask = a->mask;
    c.rows = a->rows;
    c.V = a->vocab;
    c.K = a->dim;
    c.ldh = a->ldh;
    c.mask_ld = a->mask_ld;
    c.mask_kind = a->mask_kind;
    c.T = a->temperature;
    c.greedy = false;
    c.score = true;
    c.tokens = a->tokens;
    c.logp = a->logp;
    c.ent = a->entropy;
    c.status = a->status;
    c.logits = a->logits;
    return readout_run(c);
}
