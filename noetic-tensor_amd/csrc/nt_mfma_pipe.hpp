// The bf16 MFMA pipeline of a 256 x 256 output tile on gfx950, shared by the readout-fused
// sampler's pass 1 (rl_readout.hip) and the reduced-precision matmul (matmul.hip): one 256-thread
// workgroup, a wave per SIMD, each wave 256 rows x 64 columns as 8 x 2 v_mfma_f32_32x32x16_bf16
// tiles in its AGPRs, over K / 16 k-steps of operands in fragment order.
//
// Fragment order: the MFMA operands of 32 rows (or columns) g 32 .. g 32 + 31 for k-step s
// (k 16 s .. 16 s + 15) are one 1 KiB fragment, lane l's 16 bytes at 16 l holding row
// g 32 + l % 32 at k 16 s + 8 (l / 32) .. + 7. The row operand ("h"): row group g's fragment of
// step s at (g S + s) KiB from the tile's first row group. The column operand (the "weight"),
// tile-major: column group gi of the tile at (s 8 + gi) KiB, a tile's eight fragments of one step
// 8 KiB contiguous.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace nt {
namespace pipe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void *lds_ptr_t;

constexpr int kPipeDepth = 12;         // k-steps in flight: the column operand's register ring
constexpr int kPipeStages = 14;        // the row operand's LDS stages (one k-step each)
constexpr int kPipeStageBytes = 8192;  // one k-step of the row operand: eight fragments of 1 KiB
constexpr int kBufferWord3 = 0x00020000;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}


// Eight reads of 16 bytes: h's fragments of the eight row groups (1 KiB apart), and the wait
// for them, in one statement: the data came from LDS DMA, which the compiler's own wait insertion
// would treat as outstanding vector memory (a wait for every load in flight).
__device__ __forceinline__ void lds_read_a8(uint32_t a, v4u (&fa)[8]) {
    asm volatile(
        "ds_read_b128 %0, %8\n\t"
        "ds_read_b128 %1, %8 offset:1024\n\t"
        "ds_read_b128 %2, %8 offset:2048\n\t"
        "ds_read_b128 %3, %8 offset:3072\n\t"
        "ds_read_b128 %4, %8 offset:4096\n\t"
        "ds_read_b128 %5, %8 offset:5120\n\t"
        "ds_read_b128 %6, %8 offset:6144\n\t"
        "ds_read_b128 %7, %8 offset:7168\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(fa[0]), "=&v"(fa[1]), "=&v"(fa[2]), "=&v"(fa[3]), "=&v"(fa[4]), "=&v"(fa[5]), "=&v"(fa[6]), "=&v"(fa[7])
        : "v"(a)
        : "memory");
}

// One h fragment of a later k-step (OFF bytes past `a` in LDS) into `na`, issued only: the
// register is in flight until lds_wait_a8 below, and nothing may read it before it.
template <int OFF>
__device__ __forceinline__ void lds_issue_a1(uint32_t a, v4u &na) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(na) : "v"(a), "i"(OFF) : "memory");
}

// The wait for the eight lds_issue_a1 reads of a k-step; it takes the registers as in-out
// operands, so that every use of them comes after it.
__device__ __forceinline__ void lds_wait_a8(v4u (&na)[8]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(na[0]), "+v"(na[1]), "+v"(na[2]), "+v"(na[3]), "+v"(na[4]), "+v"(na[5]), "+v"(na[6]),
                   "+v"(na[7])
                 :
                 : "memory");
}

// The pipeline's state between run() and last_odd_step(): the column operand's register ring and
// the row operand's fragments of the last even step.
template <bool SWAP>
struct MfmaPipe {
    v4u br[kPipeDepth][2];
    v4u fx[8], fy[8];  // even steps' row fragments, odd steps'

    // acc += the tile's product over k-steps 0 .. 2 (S / 2) - 1. `lds` is kPipeStages *
    // kPipeStageBytes bytes; hres covers the tile's row operand (hoff: this wave's first byte,
    // 2 wave S 1024 + 16 lane); wrs the tile's column operand as four scalar words (woff:
    // 2 wave 1024 + 16 lane). Every load has landed on return, and every wave is past its last
    // read of the stages only after a barrier the caller places.
    __device__ __forceinline__ void run(uint8_t *lds, __amdgpu_buffer_rsrc_t hres, int hoff, const v4u &wrs, int woff,
                                        int S, int wave, int lane, f32x16_t (&acc)[8][2]) {
        const uint32_t lbase = uint32_t((uintptr_t)(lds_ptr_t)(lds)) + lane * 16;
    auto issue_a = [&](int t) {
        uint8_t *st = lds + (t % kPipeStages) * kPipeStageBytes + 2 * wave * 1024;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(hres, (lds_ptr_t)(st), 16, hoff + t * 1024, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(hres, (lds_ptr_t)(st + 1024), 16, hoff + S * 1024 + t * 1024, 0, 0,
                                                 0);
    };
    // The weight loads are written out, not left to the compiler: it cannot follow a register
    // ring across loop iterations and would wait for every load in flight before each step. The
    // waits below (for h's DMAs that this wave issued after these loads) cover them; nothing reads
    // the registers before that.
    auto load_b = [&](int t, v4u &b0, v4u &b1) {
        asm volatile(
            "buffer_load_dwordx4 %0, %2, %3, 0 offen\n\t"
            "buffer_load_dwordx4 %1, %2, %3, 0 offen offset:1024"
            : "=&v"(b0), "=&v"(b1)
            : "v"(woff + t * 8192), "s"(wrs)
            : "memory");
    };
    auto stage = [&](int t) { return lbase + (t % kPipeStages) * kPipeStageBytes; };
    // Steps go in pairs u, u + 1 (u even): a group is their four DMAs of h, then their four
    // weight loads, and every wave issues its groups in order. Group u + 12 goes out in the
    // iteration of steps u, u + 1. "Group u's DMAs have landed" is then "at most 4 + 8 n vector
    // memory operations outstanding", n the later groups issued; it also means every earlier
    // group, weights included, has landed.
#pragma unroll
    for (int u = 0; u < kPipeDepth; u += 2) {
        issue_a(u);
        issue_a(u + 1);
        asm volatile("" ::: "memory");
        load_b(u, br[u][0], br[u][1]);
        load_b(u + 1, br[u + 1][0], br[u + 1][1]);
        asm volatile("" ::: "memory");
    }
    constexpr int kGroupsAhead = kPipeDepth / 2 - 1;  // groups issued after the one awaited
    static_assert(4 + 8 * kGroupsAhead == 44, "the wait below");
    asm volatile("s_waitcnt vmcnt(44)" ::: "memory");  // group 0's DMAs
    // a bare barrier: each wave has waited for its own DMAs, and LDS is coherent within the
    // workgroup (__syncthreads' fence would wait for every DMA in flight)
    asm volatile("s_barrier" ::: "memory");
    lds_read_a8(stage(0), fx);
    // Iteration i: steps u = 2 i and u + 1, the matrix cores kept fed across the iteration's other
    // work by placing it between the MFMAs (one wave per SIMD: an instruction that is not an MFMA
    // runs while the MFMA before it executes, and a run of them leaves the matrix core idle).
    //  - wait for this wave's weight of step u;
    //  - step u's sixteen MFMAs (h in fx). Between the first eight go the eight reads of step
    //    u + 1's h fragments into fy (stage u + 1, complete for every wave since the previous
    //    iteration's barrier; fy's last reader, step u - 1's block, has issued). After the
    //    first two: the wait for group u + 2 (this wave's DMAs of steps u + 2, u + 3) and the
    //    barrier (every wave's have landed, and every wave is done reading stages u - 2 and
    //    u - 1, which the next DMAs reuse); between MFMAs 8 to 12, group u + 12's four DMAs;
    //  - step u + 1's sixteen MFMAs (h in fy), with step u + 2's reads into fx between the first
    //    eight and step u + 12's weight loads after the first (ring slot 2 k: step u's MFMAs
    //    have all issued); step u + 13's weight loads into slot 2 k + 1 after its last reader.
    // Each wave issues per group: h(u + 12) and h(u + 13) (four DMAs), then the weight of u + 12
    // and of u + 13 (two loads each), in that order, so "at most n vector memory operations
    // outstanding" names a point in that sequence: the weight of step u has landed at 42 (the
    // weight of u + 1 and five later groups after it), group u + 2's DMAs at 36.
    // (SWAP: the weight is the A operand and h the B one, tile (i, j) of the output then being
    // the transposed [32 columns][32 rows] block; else h is A and the output block [32 rows][32
    // columns])
    auto mfma1 = [&](int i, int j, const v4u &a, const v4u &b) {
        if constexpr (SWAP)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, b),
                                                                __builtin_bit_cast(bf16x8_t, a), acc[i][j], 0, 0, 0);
        else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                                __builtin_bit_cast(bf16x8_t, b), acc[i][j], 0, 0, 0);
    };
    auto dma_half = [&](int t, int g) {  // one of issue_a(t)'s two DMAs (row group 2 wave + g)
        uint8_t *st = lds + (t % kPipeStages) * kPipeStageBytes + (2 * wave + g) * 1024;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(hres, (lds_ptr_t)(st), 16, hoff + g * S * 1024 + t * 1024, 0, 0, 0);
    };
    // MFMA pair r of a step (h fragment r against both weight fragments), each followed by one
    // read of the next step's fragments (2 r, then 2 r + 1) into `nx`, pinned in that order.
#define NT_PIPE_PAIR_RD(r, fa, bb, nx, sa)                      \
    mfma1(r, 0, fa[r], bb[0]);                                \
    __builtin_amdgcn_sched_barrier(0);                        \
    lds_issue_a1<(2 * (r)) * 1024>(sa, nx[2 * (r)]);          \
    __builtin_amdgcn_sched_barrier(0);                        \
    mfma1(r, 1, fa[r], bb[1]);                                \
    __builtin_amdgcn_sched_barrier(0);                        \
    lds_issue_a1<(2 * (r) + 1) * 1024>(sa, nx[2 * (r) + 1]);  \
    __builtin_amdgcn_sched_barrier(0);
    const int NI = S / 2;
    int i0 = 0;
    static_assert(2 + 8 * (kGroupsAhead - 1) + 8 == 42 && 4 + 8 * (kGroupsAhead - 1) == 36, "the waits below");
    while (i0 < NI) {
#pragma unroll
        for (int k = 0; k < kPipeDepth / 2; k++) {
            const int i = i0 + k, u = 2 * i;
            if (i < NI) {
                v4u(&b)[2] = br[2 * k];
                v4u(&c)[2] = br[2 * k + 1];
                const uint32_t s1 = stage(u + 1), s2 = stage(u + 2);
                // (each wait is an asm statement that takes the weight registers it covers as
                // in-out operands: nothing that reads them can be placed before it)
                asm volatile("s_waitcnt vmcnt(42)" : "+v"(b[0]), "+v"(b[1]) : : "memory");
                __builtin_amdgcn_sched_barrier(0);
                NT_PIPE_PAIR_RD(0, fx, b, fy, s1)
                asm volatile("s_waitcnt vmcnt(36)" : "+v"(c[0]), "+v"(c[1]) : : "memory");
                asm volatile("s_barrier" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
                NT_PIPE_PAIR_RD(1, fx, b, fy, s1)
                NT_PIPE_PAIR_RD(2, fx, b, fy, s1)
                NT_PIPE_PAIR_RD(3, fx, b, fy, s1)
                mfma1(4, 0, fx[4], b[0]);
                __builtin_amdgcn_sched_barrier(0);
                dma_half(u + kPipeDepth, 0);
                __builtin_amdgcn_sched_barrier(0);
                mfma1(4, 1, fx[4], b[1]);
                __builtin_amdgcn_sched_barrier(0);
                dma_half(u + kPipeDepth, 1);
                __builtin_amdgcn_sched_barrier(0);
                mfma1(5, 0, fx[5], b[0]);
                __builtin_amdgcn_sched_barrier(0);
                dma_half(u + kPipeDepth + 1, 0);
                __builtin_amdgcn_sched_barrier(0);
                mfma1(5, 1, fx[5], b[1]);
                __builtin_amdgcn_sched_barrier(0);
                dma_half(u + kPipeDepth + 1, 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int r = 6; r < 8; r++) {
                    mfma1(r, 0, fx[r], b[0]);
                    mfma1(r, 1, fx[r], b[1]);
                }
                __builtin_amdgcn_sched_barrier(0);
                lds_wait_a8(fy);
                __builtin_amdgcn_sched_barrier(0);
                mfma1(0, 0, fy[0], c[0]);
                __builtin_amdgcn_sched_barrier(0);
                lds_issue_a1<0>(s2, fx[0]);
                __builtin_amdgcn_sched_barrier(0);
                load_b(u + kPipeDepth, b[0], b[1]);
                __builtin_amdgcn_sched_barrier(0);
                mfma1(0, 1, fy[0], c[1]);
                __builtin_amdgcn_sched_barrier(0);
                lds_issue_a1<1024>(s2, fx[1]);
                __builtin_amdgcn_sched_barrier(0);
                NT_PIPE_PAIR_RD(1, fy, c, fx, s2)
                NT_PIPE_PAIR_RD(2, fy, c, fx, s2)
                NT_PIPE_PAIR_RD(3, fy, c, fx, s2)
#pragma unroll
                for (int r = 4; r < 8; r++) {
                    mfma1(r, 0, fy[r], c[0]);
                    mfma1(r, 1, fy[r], c[1]);
                }
                __builtin_amdgcn_sched_barrier(0);
                load_b(u + kPipeDepth + 1, c[0], c[1]);
                lds_wait_a8(fx);
                asm volatile("" ::: "memory");
            }
        }
        i0 += kPipeDepth / 2;
    }
#undef NT_PIPE_PAIR_RD
    // Every copy, the ones past the last step included, lands before the stages are reused, and
    // every weight load lands before its registers can be given to anything else: the ring's
    // last loads are never read, so the wait takes the registers as in-out operands (a load into
    // a register the compiler thinks free would overwrite whatever it put there).
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(br[0][0]), "+v"(br[0][1]), "+v"(br[1][0]), "+v"(br[1][1]), "+v"(br[2][0]), "+v"(br[2][1]),
                   "+v"(br[3][0]), "+v"(br[3][1]), "+v"(br[4][0]), "+v"(br[4][1]), "+v"(br[5][0]), "+v"(br[5][1])
                 :
                 : "memory");
    asm volatile(""
                 : "+v"(br[6][0]), "+v"(br[6][1]), "+v"(br[7][0]), "+v"(br[7][1]), "+v"(br[8][0]), "+v"(br[8][1]),
                   "+v"(br[9][0]), "+v"(br[9][1]), "+v"(br[10][0]), "+v"(br[10][1]), "+v"(br[11][0]), "+v"(br[11][1])
                 :
                 : "memory");
    static_assert(kPipeDepth == 12, "the drain above names every ring slot");
    }

    // The last step when S is odd (its fragments are in fx, its column operand in the ring).
    __device__ __forceinline__ void last_odd_step(int S, f32x16_t (&acc)[8][2]) {
        auto mfmas = [&](const v4u(&fa)[8], const v4u &b0, const v4u &b1) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if constexpr (SWAP) {
                    acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, b0),
                                                                        __builtin_bit_cast(bf16x8_t, fa[i]), acc[i][0], 0, 0, 0);
                    acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, b1),
                                                                        __builtin_bit_cast(bf16x8_t, fa[i]), acc[i][1], 0, 0, 0);
                } else {
                    acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, fa[i]),
                                                                        __builtin_bit_cast(bf16x8_t, b0), acc[i][0], 0, 0, 0);
                    acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, fa[i]),
                                                                        __builtin_bit_cast(bf16x8_t, b1), acc[i][1], 0, 0, 0);
                }
            }
        };
    if (S & 1) {  // the last step, S - 1 = 2 NI: its fragments are in fx, its weight in slot (S - 1) % 12
        const int slot = (S - 1) % kPipeDepth;
        v4u b0 = br[0][0], b1 = br[0][1];
#pragma unroll
        for (int k = 1; k < kPipeDepth; k++)
            if (slot == k) {
                b0 = br[k][0];
                b1 = br[k][1];
            }
        mfmas(fx, b0, b1);
    }
    }
};

}  // namespace pipe
}  // namespace nt
