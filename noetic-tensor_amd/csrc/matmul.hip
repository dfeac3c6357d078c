// Batched f32 matmul of a Device::Hip tensor (GpuBackend::matmul, src/tensor/gpu/mod.rs:155-156),
// bit for bit the reference's product. The reference fixes the arithmetic of every output
// (src/tensor/cuda/kernels.rs:14-20, the order of matrixmultiply 0.3.11's sgemm that CpuRef calls
// per batch, src/tensor/kernels.rs:415-420): an fma chain from zero over k in order, closed every
// 256 k; the first block's chain is the total and each later block's chain is added to it. That
// order allows no split of one output's chain over lanes and no matrix-core instruction (an MFMA
// sums several products before it rounds), so this is a VALU kernel: each of a block's 256
// threads owns an 8x8 (or 4x4) register tile of outputs and runs their 64 (16) chains side by
// side, one v_fma_f32 per product, on A and B panels staged through LDS.
//
// Layout of a 128x128 block tile: thread (tx, ty) = (tid % 16, tid / 16) owns rows
// {ty*4 + i, 64 + ty*4 + i} and columns {tx*4 + j, 64 + tx*4 + j} (i, j < 4), so each k step
// reads its 8 A values and 8 B values as four 16-byte LDS reads (A's are broadcast: a wave spans
// four ty). The panels are double-buffered (one barrier per 16 k). Workgroups are renumbered so
// that each of the 8 XCDs (which the hardware deals consecutive workgroups to in turn) works on a
// contiguous run of tiles, whose A panels then stay in that XCD's L2.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "../../include/noetic_hip.h"
#include "../../include/noetic_ops.h"
#include "nt_internal.hpp"
#include "nt_mfma_pipe.hpp"

#ifndef NT_KERNELS_SHA
#define NT_KERNELS_SHA "unknown"
#endif

namespace nt {
namespace {

constexpr int kMmThreads = 256;
constexpr int kBK = 16;    // k per LDS stage
constexpr int kKC = 256;   // the chain is closed every kKC k
constexpr int kMaxBatchDims = NT_MAX_RANK - 2;
constexpr int kPad = 4;    // LDS row padding (keeps 16-byte alignment, spreads the stores' banks)

struct MatmulP {
    const float *a, *b;
    float *c;
    int64_t a_off, b_off;          // element offsets of batch 0
    int64_t a_rs, a_cs, b_rs, b_cs;
    int64_t bshape[kMaxBatchDims]; // the output's batch dimensions
    int64_t a_bs[kMaxBatchDims];   // per batch dimension: A's stride (0 where A broadcasts)
    int64_t b_bs[kMaxBatchDims];
    int64_t blocks;                // splits * batches * tiles_m * tiles_n
    float *slices;                 // split-k: [ceil(k / 256)][batches * m * n], one per 256-k block
    int64_t outputs;               // batches * m * n
    int32_t m, n, k;
    int32_t tm, tn;                // tiles along m and n
    int32_t nbd;                   // batch dimensions
    int32_t kc_per;                // split-k: 256-k blocks per split
    int32_t avec, bvec;            // matmul_half: the operand may be staged with 16-byte loads
};

// H = 2: 128x128 tile, 8x8 outputs per thread; H = 1: 64x64 tile, 4x4 per thread.
// AK: A is read along k (a_cs == 1); otherwise along m. BN: B is read along n (b_cs == 1);
// otherwise along k. Either way consecutive lanes read consecutive addresses when the view is
// contiguous along that dimension.
// SPLIT: the workgroup covers kc_per 256-k blocks of its tile and writes each block's chain to
// that block's slice; k_fold then closes the chains in order (the same arithmetic, more
// workgroups for outputs too few to fill the chip).
template <int H, bool AK, bool BN, bool SPLIT>
__device__ __forceinline__ void matmul_body(const MatmulP &p) {
    constexpr int T = 64 * H;             // tile edge
    constexpr int LPT = T * kBK / kMmThreads;  // elements of each panel a thread loads per stage
    __shared__ __attribute__((aligned(16))) float As[2][kBK][T + kPad];
    __shared__ __attribute__((aligned(16))) float Bs[2][kBK][T + kPad];

    const int tid = threadIdx.x;
    const int tx = tid % 16, ty = tid / 16;
    int64_t wg = blockIdx.x;
    const int64_t full = p.blocks / 8 * 8;
    if (wg < full) wg = (wg % 8) * (full / 8) + wg / 8;
    const int64_t per_batch = int64_t(p.tm) * p.tn;
    int64_t zs = wg / per_batch;  // split * batches + batch
    const int64_t rem = wg - zs * per_batch;
    int kbeg = 0, kend = p.k;
    if constexpr (SPLIT) {
        int64_t nbat = 1;
        for (int d = 0; d < p.nbd; d++) nbat *= p.bshape[d];
        const int sp = int(zs / nbat);
        zs -= int64_t(sp) * nbat;
        kbeg = sp * p.kc_per * kKC;
        kend = min(p.k, kbeg + p.kc_per * kKC);
    }
    const int64_t z = zs;
    const int row0 = int(rem / p.tn) * T, col0 = int(rem % p.tn) * T;
    int64_t ao = p.a_off, bo = p.b_off;
    {
        int64_t q = z;
        for (int d = p.nbd - 1; d >= 0; --d) {
            const int64_t i = q % p.bshape[d];
            q /= p.bshape[d];
            ao += i * p.a_bs[d];
            bo += i * p.b_bs[d];
        }
    }
    const float *a = p.a + ao;
    const float *b = p.b + bo;
    const int M = p.m, N = p.n, K = p.k;

    float ra[LPT], rb[LPT];
    // Interior panels of a view contiguous along one axis (16-byte aligned) load four values per
    // instruction. Along k (A row-major, B transposed): group g is row or column g / 4, k (g % 4) * 4
    // .. + 3. Along m or n (A transposed, B row-major): group g is k g / (T / 4), rows or columns
    // (g % (T / 4)) * 4 .. + 3.
    constexpr int V4 = LPT / 4;
    auto vec_a = [&](int k0) { return p.avec && row0 + T <= M && k0 + kBK <= K; };
    auto vec_b = [&](int k0) { return p.bvec && col0 + T <= N && k0 + kBK <= K; };
    auto load = [&](int k0) {
        const bool va = vec_a(k0), vb = vec_b(k0);
        if (va) {
#pragma unroll
            for (int q = 0; q < V4; q++) {
                const int g = tid + kMmThreads * q;
                const float *src = AK ? a + int64_t(row0 + g / 4) * p.a_rs + k0 + (g % 4) * 4
                                      : a + int64_t(k0 + g / (T / 4)) * p.a_cs + row0 + (g % (T / 4)) * 4;
                const float4 v = *reinterpret_cast<const float4 *>(src);
                ra[4 * q] = v.x;
                ra[4 * q + 1] = v.y;
                ra[4 * q + 2] = v.z;
                ra[4 * q + 3] = v.w;
            }
        }
        if (vb) {
#pragma unroll
            for (int q = 0; q < V4; q++) {
                const int g = tid + kMmThreads * q;
                const float *src = BN ? b + int64_t(k0 + g / (T / 4)) * p.b_rs + col0 + (g % (T / 4)) * 4
                                      : b + int64_t(col0 + g / 4) * p.b_cs + k0 + (g % 4) * 4;
                const float4 v = *reinterpret_cast<const float4 *>(src);
                rb[4 * q] = v.x;
                rb[4 * q + 1] = v.y;
                rb[4 * q + 2] = v.z;
                rb[4 * q + 3] = v.w;
            }
        }
#pragma unroll
        for (int i = 0; i < LPT; i++) {
            const int e = tid + kMmThreads * i;
            int r, kk;
            if constexpr (AK) {
                kk = e % kBK;
                r = e / kBK;
            } else {
                r = e % T;
                kk = e / T;
            }
            const int gr = row0 + r, gk = k0 + kk;
            if (!va) ra[i] = (gr < M && gk < K) ? a[int64_t(gr) * p.a_rs + int64_t(gk) * p.a_cs] : 0.0f;
            int cc;
            if constexpr (BN) {
                cc = e % T;
                kk = e / T;
            } else {
                kk = e % kBK;
                cc = e / kBK;
            }
            const int gc = col0 + cc, gk2 = k0 + kk;
            if (!vb) rb[i] = (gc < N && gk2 < K) ? b[int64_t(gk2) * p.b_rs + int64_t(gc) * p.b_cs] : 0.0f;
        }
    };
    auto stash = [&](int s, int k0) {
        if (vec_a(k0)) {
#pragma unroll
            for (int q = 0; q < V4; q++) {
                const int g = tid + kMmThreads * q;
                if constexpr (AK) {
#pragma unroll
                    for (int j = 0; j < 4; j++) As[s][(g % 4) * 4 + j][g / 4] = ra[4 * q + j];
                } else {
                    *reinterpret_cast<float4 *>(&As[s][g / (T / 4)][(g % (T / 4)) * 4]) =
                        make_float4(ra[4 * q], ra[4 * q + 1], ra[4 * q + 2], ra[4 * q + 3]);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < LPT; i++) {
                const int e = tid + kMmThreads * i;
                if constexpr (AK) As[s][e % kBK][e / kBK] = ra[i];
                else As[s][e / T][e % T] = ra[i];
            }
        }
        if (vec_b(k0)) {
#pragma unroll
            for (int q = 0; q < V4; q++) {
                const int g = tid + kMmThreads * q;
                if constexpr (BN) {
                    *reinterpret_cast<float4 *>(&Bs[s][g / (T / 4)][(g % (T / 4)) * 4]) =
                        make_float4(rb[4 * q], rb[4 * q + 1], rb[4 * q + 2], rb[4 * q + 3]);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++) Bs[s][(g % 4) * 4 + j][g / 4] = rb[4 * q + j];
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < LPT; i++) {
                const int e = tid + kMmThreads * i;
                if constexpr (BN) Bs[s][e / T][e % T] = rb[i];
                else Bs[s][e % kBK][e / kBK] = rb[i];
            }
        }
    };

    float acc[4 * H][4 * H], tot[SPLIT ? 1 : 4 * H][SPLIT ? 1 : 4 * H];
#pragma unroll
    for (int i = 0; i < 4 * H; i++)
#pragma unroll
        for (int j = 0; j < 4 * H; j++) acc[i][j] = 0.0f;
    if constexpr (!SPLIT) {
#pragma unroll
        for (int i = 0; i < 4 * H; i++)
#pragma unroll
            for (int j = 0; j < 4 * H; j++) tot[i][j] = 0.0f;
    }
    // split-k: a closed chain goes to its 256-k block's slice, at the tile's outputs
    auto put_slice = [&](int kc) {
        float *sl = p.slices + int64_t(kc) * p.outputs + z * int64_t(p.m) * p.n;
#pragma unroll
        for (int hr = 0; hr < H; hr++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = row0 + hr * 64 + ty * 4 + i;
                if (r >= p.m) continue;
#pragma unroll
                for (int hc = 0; hc < H; hc++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int cc = col0 + hc * 64 + tx * 4 + j;
                        if (cc < p.n) sl[int64_t(r) * p.n + cc] = acc[hr * 4 + i][hc * 4 + j];
                    }
            }
    };

    auto step = [&](int s, int kk) {
        float av[4 * H], bv[4 * H];
#pragma unroll
        for (int h = 0; h < H; h++) {
            const float4 x = *reinterpret_cast<const float4 *>(&As[s][kk][h * 64 + ty * 4]);
            const float4 y = *reinterpret_cast<const float4 *>(&Bs[s][kk][h * 64 + tx * 4]);
            av[4 * h] = x.x;
            av[4 * h + 1] = x.y;
            av[4 * h + 2] = x.z;
            av[4 * h + 3] = x.w;
            bv[4 * h] = y.x;
            bv[4 * h + 1] = y.y;
            bv[4 * h + 2] = y.z;
            bv[4 * h + 3] = y.w;
        }
#pragma unroll
        for (int i = 0; i < 4 * H; i++)
#pragma unroll
            for (int j = 0; j < 4 * H; j++) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
    };

    load(kbeg);
    stash(0, kbeg);
    __syncthreads();
    int s = 0;
    for (int k0 = kbeg; k0 < kend; k0 += kBK) {
        const bool more = k0 + kBK < kend;
        if (more) load(k0 + kBK);  // the next panels' loads are in flight during this stage
        if (k0 + kBK <= K) {
#pragma unroll
            for (int kk = 0; kk < kBK; kk++) step(s, kk);
        } else {
            const int kmax = K - k0;
            for (int kk = 0; kk < kmax; kk++) step(s, kk);
        }
        if ((k0 + kBK) % kKC == 0 || !more) {
            if constexpr (SPLIT) {
                put_slice(k0 / kKC);
#pragma unroll
                for (int i = 0; i < 4 * H; i++)
#pragma unroll
                    for (int j = 0; j < 4 * H; j++) acc[i][j] = 0.0f;
            } else {
                const bool first = k0 < kKC;
#pragma unroll
                for (int i = 0; i < 4 * H; i++)
#pragma unroll
                    for (int j = 0; j < 4 * H; j++) {
                        tot[i][j] = first ? acc[i][j] : acc[i][j] + tot[i][j];
                        acc[i][j] = 0.0f;
                    }
            }
        }
        if (more) stash(s ^ 1, k0 + kBK);  // the other buffer was last read before the previous barrier
        __syncthreads();
        s ^= 1;
    }
    if constexpr (SPLIT) return;

    float *c = p.c + z * int64_t(M) * N;
    const bool vec = (N % 4) == 0;
#pragma unroll
    for (int hr = 0; hr < H; hr++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = row0 + hr * 64 + ty * 4 + i;
            if (r >= M) continue;
            float *crow = c + int64_t(r) * N;
#pragma unroll
            for (int hc = 0; hc < H; hc++) {
                const int c0 = col0 + hc * 64 + tx * 4;
                const int ri = SPLIT ? 0 : hr * 4 + i, cj = SPLIT ? 0 : hc * 4;
                if (vec && c0 + 3 < N) {
                    *reinterpret_cast<float4 *>(crow + c0) =
                        make_float4(tot[ri][SPLIT ? 0 : cj], tot[ri][SPLIT ? 0 : cj + 1], tot[ri][SPLIT ? 0 : cj + 2],
                                    tot[ri][SPLIT ? 0 : cj + 3]);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        if (c0 + j < N) crow[c0 + j] = tot[ri][SPLIT ? 0 : cj + j];
                }
            }
        }
}

// The 128 tile's 128 accumulators fill the register file at one wave per SIMD; asking for two
// waves per SIMD spills a few rarely used registers to scratch and lets one wave's fmas cover the
// other's LDS reads (3.39 -> 2.33 ms at 4096^3). The 64 tile keeps its 4-5 waves per SIMD.
template <bool AK, bool BN, bool SPLIT>
__global__ __launch_bounds__(kMmThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_matmul128(MatmulP p) {
    matmul_body<2, AK, BN, SPLIT>(p);
}

template <bool AK, bool BN, bool SPLIT>
__global__ __launch_bounds__(kMmThreads) void k_matmul64(MatmulP p) {
    matmul_body<1, AK, BN, SPLIT>(p);
}

// Split-k's closing pass: per output, the first 256-k block's chain is the total and each later
// block's chain is added to it, in order (the unsplit kernel's closure, element for element).
__global__ void k_fold(const float *slices, int64_t outputs, int nkc, float *out) {
    for (int64_t o = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; o < outputs;
         o += int64_t(gridDim.x) * blockDim.x) {
        float t = slices[o];
        for (int j = 1; j < nkc; j++) t = slices[int64_t(j) * outputs + o] + t;
        out[o] = t;
    }
}

// ---------------------------------------------------------------------------- matmul_half
// The reduced-precision product (GpuBackend::matmul_half, gpu/mod.rs:157-162; the CUDA backend's
// hgemm_bf16_f32acc, cuda/half_gemm.rs:32-...): f32 operands rounded to bf16 (nearest even) as
// they are staged, products summed in f32 on the matrix cores. A 256-thread workgroup computes a
// 128x128 tile: each wave a 64x64 quarter as 2x2 v_mfma_f32_32x32x16_bf16 tiles, over k panels of
// 32 staged through LDS as bf16 ([row][k] for A, [column][k] for B, so that every MFMA operand
// is one 16-byte LDS read: lane l takes row or column l % 32 and k 8 (l / 32) .. 8 (l / 32) + 7).
// (The 64x64 tile takes k panels of 64.)
// The next panel's f32 loads are issued before the current panel's MFMAs. Interior panels of an
// operand whose view is contiguous along one axis (16-byte aligned) are staged four values per
// load: along k they go to LDS as they are, along m or n each thread loads a 4x4 block and
// transposes it in registers, so that every LDS store writes four bf16 of one row.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
constexpr int kHPad = 8;  // bf16 padding per LDS row (rows stay 16-byte aligned)

__device__ __forceinline__ uint16_t bf16_bits(float x) {
    uint32_t r;
    asm("v_cvt_pk_bf16_f32 %0, %1, %1" : "=v"(r) : "v"(x));
    return uint16_t(r);
}

// T = 128: each wave a 64x64 quarter (2x2 MFMA tiles); T = 64 (outputs too few for 512 workgroups
// of 128): each wave a 32x32 quarter (one MFMA tile).
template <int T, bool AK, bool BN>
__global__ __launch_bounds__(kMmThreads) void k_matmul_half(MatmulP p) {
    constexpr int kHT = T;
    // k per panel: 64 for the 64 tile (longer panels cover more of the loads' latency); 32 for the
    // 128 tile, whose registers would otherwise hold it to one wave per SIMD
    constexpr int kHK = T == 64 ? 64 : 32;
    constexpr int W = T / 64;                         // MFMA tiles per wave along m and along n
    constexpr int kHLoads = kHT * kHK / kMmThreads;   // scalar f32 loads per operand and thread
    constexpr int kQuads = kHT * (kHK / 4) / kMmThreads;  // 16-byte loads along k per thread
    constexpr int kRG = kHT / 4;                      // 4x4 blocks along m or n
    constexpr int kQ4 = kHK / 4;                      // 4-k groups along k
    constexpr int kBlk = (kRG * kQ4 + kMmThreads - 1) / kMmThreads;  // 4x4 blocks per thread
    constexpr int kRegs = kHLoads > 16 * kBlk ? kHLoads : 16 * kBlk;
    __shared__ __attribute__((aligned(16))) uint16_t As[kHT][kHK + kHPad];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[kHT][kHK + kHPad];
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    int64_t wg = blockIdx.x;
    const int64_t full = p.blocks / 8 * 8;
    if (wg < full) wg = (wg % 8) * (full / 8) + wg / 8;
    const int64_t per_batch = int64_t(p.tm) * p.tn;
    const int64_t z = wg / per_batch;
    const int64_t rem = wg - z * per_batch;
    const int row0 = int(rem / p.tn) * kHT, col0 = int(rem % p.tn) * kHT;
    int64_t ao = p.a_off, bo = p.b_off;
    {
        int64_t q = z;
        for (int d = p.nbd - 1; d >= 0; --d) {
            const int64_t i = q % p.bshape[d];
            q /= p.bshape[d];
            ao += i * p.a_bs[d];
            bo += i * p.b_bs[d];
        }
    }
    const float *a = p.a + ao;
    const float *b = p.b + bo;
    const int M = p.m, N = p.n, K = p.k;

    float ra[kRegs], rb[kRegs];
    // 16-byte staging for this panel? (an interior panel of a vector-eligible view)
    auto vec_a = [&](int k0) { return p.avec && row0 + kHT <= M && k0 + kHK <= K; };
    auto vec_b = [&](int k0) { return p.bvec && col0 + kHT <= N && k0 + kHK <= K; };
    auto load = [&](int k0) {
        if (vec_a(k0)) {
            if constexpr (AK) {  // along k: group g covers row g / kQ4, k (g % kQ4) * 4 .. + 3
#pragma unroll
                for (int q = 0; q < kQuads; q++) {
                    const int g = tid + kMmThreads * q;
                    const float4 v =
                        *reinterpret_cast<const float4 *>(a + int64_t(row0 + g / kQ4) * p.a_rs + k0 + (g % kQ4) * 4);
                    ra[4 * q] = v.x;
                    ra[4 * q + 1] = v.y;
                    ra[4 * q + 2] = v.z;
                    ra[4 * q + 3] = v.w;
                }
            } else {  // along m: block id: rows (id % kRG) * 4 .. + 3 at k (id / kRG) * 4 + q
#pragma unroll
                for (int bb = 0; bb < kBlk; bb++) {
                    const int id = tid + kMmThreads * bb, rg = id % kRG, kg = id / kRG;
                    if (kg >= kQ4) continue;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float4 v =
                            *reinterpret_cast<const float4 *>(a + row0 + rg * 4 + int64_t(k0 + kg * 4 + q) * p.a_cs);
                        ra[16 * bb + 4 * q] = v.x;
                        ra[16 * bb + 4 * q + 1] = v.y;
                        ra[16 * bb + 4 * q + 2] = v.z;
                        ra[16 * bb + 4 * q + 3] = v.w;
                    }
                }
            }
        }
        if (vec_b(k0)) {
            if constexpr (BN) {  // along n: block id: columns (id % kRG) * 4 .. + 3 at k (id / kRG) * 4 + q
#pragma unroll
                for (int bb = 0; bb < kBlk; bb++) {
                    const int id = tid + kMmThreads * bb, rg = id % kRG, kg = id / kRG;
                    if (kg >= kQ4) continue;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float4 v =
                            *reinterpret_cast<const float4 *>(b + int64_t(k0 + kg * 4 + q) * p.b_rs + col0 + rg * 4);
                        rb[16 * bb + 4 * q] = v.x;
                        rb[16 * bb + 4 * q + 1] = v.y;
                        rb[16 * bb + 4 * q + 2] = v.z;
                        rb[16 * bb + 4 * q + 3] = v.w;
                    }
                }
            } else {  // along k: group g covers column g / kQ4, k (g % kQ4) * 4 .. + 3
#pragma unroll
                for (int q = 0; q < kQuads; q++) {
                    const int g = tid + kMmThreads * q;
                    const float4 v =
                        *reinterpret_cast<const float4 *>(b + int64_t(col0 + g / kQ4) * p.b_cs + k0 + (g % kQ4) * 4);
                    rb[4 * q] = v.x;
                    rb[4 * q + 1] = v.y;
                    rb[4 * q + 2] = v.z;
                    rb[4 * q + 3] = v.w;
                }
            }
        }
        const bool sa = !vec_a(k0), sb = !vec_b(k0);
#pragma unroll
        for (int i = 0; i < kHLoads; i++) {
            const int e = tid + kMmThreads * i;
            int r, kk;
            if constexpr (AK) {
                kk = e % kHK;
                r = e / kHK;
            } else {
                r = e % kHT;
                kk = e / kHT;
            }
            const int gr = row0 + r, gk = k0 + kk;
            if (sa) ra[i] = (gr < M && gk < K) ? a[int64_t(gr) * p.a_rs + int64_t(gk) * p.a_cs] : 0.0f;
            int cc;
            if constexpr (BN) {
                cc = e % kHT;
                kk = e / kHT;
            } else {
                kk = e % kHK;
                cc = e / kHK;
            }
            const int gc = col0 + cc, gk2 = k0 + kk;
            if (sb) rb[i] = (gc < N && gk2 < K) ? b[int64_t(gk2) * p.b_rs + int64_t(gc) * p.b_cs] : 0.0f;
        }
    };
    // four bf16 of one LDS row (k .. k + 3) in one 8-byte store
    auto put4 = [](uint16_t *dst, float x0, float x1, float x2, float x3) {
        uint32_t lo, hi;
        asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(lo) : "v"(x0), "v"(x1));
        asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(hi) : "v"(x2), "v"(x3));
        *reinterpret_cast<uint2 *>(dst) = make_uint2(lo, hi);
    };
    auto stash = [&](int k0) {
        if (vec_a(k0)) {
            if constexpr (AK) {
#pragma unroll
                for (int q = 0; q < kQuads; q++) {
                    const int g = tid + kMmThreads * q;
                    put4(&As[g / kQ4][(g % kQ4) * 4], ra[4 * q], ra[4 * q + 1], ra[4 * q + 2], ra[4 * q + 3]);
                }
            } else {
#pragma unroll
                for (int bb = 0; bb < kBlk; bb++) {
                    const int id = tid + kMmThreads * bb, rg = id % kRG, kg = id / kRG;
                    if (kg >= kQ4) continue;
                    const float *w = ra + 16 * bb;
#pragma unroll
                    for (int j = 0; j < 4; j++)  // row rg * 4 + j, k kg * 4 .. + 3
                        put4(&As[rg * 4 + j][kg * 4], w[j], w[4 + j], w[8 + j], w[12 + j]);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kHLoads; i++) {
                const int e = tid + kMmThreads * i;
                if constexpr (AK) As[e / kHK][e % kHK] = bf16_bits(ra[i]);
                else As[e % kHT][e / kHT] = bf16_bits(ra[i]);
            }
        }
        if (vec_b(k0)) {
            if constexpr (BN) {
#pragma unroll
                for (int bb = 0; bb < kBlk; bb++) {
                    const int id = tid + kMmThreads * bb, rg = id % kRG, kg = id / kRG;
                    if (kg >= kQ4) continue;
                    const float *w = rb + 16 * bb;
#pragma unroll
                    for (int j = 0; j < 4; j++)  // column rg * 4 + j, k kg * 4 .. + 3
                        put4(&Bs[rg * 4 + j][kg * 4], w[j], w[4 + j], w[8 + j], w[12 + j]);
                }
            } else {
#pragma unroll
                for (int q = 0; q < kQuads; q++) {
                    const int g = tid + kMmThreads * q;
                    put4(&Bs[g / kQ4][(g % kQ4) * 4], rb[4 * q], rb[4 * q + 1], rb[4 * q + 2], rb[4 * q + 3]);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kHLoads; i++) {
                const int e = tid + kMmThreads * i;
                if constexpr (BN) Bs[e % kHT][e / kHT] = bf16_bits(rb[i]);
                else Bs[e / kHK][e % kHK] = bf16_bits(rb[i]);
            }
        }
    };

    f32x16_t acc[W][W];
#pragma unroll
    for (int i = 0; i < W; i++)
#pragma unroll
        for (int j = 0; j < W; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;
    const int wm = (wave / 2) * 32 * W, wn = (wave % 2) * 32 * W;
    const int fr = lane % 32, fk = 8 * (lane / 32);

    load(0);
    for (int k0 = 0; k0 < K; k0 += kHK) {
        stash(k0);
        __syncthreads();
        if (k0 + kHK < K) load(k0 + kHK);  // in flight during this panel's MFMAs
#pragma unroll
        for (int ks = 0; ks < kHK; ks += 16) {
            bf16x8_t af[W], bf[W];
#pragma unroll
            for (int t = 0; t < W; t++) {
                af[t] = *reinterpret_cast<const bf16x8_t *>(&As[wm + t * 32 + fr][ks + fk]);
                bf[t] = *reinterpret_cast<const bf16x8_t *>(&Bs[wn + t * 32 + fr][ks + fk]);
            }
#pragma unroll
            for (int i = 0; i < W; i++)
#pragma unroll
                for (int j = 0; j < W; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    float *c = p.c + z * int64_t(M) * N;
#pragma unroll
    for (int i = 0; i < W; i++)
#pragma unroll
        for (int j = 0; j < W; j++) {
            const int col = col0 + wn + j * 32 + fr;
            if (col >= N) continue;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = row0 + wm + i * 32 + 8 * (v / 4) + 4 * (lane / 32) + (v % 4);
                if (row < M) c[int64_t(row) * N + col] = acc[i][j][v];
            }
        }
}

// ------------------------------------------------- matmul_half, packed operands (large products)
// For products of many 256 x 256 output tiles the operands are rounded to bf16 once, into the
// matrix cores' fragment order (the row operand A in row groups of 32, the column operand B
// tile-major in tiles of 256 columns; rows, columns and k past the ends are zeros), and each
// workgroup then runs the bf16 MFMA pipeline of nt_mfma_pipe.hpp over one 256 x 256 tile of one
// batch: the same instruction over the same k order from zero as the staged kernel above, so each
// output is the same sum. The packing reads each f32 operand once and writes half its bytes; the
// tiles then read bf16 fragments only, 16 or 32 bytes per lane per load.

// The batch element offsets of A and B for output batch z (broadcast dimensions repeat).
__device__ __forceinline__ void batch_offsets(const MatmulP &p, int64_t z, int64_t *ao, int64_t *bo) {
    int64_t a = p.a_off, b = p.b_off, q = z;
    for (int d = p.nbd - 1; d >= 0; --d) {
        const int64_t i = q % p.bshape[d];
        q /= p.bshape[d];
        a += i * p.a_bs[d];
        b += i * p.b_bs[d];
    }
    *ao = a;
    *bo = b;
}

// Eight f32 at src + e stride (e < 8, those at or past `lim` zero) as eight bf16, nearest even
// (two 16-byte loads when the eight are contiguous and aligned).
__device__ __forceinline__ uint4 pack8(const float *src, int64_t stride, int lim) {
    float x[8];
    if (stride == 1 && lim == 8 && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
        const float4 u = reinterpret_cast<const float4 *>(src)[0], v = reinterpret_cast<const float4 *>(src)[1];
        x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w;
        x[4] = v.x; x[5] = v.y; x[6] = v.z; x[7] = v.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = e < lim ? src[e * stride] : 0.0f;
    }
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; q++) asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(w[q]) : "v"(x[2 * q]), "v"(x[2 * q + 1]));
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// One batch's A (row-group fragments) and B (tile-major column fragments) in one launch, batch
// z = blockIdx.y; the first `ablocks` blocks of a row of the grid take A's lanes, the rest B's.
// A: fragment (g, s) of G x S at (g S + s) KiB from the batch's start (G S KiB apart); lane l's
// 16 bytes are row 32 g + l % 32, k 16 s + 8 (l / 32) .. + 7.
// B: tile t of T, step s, column group gi at ((t S + s) 8 + gi) KiB from the batch's start
// (T S 8 KiB apart); lane l's 16 bytes are column 32 (8 t + gi) + l % 32, k 16 s + 8 (l / 32) ..
// + 7. One thread per lane of a fragment.
__global__ void k_pack_half(MatmulP p, int G, int T, int S, int ablocks, uint8_t *pa, uint8_t *pb) {
    const int64_t z = blockIdx.y;
    int64_t ao, bo;
    batch_offsets(p, z, &ao, &bo);
    if (int(blockIdx.x) < ablocks) {
        const int64_t total = int64_t(G) * S * 64;
        for (int64_t idx = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; idx < total;
             idx += int64_t(ablocks) * blockDim.x) {
            const int l = int(idx % 64);
            const int64_t q = idx / 64;
            const int s = int(q % S), g = int(q / S);
            const int row = 32 * g + (l & 31), k0 = 16 * s + 8 * (l >> 5);
            const int lim = row < p.m ? min(8, p.k - k0) : 0;
            const uint4 v = pack8(p.a + ao + int64_t(row < p.m ? row : 0) * p.a_rs + int64_t(k0) * p.a_cs, p.a_cs, lim);
            *reinterpret_cast<uint4 *>(pa + (z * G * S + (int64_t(g) * S + s)) * 1024 + l * 16) = v;
        }
    } else {
        const int64_t total = int64_t(T) * S * 8 * 64;
        const int bblocks = int(gridDim.x) - ablocks;
        for (int64_t idx = (blockIdx.x - ablocks) * int64_t(blockDim.x) + threadIdx.x; idx < total;
             idx += int64_t(bblocks) * blockDim.x) {
            const int l = int(idx % 64);
            const int64_t q = idx / 64;  // (t S + s) 8 + gi
            const int gi = int(q % 8);
            const int64_t ts = q / 8;
            const int s = int(ts % S), t = int(ts / S);
            const int col = 32 * (8 * t + gi) + (l & 31), k0 = 16 * s + 8 * (l >> 5);
            const int lim = col < p.n ? min(8, p.k - k0) : 0;
            const uint4 v = pack8(p.b + bo + int64_t(col < p.n ? col : 0) * p.b_cs + int64_t(k0) * p.b_rs, p.b_rs, lim);
            *reinterpret_cast<uint4 *>(pb + (z * T * S * 8 + q) * 1024 + l * 16) = v;
        }
    }
}

// The packed path from this many 256 x 256 output tiles and this k (below them the staged kernel,
// whose operands need no second pass).
constexpr int64_t kHalfPackedTiles = 64;
constexpr int64_t kHalfPackedK = 256;

// One 256 x 256 output tile (tm_i, tn_i) of batch z per workgroup. Workgroup w is tile
// (w / (tm tn)) of the batches, then row tiles in order within a column tile: consecutive
// workgroups share their B tile, and the 8 XCDs (dealt workgroups in turn) each hold every
// eighth row tile of it.
__global__ __launch_bounds__(256) void k_half_tiles(MatmulP p, const uint8_t *pa, const uint8_t *pb, int G, int T,
                                                     int S) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[pipe::kPipeStages * pipe::kPipeStageBytes];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t wg = blockIdx.x, per_batch = int64_t(p.tm) * p.tn;
    const int64_t z = wg / per_batch;
    const int rem = int(wg - z * per_batch);
    const int tn_i = rem / p.tm, tm_i = rem % p.tm;
    // this tile's row groups of A (rows past the batch's last group read as zeros: the range)
    const int g0 = 8 * tm_i, ng = min(8, G - g0);
    const __amdgpu_buffer_rsrc_t hres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(pa + (z * G + g0) * int64_t(S) * 1024), short(0), ng * S * 1024, pipe::kBufferWord3);
    const int hoff = 2 * wave * S * 1024 + lane * 16, woff = 2 * wave * 1024 + lane * 16;
    const uint64_t wbase = reinterpret_cast<uint64_t>(pb + (z * T + tn_i) * int64_t(S) * 8192);
    const pipe::v4u wrs = {uint32_t(wbase), uint32_t(wbase >> 32), uint32_t(S * 8192), uint32_t(pipe::kBufferWord3)};
    pipe::f32x16_t acc[8][2];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;
    pipe::MfmaPipe<false> pp;
    pp.run(lds, hres, hoff, wrs, woff, S, wave, lane, acc);
    pp.last_odd_step(S, acc);
    // lane l holds rows 32 i + 8 (v / 4) + 4 (l / 32) + v % 4, column 64 wave + 32 j + l % 32
    float *c = p.c + z * int64_t(p.m) * p.n;
    const int row0 = 256 * tm_i, col0 = 256 * tn_i + 64 * wave + (lane & 31);
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int col = col0 + 32 * j;
        if (col >= p.n) continue;
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int row = row0 + 32 * i + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
                if (row < p.m) c[int64_t(row) * p.n + col] = acc[i][j][v];
            }
    }
}

template <int H, bool SPLIT>
int launch_matmul(const MatmulP &p, bool ak, bool bn, hipStream_t s) {
    const dim3 grid(unsigned(p.blocks)), block(kMmThreads);
    if constexpr (H == 2) {
        if (ak && bn) hipLaunchKernelGGL((k_matmul128<true, true, SPLIT>), grid, block, 0, s, p);
        else if (ak) hipLaunchKernelGGL((k_matmul128<true, false, SPLIT>), grid, block, 0, s, p);
        else if (bn) hipLaunchKernelGGL((k_matmul128<false, true, SPLIT>), grid, block, 0, s, p);
        else hipLaunchKernelGGL((k_matmul128<false, false, SPLIT>), grid, block, 0, s, p);
    } else {
        if (ak && bn) hipLaunchKernelGGL((k_matmul64<true, true, SPLIT>), grid, block, 0, s, p);
        else if (ak) hipLaunchKernelGGL((k_matmul64<true, false, SPLIT>), grid, block, 0, s, p);
        else if (bn) hipLaunchKernelGGL((k_matmul64<false, true, SPLIT>), grid, block, 0, s, p);
        else hipLaunchKernelGGL((k_matmul64<false, false, SPLIT>), grid, block, 0, s, p);
    }
    return launched("k_matmul");
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" {

int nt_hip_matmul(const float *a, const NtLayout *al, const float *b, const NtLayout *bl, float *out) {
    if (!al || !bl) return fail(NT_E_ARG, "matmul: null layout");
    const int r = al->rank;
    if (r < 2 || r > NT_MAX_RANK || bl->rank != r || al->shape[r - 1] != bl->shape[r - 2])
        return fail(NT_E_ARG, "matmul: shapes [" + std::to_string(r) + "-d] do not multiply (rank >= 2, equal "
                              "ranks, a's last dimension equal to b's second last)");
    for (int d = 0; d < r; d++)
        if (al->shape[d] < 0 || bl->shape[d] < 0 || al->strides[d] < 0 || bl->strides[d] < 0 || al->offset < 0 ||
            bl->offset < 0)
            return fail(NT_E_ARG, "matmul: negative shape, stride or offset");
    MatmulP p{};
    p.nbd = r - 2;
    int64_t nb = 1;
    for (int d = 0; d < r - 2; d++) {
        const int64_t x = al->shape[d], y = bl->shape[d];
        if (x != y && x != 1 && y != 1)
            return fail(NT_E_ARG, "matmul: batch dimension " + std::to_string(d) + " does not broadcast (" +
                                      std::to_string(x) + " against " + std::to_string(y) + ")");
        p.bshape[d] = x == 1 ? y : x;
        p.a_bs[d] = x == 1 ? 0 : al->strides[d];
        p.b_bs[d] = y == 1 ? 0 : bl->strides[d];
        nb *= p.bshape[d];
    }
    const int64_t m = al->shape[r - 2], k = al->shape[r - 1], n = bl->shape[r - 1];
    if (m >= (int64_t(1) << 31) - 256 || n >= (int64_t(1) << 31) - 256 || k >= (int64_t(1) << 31) - 256)
        return fail(NT_E_ARG, "matmul: m, k and n must each be below 2^31 - 256");
    if (nb == 0 || m == 0 || n == 0) return 0;
    if (!a || !b || !out) return fail(NT_E_ARG, "matmul: null buffer");
    p.a = a;
    p.b = b;
    p.c = out;
    p.a_off = al->offset;
    p.b_off = bl->offset;
    p.a_rs = al->strides[r - 2];
    p.a_cs = al->strides[r - 1];
    p.b_rs = bl->strides[r - 2];
    p.b_cs = bl->strides[r - 1];
    p.m = int32_t(m);
    p.n = int32_t(n);
    p.k = int32_t(k);
    // 128x128 tiles when they give at least two workgroups per CU of the 256, else 64x64.
    const int64_t big = nb * ((m + 127) / 128) * ((n + 127) / 128);
    const int H = big >= 512 ? 2 : 1;
    const int T = 64 * H;
    p.tm = int32_t((m + T - 1) / T);
    p.tn = int32_t((n + T - 1) / T);
    const int64_t tiles = nb * p.tm * p.tn;
    p.outputs = nb * m * n;
    // Split k over more workgroups when the tiles alone leave CUs idle: each workgroup takes
    // kc_per of the ceil(k / 256) chains, so that about 1024 workgroups run in all.
    const int64_t nkc = (k + kKC - 1) / kKC;
    int64_t splits = 1;
    // (the slices take 4 bytes per output and 256-k block; past 1 GiB the tiles run unsplit)
    if (tiles < 1024 && nkc > 1 && nkc * p.outputs <= (int64_t(1) << 28)) {
        const int64_t want = (1024 + tiles - 1) / tiles;
        const int64_t per = (nkc + std::min(want, nkc) - 1) / std::min(want, nkc);
        p.kc_per = int32_t(per);
        splits = (nkc + per - 1) / per;
    }
    p.blocks = tiles * splits;
    if (p.blocks > int64_t(0x7fffffff)) return fail(NT_E_ARG, "matmul: too many output tiles");
    const bool ak = k == 1 || p.a_cs == 1;
    const bool bn = n == 1 || p.b_cs == 1;
    {
        // 16-byte panel loads: a view contiguous along its read axis whose other stride, batch
        // offsets and base are 16-byte aligned
        auto aligned = [&](const int64_t *bs, int64_t off, int64_t other, const float *base) {
            if (off % 4 != 0 || other % 4 != 0 || (reinterpret_cast<uintptr_t>(base) & 15) != 0) return false;
            for (int d = 0; d < r - 2; d++)
                if (bs[d] % 4 != 0) return false;
            return true;
        };
        p.avec = ak ? (p.a_cs == 1 && aligned(p.a_bs, p.a_off, p.a_rs, a))
                    : (p.a_rs == 1 && aligned(p.a_bs, p.a_off, p.a_cs, a));
        p.bvec = bn ? (p.b_cs == 1 && aligned(p.b_bs, p.b_off, p.b_rs, b))
                    : (p.b_rs == 1 && aligned(p.b_bs, p.b_off, p.b_cs, b));
    }
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    hipStream_t st = ctx().stream;
    if (splits == 1) return H == 2 ? launch_matmul<2, false>(p, ak, bn, st) : launch_matmul<1, false>(p, ak, bn, st);
    void *sl = nullptr;
    if (int rc = scratch_alloc(size_t(nkc) * size_t(p.outputs) * sizeof(float), &sl)) return rc;
    p.slices = static_cast<float *>(sl);
    int rc = H == 2 ? launch_matmul<2, true>(p, ak, bn, st) : launch_matmul<1, true>(p, ak, bn, st);
    if (!rc) {
        const int64_t fb = std::min<int64_t>((p.outputs + kMmThreads - 1) / kMmThreads, 4096);
        hipLaunchKernelGGL(k_fold, dim3(unsigned(fb)), dim3(kMmThreads), 0, st, p.slices, p.outputs, int(nkc), out);
        rc = launched("k_fold");
    }
    const int rf = scratch_release(sl);
    return rc ? rc : rf;
}

int nt_hip_matmul_half(const float *a, const NtLayout *al, const float *b, const NtLayout *bl, float *out) {
    if (!al || !bl) return fail(NT_E_ARG, "matmul_half: null layout");
    const int r = al->rank;
    if (r < 2 || r > NT_MAX_RANK || bl->rank != r || al->shape[r - 1] != bl->shape[r - 2])
        return fail(NT_E_ARG, "matmul_half: shapes [" + std::to_string(r) + "-d] do not multiply (rank >= 2, equal "
                              "ranks, a's last dimension equal to b's second last)");
    for (int d = 0; d < r; d++)
        if (al->shape[d] < 0 || bl->shape[d] < 0 || al->strides[d] < 0 || bl->strides[d] < 0 || al->offset < 0 ||
            bl->offset < 0)
            return fail(NT_E_ARG, "matmul_half: negative shape, stride or offset");
    MatmulP p{};
    p.nbd = r - 2;
    int64_t nb = 1;
    for (int d = 0; d < r - 2; d++) {
        const int64_t x = al->shape[d], y = bl->shape[d];
        if (x != y && x != 1 && y != 1)
            return fail(NT_E_ARG, "matmul_half: batch dimension " + std::to_string(d) + " does not broadcast (" +
                                      std::to_string(x) + " against " + std::to_string(y) + ")");
        p.bshape[d] = x == 1 ? y : x;
        p.a_bs[d] = x == 1 ? 0 : al->strides[d];
        p.b_bs[d] = y == 1 ? 0 : bl->strides[d];
        nb *= p.bshape[d];
    }
    const int64_t m = al->shape[r - 2], k = al->shape[r - 1], n = bl->shape[r - 1];
    if (m >= (int64_t(1) << 31) - 256 || n >= (int64_t(1) << 31) - 256 || k >= (int64_t(1) << 31) - 256)
        return fail(NT_E_ARG, "matmul_half: m, k and n must each be below 2^31 - 256");
    if (nb == 0 || m == 0 || n == 0) return 0;
    if (!a || !b || !out) return fail(NT_E_ARG, "matmul_half: null buffer");
    p.a = a;
    p.b = b;
    p.c = out;
    p.a_off = al->offset;
    p.b_off = bl->offset;
    p.a_rs = al->strides[r - 2];
    p.a_cs = al->strides[r - 1];
    p.b_rs = bl->strides[r - 2];
    p.b_cs = bl->strides[r - 1];
    p.m = int32_t(m);
    p.n = int32_t(n);
    p.k = int32_t(k);
    // Packed operands and 256 x 256 tiles for a product of many such tiles (see k_half_tiles);
    // NOETIC_HIP_HALF_GEMM=packed|staged picks one path (a tuning knob). The packed path keeps
    // every offset in 32 bits: k <= 65536, at most 65535 batches and 1 GiB of packed operands.
    {
        const int64_t S = (k + 15) / 16, G = (m + 31) / 32, T256 = (n + 255) / 256, TM = (m + 255) / 256;
        const int64_t tiles = nb * TM * T256;
        const int64_t bytes_a = nb * G * S * 1024, bytes_b = nb * T256 * S * 8192;
        const bool fits = k <= 65536 && nb <= 65535 && bytes_a + bytes_b <= (int64_t(1) << 30) && tiles <= 0x7fffffff;
        bool packed = fits && tiles >= kHalfPackedTiles && k >= kHalfPackedK;
        if (const char *e = std::getenv("NOETIC_HIP_HALF_GEMM")) {
            if (std::strcmp(e, "packed") == 0) packed = fits;
            else if (std::strcmp(e, "staged") == 0) packed = false;
        }
        if (packed) {
            p.tm = int32_t(TM);
            p.tn = int32_t(T256);
            std::unique_lock<std::mutex> lk;
            if (int rc = enter(&lk)) return rc;
            hipStream_t st = ctx().stream;
            void *ws = nullptr;
            if (int rc = scratch_alloc(size_t(bytes_a + bytes_b), &ws)) return rc;
            uint8_t *pa = static_cast<uint8_t *>(ws), *pb = pa + bytes_a;
            // both operands in one launch, blocks in proportion to their fragments
            const int64_t ta = G * S * 64, tb = T256 * S * 8 * 64;
            const int64_t ba = std::min<int64_t>((ta + 255) / 256, 4096), bb = std::min<int64_t>((tb + 255) / 256, 4096);
            hipLaunchKernelGGL(k_pack_half, dim3(unsigned(ba + bb), unsigned(nb)), dim3(256), 0, st, p, int(G),
                               int(T256), int(S), int(ba), pa, pb);
            int rc = launched("k_pack_half");
            if (!rc) {
                hipLaunchKernelGGL(k_half_tiles, dim3(unsigned(tiles)), dim3(256), 0, st, p, pa, pb, int(G),
                                   int(T256), int(S));
                rc = launched("k_half_tiles");
            }
            const int rf = scratch_release(ws);
            return rc ? rc : rf;
        }
    }
    // 128x128 tiles when they give at least 512 workgroups, else 64x64
    const int64_t big = nb * ((m + 127) / 128) * ((n + 127) / 128);
    const int T = big >= 512 ? 128 : 64;
    p.tm = int32_t((m + T - 1) / T);
    p.tn = int32_t((n + T - 1) / T);
    p.blocks = nb * p.tm * p.tn;
    if (p.blocks > int64_t(0x7fffffff)) return fail(NT_E_ARG, "matmul_half: too many output tiles");
    const bool ak = k == 1 || p.a_cs == 1;
    const bool bn = n == 1 || p.b_cs == 1;
    // 16-byte staging: the view contiguous along its read axis, the other stride, the offsets of
    // every batch and the base address all multiples of 4 elements / 16 bytes
    auto batch_aligned = [&](const int64_t *bs, int64_t off, const float *base) {
        if (off % 4 != 0 || (reinterpret_cast<uintptr_t>(base) & 15) != 0) return false;
        for (int d = 0; d < r - 2; d++)
            if (bs[d] % 4 != 0) return false;
        return true;
    };
    const bool a_ok = batch_aligned(p.a_bs, p.a_off, a);
    const bool b_ok = batch_aligned(p.b_bs, p.b_off, b);
    p.avec = a_ok && (ak ? (p.a_cs == 1 && p.a_rs % 4 == 0) : (p.a_rs == 1 && p.a_cs % 4 == 0));
    p.bvec = b_ok && (bn ? (p.b_cs == 1 && p.b_rs % 4 == 0) : (p.b_rs == 1 && p.b_cs % 4 == 0));
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    hipStream_t st = ctx().stream;
    const dim3 grid(unsigned(p.blocks)), block(kMmThreads);
    if (T == 128) {
        if (ak && bn) hipLaunchKernelGGL((k_matmul_half<128, true, true>), grid, block, 0, st, p);
        else if (ak) hipLaunchKernelGGL((k_matmul_half<128, true, false>), grid, block, 0, st, p);
        else if (bn) hipLaunchKernelGGL((k_matmul_half<128, false, true>), grid, block, 0, st, p);
        else hipLaunchKernelGGL((k_matmul_half<128, false, false>), grid, block, 0, st, p);
    } else {
        if (ak && bn) hipLaunchKernelGGL((k_matmul_half<64, true, true>), grid, block, 0, st, p);
        else if (ak) hipLaunchKernelGGL((k_matmul_half<64, true, false>), grid, block, 0, st, p);
        else if (bn) hipLaunchKernelGGL((k_matmul_half<64, false, true>), grid, block, 0, st, p);
        else hipLaunchKernelGGL((k_matmul_half<64, false, false>), grid, block, 0, st, p);
    }
    return launched("k_matmul_half");
}

int nt_hip_half_gemm_key(char *buf, size_t cap) {
    if (!buf || cap == 0) return fail(NT_E_ARG, "nt_hip_half_gemm_key: empty buffer");
    std::string sha(NT_KERNELS_SHA);
    const std::string key = "gemm-bf16-mfma32x32x16-f32acc-kernels-" + sha.substr(0, 16);
    if (key.size() + 1 > cap) return fail(NT_E_ARG, "nt_hip_half_gemm_key: buffer too small");
    std::snprintf(buf, cap, "%s", key.c_str());
    return 0;
}

}  // extern "C"
