// The nn::rl samplers' device code for gfx950 (MI355X): the streaming sampler, the
// register-resident sampler (one workgroup per row) and the segmented sampler (a row across
// several workgroups). One source for both ways the library builds them: compiled ahead of time
// into libnoetic_hip.so (rl_sample.hip includes this file), and compiled at run time by hiprtc
// from the text embedded in the library (rtc.cpp), which names each template instance it needs.
// The row layout, arithmetic and determinism rules they share are described in rl_kernels.hip.
#pragma once

#include "nt_rows.hpp"

namespace nt {
namespace {

// ------------------------------------------------------------------ sampler

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
    if constexpr (MK != NT_MASK_NONE) mrow = static_cast<const char *>(p.mask) + mask_row_at(p.mm, row) * MaskWords<MK>::kBytes;

    // ---- phase 1: stream the row once, per-chunk (max, sum exp[, sum exp * d]) into LDS.
    // Aligned 16-bit rows (below 2^31 bytes of mask) load through per-row buffer resources,
    // non-temporal (every input is read once); a group past the row's end reads zeros and is set
    // to -inf (a lane's 8 elements lie wholly inside the row or wholly past it, V % 8 == 0).
    constexpr bool kBuf = AL && DT != NT_F32;
    const int Vb = kBuf ? int(p.V) : 0;
    const __amdgpu_buffer_rsrc_t xres =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(xrow), short(0), Vb * Elem<DT>::kBytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t mres =
        MK != NT_MASK_NONE ? __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(mrow), short(0),
                                                               Vb * MaskWords<MK>::kBytes, kBufferWord3)
                           : xres;
    // An f32 mask on such rows goes through LDS: each wave's batch of chunks has its own slots
    // after the per-chunk records (16-byte aligned; the launch sizes them), filled by the load
    // unit one contiguous KiB per instruction (buffer_load ... lds), where two 16-byte loads per
    // lane 32 bytes apart would each touch every 128-byte line half.
    constexpr bool kMl = kBuf && MK == NT_MASK_F32;
    constexpr int kSB = kMl ? kMaskStage : kBatch;  // chunks per wave with loads in flight together
    constexpr int kMB = kChunk * 4;                 // f32 mask bytes per chunk
    uint8_t *const mstage = reinterpret_cast<uint8_t *>(smem) + ((p.nc * (ENT ? 3 : 2) * 4 + 15) & ~15);
    const uint32_t mslot = uint32_t((uintptr_t)(lds_ptr_t)(mstage)) + uint32_t(wave * kSB * kMB) + uint32_t(lane * 32);
    for (int c0 = wave; c0 < p.nc; c0 += nw * kSB) {
        Raw<DT, MK> raw[kSB];
#pragma unroll
        for (int b = 0; b < kSB; b++) {
            const int c = c0 + b * nw;
            const int64_t e0 = int64_t(c < p.nc ? c : 0) * kChunk + lane * kEpl;
            if constexpr (kBuf) {
                const int eb = c < p.nc ? int(e0) : Vb;
                const auto xa = __builtin_amdgcn_raw_buffer_load_b128(xres, eb * 2, 0, kCachePolicyNT);
                for (int i = 0; i < 4; i++) raw[b].x[i] = xa[i];
                if constexpr (MK == NT_MASK_U8) {
                    const auto k = __builtin_amdgcn_raw_buffer_load_b64(mres, eb, 0, kCachePolicyNT);
                    raw[b].m[0] = k[0];
                    raw[b].m[1] = k[1];
                } else if constexpr (MK == NT_MASK_F32) {
                    // (a chunk past the row reads zeros)
                    const int mb = c < p.nc ? c * kMB : Vb * 4;
                    uint8_t *slot = mstage + (wave * kSB + b) * kMB;
#pragma unroll
                    for (int d = 0; d < 2; d++)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(mres, (lds_ptr_t)(slot + d * 1024), 16,
                                                                 mb + d * 1024 + 16 * lane, 0, 0, kCachePolicyNT);
                } else {
                    raw[b].m[0] = 0;
                }
                if (eb >= Vb) {
                    for (int i = 0; i < 4; i++) raw[b].x[i] = Elem<DT>::kNegInf;
                }
                // (each chunk's three loads stay together, in chunk order, for the waits below)
                if constexpr (kMl) __builtin_amdgcn_sched_barrier(0);
            } else {
                load_raw<DT, MK, AL>(raw[b], xrow, mrow, c < p.nc ? e0 : p.V, p.V);
            }
        }
#pragma unroll
        for (int b = 0; b < kSB; b++) {
            const int c = c0 + b * nw;
            if constexpr (kMl) {
                // chunk b's three loads are done once at most the later chunks' three each are out
                static_for<0, kSB>([&](auto i) {
                    if (b == decltype(i)::value) wait_vmcnt<3 * (kSB - 1 - decltype(i)::value)>();
                });
                lds_mask_words<NT_MASK_F32, kEpl>(mslot + uint32_t(b * kMB), raw[b].m);
            }
            if (c < p.nc) {
            float v[kEpl];
            decode<DT, MK>(raw[b], v, p.tau, tau_one);
            // (cross-lane steps by DPP, no LDS round trips: the sums' order is fixed, rows of 16
            // lanes and then the four rows in order)
            const float cm = wave_max3_dpp(max8_hw(v));
            const float sh = (cm == -INFINITY) ? 0.0f : cm;
            float w[kEpl], h[kEpl];
#pragma unroll
            for (int j = 0; j < kEpl; j++) {
                const float d = (v[j] - sh) * p.c;
                w[j] = exp2_hw(d);
                if constexpr (ENT) h[j] = w[j] * fmaxf(d, -FLT_MAX);
            }
            auto rows4 = [](float x) {
                const float r = row_sum_dpp(x);
                return ((readlane_f(r, 0) + readlane_f(r, 16)) + readlane_f(r, 32)) + readlane_f(r, 48);
            };
            const float cs = rows4(tree8(w));
            float ce = 0.0f;
            if constexpr (ENT) ce = rows4(tree8(h));
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
    // (nothing allowed, or every allowed logit below -FLT_MAX T, whose tempered value is -inf)
    if (a == -INFINITY || (MK != NT_MASK_F32 && p.tau_one == 0 && a / p.tau == -INFINITY)) {
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

template <int DT, int MK, int K, bool ENT, int EPL, int WN = kRRWindow>
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
        mrow = static_cast<const uint8_t *>(p.mask) + mask_row_at(p.mm, row) * MaskWords<MK>::kBytes;
    const uint32_t mbase = uint32_t((uintptr_t)(lds_ptr_t)(mlds));
    // The row's uniform, read now so that its latency hides under the row's loads.
    const double u_row = p.greedy ? 0.0 : p.u[row];

    // ---- loads: the first W chunks now, chunk k + W while chunk k is consumed.
    constexpr int W = K < WN ? K : WN;
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
    // (nothing allowed, or every allowed logit below -FLT_MAX T, whose tempered value is -inf)
    if (M == -INFINITY || (MK != NT_MASK_F32 && M <= p.m_ovf)) {
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
    // inside the lane, compared against the f64 target): every comparison at once, then the
    // first that passes.
    int jsel;
    {
        const double t0 = tloc - (cincl - ls);
        float C[EPL];
        C[0] = w[0];
#pragma unroll
        for (int j = 1; j < EPL; j++) C[j] = C[j - 1] + w[j];
        uint32_t crossed = 0;
#pragma unroll
        for (int j = 0; j < EPL; j++) crossed |= uint32_t(double(C[j]) > t0) << j;
        jsel = (!none && crossed != 0u) ? __builtin_ctz(crossed) : jlast;
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

// ------------------------------------------------------------------ queued sampler (u8 keep-masks)
//
// With a u8 keep-mask an excluded token's value is -inf whatever its logit (NaN and +inf
// included), so its logit never needs to be read or weighed. This kernel is the
// register-resident sampler reorganised around that: one 1024-thread workgroup per row, each
// wave owning K consecutive chunks of 512 elements, taken in NS stages of KS = K / NS chunks.
//  - The mask comes first: the wave's mask bytes of stage s + 1 stream into LDS (1 KiB per
//    instruction) while stage s is queued.
//  - Queue: a lane group is 8 consecutive elements (one 16-byte bf16 load, two f32 ones). The
//    groups of a stage's chunks that keep a token are listed in index order in LDS (a ballot and
//    a lane count per chunk).
//  - Slot j of stage s holds the stage's queue entries [64 j, 64 j + 64), one per lane; its
//    logits are loaded straight from HBM into the slot's registers. Lanes past the queue's end,
//    and slots past it, load through an out-of-range buffer offset: no memory is read and they
//    weigh nothing. A row whose kept tokens lie in runs reads only the 128-byte lines that hold
//    one.
//  - Slots are weighed as the register-resident sampler weighs chunks (the same exponent
//    reference rule, the same four 16-lane partials per slot), one stage behind the loads.
// A wave whose first stage keeps a token in more than kRqDense of its lane groups reads the
// rest of its chunks as the register-resident sampler does instead (dense path): every lane
// group loaded in place with its chunk's mask, one chunk ahead of the one being weighed, so a
// dense mask pays only the first stage's wait for its mask bytes. Each wave keeps, per slot and
// lane, the LDS address of its group's mask bytes (a zero word for an empty lane), from which the
// group's element index and its mask are read again when the draw lands in it.
// Phases 2 and 3 are the register-resident sampler's with slots in place of chunks: within a
// wave the slots are in index order (queue entries, or chunks), so the waves' slots in order
// run through the row's kept elements in order. Every load and wait on either path is in a fixed
// order whatever the mask (empty slots load nothing but still issue), so each wait count is a
// compile-time constant.

// The share of a first stage's lane groups with a kept token above which a wave takes the dense
// path.
constexpr int kRqDensePct = 70;

// SH: the launch's mask rows are each read by several logits rows (a stride 0 over a dimension
// longer than one, mask_shared): they are loaded through the caches, where the other rows find
// them; otherwise each row's mask is read once, non-temporal.
template <int DT, int K, bool ENT, int NS, bool SH>
__global__ __launch_bounds__(kRRThreads) void k_sample_rq(SampleP p) {
    constexpr int MK = NT_MASK_U8;
    constexpr int EPL = 8;
    constexpr int CH = kWave * EPL;                // elements (and mask bytes) per chunk
    constexpr int NCH = K * kRRWaves;
    constexpr int KS = K / NS;                     // chunks per stage = slots per stage
    static_assert(K % NS == 0 && KS % 4 == 0, "stages of a multiple of 4 chunks");
    constexpr int MD = KS * CH / 1024;             // 1 KiB mask DMAs per stage
    constexpr int LX = RRX<DT, EPL>::kPieces;      // 16-byte logit loads per lane group
    __shared__ __attribute__((aligned(16))) uint8_t mlds[NCH * CH];            // the row's mask bytes
    __shared__ __attribute__((aligned(16))) uint16_t qpos[kRRWaves * KS * kWave];  // per wave: a stage's queue
    __shared__ __attribute__((aligned(16))) float csum4[NCH * 4];  // per slot and 16-lane row: sum of 2^(v c - wref)
    __shared__ __attribute__((aligned(16))) float cent4[ENT ? NCH * 4 : 4];  // per slot and row: sum of w (v c - wref)
    __shared__ float wref[kRRWaves];
    __shared__ float wmax[kRRWaves];
    __shared__ double wtot[kRRWaves];
    __shared__ double went[ENT ? kRRWaves : 1];
    __shared__ int wpick[kRRWaves];
    __shared__ __attribute__((aligned(8))) uint32_t zmask[2];  // the mask words of an empty lane

    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const float c = p.c;
    const bool tau_one = p.tau_one != 0;
    const void *xrow = static_cast<const char *>(p.logits) + row * p.ld * Elem<DT>::kBytes;
    const uint8_t *mrow = static_cast<const uint8_t *>(p.mask) + mask_row_at(p.mm, row);
    const uint32_t mbase = uint32_t((uintptr_t)(lds_ptr_t)(mlds));
    const uint32_t zaddr = uint32_t((uintptr_t)(lds_ptr_t)(zmask));
    const double u_row = p.greedy ? 0.0 : p.u[row];
    const int Vi = int(p.V);
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(xrow), short(0), int(p.V * Elem<DT>::kBytes), kBufferWord3);
    const __amdgpu_buffer_rsrc_t mres =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(mrow), short(0), Vi, kBufferWord3);
    // Offsets past every row: such a load reads nothing and returns zeros. Each slot has its
    // own, so that no two of a wave's loads are ever the same load (the compiler would merge
    // those, and the waits below count loads).
    constexpr int kNoRead = 0x40000000;
    // Every wave zeroes the empty lane's words itself (the same bits), so its own reads of
    // them follow its own store.
    if (lane < 2) zmask[lane] = 0u;
    constexpr int kMaskPolicy = SH ? 0 : kCachePolicyNT;

    RRX<DT, EPL> raw[K];  // slot k's logit words
    uint32_t ma[K];       // slot k: the LDS address of this lane's group's mask bytes (zmask: none)
    uint16_t *const q = qpos + wave * KS * kWave;

    // The wave's mask bytes of stage s into mlds (the row's bytes at their own offsets), with
    // non-temporal loads: at C4 (256 rows of V = 128256 bf16, a runs mask, tau 0.7, each process
    // timing one policy) 16.8 -> 15.7 us per launch HBM-cold and 15.4 -> 14.5 us re-reading one
    // input; non-temporal logit loads as well measured 15.6 and 15.1 us.
    auto issue_mask = [&](auto sc) {
        constexpr int s = decltype(sc)::value;
        const int b0 = (wave * K + s * KS) * CH;
        static_for<0, MD>([&](auto dc) {
            constexpr int d = decltype(dc)::value;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(mres, (lds_ptr_t)(mlds + b0 + d * 1024), 16,
                                                     b0 + d * 1024 + 16 * lane, 0, 0, kMaskPolicy);
        });
        __builtin_amdgcn_sched_barrier(0);
    };
    // Queue stage s's lane groups that keep a token, in index order; returns the count (uniform).
    auto build = [&](auto sc) -> int {
        constexpr int s = decltype(sc)::value;
        const int e00 = (wave * K + s * KS) * CH + lane * EPL;  // this lane's group in the stage's first chunk
        int cnt = 0;
        static_for<0, KS / 4>([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            uint2 m[4];
            lds_read4_b64<(4 * g) * CH, (4 * g + 1) * CH, (4 * g + 2) * CH, (4 * g + 3) * CH>(
                mbase + e00, m[0], m[1], m[2], m[3]);
            static_for<0, 4>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                constexpr int cl = 4 * g + i;
                const bool act = ((m[i].x | m[i].y) != 0u) && e00 + cl * CH < Vi;
                const uint64_t bal = __ballot(act);
                if (act)
                    q[cnt + int(__builtin_amdgcn_mbcnt_hi(uint32_t(bal >> 32),
                                                          __builtin_amdgcn_mbcnt_lo(uint32_t(bal), 0u)))] =
                        uint16_t(cl * kWave + lane);
                cnt += __builtin_popcountll(bal);
            });
        });
        return cnt;
    };
    // Stage s's slot loads: lane l of slot j takes queue entry 64 j + l.
    auto issue_queued = [&](auto sc, int cnt) {
        constexpr int s = decltype(sc)::value;
        const int sb = (wave * K + s * KS) * CH;
        static_for<0, KS>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            const int idx = j * kWave + lane;
            const bool valid = idx < cnt;
            const int e0 = sb + int(q[valid ? idx : 0]) * EPL;
            ma[s * KS + j] = valid ? mbase + uint32_t(e0) : zaddr;
            const int xo = valid ? e0 * Elem<DT>::kBytes : kNoRead + 4096 * (s * KS + j);
#pragma unroll
            for (int pc = 0; pc < LX; pc++) {
                const auto a = __builtin_amdgcn_raw_buffer_load_b128(xres, xo + 16 * pc, 0, 0);
                raw[s * KS + j].x[4 * pc] = a[0];
                raw[s * KS + j].x[4 * pc + 1] = a[1];
                raw[s * KS + j].x[4 * pc + 2] = a[2];
                raw[s * KS + j].x[4 * pc + 3] = a[3];
            }
        });
        __builtin_amdgcn_sched_barrier(0);
    };

    // ---- phase 1, weighing: as the register-resident sampler's, per slot.
    float *const cpart = csum4 + 4 * K * wave + lane / 16;
    float *const epart = ENT ? cent4 + 4 * K * wave + lane / 16 : nullptr;
    const bool row_leader = (lane & 15) == 0;
    bool have_ref = false;
    float lmax = -INFINITY;
    float sref = -INFINITY;
    float sref_v = -INFINITY;
    // Weigh slot k; its mask words are read here (the caller has waited for its loads, which
    // follow its mask bytes).
    auto weigh_slot = [&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const uint2 m2 = lds_read_b64(ma[k]);
        const uint32_t mw[2] = {m2.x, m2.y};
        float v[EPL];
        decode_e<DT, MK, EPL>(raw[k].x, mw, v, p.tau, tau_one);
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
            for (int jj = 0; jj < EPL; jj++) {
                const float d = fmaf(v[jj], c, -sref);
                w[jj] = exp2_hw(d);
                if constexpr (ENT) h[jj] = w[jj] * fmaxf(d, -FLT_MAX);
            }
            gs = tree_sum<EPL>(w);
            if constexpr (ENT) gh = tree_sum<EPL>(h);
        };
        if (have_ref) {
            weigh();
            bool move = !(gs < INFINITY);
            if constexpr (ENT) move = !(gs <= kChunkSumCap);
            if (__ballot(move) != 0) {
                const float wm = wave_max3_dpp(max_hw<EPL>(v));
                const float nref = wm * c;
                if (nref > sref) {
                    const float dk = sref - nref, f = exp2_hw(dk);
                    if ((lane & 15) == 0) {
                        static_for<0, k>([&](auto kc2) {
                            constexpr int kk = decltype(kc2)::value;
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
        const float cs = row_sum_dpp(gs);
        float ce = 0.0f;
        if constexpr (ENT) ce = row_sum_dpp(gh);
        if (row_leader) {
            cpart[4 * k] = cs;
            if constexpr (ENT) epart[4 * k] = ce;
        }
    };
    // An empty slot weighs nothing (its partials are read with the others').
    auto empty_slot = [&](auto kc) {
        constexpr int k = decltype(kc)::value;
        ma[k] = zaddr;
        if (row_leader) {
            cpart[4 * k] = 0.0f;
            if constexpr (ENT) epart[4 * k] = 0.0f;
        }
    };
    // Weigh stage s's slots that hold entries; `after` is the number of loads issued after the
    // stage's last one.
    auto weigh_stage = [&](auto sc, auto afterc, int cnt) {
        constexpr int s = decltype(sc)::value;
        constexpr int after = decltype(afterc)::value;
        const int nb = (cnt + kWave - 1) / kWave;
        static_for<0, KS>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            if (j < nb) {
                wait_vmcnt<after + (KS - 1 - j) * LX>();
                weigh_slot(std::integral_constant<int, s * KS + j>{});
            } else {
                empty_slot(std::integral_constant<int, s * KS + j>{});
            }
        });
    };

    // ---- the first stage's mask, then the path.
    issue_mask(std::integral_constant<int, 0>{});
    wait_vmcnt<0>();
    const int cnt0 = build(std::integral_constant<int, 0>{});
    if (cnt0 * 100 > kRqDensePct * KS * kWave) {
        // Dense path: chunk k's logits in place (and, past the first stage, its mask bytes,
        // 4 per lane, as the register-resident sampler brings them), chunk k + 1 issued before
        // chunk k is weighed.
        constexpr int DMB = CH / (4 * kWave);  // mask DMAs per chunk past the first stage
        auto issue_dense = [&](auto kc) {
            constexpr int k = decltype(kc)::value;
            const int ch = wave * K + k;
            const int e0 = ch * CH + lane * EPL;
            const bool in = e0 < Vi;
            ma[k] = in ? mbase + uint32_t(e0) : zaddr;
            const int xo = in ? e0 * Elem<DT>::kBytes : kNoRead + 4096 * k;
#pragma unroll
            for (int pc = 0; pc < LX; pc++) {
                const auto a = __builtin_amdgcn_raw_buffer_load_b128(xres, xo + 16 * pc, 0, 0);
                raw[k].x[4 * pc] = a[0];
                raw[k].x[4 * pc + 1] = a[1];
                raw[k].x[4 * pc + 2] = a[2];
                raw[k].x[4 * pc + 3] = a[3];
            }
            if constexpr (k >= KS) {
                static_for<0, DMB>([&](auto dc) {
                    constexpr int d = decltype(dc)::value;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(mres, (lds_ptr_t)(mlds + ch * CH + d * 4 * kWave), 4,
                                                             ch * CH + d * 4 * kWave + 4 * lane, 0, 0, kMaskPolicy);
                });
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        issue_dense(std::integral_constant<int, 0>{});
        static_for<0, K>([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            if constexpr (k + 1 < K) {
                issue_dense(std::integral_constant<int, k + 1>{});
                wait_vmcnt<LX + (k + 1 >= KS ? DMB : 0)>();
            } else {
                wait_vmcnt<0>();
            }
            weigh_slot(kc);
        });
    } else {
        // Queued path: M_0 | queue 0, M_1, L_0 | wait M_s, queue s, M_{s+1}, L_s, weigh s - 1 |
        // weigh the last stage. After M_s only L_{s-1} is issued, so its wait leaves KS LX loads
        // in flight.
        int cnt[NS];
        cnt[0] = cnt0;
        static_for<0, NS>([&](auto sc) {
            constexpr int s = decltype(sc)::value;
            if constexpr (s > 0) {
                wait_vmcnt<KS * LX>();
                cnt[s] = build(sc);
            }
            if constexpr (s + 1 < NS) issue_mask(std::integral_constant<int, s + 1>{});
            issue_queued(sc, cnt[s]);
            if constexpr (s >= 1)
                weigh_stage(std::integral_constant<int, s - 1>{},
                            std::integral_constant<int, KS * LX + (s + 1 < NS ? MD : 0)>{}, cnt[s - 1]);
        });
        weigh_stage(std::integral_constant<int, NS - 1>{}, std::integral_constant<int, 0>{}, cnt[NS - 1]);
    }

    // ---- end of phase 1: lane k < K takes slot k's sum in f64; the f64 prefix over the wave's
    // slots stays in registers and the wave's totals go to LDS.
    double wcs = 0.0, wce = 0.0;
    if (lane < K) {
        const float4 qs = *reinterpret_cast<const float4 *>(csum4 + 4 * (wave * K + lane));
        wcs = double((qs.x + qs.y) + (qs.z + qs.w));
        if constexpr (ENT) {
            const float4 e = *reinterpret_cast<const float4 *>(cent4 + 4 * (wave * K + lane));
            wce = double((e.x + e.y) + (e.z + e.w));
        }
    }
    const double wincl = row_scan_dpp(wcs);
    {
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

    // ---- phase 2: the register-resident sampler's.
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
    // (nothing allowed, or every allowed logit below -FLT_MAX T, whose tempered value is -inf)
    if (M == -INFINITY || (MK != NT_MASK_F32 && M <= p.m_ovf)) {
        refuse(NT_ROW_NO_TOKEN, tid == 0);
        return;
    }
    const float A = M * c;
    const bool wlive = rw != -INFINITY;
    const float wf = wlive ? exp2_hw(rw - A) : 0.0f;
    const double wt = wlive ? double(wf) * tw : 0.0;
    const double incl = row_scan_dpp(wt);
    const double S = readlane_d(incl, kRRWaves - 1);
    if (!(S == S)) {
        refuse(NT_ROW_NAN, tid == 0);
        return;
    }
    auto entropy_sum = [&]() -> double {
        if constexpr (!ENT) return 0.0;
        const double lh = (wlive && tw > 0.0) ? double(wf) * (hw + double(rw - A) * tw) : 0.0;
        return readlane_d(row_scan_dpp(lh), kRRWaves - 1);
    };
    auto write_row = [&](int64_t id, float vz, double H) {
        const double shiftA = double(A) - double(M) * double(c);
        const double lnS = ln_fast(S) + shiftA * kLn2;
        const float zid = tau_one ? vz : vz / p.tau;
        const float mz = tau_one ? M : M / p.tau;
        p.ids[row] = int32_t(id);
        if (p.logp) p.logp[row] = float((double(zid) - double(mz)) - lnS);
        if (p.ent) p.ent[row] = float(lnS - kLn2 * (H / S + shiftA));
        p.status[row] = NT_ROW_OK;
    };
    // A weighed slot's values, its mask read again (an empty lane reads the zero words: -inf).
    auto slot_values = [&](const RRX<DT, EPL> &r, uint32_t a, float *v) {
        const uint2 m2 = lds_read_b64(a);
        const uint32_t mw[2] = {m2.x, m2.y};
        decode_e<DT, MK, EPL>(r.x, mw, v, p.tau, tau_one);
    };

    if (p.greedy) {
        int first = 0x7fffffff;
        static_for<0, K>([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            if (ma[k] != zaddr) {
                float v[EPL];
                slot_values(raw[k], ma[k], v);
#pragma unroll
                for (int j = EPL - 1; j >= 0; j--)
                    if (v[j] == M) first = min(first, int(ma[k] - mbase) + j);
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

    const double t = u_row * S;
    const bool wl = lane < kRRWaves;
    int wsel = first_lane(__ballot(wl && incl > t && wt > 0.0));
    if (wsel < 0) wsel = last_lane(__ballot(wl && wt > 0.0));
    if (wsel < 0) {
        refuse(NT_ROW_NAN, tid == 0);
        return;
    }
    if (wave != wsel) return;
    // ---- phase 3 (that wave alone): the crossing slot from the prefix, then its registers.
    const double tl = readlane_d((t - (incl - wt)) * double(exp2_hw(A - rw)), wsel);
    const bool lk = lane < K;
    int kstar = first_lane(__ballot(lk && wincl > tl && wcs > 0.0));
    if (kstar < 0) kstar = last_lane(__ballot(lk && wcs > 0.0));
    if (kstar < 0) {
        refuse(NT_ROW_NAN, lane == 0);
        return;
    }
    const double tloc = readlane_d(tl - (wincl - wcs), kstar);
    const double H = entropy_sum();
    RRX<DT, EPL> r = raw[0];
    uint32_t ar = ma[0];
    static_for<1, K>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        if (k == kstar) {
            r = raw[k];
            ar = ma[k];
        }
    });
    float v[EPL];
    slot_values(r, ar, v);
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
    if (none) lsel = last_lane(__ballot(jlast >= 0));
    if (lsel < 0) {
        refuse(NT_ROW_NAN, lane == 0);
        return;
    }
    int jsel;  // (the register-resident sampler's walk)
    {
        const double t0 = tloc - (cincl - ls);
        float C[EPL];
        C[0] = w[0];
#pragma unroll
        for (int j = 1; j < EPL; j++) C[j] = C[j - 1] + w[j];
        uint32_t crossed = 0;
#pragma unroll
        for (int j = 0; j < EPL; j++) crossed |= uint32_t(double(C[j]) > t0) << j;
        jsel = (!none && crossed != 0u) ? __builtin_ctz(crossed) : jlast;
    }
    if (lane == lsel) {
        if (jsel < 0) jsel = 0;
        float vz = v[0];
#pragma unroll
        for (int j = 1; j < EPL; j++)
            if (j == jsel) vz = v[j];
        write_row(int64_t(ar - mbase) + jsel, vz, H);
    }
}

// ------------------------------------------------------------------ segmented sampler
//
// Rows too few to fill the chip (C2's 64 rows on 256 CUs), and rows whose tail should overlap
// other rows' streaming, are cut into G segments of NW K chunks, one workgroup each, so that a
// row's bytes stream through G compute units. Each wave of a segment runs phase 1 of the
// register-resident sampler on its K chunks, then publishes a wave record in device scratch:
// its exponent reference, its maximum (or the value its reference came from), the first index of
// its maximum (greedy), its f64 totals and its K f32 chunk sums, with agent-scope atomic stores
// (coherent across the XCDs' L2s). The workgroup waits until those stores have completed, then
// increments the row's arrival counter with one agent-scope vector atomic; the last arriver reads
// the records with agent-scope atomic loads. No workgroup waits for another: every one but the
// last to arrive exits;
// the last one's first wave merges the G NW wave records of the row in index order (phase 2 over
// up to 64 records, one per lane), finds the crossing wave and chunk from the records, reads the
// crossing chunk again (512 elements, about 1.5 KB, from the caches in practice) and resolves
// the draw as the register-resident sampler's phase 3 does. It resets the counter for the next
// launch. Which workgroup arrives last changes from run to run, but the merge reads the same
// records in the same order, so the result bits do not.

// The record a wave publishes: 32 bytes, then its K chunk sums (f32).
struct SegRec {
    float ref;     // RN(s c): the wave's exponent reference (-inf: no allowed value)
    float vmax;    // greedy: the wave's exact maximum; else the value its reference came from
    int first;     // greedy: the first index of vmax in the wave's chunks (INT_MAX: none)
    int pad;
    double total;  // sum of the wave's weights 2^(v c - ref)
    double ent;    // sum of w (v c - ref) (entropy numerator)
};
static_assert(sizeof(SegRec) == 32, "wave record header");

struct SegP {
    SampleP s;
    int G;              // segments per row
    int nwr;            // wave records per row (G NW, at most 64)
    int rec_bytes;      // 32 + 4 K
    uint8_t *recs;      // [rows][nwr] records
    uint32_t *count;    // [rows] arrival counters: zero between launches
};

constexpr int kSegMaxRecords = 64;

template <int DT, int MK, int K, bool ENT, int NW, int WN = kRRWindow>
__global__ __launch_bounds__(NW * kWave) void k_sample_seg(SegP q) {
    constexpr int EPL = 8;
    constexpr int CH = kWave * EPL;                // elements per chunk
    constexpr int NCH = K * NW;                    // chunks per segment
    constexpr int LX = RRX<DT, EPL>::kPieces;
    constexpr int LD = RRMask<MK, EPL>::kDma;
    constexpr int MB = RRMask<MK, EPL>::kBytes;
    constexpr int DB = RRMask<MK, EPL>::kDmaBytes;
    constexpr int L = LX + LD;
    const SampleP &p = q.s;
    __shared__ __attribute__((aligned(16))) uint8_t mlds[MK == NT_MASK_NONE ? 16 : NCH * MB];
    __shared__ __attribute__((aligned(16))) float csum4[NCH * 4];
    __shared__ __attribute__((aligned(16))) float cent4[ENT ? NCH * 4 : 4];
    __shared__ int s_last;

    const int G = q.G;
    const int64_t row = blockIdx.x / G;
    const int seg = blockIdx.x - int(row) * G;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int wg = seg * NW + wave;  // the wave's index in the row: chunks wg K .. wg K + K - 1
    const int nc = p.nc;
    const float c = p.c;
    const bool tau_one = p.tau_one != 0;
    const void *xrow = static_cast<const char *>(p.logits) + row * p.ld * Elem<DT>::kBytes;
    const uint8_t *mrow = nullptr;
    if constexpr (MK != NT_MASK_NONE)
        mrow = static_cast<const uint8_t *>(p.mask) + mask_row_at(p.mm, row) * MaskWords<MK>::kBytes;
    const uint32_t mbase = uint32_t((uintptr_t)(lds_ptr_t)(mlds));
    // The row's uniform, read now (every segment reads it; the one that resolves uses it).
    const double u_row = p.greedy ? 0.0 : p.u[row];

    constexpr int W = K < WN ? K : WN;
    RRX<DT, EPL> raw[K];
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(xrow), short(0), int(p.V * Elem<DT>::kBytes), kBufferWord3);
    __amdgpu_buffer_rsrc_t mres;
    if constexpr (MK != NT_MASK_NONE)
        mres = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(mrow), short(0),
                                                 int(p.V * MaskWords<MK>::kBytes), kBufferWord3);
    auto issue = [&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const int ch = wg * K + k;       // chunk of the row
        const int lc = wave * K + k;     // its slot in this workgroup
        const int xo = (ch * CH + lane * EPL) * Elem<DT>::kBytes;
#pragma unroll
        for (int qq = 0; qq < LX; qq++) {
            const auto a = __builtin_amdgcn_raw_buffer_load_b128(xres, xo + 16 * qq, 0, 0);
            raw[k].x[4 * qq] = a[0];
            raw[k].x[4 * qq + 1] = a[1];
            raw[k].x[4 * qq + 2] = a[2];
            raw[k].x[4 * qq + 3] = a[3];
        }
        if constexpr (MK != NT_MASK_NONE) {
#pragma unroll
            for (int d = 0; d < LD; d++) {
                if constexpr (DB == 16)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(mres, (lds_ptr_t)(mlds + lc * MB + d * DB * kWave), 16,
                                                             ch * MB + d * DB * kWave + DB * lane, 0, 0, 0);
                else
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(mres, (lds_ptr_t)(mlds + lc * MB + d * DB * kWave), 4,
                                                             ch * MB + d * DB * kWave + DB * lane, 0, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    static_for<0, W>(issue);

    // ---- phase 1: the register-resident sampler's, on this wave's K chunks.
    float *const cpart = csum4 + 4 * K * wave + lane / 16;
    float *const epart = ENT ? cent4 + 4 * K * wave + lane / 16 : nullptr;
    const bool row_leader = (lane & 15) == 0;
    const int Vi = int(p.V);
    const uint32_t mlw = mbase + wave * K * MB + lane * EPL * MaskWords<MK>::kBytes;
    bool have_ref = false;
    float lmax = -INFINITY;
    float sref = -INFINITY;
    float sref_v = -INFINITY;
    static_for<0, K>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const int ch = wg * K + k;
        if (ch < nc) {
            const int64_t e0 = int64_t(ch) * CH + lane * EPL;
            uint32_t mw[RRMask<MK, EPL>::kWords];
            if constexpr (MK != NT_MASK_NONE) {
                wait_vmcnt<L * ((K < k + W ? K : k + W) - 1 - k)>();
                constexpr int kOff = k * MB;
                if constexpr (MK == NT_MASK_U8 && kOff < 65536) {
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
            if ((ch + 1) * CH > Vi) {
#pragma unroll
                for (int j = 0; j < EPL; j++)
                    if (e0 + j >= p.V) v[j] = -INFINITY;
            }
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
                bool move = !(gs < INFINITY);
                if constexpr (ENT) move = !(gs <= kChunkSumCap);
                if (__ballot(move) != 0) {
                    const float wm = wave_max3_dpp(max_hw<EPL>(v));
                    const float nref = wm * c;
                    if (nref > sref) {
                        const float dk = sref - nref, f = exp2_hw(dk);
                        if ((lane & 15) == 0) {
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
            const float cs = row_sum_dpp(gs);
            float ce = 0.0f;
            if constexpr (ENT) ce = row_sum_dpp(gh);
            if (row_leader) {
                cpart[4 * k] = cs;
                if constexpr (ENT) epart[4 * k] = ce;
            }
        }
        if constexpr (k + W < K) {
            if (!(ch < nc)) issue(std::integral_constant<int, k + W>{});
        }
    });

    // ---- the wave's record: chunk sums (lane k < K, the four partials in a fixed order), the f64
    // totals by the same 16-lane scan the register-resident sampler takes, the reference and,
    // when greedy, the first index of the wave's maximum.
    SegRec *rec = reinterpret_cast<SegRec *>(q.recs + (row * q.nwr + wg) * int64_t(q.rec_bytes));
    float *rec_cs = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(rec) + sizeof(SegRec));
    float cs32 = 0.0f;
    double wce = 0.0;
    {
        const int ch = wg * K + lane;
        if (lane < K && ch < nc) {
            const float4 qs = *reinterpret_cast<const float4 *>(csum4 + 4 * (wave * K + lane));
            cs32 = (qs.x + qs.y) + (qs.z + qs.w);
            if constexpr (ENT) {
                const float4 e = *reinterpret_cast<const float4 *>(cent4 + 4 * (wave * K + lane));
                wce = double((e.x + e.y) + (e.z + e.w));
            }
        }
    }
    const double wincl = row_scan_dpp(double(cs32));
    double wh = 0.0;
    if constexpr (ENT) wh = row_scan_dpp(wce);
    float wm = sref_v;
    int wfirst = 0x7fffffff;
    if (p.greedy) {
        wm = wave_max3_dpp(lmax);
        int first = 0x7fffffff;
        static_for<0, K>([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            const int ch = wg * K + k;
            if (ch < nc) {
                uint32_t mw[RRMask<MK, EPL>::kWords];
                lds_mask_words<MK, EPL>(mbase + (wave * K + k) * MB + lane * EPL * MaskWords<MK>::kBytes, mw);
                float v[EPL];
                decode_e<DT, MK, EPL>(raw[k].x, mw, v, p.tau, tau_one);
#pragma unroll
                for (int j = EPL - 1; j >= 0; j--) {
                    const int64_t e = int64_t(ch) * CH + lane * EPL + j;
                    if (e < p.V && v[j] == wm) first = min(first, int(e));
                }
            }
        });
        wfirst = wave_min_i(first);
    }
    // Records are shared across compute units (and the L2s of different XCDs) through
    // agent-scope atomic stores and loads: the accesses are coherent at the device's point of
    // coherence (no whole-cache write-back or invalidate, which measured about 0.12 us per
    // workgroup, serialised), and the only ordering needed is that a segment's record stores are
    // complete before its arrival is counted, an explicit wait for the vector memory counter.
    auto st_f = [](float *a, float v) { __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto st_i = [](int *a, int v) { __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto st_d = [](double *a, double v) { __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    if (lane < K) st_f(rec_cs + lane, cs32);
    if (lane == kRRWaves - 1) {
        st_d(&rec->total, wincl);
        st_d(&rec->ent, wh);
    }
    if (lane == 0) {
        st_f(&rec->ref, sref);
        st_f(&rec->vmax, wm);
        st_i(&rec->first, wfirst);
    }
    wait_vmcnt<0>();
    __syncthreads();
    if (G > 1) {
        if (tid == 0) {
            const uint32_t old = __hip_atomic_fetch_add(q.count + row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = old == uint32_t(G - 1);
        }
        __syncthreads();
        if (!s_last) return;
    }
    if (wave != 0) return;
    // The last segment of the row: ready the counter for the next launch (the kernel's end
    // orders it before that launch).
    if (G > 1 && lane == 0) __hip_atomic_store(q.count + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // ---- phase 2 (one wave): lane l < nwr takes wave record l of the row, in index order, and
    // its K chunk sums, all in one round of loads.
    auto ld_f = [](const float *a) { return __hip_atomic_load(const_cast<float *>(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto ld_i = [](const int *a) { return __hip_atomic_load(const_cast<int *>(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto ld_d = [](const double *a) { return __hip_atomic_load(const_cast<double *>(a), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    const bool lv = lane < q.nwr;
    const SegRec *rl = reinterpret_cast<const SegRec *>(q.recs + (row * q.nwr + (lv ? lane : 0)) * int64_t(q.rec_bytes));
    const float *rl_cs = reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(rl) + sizeof(SegRec));
    float rw = -INFINITY, vm = -INFINITY;
    double tw = 0.0, hw = 0.0;
    int fi = 0x7fffffff;
    float lcs[K];
    if (lv) {
        rw = ld_f(&rl->ref);
        vm = ld_f(&rl->vmax);
        tw = ld_d(&rl->total);
        if constexpr (ENT) hw = ld_d(&rl->ent);
        if (p.greedy) fi = ld_i(&rl->first);
#pragma unroll
        for (int k = 0; k < K; k++) lcs[k] = ld_f(rl_cs + k);
    } else {
#pragma unroll
        for (int k = 0; k < K; k++) lcs[k] = 0.0f;
    }
    const float M = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(wave_max3_dpp(vm))));
    auto refuse = [&](uint8_t st) {
        if (lane == 0) {
            p.ids[row] = -1;
            if (p.logp) p.logp[row] = NAN;
            if (p.ent) p.ent[row] = NAN;
            p.status[row] = st;
        }
    };
    // (nothing allowed, or every allowed logit below -FLT_MAX T, whose tempered value is -inf)
    if (M == -INFINITY || (MK != NT_MASK_F32 && M <= p.m_ovf)) {
        refuse(NT_ROW_NO_TOKEN);
        return;
    }
    const float A = M * c;
    const bool wlive = rw != -INFINITY;
    const float wf = wlive ? exp2_hw(rw - A) : 0.0f;
    const double wt = wlive ? double(wf) * tw : 0.0;
    const double incl = wave_scan_dpp(wt);
    const double S = readlane_d(incl, kWave - 1);
    if (!(S == S)) {
        refuse(NT_ROW_NAN);
        return;
    }
    double H = 0.0;
    if constexpr (ENT) {
        const double lh = (wlive && tw > 0.0) ? double(wf) * (hw + double(rw - A) * tw) : 0.0;
        H = readlane_d(wave_scan_dpp(lh), kWave - 1);
    }
    auto write_row = [&](int64_t id, float vz) {
        const double shiftA = double(A) - double(M) * double(c);
        const double lnS = ln_fast(S) + shiftA * kLn2;
        const bool zv = MK == NT_MASK_F32 || tau_one;
        const float zid = zv ? vz : vz / p.tau;
        const float mz = zv ? M : M / p.tau;
        p.ids[row] = int32_t(id);
        if (p.logp) p.logp[row] = float((double(zid) - double(mz)) - lnS);
        if (p.ent) p.ent[row] = float(lnS - kLn2 * (H / S + shiftA));
        p.status[row] = NT_ROW_OK;
    };
    if (p.greedy) {
        const int best = wave_min_i(lv && vm == M ? fi : 0x7fffffff);
        if (lane == 0) write_row(best, M);
        return;
    }
    const double t = u_row * S;
    int wsel = first_lane(__ballot(lv && incl > t && wt > 0.0));
    if (wsel < 0) wsel = last_lane(__ballot(lv && wt > 0.0));
    if (wsel < 0) {
        refuse(NT_ROW_NAN);
        return;
    }
    const float sr = readlane_f(rw, wsel);
    const double tl = readlane_d((t - (incl - wt)) * double(exp2_hw(A - rw)), wsel);
    // ---- phase 3: the crossing chunk from the crossing wave's chunk sums (lane k takes chunk k's,
    // from the crossing lane's registers), then its elements.
    float mycs = 0.0f;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const float ck = readlane_f(lcs[k], wsel);
        if (lane == k) mycs = ck;
    }
    const bool lk = lane < K;
    const double wcs = lk ? double(mycs) : 0.0;
    const double cincl_w = row_scan_dpp(wcs);
    int kstar = first_lane(__ballot(lk && cincl_w > tl && wcs > 0.0));
    if (kstar < 0) kstar = last_lane(__ballot(lk && wcs > 0.0));
    if (kstar < 0) {
        refuse(NT_ROW_NAN);
        return;
    }
    const double tloc = readlane_d(tl - (cincl_w - wcs), kstar);
    const int cstar = wsel * K + kstar;
    // The crossing chunk again, straight from memory (the caches hold it in practice).
    uint32_t xw[RRX<DT, EPL>::kWords];
    uint32_t mw[RRMask<MK, EPL>::kWords];
    {
        const int xo = (cstar * CH + lane * EPL) * Elem<DT>::kBytes;
#pragma unroll
        for (int qq = 0; qq < LX; qq++) {
            const auto a = __builtin_amdgcn_raw_buffer_load_b128(xres, xo + 16 * qq, 0, 0);
            xw[4 * qq] = a[0];
            xw[4 * qq + 1] = a[1];
            xw[4 * qq + 2] = a[2];
            xw[4 * qq + 3] = a[3];
        }
        if constexpr (MK == NT_MASK_U8) {
            const auto m2 = __builtin_amdgcn_raw_buffer_load_b64(mres, cstar * CH + lane * EPL, 0, 0);
            mw[0] = m2[0];
            mw[1] = m2[1];
        } else if constexpr (MK == NT_MASK_F32) {
#pragma unroll
            for (int qq = 0; qq < EPL / 4; qq++) {
                const auto a = __builtin_amdgcn_raw_buffer_load_b128(mres, (cstar * CH + lane * EPL) * 4 + 16 * qq, 0, 0);
                mw[4 * qq] = a[0];
                mw[4 * qq + 1] = a[1];
                mw[4 * qq + 2] = a[2];
                mw[4 * qq + 3] = a[3];
            }
        } else {
            mw[0] = 0;
        }
    }
    float v[EPL];
    decode_e<DT, MK, EPL>(xw, mw, v, p.tau, tau_one);
    {
        const int64_t e0 = int64_t(cstar) * CH + lane * EPL;
#pragma unroll
        for (int j = 0; j < EPL; j++)
            if (e0 + j >= p.V) v[j] = -INFINITY;
    }
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
    if (none) lsel = last_lane(__ballot(jlast >= 0));
    if (lsel < 0) {
        refuse(NT_ROW_NAN);
        return;
    }
    int jsel = -1;
    {
        const double t0 = tloc - (cincl - ls);
        float Cs = 0.0f;
#pragma unroll
        for (int j = 0; j < EPL; j++) {
            Cs += w[j];
            if (jsel < 0 && !none && double(Cs) > t0) jsel = j;
        }
        if (jsel < 0) jsel = jlast;
    }
    if (lane == lsel) {
        if (jsel < 0) jsel = 0;
        float vz = v[0];
#pragma unroll
        for (int j = 1; j < EPL; j++)
            if (j == jsel) vz = v[j];
        write_row(int64_t(cstar) * CH + lane * EPL + jsel, vz);
    }
}

}  // namespace
}  // namespace nt
