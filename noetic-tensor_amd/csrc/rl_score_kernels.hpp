// The nn::rl scorer and its fused backward, device code for gfx950 (MI355X): per-token
// log-probabilities, the exact KL to a frozen reference and the entropy in one pass over a row
// (k_score), and the gradient of a weighted sum of the three with respect to the logits
// (k_score_grad). One source for both ways the library builds them: compiled ahead of time into
// libnoetic_hip.so (rl_kernels.hip includes this file), and compiled at run time by hiprtc from
// the text embedded in the library (rtc.cpp), which names each template instance it needs. The
// row layout, arithmetic and determinism rules are described in rl_kernels.hip.
#pragma once

#include "nt_rows.hpp"

namespace nt {
namespace {

// ------------------------------------------------------------------ scorer

struct ScoreP {
    const void *logits;
    const void *ref;
    const void *mask;
    int64_t V, ld;
    MaskMap mm;  // the mask row of each logits row
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
    if constexpr (MK != NT_MASK_NONE) mrow = static_cast<const char *>(p.mask) + mask_row_at(p.mm, row) * MaskWords<MK>::kBytes;

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
    // The value-space max as the reference's f32 max of the tempered logits.
    auto zmax = [&](float a) -> float {
        if constexpr (MK != NT_MASK_F32) return tau_one ? a : a / p.tau;
        else return a;
    };
    int stt = NT_ROW_OK;
    // (nothing allowed, or every allowed logit below -FLT_MAX T, whose tempered value is -inf)
    if (af == -INFINITY || zmax(af) == -INFINITY) stt = NT_ROW_NO_TOKEN;
    else if (!(S == S)) stt = NT_ROW_NAN;
    const double lnS = log(S);
    // The tempered logit of one token, with the reference's f32 arithmetic.
    auto ztok = [&](const void *rowp, int64_t tok) -> float {
        float x;
        if constexpr (DT == NT_F32) x = static_cast<const float *>(rowp)[tok];
        else x = widen16<DT>(uint32_t(static_cast<const uint16_t *>(rowp)[tok]));
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
    int64_t V, ld, gld;
    MaskMap mm;  // the mask row of each logits row
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
// Two gradients in a 16-bit dtype, a in the low half: bf16 as above, or f16 rounded to nearest
// even (v_cvt_f16_f32 in the default rounding mode; beyond 65504 they round to infinity).
template <int GDT>
__device__ __forceinline__ uint32_t pack16(float a, float b) {
    if constexpr (GDT == NT_BF16) return pack_bf16(a, b);
    else return uint32_t(__builtin_bit_cast(uint16_t, _Float16(a))) | (uint32_t(__builtin_bit_cast(uint16_t, _Float16(b))) << 16);
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

// The tempered logit as tempered_logits computes it: x / T (an f32 divide), then the mask
// (TAU1: x is already divided, or T is 1).
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
    // x / T for the step's 8 elements at once (div_tau: the IEEE quotient, three instructions each
    // where the division takes about ten), then the mask
    float x[kEpl], xr[kEpl];
#pragma unroll
    for (int j = 0; j < kEpl; j++) {
        x[j] = logit<DT>(rx.x, j);
        xr[j] = KL ? logit<DT>(ry.x, j) : 0.0f;
    }
    if constexpr (!TAU1) {
        div_tau<kEpl>(x, tau);
        if constexpr (KL) div_tau<kEpl>(xr, tau);
    }
#pragma unroll
    for (int j = 0; j < kEpl; j++) {
        const uint32_t mword = MK == NT_MASK_U8 ? rx.m[j / 4] : (MK == NT_MASK_F32 ? rx.m[j] : 0u);
        const float z = grad_tempered<MK, true>(x[j], tau, mword, j);
        const float zr = KL ? grad_tempered<MK, true>(xr[j], tau, mword, j) : 0.0f;
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
            const_cast<char *>(static_cast<const char *>(p.mask) + mask_row_at(p.mm, row) * MB), short(0), V * MB,
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
            const v4u w = {pack16<GDT>(o[0], o[1]), pack16<GDT>(o[2], o[3]), pack16<GDT>(o[4], o[5]), pack16<GDT>(o[6], o[7])};
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
    const char *mrow = MK != NT_MASK_NONE ? static_cast<const char *>(p.mask) + mask_row_at(p.mm, row) * MaskWords<MK>::kBytes
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
                const uint32_t w = pack16<GDT>(o[j], o[j + 1]);
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

}  // namespace
}  // namespace nt
