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
#include "nt_launch.hpp"
#include "nt_rows.hpp"
#include "rl_score_kernels.hpp"

namespace nt {
namespace {

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

template <int DT, int MK, bool REF, bool KL, bool ENT>
void pick_al_score(bool al, const ScoreP &p, int64_t rows, hipStream_t s) {
    char nm[96];
    std::snprintf(nm, sizeof nm, "nt::k_score<%d, %d, %s, %s, %s, %s>", DT, MK, rtc_bool(REF), rtc_bool(KL),
                  rtc_bool(ENT), rtc_bool(al));
    if (al) launch_path(k_score<DT, MK, REF, KL, ENT, true>, nm, dim3(unsigned(rows)), dim3(kScoreThreads), 0, s, p);
    else launch_path(k_score<DT, MK, REF, KL, ENT, false>, nm, dim3(unsigned(rows)), dim3(kScoreThreads), 0, s, p);
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

int nt_hip_rl_score(const NtRlScoreArgs *a) {
    if (!a) return fail(NT_E_ARG, "nt_hip_rl_score: null args");
    if (int rc = check_rows(a->rows, a->vocab, a->ld, a->dtype, a->mask_kind, a->mask, a->mask_ld, "nt_hip_rl_score"))
        return rc;
    MaskMap mm;
    if (int rc = mask_map(a->mask_rows, a->rows, a->vocab, a->mask_kind, a->mask_ld, "nt_hip_rl_score", &mm)) return rc;
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
    p.mm = mm;
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
    bool al = aligned_rows(a->logits, a->vocab, a->ld, a->dtype, a->mask_kind, a->mask, mm) &&
              a->vocab * 4 <= int64_t(0x7fffffff);
    if (ref) al = al && reinterpret_cast<uintptr_t>(a->ref_logits) % 16 == 0;
    hipStream_t s = ctx().stream;
    rtc_status() = 0;
    if (a->dtype == NT_F32) pick_mk_score<NT_F32>(a->mask_kind, ref, kl, ent, al, p, a->rows, s);
    else if (a->dtype == NT_BF16) pick_mk_score<NT_BF16>(a->mask_kind, ref, kl, ent, al, p, a->rows, s);
    else pick_mk_score<NT_F16>(a->mask_kind, ref, kl, ent, al, p, a->rows, s);
    return rtc_status() ? rtc_status() : launched("nt_hip_rl_score");
}

int nt_hip_rl_score_backward(const NtRlScoreGradArgs *a) {
    if (!a) return fail(NT_E_ARG, "nt_hip_rl_score_backward: null args");
    if (int rc = check_rows(a->rows, a->vocab, a->ld, a->dtype, a->mask_kind, a->mask, a->mask_ld,
                            "nt_hip_rl_score_backward"))
        return rc;
    MaskMap mm;
    if (int rc = mask_map(a->mask_rows, a->rows, a->vocab, a->mask_kind, a->mask_ld, "nt_hip_rl_score_backward", &mm))
        return rc;
    if (!(a->temperature > 0.0) || !std::isfinite(a->temperature))
        return fail(NT_E_ARG, "tempered_logits: temperature " + std::to_string(a->temperature) + " (must be positive)");
    if (!a->logits || !a->grad || !a->lse_base || !a->lse_rest)
        return fail(NT_E_ARG, "nt_hip_rl_score_backward: null logits, grad or log-sum-exp statistics");
    if (a->grad_dtype != NT_F32 && a->grad_dtype != NT_BF16 && a->grad_dtype != NT_F16)
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
    p.mm = mm;
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
    bool al = aligned_rows(a->logits, a->vocab, a->ld, a->dtype, a->mask_kind, a->mask, mm) &&
              reinterpret_cast<uintptr_t>(a->grad) % 16 == 0 && a->grad_ld % kEpl == 0 &&
              a->vocab * 4 <= int64_t(0x7fffffff);
    if (kl) al = al && reinterpret_cast<uintptr_t>(a->ref_logits) % 16 == 0;
    hipStream_t s = ctx().stream;
    auto go = [&](auto dt, auto mk) {
        constexpr int DT = decltype(dt)::value, MK = decltype(mk)::value;
        auto launch = [&](auto klc, auto gdt, auto alc) {
            constexpr bool KL = decltype(klc)::value, AL = decltype(alc)::value;
            constexpr int GDT = decltype(gdt)::value;
            char nm[96];
            std::snprintf(nm, sizeof nm, "nt::k_score_grad<%d, %d, %s, %d, %s>", DT, MK, rtc_bool(KL), GDT,
                          rtc_bool(AL));
            launch_path(k_score_grad<DT, MK, KL, GDT, AL>, nm, dim3(unsigned(a->rows)), dim3(kGradThreads), 0, s, p);
        };
        auto by_al = [&](auto klc, auto gdt) {
            if (al) launch(klc, gdt, std::true_type{});
            else launch(klc, gdt, std::false_type{});
        };
        auto by_gdt = [&](auto klc) {
            if (a->grad_dtype == NT_F32) by_al(klc, std::integral_constant<int, NT_F32>{});
            else if (a->grad_dtype == NT_BF16) by_al(klc, std::integral_constant<int, NT_BF16>{});
            else by_al(klc, std::integral_constant<int, NT_F16>{});
        };
        if (kl) by_gdt(std::true_type{});
        else by_gdt(std::false_type{});
    };
    auto by_mk = [&](auto dt) {
        if (a->mask_kind == NT_MASK_U8) go(dt, std::integral_constant<int, NT_MASK_U8>{});
        else if (a->mask_kind == NT_MASK_F32) go(dt, std::integral_constant<int, NT_MASK_F32>{});
        else go(dt, std::integral_constant<int, NT_MASK_NONE>{});
    };
    rtc_status() = 0;
    if (a->dtype == NT_F32) by_mk(std::integral_constant<int, NT_F32>{});
    else if (a->dtype == NT_BF16) by_mk(std::integral_constant<int, NT_BF16>{});
    else by_mk(std::integral_constant<int, NT_F16>{});
    return rtc_status() ? rtc_status() : launched("nt_hip_rl_score_backward");
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
