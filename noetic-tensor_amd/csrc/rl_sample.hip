// The nn::rl samplers' dispatch and their C-ABI entry point nt_hip_rl_sample. The kernels
// (rl_sample_kernels.hpp) launch either from this library's code objects or, compiled at run
// time by hiprtc, through hipModuleLaunchKernel (rtc.cpp), as the library's kernel path says.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "nt_launch.hpp"
#include "rl_sample_kernels.hpp"

namespace nt {
namespace {

// ------------------------------------------------------------------ dispatch

template <int DT, int MK, bool ENT, bool AL>
void launch_sample(const SampleP &p, int64_t rows, int threads, size_t shm, hipStream_t s) {
    char nm[96];
    std::snprintf(nm, sizeof nm, "nt::k_sample<%d, %d, %s, %s>", DT, MK, rtc_bool(ENT), rtc_bool(AL));
    launch_path(k_sample<DT, MK, ENT, AL>, nm, dim3(unsigned(rows)), dim3(threads), shm, s, p);
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
// Unmasked f32 rows stop at 4 chunks per wave: at 8 the kernel needs more than 128 registers and
// spills, and segments or the streaming kernel measured faster for those rows at every row count.
int rr_kmax(int dtype, int mk, int epl) {
    int k = (dtype != NT_F32 ? 128 : 64) / epl;
    if (mk == NT_MASK_F32) k = k < 32 / epl ? k : 32 / epl;  // 16 waves * K * 256 EPL bytes <= 128 KiB
    if (dtype == NT_F32 && mk == NT_MASK_NONE) k = k < 32 / epl ? k : 32 / epl;
    return k;
}

template <int DT, int MK, int K, int EPL, int WN>
void launch_rr_kw(bool ent, const SampleP &p, int64_t rows, hipStream_t s) {
    char nm[96];
    std::snprintf(nm, sizeof nm, "nt::k_sample_rr<%d, %d, %d, %s, %d, %d>", DT, MK, K, rtc_bool(ent), EPL, WN);
    if (ent) launch_path(k_sample_rr<DT, MK, K, true, EPL, WN>, nm, dim3(unsigned(rows)), dim3(kRRThreads), 0, s, p);
    else launch_path(k_sample_rr<DT, MK, K, false, EPL, WN>, nm, dim3(unsigned(rows)), dim3(kRRThreads), 0, s, p);
}

// Every chunk's loads in flight at once (allw) for K of 2 or 4: a launch of few rows is bound by
// the latency of each compute unit's reads, not by its VALU.
template <int DT, int MK, int K, int EPL>
void launch_rr_k(bool ent, bool allw, const SampleP &p, int64_t rows, hipStream_t s) {
    if constexpr (K == 2 || K == 4) {
        if (allw) {
            launch_rr_kw<DT, MK, K, EPL, K>(ent, p, rows, s);
            return;
        }
    }
    launch_rr_kw<DT, MK, K, EPL, kRRWindow>(ent, p, rows, s);
}

// K is a power of two up to rr_kmax(DT, MK, EPL); the instantiations are exactly those.
template <int DT, int MK, int EPL>
void launch_rr_mk(int K, bool ent, bool allw, const SampleP &p, int64_t rows, hipStream_t s) {
    constexpr int KREG = (DT != NT_F32 ? 128 : 64) / EPL;
    constexpr int KMAX = (MK == NT_MASK_F32 || (DT == NT_F32 && MK == NT_MASK_NONE)) && 32 / EPL < KREG ? 32 / EPL : KREG;
    switch (K) {
        case 1: launch_rr_k<DT, MK, 1, EPL>(ent, allw, p, rows, s); break;
        case 2: launch_rr_k<DT, MK, 2, EPL>(ent, allw, p, rows, s); break;
        case 4: if constexpr (KMAX >= 4) launch_rr_k<DT, MK, 4, EPL>(ent, allw, p, rows, s); break;
        case 8: if constexpr (KMAX >= 8) launch_rr_k<DT, MK, 8, EPL>(ent, allw, p, rows, s); break;
        case 16: if constexpr (KMAX >= 16) launch_rr_k<DT, MK, 16, EPL>(ent, allw, p, rows, s); break;
        default: break;
    }
}

template <int EPL>
void launch_rr(int dtype, int mk, int K, bool ent, bool allw, const SampleP &p, int64_t rows, hipStream_t s) {
    if (dtype == NT_F32) {
        if (mk == NT_MASK_U8) launch_rr_mk<NT_F32, NT_MASK_U8, EPL>(K, ent, allw, p, rows, s);
        else if (mk == NT_MASK_F32) launch_rr_mk<NT_F32, NT_MASK_F32, EPL>(K, ent, allw, p, rows, s);
        else launch_rr_mk<NT_F32, NT_MASK_NONE, EPL>(K, ent, allw, p, rows, s);
    } else if (dtype == NT_BF16) {
        if (mk == NT_MASK_U8) launch_rr_mk<NT_BF16, NT_MASK_U8, EPL>(K, ent, allw, p, rows, s);
        else if (mk == NT_MASK_F32) launch_rr_mk<NT_BF16, NT_MASK_F32, EPL>(K, ent, allw, p, rows, s);
        else launch_rr_mk<NT_BF16, NT_MASK_NONE, EPL>(K, ent, allw, p, rows, s);
    } else {
        if (mk == NT_MASK_U8) launch_rr_mk<NT_F16, NT_MASK_U8, EPL>(K, ent, allw, p, rows, s);
        else if (mk == NT_MASK_F32) launch_rr_mk<NT_F16, NT_MASK_F32, EPL>(K, ent, allw, p, rows, s);
        else launch_rr_mk<NT_F16, NT_MASK_NONE, EPL>(K, ent, allw, p, rows, s);
    }
}

// The queued sampler (u8 keep-masks): K chunks per wave in stages of 4 (K = 4) or 8 (K = 16)
// chunks, two stages from K = 8 on; SH when mask rows are shared by several logits rows.
template <int DT, int K, bool SH>
void launch_rq_k(bool ent, const SampleP &p, int64_t rows, hipStream_t s) {
    constexpr int NS = K >= 8 ? 2 : 1;
    char nm[96];
    std::snprintf(nm, sizeof nm, "nt::k_sample_rq<%d, %d, %s, %d, %s>", DT, K, rtc_bool(ent), NS, rtc_bool(SH));
    if (ent) launch_path(k_sample_rq<DT, K, true, NS, SH>, nm, dim3(unsigned(rows)), dim3(kRRThreads), 0, s, p);
    else launch_path(k_sample_rq<DT, K, false, NS, SH>, nm, dim3(unsigned(rows)), dim3(kRRThreads), 0, s, p);
}

template <int DT, bool SH>
void launch_rq_dt(int K, bool ent, const SampleP &p, int64_t rows, hipStream_t s) {
    if (K == 4) {
        launch_rq_k<DT, 4, SH>(ent, p, rows, s);
    } else if constexpr (DT == NT_F32) {
        launch_rq_k<DT, 8, SH>(ent, p, rows, s);  // (f32 rows take at most 8 chunks per wave)
    } else {
        if (K == 8) launch_rq_k<DT, 8, SH>(ent, p, rows, s);
        else launch_rq_k<DT, 16, SH>(ent, p, rows, s);
    }
}

// Whether several of the launch's logits rows read one mask row: a stride 0 over a dimension of
// the row map longer than one (rows = S T B).
bool mask_shared(const MaskMap &m, int64_t rows) {
    return (m.ld == 0 && m.T > 1u) || (m.ld_b == 0 && m.B > 1u) || (m.ld_s == 0 && rows > int64_t(m.T) * m.B);
}

void launch_rq(int dtype, int K, bool ent, const SampleP &p, int64_t rows, hipStream_t s) {
    const bool sh = mask_shared(p.mm, rows);
    if (dtype == NT_F32) {
        if (sh) launch_rq_dt<NT_F32, true>(K, ent, p, rows, s);
        else launch_rq_dt<NT_F32, false>(K, ent, p, rows, s);
    } else if (dtype == NT_BF16) {
        if (sh) launch_rq_dt<NT_BF16, true>(K, ent, p, rows, s);
        else launch_rq_dt<NT_BF16, false>(K, ent, p, rows, s);
    } else {
        if (sh) launch_rq_dt<NT_F16, true>(K, ent, p, rows, s);
        else launch_rq_dt<NT_F16, false>(K, ent, p, rows, s);
    }
}

// Whether a u8-masked launch of K chunks per wave takes the queued sampler: K of 4 or more (the
// queue's stages are 4 chunks at least), a mask whose rows start on 16 bytes (the mask comes in
// 16-byte pieces per lane), and no NOETIC_HIP_SAMPLE_QUEUE=off (a tuning knob that keeps the
// register-resident sampler). Measured on MI355X at 256 rows of V = 128256 bf16, tau 0.7, HBM-cold
// inputs: a grammar mask of runs (30% kept) 20.2 -> 16.8 us, a Bernoulli(0.9) mask 20.2 -> 20.4 us
// (its waves take the dense path); at V = 50304 f32, runs 14.6 -> 10.2 us, Bernoulli 14.6 -> 14.4 us.
bool use_queue(int mk, int K, const void *mask, const MaskMap &mm) {
    if (mk != NT_MASK_U8 || K < 4) return false;
    if (reinterpret_cast<uintptr_t>(mask) % 16 != 0 || mm.ld % 16 != 0 || mm.ld_b % 16 != 0 || mm.ld_s % 16 != 0)
        return false;
    const char *env = std::getenv("NOETIC_HIP_SAMPLE_QUEUE");
    return !(env && std::strcmp(env, "off") == 0);
}

// ------------------------------------------------------------------ segmented dispatch

// Arrival counters of the segmented sampler: one u32 per row at the start of its workspace, for
// up to kSegMaxRows rows; the wave records follow. The counters are zero between launches: the
// resolver of each row resets its own before the launch ends.
constexpr int64_t kSegMaxRows = kSegCounterBytes / sizeof(uint32_t);

struct SegShape {
    int nw = 0, k = 0, g = 0;  // waves per segment, chunks per wave, segments per row (0: none)
};

// The (NW, K) pairs the segmented sampler is instantiated for: 4 or 8 waves, 4, 8 or 16 chunks
// per wave (at most 8 for f32 rows: 8 logit words per chunk in registers), and an f32 mask's
// 2 KiB per chunk within 128 KiB of LDS.
bool seg_built(int dtype, int mk, int nw, int k) {
    if (nw != 4 && nw != 8) return false;
    if (k != 4 && k != 8 && k != 16) return false;
    if (dtype == NT_F32 && k > 8) return false;
    if (mk == NT_MASK_F32 && nw * k > 64) return false;
    return true;
}

// How a launch of `rows` aligned rows of `nch` chunks is cut. NOETIC_HIP_SAMPLE_SEG=off keeps one
// workgroup per row; NOETIC_HIP_SAMPLE_SEG=NW,K forces segments of NW waves of K chunks (a tuning
// knob; shapes the library is not built for, or that give fewer than two segments, keep one
// workgroup per row).
SegShape seg_shape(int dtype, int mk, int64_t rows, int64_t nch) {
    SegShape s;
    if (rows > kSegMaxRows) return s;
    int nw = 0, k = 0;
    const char *env = std::getenv("NOETIC_HIP_SAMPLE_SEG");
    if (env && *env) {
        if (std::sscanf(env, "%d,%d", &nw, &k) != 2 || !seg_built(dtype, mk, nw, k)) return s;
    } else {
        // Measured on MI355X (logits re-read, as a decode step's are): segments pay for their
        // merge (an arrival counter, the wave records and the crossing chunk read again, about
        // 3 us of latency on the row's critical path) only when few rows each stream many
        // chunks. V = 128256 bf16 with a u8 mask: 1 row 12.0 -> 6.2 us, 16 rows 12.3 -> 7.3 us,
        // 64 rows 12.8 -> 9.0 us, 256 rows 17.0 -> 21.0 us; V = 32000 f32: one workgroup per row
        // is faster at every row count.
        //
        // Unmasked f32 rows of 65 to 128 chunks (32768 < V <= 65536) would need the
        // register-resident kernel at 8 chunks per wave, which spills; V = 50304 f32 measured
        // (us, rows 16 / 64 / 256 / 1024 / 4096): that kernel 7.6 / 8.2 / 13.0 / 42.6 / 185,
        // segments of 8 waves x 4 chunks 6.1 / 6.8 / 13.2 / 37.4 / 174, of 8 x 8 chunks
        // 7.4 / 7.7 / 11.8 / 38.5 / 167, the streaming kernel 9.5 / 9.8 / 13.8 / 35.7 / 146.
        // Those rows take segments up to 256 rows and the streaming kernel beyond.
        const bool f32_k8 = dtype == NT_F32 && mk == NT_MASK_NONE && nch > 64 && nch <= 128;
        if (rows <= 64 && (nch >= 96 || f32_k8)) {
            nw = 8;
            k = 4;
        } else if (f32_k8 && rows <= 256) {
            nw = 8;
            k = 8;
        } else {
            return s;
        }
    }
    const int64_t g = (nch + int64_t(nw) * k - 1) / (int64_t(nw) * k);
    if (g < 2 || g * nw > kSegMaxRecords) return s;
    s.nw = nw;
    s.k = k;
    s.g = int(g);
    return s;
}

// Whether each wave issues all its chunks' loads at once: NOETIC_HIP_SAMPLE_WINDOW=all or one
// forces it (a tuning knob); otherwise launches of fewer rows than compute units do, where each
// compute unit's read latency, not its VALU, bounds the launch.
bool all_in_flight(int64_t workgroups) {
    const char *env = std::getenv("NOETIC_HIP_SAMPLE_WINDOW");
    if (env && std::strcmp(env, "all") == 0) return true;
    if (env && std::strcmp(env, "one") == 0) return false;
    return workgroups < 256;
}

size_t seg_workspace_bytes(int64_t rows, const SegShape &s) {
    return kSegCounterBytes + size_t(rows) * size_t(s.g * s.nw) * (sizeof(SegRec) + 4 * size_t(s.k));
}

// The library's workspace of the segmented sampler on the claimed device: allocated on first use,
// reallocated (after the stream drains) when a launch needs more, counters zeroed by a kernel on
// the library stream, kept until the process ends.
struct SegWorkspace {
    uint8_t *base = nullptr;
    size_t bytes = 0;
};
SegWorkspace g_seg_ws;

int seg_workspace(size_t need, uint8_t **out) {
    if (need > g_seg_ws.bytes) {
        size_t nb = need < (size_t(4) << 20) ? (size_t(4) << 20) : need;
        nb = (nb + 0xfffff) & ~size_t(0xfffff);
        if (g_seg_ws.base) {
            if (int rc = hip_check(hipStreamSynchronize(ctx().stream), "hipStreamSynchronize")) return rc;
            if (int rc = hip_check(hipFree(g_seg_ws.base), "hipFree")) return rc;
            g_seg_ws = SegWorkspace{};
        }
        void *p = nullptr;
        if (int rc = hip_check(hipMalloc(&p, nb), "hipMalloc")) return rc;
        if (int rc = zero_words(static_cast<uint32_t *>(p), kSegCounterBytes / sizeof(uint32_t))) {
            (void)hipFree(p);
            return rc;
        }
        g_seg_ws.base = static_cast<uint8_t *>(p);
        g_seg_ws.bytes = nb;
    }
    *out = g_seg_ws.base;
    return 0;
}

template <int DT, int MK, int K, int NW, int WN>
void launch_seg_kw(bool ent, const SegP &q, int64_t rows, hipStream_t s) {
    const dim3 grid(unsigned(rows * q.G));
    char nm[96];
    std::snprintf(nm, sizeof nm, "nt::k_sample_seg<%d, %d, %d, %s, %d, %d>", DT, MK, K, rtc_bool(ent), NW, WN);
    if (ent) launch_path(k_sample_seg<DT, MK, K, true, NW, WN>, nm, grid, dim3(NW * kWave), 0, s, q);
    else launch_path(k_sample_seg<DT, MK, K, false, NW, WN>, nm, grid, dim3(NW * kWave), 0, s, q);
}

template <int DT, int MK, int K, int NW>
void launch_seg_k(bool ent, bool allw, const SegP &q, int64_t rows, hipStream_t s) {
    if constexpr (K == 4) {
        if (allw) {
            launch_seg_kw<DT, MK, K, NW, K>(ent, q, rows, s);
            return;
        }
    }
    launch_seg_kw<DT, MK, K, NW, kRRWindow>(ent, q, rows, s);
}

template <int DT, int MK, int NW>
void launch_seg_nw(int k, bool ent, bool allw, const SegP &q, int64_t rows, hipStream_t s) {
    if (k == 4) launch_seg_k<DT, MK, 4, NW>(ent, allw, q, rows, s);
    else if (k == 8) launch_seg_k<DT, MK, 8, NW>(ent, allw, q, rows, s);
    else if constexpr (DT != NT_F32 && (MK != NT_MASK_F32 || NW * 16 <= 64))
        launch_seg_k<DT, MK, 16, NW>(ent, allw, q, rows, s);
}

template <int DT, int MK>
void launch_seg_mk(int nw, int k, bool ent, bool allw, const SegP &q, int64_t rows, hipStream_t s) {
    if (nw == 4) launch_seg_nw<DT, MK, 4>(k, ent, allw, q, rows, s);
    else launch_seg_nw<DT, MK, 8>(k, ent, allw, q, rows, s);
}

void launch_seg(int dtype, int mk, const SegShape &sh, bool ent, bool allw, const SegP &q, int64_t rows, hipStream_t s) {
    if (dtype == NT_F32) {
        if (mk == NT_MASK_U8) launch_seg_mk<NT_F32, NT_MASK_U8>(sh.nw, sh.k, ent, allw, q, rows, s);
        else if (mk == NT_MASK_F32) launch_seg_mk<NT_F32, NT_MASK_F32>(sh.nw, sh.k, ent, allw, q, rows, s);
        else launch_seg_mk<NT_F32, NT_MASK_NONE>(sh.nw, sh.k, ent, allw, q, rows, s);
    } else if (dtype == NT_BF16) {
        if (mk == NT_MASK_U8) launch_seg_mk<NT_BF16, NT_MASK_U8>(sh.nw, sh.k, ent, allw, q, rows, s);
        else if (mk == NT_MASK_F32) launch_seg_mk<NT_BF16, NT_MASK_F32>(sh.nw, sh.k, ent, allw, q, rows, s);
        else launch_seg_mk<NT_BF16, NT_MASK_NONE>(sh.nw, sh.k, ent, allw, q, rows, s);
    } else {
        if (mk == NT_MASK_U8) launch_seg_mk<NT_F16, NT_MASK_U8>(sh.nw, sh.k, ent, allw, q, rows, s);
        else if (mk == NT_MASK_F32) launch_seg_mk<NT_F16, NT_MASK_F32>(sh.nw, sh.k, ent, allw, q, rows, s);
        else launch_seg_mk<NT_F16, NT_MASK_NONE>(sh.nw, sh.k, ent, allw, q, rows, s);
    }
}


}  // namespace

// nt_hip_rl_sample's dispatch, with the segmented sampler's workspace from `workspace` (the
// library's allocation for nt_hip_rl_sample); `nofree` skips the deferred frees of enter().
int sample_entry(const NtRlSampleArgs *a, WorkspaceFn workspace, bool nofree, const char *who) {
    if (!a) return fail(NT_E_ARG, std::string(who) + ": null args");
    if (int rc = check_rows(a->rows, a->vocab, a->ld, a->dtype, a->mask_kind, a->mask, a->mask_ld, who)) return rc;
    MaskMap mm;
    if (int rc = mask_map(a->mask_rows, a->rows, a->vocab, a->mask_kind, a->mask_ld, who, &mm)) return rc;
    if (!(a->temperature >= 0.0) || !std::isfinite(a->temperature))
        return fail(NT_E_ARG, "sample_categorical: temperature " + std::to_string(a->temperature) + " (must be ≥ 0)");
    const bool greedy = a->temperature == 0.0;
    if (!a->logits || !a->ids || !a->status || (!greedy && !a->uniforms))
        return fail(NT_E_ARG, std::string(who) + ": null logits, ids, status or uniforms");
    std::unique_lock<std::mutex> lk;
    if (int rc = nofree ? enter_nofree(&lk) : enter(&lk)) return rc;
    if (a->rows == 0) return 0;
    const int64_t nc = (a->vocab + kChunk - 1) / kChunk;
    const bool ent = a->entropy != nullptr;
    const size_t shm = size_t(nc) * sizeof(float) * (ent ? 3 : 2);
    if (shm > 64 * 1024) return fail(NT_E_UNSUPPORTED, std::string(who) + ": V " + std::to_string(a->vocab) + " too large");
    SampleP p;
    p.logits = a->logits;
    p.mask = a->mask;
    p.V = a->vocab;
    p.ld = a->ld;
    p.mm = mm;
    const double T = greedy ? 1.0 : a->temperature;
    p.tau = float(T);
    p.tau_one = (T == 1.0);
    p.c = (a->mask_kind == NT_MASK_F32 || T == 1.0) ? kLog2e : float(double(kLog2e) / double(p.tau));
    p.m_ovf = p.tau_one ? -INFINITY : neg_overflow_bound(p.tau);
    p.greedy = greedy;
    p.nc = int(nc);
    p.u = a->uniforms;
    p.ids = a->ids;
    p.logp = a->logp;
    p.ent = a->entropy;
    p.status = a->status;
    // Waves per row of the streaming kernel: about four chunks per wave, at most 16; many rows get
    // smaller groups.
    int nw = int(nc / 4);
    nw = nw < 1 ? 1 : (nw > 16 ? 16 : nw);
    if (a->rows >= 2048 && nw > 4) nw = 4;
    const bool al = aligned_rows(a->logits, a->vocab, a->ld, a->dtype, a->mask_kind, a->mask, mm);
    hipStream_t s = ctx().stream;
    // Aligned rows: segments when few rows each hold many chunks, else one workgroup per row when
    // the row fits its registers (chunks per wave K = 1..16); the streaming kernel takes the rest
    // (unaligned rows, larger V).
    if (al) {
        // 8 elements per lane (512-element chunks): 16 per lane measured slower on MI355X at c4
        // (19.37 us, or 18.81 with a one-chunk window, against 18.24-18.52 us at 8).
        constexpr int epl = 8;
        const int64_t nch = (a->vocab + kWave * epl - 1) / (kWave * epl);
        const SegShape sg = seg_shape(a->dtype, a->mask_kind, a->rows, nch);
        if (sg.g > 0) {
            uint8_t *ws = nullptr;
            const size_t need = seg_workspace_bytes(a->rows, sg);
            if (int rc = workspace(need, &ws)) return rc;
            SegP q;
            q.s = p;
            q.s.nc = int(nch);
            q.G = sg.g;
            q.nwr = sg.g * sg.nw;
            q.rec_bytes = int(sizeof(SegRec)) + 4 * sg.k;
            q.count = reinterpret_cast<uint32_t *>(ws);
            q.recs = ws + kSegCounterBytes;
            rtc_status() = 0;
            launch_seg(a->dtype, a->mask_kind, sg, ent, all_in_flight(a->rows * sg.g), q, a->rows, s);
            return rtc_status() ? rtc_status() : launched(who);
        }
        const int kmax = rr_kmax(a->dtype, a->mask_kind, epl);
        const char *rr_env = std::getenv("NOETIC_HIP_SAMPLE_RR");  // "off": the streaming kernel (a tuning knob)
        if (nch <= int64_t(kRRWaves) * kmax && !(rr_env && std::strcmp(rr_env, "off") == 0)) {
            int K = 1;
            while (int64_t(kRRWaves) * K < nch) K *= 2;
            p.nc = int(nch);
            rtc_status() = 0;
            if (use_queue(a->mask_kind, K, a->mask, mm)) launch_rq(a->dtype, K, ent, p, a->rows, s);
            else launch_rr<8>(a->dtype, a->mask_kind, K, ent, all_in_flight(a->rows), p, a->rows, s);
            return rtc_status() ? rtc_status() : launched(who);
        }
    }
    // An f32 mask on aligned 16-bit rows is staged through LDS after the per-chunk records:
    // kMaskStage chunks of f32 words (2 KiB each) per wave, at 16 bytes.
    const size_t shs = al && a->dtype != NT_F32 && a->mask_kind == NT_MASK_F32
                           ? ((shm + 15) & ~size_t(15)) + size_t(nw) * kMaskStage * kChunk * sizeof(float)
                           : shm;
    rtc_status() = 0;
    if (a->dtype == NT_F32) pick_mk_sample<NT_F32>(a->mask_kind, ent, al, p, a->rows, nw * kWave, shs, s);
    else if (a->dtype == NT_BF16) pick_mk_sample<NT_BF16>(a->mask_kind, ent, al, p, a->rows, nw * kWave, shs, s);
    else pick_mk_sample<NT_F16>(a->mask_kind, ent, al, p, a->rows, nw * kWave, shs, s);
    return rtc_status() ? rtc_status() : launched(who);
}

namespace {
__global__ void k_zero_words(uint32_t *p, int64_t n) {
    for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
        p[i] = 0;
}
}  // namespace

int zero_words(uint32_t *p, size_t n) {
    hipLaunchKernelGGL(k_zero_words, dim3(64), dim3(256), 0, ctx().stream, p, int64_t(n));
    return launched("zero_words");
}

}  // namespace nt

using namespace nt;

extern "C" {

int nt_hip_rl_sample(const NtRlSampleArgs *a) { return sample_entry(a, seg_workspace, false, "nt_hip_rl_sample"); }

}  // extern "C"
