// The reference's Gumbel-max sampler on the device: sample_categorical (src/nn/rl.rs:488-529)
// for a Hip tensor, with the reference's contract kept whole: one u64 of the caller's ChaCha20
// stream per logit in row-major order, the draw u = ((k >> 11) + 0.5) / 2^53, the f64 noise
// -ln(-ln u) rounded once to f32, the f32 sum z + g and the first maximum of each row.
//
// The reference draws the noise on the host and uploads it (rows x V f64 values turned into
// f32, then an add kernel and an argmax kernel). Here the noise is generated where it is used:
// ChaCha20 is a counter-mode stream, so word w of the keystream is word w % 16 of block w / 16
// and every element's u64 is computed from the stream's key and starting word position alone.
// One workgroup takes one row (rl_gumbel_kernels.hpp):
//  - the row is cut into blocks of 8 elements, one keystream block each; a block whose eight
//    logits are all excluded (-inf) is skipped without generating it (such an element can never
//    be the maximum of an accepted row; a row with no other candidate is refused);
//  - each wave queues its blocks that hold an allowed element in LDS and generates their
//    keystream by full waves;
//  - every allowed element's draw is first screened in f32 (hardware logarithms, within 1e-5 of
//    the exact f32 value); only the elements within a margin of the row's largest screened value
//    (1e-3, or four ulps of it where that is wider) can be the row's maximum. A single one is the
//    answer; several are evaluated exactly, in f64 as the reference does, and the row's first
//    maximum is taken among them with "greater value, else smaller index", which is associative,
//    so the result is the sequential first maximum whatever the timing (a thread with more than
//    four candidates sends its row to the exact evaluation of every element);
//  - rows whose first u64 starts a block, on aligned rows, read a block's 8 logits and mask
//    entries with vector loads issued two steps ahead; others read element by element.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/noetic_hip.h"
#include "nt_internal.hpp"
#include "nt_launch.hpp"
#include "rl_gumbel_kernels.hpp"

namespace nt {
namespace {

template <int DT, int MK, bool ODD, bool GREEDY>
void launch_gumbel(const GumbelP &p, int64_t rows, int threads, hipStream_t s) {
    char nm[96];
    std::snprintf(nm, sizeof nm, "nt::k_sample_gumbel<%d, %d, %s, %s>", DT, MK, rtc_bool(ODD), rtc_bool(GREEDY));
    launch_path(k_sample_gumbel<DT, MK, ODD, GREEDY>, nm, dim3(unsigned(rows)), dim3(threads),
                gumbel_queue_bytes(threads, GREEDY), s, p);
}

template <int DT, int MK>
void pick_gumbel(bool odd, bool greedy, const GumbelP &p, int64_t rows, int threads, hipStream_t s) {
    if (greedy) launch_gumbel<DT, MK, false, true>(p, rows, threads, s);
    else if (odd) launch_gumbel<DT, MK, true, false>(p, rows, threads, s);
    else launch_gumbel<DT, MK, false, false>(p, rows, threads, s);
}

template <int DT>
void pick_gumbel_mk(int mk, bool odd, bool greedy, const GumbelP &p, int64_t rows, int threads, hipStream_t s) {
    if (mk == NT_MASK_U8) pick_gumbel<DT, NT_MASK_U8>(odd, greedy, p, rows, threads, s);
    else if (mk == NT_MASK_F32) pick_gumbel<DT, NT_MASK_F32>(odd, greedy, p, rows, threads, s);
    else pick_gumbel<DT, NT_MASK_NONE>(odd, greedy, p, rows, threads, s);
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" int nt_hip_rl_sample_gumbel(const NtRlGumbelArgs *a) {
    if (!a) return fail(NT_E_ARG, "nt_hip_rl_sample_gumbel: null args");
    const int64_t rows = a->rows, V = a->vocab;
    if (rows < 0 || V < 1 || a->ld < V || (a->dtype != NT_F32 && a->dtype != NT_BF16 && a->dtype != NT_F16) ||
        a->mask_kind < NT_MASK_NONE || a->mask_kind > NT_MASK_F32 ||
        ((a->mask_kind == NT_MASK_NONE) != (a->mask == nullptr)) || (a->mask_ld != 0 && a->mask_ld < V) ||
        rows > 0x7fffffffLL || V > 0x7fffffffLL || a->word < 0 || a->word > 15)
        return fail(NT_E_ARG, "nt_hip_rl_sample_gumbel: invalid rows " + std::to_string(rows) + ", V " +
                                  std::to_string(V) + ", ld " + std::to_string(a->ld) + ", dtype, mask or word " +
                                  std::to_string(a->word));
    if (!(a->temperature >= 0.0) || !std::isfinite(a->temperature))
        return fail(NT_E_ARG, "sample_categorical: temperature " + std::to_string(a->temperature) + " (must be ≥ 0)");
    if (!a->logits || !a->ids || !a->status)
        return fail(NT_E_ARG, "nt_hip_rl_sample_gumbel: null logits, ids or status");
    MaskMap mm;
    if (int rc = mask_map(a->mask_rows, rows, V, a->mask_kind, a->mask_ld, "nt_hip_rl_sample_gumbel", &mm)) return rc;
    // The stream's block counter is 64-bit: the draws of this call must not wrap it.
    const uint64_t words = 2 * uint64_t(rows) * uint64_t(V);
    if (a->block > (~uint64_t(0) >> 5) || words > (uint64_t(1) << 62))
        return fail(NT_E_ARG, "nt_hip_rl_sample_gumbel: stream position or draw count out of range");
    std::unique_lock<std::mutex> lk;
    if (int rc = enter(&lk)) return rc;
    if (rows == 0) return 0;
    const bool greedy = a->temperature == 0.0;
    GumbelP p;
    p.logits = a->logits;
    p.mask = a->mask;
    p.V = V;
    p.ld = a->ld;
    p.mm = mm;
    const double T = greedy ? 1.0 : a->temperature;
    p.tau = float(T);  // the reference divides by `temperature as f32` (float.rs:494-499)
    p.tau_one = T == 1.0;
    for (int i = 0; i < 8; i++) p.key.k[i] = a->key[i];
    const uint64_t w0 = 16 * a->block + uint64_t(a->word);
    p.h = w0 >> 1;
    const bool odd = (w0 & 1) != 0;
    p.ids = a->ids;
    p.status = a->status;
    // the aligned path: rows and mask rows start on their vector loads' alignment, V is a whole
    // number of 8-element blocks (so no 16- or 8-byte load ends partly past the row's bytes, and
    // what a load past the end returns is all zeros), and a row's bytes fit a buffer resource's
    // 32-bit range
    const int esz = a->dtype == NT_F32 ? 4 : 2, msz = a->mask_kind == NT_MASK_F32 ? 4 : 1;
    const bool mask_vec = a->mask_kind == NT_MASK_NONE ||
                          (reinterpret_cast<uintptr_t>(a->mask) % (a->mask_kind == NT_MASK_F32 ? 16 : 8) == 0 &&
                           (mm.ld * msz) % (a->mask_kind == NT_MASK_F32 ? 16 : 8) == 0 &&
                           (mm.ld_b * msz) % (a->mask_kind == NT_MASK_F32 ? 16 : 8) == 0 &&
                           (mm.ld_s * msz) % (a->mask_kind == NT_MASK_F32 ? 16 : 8) == 0);
    p.vec = reinterpret_cast<uintptr_t>(a->logits) % 16 == 0 && (a->ld * esz) % 16 == 0 && mask_vec && V % 8 == 0 &&
            V * 4 <= int64_t(0x7fffffff);
    // Threads per row: one per keystream block of the row, in whole waves, at most 1024.
    const int64_t nblk = V / 8 + 2;
    int threads = int(((nblk + 63) / 64) * 64);
    threads = threads > kGumbelMaxThreads ? kGumbelMaxThreads : threads;
    hipStream_t s = ctx().stream;
    rtc_status() = 0;
    if (a->dtype == NT_F32) pick_gumbel_mk<NT_F32>(a->mask_kind, odd, greedy, p, rows, threads, s);
    else if (a->dtype == NT_BF16) pick_gumbel_mk<NT_BF16>(a->mask_kind, odd, greedy, p, rows, threads, s);
    else pick_gumbel_mk<NT_F16>(a->mask_kind, odd, greedy, p, rows, threads, s);
    return rtc_status() ? rtc_status() : launched("nt_hip_rl_sample_gumbel");
}
