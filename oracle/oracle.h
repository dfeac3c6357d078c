/*
 * CPU oracle for the nn::rl vocabulary-row hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP library under
 * noetic-tensor_amd/) links, loads or calls this code; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
 * checker and as the timed CPU baseline.
 *
 * Two kinds of function live here:
 *  - or_*      : the f64 restatement of shyble/noetic-tensor 0.7.0 `src/nn/rl.rs` used as
 *                the parity oracle (every float input is the f32 value the reference computes
 *                with; the arithmetic after it runs in f64);
 *  - or_cpuref_*: the reference's `Cpu(Reference)` op sequence in f32 (same op order,
 *                materialised [rows, V] intermediates, glibc expf/logf), used for the timed
 *                CPU baseline and for comparing against the reference's own f32 rounding.
 *
 * Parity pins (the tests that check each function) are listed in tests/test_oracle.py. The
 * inverse-CDF sampler has no reference definition (the reference samples by Gumbel-max); it
 * is pinned by brute force on tiny rows and by the reference's frequency test.
 */
#ifndef NOETIC_ORACLE_H
#define NOETIC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- hashing and seeded streams (src/hash.rs, src/rng.rs) ---------------------------- */

/* SHA-256 (FIPS 180-4), as sha2 0.10.9 computes it (src/hash.rs:6-7). */
void or_sha256(const uint8_t *data, size_t len, uint8_t out[32]);

/* ChaCha20Rng of rand_chacha 0.3.1: 20 rounds, 256-bit key = the seed, 64-bit block counter
 * in state words 12-13 starting at 0, 64-bit stream id 0 in words 14-15, keystream consumed
 * as consecutive little-endian u32 words; next_u64 = lo | hi << 32 of the next two words. */
typedef struct {
    uint32_t key[8];
    uint64_t counter; /* the next block to generate */
    uint32_t buf[16];
    int idx; /* next unread word of buf; 16 = empty */
} or_chacha;

void or_chacha_block(const uint32_t key[8], uint64_t counter, uint64_t stream, uint32_t out[16]);
void or_chacha_block_rounds(const uint32_t key[8], uint64_t counter, uint64_t stream, int rounds, uint32_t out[16]);
void or_seed_from_u64(uint64_t state, uint64_t inc, uint8_t seed[32]);
void or_reference_rnd_f32(uint64_t seed, uint64_t inc, int64_t n, float lo, float hi, float *out);
void or_reference_rnd_f64(uint64_t seed, uint64_t inc, int64_t n, double lo, double hi, double *out);
/* One f32 product in the reference's matmul order: fmaf chains over k closed every 256. */
void or_matmul_f32(const float *a, int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs, int64_t b_cs,
                   int64_t m, int64_t k, int64_t n, float *c);
void or_chacha_seed(or_chacha *r, const uint8_t seed[32]);
/* rng::derive(root, label): ChaCha20Rng::from_seed(SHA-256(root.to_le_bytes() || label))
 * (src/rng.rs:9-17). */
void or_rng_derive(or_chacha *r, uint64_t root, const char *label, size_t label_len);
uint32_t or_chacha_next_u32(or_chacha *r);
uint64_t or_chacha_next_u64(or_chacha *r);
/* The reference's uniform on the open interval (0,1): ((k >> 11) + 0.5) / 2^53
 * (src/nn/rl.rs:493-494). */
double or_uniform_open01(uint64_t k);
/* n uniforms, one next_u64 each, in order. */
void or_rng_uniforms(or_chacha *r, size_t n, double *out);
/* rand 0.8 `gen::<f64>()` ((k >> 11) * 2^-53) and the Box-Muller normal of
 * src/nn/init.rs:28-37: two draws per value, cos branch. */
double or_rng_gen_f64(or_chacha *r);
double or_rng_normal(or_chacha *r);

/* ---- bf16 (src/tensor/half.rs:16-27) --------------------------------------------------- */
uint16_t or_bf16_from_f32(float x);
float or_bf16_to_f32(uint16_t b);

/* ---- tempered logits (src/nn/rl.rs:475-486, float.rs:494-499) -------------------------- */
/* z = x / (float)tau (skipped at tau == 1) + mask. Exactly one of addmask (an additive f32
 * mask row, length V) or keep (a u8 row: 0 excludes the token, i.e. adds -inf) may be
 * non-NULL. f32 arithmetic, as the reference computes f32 and bf16 tensors. */
void or_tempered_row(const float *x, int64_t V, double tau, const float *addmask,
                     const uint8_t *keep, float *z);

/* ---- f64 row oracle ------------------------------------------------------------------ */
typedef struct {
    double m;    /* first maximum of z (NaN if the row holds a NaN) */
    double S;    /* sum_v exp(z_v - m) */
    double lse;  /* m + ln S */
    int64_t argmax; /* first index of the maximum (reference argmax_dim, kernels.rs:184-209) */
    int status;  /* 0 ok, 1 every entry -inf, 2 NaN (rl.rs:516-519) */
} or_rowstats;

or_rowstats or_row_stats(const float *z, int64_t V);
/* log_softmax(z)[tok] (rl.rs:134-141, activation.rs:30-42) in f64. */
double or_token_logp(const float *z, int64_t V, int64_t tok);
/* H = -sum p log p, terms with log p == -inf give 0 (rl.rs:405-414). */
double or_entropy(const float *z, int64_t V);
/* KL(softmax z || softmax r) = sum p (log p - log r), terms with log p == -inf give 0
 * (rl.rs:327-338). */
double or_kl(const float *z, const float *r, int64_t V);
/* The gradient with respect to z of g_lp * logp(tok) + g_kl * KL(softmax z || softmax r) +
 * g_h * H(softmax z) for one row, in f64 (the reference's autograd through log_softmax
 * activation.rs:36-41, gather, categorical_kl rl.rs:327-338 with r detached, and
 * categorical_entropy rl.rs:405-414): out_v = [v == tok] g_lp - pi_v (g_lp + g_kl (KL -
 * (log pi_v - log pi_r,v)) + g_h (log pi_v + H)), 0 softmax term where pi_v = 0. r may be NULL
 * when g_kl is 0; tok < 0 means no token term. Returns 0, or -1 for a refused row (out NaN). */
int or_score_grad_row(const float *z, const float *r, int64_t V, int64_t tok, double g_lp, double g_kl, double g_h,
                      double *out);

/* The inverse-CDF sampler (the build's definition; the reference's sampler is Gumbel-max):
 * with w_v = exp(z_v - m) and S = sum w, return min{v : sum_{j<=v} w_j > u*S}; if rounding
 * leaves no crossing, the last v with w_v > 0. temperature 0 (greedy) is the first argmax.
 * *edge (optional) = min |u - F| over the two CDF edges around the chosen token, F = C/S. */
int64_t or_sample_invcdf(const float *z, int64_t V, double u, double *edge);

/* k1/k2/k3 of rl.rs:380-400 on per-token values: delta = lr - lp, zeroed where mask == 0,
 * clamped to [-clamp, clamp] when clamp > 0; est 1, 2, 3. mask may be NULL (all scored). */
void or_kl_estimate(const double *lp, const double *lr, const double *mask, int64_t n, int est,
                    double clamp, double *out);

/* reduce_tokens (rl.rs:69-92) of per-token values [S,B,T] (already zero at masked positions):
 * reduction 0 None, 1 Sum [S], 2 TokenMean [S], 3 PerSequence [S,B], 4 SequenceMean [S].
 * Returns the number of outputs written. */
int64_t or_reduce_tokens(const double *per, const double *mask, int64_t S, int64_t B, int64_t T,
                         int reduction, double *out);

/* group_advantages (rl.rs:436-463): norm 0 MeanOnly, 1 Std. Returns 0, or -1 for an invalid
 * call (groups of n must divide len; eps >= 0; unbiased needs n >= 2). */
void or_policy_loss(int kind, int64_t n, int64_t T, const double *lp, const double *old, const double *w,
                    int per_seq, const double *mask, double low, double high, double dual, double clamp,
                    double *loss, double *dloss, double *hit);
void or_reduce_tokens_backward(const double *mask, int64_t S, int64_t B, int64_t T, int reduction, const double *up,
                               double scale, const double *local, double *out);
void or_kl_estimate_grad(const double *lp, const double *lr, const double *mask, int64_t n, int est, double clamp,
                         double *out);
int or_group_advantages(const double *rewards, int64_t len, int64_t n, int norm, double eps,
                        int unbiased, double *out);

/* ---- Cpu(Reference) op sequence in f32 (the timed CPU baseline) ---------------------- */
/* ndarray's 8-partial unrolled sum (kernels.rs:122-148). */
double or_unrolled_sum_f64(const double *x, int64_t n);
void or_cpuref_log_softmax_f64(const double *x, int64_t rows, int64_t V, double *y);
float or_unrolled_sum_f32(const float *x, int64_t n);
/* log_softmax along the last axis, in the reference's op order with materialised
 * intermediates: max_dim, x - max, exp, sum_dim, log, shifted - lse (activation.rs:30-42). */
void or_cpuref_log_softmax(const float *x, int64_t rows, int64_t V, float *y);
/* The reference's sample_categorical (rl.rs:510-529) followed by token_log_probs of the
 * tempered logits at the sampled ids, on Cpu(Reference): tempered_logits, max_dim check,
 * one Gumbel draw per logit from the stream, argmax, log_softmax, gather. x: [rows, V] f32
 * (bf16 inputs pass their exact f32 values). keep: u8 [rows or 1, V] or NULL (keep_ld 0 =
 * shared row). Returns 0, or 1 + the first refused row. */
int64_t or_cpuref_sample_logp(const float *x, int64_t rows, int64_t V, double tau,
                              const uint8_t *keep, int64_t keep_ld, or_chacha *rng,
                              int64_t *ids, float *logp);
/* sample_categorical alone (rl.rs:510-529) on Cpu(Reference), with either mask form: addmask
 * is an additive f32 mask [rows or 1, V] (add_ld 0 = one shared row), keep a u8 keep-mask
 * (0 = -inf). The refusal check (first maximum NaN or -inf, rl.rs:515-519) runs before any
 * draw, so a refused call leaves the stream untouched. Returns 0, or 1 + the first refused row. */
int64_t or_cpuref_sample_gumbel(const float *x, int64_t rows, int64_t V, double tau, const float *addmask,
                                int64_t add_ld, const uint8_t *keep, int64_t keep_ld, or_chacha *rng, int64_t *ids);
/* The same sequence (sample_categorical, then token_log_probs) on the reference's Cpu(Fast)
 * backend (src/tensor/backend.rs:57-239) with `threads` workers: threaded maps from 2^20
 * elements, equal-shape zips from 2^22, last-axis sums from 2^22 by 16 accumulators; the rest
 * as Cpu(Reference). The tokens equal or_cpuref_sample_logp's for the same stream; a log-prob may
 * differ in its last bits (the sum order). The timed Cpu(Fast) baseline. */
int64_t or_cpufast_sample_logp(const float *x, int64_t rows, int64_t V, double tau, const uint8_t *keep,
                               int64_t keep_ld, or_chacha *rng, int threads, int64_t *ids, float *logp);
/* The same sequence with the inverse-CDF draw in place of Gumbel-max (one uniform per row),
 * still unfused and in f32 where the reference is f32: the "port" CPU baseline of the fused
 * path. threads > 1 splits rows across pthreads (Cpu(Fast)-style, backend.rs:59-72). */
int64_t or_cpu_sample_logp_invcdf(const float *x, int64_t rows, int64_t V, double tau,
                                  const uint8_t *keep, int64_t keep_ld, const double *u,
                                  int64_t *ids, float *logp, int threads);

#ifdef __cplusplus
}
#endif
#endif
