/*
 * noetic_synth.h — synthetic workload generators of libnoetic_hip.so.
 *
 * No counterpart in the reference: these fill device buffers with the seeded synthetic inputs
 * of the benchmark configurations (normal logits, spikes, Zipf rank biases, Bernoulli and
 * run-structured vocabulary masks, target tokens), so that multi-GB inputs are generated on
 * the GPU instead of uploaded. Every value is a function of a ChaCha20 stream
 * (nt_rng_derive's key) and the element index only, so a generator is reproducible.
 *
 * Stream layout: for a stream keyed by `key`, keystream u32 word i is word i % 16 of ChaCha20
 * block i / 16 (block counter = i / 16, stream id 0), i.e. the same words a sequential
 * ChaCha20Rng(key) returns. Normal value i uses u64 draws 2i and 2i+1 with the Box-Muller
 * convention of src/nn/init.rs:28-37: u1 = max((k1 >> 11) 2^-53, 1e-300), u2 = (k2 >> 11) 2^-53,
 * z = sqrt(-2 ln u1) cos(2 pi u2).
 */
#ifndef NOETIC_SYNTH_H
#define NOETIC_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct NtSynthNormal {
    void *out;            /* [rows, V] contiguous, f32 or bf16 (NT_F32 / NT_BF16) */
    int32_t dtype;
    int64_t rows, vocab;
    uint32_t key[8];      /* value stream */
    double mean, std;     /* out = mean + std * z (+ bias) */
    double zipf_s;        /* > 0: add -zipf_s * ln(1 + ((v + rot_r) mod V)), rot_r = u64 draw r of
                             rot_key's stream mod V (a Zipf(s) rank bias, per-row rotation) */
    uint32_t rot_key[8];
    const void *base;     /* NULL, or [rows, V] of `dtype`: out = round(base + std * z) */
} NtSynthNormal;
int nt_synth_normal(const NtSynthNormal *a);

/* Add `value` to k distinct tokens of each row: token j of row r is (b_r + j * (V / k)) mod V,
 * b_r = u64 draw r of key's stream mod V. x: [rows, V] contiguous f32 or bf16. */
int nt_synth_spikes(void *x, int32_t dtype, int64_t rows, int64_t vocab, int32_t k, const uint32_t key[8],
                    double value);

/* u8 Bernoulli(p) keep-mask: byte i = (u32 word i < p * 2^32). */
int nt_synth_bernoulli_mask(uint8_t *out, int64_t n, const uint32_t key[8], double p);

/* Tokens uniform in [0, V): token i = u64 draw i mod V. */
int nt_synth_tokens(int32_t *out, int64_t n, const uint32_t key[8], int64_t vocab);

/* Set mask[r, tokens[r]] = 1 for every row (a scored token is always allowed; it also keeps
 * at least one token per row). */
int nt_synth_keep_tokens(uint8_t *mask, int64_t rows, int64_t mask_ld, const int32_t *tokens);

/* HOST function: a grammar-like u8 keep-mask [rows, V] of contiguous allowed runs. Each row
 * alternates kept and excluded runs with lengths uniform in [1, 2*mean_kept - 1] and
 * [1, 2*mean_gap - 1], starting with a gap of random phase; at least one token per row is kept.
 * Draws come from rng::derive(root, label) in row order. out is host memory. */
int nt_synth_runs_mask_host(uint8_t *out, int64_t rows, int64_t vocab, uint64_t root, const char *label,
                            size_t label_len, int32_t mean_kept, int32_t mean_gap);

#ifdef __cplusplus
}
#endif
#endif
