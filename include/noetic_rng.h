/*
 * noetic_rng.h — the seeded host streams of libnoetic_hip.so (no GPU needed).
 *
 * The fused sampler reads one uniform per row drawn on the host from an engine stream, as the
 * reference draws its Gumbel noise on the host (src/nn/rl.rs:488-498): these functions are
 * the stream. They replace `rng::derive` (src/rng.rs:9-17) and the `next_u64` calls of
 * rand_chacha 0.3.1's ChaCha20Rng (src/nn/rl.rs:493).
 */
#ifndef NOETIC_RNG_H
#define NOETIC_RNG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ChaCha20Rng state: 256-bit key, 64-bit block counter (state words 12-13), stream 0
 * (words 14-15), the current block's 16 keystream words and the next unread word. */
typedef struct NtRng {
    uint32_t key[8];
    uint64_t counter;
    uint32_t buf[16];
    int32_t idx;
} NtRng;

/* rng::derive(root, label): seed = SHA-256(root.to_le_bytes() || label) (src/rng.rs:9-17). */
int nt_rng_derive(NtRng *r, uint64_t root, const char *label, size_t label_len);
/* ChaCha20Rng::from_seed(seed). */
int nt_rng_from_seed(NtRng *r, const uint8_t seed[32]);
uint32_t nt_rng_next_u32(NtRng *r);
uint64_t nt_rng_next_u64(NtRng *r);
/* n uniforms on (0,1), one next_u64 each: ((k >> 11) + 0.5) / 2^53 (src/nn/rl.rs:493-494). */
int nt_rng_uniforms(NtRng *r, size_t n, double *out);
/* The stream's word position, rand_chacha 0.3.1's `get_word_pos` in two parts: the next unread
 * keystream word is word `*word` (0..15) of block `*block`. The Gumbel sampler
 * (nt_hip_rl_sample_gumbel) takes this position and generates the draws on the device. */
int nt_rng_word_pos(const NtRng *r, uint64_t *block, int32_t *word);
/* rand_chacha's `set_word_pos`: move the stream to word `word` (0..15) of block `block`. */
int nt_rng_set_word_pos(NtRng *r, uint64_t block, int32_t word);
/* Advance the stream by n u64 draws (2n keystream words) without handing them out: the state
 * after n calls of nt_rng_next_u64 (the reference's sampler consumes one u64 per logit,
 * src/nn/rl.rs:490-498, src/nn/tests/rl.rs:596-599). */
int nt_rng_skip_u64(NtRng *r, uint64_t n);
/* SHA-256 of data (src/hash.rs:6-7). */
int nt_sha256(const void *data, size_t len, uint8_t out[32]);

#ifdef __cplusplus
}
#endif
#endif
