// The product's seeded host streams: SHA-256 and ChaCha20Rng as rng::derive uses them
// (src/rng.rs:9-17, src/hash.rs:6-7). Host-only code; it runs without a GPU.
#include <array>
#include <cstring>
#include <vector>

#include "../../include/noetic_rng.h"

namespace {

constexpr std::array<uint32_t, 64> kRound = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
    0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
    0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
    0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
    0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
    0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

inline uint32_t ror(uint32_t x, unsigned n) { return (x >> n) | (x << (32u - n)); }
inline uint32_t rol(uint32_t x, unsigned n) { return (x << n) | (x >> (32u - n)); }

class Sha256 {
  public:
    void update(const uint8_t *p, size_t n) {
        total_ += n;
        while (n > 0) {
            size_t take = std::min(n, sizeof(block_) - fill_);
            std::memcpy(block_ + fill_, p, take);
            fill_ += take;
            p += take;
            n -= take;
            if (fill_ == sizeof(block_)) {
                compress(block_);
                fill_ = 0;
            }
        }
    }
    void finish(uint8_t out[32]) {
        uint64_t bits = total_ * 8u;
        uint8_t pad = 0x80;
        update(&pad, 1);
        uint8_t zero = 0;
        while (fill_ != 56) update(&zero, 1);
        uint8_t len[8];
        for (int i = 0; i < 8; i++) len[i] = uint8_t(bits >> (56 - 8 * i));
        update(len, 8);
        for (int i = 0; i < 8; i++)
            for (int b = 0; b < 4; b++) out[4 * i + b] = uint8_t(h_[i] >> (24 - 8 * b));
    }

  private:
    void compress(const uint8_t *blk) {
        uint32_t w[64];
        for (int i = 0; i < 16; i++)
            w[i] = uint32_t(blk[4 * i]) << 24 | uint32_t(blk[4 * i + 1]) << 16 | uint32_t(blk[4 * i + 2]) << 8 |
                   uint32_t(blk[4 * i + 3]);
        for (int i = 16; i < 64; i++)
            w[i] = w[i - 16] + (ror(w[i - 15], 7) ^ ror(w[i - 15], 18) ^ (w[i - 15] >> 3)) + w[i - 7] +
                   (ror(w[i - 2], 17) ^ ror(w[i - 2], 19) ^ (w[i - 2] >> 10));
        std::array<uint32_t, 8> v;
        std::copy(h_, h_ + 8, v.begin());
        for (int i = 0; i < 64; i++) {
            uint32_t t1 = v[7] + (ror(v[4], 6) ^ ror(v[4], 11) ^ ror(v[4], 25)) + ((v[4] & v[5]) ^ (~v[4] & v[6])) +
                          kRound[i] + w[i];
            uint32_t t2 = (ror(v[0], 2) ^ ror(v[0], 13) ^ ror(v[0], 22)) + ((v[0] & v[1]) ^ (v[0] & v[2]) ^ (v[1] & v[2]));
            for (int k = 7; k > 0; k--) v[k] = v[k - 1];
            v[4] += t1;
            v[0] = t1 + t2;
        }
        for (int i = 0; i < 8; i++) h_[i] += v[i];
    }
    uint32_t h_[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                      0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    uint8_t block_[64];
    size_t fill_ = 0;
    uint64_t total_ = 0;
};

// One ChaCha20 block: "expand 32-byte k", key, 64-bit counter, 64-bit stream 0; 10 double rounds.
void chacha_block(const uint32_t key[8], uint64_t counter, uint32_t out[16]) {
    uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
    for (int i = 0; i < 8; i++) in[4 + i] = key[i];
    in[12] = uint32_t(counter);
    in[13] = uint32_t(counter >> 32);
    in[14] = 0;
    in[15] = 0;
    uint32_t x[16];
    std::memcpy(x, in, sizeof x);
    auto quarter = [&x](int a, int b, int c, int d) {
        x[a] += x[b]; x[d] = rol(x[d] ^ x[a], 16);
        x[c] += x[d]; x[b] = rol(x[b] ^ x[c], 12);
        x[a] += x[b]; x[d] = rol(x[d] ^ x[a], 8);
        x[c] += x[d]; x[b] = rol(x[b] ^ x[c], 7);
    };
    for (int round = 0; round < 10; round++) {
        quarter(0, 4, 8, 12); quarter(1, 5, 9, 13); quarter(2, 6, 10, 14); quarter(3, 7, 11, 15);
        quarter(0, 5, 10, 15); quarter(1, 6, 11, 12); quarter(2, 7, 8, 13); quarter(3, 4, 9, 14);
    }
    for (int i = 0; i < 16; i++) out[i] = x[i] + in[i];
}

}  // namespace

extern "C" {

int nt_sha256(const void *data, size_t len, uint8_t out[32]) {
    if (!out || (!data && len)) return -1;
    Sha256 h;
    h.update(static_cast<const uint8_t *>(data), len);
    h.finish(out);
    return 0;
}

int nt_rng_from_seed(NtRng *r, const uint8_t seed[32]) {
    if (!r || !seed) return -1;
    for (int i = 0; i < 8; i++)
        r->key[i] = uint32_t(seed[4 * i]) | uint32_t(seed[4 * i + 1]) << 8 | uint32_t(seed[4 * i + 2]) << 16 |
                    uint32_t(seed[4 * i + 3]) << 24;
    r->counter = 0;
    r->idx = 16;
    std::memset(r->buf, 0, sizeof r->buf);
    return 0;
}

int nt_rng_derive(NtRng *r, uint64_t root, const char *label, size_t label_len) {
    if (!r || (!label && label_len)) return -1;
    uint8_t le[8];
    for (int i = 0; i < 8; i++) le[i] = uint8_t(root >> (8 * i));
    Sha256 h;
    h.update(le, 8);
    h.update(reinterpret_cast<const uint8_t *>(label), label_len);
    uint8_t seed[32];
    h.finish(seed);
    return nt_rng_from_seed(r, seed);
}

uint32_t nt_rng_next_u32(NtRng *r) {
    if (r->idx >= 16) {
        chacha_block(r->key, r->counter++, r->buf);
        r->idx = 0;
    }
    return r->buf[r->idx++];
}

uint64_t nt_rng_next_u64(NtRng *r) {
    uint64_t lo = nt_rng_next_u32(r);
    return lo | uint64_t(nt_rng_next_u32(r)) << 32;
}

int nt_rng_word_pos(const NtRng *r, uint64_t *block, int32_t *word) {
    if (!r || !block || !word || r->idx < 0 || r->idx > 16) return -1;
    // buf holds block counter - 1 and idx is its next unread word; idx 16 (empty) is word 0 of
    // block counter.
    if (r->idx == 16) {
        *block = r->counter;
        *word = 0;
    } else {
        *block = r->counter - 1;
        *word = r->idx;
    }
    return 0;
}

int nt_rng_set_word_pos(NtRng *r, uint64_t block, int32_t word) {
    if (!r || word < 0 || word > 15) return -1;
    if (word == 0) {
        r->counter = block;
        r->idx = 16;
    } else {
        chacha_block(r->key, block, r->buf);
        r->counter = block + 1;
        r->idx = word;
    }
    return 0;
}

int nt_rng_skip_u64(NtRng *r, uint64_t n) {
    uint64_t block;
    int32_t word;
    if (nt_rng_word_pos(r, &block, &word)) return -1;
    // 2n words past (block, word); n < 2^63
    const uint64_t w = uint64_t(word) + 2 * (n % 8);
    return nt_rng_set_word_pos(r, block + n / 8 + w / 16, int32_t(w % 16));
}

int nt_rng_uniforms(NtRng *r, size_t n, double *out) {
    if (!r || (!out && n)) return -1;
    for (size_t i = 0; i < n; i++) out[i] = (double(nt_rng_next_u64(r) >> 11) + 0.5) * 0x1p-53;
    return 0;
}

}  // extern "C"
