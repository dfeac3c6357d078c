// The ChaCha20 block function on the device, as rand_chacha 0.3.1's ChaCha20Rng lays out its
// state (the stream behind rng::derive, src/rng.rs:9-17): "expand 32-byte k", the 256-bit key,
// a 64-bit block counter in words 12-13 and the 64-bit stream id 0 in words 14-15; 10 double
// rounds; the keystream is the 16 output words in order. Word w of the stream is word w % 16
// of block w / 16, so any position is reached without generating what comes before it.
#pragma once

#ifndef __HIPCC_RTC__  // (hiprtc: the device part of the library's headers, stdint from nt_rows.hpp)
#include <hip/hip_runtime.h>

#include <cstdint>
#endif

namespace nt {

struct ChachaKey {
    uint32_t k[8];
};

__device__ __forceinline__ uint32_t chacha_rotl(uint32_t x, int n) { return (x << n) | (x >> (32 - n)); }

// Block `counter` of the keystream keyed by `key` (stream id 0), into out[16].
__device__ __forceinline__ void chacha_block_dev(const ChachaKey &key, uint64_t counter, uint32_t out[16]) {
    const uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
                            key.k[0], key.k[1], key.k[2], key.k[3], key.k[4], key.k[5], key.k[6], key.k[7],
                            uint32_t(counter), uint32_t(counter >> 32), 0u, 0u};
    uint32_t x[16];
#pragma unroll
    for (int i = 0; i < 16; i++) x[i] = s[i];
#define NT_QR(a, b, c, d)                                   \
    x[a] += x[b]; x[d] = chacha_rotl(x[d] ^ x[a], 16);      \
    x[c] += x[d]; x[b] = chacha_rotl(x[b] ^ x[c], 12);      \
    x[a] += x[b]; x[d] = chacha_rotl(x[d] ^ x[a], 8);       \
    x[c] += x[d]; x[b] = chacha_rotl(x[b] ^ x[c], 7);
    for (int r = 0; r < 10; r++) {
        NT_QR(0, 4, 8, 12) NT_QR(1, 5, 9, 13) NT_QR(2, 6, 10, 14) NT_QR(3, 7, 11, 15)
        NT_QR(0, 5, 10, 15) NT_QR(1, 6, 11, 12) NT_QR(2, 7, 8, 13) NT_QR(3, 4, 9, 14)
    }
#undef NT_QR
#pragma unroll
    for (int i = 0; i < 16; i++) out[i] = x[i] + s[i];
}

}  // namespace nt
