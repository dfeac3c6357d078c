/*
 * CPU oracle for the nn::rl vocabulary-row hot path. TEST INFRASTRUCTURE ONLY: the product
 * never links or calls it (see oracle.h). Citations are to shyble/noetic-tensor 0.7.0.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ===================================================================== SHA-256 (FIPS 180-4)
 * sha2 0.10.9, called by rng::derive (src/rng.rs:10-13) and hash::sha256_hex (src/hash.rs:6). */
static const uint32_t K256[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u,
    0xab1c5ed5u, 0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu,
    0x9bdc06a7u, 0xc19bf174u, 0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu,
    0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau, 0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u,
    0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u, 0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu,
    0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u, 0xa2bfe8a1u, 0xa81a664bu,
    0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u, 0x19a4c116u,
    0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
    0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u,
    0xc67178f2u};

static uint32_t rotr32(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static void sha256_compress(uint32_t h[8], const uint8_t blk[64]) {
    uint32_t w[64];
    for (int i = 0; i < 16; i++)
        w[i] = ((uint32_t)blk[4 * i] << 24) | ((uint32_t)blk[4 * i + 1] << 16) |
               ((uint32_t)blk[4 * i + 2] << 8) | (uint32_t)blk[4 * i + 3];
    for (int i = 16; i < 64; i++) {
        uint32_t s0 = rotr32(w[i - 15], 7) ^ rotr32(w[i - 15], 18) ^ (w[i - 15] >> 3);
        uint32_t s1 = rotr32(w[i - 2], 17) ^ rotr32(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int i = 0; i < 64; i++) {
        uint32_t S1 = rotr32(e, 6) ^ rotr32(e, 11) ^ rotr32(e, 25);
        uint32_t ch = (e & f) ^ (~e & g);
        uint32_t t1 = hh + S1 + ch + K256[i] + w[i];
        uint32_t S0 = rotr32(a, 2) ^ rotr32(a, 13) ^ rotr32(a, 22);
        uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
        uint32_t t2 = S0 + mj;
        hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
}

void or_sha256(const uint8_t *data, size_t len, uint8_t out[32]) {
    uint32_t h[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                     0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    size_t full = len / 64;
    for (size_t i = 0; i < full; i++) sha256_compress(h, data + 64 * i);
    uint8_t tail[128];
    size_t rem = len - 64 * full;
    memset(tail, 0, sizeof tail);
    memcpy(tail, data + 64 * full, rem);
    tail[rem] = 0x80;
    size_t tl = (rem + 1 + 8 <= 64) ? 64 : 128;
    uint64_t bits = (uint64_t)len * 8u;
    for (int i = 0; i < 8; i++) tail[tl - 1 - i] = (uint8_t)(bits >> (8 * i));
    sha256_compress(h, tail);
    if (tl == 128) sha256_compress(h, tail + 64);
    for (int i = 0; i < 8; i++) {
        out[4 * i] = (uint8_t)(h[i] >> 24);
        out[4 * i + 1] = (uint8_t)(h[i] >> 16);
        out[4 * i + 2] = (uint8_t)(h[i] >> 8);
        out[4 * i + 3] = (uint8_t)h[i];
    }
}

/* ===================================================================== ChaCha20 (RFC 8439 core)
 * rand_chacha 0.3.1's ChaCha20Rng (Cargo.lock:155-161), used through rng::derive (src/rng.rs:16)
 * and next_u64 (src/nn/rl.rs:493). */
#define QR(a, b, c, d)                                                                     \
    a += b; d ^= a; d = (d << 16) | (d >> 16);                                             \
    c += d; b ^= c; b = (b << 12) | (b >> 20);                                             \
    a += b; d ^= a; d = (d << 8) | (d >> 24);                                              \
    c += d; b ^= c; b = (b << 7) | (b >> 25);

/* The block function with `rounds` rounds (20 for ChaCha20Rng, 8 for ChaCha8Rng). */
void or_chacha_block_rounds(const uint32_t key[8], uint64_t counter, uint64_t stream, int rounds, uint32_t out[16]) {
    uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
    for (int i = 0; i < 8; i++) s[4 + i] = key[i];
    s[12] = (uint32_t)counter;
    s[13] = (uint32_t)(counter >> 32);
    s[14] = (uint32_t)stream;
    s[15] = (uint32_t)(stream >> 32);
    uint32_t x[16];
    memcpy(x, s, sizeof x);
    for (int r = 0; r < rounds / 2; r++) {
        QR(x[0], x[4], x[8], x[12]);
        QR(x[1], x[5], x[9], x[13]);
        QR(x[2], x[6], x[10], x[14]);
        QR(x[3], x[7], x[11], x[15]);
        QR(x[0], x[5], x[10], x[15]);
        QR(x[1], x[6], x[11], x[12]);
        QR(x[2], x[7], x[8], x[13]);
        QR(x[3], x[4], x[9], x[14]);
    }
    for (int i = 0; i < 16; i++) out[i] = x[i] + s[i];
}

void or_chacha_block(const uint32_t key[8], uint64_t counter, uint64_t stream, uint32_t out[16]) {
    or_chacha_block_rounds(key, counter, stream, 20, out);
}

void or_chacha_seed(or_chacha *r, const uint8_t seed[32]) {
    for (int i = 0; i < 8; i++)
        r->key[i] = (uint32_t)seed[4 * i] | ((uint32_t)seed[4 * i + 1] << 8) |
                    ((uint32_t)seed[4 * i + 2] << 16) | ((uint32_t)seed[4 * i + 3] << 24);
    r->counter = 0;
    r->idx = 16;
}

void or_rng_derive(or_chacha *r, uint64_t root, const char *label, size_t label_len) {
    size_t n = 8 + label_len;
    uint8_t *msg = (uint8_t *)malloc(n);
    for (int i = 0; i < 8; i++) msg[i] = (uint8_t)(root >> (8 * i)); /* root.to_le_bytes() */
    memcpy(msg + 8, label, label_len);
    uint8_t digest[32];
    or_sha256(msg, n, digest);
    free(msg);
    or_chacha_seed(r, digest);
}

uint32_t or_chacha_next_u32(or_chacha *r) {
    if (r->idx >= 16) {
        or_chacha_block(r->key, r->counter, 0, r->buf);
        r->counter++;
        r->idx = 0;
    }
    return r->buf[r->idx++];
}

uint64_t or_chacha_next_u64(or_chacha *r) {
    uint64_t lo = or_chacha_next_u32(r);
    uint64_t hi = or_chacha_next_u32(r);
    return lo | (hi << 32);
}

double or_uniform_open01(uint64_t k) { return ((double)(k >> 11) + 0.5) / 9007199254740992.0; }

void or_rng_uniforms(or_chacha *r, size_t n, double *out) {
    for (size_t i = 0; i < n; i++) out[i] = or_uniform_open01(or_chacha_next_u64(r));
}

double or_rng_gen_f64(or_chacha *r) {
    return (double)(or_chacha_next_u64(r) >> 11) * (1.0 / 9007199254740992.0);
}

double or_rng_normal(or_chacha *r) {
    double u1 = or_rng_gen_f64(r);
    if (u1 < 1e-300) u1 = 1e-300;
    double u2 = or_rng_gen_f64(r);
    return sqrt(-2.0 * log(u1)) * cos(2.0 * 3.14159265358979323846 * u2);
}

/* ===================================================================== bf16 (half.rs:16-27) */
uint16_t or_bf16_from_f32(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    if (x != x) return (uint16_t)((b >> 16) | 0x0040u);
    uint32_t round = 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)((b + round) >> 16);
}

float or_bf16_to_f32(uint16_t h) {
    uint32_t b = (uint32_t)h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* ===================================================================== tempered logits
 * rl.rs:475-486: z = logits / temperature (skipped at exactly 1) + mask; the divide is
 * `a / (tau as f32)` in f32 (float.rs:494-499). A u8 keep-mask excludes with -inf. */
void or_tempered_row(const float *x, int64_t V, double tau, const float *addmask,
                     const uint8_t *keep, float *z) {
    float t = (float)tau;
    for (int64_t v = 0; v < V; v++) {
        float a = (tau == 1.0) ? x[v] : x[v] / t;
        if (addmask) a = a + addmask[v];
        if (keep && keep[v] == 0) a = -INFINITY;
        z[v] = a;
    }
}

/* ===================================================================== f64 row oracle */
or_rowstats or_row_stats(const float *z, int64_t V) {
    or_rowstats s;
    /* First maximum, NaN-propagating (kernels.rs:184-209). */
    float best = z[0];
    int64_t idx = 0;
    for (int64_t k = 0; k < V; k++) {
        float e = z[k];
        if (best != best) break;
        if (e != e || e > best) {
            best = e;
            idx = k;
        }
    }
    s.m = (double)best;
    s.argmax = idx;
    s.status = (best != best) ? 2 : (best == -INFINITY ? 1 : 0);
    double S = 0.0;
    if (s.status == 0)
        for (int64_t v = 0; v < V; v++) S += exp((double)z[v] - s.m);
    s.S = (s.status == 0) ? S : NAN;
    s.lse = s.m + log(s.S);
    return s;
}

double or_token_logp(const float *z, int64_t V, int64_t tok) {
    or_rowstats s = or_row_stats(z, V);
    if (s.status != 0) return NAN;
    if (z[tok] == -INFINITY) return -INFINITY;
    return ((double)z[tok] - s.m) - log(s.S);
}

double or_entropy(const float *z, int64_t V) {
    or_rowstats s = or_row_stats(z, V);
    if (s.status != 0) return NAN;
    double ls = log(s.S), h = 0.0;
    for (int64_t v = 0; v < V; v++) {
        if (z[v] == -INFINITY) continue; /* log p == -inf: a zero term (rl.rs:409-411) */
        double lp = ((double)z[v] - s.m) - ls;
        h -= exp(lp) * lp;
    }
    return h;
}

double or_kl(const float *z, const float *r, int64_t V) {
    or_rowstats sp = or_row_stats(z, V), sr = or_row_stats(r, V);
    if (sp.status != 0 || sr.status != 0) return NAN;
    double lsp = log(sp.S), lsr = log(sr.S), kl = 0.0;
    for (int64_t v = 0; v < V; v++) {
        if (z[v] == -INFINITY) continue; /* the mask_fill of rl.rs:333-334 */
        double lp = ((double)z[v] - sp.m) - lsp;
        double lr = (r[v] == -INFINITY) ? -INFINITY : ((double)r[v] - sr.m) - lsr;
        kl += exp(lp) * (lp - lr);
    }
    return kl;
}

int or_score_grad_row(const float *z, const float *r, int64_t V, int64_t tok, double g_lp, double g_kl, double g_h,
                      double *out) {
    or_rowstats sp = or_row_stats(z, V);
    if (sp.status != 0 || (g_kl != 0.0 && !r)) {
        for (int64_t v = 0; v < V; v++) out[v] = NAN;
        return -1;
    }
    const double lsp = log(sp.S);
    double kl = 0.0, h = 0.0, lsr = 0.0;
    or_rowstats sr = {0};
    if (g_kl != 0.0) {
        sr = or_row_stats(r, V);
        if (sr.status != 0) {
            for (int64_t v = 0; v < V; v++) out[v] = NAN;
            return -1;
        }
        lsr = log(sr.S);
        kl = or_kl(z, r, V);
    }
    if (g_h != 0.0) h = or_entropy(z, V);
    for (int64_t v = 0; v < V; v++) {
        double g = (v == tok) ? g_lp : 0.0;
        if (z[v] != -INFINITY) {
            const double lp = ((double)z[v] - sp.m) - lsp;
            const double pi = exp(lp);
            if (pi > 0.0) {
                double t = g_lp;
                if (g_kl != 0.0) {
                    const double lr = (r[v] == -INFINITY) ? -INFINITY : ((double)r[v] - sr.m) - lsr;
                    t += g_kl * (kl - (lp - lr));
                }
                if (g_h != 0.0) t += g_h * (lp + h);
                g -= pi * t;
            }
        }
        out[v] = g;
    }
    return 0;
}

int64_t or_sample_invcdf(const float *z, int64_t V, double u, double *edge) {
    or_rowstats s = or_row_stats(z, V);
    if (s.status != 0) {
        if (edge) *edge = NAN;
        return -1;
    }
    double S = 0.0;
    for (int64_t v = 0; v < V; v++) S += exp((double)z[v] - s.m);
    double t = u * S, C = 0.0;
    int64_t last = -1;
    for (int64_t v = 0; v < V; v++) {
        double w = exp((double)z[v] - s.m);
        if (w > 0.0) last = v;
        double prev = C;
        C += w;
        if (C > t) {
            if (edge) {
                double a = fabs(u - prev / S), b = fabs(u - C / S);
                *edge = a < b ? a : b;
            }
            return v;
        }
    }
    if (edge) *edge = 0.0; /* no crossing: u sits on the last edge */
    return last;
}

/* ===================================================================== per-token estimators */
void or_kl_estimate(const double *lp, const double *lr, const double *mask, int64_t n, int est,
                    double clamp, double *out) {
    for (int64_t i = 0; i < n; i++) {
        int scored = mask ? (mask[i] != 0.0) : 1;
        /* zero_masked is a select (rl.rs:100-102), then the optional clamp (rl.rs:389-392). */
        double d = scored ? (lr[i] - lp[i]) : 0.0;
        if (clamp > 0.0) d = d < -clamp ? -clamp : (d > clamp ? clamp : d);
        double k;
        if (est == 1) k = -d;
        else if (est == 2) k = d * d / 2.0;
        else k = exp(d) - d - 1.0;
        out[i] = scored ? k : 0.0;
    }
}

int64_t or_reduce_tokens(const double *per, const double *mask, int64_t S, int64_t B, int64_t T,
                         int reduction, double *out) {
    int64_t n = S * B * T;
    if (reduction == 0) {
        memcpy(out, per, (size_t)n * sizeof(double));
        return n;
    }
    for (int64_t s = 0; s < S; s++) {
        double tot = 0.0, cnt = 0.0, seqsum = 0.0, nonempty = 0.0;
        for (int64_t b = 0; b < B; b++) {
            double v = 0.0, m = 0.0;
            for (int64_t t = 0; t < T; t++) {
                int64_t i = (s * B + b) * T + t;
                v += per[i];
                m += mask ? mask[i] : 1.0;
            }
            tot += v;
            cnt += m;
            double ps = v / (m > 1.0 ? m : 1.0);
            if (reduction == 3) out[s * B + b] = ps;
            seqsum += ps;
            nonempty += (m > 1.0 ? 1.0 : m); /* min(count, 1) on integer counts (rl.rs:80) */
        }
        if (reduction == 1) out[s] = tot;
        else if (reduction == 2) out[s] = tot / (cnt > 1.0 ? cnt : 1.0);
        else if (reduction == 4) out[s] = seqsum / (nonempty > 1.0 ? nonempty : 1.0);
    }
    return reduction == 3 ? S * B : S;
}

int or_group_advantages(const double *r, int64_t len, int64_t n, int norm, double eps,
                        int unbiased, double *out) {
    if (n < 1 || len % n != 0) return -1;
    if (norm == 1 && (eps < 0.0 || (unbiased && n < 2))) return -1;
    for (int64_t g = 0; g < len; g += n) {
        double lo = INFINITY, hi = -INFINITY, sum = 0.0;
        for (int64_t i = 0; i < n; i++) {
            lo = r[g + i] < lo ? r[g + i] : lo;
            hi = r[g + i] > hi ? r[g + i] : hi;
        }
        if (lo == hi) { /* equal rewards: exact zeros (rl.rs:451-454) */
            for (int64_t i = 0; i < n; i++) out[g + i] = 0.0;
            continue;
        }
        for (int64_t i = 0; i < n; i++) sum += r[g + i];
        double mean = sum / (double)n, scale = 1.0;
        if (norm == 1) {
            double ss = 0.0;
            for (int64_t i = 0; i < n; i++) ss += (r[g + i] - mean) * (r[g + i] - mean);
            double var = ss / (unbiased ? (double)(n - 1) : (double)n);
            scale = sqrt(var) + eps;
        }
        for (int64_t i = 0; i < n; i++) out[g + i] = (r[g + i] - mean) / scale;
    }
    return 0;
}

/* ===================================================================== Cpu(Reference), f32 */
float or_unrolled_sum_f32(const float *x, int64_t n) {
    float p0 = 0, p1 = 0, p2 = 0, p3 = 0, p4 = 0, p5 = 0, p6 = 0, p7 = 0, acc = 0;
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) {
        p0 = p0 + x[i]; p1 = p1 + x[i + 1]; p2 = p2 + x[i + 2]; p3 = p3 + x[i + 3];
        p4 = p4 + x[i + 4]; p5 = p5 + x[i + 5]; p6 = p6 + x[i + 6]; p7 = p7 + x[i + 7];
    }
    acc = acc + (p0 + p4);
    acc = acc + (p1 + p5);
    acc = acc + (p2 + p6);
    acc = acc + (p3 + p7);
    for (; i < n; i++) acc = acc + x[i];
    return acc;
}

/* The same unrolled fold in f64 (kernels.rs:120-151 is generic over the element type). */
double or_unrolled_sum_f64(const double *x, int64_t n) {
    double p0 = 0, p1 = 0, p2 = 0, p3 = 0, p4 = 0, p5 = 0, p6 = 0, p7 = 0, acc = 0;
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) {
        p0 = p0 + x[i]; p1 = p1 + x[i + 1]; p2 = p2 + x[i + 2]; p3 = p3 + x[i + 3];
        p4 = p4 + x[i + 4]; p5 = p5 + x[i + 5]; p6 = p6 + x[i + 6]; p7 = p7 + x[i + 7];
    }
    acc = acc + (p0 + p4);
    acc = acc + (p1 + p5);
    acc = acc + (p2 + p6);
    acc = acc + (p3 + p7);
    for (; i < n; i++) acc = acc + x[i];
    return acc;
}

/* log_softmax along rows in the reference's operation order (activation.rs:30-42) in f64:
 * shifted = x - max, lse = log(unrolled_sum(exp(shifted))), y = shifted - lse. The f32 form is
 * or_cpuref_log_softmax. */
void or_cpuref_log_softmax_f64(const double *x, int64_t rows, int64_t V, double *y) {
    double *e = (double *)malloc((size_t)V * sizeof(double));
    for (int64_t r = 0; r < rows; r++) {
        const double *xr = x + r * V;
        double m = xr[0];
        for (int64_t k = 1; k < V; k++) m = xr[k] > m ? xr[k] : m;
        for (int64_t k = 0; k < V; k++) e[k] = exp(xr[k] - m);
        const double lse = log(or_unrolled_sum_f64(e, V));
        for (int64_t k = 0; k < V; k++) y[r * V + k] = (xr[k] - m) - lse;
    }
    free(e);
}

static float first_max_f32(const float *x, int64_t V, int64_t *idx_out) {
    float best = x[0];
    int64_t idx = 0;
    for (int64_t k = 0; k < V; k++) {
        float e = x[k];
        if (best != best) break;
        if (e != e || e > best) {
            best = e;
            idx = k;
        }
    }
    if (idx_out) *idx_out = idx;
    return best;
}

void or_cpuref_log_softmax(const float *x, int64_t rows, int64_t V, float *y) {
    size_t n = (size_t)rows * (size_t)V;
    float *mx = (float *)malloc((size_t)rows * sizeof(float));
    float *shifted = (float *)malloc(n * sizeof(float));
    float *e = (float *)malloc(n * sizeof(float));
    float *lse = (float *)malloc((size_t)rows * sizeof(float));
    for (int64_t r = 0; r < rows; r++) mx[r] = first_max_f32(x + r * V, V, NULL);
    for (size_t i = 0; i < n; i++) shifted[i] = x[i] - mx[i / (size_t)V];
    for (size_t i = 0; i < n; i++) e[i] = expf(shifted[i]);
    for (int64_t r = 0; r < rows; r++) lse[r] = or_unrolled_sum_f32(e + r * V, V);
    for (int64_t r = 0; r < rows; r++) lse[r] = logf(lse[r]);
    for (size_t i = 0; i < n; i++) y[i] = shifted[i] - lse[i / (size_t)V];
    free(mx); free(shifted); free(e); free(lse);
}

/* tempered_logits (rl.rs:475-486) as CpuRef materialises it: div_scalar (skipped at tau 1,
 * float.rs:494-499), then the broadcast add of the additive mask, f32 throughout. A u8 keep
 * row is this library's mask kind, not the reference's: it selects, as mask_fill does
 * (float.rs:984-1000), so an excluded token is -inf whatever its logit (a NaN or +inf there does
 * not reach the row), the rule every device kernel applies to a u8 mask. */
static float *cpuref_tempered_add(const float *x, int64_t rows, int64_t V, double tau,
                                  const float *addmask, int64_t add_ld, const uint8_t *keep, int64_t keep_ld) {
    size_t n = (size_t)rows * (size_t)V;
    float *z = (float *)malloc(n * sizeof(float));
    float t = (float)tau;
    if (tau == 1.0) memcpy(z, x, n * sizeof(float));
    else for (size_t i = 0; i < n; i++) z[i] = x[i] / t;
    if (addmask) {
        float *z2 = (float *)malloc(n * sizeof(float));
        for (int64_t r = 0; r < rows; r++)
            for (int64_t v = 0; v < V; v++) z2[r * V + v] = z[r * V + v] + addmask[r * add_ld + v];
        free(z);
        z = z2;
    }
    if (keep) {
        float *z2 = (float *)malloc(n * sizeof(float));
        for (int64_t r = 0; r < rows; r++)
            for (int64_t v = 0; v < V; v++)
                z2[r * V + v] = keep[(keep_ld ? r * keep_ld : 0) + v] ? z[r * V + v] : -INFINITY;
        free(z);
        z = z2;
    }
    return z;
}

static float *cpuref_tempered(const float *x, int64_t rows, int64_t V, double tau,
                              const uint8_t *keep, int64_t keep_ld) {
    return cpuref_tempered_add(x, rows, V, tau, NULL, 0, keep, keep_ld);
}

int64_t or_cpuref_sample_gumbel(const float *x, int64_t rows, int64_t V, double tau, const float *addmask,
                                int64_t add_ld, const uint8_t *keep, int64_t keep_ld, or_chacha *rng, int64_t *ids) {
    size_t n = (size_t)rows * (size_t)V;
    float *z = cpuref_tempered_add(x, rows, V, tau == 0.0 ? 1.0 : tau, addmask, add_ld, keep, keep_ld);
    for (int64_t r = 0; r < rows; r++) { /* max_dim + host check (rl.rs:515-519), before any draw */
        float m = first_max_f32(z + r * V, V, NULL);
        if (m != m || m == -INFINITY) {
            free(z);
            return 1 + r;
        }
    }
    if (tau != 0.0) {
        /* gumbel (rl.rs:490-498): one u64 per element in row-major order, f64 noise, cast to
         * f32 by from_f64s (float.rs:257-260), then z + g in f32. */
        for (size_t i = 0; i < n; i++) {
            double u = or_uniform_open01(or_chacha_next_u64(rng));
            float g = (float)(-log(-log(u)));
            z[i] = z[i] + g;
        }
    }
    for (int64_t r = 0; r < rows; r++) first_max_f32(z + r * V, V, &ids[r]);
    free(z);
    return 0;
}

int64_t or_cpuref_sample_logp(const float *x, int64_t rows, int64_t V, double tau,
                              const uint8_t *keep, int64_t keep_ld, or_chacha *rng,
                              int64_t *ids, float *logp) {
    size_t n = (size_t)rows * (size_t)V;
    float *z = cpuref_tempered(x, rows, V, tau == 0.0 ? 1.0 : tau, keep, keep_ld);
    for (int64_t r = 0; r < rows; r++) { /* max_dim + host check (rl.rs:515-519) */
        float m = first_max_f32(z + r * V, V, NULL);
        if (m != m || m == -INFINITY) {
            free(z);
            return 1 + r;
        }
    }
    float *zg = (float *)malloc(n * sizeof(float));
    if (tau == 0.0) {
        memcpy(zg, z, n * sizeof(float));
    } else {
        /* gumbel (rl.rs:490-498): f64 draws, cast to the logits' dtype, then z + g. */
        double *g = (double *)malloc(n * sizeof(double));
        for (size_t i = 0; i < n; i++) {
            double u = or_uniform_open01(or_chacha_next_u64(rng));
            g[i] = -log(-log(u));
        }
        float *gf = (float *)malloc(n * sizeof(float));
        for (size_t i = 0; i < n; i++) gf[i] = (float)g[i];
        for (size_t i = 0; i < n; i++) zg[i] = z[i] + gf[i];
        free(g);
        free(gf);
    }
    for (int64_t r = 0; r < rows; r++) first_max_f32(zg + r * V, V, &ids[r]);
    float *y = (float *)malloc(n * sizeof(float));
    or_cpuref_log_softmax(z, rows, V, y);
    for (int64_t r = 0; r < rows; r++) logp[r] = y[r * V + ids[r]];
    free(y);
    free(zg);
    free(z);
    return 0;
}

/* ===================================================================== Cpu(Fast)
 * The reference's Cpu(Fast) backend (src/tensor/backend.rs:57-239) as the sampler's op sequence
 * meets it: elementwise maps run on threads from FAST_MIN_MAP = 2^20 elements, zips of equal
 * shapes from FAST_MIN_ZIP = 2^22, last-axis sums from FAST_MIN_SUM = 2^22 with the 16-accumulator
 * lane sum (simd_sum); everything else (max_dim, argmax, broadcast zips, the Gumbel draws, the
 * gather) runs as Cpu(Reference) does. Threads are spawned per op call, as the reference's
 * scoped threads are, each taking one contiguous part of ceil(n / threads) elements. */
#define OR_FAST_MIN_MAP ((size_t)1 << 20)
#define OR_FAST_MIN_ZIP ((size_t)1 << 22)
#define OR_FAST_MIN_SUM ((size_t)1 << 22)

typedef struct {
    int op; /* 0: y = x / t, 1: y = a + b, 2: y = expf(x), 3: lane sums, 4: y = b != 0 ? a : -inf */
    const float *a, *b;
    float *y;
    float t;
    size_t lo, hi; /* elements (ops 0-2) or lanes (op 3) */
    int64_t n;     /* lane length (op 3) */
} fast_job;

/* simd_sum (backend.rs:92-115): 16 accumulators over chunks of 16, added in order, then the
 * remainder. */
static float fast_simd_sum(const float *x, int64_t n) {
    float acc[16] = {0};
    int64_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int k = 0; k < 16; k++) acc[k] = acc[k] + x[i + k];
    float total = 0.0f;
    for (int k = 0; k < 16; k++) total = total + acc[k];
    for (; i < n; i++) total = total + x[i];
    return total;
}

static void *fast_run(void *arg) {
    fast_job *j = (fast_job *)arg;
    switch (j->op) {
        case 0: for (size_t i = j->lo; i < j->hi; i++) j->y[i] = j->a[i] / j->t; break;
        case 1: for (size_t i = j->lo; i < j->hi; i++) j->y[i] = j->a[i] + j->b[i]; break;
        case 2: for (size_t i = j->lo; i < j->hi; i++) j->y[i] = expf(j->a[i]); break;
        case 4: for (size_t i = j->lo; i < j->hi; i++) j->y[i] = j->b[i] != 0.0f ? j->a[i] : -INFINITY; break;
        default: for (size_t l = j->lo; l < j->hi; l++) j->y[l] = fast_simd_sum(j->a + (int64_t)l * j->n, j->n); break;
    }
    return NULL;
}

/* One op over [0, n) on `parts` threads (fill, backend.rs:74-89). */
static void fast_par(int op, const float *a, const float *b, float *y, float t, size_t n, int64_t lane, int parts) {
    size_t per = (n + (size_t)parts - 1) / (size_t)parts;
    if (per == 0) per = 1;
    int used = (int)((n + per - 1) / per);
    pthread_t th[256];
    fast_job jobs[256];
    if (used > 256) used = 256;
    for (int i = 0; i < used; i++) {
        size_t lo = (size_t)i * per, hi = lo + per < n ? lo + per : n;
        fast_job j = {op, a, b, y, t, lo, hi, lane};
        jobs[i] = j;
        pthread_create(&th[i], NULL, fast_run, &jobs[i]);
    }
    for (int i = 0; i < used; i++) pthread_join(th[i], NULL);
}

int64_t or_cpufast_sample_logp(const float *x, int64_t rows, int64_t V, double tau, const uint8_t *keep,
                               int64_t keep_ld, or_chacha *rng, int threads, int64_t *ids, float *logp) {
    size_t n = (size_t)rows * (size_t)V;
    const int parts = threads < 1 ? 1 : (threads > 256 ? 256 : threads);
    const double tt = tau == 0.0 ? 1.0 : tau;
    /* tempered_logits: div_scalar (a map), then the u8 keep-mask as a select (a zip of equal
     * shapes, or a broadcast zip for a shared mask row): an excluded token is -inf whatever its
     * logit, the device kernels' rule */
    float *z = (float *)malloc(n * sizeof(float));
    if (tt == 1.0) memcpy(z, x, n * sizeof(float));
    else if (n >= OR_FAST_MIN_MAP && parts > 1) fast_par(0, x, NULL, z, (float)tt, n, 0, parts);
    else for (size_t i = 0; i < n; i++) z[i] = x[i] / (float)tt;
    if (keep) {
        int64_t mrows = keep_ld == 0 ? 1 : rows;
        float *kf = (float *)malloc((size_t)mrows * (size_t)V * sizeof(float));  /* the condition tensor */
        for (int64_t r = 0; r < mrows; r++)
            for (int64_t v = 0; v < V; v++) kf[r * V + v] = keep[r * keep_ld + v] ? 1.0f : 0.0f;
        float *z2 = (float *)malloc(n * sizeof(float));
        if (mrows == rows && n >= OR_FAST_MIN_ZIP && parts > 1) fast_par(4, z, kf, z2, 0.0f, n, 0, parts);
        else
            for (int64_t r = 0; r < rows; r++)
                for (int64_t v = 0; v < V; v++)
                    z2[r * V + v] = kf[(keep_ld ? r : 0) * V + v] != 0.0f ? z[r * V + v] : -INFINITY;
        free(kf);
        free(z);
        z = z2;
    }
    for (int64_t r = 0; r < rows; r++) { /* max_dim (Reference) + the host check */
        float m = first_max_f32(z + r * V, V, NULL);
        if (m != m || m == -INFINITY) {
            free(z);
            return 1 + r;
        }
    }
    float *zg = (float *)malloc(n * sizeof(float));
    if (tau == 0.0) {
        memcpy(zg, z, n * sizeof(float));
    } else {
        /* the Gumbel draws: the host loop of rl.rs:490-498, one thread (the stream is sequential),
         * cast to f32 by from_f64s, then z + g (a zip of equal shapes) */
        float *gf = (float *)malloc(n * sizeof(float));
        for (size_t i = 0; i < n; i++) gf[i] = (float)(-log(-log(or_uniform_open01(or_chacha_next_u64(rng)))));
        if (n >= OR_FAST_MIN_ZIP && parts > 1) fast_par(1, z, gf, zg, 0.0f, n, 0, parts);
        else for (size_t i = 0; i < n; i++) zg[i] = z[i] + gf[i];
        free(gf);
    }
    for (int64_t r = 0; r < rows; r++) first_max_f32(zg + r * V, V, &ids[r]); /* argmax (Reference) */
    /* token_log_probs: log_softmax = max_dim, a broadcast sub (Reference), exp (a map), sum_dim
     * on the last axis (simd_sum per lane on threads), ln of the row sums (a map of `rows`
     * elements), a broadcast sub; then the gather */
    float *mx = (float *)malloc((size_t)rows * sizeof(float));
    float *sh = (float *)malloc(n * sizeof(float));
    float *e = (float *)malloc(n * sizeof(float));
    float *lse = (float *)malloc((size_t)rows * sizeof(float));
    for (int64_t r = 0; r < rows; r++) mx[r] = first_max_f32(z + r * V, V, NULL);
    for (size_t i = 0; i < n; i++) sh[i] = z[i] - mx[i / (size_t)V];
    if (n >= OR_FAST_MIN_MAP && parts > 1) fast_par(2, sh, NULL, e, 0.0f, n, 0, parts);
    else for (size_t i = 0; i < n; i++) e[i] = expf(sh[i]);
    if (n >= OR_FAST_MIN_SUM && parts > 1) fast_par(3, e, NULL, lse, 0.0f, (size_t)rows, V, parts);
    else for (int64_t r = 0; r < rows; r++) lse[r] = or_unrolled_sum_f32(e + r * V, V);
    for (int64_t r = 0; r < rows; r++) lse[r] = logf(lse[r]);
    for (int64_t r = 0; r < rows; r++) logp[r] = sh[r * V + ids[r]] - lse[r];
    free(mx); free(sh); free(e); free(lse); free(zg); free(z);
    return 0;
}

typedef struct {
    const float *x;
    int64_t r0, r1, V;
    double tau;
    const uint8_t *keep;
    int64_t keep_ld;
    const double *u;
    int64_t *ids;
    float *logp;
    int64_t refused;
} invcdf_job;

static void *invcdf_run(void *arg) {
    invcdf_job *j = (invcdf_job *)arg;
    int64_t V = j->V;
    j->refused = 0;
    for (int64_t r = j->r0; r < j->r1; r++) {
        const uint8_t *kp = j->keep ? j->keep + r * j->keep_ld : NULL;
        float *z = cpuref_tempered(j->x + r * V, 1, V, j->tau == 0.0 ? 1.0 : j->tau, kp, 0);
        int64_t am;
        float m = first_max_f32(z, V, &am);
        if (m != m || m == -INFINITY) {
            free(z);
            if (!j->refused) j->refused = 1 + r;
            continue;
        }
        float *e = (float *)malloc((size_t)V * sizeof(float));
        for (int64_t v = 0; v < V; v++) e[v] = expf(z[v] - m);
        float S = or_unrolled_sum_f32(e, V);
        int64_t id = am;
        if (j->tau != 0.0) {
            double t = j->u[r] * (double)S, C = 0.0;
            int64_t last = -1;
            id = -1;
            for (int64_t v = 0; v < V; v++) {
                if (e[v] > 0.0f) last = v;
                C += (double)e[v];
                if (C > t) {
                    id = v;
                    break;
                }
            }
            if (id < 0) id = last;
        }
        j->ids[r] = id;
        j->logp[r] = (z[id] - m) - logf(S);
        free(e);
        free(z);
    }
    return NULL;
}

int64_t or_cpu_sample_logp_invcdf(const float *x, int64_t rows, int64_t V, double tau,
                                  const uint8_t *keep, int64_t keep_ld, const double *u,
                                  int64_t *ids, float *logp, int threads) {
    if (threads < 1) threads = 1;
    if (threads > rows) threads = (int)(rows > 0 ? rows : 1);
    invcdf_job *jobs = (invcdf_job *)calloc((size_t)threads, sizeof(invcdf_job));
    pthread_t *th = (pthread_t *)calloc((size_t)threads, sizeof(pthread_t));
    int64_t per = (rows + threads - 1) / threads;
    for (int i = 0; i < threads; i++) {
        invcdf_job *j = &jobs[i];
        j->x = x; j->V = V; j->tau = tau; j->keep = keep; j->keep_ld = keep_ld; j->u = u;
        j->ids = ids; j->logp = logp;
        j->r0 = i * per;
        j->r1 = (i + 1) * per < rows ? (i + 1) * per : rows;
        if (j->r0 > j->r1) j->r0 = j->r1;
        if (threads == 1) invcdf_run(j);
        else pthread_create(&th[i], NULL, invcdf_run, j);
    }
    int64_t refused = 0;
    for (int i = 0; i < threads; i++) {
        if (threads > 1) pthread_join(th[i], NULL);
        if (jobs[i].refused && (!refused || jobs[i].refused < refused)) refused = jobs[i].refused;
    }
    free(jobs);
    free(th);
    return refused;
}

/* ------------------------------------------------------------------ policy losses per token */

/* policy_gradient_loss (rl.rs:228-235, kind 0) and clipped_policy_loss (rl.rs:265-287, kind 1)
 * per token in f64, before reduce_tokens: the loss (0 at masked positions), its derivative with
 * respect to logp as the op sequence's autograd propagates it (the select gives the gradient to
 * the chosen branch, the clamps pass it inside their range only, exp's derivative is its value),
 * and clip_fraction's per-token indicator (rl.rs:293-317) times the mask. w holds per-token
 * weights, or per-sequence ones (per_seq: index i / T). dual <= 0: no dual clip; clamp <= 0: no
 * log-ratio clamp. Any output may be NULL. */
void or_policy_loss(int kind, int64_t n, int64_t T, const double *lp, const double *old, const double *w,
                    int per_seq, const double *mask, double low, double high, double dual, double clamp,
                    double *loss, double *dloss, double *hit) {
    const double lo = 1.0 - low, hi = 1.0 + high;
    for (int64_t i = 0; i < n; i++) {
        const double m = mask ? mask[i] : 1.0;
        const int scored = m != 0.0;
        const double a = per_seq ? w[i / T] : w[i];
        double per, dper, h = 0.0;
        if (kind == 0) {
            per = -(lp[i] * a);
            dper = -a;
        } else {
            const double d = scored ? lp[i] - old[i] : 0.0;
            double dc = d, gate = 1.0;
            if (clamp > 0.0) {
                dc = d < -clamp ? -clamp : (d > clamp ? clamp : d);
                gate = (d >= -clamp && d <= clamp) ? 1.0 : 0.0;
            }
            const double r = exp(dc);
            const double rc = r < lo ? lo : (r > hi ? hi : r);
            const double un = -(r * a), cl = -(rc * a);
            const int un_wins = (un - cl) > 0.0;
            double v = un_wins ? un : cl;
            double gr = (un_wins || (r >= lo && r <= hi)) ? -a : 0.0;
            if (dual > 0.0 && a < 0.0) {
                const double cap = -dual * a;
                const int keep = (cap - v) > 0.0; /* min(v, -c A): v where v < -c A */
                v = keep ? v : cap;
                gr = keep ? gr : 0.0;
            }
            per = v;
            dper = gr * r * gate;
            const double r0 = exp(d);
            h = ((a > 0.0 && r0 > hi) ? 1.0 : 0.0) + ((a < 0.0 && r0 < lo) ? 1.0 : 0.0);
            if (dual > 0.0 && a < 0.0 && r0 > dual) h += 1.0;
            if (clamp > 0.0 && fabs(d) > clamp) h += 1.0;
            h = (h > 1.0 ? 1.0 : h) * m;
        }
        if (loss) loss[i] = scored ? per : 0.0;
        if (dloss) dloss[i] = scored ? dper : 0.0;
        if (hit) hit[i] = scored ? h : 0.0;
    }
}

/* The backward of reduce_tokens after zero_masked (rl.rs:69-102): the derivative of each
 * reduced output with respect to each position's value, times the output's upstream gradient
 * (up NULL: ones), times scale and local[i] (NULL: ones); 0 at masked positions. */
void or_reduce_tokens_backward(const double *mask, int64_t S, int64_t B, int64_t T, int reduction, const double *up,
                               double scale, const double *local, double *out) {
    for (int64_t s = 0; s < S; s++) {
        double cnt = 0.0, nonempty = 0.0;
        for (int64_t b = 0; b < B; b++) {
            double m = 0.0;
            for (int64_t t = 0; t < T; t++) m += mask ? mask[(s * B + b) * T + t] : 1.0;
            cnt += m;
            nonempty += m > 1.0 ? 1.0 : m;
        }
        cnt = cnt > 1.0 ? cnt : 1.0;
        nonempty = nonempty > 1.0 ? nonempty : 1.0;
        for (int64_t b = 0; b < B; b++) {
            double m_seq = 0.0;
            for (int64_t t = 0; t < T; t++) m_seq += mask ? mask[(s * B + b) * T + t] : 1.0;
            m_seq = m_seq > 1.0 ? m_seq : 1.0;
            for (int64_t t = 0; t < T; t++) {
                const int64_t i = (s * B + b) * T + t;
                const double m = mask ? mask[i] : 1.0;
                double g;
                if (reduction == 0) g = up ? up[i] : 1.0;
                else if (reduction == 1) g = up ? up[s] : 1.0;
                else if (reduction == 2) g = (up ? up[s] : 1.0) / cnt;
                else if (reduction == 3) g = (up ? up[s * B + b] : 1.0) / m_seq;
                else g = (up ? up[s] : 1.0) / (nonempty * m_seq);
                out[i] = m != 0.0 ? scale * g * (local ? local[i] : 1.0) : 0.0;
            }
        }
    }
}

/* d kl_estimate / d logp per token (rl.rs:380-400): with delta = lr - lp, 1 (k1), -delta (k2),
 * 1 - exp(delta) (k3); 0 at masked positions and where the clamp is active. */
void or_kl_estimate_grad(const double *lp, const double *lr, const double *mask, int64_t n, int est, double clamp,
                         double *out) {
    for (int64_t i = 0; i < n; i++) {
        const int scored = mask ? (mask[i] != 0.0) : 1;
        const double d = scored ? (lr[i] - lp[i]) : 0.0;
        const int active = clamp > 0.0 && !(d >= -clamp && d <= clamp);
        double g;
        if (est == 1) g = 1.0;
        else if (est == 2) g = -d;
        else g = -expm1(d);
        out[i] = (scored && !active) ? g : 0.0;
    }
}


/* ------------------------------------------------------------------ the reference's test inputs */

/* rand_core 0.6.4's SeedableRng::seed_from_u64: PCG32 steps (state = state * mul + inc, then the
 * XSH-RR output: ((state >> 18) ^ state) >> 27 rotated right by state >> 59) fill the 32-byte
 * seed four little-endian bytes at a time. */
void or_seed_from_u64(uint64_t state, uint64_t inc, uint8_t seed[32]) {
    for (int i = 0; i < 8; i++) {
        state = state * 6364136223846793005ull + inc;
        const uint32_t xs = (uint32_t)(((state >> 18) ^ state) >> 27);
        const uint32_t rot = (uint32_t)(state >> 59);
        const uint32_t x = (xs >> rot) | (xs << ((32u - rot) & 31u));
        for (int b = 0; b < 4; b++) seed[4 * i + b] = (uint8_t)(x >> (8 * b));
    }
}

/* The reference's test helper rnd (src/tensor/tests/mod.rs:28-31): ChaCha8Rng::seed_from_u64(seed),
 * then n draws of rand 0.8's gen_range(lo..hi) for f32: a u32 from the stream, its top 23 bits as
 * the mantissa of a value in [1, 2), minus 1, times (hi - lo), plus lo (f32 arithmetic, no fused
 * multiply-add), drawn again in the rare case the result reaches hi. The stream is consumed one
 * 16-word block after another, each block's words in order (counter in words 12-13, stream 0). */
void or_reference_rnd_f32(uint64_t seed, uint64_t inc, int64_t n, float lo, float hi, float *out) {
    uint8_t sd[32];
    or_seed_from_u64(seed, inc, sd);
    or_chacha r;
    or_chacha_seed(&r, sd);
    const float scale = hi - lo;
    for (int64_t i = 0; i < n; i++) {
        for (;;) {
            if (r.idx >= 16) {
                or_chacha_block_rounds(r.key, r.counter, 0, 8, r.buf);
                r.counter++;
                r.idx = 0;
            }
            const uint32_t u = r.buf[r.idx++];
            union { uint32_t b; float f; } v;
            v.b = (u >> 9) | 0x3f800000u;
            volatile float v01 = v.f - 1.0f;
            volatile float prod = v01 * scale;
            const float res = prod + lo;
            if (res < hi) {
                out[i] = res;
                break;
            }
        }
    }
}

/* The nn tests' helper rnd (src/nn/tests/mod.rs:35-38): ChaCha8Rng::seed_from_u64(seed), then n
 * draws of rand 0.8's gen_range(lo..hi) for f64: a u64 from the stream (two consecutive words,
 * low first), its top 52 bits as the mantissa of a value in [1, 2), minus 1, times (hi - lo),
 * plus lo (f64 arithmetic, no fused multiply-add), drawn again in the rare case the result
 * reaches hi. */
void or_reference_rnd_f64(uint64_t seed, uint64_t inc, int64_t n, double lo, double hi, double *out) {
    uint8_t sd[32];
    or_seed_from_u64(seed, inc, sd);
    or_chacha r;
    or_chacha_seed(&r, sd);
    const double scale = hi - lo;
    for (int64_t i = 0; i < n; i++) {
        for (;;) {
            uint32_t w[2];
            for (int h = 0; h < 2; h++) {
                if (r.idx >= 16) {
                    or_chacha_block_rounds(r.key, r.counter, 0, 8, r.buf);
                    r.counter++;
                    r.idx = 0;
                }
                w[h] = r.buf[r.idx++];
            }
            const uint64_t u = (uint64_t)w[0] | ((uint64_t)w[1] << 32);
            union { uint64_t b; double f; } v;
            v.b = (u >> 12) | 0x3ff0000000000000ull;
            volatile double v01 = v.f - 1.0;
            volatile double prod = v01 * scale;
            const double res = prod + lo;
            if (res < hi) {
                out[i] = res;
                break;
            }
        }
    }
}

/* ===================================================================== matmul and sort */
/* One [m, k] x [k, n] product in the reference's arithmetic (src/tensor/cuda/kernels.rs:14-20,
 * the order of matrixmultiply 0.3.11's sgemm that CpuRef calls per batch,
 * src/tensor/kernels.rs:415-420): each output is an fmaf chain from zero over k in order, closed
 * every 256 k; the first block's chain is the total and each later block's chain is added to it.
 * Element strides a_rs/a_cs and b_rs/b_cs; c is contiguous [m, n]. */
void or_matmul_f32(const float *a, int64_t a_rs, int64_t a_cs, const float *b, int64_t b_rs, int64_t b_cs,
                   int64_t m, int64_t k, int64_t n, float *c) {
    /* a row of outputs at a time, each output's chain still in k order (the loops over j only
     * interleave independent chains) */
    float *acc = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    for (int64_t i = 0; i < m; i++) {
        float *tot = c + i * n;
        for (int64_t j = 0; j < n; j++) tot[j] = 0.0f;
        for (int64_t k0 = 0; k0 < k; k0 += 256) {
            const int64_t k1 = k0 + 256 < k ? k0 + 256 : k;
            for (int64_t j = 0; j < n; j++) acc[j] = 0.0f;
            for (int64_t l = k0; l < k1; l++) {
                const float x = a[i * a_rs + l * a_cs];
                const float *brow = b + l * b_rs;
                for (int64_t j = 0; j < n; j++) acc[j] = fmaf(x, brow[j * b_cs], acc[j]);
            }
            for (int64_t j = 0; j < n; j++) tot[j] = k0 == 0 ? acc[j] : acc[j] + tot[j];
        }
    }
    free(acc);
}
