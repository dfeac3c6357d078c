/*
 * noetic_hip.h — the C ABI of libnoetic_hip.so, the MI355X (gfx950) backend of noetic-tensor's
 * `nn::rl` vocabulary-row hot path.
 *
 * Conventions (all entry points):
 *  - Plain pointers and sizes; no framework types cross the boundary.
 *  - Return 0 on success, else an NT_E_* code or a hipError_t value (> 0); the text of the
 *    last failure on this thread is nt_hip_last_error().
 *  - Device pointers come from nt_hip_alloc (or any HIP allocation on the claimed device).
 *    Every launch goes to the library's one stream (one process-wide non-blocking stream, as
 *    the reference's CUDA backend keeps, src/tensor/cuda/backend.rs:205-206); results are
 *    ready after nt_hip_sync() or a download.
 *  - Every device entry point is serialised by one process-wide mutex (the reference's
 *    `CTX: OnceLock<Mutex<Ctx>>`, src/tensor/cuda/backend.rs:104,148-159).
 *  - Kernels use no atomics and reduce in a fixed order, so a rerun on the same inputs is
 *    bit-identical (the reference's determinism contract, src/nn/tests/gpu/rl.rs:125-128).
 *
 * A Rust caller binds these with a hand-written `extern "C"` block, the reference's FFI style
 * (src/tensor/cuda/ffi.rs:30-117), from optional GpuBackend methods.
 */
#ifndef NOETIC_HIP_H
#define NOETIC_HIP_H

#ifndef __HIPCC_RTC__ /* the library's kernels compiled at run time by hiprtc see size_t from it */
#include <stddef.h>
#endif
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes (the library's own; hipError_t values are passed through) ---------- */
#define NT_OK 0
#define NT_E_ARG (-1)         /* an invalid argument (shape, dtype, null pointer, ...) */
#define NT_E_UNCLAIMED (-2)   /* no device claimed in this process */
#define NT_E_CLAIMED (-3)     /* another device is already claimed by this process */
#define NT_E_UNSUPPORTED (-4) /* a valid request this build does not implement */
#define NT_E_RTC (-5)         /* the run-time kernel compiler (hiprtc) failed; the log is in nt_hip_last_error */

/* ---- dtypes and mask kinds ------------------------------------------------------------ */
#define NT_F32 0  /* f32 logits */
#define NT_BF16 1 /* bf16 logits, stored as their bit patterns (src/tensor/half.rs:10-12) */
#define NT_F16 2  /* f16 logits, IEEE binary16 bit patterns (src/tensor/half.rs:40-70), widened
                     exactly as the reference computes 16-bit values in f32 (float.rs:43-58) */

#define NT_MASK_NONE 0 /* no vocabulary mask */
#define NT_MASK_U8 1   /* u8 keep-mask: 0 excludes the token, any other value keeps it. An excluded
                          token's logit is replaced by -inf, whatever it holds, so a NaN or +inf
                          there does not reach the row (a -inf entry of an f32 mask is added
                          instead, and NaN + -inf or inf + -inf refuses the row, as the
                          reference's additive masks do) */
#define NT_MASK_F32 2  /* additive f32 mask (0, -inf, -1e9, any value), added after the divide
                          by the temperature: rl.rs:475-486 `logits / temperature + mask` */

/* A mask of the logits' rank that broadcasts over any of the leading dimensions (rl.rs:477-483:
 * each mask dimension equals the logits' or is 1). The logits rows are (s, b, t) positions, t
 * fastest: row r = (s B + b) T + t with T = t_rows and B = b_rows, and it reads the mask row that
 * starts at element s ld_s + b ld_b + t mask_ld (mask_ld being the args' own field). All zero (the
 * default) is one group, T = rows and B = 1: row r reads the mask at r mask_ld. Each stride is 0
 * (a broadcast dimension) or at least vocab; rows must be a multiple of T B. A logits tensor of
 * any rank folds its leading dimensions into these three: adjacent dimensions that are both
 * broadcast, or both read contiguously, merge. */
typedef struct NtMaskRows {
    int64_t t_rows, b_rows; /* T and B; 0 and 0 = one group of all rows */
    int64_t ld_b, ld_s;     /* mask elements between consecutive b and s (0 = broadcast) */
} NtMaskRows;

/* ---- per-row status ------------------------------------------------------------------- */
#define NT_ROW_OK 0
#define NT_ROW_NO_TOKEN 1 /* every logit -inf after the mask: rl.rs:516-519 refuses the row */
#define NT_ROW_NAN 2      /* a NaN reached the row's sum: rl.rs:516-519 refuses the row */
#define NT_ROW_BAD_TOKEN 3 /* a scored token outside [0, V): the reference's gather panics
                            (src/tensor/kernels.rs:224) */

/* ===================================================================== runtime
 * Replaces the device/context/memory slice of the reference's GpuBackend trait
 * (src/tensor/gpu/mod.rs:137-207) for a new `Device::Hip(i)` (src/tensor/device.rs:23-27). */

/* Claim HIP device `device` for this process (one device per process, as `claim` in
 * src/tensor/cuda/backend.rs:115-138): sets it current and creates the library's stream.
 * Claiming the claimed device again is a no-op. */
int nt_hip_claim(int device);
/* Number of visible HIP devices (0 without a GPU; never fails). */
int nt_hip_device_count(void);
/* The text of the last failure on the calling thread ("" if none). */
const char *nt_hip_last_error(void);
/* Provenance key, "hip-<gcnArchName>-hiprt<runtime version>-kernels-<sha16 of the device
 * sources>" (cf. `key`, src/tensor/cuda/backend.rs:962-966); written NUL-terminated into buf. */
int nt_hip_key(char *buf, size_t cap);
/* What the device's results depend on outside the library's sources (cf. `platform_details`,
 * src/tensor/gpu/mod.rs:199, src/tensor/cuda/backend.rs:968-974, used by `gpu_platform_key`,
 * gpu/mod.rs:699-700): "hipdriver<version>-amdgpu-<kernel driver release or inbox>-clang-<the
 * compiler version and release that built the code objects>", NUL-terminated into buf; an
 * error when cap cannot hold it. */
int nt_hip_platform_details(char *buf, size_t cap);
/* GpuBackend::alloc / upload / download / sync (src/tensor/gpu/mod.rs:139-140,181-184).
 * nt_hip_alloc takes memory from the device's stream-ordered pool when it has one: it is valid for
 * work queued on the library stream after the call. nt_hip_free only records the pointer and
 * returns at once (the reference's Mem drop, src/tensor/cuda/backend.rs:35-45); the next entry
 * point frees it on the stream, after the work queued before the release. */
int nt_hip_alloc(size_t bytes, void **out);
int nt_hip_free(void *ptr);
int nt_hip_upload(void *dst, const void *src, size_t bytes);   /* host -> device, synchronous */
int nt_hip_download(void *dst, const void *src, size_t bytes); /* device -> host, synchronous */
int nt_hip_memset(void *dst, int value, size_t bytes);          /* device fill, on the stream */
int nt_hip_sync(void);
/* The library's stream as a hipStream_t (for callers that record events on it). */
int nt_hip_stream(void **out);
/* Launch counter (the reference's `launches()`, src/tensor/cuda/backend.rs:1034-1036). */
uint64_t nt_hip_launches(void);

/* Where the nn::rl row kernels (nt_hip_rl_sample, nt_hip_rl_sample_gumbel, nt_hip_rl_score,
 * nt_hip_rl_score_backward) launch from; nt_hip_rl_sample_noalloc always launches the ahead-of-time
 * code objects, since a run-time instance's first launch allocates. The CUDA
 * backend compiles its kernels with NVRTC at first use and caches the functions
 * (src/tensor/cuda/mod.rs:169-218, cuda/backend.rs:281-293, 322-358); here both ways exist for
 * one device source: NT_KERNELS_AOT, the code objects hipcc built into this library (the
 * default), and NT_KERNELS_RTC, each template instance compiled by hiprtc at its first launch
 * from the source embedded in the library (0.2-1.3 s each), loaded with hipModuleLoadData, launched
 * with hipModuleLaunchKernel and cached per process and on disk (NOETIC_HIP_CACHE_DIR, else
 * $HOME/.cache/noetic-hip). The environment's NOETIC_HIP_KERNELS=aot|rtc sets the first value;
 * nt_hip_set_kernel_path changes it for the process and returns the previous path (or NT_E_ARG).
 * With NT_KERNELS_RTC, nt_hip_key also names hiprtc's version and the embedded source's SHA-256. */
#define NT_KERNELS_AOT 0
#define NT_KERNELS_RTC 1
int nt_hip_set_kernel_path(int path);
int nt_hip_kernel_path(void);

/* ===================================================================== nn::rl fused rows
 * Logits are row-major [rows, V] (rows = S*B*T of `[S, B, T, V]`, rl.rs:8-14) with row stride
 * `ld` elements (ld >= V). A row is one (s, b, t) position. The float arithmetic is f32 with
 * bf16 and f16 inputs converted exactly (float.rs:43-67); per-row scalars are combined in f64. */

/* Gumbel-max categorical sample of each row: the reference's own sampler,
 *   ids = sample_categorical(logits, temperature, mask, rng)        (rl.rs:488-529)
 * for a Hip tensor. z = tempered_logits(logits, temperature, mask) in f32 (rl.rs:475-486: the
 * f32 divide, skipped at temperature 1, then the f32 mask add; a u8 keep-mask puts -inf at an
 * excluded token); g_i = f32(-ln(-ln u_i)) with u_i = ((k_i >> 11) + 0.5) / 2^53 from the i-th
 * u64 k_i of the stream in row-major element order (one u64 per logit, rl.rs:490-498); the
 * token is the first index of the maximum of z + g (argmax_dim, src/tensor/kernels.rs:183-209).
 * The draws are generated on the device from the stream's ChaCha20 key and word position, so
 * nothing of size rows x V crosses PCIe. The call does not move the caller's stream: after it
 * has checked the status (a refused row draws nothing, as the reference panics before its
 * draw, rl.rs:515-519), the caller advances the stream by rows x V u64 (nt_rng_skip_u64, or
 * rand_chacha's set_word_pos) when temperature > 0. Temperature 0 is greedy: the first argmax
 * of the masked logits, no draws. */
typedef struct NtRlGumbelArgs {
    const void *logits;       /* [rows, ld] f32, bf16 or f16 */
    int32_t dtype;            /* NT_F32 | NT_BF16 | NT_F16 */
    int32_t mask_kind;        /* NT_MASK_* */
    int64_t rows, vocab, ld;
    const void *mask;         /* u8 or f32 rows of vocab entries; NULL with NT_MASK_NONE */
    int64_t mask_ld;          /* mask row stride (over t, see NtMaskRows); 0 = one row shared */
    double temperature;       /* >= 0 and finite; 0 = greedy */
    uint32_t key[8];          /* the stream's ChaCha20 key (its 32-byte seed as little-endian words) */
    uint64_t block;           /* the stream's position: its next u64 starts at word `word` of */
    int32_t word;             /*   keystream block `block` (nt_rng_word_pos); word in 0..15 */
    int32_t pad0;
    int32_t *ids;             /* [rows] out: the sampled token (-1 on a refused row) */
    uint8_t *status;          /* [rows] out: NT_ROW_OK, NT_ROW_NO_TOKEN or NT_ROW_NAN (required) */
    NtMaskRows mask_rows;     /* a mask broadcast over leading dimensions (zero: rows of mask_ld) */
} NtRlGumbelArgs;
int nt_hip_rl_sample_gumbel(const NtRlGumbelArgs *a);

/* Fused masked categorical sample + log-probability (+ entropy) of each row by the inverse
 * CDF of one uniform per row: one pass over the logits and the mask. This is a new nn::rl
 * entry (`sample_categorical_inv_cdf`; the reference has no counterpart), which does, for a
 * Hip tensor, what the op sequence
 *   ids  = <an inverse-CDF draw of softmax(z)>                      (cf. rl.rs:510-529)
 *   logp = token_log_probs(tempered_logits(logits, temperature, mask), ids)  (rl.rs:134-141)
 *   ent  = categorical_entropy(tempered_logits(...), None, TokenReduction::None) (rl.rs:405-414)
 * would: with z the tempered logits, m = max z, w_v = exp(z_v - m) and S = sum w, the token is
 * min{v : sum_{j<=v} w_j > u*S} (excluded tokens have w = 0 and are never drawn; if rounding
 * leaves no crossing, the last token with w > 0). temperature 0 is greedy: the first argmax
 * of the masked logits (rl.rs:510-513), no uniform read; logp/entropy are then those of the
 * temperature-1 distribution (rl.rs:514). */
typedef struct NtRlSampleArgs {
    const void *logits;       /* [rows, ld] f32, bf16 or f16 */
    int32_t dtype;            /* NT_F32 | NT_BF16 | NT_F16 */
    int32_t mask_kind;        /* NT_MASK_* */
    int64_t rows, vocab, ld;
    const void *mask;         /* u8 or f32 rows of vocab entries; NULL with NT_MASK_NONE */
    int64_t mask_ld;          /* mask row stride (over t, see NtMaskRows); 0 = one row shared */
    double temperature;       /* >= 0 and finite; 0 = greedy */
    const double *uniforms;   /* [rows] device, each in (0,1); unused when greedy */
    int32_t *ids;             /* [rows] out: the sampled token (-1 on a refused row) */
    float *logp;              /* [rows] out or NULL */
    float *entropy;           /* [rows] out or NULL */
    uint8_t *status;          /* [rows] out: NT_ROW_* (required) */
    NtMaskRows mask_rows;     /* a mask broadcast over leading dimensions (zero: rows of mask_ld) */
} NtRlSampleArgs;
int nt_hip_rl_sample(const NtRlSampleArgs *a);

/* nt_hip_rl_sample without allocation. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Same arguments, kernels and results as nt_hip_rl_sample; the segmented
 * sampler's workspace (its per-row arrival counters and wave records) is a fixed device array
 * of 2 MiB per GPU instead of the library's allocation, and a launch that needs more is refused
 * (NT_E_ARG) before anything runs. The call makes no hipMalloc, hipFree or other allocating call
 * (pointers released with nt_hip_free are freed by the next other entry point), and it launches
 * the library's ahead-of-time code objects whatever nt_hip_set_kernel_path chose: compiling and
 * loading a hiprtc instance allocates device memory. Calls share that
 * GPU's array and leave the last call's records in it; they are ordered on the library's stream,
 * and calls that overlap on one GPU race. */
int nt_hip_rl_sample_noalloc(const NtRlSampleArgs *a);

/* The readout-fused sampler: one decode step's readout product and its inverse-CDF sample +
 * log-probability, with the logits never written. For each row r,
 *   logits[r, v] = sum_k hidden[r, k] W[k, v]          (the decoder's readout x . W,
 *                                                        src/nn/decoder.rs:272,286; linear.rs:1-3)
 * in f32 from bf16 operands on the matrix cores (the reference's half-precision product,
 * src/tensor/gpu/half_gemm.rs:1-10; it stands for the decoder's product only when the caller's
 * matmul precision is MatmulPrecision::Half, src/tensor/precision.rs:4-8, 59-63: at the default
 * F32 the caller multiplies and samples the written logits), then exactly nt_hip_rl_sample's draw on those logits
 * (tempered by the temperature, the u8 keep-mask applied; one uniform per row; temperature 0 is
 * the first argmax). The weight is packed once, when loaded, into the order the matrix cores
 * read it (nt_hip_rl_readout_pack_weight, from the reference's [d, V] layout or a [V, d] one).
 * rows <= 256; vocab <= 262144; dim a multiple of 16, at most 16384; a bf16 hidden has ldh a
 * multiple of 8 and is 16-byte aligned (an f32 or f16 one: aligned to its element, one more launch
 * rounds it); a
 * u8 mask with one row per logits row (mask_ld >= vocab) or one row shared by all (mask_ld 0).
 * Three launches on the
 * library stream: h into the same order (2 MB at 256 x 4096), the product with the sampler's
 * per-row records in its epilogue, then one workgroup per row that merges them and recomputes
 * only the 32 logits of the block holding the draw. The debug pointers (NULL in use) write the
 * f32 logits, the recomputed block and its index, for the parity tests. */
#define NT_READOUT_W_DV 0 /* the reference's Linear weight [d, V]: W[k, v] at w + k ld + v */
#define NT_READOUT_W_VD 1 /* vocabulary-major [V, d]: W[k, v] at w + v ld + k */
/* Bytes of the packed weight: ceil(vocab / 256) 256 dim 2, the vocabulary padded with zero
 * columns to whole tiles of 256 (-1 for an invalid shape). */
int64_t nt_hip_rl_readout_packed_bytes(int64_t vocab, int64_t dim);
/* Pack a readout weight (dtype NT_BF16, or NT_F32 or NT_F16 rounded to bf16 to nearest-even as it
 * is packed, the half-precision product's rounding of its operands, src/tensor/precision.rs:4-8;
 * an f16 value widens to f32 exactly first, so it is rounded once; layout
 * NT_READOUT_W_*, row stride ld) into `packed` (device, nt_hip_rl_readout_packed_bytes bytes,
 * 16-byte aligned): one kernel on the library stream. */
int nt_hip_rl_readout_pack_weight(const void *weight, int32_t dtype, int32_t layout, int64_t vocab, int64_t dim,
                                  int64_t ld, void *packed);
typedef struct NtRlReadoutSampleArgs {
    const void *hidden;        /* [rows, ldh] hidden_dtype: the readout's input */
    const void *weight_packed; /* the readout weight, packed by nt_hip_rl_readout_pack_weight */
    int64_t rows, vocab, dim, ldh;
    int32_t mask_kind;         /* NT_MASK_NONE | NT_MASK_U8 */
    int32_t hidden_dtype;      /* NT_BF16, or NT_F32 / NT_F16 (rounded to bf16 to nearest-even
                                  first, as the weight is packed) */
    const void *mask;          /* u8 [rows, mask_ld] (mask_ld 0: one row shared) or NULL */
    int64_t mask_ld;
    double temperature;        /* >= 0 and finite; 0 = greedy */
    const double *uniforms;    /* [rows] device, each in (0,1); unused when greedy */
    int32_t *ids;              /* [rows] out: the sampled token (-1 on a refused row) */
    float *logp;               /* [rows] out or NULL */
    uint8_t *status;           /* [rows] out: NT_ROW_* */
    float *logits;             /* debug: [rows, vocab] f32 out or NULL */
    float *debug_block;        /* debug: [rows, 32] the crossing block's recomputed logits, or NULL */
    int32_t *debug_block_index; /* debug: [rows] that block's index (columns 32 b .. 32 b + 31), or NULL */
} NtRlReadoutSampleArgs;
int nt_hip_rl_readout_sample(const NtRlReadoutSampleArgs *a);

/* The readout-fused scorer: the same readout product, then for each row
 *   logp[r]    = token_log_probs(z, tokens)[r]       (rl.rs:134-141)
 *   entropy[r] = categorical_entropy(z)[r]          (rl.rs:405-414)
 * with z = tempered_logits(hidden . W, T, mask) (rl.rs:475-486), as nt_hip_rl_score computes
 * them on written logits (same refusals and statuses: an excluded token has logp -inf, a token
 * outside [0, vocab) gives NT_ROW_BAD_TOKEN and logp NaN), with the logits never written: the
 * scoring pass of an RL step from the decoder's hidden states (decoder.rs:272,286). Shapes,
 * packing and limits as nt_hip_rl_readout_sample; temperature > 0. Three launches: h into the
 * matrix cores' order, the product with per-row records in its epilogue (block sums, for the
 * entropy each block's sum of w (x c - ref), and each row's token logit), then one workgroup per
 * row that merges the records. */
typedef struct NtRlReadoutScoreArgs {
    const void *hidden;        /* [rows, ldh] hidden_dtype */
    const void *weight_packed; /* packed by nt_hip_rl_readout_pack_weight */
    int64_t rows, vocab, dim, ldh;
    int32_t mask_kind;         /* NT_MASK_NONE | NT_MASK_U8 */
    int32_t hidden_dtype;      /* NT_BF16 | NT_F32 | NT_F16 */
    const void *mask;          /* u8 [rows, mask_ld] (mask_ld 0: one row shared) or NULL */
    int64_t mask_ld;
    double temperature;        /* > 0 and finite */
    const int32_t *tokens;     /* [rows] device, or NULL when only the entropy is asked for */
    float *logp;               /* [rows] out or NULL */
    float *entropy;            /* [rows] out or NULL (one of logp, entropy) */
    uint8_t *status;           /* [rows] out: NT_ROW_* */
    float *logits;             /* debug: [rows, vocab] f32 out or NULL */
} NtRlReadoutScoreArgs;
int nt_hip_rl_readout_score(const NtRlReadoutScoreArgs *a);

/* Fused row scoring: for each row, any of
 *   logp[r]     = token_log_probs(z, tokens)[r]                 (rl.rs:134-141)
 *   ref_logp[r] = token_log_probs(zr, tokens)[r]                (rl.rs:134-141, reference)
 *   kl[r]       = categorical_kl(z, zr) per position (exact)    (rl.rs:327-338)
 *   entropy[r]  = categorical_entropy(z) per position           (rl.rs:405-414)
 * with z = tempered_logits(logits, T, mask) and zr = tempered_logits(ref_logits, T, mask)
 * (`reference_kl`, rl.rs:347-351; T = 1 and no mask give `categorical_kl`). One pass reads
 * each logit (and the mask) once. A token excluded by the mask gives logp -inf, as the
 * reference does (rl.rs:136-137). */
typedef struct NtRlScoreArgs {
    const void *logits;       /* [rows, ld] policy logits */
    const void *ref_logits;   /* [rows, ld] reference logits or NULL (no ref_logp / kl) */
    int32_t dtype;            /* NT_F32 | NT_BF16 | NT_F16 (both inputs) */
    int32_t mask_kind;
    int64_t rows, vocab, ld;
    const void *mask;
    int64_t mask_ld;
    double temperature;       /* > 0 and finite */
    const int32_t *tokens;    /* [rows] device, each in [0, V); NULL when no logp is asked */
    float *logp;              /* [rows] out or NULL */
    float *ref_logp;          /* [rows] out or NULL */
    float *kl;                /* [rows] out or NULL */
    float *entropy;           /* [rows] out or NULL */
    uint8_t *status;          /* [rows] out or NULL: NT_ROW_* of the policy row */
    /* The row's log-sum-exp, for nt_hip_rl_score_backward: lse = lse_base + lse_rest with
     * lse_base a finite point at most 5 ln 2 below the maximum of the tempered logits and
     * lse_rest = ln sum exp(z - lse_base); both NaN on a refused row. Any of the four may be
     * NULL. */
    float *lse_base;          /* [rows] out or NULL (policy) */
    float *lse_rest;          /* [rows] out or NULL (policy) */
    float *ref_lse_base;      /* [rows] out or NULL (reference; needs ref_logits) */
    float *ref_lse_rest;      /* [rows] out or NULL (reference) */
    NtMaskRows mask_rows;     /* a mask broadcast over leading dimensions (zero: rows of mask_ld) */
} NtRlScoreArgs;
int nt_hip_rl_score(const NtRlScoreArgs *a);

/* The fused backward of nt_hip_rl_score: for each row, the gradient with respect to the raw
 * logits x of
 *   g_logp[r] * logp[r] + g_kl[r] * kl[r] + g_entropy[r] * entropy[r]
 * with z = x / T + mask (tempered_logits, rl.rs:475-486), pi = softmax(z), log pi_v =
 * (z_v - lse_base) - lse_rest:
 *   dlogp/dz_v    = [v == token] - pi_v                     (log_softmax backward,
 *                                                            activation.rs:36-41, gathered)
 *   dkl/dz_v      = pi_v ((log pi_v - log pi_ref,v) - kl)   (categorical_kl, rl.rs:327-338;
 *                                                            the reference is detached)
 *   dentropy/dz_v = -pi_v (log pi_v + entropy)              (categorical_entropy, rl.rs:405-414)
 *   dL/dx_v       = dL/dz_v / T                             (the divide's backward)
 * An entry with pi_v = 0 (excluded, or -inf) gets only the token term. Inputs are the forward's
 * outputs for the same logits, temperature and mask (the statistics from nt_hip_rl_score). The
 * gradient is written in grad_dtype (bf16 by round-to-nearest-even from the f32 value, as the
 * reference stores a bf16 tensor's gradient), row stride grad_ld. One pass reads each logit
 * (and reference logit) once and writes each gradient element once. */
typedef struct NtRlScoreGradArgs {
    const void *logits;       /* [rows, ld] policy logits (NT_F32 | NT_BF16 | NT_F16) */
    const void *ref_logits;   /* [rows, ld] reference logits; needed when g_kl is given */
    int32_t dtype;
    int32_t mask_kind;
    int64_t rows, vocab, ld;
    const void *mask;
    int64_t mask_ld;
    double temperature;       /* > 0 and finite; the forward's */
    const int32_t *tokens;    /* [rows]; needed when g_logp is given */
    const float *lse_base, *lse_rest;          /* [rows] from the forward (policy) */
    const float *ref_lse_base, *ref_lse_rest;  /* [rows] from the forward (reference) */
    const float *kl;          /* [rows] the forward's exact KL; needed when g_kl is given */
    const float *entropy;     /* [rows] the forward's entropy; needed when g_entropy is given */
    const float *g_logp;      /* [rows] upstream gradients, or NULL (zero) */
    const float *g_kl;
    const float *g_entropy;
    void *grad;               /* [rows, grad_ld] out */
    int32_t grad_dtype;       /* NT_F32 | NT_BF16 | NT_F16 (16-bit: the f32 gradient rounded to nearest even) */
    int32_t pad0;
    int64_t grad_ld;
    NtMaskRows mask_rows;     /* the forward's */
} NtRlScoreGradArgs;
int nt_hip_rl_score_backward(const NtRlScoreGradArgs *a);

/* kl_estimate per sampled token (rl.rs:380-400), elementwise over n = S*B*T values:
 * delta = ref_logp - logp, zeroed where mask == 0 (a select, rl.rs:100-102), clamped to
 * [-clamp, clamp] when clamp > 0; estimator 1: -delta, 2: delta^2/2, 3: exp(delta)-delta-1;
 * the result is zero at masked positions. mask (f32 0/1) may be NULL. */
int nt_hip_rl_kl_estimate(const float *logp, const float *ref_logp, const float *mask, int64_t n,
                          int32_t estimator, double clamp, float *out);

/* zero_masked (rl.rs:100-102): out = mask != 0 ? x : 0, a select (a non-finite value at a
 * masked position does not leak). */
int nt_hip_rl_zero_masked(const float *x, const float *mask, int64_t n, float *out);

/* reduce_tokens (rl.rs:69-92) of per-token values [S,B,T] that are already zero at masked
 * positions, mask f32 [S,B,T] (NULL = every position scored): reduction 1 Sum [S],
 * 2 TokenMean [S], 3 PerSequence [S,B], 4 SequenceMean [S]. Each output is summed in a fixed
 * order by one thread. */
int nt_hip_rl_reduce_tokens(const float *per, const float *mask, int64_t S, int64_t B, int64_t T,
                            int32_t reduction, float *out);

/* The backward of reduce_tokens after zero_masked (rl.rs:69-102): for each position of
 * [S,B,T], out = mask != 0 ? scale * upstream[o] * dR/dper * local : 0, where o is the reduced
 * output the position feeds and dR/dper is 1 (None, Sum), 1/max(sum_s m, 1) (TokenMean),
 * 1/max(sum_t m, 1) (PerSequence) or 1/(max(sum_t m, 1) * max(sequences of the seed with a
 * scored position, 1)) (SequenceMean). upstream has the reduced shape ([S,B,T] for None, [S,B]
 * for PerSequence, [S] otherwise); NULL means ones. local ([S,B,T], NULL = ones) is the
 * per-token derivative of the loss being reduced (nt_hip_rl_policy_loss's dloss), so that out is
 * that loss's gradient with respect to logp. mask NULL scores every position. */
int nt_hip_rl_reduce_tokens_backward(const float *mask, int64_t S, int64_t B, int64_t T, int32_t reduction,
                                     const float *upstream, double scale, const float *local, float *out);

/* kl_estimate's derivative with respect to logp per sampled token (rl.rs:380-400), with the
 * same arguments as nt_hip_rl_kl_estimate: with delta = ref_logp - logp, 1 (k1), -delta (k2),
 * 1 - exp(delta) (k3); zero where the clamp is active (|delta| > clamp) and at masked
 * positions. */
int nt_hip_rl_kl_estimate_backward(const float *logp, const float *ref_logp, const float *mask, int64_t n,
                                   int32_t estimator, double clamp, float *out);

/* group_advantages_tensor (rl.rs:416-469) on the device: rewards [groups, n] (f32, row-major),
 * each reward minus its group's mean, divided by the group's standard deviation plus eps when
 * norm is 1 (GroupNorm::Std; unbiased 1: the sample standard deviation, n - 1, which needs
 * n >= 2; 0: the population one) or by 1 when norm is 0 (MeanOnly); a group whose rewards are all
 * equal gives exact zeros. In f64, with the group's sums taken left to right as the reference's
 * host loop takes them, then rounded to f32. */
int nt_hip_rl_group_advantages(const float *rewards, int64_t groups, int64_t n, int32_t norm, double eps,
                               int32_t unbiased, float *out);

enum { NT_LOSS_PG = 0, NT_LOSS_PPO = 1 };

/* The policy losses per token (rl.rs:228-317), before reduce_tokens.
 *   kind NT_LOSS_PG:  policy_gradient_loss (rl.rs:228-235), loss = -(w * logp);
 *   kind NT_LOSS_PPO: clipped_policy_loss (rl.rs:265-287): d = logp - old_logp (0 at masked
 *     positions), clamped to [-log_ratio_clamp, log_ratio_clamp] when log_ratio_clamp > 0;
 *     r = exp(d); loss = max(-r A, -clip(r, 1 - clip_low, 1 + clip_high) A) by a select; with a
 *     dual clip c (dual > 0, c > 1) a token with A < 0 has min(loss, -c A).
 * weights are the weights (PG) or advantages (PPO), per token [S,B,T] or per sequence [S,B]
 * (weights_per_sequence = 1). mask f32 [S,B,T], NULL = every position scored. Outputs, each
 * [S,B,T] and optional:
 *   loss   the per-token loss, 0 at masked positions (TokenReduction::None's values);
 *   dloss  d loss / d logp per token (0 at masked positions and where a bound is active; the
 *          op sequence's autograd, including its NaN for an overflowed ratio without the clamp);
 *   hit    clip_fraction's numerator (rl.rs:293-317): 1 where the token gets no gradient
 *          through a bound (A > 0, r > 1 + high; A < 0, r < 1 - low; A < 0, r > c under a dual
 *          clip; |d| beyond the clamp), times the mask; its TokenMean is clip_fraction.
 * Arguments follow Clip::check (rl.rs:189-200): 0 <= clip_low < 1, 0 <= clip_high, dual 0 or
 * c > 1, log_ratio_clamp 0 (unbounded) or b > 0. */
typedef struct NtRlPolicyLossArgs {
    const float *logp;
    const float *old_logp; /* PPO only */
    const float *weights;
    const float *mask;
    int64_t S, B, T;
    int32_t kind;
    int32_t weights_per_sequence;
    double clip_low, clip_high, dual, log_ratio_clamp;
    float *loss, *dloss, *hit;
} NtRlPolicyLossArgs;

int nt_hip_rl_policy_loss(const NtRlPolicyLossArgs *a);

#ifdef __cplusplus
}
#endif
#endif
