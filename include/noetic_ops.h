/* noetic_ops.h: the general device ops of a Device::Hip tensor that the nn::rl chain uses around
 * the fused entry points (noetic_hip.h): strided copies and writes, casts, elementwise unary,
 * compare, binary and mask_fill, reductions along one dimension or over everything, and the
 * indexing ops. Each entry point is one method of the reference's `GpuBackend` trait
 * (src/tensor/gpu/mod.rs:137-207) with the trait's argument meaning:
 *   - every output is fresh, contiguous and row-major over the op's shape (the caller allocates
 *     it with nt_hip_alloc and passes it in);
 *   - inputs are read in place through an NtLayout (a view: shape, element strides, element
 *     offset; a stride of 0 broadcasts), as the reference's kernels read a Layout;
 *   - float kernels compute in f32 (f16 and bf16 are cast to f32 first, as the reference's
 *     dispatch does, gpu/mod.rs:336-342).
 * Calls are stream-ordered on the library's stream (nt_hip_stream) and return 0 or an NT_E_*
 * code (noetic_hip.h) with nt_hip_last_error() text. No entry point allocates device memory.
 */
#ifndef NOETIC_OPS_H
#define NOETIC_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NT_MAX_RANK 8

/* A view of a buffer: element i of the row-major iteration over `shape` is the element at
 * offset + sum_d coord_d * strides[d] (elements, not bytes). Layout, src/tensor/layout.rs:8-12.
 * The reference's broadcast (layout.rs:71-80) gives stride 0 on expanded dimensions. */
typedef struct NtLayout {
    int32_t rank; /* 0..NT_MAX_RANK (rank 0 is one element) */
    int32_t pad_;
    int64_t offset;
    int64_t shape[NT_MAX_RANK];
    int64_t strides[NT_MAX_RANK];
} NtLayout; /* 144 bytes */

/* Element types of a GPU buffer (DType, src/tensor/dtype.rs:9-18; F64 is not a device type
 * here, as on the reference's CUDA backend). NT_F32 and NT_BF16 are those of noetic_hip.h. */
#define NT_DT_F32 0
#define NT_DT_BF16 1
#define NT_DT_F16 2
#define NT_DT_BOOL 3 /* one byte, 0 or 1 */
#define NT_DT_U8 4
#define NT_DT_I32 5
#define NT_DT_I64 6

/* UnaryOp codes (gpu/mod.rs:68-103, `UnaryOp::code`). */
#define NT_UN_NEG 0
#define NT_UN_EXP 1
#define NT_UN_LOG 2
#define NT_UN_SQRT 3
#define NT_UN_RECIP 4
#define NT_UN_ABS 5
#define NT_UN_SIGN 6
#define NT_UN_SIGMOID 7 /* 1 / (1 + e^-x) for x >= 0, e^x / (1 + e^x) below, in f32 */
#define NT_UN_ADD_SCALAR 8
#define NT_UN_SUB_SCALAR 9
#define NT_UN_MUL_SCALAR 10
#define NT_UN_DIV_SCALAR 11
#define NT_UN_POW_SCALAR 12 /* C99 powf */

/* CmpOp codes (gpu/mod.rs:107-114). */
#define NT_CMP_GT 0
#define NT_CMP_GE 1
#define NT_CMP_LT 2
#define NT_CMP_LE 3
#define NT_CMP_EQ 4

/* BinaryOp codes (gpu/mod.rs:116-122). */
#define NT_BIN_ADD 0
#define NT_BIN_SUB 1
#define NT_BIN_MUL 2
#define NT_BIN_DIV 3

/* ReduceOp codes (gpu/mod.rs:124-133). */
#define NT_RED_SUM 0
#define NT_RED_MAX 1
#define NT_RED_ARGMAX 2

/* GpuBackend::copy (gpu/mod.rs:140-141): the elements `xl` selects, contiguous, any element type
 * (elem_bytes 1, 2, 4 or 8). */
int nt_hip_copy(const void *x, const NtLayout *xl, int32_t elem_bytes, void *out);

/* GpuBackend::write (gpu/mod.rs:179-180): copy the view `sl` of src into the view `dl` of dst
 * (same shape, same element type); dst is changed in place. */
int nt_hip_write(void *dst, const NtLayout *dl, const void *src, const NtLayout *sl, int32_t elem_bytes);

/* GpuBackend::cast (gpu/mod.rs:142-144): f16/bf16/bool -> f32, f32 -> f16/bf16 (round to
 * nearest even, NaN kept quiet: half.rs:14-60), f16 <-> bf16 through f32, same type = copy. */
int nt_hip_cast(const void *x, const NtLayout *xl, int32_t from, int32_t to, void *out);

/* GpuBackend::unary (gpu/mod.rs:145): out = op(x) (f32). exp, ln and pow are rounded to f32 from
 * an f64 evaluation (the nearest f32 except when the exact value lies within about 2^-29 ulp
 * of a rounding midpoint). */
int nt_hip_unary(int32_t op, float scalar, const float *x, const NtLayout *xl, float *out);

/* GpuBackend::compare (gpu/mod.rs:146-147): out = (x op scalar) as bool bytes (a NaN compares
 * false). */
int nt_hip_compare(int32_t op, float scalar, const float *x, const NtLayout *xl, uint8_t *out);

/* GpuBackend::binary (gpu/mod.rs:148-149): out = a op b over al's shape; al and bl are already
 * broadcast to that shape (equal shapes, stride 0 on expanded dimensions). */
int nt_hip_binary(int32_t op, const float *a, const NtLayout *al, const float *b, const NtLayout *bl, float *out);

/* GpuBackend::mask_fill (gpu/mod.rs:150-151): out = mask != 0 ? value : x; ml broadcast to xl's
 * shape. */
int nt_hip_mask_fill(const float *x, const NtLayout *xl, const uint8_t *mask, const NtLayout *ml, float value,
                     float *out);

/* GpuBackend::reduce_dim (gpu/mod.rs:152-153) of contiguous f32 x read as [outer, n, inner],
 * the dimension kept (size 1): out is f32 [outer, inner] (Sum, Max) or int32 (ArgMax).
 * Sum follows CpuRef's order exactly (kernels.rs:120-174): along the last axis (last_axis != 0)
 * each lane is folded with eight partial sums (ndarray's unrolled_fold), along any other axis the
 * slices are added in order from zero; the results equal CpuRef's bit for bit. Max and ArgMax
 * take the first maximum, NaN-propagating (the first NaN is the maximum). n == 0 is refused for
 * Max and ArgMax. */
int nt_hip_reduce_dim(int32_t op, const float *x, int64_t outer, int64_t n, int64_t inner, int32_t last_axis,
                      void *out);

/* GpuBackend::reduce_all (gpu/mod.rs:154-155): Sum (the eight-partial fold over all n) or Max
 * (NaN-propagating) of contiguous f32 x, one f32. */
int nt_hip_reduce_all(int32_t op, const float *x, int64_t n, float *out);

/* GpuBackend::gather (gpu/mod.rs:169-170): out[o, k, i] = x[o, idx[o, k, i], i] for contiguous
 * x [outer, n, inner] and int32 idx [outer, m, inner]. The reference's host checks the indices
 * first (src/tensor/infer.rs:110-125); an index outside [0, n) gives NaN here, never a read out of
 * bounds. */
int nt_hip_gather(const float *x, int64_t outer, int64_t n, int64_t inner, const int32_t *idx, int64_t m, float *out);

/* GpuBackend::index_select (gpu/mod.rs:171-172): out[o, k, i] = x[o, idx[k], i] (m indices). */
int nt_hip_index_select(const float *x, int64_t outer, int64_t n, int64_t inner, const int32_t *idx, int64_t m,
                        float *out);

/* GpuBackend::one_hot (gpu/mod.rs:173-174): out[c, j] = idx[c] == j ? 1 : 0, f32 [count, n]. */
int nt_hip_one_hot(const int32_t *idx, int64_t count, int64_t n, float *out);

/* GpuBackend::scatter_add (gpu/mod.rs:175-176): out[o, j, i] = the sum, in ascending k, of
 * v[o, k, i] over the k with idx[o, k, i] == j (zeros elsewhere): out f32 [outer, n, inner] from
 * v and idx [outer, m, inner]. Deterministic: one thread per target, no atomics. */
int nt_hip_scatter_add(const int32_t *idx, const float *v, int64_t outer, int64_t n, int64_t inner, int64_t m,
                       float *out);

/* GpuBackend::index_add (gpu/mod.rs:177-178): out[o, j, i] = the sum, in ascending k, of
 * v[o, k, i] over the k with idx[k] == j. */
int nt_hip_index_add(const int32_t *idx, const float *v, int64_t outer, int64_t n, int64_t inner, int64_t m,
                     float *out);

/* GpuBackend::fill (gpu/mod.rs:190-193): n f32 elements equal to value. */
int nt_hip_fill(float *out, int64_t n, float value);

/* GpuBackend::matmul (gpu/mod.rs:155-156; the CUDA backend's matmul, cuda/backend.rs:784-830):
 * the batched product of two f32 views a [..., m, k] and b [..., k, n] of equal rank >= 2, batch
 * dimensions broadcast where one side is 1, into contiguous out [batch..., m, n]. Every output is
 * the reference's arithmetic (cuda/kernels.rs:14-20, CpuRef's matrixmultiply order): an fma chain
 * from zero over k in order, closed every 256 k, the first block's chain the total and each later
 * block's chain added to it; so the result equals CpuRef's bit for bit. k = 0 gives zeros. */
int nt_hip_matmul(const float *a, const NtLayout *al, const float *b, const NtLayout *bl, float *out);

/* GpuBackend::matmul_half (gpu/mod.rs:157-162; the CUDA backend's hgemm_bf16_f32acc,
 * cuda/half_gemm.rs:32-..., backend.rs:750-773): the same batched product of two f32 views with
 * each operand rounded to bf16 (nearest even) and the products summed in f32 on the matrix cores
 * (v_mfma_f32_32x32x16_bf16). Compared with a stated tolerance, not byte for byte: within
 * 2^-21 k sum|a||b| of the rounded operands' exact product (src/tensor/tests/gpu/half_gemm.rs:73-104);
 * the same bits run to run. */
int nt_hip_matmul_half(const float *a, const NtLayout *al, const float *b, const NtLayout *bl, float *out);
/* GpuBackend::half_gemm_key (gpu/mod.rs:163-167; cuda/backend.rs:775-783): the reduced-precision
 * product's key part, "gemm-bf16-mfma32x32x16-f32acc-kernels-<sha16 of the device sources>",
 * NUL-terminated into buf. */
int nt_hip_half_gemm_key(char *buf, size_t cap);

/* GpuBackend::sort_desc (gpu/mod.rs:186-191; CpuRef's order, kernels.rs:374-413): along the
 * middle of contiguous f32 x [outer, n, inner], descending: every NaN first (all NaNs equal),
 * then total_cmp (+0 before -0), ties in ascending source position. vals gets the source values
 * (NaN payloads kept), idx their I32 positions along the lane, both [outer, n, inner]. Every
 * lane length runs on the device (the CUDA backend sends lanes past 4096 through the host,
 * cuda/backend.rs:919-937); lanes past 8192 take 16 bytes of scratch per element. */
int nt_hip_sort_desc(const float *x, int64_t outer, int64_t n, int64_t inner, float *vals, int32_t *idx);

#ifdef __cplusplus
}
#endif

#endif /* NOETIC_OPS_H */
