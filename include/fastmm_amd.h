/*
 * fastmm_amd.h -- C ABI of the MI355X (gfx950) fast-matmul Linear backend.
 *
 * The reference (chelokot/rdna3-fastmm) is Python + Triton and has no FFI of
 * its own: its plan methods launch one Triton kernel (or one torch.bmm) per
 * stage. Each entry point below replaces exactly one of those launches, with
 * the same meaning, so the Python host layer (rdna3_fastmm.runtime / .linear)
 * can keep the reference's plan and operator API and call these instead.
 * Reference citations are paths in the reference repository.
 *
 * Conventions for every entry point:
 *   - all pointers are device pointers on the current HIP device, contiguous,
 *     row-major, and must not overlap (the host layer checks this);
 *   - `stream` is a hipStream_t (NULL = the legacy default stream); work is
 *     enqueued asynchronously, nothing synchronizes;
 *   - returns FASTMM_OK or an error code; fastmm_last_error() then describes
 *     the failure (thread-local). Argument errors are reported before any
 *     launch, so a failed call leaves every buffer untouched;
 *   - block sizes follow the scheme's partition: with s = scheme size,
 *     Mb = ceil(rows/s), Kb = ceil(inner/s), Nb = ceil(columns/s)
 *     (runtime.py:66-78); rows/columns past the matrix read as zero.
 *
 * Layouts:
 *   x / input      [rows, inner]            dtype (bf16 or fp16)
 *   weight         [columns, inner]         dtype  (F.linear layout)
 *   right          [inner, columns]         dtype  (mm path)
 *   left_transformed  A'[R, Mb, Kb]         fp16 or bf16 (operand layout below)
 *   right_transformed B'[R, Nb, Kb]         fp16 or bf16 (operand layout below; the
 *        reference stores [R, Kb, Nb] and transposes inside torch.bmm)
 *   products       P[R, Mb, Nb]             fp16, bf16 or fp32, row-major
 *   bias           [columns]                dtype
 *   output         [rows, columns]          dtype
 *
 * Operand layout of A' and B' (same element count as [R, rows, Kb]): when
 * Kb % 32 == 0 each plane is K-slab-major, element (row, k) at
 *     ((k / 32) * rows + row) * 32 + k % 32        (rows = Mb or Nb),
 * so the 32-wide K slice of a run of rows is contiguous; otherwise each plane
 * is row-major, element (row, k) at row * Kb + k. The transforms write and
 * fastmm_leaf_products reads this layout; buffers written by one library
 * version are only valid for the same FASTMM_ABI_VERSION.
 */
#ifndef FASTMM_AMD_H
#define FASTMM_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FASTMM_ABI_VERSION 5

#define FASTMM_OK 0
#define FASTMM_ERROR_ARGUMENT 1    /* bad pointer, size, dtype or scheme */
#define FASTMM_ERROR_UNSUPPORTED 2 /* valid request this build does not run */
#define FASTMM_ERROR_LAUNCH 3      /* the HIP runtime rejected a launch */

#define FASTMM_BF16 0
#define FASTMM_FP16 1
#define FASTMM_FP32 2

#define FASTMM_SCHEME_RANK7 0  /* <2,2,2> rank 7  (certificate 2x2x2_rank7_15add) */
#define FASTMM_SCHEME_RANK48 1 /* <4,4,4> rank 48 (certificate 4x4x4_rank48_accurate) */
#define FASTMM_SCHEME_RANK49 2 /* <4,4,4> rank 49 (certificate 4x4x4_rank49_159add) */
#define FASTMM_SCHEME_RANK343 3 /* <8,8,8> rank 343 (certificate 8x8x8_rank343_1661add); fp16 only */

/* Library identity. */
int fastmm_abi_version(void);
const char* fastmm_last_error(void);

/* Scheme metadata compiled into the kernels; the host layer compares the
 * digest with the certificate it verified, as the reference checks its
 * generated modules at import (runtime.py:16-53). Returns FASTMM_OK or
 * FASTMM_ERROR_ARGUMENT. */
int fastmm_scheme_info(int scheme, int* size, int* rank);
const char* fastmm_scheme_sha256(int scheme);

/* A-side transform x[rows, inner] (dtype) -> A'[R, Mb, Kb] in plane_dtype
 * (FASTMM_FP16 or FASTMM_BF16: the plan's compute dtype, fp32 program value
 * rounded to nearest even). Replaces _LinearPlan._transform_left +
 * left_transform_kernel (runtime.py:597-615; generated/rank7_2x2x2.py:9-62),
 * whose planes have the plan's compute dtype (runtime.py:216-252). */
int fastmm_left_transform(int scheme, int dtype, int plane_dtype, const void* input,
                          void* left_transformed, int64_t rows, int64_t inner, void* stream);

/* Weight transform W[columns, inner] -> B'[R, Nb, Kb] in plane_dtype (prepack
 * and the dynamic path). Replaces _LinearPlan._transform_weight +
 * right_transform_weight_kernel (runtime.py:637-655; rank7_2x2x2.py:121-204). */
int fastmm_weight_transform(int scheme, int dtype, int plane_dtype, const void* weight,
                            void* right_transformed, int64_t columns, int64_t inner, void* stream);

/* Right transform right[inner, columns] -> B'[R, Nb, Kb] in plane_dtype (mm
 * path). Replaces _LinearPlan._transform_right + right_transform_kernel
 * (runtime.py:617-635; rank7_2x2x2.py:65-118). */
int fastmm_right_transform(int scheme, int dtype, int plane_dtype, const void* right,
                           void* right_transformed, int64_t inner, int64_t columns, void* stream);

/* Leaf products P[r] = A'[r] @ B'[r]^T for r < rank on FP16 or BF16 MFMA
 * (operand_dtype = the planes' type) with fp32 accumulation, stored as
 * products_dtype: operand_dtype (the reference's torch.bmm rounding) or
 * FASTMM_FP32 (no product rounding).
 * Replaces torch.bmm(A', B', out=P) (runtime.py:728-732, 768-772).
 *
 * scratch / scratch_bytes: caller-owned device memory (16-byte aligned) for
 * the split-K tail, at least fastmm_leaf_scratch_bytes() for the same
 * arguments on the current device, or NULL / 0. With it, the last partial
 * round of 256x256 tiles is split along K over the idle compute units and
 * its fp32 parts are added in K order before the one products rounding;
 * without it the tail runs as whole tiles (same results up to fp32 summation
 * order). Calls that share one scratch buffer must not overlap. */
int fastmm_leaf_products(int rank, int operand_dtype, const void* left_transformed,
                         const void* right_transformed, void* products, int products_dtype,
                         int64_t block_rows, int64_t block_inner, int64_t block_columns,
                         void* scratch, int64_t scratch_bytes, void* stream);

/* fastmm_leaf_products without caller scratch and without any allocation: the
 * split-K tail's fp32 parts go to a device array that the library holds
 * (FASTMM_STATIC_SCRATCH_BYTES = 48 MiB, one copy per GPU the library runs
 * on, kept until the process ends), so the results are the same bits as
 * fastmm_leaf_products given enough scratch. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). It calls no
 * hipMalloc/hipFree. Shapes whose tail would need more than the array return
 * FASTMM_ERROR_UNSUPPORTED (on a 256-CU MI355X the tail never needs more).
 * Every call on one GPU shares that GPU's array: calls that overlap in time
 * on one GPU (other streams, other host threads) race and must not be issued;
 * calls on one stream are ordered and safe. */
#define FASTMM_STATIC_SCRATCH_BYTES (48LL << 20)
int fastmm_leaf_products_noalloc(int rank, int operand_dtype, const void* left_transformed,
                                 const void* right_transformed, void* products, int products_dtype,
                                 int64_t block_rows, int64_t block_inner, int64_t block_columns, void* stream);

/* Scratch bytes fastmm_leaf_products can use for these arguments on the
 * current device (0 when the shape runs no split-K tail). No counterpart in
 * the reference (torch.bmm manages its own workspace). */
int fastmm_leaf_scratch_bytes(int rank, int operand_dtype, int products_dtype, int64_t block_rows,
                              int64_t block_inner, int64_t block_columns, int64_t* bytes);

/* Output recombination P[R, Mb, Nb] (products_dtype: fp16, bf16 or fp32) ->
 * output[rows, columns] in dtype, with an optional bias[columns] (NULL = none)
 * added in fp32 after the scheme's sum. Replaces _reconstruct / _reconstruct_bias + output_transform[_bias]_kernel
 * (runtime.py:657-698; rank7_2x2x2.py:207-345).
 * The 8x8-block scheme runs the reference's dense form instead
 * (Rank343Plan._reconstruct, runtime.py:938-962: every output block as one
 * fp32-accumulated MFMA contraction of the products with the scheme's -1/0/1
 * output matrix) when the products are fp16, there is no bias, columns % 64
 * == 0 (whole 8-column blocks of whole 8-position groups), the products are
 * 16-byte aligned and the output 8-byte aligned; its other inputs run the
 * output circuit. The two forms agree up to fp32 summation order, so results
 * can differ in the last bit between them. */
int fastmm_reconstruct(int scheme, int products_dtype, const void* products, const void* bias,
                       int dtype, void* output, int64_t rows, int64_t columns, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FASTMM_AMD_H */
