/*
 * w6a16.h -- C ABI of the weight-only 6-bit GEMM in librwkv7_hip.so (gfx950).
 *
 * Replaces the reference's W6A16 Triton GEMM/GEMV `_w6a16` and its launcher `_impl`
 * (rwkv_next/kernels/int6_gemm.py:156-215, 253-287), behind the op `rwkv_next::int6_matmul` (int6_gemm.py:316-323)
 * that the model's quantised linear layers call (rwkv_next/model.py:63-66).  The weight format is the reference's
 * own (int6_gemm.py:14-38, 73-112), so weights quantised by the reference load unchanged:
 *   lo     uint8 [B'][K/2][N]   lo[c*32 + j][n] = lo4(row c*64 + j) | lo4(row c*64 + j + 32) << 4, j < 32
 *   hi     uint8 [B'][K/4][N]   hi[c*16 + j][n] = hi2(j) | hi2(j + 16) << 2 | hi2(j + 32) << 4 | hi2(j + 48) << 6
 *   scales fp16  [B'][K/group_k][N]
 * with u = q + 32 in [0, 63] the stored code of q in [-32, 31] and w = scale * q.
 *
 * C[b][m][n] = sum_k A[b][m][k] * w[b][k][n], A bf16 or fp16 row-major (k contiguous), fp32 accumulation.
 * Return codes are the WKV7_* codes of wkv7.h.
 */
#ifndef RWKV_NEXT_AMD_W6A16_H
#define RWKV_NEXT_AMD_W6A16_H

#include <stddef.h>
#include <stdint.h>

#include "wkv7.h"

#ifdef __cplusplus
extern "C" {
#endif

#define W6A16_OUT_BF16 0
#define W6A16_OUT_F16 1
#define W6A16_OUT_F32 2

/* Activation types of w6a16_args.a_dtype (the reference takes a.dtype, int6_gemm.py:144-147, 253-287) */
#define W6A16_IN_BF16 0
#define W6A16_IN_F16 1

/* Weight formats of w6a16_args.format */
#define W6A16_FORMAT_PLANES 0   /* the reference's planes: lo, hi, scales as above */
#define W6A16_FORMAT_PACKED 1   /* w6a16_pack's layout: lo = packed weight, scales = packed scales, hi unused */

typedef struct w6a16_args {
    const uint16_t *a;                 /* activations [B][M][K], bf16 or fp16 (a_dtype) */
    int64_t a_batch_stride, a_row_stride;          /* elements; row stride >= K, multiples of 8 */
    const uint8_t *lo, *hi;            /* weight planes; batch strides 0 to share one weight across the batch */
    int64_t lo_batch_stride, hi_batch_stride;      /* bytes */
    const uint16_t *scales;            /* fp16, 4-byte aligned */
    int64_t scales_batch_stride;       /* elements */
    void *out;                         /* [B][M][N] bf16, fp16 or fp32 (out_dtype) */
    int64_t out_batch_stride, out_row_stride;      /* elements */
    void *workspace;                   /* split_k > 1 or M > 32: w6a16_workspace_size bytes, 256-byte aligned */
    size_t workspace_bytes;
    int32_t B, M, N, K;                /* K % 64 == 0, N % 16 == 0; M <= 32: B * ceil(M / 16) <= 65535,
                                          M > 32: B <= 65535 */
    int32_t group_k;                   /* % 64 == 0, divides K */
    int32_t split_k;                   /* 1 .. 256: K is cut into split_k ranges of 64-row chunks */
    int32_t out_dtype;                 /* W6A16_OUT_BF16, W6A16_OUT_F16 or W6A16_OUT_F32 */
    int32_t format;                    /* W6A16_FORMAT_PLANES or W6A16_FORMAT_PACKED */
    int32_t a_dtype;                   /* W6A16_IN_BF16 (0) or W6A16_IN_F16 */
} w6a16_args;

/* sizeof(w6a16_args) as compiled into the library (bindings check their struct layout against it). */
size_t w6a16_args_size(void);

/* Bytes of workspace `w6a16_matmul` needs (0 for split_k == 1 and M <= 32, for W6A16_FORMAT_PACKED with M > 256 (the
 * large-M kernel), and for M <= 32 with split_k 2..8 where the
 * in-workgroup split-K kernel runs: always for W6A16_FORMAT_PACKED, and for the planes when B * ceil(M / 16) *
 * ceil(N / 128) reaches the device's CU count; that kernel sums its split_k partial tiles in LDS): a fixed 1 MiB region of u32 arrival
 * counters (one per output tile; a call with more than 262144 tiles is refused with WKV7_ERR_SHAPE), then fp32
 * partial tiles (split_k > 1), then, for M > 32, the per-row sums of A that a small first launch computes and the
 * GEMM kernel reads.  The split that completes a tile last reduces it inside the kernel.  Contract: the counter
 * region (the first 1 MiB) must be zero before the workspace's first use; every completed call leaves it zero again
 * and never writes partials into it, so one workspace serves any number of calls of any shapes issued one after
 * another (stream order).  Calls that can run at the same time (different streams) need different workspaces. */
int w6a16_workspace_size(const w6a16_args *args, size_t *bytes);

/* Split-K for a shape: the smallest power of two (<= 64, every range keeping at least one 64-row chunk) that gives
 * every CU at least one workgroup, then doubled while ranges keep at least sixteen 64-row chunks and the launch stays
 * within two workgroups per CU.  Replaces the split-K rule of plan_int6 (rwkv_next/kernels/int6_gemm.py:239-250). */
int w6a16_plan_split(int32_t B, int32_t M, int32_t N, int32_t K);

/* split_k for the packed layout (W6A16_FORMAT_PACKED), whose in-workgroup kernel prefers a shallower split where it
 * runs half strips; otherwise equal to w6a16_plan_split.  No counterpart in the reference (its weights come only as
 * planes); for callers that pass packed weights.  Results depend on split_k: a packed call gives the planes' bits
 * only at the same split_k. */
int w6a16_plan_split_packed(int32_t B, int32_t M, int32_t N, int32_t K);

/* C = A @ dequant(W) on `stream` (hipStream_t).  Replaces `_impl` + `_w6a16` (int6_gemm.py:253-287, 156-215).
 * W6A16_FORMAT_PACKED with M > 256 runs the large-M kernel: A times the weight dequantised to A's type (s q rounded
 * once, the values w6a16_dequantize writes), fp32 accumulation, no workspace; split_k is not used there. */
int w6a16_matmul(const w6a16_args *args, void *stream);

/* w[b][k][n] = scale * q ([B][K][N], batch stride in elements) as bf16, fp16 or fp32 (W6A16_OUT_*):
 * the Python layer's path above M = 256, where a library GEMM on the dequantised weight is faster than the large-M
 * kernel (measured at K = 4096, N = 16384) except near M = 1024.  Replaces dequantize_int6
 * (int6_gemm.py:115-131) on the device.  N % 16 == 0; all pointers 16-byte aligned. */
int w6a16_dequantize(const uint8_t *lo, const uint8_t *hi, const uint16_t *scales, void *w, int32_t B, int32_t K,
                     int32_t N, int32_t group_k, int64_t lo_batch_stride, int64_t hi_batch_stride,
                     int64_t scales_batch_stride, int64_t w_batch_stride, int32_t out_dtype, void *stream);

/* The packed layout (no counterpart in the reference; a load-time re-layout of the same bits): per (batch, 128-column
 * strip, 64-row chunk) one contiguous 6144-byte block in MFMA operand order, and per (batch, strip, group) 128 fp16
 * scales.  Sizes for a (B, K, N) weight; columns are padded to whole strips. */
int w6a16_packed_size(int32_t B, int32_t K, int32_t N, int32_t group_k, size_t *weight_bytes, size_t *scale_bytes);

/* Re-lay out reference planes (as passed to w6a16_matmul in W6A16_FORMAT_PLANES) into the packed layout on `stream`.
 * Packed batches are contiguous: batch strides w6a16_packed_size(1, ...).  Used with W6A16_FORMAT_PACKED, a call
 * streams each wavefront's weight linearly and skips the LDS transposition the planes need. */
int w6a16_pack(const uint8_t *lo, const uint8_t *hi, const uint16_t *scales, int32_t B, int32_t K, int32_t N,
               int32_t group_k, int64_t lo_batch_stride, int64_t hi_batch_stride, int64_t scales_batch_stride,
               void *packed, uint16_t *packed_scales, void *stream);

/* w6a16_dequantize for the packed layout (batches contiguous, as w6a16_pack writes them). */
int w6a16_dequantize_packed(const void *packed, const uint16_t *packed_scales, void *w, int32_t B, int32_t K,
                            int32_t N, int32_t group_k, int64_t w_batch_stride, int32_t out_dtype, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RWKV_NEXT_AMD_W6A16_H */
