/*
 * wkv7.h -- C ABI of the MI355X (gfx950) WKV7 recurrence library, librwkv7_hip.so.
 *
 * Drop-in replacement for the WKV7 hot path of OpenMOSE/RWKV-Infer-Next.  In the reference every caller of the
 * recurrence -- the functional op, the varlen prefill call and the in-place rollback replay -- ends in one
 * launcher, `_launch(r, w, k, v, a, b, h0, ht, cu, nkeep, store_o, H, K)` (rwkv_next/kernels/wkv7.py:89-104),
 * which runs the Triton program `_wkv7_raw` (rwkv_next/kernels/wkv7.py:38-79).  `wkv7_run` below takes the same
 * arguments (plus the slot-pool, snapshot and workspace extensions) and is what a binding of that launcher
 * calls.
 *
 * Math (rwkv_next/kernels/wkv7.py:4-7), per (sequence, head), state S = K x V fp32 with V contiguous:
 *     S_t = diag(d_t) S_{t-1} + b_t (a_t^T S_{t-1}) + k_t v_t^T,   d_t = exp(-exp(w_t)),   o_t = S_t^T r_t
 * with the RAW w (the decay is computed in fp32 inside the kernels).  Head size K = V = 64.
 *
 * Plain C: no HIP, CUDA or torch types.  Pointers are device pointers; `stream` is a hipStream_t passed as
 * void*.  No function allocates device memory or synchronises the host, and every call is reentrant and can be
 * recorded into a hipGraph (scratch memory comes from the caller's workspace).  Global state: a per-device cache of
 * the compute-unit count.  (The allocation-free variant of wkv7_run, with its static device scratch array, is a
 * separate library: include/wkv7_noalloc.h.)
 */
#ifndef RWKV_NEXT_AMD_WKV7_H
#define RWKV_NEXT_AMD_WKV7_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WKV7_ABI_VERSION 2

/* Return codes.  Negative: argument validation failed before anything was launched.  Positive: the hipError_t
 * of a failed launch (the reference surfaces Triton/GPU errors as Python exceptions, engine.py:486-495). */
#define WKV7_OK 0
#define WKV7_ERR_NULL (-1)       /* a required pointer is NULL */
#define WKV7_ERR_SHAPE (-2)      /* head_size outside 1..256, H < 1, negative sizes, T too large */
#define WKV7_ERR_ALIGN (-3)      /* operand/state pointers not 16-byte aligned, or strides not multiples of 8 */
#define WKV7_ERR_WORKSPACE (-4)  /* workspace missing or smaller than wkv7_workspace_size() */
#define WKV7_ERR_ARG (-5)        /* inconsistent arguments (snapshots on the chunked path, bad algo, ...) */
#define WKV7_ERR_SCRATCH_LIMIT (-6) /* wkv7_run_noalloc (wkv7_noalloc.h): the call needs more than its scratch */

/* Bits of the optional device status word (wkv7_args.status).  The recurrence kernels never follow an index outside
 * its buffer: they go on as documented for each case below, so every kernel exits normally.  When status is set,
 * wkv7_run first launches one small check over the call's per-sequence indices (in stream order, before the
 * recurrence) that ORs the bits of every such case into the word; it never reads or clears it.  Calls with status ==
 * NULL launch nothing extra.  In the reference the same inputs raise from torch indexing
 * (rwkv_next/model.py:366-396: index_select / index_copy_ / pool views). */
#define WKV7_STATUS_H0_SLOT 1   /* an h0 index outside [0, h0_rows): that sequence started from a zero state */
#define WKV7_STATUS_HT_SLOT 2   /* an ht index outside [0, ht_rows): that final state was not stored */
#define WKV7_STATUS_SEQLENS 4   /* cu_seqlens entries not non-decreasing within [0, total_tokens], or a row longer
                                 * than the bound T > 0: extents clamped (such a row is cut to its first T tokens) */
#define WKV7_STATUS_NKEEP 8     /* a negative n_keep entry: treated as 0 */
#define WKV7_STATUS_DECAY 16    /* some w of a token that the chunked, segmented or chain kernels run (rows longer
                                 * than the token-serial threshold, within n_keep) exceeds WKV7_CHUNK_W_MAX: those
                                 * rows' results are not finite; run such calls with WKV7_ALGO_RECURRENT */
#define WKV7_STATUS_SLOT_CLASH 32  /* (calls of at most WKV7_STATUS_CLASH_MAX_SEQS sequences) two sequences store their
                                    * final states to the same ht slot, or, with h0 and ht one pool, a sequence stores
                                    * to a slot another sequence reads its initial state from: the result depends on
                                    * the order in which the kernels reach them */
#define WKV7_STATUS_CLASH_MAX_SEQS 1024
#define WKV7_STATUS_SEGMENT_WAIT 64  /* the segmented prefill kernel gave up a bounded wait (an internal hand-off did not
                                      * arrive): that row's results are wrong and the workspace's hand-off flags must
                                      * be zeroed again before the next call */

/* Largest raw w the chunked form handles.  It references each chunk's decay factors to the chunk midpoint, so factors
 * up to exp(32 exp(w)) must fit fp32: w <= 1.0 (32 e^1.0 = 87 < 88.7).  RWKV-7 produces w = -softplus(-x) - 0.5
 * <= -0.5 (rwkv_next/model.py:142-144).  The token-serial kernels take any w. */
#define WKV7_CHUNK_W_MAX 1.0f

/* Algorithm selection (wkv7_args.algo). */
#define WKV7_ALGO_AUTO 0       /* dense rows of at most rec_max_len tokens token-serial, longer ones on the segmented
                                * kernel (the chunked one for calls of fewer than 8 x CUs 32-token chunk-heads); a
                                * ragged call in one segmented dispatch, its short rows token-serial in the
                                * kernel's tail (beyond 4096 rows: token-serial + two-kernel chunked) */
#define WKV7_ALGO_RECURRENT 1  /* token-serial kernel for every row */
#define WKV7_ALGO_CHUNKED 2    /* chunked MFMA prefill for every row */
#define WKV7_ALGO_SEGMENTED 4  /* the segmented chunked kernel (32-token chunks, rows cut into segments, one
                                * dispatch; needs a workspace): every row, or with rec_max_len >= 0 the rows longer
                                * than it, the others token-serially in the same launch.  WKV7_ERR_SHAPE when
                                * a token stride exceeds 2^24 or the grid needs more flags than the flag region holds (AUTO
                                * then takes the chunked path) */
#define WKV7_ALGO_CHAIN 3      /* one dispatch: rows of at most rec_max_len tokens token-serial, longer rows chunked with
                                * each (row, head) chain walked by one workgroup (no workspace; num_seqs <= 512) */

/*
 * One call.  Operand element (token t, head h, channel i) is at ptr[t * in_tok_stride + h * 64 + i] (bf16 bit
 * patterns); the reference's layout (B, T, H*K) contiguous has in_tok_stride = H * 64 and token index
 * t = b * T + tau.
 */
typedef struct wkv7_args {
    /* operands, bf16: r, w (raw log-log decay), k, v, a, b -- rwkv_next/kernels/wkv7.py:39, 60-73 */
    const uint16_t *r, *w, *k, *v, *a, *b;  /* chunked / chain paths: w <= WKV7_CHUNK_W_MAX (see above) */
    int64_t in_tok_stride;        /* elements between consecutive tokens (multiple of 8) */
    uint16_t *o;                  /* output o, bf16, or NULL for STORE_O = False (wkv7.py:76-77, 93) */
    int64_t o_tok_stride;         /* elements between consecutive output tokens (multiple of 8) */

    /* states, fp32 [rows][H][64][64] -- h0 / ht of wkv7.py:62-64, 78-79 */
    const float *h0;              /* initial states, or NULL for zeros (HAS_H0 = False) */
    const int64_t *h0_idx;        /* NULL: sequence n reads h0 row n; else row h0_idx[n] (slot pool) */
    int64_t h0_rows;              /* rows addressable through h0 (slot indices outside [0, h0_rows) read zeros) */
    float *ht;                    /* final states, or NULL for final=False (STORE_HT, wkv7.py:78-79, 119) */
    const int64_t *ht_idx;        /* NULL: row n; else row ht_idx[n].  ht == h0 with equal indices = in place */
    int64_t ht_rows;              /* rows addressable through ht (indices outside are not written) */
    const uint8_t *fresh;         /* NULL, or per sequence: nonzero = start from zeros (model.py:382-383) */

    /* sequences -- wkv7.py:46-54 */
    const int32_t *cu_seqlens;    /* NULL: dense, sequence n = tokens [n*T, (n+1)*T); else [num_seqs + 1] */
    const int64_t *n_keep;        /* NULL, or per sequence: run only the first min(len, n_keep[n]) tokens */
    float *snapshots;             /* NULL, or [num_seqs][T][H][K][K]: state after each token t < len of each row
                                   * (the others untouched; ragged calls need T >= 1), recurrent kernel */

    void *workspace;              /* device scratch of the chunked paths (see wkv7_workspace_size), 256-byte aligned.
                                   * Its first WKV7_SEG_FLAG_BYTES hold the segmented kernel's hand-off flags: they
                                   * must be zero before the workspace's first call, and every call that completes
                                   * leaves them zero (WKV7_STATUS_SEGMENT_WAIT aside), so a workspace serves any
                                   * number of calls in stream order without clearing */
    size_t workspace_bytes;

    int32_t num_seqs;             /* N: B when dense, cu_seqlens entries - 1 when ragged */
    int32_t T;                    /* dense: tokens per sequence.  Ragged: an upper bound on any row's length
                                   * (0 = total_tokens; a longer row is cut to T tokens, see WKV7_STATUS_SEQLENS);
                                   * the snapshot time stride in both cases */
    int64_t total_tokens;         /* operand rows: N*T dense, the packed length when ragged */
    int32_t H;                    /* heads */
    int32_t head_size;            /* K == V: 64 (every RWKV-7 model) runs the kernels above; any other 1..256 (the
                                   * reference pads K to a power of two and masks, wkv7.py:55-59, 96) runs one
                                   * generic token-serial kernel on every row, no workspace, algo AUTO or RECURRENT
                                   * (others: WKV7_ERR_ARG); states and snapshots are then [..][K][K], operand rows
                                   * [token][H][K] (2-byte aligned; states 4-byte aligned) */
    int32_t algo;                 /* WKV7_ALGO_* */
    int32_t rec_max_len;          /* AUTO: rows of at most this many tokens run token-serial; -1 = default */
    int32_t *status;              /* NULL, or one device int32 that receives WKV7_STATUS_* bits (see above) */
} wkv7_args;

/* Bytes at the start of a workspace reserved for the segmented kernel's hand-off flags (zero between calls). */
#define WKV7_SEG_FLAG_BYTES (256u << 10)

/* Bytes of device workspace `wkv7_run` needs for these arguments (0 when only the token-serial kernel runs).
 * Depends only on host-side sizes and flags, never on device data.  No reference counterpart: the reference's
 * launcher allocates its outputs through the torch caching allocator (wkv7.py:93, 119, 135). */
int wkv7_workspace_size(const wkv7_args *args, size_t *bytes);

/* Run the recurrence for `args` on `stream` (a hipStream_t).  Replaces `_launch` + `_wkv7_raw`
 * (rwkv_next/kernels/wkv7.py:89-104, 38-79), i.e. the bodies of
 *   wkv7()          functional / varlen forward  (wkv7.py:126-138; torch op rwkv_next::wkv7_fwd, 113-123)
 *   wkv7_replay()   in-place rollback over the first n_keep[b] tokens (wkv7.py:141-147)
 * and the model's pool traffic around them (model.py:366-371 decode, 382-396 prefill gather/scatter,
 * 485 verify with final=False) when h0/ht address the slot pool through h0_idx/ht_idx.
 * Asynchronous; returns after launching. */
int wkv7_run(const wkv7_args *args, void *stream);

/*
 * Slot-pool maintenance on a pool of `layers` consecutive fp32 [rows][H][64][64] arrays (a model's per-layer state
 * pools, the reference's `wkv (L, S, Hl, 64, 64)`, rwkv_next/model.py:302).  Slot indices outside [0, rows) are
 * ignored.  Asynchronous on `stream`; no allocation, no memset, so they can be recorded into a hipGraph.
 */

/* pool[l][idx[i]] := 0 for every layer l and i < n.  Replaces the WKV part of `reset_slots`
 * (rwkv_next/model.py:310-311). */
int wkv7_pool_reset(float *pool, int32_t layers, int64_t rows, int32_t H, const int64_t *idx, int32_t n,
                    void *stream);

/* pool[l][dst[i]] := pool[l][src[i]] for every layer l and i < n, with gather-then-scatter semantics: every source
 * is read before any destination is written, so swaps and chains are exact.  dst entries must be distinct.
 * n <= 1024.  Replaces the WKV part of `move_slots` (rwkv_next/model.py:313-316). */
int wkv7_pool_move(float *pool, int32_t layers, int64_t rows, int32_t H, const int64_t *src, const int64_t *dst,
                   int32_t n, void *stream);

/* Rollback after a speculative verify that wrote per-token snapshots [num_seqs][T][H][64][64]:
 * pool[slots[b]] := snapshots[b][n_accepted[b] - 1] for n_accepted[b] in [1, T]; other rows keep the pool's state.
 * One layer.  Replaces the per-layer `wkv7_replay` pass of `rollback` (rwkv_next/model.py:498-508;
 * rwkv_next/kernels/wkv7.py:141-147) with a copy. */
int wkv7_snapshot_restore(float *pool, int64_t rows, int32_t H, const int64_t *slots, const float *snapshots,
                          int32_t T, const int64_t *n_accepted, int32_t num_seqs, void *stream);

/*
 * Time-mix work around the recurrence, fused (one pass each instead of the reference's chain of elementwise torch
 * ops).  All tensors bf16, rows of H*64 channels; head size 64, 1 <= H <= 65536.  Every pointer 16-byte aligned and
 * row strides multiples of 8 elements (WKV7_ERR_ALIGN otherwise).  fp32 arithmetic, one bf16 rounding per output.
 * Outputs must not overlap the inputs.
 */

/* Operand prologue, rwkv_next/model.py:142-152:
 *   w = -softplus(-(b_w + o_w)) - 0.5;  a = sigmoid(b_a + o_a);
 *   v' = v (v_first == NULL: first layer) or v + (v_first - v) * sigmoid(b_v + o_v);
 *   kk = L2-normalise(k * kk_mul) per head (eps 1e-12);  k' = k * (1 + (a - 1) * ka_mul);
 *   outputs w, k', v', a_out = -kk, b_out = kk * a  -- with r, the six WKV operands. */
typedef struct wkv7_prologue_args {
    const uint16_t *k, *v;                   /* projections [tokens][in_stride] */
    const uint16_t *o_v, *o_w, *o_a;         /* LoRA outputs o[0], o[1], o[2] (model.py:135-140), same layout */
    const uint16_t *v_first;                 /* the first layer's v, or NULL on the first layer */
    const uint16_t *b_w, *b_a, *b_v, *kk_mul, *ka_mul;  /* per-channel parameters [H*64] (b_v unused if no v_first) */
    uint16_t *w_out, *k_out, *v_out, *a_out, *b_out;    /* [tokens][out_stride] */
    int64_t tokens, in_stride, out_stride;  /* strides in elements, >= H*64 */
    int32_t H, head_size;
} wkv7_prologue_args;

/* Epilogue up to the output projection, rwkv_next/model.py:156-158:
 *   out = (group_norm(y; one group per head, lnx_w, lnx_b, eps) + sum_c(r * k' * r_k) * v') * g */
typedef struct wkv7_epilogue_args {
    const uint16_t *y, *r, *k, *v, *g;       /* recurrence output, r, k', v', gate [tokens][in_stride] */
    const uint16_t *lnx_w, *lnx_b;           /* group-norm affine [H*64] */
    const uint16_t *r_k;                     /* bonus weights [H][64] */
    uint16_t *out;                           /* [tokens][out_stride] */
    int64_t tokens, in_stride, out_stride;
    float eps;                               /* the model's 1e-5 * head_size_divisor^2 (model.py:266) */
    int32_t H, head_size;
} wkv7_epilogue_args;

int wkv7_timemix_prologue(const wkv7_prologue_args *args, void *stream);
int wkv7_timemix_epilogue(const wkv7_epilogue_args *args, void *stream);

/* Static description of a return code. */
const char *wkv7_strerror(int code);

/* WKV7_ABI_VERSION of the loaded library. */
int wkv7_abi_version(void);

/* sizeof(wkv7_args) as compiled into the library, so a binding can check its struct layout. */
size_t wkv7_args_size(void);

/* Byte offsets of the fields of wkv7_args in declaration order, written to offsets[0 .. min(n, count) - 1]; returns
 * the number of fields (count).  Lets a binding check every field's position, not only the total size. */
int wkv7_args_layout(size_t *offsets, int n);

#ifdef __cplusplus
}
#endif

#endif /* RWKV_NEXT_AMD_WKV7_H */
