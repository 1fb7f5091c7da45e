// wkv7_capi.hip -- the extern "C" entry points of include/wkv7.h: argument validation, the host-side choice
// between the token-serial and the chunked kernels, and the launches.
//
// Everything here is decided from host-known sizes and flags (never from device data), so a call can be
// recorded into a hipGraph and replayed with new device-side lengths, slots or n_keep values.
#include <stddef.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>

#include "wkv7.h"
#include "wkv7_launch.h"

namespace wkv7 {

int device_cu_count() {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cache[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) return 256;
    cache[dev].store(v, std::memory_order_relaxed);
    return v;
}

}  // namespace wkv7

namespace {

using wkv7::Params;

// AUTO threshold: rows of at most this many tokens run the token-serial kernel.  Below it one wavefront walking
// the tokens beats the chunked paths' fixed cost (a chunk transition built on MFMA per row).
constexpr int kDefaultRecMaxLen = 32;
// AUTO on dense rows: the segmented kernel from this many 32-token chunk-heads per CU up (measured crossover near 8)
constexpr int kSegMinChunkHeadsPerCu = 8;

struct Plan {
    bool run_generic = false;  // head size other than 64
    bool run_recurrent = false;
    bool run_chunked = false;
    bool run_chain = false;
    bool run_seg = false;
    bool seg_short = false;  // the segmented launch also runs the short rows (no token-serial launch)
    int rec_len_rec = -1;    // Params.rec_max_len of the token-serial launch (-1: all rows)
    int rec_len_chunk = -1;  // Params.rec_max_len of the chunked launch (-1: all rows)
    wkv7::ChunkWorkspace ws{};
    wkv7::SegWorkspace sws{};
};

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Head sizes other than 64: the generic token-serial kernel, with scalar accesses (2-byte operands, 4-byte states).
int validate_generic(const wkv7_args* a) {
    if (a->algo != WKV7_ALGO_AUTO && a->algo != WKV7_ALGO_RECURRENT) return WKV7_ERR_ARG;  // K = 64 forms only
    if ((int64_t)a->num_seqs * a->H > ((int64_t)1 << 31)) return WKV7_ERR_SHAPE;
    if (!a->cu_seqlens && (int64_t)a->num_seqs * a->T > a->total_tokens) return WKV7_ERR_SHAPE;
    if (a->T > (1 << 30) || a->total_tokens > ((int64_t)1 << 40)) return WKV7_ERR_SHAPE;
    const int64_t K = a->head_size;
    if (a->num_seqs > 0 && a->total_tokens > 0) {
        const uint16_t* ops[6] = {a->r, a->w, a->k, a->v, a->a, a->b};
        for (const uint16_t* p : ops) {
            if (!p) return WKV7_ERR_NULL;
            if (!aligned(p, 2)) return WKV7_ERR_ALIGN;
        }
        if (a->in_tok_stride < a->H * K) return WKV7_ERR_ALIGN;
        if (a->o && (!aligned(a->o, 2) || a->o_tok_stride < a->H * K)) return WKV7_ERR_ALIGN;
    }
    // grid: one wavefront per (sequence, head, 16 state columns), four per workgroup
    if (((int64_t)a->num_seqs * a->H * ((K + 15) / 16) + 3) / 4 > 0x7FFFFFFF) return WKV7_ERR_SHAPE;
    if ((a->h0 && !aligned(a->h0, 4)) || (a->ht && !aligned(a->ht, 4))) return WKV7_ERR_ALIGN;
    if (a->h0_idx && !a->h0) return WKV7_ERR_ARG;
    if (a->ht_idx && !a->ht) return WKV7_ERR_ARG;
    if ((a->h0 && a->h0_rows < 0) || (a->ht && a->ht_rows < 0)) return WKV7_ERR_SHAPE;
    if (a->rec_max_len < -1) return WKV7_ERR_ARG;
    if (a->snapshots) {
        if (!aligned(a->snapshots, 4)) return WKV7_ERR_ALIGN;
        if (a->T < 1) return WKV7_ERR_ARG;
    }
    return WKV7_OK;
}

int validate(const wkv7_args* a) {
    if (a->head_size < 1 || a->head_size > wkv7::kGenericMaxK) return WKV7_ERR_SHAPE;
    if (a->H < 1 || a->num_seqs < 0 || a->T < 0 || a->total_tokens < 0) return WKV7_ERR_SHAPE;
    if (a->algo < WKV7_ALGO_AUTO || a->algo > WKV7_ALGO_SEGMENTED) return WKV7_ERR_ARG;
    if (a->head_size != wkv7::HS) return validate_generic(a);
    if (a->algo == WKV7_ALGO_SEGMENTED && a->snapshots) return WKV7_ERR_ARG;
    if (a->algo == WKV7_ALGO_SEGMENTED && (a->cu_seqlens || a->n_keep) && a->num_seqs > wkv7::kSegMaxRows)
        return WKV7_ERR_ARG;
    if (a->algo == WKV7_ALGO_CHAIN && (a->num_seqs > wkv7::kChainMaxSeqs || a->snapshots)) return WKV7_ERR_ARG;
    if (a->rec_max_len < -1) return WKV7_ERR_ARG;
    if ((int64_t)a->num_seqs * a->H > ((int64_t)1 << 31)) return WKV7_ERR_SHAPE;
    if (!a->cu_seqlens && (int64_t)a->num_seqs * a->T > a->total_tokens) return WKV7_ERR_SHAPE;
    if (a->T > (1 << 30) || a->total_tokens > ((int64_t)1 << 40)) return WKV7_ERR_SHAPE;
    const bool has_tokens = a->num_seqs > 0 && a->total_tokens > 0;
    if (has_tokens) {
        const uint16_t* ops[6] = {a->r, a->w, a->k, a->v, a->a, a->b};
        for (const uint16_t* p : ops) {
            if (!p) return WKV7_ERR_NULL;
            if (!aligned(p, 16)) return WKV7_ERR_ALIGN;
        }
        if (a->in_tok_stride < (int64_t)a->H * wkv7::HS || a->in_tok_stride % 8) return WKV7_ERR_ALIGN;
        if (a->o) {
            if (!aligned(a->o, 16)) return WKV7_ERR_ALIGN;
            if (a->o_tok_stride < (int64_t)a->H * wkv7::HS || a->o_tok_stride % 8) return WKV7_ERR_ALIGN;
        }
    }
    if (a->h0 && !aligned(a->h0, 16)) return WKV7_ERR_ALIGN;
    if (a->ht && !aligned(a->ht, 16)) return WKV7_ERR_ALIGN;
    if (a->h0_idx && !a->h0) return WKV7_ERR_ARG;
    if (a->ht_idx && !a->ht) return WKV7_ERR_ARG;
    if ((a->h0 && a->h0_rows < 0) || (a->ht && a->ht_rows < 0)) return WKV7_ERR_SHAPE;
    if (a->snapshots) {
        if (!aligned(a->snapshots, 16)) return WKV7_ERR_ALIGN;
        if (a->T < 1) return WKV7_ERR_ARG;
        if (a->algo == WKV7_ALGO_CHUNKED) return WKV7_ERR_ARG;
    }
    return WKV7_OK;
}

// The segmented launch holds one hand-off flag per unit in the workspace's flag region and addresses a chunk's operand
// and output rows with 32-bit offsets.
bool seg_fits(const Plan& pl, const wkv7_args* a) {
    return pl.sws.units <= (int64_t)(wkv7::kSegFlagRegion / sizeof(int32_t)) &&
           a->in_tok_stride <= wkv7::kSegMaxTokStride && a->o_tok_stride <= wkv7::kSegMaxTokStride;
}

Plan make_plan(const wkv7_args* a) {
    Plan pl;
    if (a->head_size != wkv7::HS) {
        pl.run_generic = true;
        return pl;
    }
    const bool varlen = a->cu_seqlens != nullptr;
    const int64_t bound = varlen ? (a->T > 0 ? a->T : a->total_tokens) : a->T;
    const int thr = a->rec_max_len >= 0 ? a->rec_max_len : kDefaultRecMaxLen;
    if (a->snapshots || a->algo == WKV7_ALGO_RECURRENT) {
        pl.run_recurrent = true;
    } else if (a->algo == WKV7_ALGO_SEGMENTED) {
        pl.run_seg = true;
        if (a->rec_max_len >= 0) {  // rows of at most rec_max_len tokens run token-serial in the same launch
            pl.seg_short = true;
            pl.rec_len_chunk = a->rec_max_len;
        }
    } else if (a->algo == WKV7_ALGO_CHAIN) {
        pl.run_chain = true;
        pl.rec_len_rec = thr;
    } else if (a->algo == WKV7_ALGO_CHUNKED) {
        pl.run_chunked = true;
    } else if (bound <= thr) {
        pl.run_recurrent = true;
    } else if (!varlen && !a->n_keep) {
        // every row has exactly T > thr tokens: one segmented dispatch, unless the call is too small to fill the
        // GPU with segments (then the chunked path's wider per-chunk parallelism wins: B = 1, T = 512 is 41 against
        // 51 us at H = 64, T = 1024 about even)
        const int64_t chunk_heads = (int64_t)a->num_seqs * ((bound + wkv7::kSegChunk - 1) / wkv7::kSegChunk) * a->H;
        if (chunk_heads >= (int64_t)kSegMinChunkHeadsPerCu * wkv7::device_cu_count()) pl.run_seg = true;
        else pl.run_chunked = true;
    } else {
        // row lengths are only known on the device: rows of at most thr tokens token-serial, the others segmented,
        // both in the segmented launch (chunked beside a token-serial launch when the segmented kernel's LDS row
        // table cannot hold the call)
        pl.rec_len_rec = pl.rec_len_chunk = thr;
        if (a->num_seqs <= wkv7::kSegMaxRows) {
            pl.run_seg = pl.seg_short = true;
        } else {
            pl.run_recurrent = pl.run_chunked = true;
        }
    }
    if (pl.run_seg) {
        pl.sws = wkv7::seg_workspace(a->num_seqs, a->H, a->total_tokens, bound, varlen || a->n_keep != nullptr,
                                     pl.rec_len_chunk, wkv7::device_cu_count());
        // AUTO falls back to the chunked path when the segmented launch cannot take the call
        if (a->algo == WKV7_ALGO_AUTO && !seg_fits(pl, a)) {
            pl.run_seg = false;
            pl.run_chunked = true;
            if (pl.seg_short) pl.run_recurrent = true;
            pl.seg_short = false;
        }
    }
    if (pl.run_chunked)
        pl.ws = wkv7::chunk_workspace(a->num_seqs, a->H, a->total_tokens, bound, varlen, pl.rec_len_chunk);
    return pl;
}

// Every path that uses a workspace leaves its first kSegFlagRegion bytes to the segmented kernel's hand-off flags, so
// one workspace can serve calls of any path in stream order.
size_t workspace_bytes(const Plan& pl) {
    if (pl.run_seg) return pl.sws.total_bytes;
    if (pl.run_chunked && pl.ws.total_bytes > 0) return wkv7::kSegFlagRegion + pl.ws.total_bytes;
    return 0;
}

Params to_params(const wkv7_args* a) {
    Params p{};
    p.r = a->r; p.w = a->w; p.k = a->k; p.v = a->v; p.a = a->a; p.b = a->b;
    p.in_tok_stride = a->in_tok_stride;
    p.o = a->o;
    p.o_tok_stride = a->o_tok_stride;
    p.h0 = a->h0;
    p.h0_idx = a->h0_idx;
    p.ht = a->ht;
    p.ht_idx = a->ht_idx;
    p.h0_rows = a->h0 ? (a->h0_idx ? a->h0_rows : (a->h0_rows > 0 ? a->h0_rows : a->num_seqs)) : 0;
    p.ht_rows = a->ht ? (a->ht_idx ? a->ht_rows : (a->ht_rows > 0 ? a->ht_rows : a->num_seqs)) : 0;
    p.fresh = a->fresh;
    p.cu = a->cu_seqlens;
    p.n_keep = a->n_keep;
    p.snap = a->snapshots;
    p.total_tokens = a->total_tokens;
    p.num_seqs = a->num_seqs;
    p.T = a->T;
    p.H = a->H;
    p.rec_max_len = -1;
    p.status = a->status;
    p.K = a->head_size;
    return p;
}

// The optional status word: one pass over the call's sequences, launched before the recurrence only when the
// caller passes a status pointer (so calls without one keep their single dispatch and pay nothing).  It checks
// exactly what the kernels skip: an h0 slot outside [0, h0_rows) on a row that reads it (not fresh), an ht slot
// outside [0, ht_rows), cu_seqlens entries that are not non-decreasing within [0, total_tokens] or span more than
// the length bound T, a negative n_keep;
// and, when the call runs the chunked, segmented or chain kernels, w against WKV7_CHUNK_W_MAX (16 bytes per thread)
// on the tokens those kernels run: rows longer than chunk_thr (every row when chunk_thr < 0), within n_keep.
__device__ __forceinline__ int row_of_token(const wkv7::Params& p, int64_t t) {
    if (!p.cu) return (int)(t / (p.T > 0 ? p.T : 1));
    int lo = 0, hi = p.num_seqs - 1;  // the last row n with cu[n] <= t
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (p.cu[mid] <= t) lo = mid; else hi = mid - 1;
    }
    return lo;
}

__global__ __launch_bounds__(256) void wkv7_status_kernel(const wkv7::Params p, int32_t* __restrict__ status,
                                                          bool check_w, int chunk_thr) {
    int bits = 0;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x, nthr = (int64_t)gridDim.x * blockDim.x;
    for (int64_t n = tid; n < p.num_seqs; n += nthr) {
        if (p.h0 && !(p.fresh && p.fresh[n])) {
            const int64_t s = p.h0_idx ? p.h0_idx[n] : n;
            if (s < 0 || s >= p.h0_rows) bits |= WKV7_STATUS_H0_SLOT;
        }
        if (p.ht) {
            const int64_t s = p.ht_idx ? p.ht_idx[n] : n;
            if (s < 0 || s >= p.ht_rows) bits |= WKV7_STATUS_HT_SLOT;
        }
        if (p.cu) {
            const int64_t b = p.cu[n], e = p.cu[n + 1];
            if (b < 0 || e < b || e > p.total_tokens || (p.T > 0 && e - b > p.T)) bits |= WKV7_STATUS_SEQLENS;
        }
        if (p.n_keep && p.n_keep[n] < 0) bits |= WKV7_STATUS_NKEEP;
    }
    if (check_w) {
        const int64_t per_tok = (int64_t)p.H * (wkv7::HS / 8);  // 16-byte pieces of one token's w
        const bool all_rows = chunk_thr < 0 && !p.n_keep;
        for (int64_t i = tid; i < p.total_tokens * per_tok; i += nthr) {
            const int64_t t = i / per_tok, j = (i - t * per_tok) * 8;
            if (!all_rows) {  // only tokens a chunked kernel runs
                const int n = row_of_token(p, t);
                int64_t bos;
                int L;
                wkv7::seq_extent(p, n, bos, L);
                if (L <= chunk_thr || t - bos >= L) continue;
            }
            const uint4 x = *reinterpret_cast<const uint4*>(p.w + t * p.in_tok_stride + j);
            const uint32_t wd[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float lo, hi;
                wkv7::bf16x2_to_f32(wd[e], lo, hi);
                if (!(lo <= WKV7_CHUNK_W_MAX) || !(hi <= WKV7_CHUNK_W_MAX)) bits |= WKV7_STATUS_DECAY;  // NaN too
            }
        }
    }
    // Slot clashes (uniform over the grid): every workgroup stages the call's in-range final-state slots and, for an
    // in-place pool, initial-state slots in LDS; workgroup b then compares each final-state slot j = b, b + G, ..
    // with every other sequence's slots, each thread holding the entries n = threadIdx.x + 256 k in registers.
    constexpr int kMax = WKV7_STATUS_CLASH_MAX_SEQS, kPer = kMax / 256;
    const int N = p.num_seqs;
    if (p.ht && N >= 2 && N <= kMax) {
        __shared__ int64_t dst[kMax], src[kMax];
        const bool same_pool = static_cast<const void*>(p.h0) == static_cast<const void*>(p.ht);
        for (int n = threadIdx.x; n < N; n += blockDim.x) {
            const int64_t d = p.ht_idx ? p.ht_idx[n] : n;
            dst[n] = (d >= 0 && d < p.ht_rows) ? d : -1;
            int64_t s = -1;
            if (same_pool && !(p.fresh && p.fresh[n])) {
                const int64_t x = p.h0_idx ? p.h0_idx[n] : n;
                if (x >= 0 && x < p.h0_rows) s = x;
            }
            src[n] = s;
        }
        __syncthreads();
        int64_t md[kPer], ms[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int n = threadIdx.x + 256 * k;
            md[k] = n < N ? dst[n] : -1;
            ms[k] = n < N ? src[n] : -1;
        }
        for (int j = blockIdx.x; j < N; j += gridDim.x) {
            const int64_t dj = dst[j];
            if (dj < 0) continue;
#pragma unroll
            for (int k = 0; k < kPer; ++k)
                if (threadIdx.x + 256 * k != j && (md[k] == dj || ms[k] == dj)) bits |= WKV7_STATUS_SLOT_CLASH;
        }
    }
    if (bits) __hip_atomic_fetch_or(status, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

extern "C" {

int wkv7_abi_version(void) { return WKV7_ABI_VERSION; }

size_t wkv7_args_size(void) { return sizeof(wkv7_args); }

int wkv7_args_layout(size_t* offsets, int n) {
    const size_t off[] = {
        offsetof(wkv7_args, r), offsetof(wkv7_args, w), offsetof(wkv7_args, k), offsetof(wkv7_args, v),
        offsetof(wkv7_args, a), offsetof(wkv7_args, b), offsetof(wkv7_args, in_tok_stride), offsetof(wkv7_args, o),
        offsetof(wkv7_args, o_tok_stride), offsetof(wkv7_args, h0), offsetof(wkv7_args, h0_idx),
        offsetof(wkv7_args, h0_rows), offsetof(wkv7_args, ht), offsetof(wkv7_args, ht_idx),
        offsetof(wkv7_args, ht_rows), offsetof(wkv7_args, fresh), offsetof(wkv7_args, cu_seqlens),
        offsetof(wkv7_args, n_keep), offsetof(wkv7_args, snapshots), offsetof(wkv7_args, workspace),
        offsetof(wkv7_args, workspace_bytes), offsetof(wkv7_args, num_seqs), offsetof(wkv7_args, T),
        offsetof(wkv7_args, total_tokens), offsetof(wkv7_args, H), offsetof(wkv7_args, head_size),
        offsetof(wkv7_args, algo), offsetof(wkv7_args, rec_max_len), offsetof(wkv7_args, status)};
    const int count = (int)(sizeof(off) / sizeof(off[0]));
    for (int i = 0; i < n && i < count && offsets; ++i) offsets[i] = off[i];
    return count;
}

const char* wkv7_strerror(int code) {
    switch (code) {
        case WKV7_OK: return "ok";
        case WKV7_ERR_NULL: return "a required pointer is NULL";
        case WKV7_ERR_SHAPE: return "invalid sizes (1 <= head_size <= 256, H >= 1, counts non-negative)";
        case WKV7_ERR_ALIGN: return "pointers must be 16-byte aligned and token strides multiples of 8 elements";
        case WKV7_ERR_WORKSPACE: return "workspace missing or smaller than wkv7_workspace_size()";
        case WKV7_ERR_ARG: return "inconsistent arguments";
        case WKV7_ERR_SCRATCH_LIMIT: return "the call needs more scratch than wkv7_run_noalloc holds";
        default: return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "unknown error";
    }
}

int wkv7_workspace_size(const wkv7_args* args, size_t* bytes) {
    if (!args || !bytes) return WKV7_ERR_NULL;
    const int rc = validate(args);
    if (rc != WKV7_OK) return rc;
    const Plan pl = make_plan(args);
    if (pl.run_seg && !seg_fits(pl, args)) return WKV7_ERR_SHAPE;
    *bytes = workspace_bytes(pl);
    return WKV7_OK;
}

int wkv7_run(const wkv7_args* args, void* stream) {
    if (!args) return WKV7_ERR_NULL;
    const int rc = validate(args);
    if (rc != WKV7_OK) return rc;
    const Plan pl = make_plan(args);
    if (pl.run_seg && !seg_fits(pl, args)) return WKV7_ERR_SHAPE;
    const size_t need = workspace_bytes(pl);
    if (need > 0) {
        if (!args->workspace || args->workspace_bytes < need) return WKV7_ERR_WORKSPACE;
        if (!aligned(args->workspace, 256)) return WKV7_ERR_ALIGN;
    }
    if (args->num_seqs == 0) return WKV7_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    Params p = to_params(args);
    if (args->status) {
        const bool check_w = pl.run_chunked || pl.run_chain || pl.run_seg;
        // the rows the chunked kernels run: those longer than the token-serial threshold of a split plan
        const int chunk_thr = pl.run_chain ? pl.rec_len_rec : pl.rec_len_chunk;
        const int64_t work = std::max<int64_t>(args->num_seqs, check_w ? args->total_tokens * args->H * 8 : 0);
        int blocks = (int)std::min<int64_t>((work + 255) / 256, 1024);
        // the slot-clash comparison (up to 1024 x 1024 slot pairs) is spread over at least 16 workgroups
        if (args->ht && args->num_seqs >= 2 && args->num_seqs <= WKV7_STATUS_CLASH_MAX_SEQS) blocks = std::max(blocks, 16);
        hipLaunchKernelGGL(wkv7_status_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p, args->status, check_w,
                           chunk_thr);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return static_cast<int>(e);
    }
    if (pl.run_generic) {
        const hipError_t e = wkv7::launch_generic(p, s);
        return e == hipSuccess ? WKV7_OK : static_cast<int>(e);
    }
    if (pl.run_chain) {
        p.rec_max_len = pl.rec_len_rec;
        const hipError_t e = wkv7::launch_chain(p, s);
        return e == hipSuccess ? WKV7_OK : static_cast<int>(e);
    }
    if (pl.run_recurrent) {
        p.rec_max_len = pl.rec_len_rec;
        const hipError_t e = wkv7::launch_recurrent(p, s);
        if (e != hipSuccess) return static_cast<int>(e);
    }
    if (pl.run_chunked) {
        p.rec_max_len = pl.rec_len_chunk;
        const hipError_t e = wkv7::launch_chunked(p, pl.ws, static_cast<char*>(args->workspace) + wkv7::kSegFlagRegion, s);
        if (e != hipSuccess) return static_cast<int>(e);
    }
    if (pl.run_seg) {
        p.rec_max_len = pl.rec_len_chunk;
        const hipError_t e = wkv7::launch_seg(p, pl.sws, args->workspace, pl.seg_short, s);
        if (e != hipSuccess) return static_cast<int>(e);
    }
    return WKV7_OK;
}

}  // extern "C"
