// wkv7_launch.h -- host-side launchers of the WKV7 kernels (internal to the library; the public interface is
// include/wkv7.h).  All launchers are asynchronous on `stream`, allocate nothing and never synchronise, so
// every call can be recorded into a hipGraph.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "wkv7.h"
#include "wkv7_device.h"

namespace wkv7 {

constexpr int kChunk = 64;                 // chunk length of the chunked prefill

// Compute units of the current device.  Queried once per device and cached (the attribute query is a driver call
// that costs microseconds; launchers run on every call).
int device_cu_count();
// Workspace record per (chunk, head): A hi/lo (bf16), H^T (fp32), Q (bf16), O_intra^T (bf16), 64 x 64 each.
constexpr int kChunkBytes = 2 * 2 * HS2 + 4 * HS2 + 2 * HS2 + 2 * HS2;

// Token-serial kernel: every row, or only rows with len <= p.rec_max_len when p.rec_max_len >= 0.
hipError_t launch_recurrent(const Params& p, hipStream_t stream);

// Workspace of the chunked path for one call.  Layout (byte offsets, each 256-aligned):
//   [plan]   int32 chunk_seq[max_chunks], chunk_idx[max_chunks], seq_off[num_seqs + 1], total   (varlen only)
//   [chunks] [max_chunks][H] records of kChunkBytes, then one trash record (stores that must not land)
struct ChunkWorkspace {
    int64_t max_chunks;
    size_t plan_bytes;
    size_t chunk_bytes;
    size_t total_bytes;
};

// max_len_bound: an upper bound on any row's length (dense: T).
ChunkWorkspace chunk_workspace(int num_seqs, int H, int64_t total_tokens, int64_t max_len_bound, bool varlen,
                               int rec_max_len);

// Rows a chain launch accepts (its row table has one entry per thread of a 512-thread workgroup).
constexpr int kChainMaxSeqs = 512;

// Single-dispatch chain kernel: rows of at most p.rec_max_len tokens token-serially, longer rows as (row, head) chains
// whose chunk records stay in LDS.  No workspace.  p.num_seqs <= kChainMaxSeqs.
hipError_t launch_chain(const Params& p, hipStream_t stream);

// Chunked path over rows with len > p.rec_max_len (all rows when p.rec_max_len < 0): plan (varlen only), prep
// (parallel over chunks), scan (sequential over chunks per (row, head, 16-column block)).
hipError_t launch_chunked(const Params& p, const ChunkWorkspace& ws, void* workspace, hipStream_t stream);

// Segmented single-dispatch chunked prefill (wkv7_seg.hip).  Chunks of kSegChunk tokens; a row of nch chunks is cut
// into nseg = ceil(nch / seg) segments, one workgroup per (row, head, segment) unit.  Ragged or n_keep calls build a
// row table in LDS and take at most kSegMaxRows rows.
constexpr int kSegChunk = 32;
constexpr int kSegMaxRows = 4096;
constexpr int kSegMinChunks = 8;
// The kernel addresses a chunk's operand and output rows with 32-bit byte offsets: in_tok_stride and o_tok_stride at
// most this many elements.
constexpr int64_t kSegMaxTokStride = int64_t(1) << 24;
// First chunk of segment s.  Segments after the first also carry the map from the row's initial state and finish
// with a correction pass, so the first segment takes a longer share, round(7 nch / (6 nseg + 1)) chunks (the measured
// per-chunk cost ratio of the two kinds is about 1.2); the later ones split the rest evenly, the last ones (with the
// longest hand-off chains) taking the shorter shares.
__host__ __device__ inline int seg_start(int nch, int nseg, int s) {
    if (s <= 0) return 0;
    const int64_t den = 6 * (int64_t)nseg + 1;
    const int first = (int)((7 * (int64_t)nch + den / 2) / den);
    if (nseg <= 1) return nch;
    return first + (int)(((int64_t)(s - 1) * (nch - first) + nseg - 2) / (nseg - 1));  // later ones no longer
}
// The workspace starts with one int32 hand-off flag per unit (at most kSegFlagRegion / 4 units).  The region must be
// zero before a workspace's first call; every call that completes leaves it zero.  No other path writes it.
constexpr size_t kSegFlagRegion = WKV7_SEG_FLAG_BYTES;
struct SegWorkspace {
    int seg;             // chunks per segment
    int64_t units;       // grid (an upper bound on the call's units)
    size_t flag_bytes, x_bytes, qp_bytes, total_bytes;
};
SegWorkspace seg_workspace(int num_seqs, int H, int64_t total_tokens, int64_t max_len_bound, bool varlen,
                           int rec_max_len, int cus);
// short_rows: the launch also runs the rows of at most p.rec_max_len tokens (token-serial, after each workgroup's
// own chunks), so a ragged call needs no second dispatch.
hipError_t launch_seg(const Params& p, const SegWorkspace& ws, void* workspace, bool short_rows, hipStream_t stream);

// Head sizes other than 64 (1 <= p.K <= kGenericMaxK): the token-serial recurrence on every row, no workspace.
constexpr int kGenericMaxK = 256;
int64_t generic_grid(const Params& p);  // workgroups of the launch
hipError_t launch_generic(const Params& p, hipStream_t stream);

}  // namespace wkv7
