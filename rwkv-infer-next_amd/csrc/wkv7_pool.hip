// wkv7_pool.hip -- slot-pool maintenance of the fp32 WKV state pool [layers][rows][H][64][64]: zeroing slots, moving
// slots (gather-then-scatter), and restoring per-token snapshots after a speculative verify.
//
// Replaces the WKV part of the reference's pool ops, which are torch indexing on (L, S, Hl, 64, 64):
//   reset_slots  self.wkv[:, idx] = 0                       (rwkv_next/model.py:310-311)
//   move_slots   self.wkv[:, d] = self.wkv[:, s]            (rwkv_next/model.py:313-316)
//   rollback     per layer, wkv7_replay over the first n[b] verify tokens (rwkv_next/model.py:498-508), here a
//                copy of the snapshot the verify already wrote
// All three are HBM-bound byte copies (16 KB per (slot, head) written; moves and restores also read 16 KB).  No
// hipMemset is used, so the calls can be recorded into a HIP graph.
#include <stdint.h>

#include "wkv7.h"
#include "wkv7_device.h"
#include "wkv7_launch.h"

namespace wkv7 {
namespace {

constexpr int kThreads = 256;
constexpr int kMoveLdsBytes = 64 * 1024;  // staging per workgroup for moves
constexpr int kMaxMoves = kMoveLdsBytes / 64;  // at least 16 floats (64 B) per move and position range

__device__ __forceinline__ f4 ldg4(const float* p) { return __builtin_nontemporal_load(reinterpret_cast<const f4*>(p)); }
__device__ __forceinline__ void stg4(float* p, f4 x) { __builtin_nontemporal_store(x, reinterpret_cast<f4*>(p)); }

// One workgroup zeroes one (layer, listed slot, head) state: 4096 floats, 4 f4 per thread.
__global__ __launch_bounds__(kThreads) void pool_reset_kernel(float* __restrict__ pool, int64_t rows, int H,
                                                              const int64_t* __restrict__ idx, int n) {
    const int64_t b = blockIdx.x;
    const int h = (int)(b % H);
    const int64_t i = (b / H) % n;
    const int64_t l = b / ((int64_t)H * n);
    const int64_t s = idx[i];
    if (s < 0 || s >= rows) return;  // indices outside the pool are ignored
    float* base = pool + ((l * rows + s) * H + h) * (int64_t)HS2;
    const f4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4; ++u) stg4(base + (u * kThreads + threadIdx.x) * 4, z);
}

// One workgroup owns positions [p0, p0 + P) of one layer's slot rows (a row is H * 4096 floats) for ALL moves: it
// stages every source range in LDS, then writes every destination range.  Other workgroups own other positions,
// so sources that are also destinations (swaps, chains) read their old values, as a gather-then-scatter does.
__global__ __launch_bounds__(kThreads) void pool_move_kernel(float* __restrict__ pool, int64_t rows, int64_t row_len,
                                                             const int64_t* __restrict__ src,
                                                             const int64_t* __restrict__ dst, int n, int P) {
    extern __shared__ __attribute__((aligned(16))) float stage[];  // [n][P]
    const int64_t ranges = row_len / P;
    const int64_t l = blockIdx.x / ranges;
    const int64_t p0 = (blockIdx.x % ranges) * P;
    float* const layer = pool + l * rows * row_len;
    const int per_move = P / 4;  // f4 per move
    const int total = n * per_move;
    for (int e = threadIdx.x; e < total; e += kThreads) {
        const int i = e / per_move, q = e % per_move;
        const int64_t s = src[i];
        const f4 x = (s >= 0 && s < rows) ? ldg4(layer + s * row_len + p0 + 4 * q) : f4{0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<f4*>(stage + i * P + 4 * q) = x;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < total; e += kThreads) {
        const int i = e / per_move, q = e % per_move;
        const int64_t d = dst[i], s = src[i];
        if (d < 0 || d >= rows || s < 0 || s >= rows) continue;
        stg4(layer + d * row_len + p0 + 4 * q, *reinterpret_cast<const f4*>(stage + i * P + 4 * q));
    }
}

// pool[slots[b]] := snaps[b][n[b] - 1] for n[b] in [1, T]; other rows keep the pool's state.  One workgroup per UPW
// consecutive (b, head) units: all their index loads, then all their states' loads, then the stores, so a workgroup
// of two units waits for one index round trip where two workgroups of one would each wait for theirs (measured at
// B = 64, H = 64, 4096 units: 24.9 us with one unit per workgroup, 24.2 with two; at H = 8, 512 units, two per
// workgroup halve an already small grid: 5.0 against 5.2 us).
template <int UPW>
__global__ __launch_bounds__(kThreads) void snapshot_restore_kernel(float* __restrict__ pool, int64_t rows, int H,
                                                                    const int64_t* __restrict__ slots,
                                                                    const float* __restrict__ snaps, int T,
                                                                    const int64_t* __restrict__ nacc, int64_t units) {
    const float* from[UPW];
    float* to[UPW];
    bool ok[UPW];
#pragma unroll
    for (int k = 0; k < UPW; ++k) {
        const uint32_t u = UPW * blockIdx.x + k;  // < 2^32: at most 2^31 - 1 workgroups
        const int64_t b = u / (uint32_t)H;
        const int h = (int)(u % (uint32_t)H);
        const int64_t nb = u < units ? nacc[b] : 0, s = u < units ? slots[b] : -1;
        ok[k] = nb >= 1 && nb <= T && s >= 0 && s < rows;
        from[k] = snaps + ((b * T + (ok[k] ? nb - 1 : 0)) * H + h) * (int64_t)HS2;
        to[k] = pool + ((ok[k] ? s : 0) * H + h) * (int64_t)HS2;
    }
    f4 x[UPW][4];
#pragma unroll
    for (int k = 0; k < UPW; ++k)
        if (ok[k])
#pragma unroll
            for (int v = 0; v < 4; ++v) x[k][v] = ldg4(from[k] + (v * kThreads + threadIdx.x) * 4);
#pragma unroll
    for (int k = 0; k < UPW; ++k)
        if (ok[k])
#pragma unroll
            for (int v = 0; v < 4; ++v) stg4(to[k] + (v * kThreads + threadIdx.x) * 4, x[k][v]);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace wkv7

extern "C" {

int wkv7_pool_reset(float* pool, int32_t layers, int64_t rows, int32_t H, const int64_t* idx, int32_t n,
                    void* stream) {
    if (layers < 0 || rows < 0 || H < 1 || n < 0) return WKV7_ERR_SHAPE;
    if (n == 0 || layers == 0 || rows == 0) return WKV7_OK;
    if (!pool || !idx) return WKV7_ERR_NULL;
    if (!wkv7::aligned16(pool)) return WKV7_ERR_ALIGN;
    const int64_t blocks = (int64_t)layers * n * H;
    if (blocks > 0x7fffffffLL) return WKV7_ERR_SHAPE;
    hipLaunchKernelGGL(wkv7::pool_reset_kernel, dim3((unsigned)blocks), dim3(wkv7::kThreads), 0,
                       static_cast<hipStream_t>(stream), pool, rows, (int)H, idx, (int)n);
    return static_cast<int>(hipGetLastError());
}

int wkv7_pool_move(float* pool, int32_t layers, int64_t rows, int32_t H, const int64_t* src, const int64_t* dst,
                   int32_t n, void* stream) {
    if (layers < 0 || rows < 0 || H < 1 || n < 0) return WKV7_ERR_SHAPE;
    if (n == 0 || layers == 0 || rows == 0) return WKV7_OK;
    if (!pool || !src || !dst) return WKV7_ERR_NULL;
    if (n > wkv7::kMaxMoves) return WKV7_ERR_SHAPE;
    if (!wkv7::aligned16(pool)) return WKV7_ERR_ALIGN;
    const int64_t row_len = (int64_t)H * wkv7::HS2;
    // positions per workgroup: as many as fit n staged copies in the LDS budget, a power of two in [16, 4096]
    int P = 4096;
    while (P > 16 && (int64_t)n * P * 4 > wkv7::kMoveLdsBytes) P >>= 1;
    const int64_t blocks = (int64_t)layers * (row_len / P);
    if (blocks > 0x7fffffffLL) return WKV7_ERR_SHAPE;
    hipLaunchKernelGGL(wkv7::pool_move_kernel, dim3((unsigned)blocks), dim3(wkv7::kThreads),
                       (size_t)n * P * sizeof(float), static_cast<hipStream_t>(stream), pool, rows, row_len, src, dst,
                       (int)n, P);
    return static_cast<int>(hipGetLastError());
}

int wkv7_snapshot_restore(float* pool, int64_t rows, int32_t H, const int64_t* slots, const float* snapshots,
                          int32_t T, const int64_t* n_accepted, int32_t num_seqs, void* stream) {
    if (rows < 0 || H < 1 || T < 1 || num_seqs < 0) return WKV7_ERR_SHAPE;
    if (num_seqs == 0 || rows == 0) return WKV7_OK;
    if (!pool || !slots || !snapshots || !n_accepted) return WKV7_ERR_NULL;
    if (!wkv7::aligned16(pool) || !wkv7::aligned16(snapshots)) return WKV7_ERR_ALIGN;
    // two units per workgroup once there are at least four per CU
    const int64_t units = (int64_t)num_seqs * H;
    const bool two = units >= 4 * (int64_t)wkv7::device_cu_count();
    const int64_t blocks = two ? (units + 1) / 2 : units;
    if (blocks > 0x7fffffffLL) return WKV7_ERR_SHAPE;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (two)
        hipLaunchKernelGGL(wkv7::snapshot_restore_kernel<2>, dim3((unsigned)blocks), dim3(wkv7::kThreads), 0, s, pool,
                           rows, (int)H, slots, snapshots, (int)T, n_accepted, units);
    else
        hipLaunchKernelGGL(wkv7::snapshot_restore_kernel<1>, dim3((unsigned)blocks), dim3(wkv7::kThreads), 0, s, pool,
                           rows, (int)H, slots, snapshots, (int)T, n_accepted, units);
    return static_cast<int>(hipGetLastError());
}

}  // extern "C"
