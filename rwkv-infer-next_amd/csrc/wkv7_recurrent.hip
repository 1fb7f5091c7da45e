// wkv7_recurrent.hip -- token-serial WKV7 kernel: decode (T = 1), speculative verify (short T) with per-token
// state snapshots, in-place rollback replay (n_keep), and the short rows of a ragged batch.
//
// Replaces the reference's fused recurrent Triton program _wkv7_raw (rwkv_next/kernels/wkv7.py:38-79) for
// these cases.  Work decomposition (MI355X, wave64):
//   * one wavefront per (sequence, head) pair at a time.  wkv7_recurrent_kernel: at most two waves per SIMD;
//     each wave walks pairs gw, gw + nwaves, ... and issues the next pair's state loads before working on the
//     current pair, so state reads, the recurrence math and state writes of different pairs overlap.
//     wkv7_decode_kernel (single-token rows, at least three pairs per SIMD): one wave per SIMD issues the loads of
//     four pairs before updating and storing the first, so the grid's state reads run ahead of its writes;
//   * lane L = 16 g + c owns state rows k = 4 i + g (i = 0..15) and columns v = 4 c .. 4 c + 3: 64 fp32 in VGPRs.
//     Load instruction i of a wave reads rows 4i .. 4i+3, i.e. 1 KB contiguous, so a 16 KB state arrives in 16
//     coalesced dwordx4 instructions.  State traffic is streamed with non-temporal loads and stores (each state
//     is touched once per call);
//   * the per-token k-side vectors (decay, a, b, k, r) are computed by lane i for channel i and broadcast through
//     a per-wave LDS slab, stored permuted (channel 4 i + g at slot 16 g + i) so each lane group reads its 16
//     channels with four ds_read_b128; v is read per lane;
//   * sa = a^T S and y = S^T r are lane-local sums over the lane's 16 rows followed by a two-step xor butterfly
//     over the four row groups.  Every lane ends with bitwise identical sums (fp add is commutative), so all
//     lanes hold the same update.  Updated rows are stored as soon as they are final.
// Decode is HBM-bound: 16 KB state read + 16 KB written per pair, plus 896 B of operands and output.
//
// The per-token arithmetic is one fixed instruction sequence with explicit fmaf (the file is built with
// -ffp-contract=off), so a snapshot taken after token t is bit-identical to a re-run over the first t+1 tokens.
#include "wkv7_device.h"
#include "wkv7_launch.h"
#include "wkv7_token.h"

namespace wkv7 {

namespace {

constexpr int kWaves = 4;            // waves per workgroup
constexpr int kWavesPerSimd = 2;     // residency target: two 16 KB states in flight per wave

__global__ __launch_bounds__(64 * kWaves, kWavesPerSimd) void wkv7_recurrent_kernel(const Params p) {
    __shared__ __attribute__((aligned(16))) float slab[kWaves][5 * HS];  // decay, a, b, k, r (permuted)
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: indices stay in SGPRs
    const int g = lane >> 4, c = lane & 15;
    // pair indices fit 32 bits (wkv7_run validates num_seqs * H <= 2^31); 64-bit divisions are software-emulated
    const uint32_t npairs = (uint32_t)p.num_seqs * (uint32_t)p.H;
    const uint32_t nwaves = gridDim.x * kWaves;
    uint32_t pa = blockIdx.x * kWaves + wv;
    if (pa >= npairs) return;  // no workgroup barriers below: waves are independent

    f4 SA[16], SB[16];
    TokenIn xa{}, xb{};
    Pair qa = pair_of(p, pa);
    prefetch_pair(p, qa, lane, g, c, SA, xa);
    // Wave w takes pairs w, w + nwaves, ...  Two buffers, unrolled by two so that the state arrays stay in
    // registers: the next pair's loads are issued before the current pair runs.
    while (true) {
        const uint32_t pb = pa + nwaves;
        Pair qb{};
        if (pb < npairs) {
            qb = pair_of(p, pb);
            prefetch_pair(p, qb, lane, g, c, SB, xb);
        }
        run_pair(p, qa, lane, g, c, SA, xa, slab[wv]);
        if (pb >= npairs) break;
        pa = pb + nwaves;
        if (pa < npairs) {
            qa = pair_of(p, pa);
            prefetch_pair(p, qa, lane, g, c, SA, xa);
        }
        run_pair(p, qb, lane, g, c, SB, xb, slab[wv]);
        if (pa >= npairs) break;
    }
}

// Single-token rows (decode): one wavefront per SIMD; each wave issues the state loads of up to kGroup pairs
// (w, w + nwaves, ...) before updating and storing the first of them, so that across the grid the state reads run
// ahead of the state writes instead of mixing with them (a decode-shaped streaming probe: 64 MiB in place in
// 22.9 us this way, 25.0 us with two pairs per wave and two waves per SIMD).
constexpr int kGroup = 4;

__global__ __launch_bounds__(64 * kWaves, 1) void wkv7_decode_kernel(const Params p) {
    __shared__ __attribute__((aligned(16))) float slab[kWaves][5 * HS];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, c = lane & 15;
    const uint32_t npairs = (uint32_t)p.num_seqs * (uint32_t)p.H;
    const uint32_t nwaves = gridDim.x * kWaves;
    for (uint32_t base = blockIdx.x * kWaves + wv; base < npairs; base += kGroup * nwaves) {
        f4 S[kGroup][16];
        TokenIn x[kGroup];
        Pair q[kGroup];
#pragma unroll
        for (int j = 0; j < kGroup; ++j) {
            const uint32_t pj = base + j * nwaves;
            q[j] = Pair{};
            if (pj < npairs) {
                q[j] = pair_of(p, pj);
                prefetch_pair(p, q[j], lane, g, c, S[j], x[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < kGroup; ++j)
            if (base + j * nwaves < npairs) run_pair(p, q[j], lane, g, c, S[j], x[j], slab[wv]);
    }
}

}  // namespace

hipError_t launch_recurrent(const Params& p, hipStream_t stream) {
    const int64_t pairs = (int64_t)p.num_seqs * p.H;
    if (pairs == 0) return hipSuccess;
    const int cus = device_cu_count();
    // Dense single-token rows (decode) with at least three pairs per SIMD: the grouped kernel.  Measured per launch
    // (B x H pairs; this kernel / the double-buffered one): 3072 pairs 20.0 / 20.6 us, 4096 25.2 / 27.1, 6144
    // 40.1 / 41.0, 8192 50.8 / 53.6; fewer pairs do not fill its groups (2560: 19.5 / 17.6 us).
    const int64_t simds = (int64_t)cus * 4;
    if (p.T == 1 && !p.cu && pairs >= 3 * simds) {
        const int64_t waves = simds;  // one wavefront per SIMD
        const int64_t blocks = (waves + kWaves - 1) / kWaves;
        hipLaunchKernelGGL(wkv7_decode_kernel, dim3((unsigned)blocks), dim3(64 * kWaves), 0, stream, p);
        return hipGetLastError();
    }
    const int64_t max_waves = (int64_t)cus * 4 * kWavesPerSimd;  // 4 SIMDs per CU
    // As many waves as fit (measured: for H = 40, 2560 pairs, 2048 waves -- 512 of them taking a second pair -- run
    // in 17.6 us per launch; 1280 waves with two pairs each in 20.0 us: more states in flight beat an even split).
    const int64_t waves = pairs < max_waves ? pairs : max_waves;
    const int64_t blocks = (waves + kWaves - 1) / kWaves;
    hipLaunchKernelGGL(wkv7_recurrent_kernel, dim3((unsigned)blocks), dim3(64 * kWaves), 0, stream, p);
    return hipGetLastError();
}

}  // namespace wkv7
