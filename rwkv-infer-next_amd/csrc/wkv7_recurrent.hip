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

namespace wkv7 {

namespace {

constexpr int kWaves = 4;            // waves per workgroup
constexpr int kWavesPerSimd = 2;     // residency target: two 16 KB states in flight per wave

struct TokenIn {
    uint16_t w, a, b, k, r;
    uint2 v;  // 4 bf16: v[4c .. 4c+3]
};

__device__ __forceinline__ f4 load_nt(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
}
__device__ __forceinline__ void store_nt(float* p, f4 x) { __builtin_nontemporal_store(x, reinterpret_cast<f4*>(p)); }

// The token/head offset is wave-uniform and kept apart from the per-lane offset, so the loads use a scalar base
// address plus a 32-bit vector offset instead of one 64-bit address per lane and operand.
__device__ __forceinline__ void load_token(const Params& p, int64_t tok, int h, int lane, int c, TokenIn& x) {
    const int64_t off = tok * p.in_tok_stride + (int64_t)h * HS;
    x.w = uniform_ptr(p.w + off)[lane];
    x.a = uniform_ptr(p.a + off)[lane];
    x.b = uniform_ptr(p.b + off)[lane];
    x.k = uniform_ptr(p.k + off)[lane];
    x.r = uniform_ptr(p.r + off)[lane];
    x.v = uniform_ptr(reinterpret_cast<const uint2*>(p.v + off))[c];
}

__device__ __forceinline__ float butterfly4(float x) {
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

// Pair geometry: sequence, head, first token, length; `run` is false for pairs another launch owns.
struct Pair {
    int n, h, L;
    int64_t bos;
    bool run;
};

__device__ __forceinline__ Pair pair_of(const Params& p, uint32_t pair) {
    Pair q;
    q.n = (int)(pair / (uint32_t)p.H);
    q.h = (int)(pair % (uint32_t)p.H);
    seq_extent(p, q.n, q.bos, q.L);
    q.run = p.rec_max_len < 0 || q.L <= p.rec_max_len;  // else a chunked launch owns this row
    return q;
}

// Issue the loads of a pair's initial state (rows 4 i + g) and of its first token's operands.
__device__ __forceinline__ void prefetch_pair(const Params& p, const Pair& q, int lane, int g, int c, f4 (&S)[16],
                                              TokenIn& x) {
    if (!q.run) return;
    if (const float* src = state_src(p, q.n, q.h)) {
        const float* s = uniform_ptr(src);
#pragma unroll
        for (int i = 0; i < 16; ++i) S[i] = load_nt(s + (4 * i + g) * HS + 4 * c);
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) S[i] = f4{0.f, 0.f, 0.f, 0.f};
    }
    if (q.L > 0) load_token(p, q.bos, q.h, lane, c, x);
}

// The recurrence over one pair's tokens, state in S (rows 4 i + g, columns 4 c .. 4 c + 3).
__device__ __forceinline__ void run_pair(const Params& p, const Pair& q, int lane, int g, int c, f4 (&S)[16],
                                         TokenIn cur, float* slab) {
    if (!q.run) return;
    float* const dvec = slab;
    float* const avec = slab + HS;
    float* const bvec = slab + 2 * HS;
    float* const kvec = slab + 3 * HS;
    float* const rvec = slab + 4 * HS;
    const int slot = (lane & 3) * 16 + (lane >> 2);  // LDS position of channel `lane`
    float* const dst = state_dst(p, q.n, q.h);
    float* const dst_u = dst ? uniform_ptr(dst) : nullptr;
    TokenIn nxt = cur;
    for (int t = 0; t < q.L; ++t) {
        dvec[slot] = decay(bf16_to_f32(cur.w));
        avec[slot] = bf16_to_f32(cur.a);
        bvec[slot] = bf16_to_f32(cur.b);
        kvec[slot] = bf16_to_f32(cur.k);
        rvec[slot] = bf16_to_f32(cur.r);
        float vj[4];
        bf16x2_to_f32(cur.v.x, vj[0], vj[1]);
        bf16x2_to_f32(cur.v.y, vj[2], vj[3]);
        if (t + 1 < q.L) load_token(p, q.bos + t + 1, q.h, lane, c, nxt);  // in flight during this token's math
        wave_lds_sync();

        // sa[j] = sum_k a_k S[k][j] over the old state (wkv7.py:75)
        float sa[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            const f4 av = *reinterpret_cast<const f4*>(avec + 16 * g + 4 * i4);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
#pragma unroll
                for (int j = 0; j < 4; ++j) sa[j] = fmaf(av[ii], S[4 * i4 + ii][j], sa[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) sa[j] = butterfly4(sa[j]);

        // S[k][j] = d_k S[k][j] + b_k sa[j] + k_k v_j;  y[j] = sum_k r_k S[k][j] (updated state, wkv7.py:75-77)
        const bool last = t + 1 == q.L;
        float* const snap = (p.snap && t < p.T)
                                ? uniform_ptr(p.snap + (((int64_t)q.n * p.T + t) * p.H + q.h) * (int64_t)HS2)
                                : nullptr;
        float y[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            const f4 dv = *reinterpret_cast<const f4*>(dvec + 16 * g + 4 * i4);
            const f4 bv = *reinterpret_cast<const f4*>(bvec + 16 * g + 4 * i4);
            const f4 kv = *reinterpret_cast<const f4*>(kvec + 16 * g + 4 * i4);
            const f4 rv = *reinterpret_cast<const f4*>(rvec + 16 * g + 4 * i4);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const int i = 4 * i4 + ii;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    S[i][j] = fmaf(dv[ii], S[i][j], fmaf(bv[ii], sa[j], kv[ii] * vj[j]));
                    y[j] = fmaf(rv[ii], S[i][j], y[j]);
                }
            }
            if (snap) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) store_nt(snap + (4 * (4 * i4 + ii) + g) * HS + 4 * c, S[4 * i4 + ii]);
            }
            if (last && dst_u) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) store_nt(dst_u + (4 * (4 * i4 + ii) + g) * HS + 4 * c, S[4 * i4 + ii]);
            }
            // keeps the scheduler from hoisting all 64 broadcast reads above the FMAs (VGPR budget)
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) y[j] = butterfly4(y[j]);

        if (p.o && g == 0) {
            uint2 pk;
            pk.x = pack_bf16x2(y[0], y[1]);
            pk.y = pack_bf16x2(y[2], y[3]);
            uniform_ptr(reinterpret_cast<uint2*>(p.o + (q.bos + t) * p.o_tok_stride + (int64_t)q.h * HS))[c] = pk;
        }
        cur = nxt;
        wave_lds_sync();  // this token's LDS reads precede the next token's writes
    }
    if (q.L == 0 && dst_u) {  // no tokens: the state passes through (wkv7.py:65-79 with L = 0)
#pragma unroll
        for (int i = 0; i < 16; ++i) store_nt(dst_u + (4 * i + g) * HS + 4 * c, S[i]);
    }
}

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
