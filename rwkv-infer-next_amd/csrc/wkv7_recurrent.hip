// wkv7_recurrent.hip -- token-serial WKV7 kernels: decode (T = 1), speculative verify (short T) with per-token
// state snapshots, in-place rollback replay (n_keep), and the short rows of a ragged batch.
//
// Replaces the reference's fused recurrent Triton program _wkv7_raw (rwkv_next/kernels/wkv7.py:38-79) for
// these cases.  Work decomposition (MI355X, wave64):
//   * wkv7_recurrent_kernel (every row shape): one wavefront per (sequence, head) pair at a time, at most two waves
//     per SIMD; each wave walks pairs gw, gw + nwaves, ... and issues the next pair's state loads before working on
//     the current pair, so state reads, the recurrence math and state writes of different pairs overlap.  Lane
//     L = 8 g + c owns state rows k = 8 i + g (i = 0..7) and columns 32 hh + 4 c .. + 3 (hh = 0, 1; the per-pair
//     code of wkv7_token.h);
//   * wkv7_decode_kernel (dense single-token rows without snapshots): half-pair units (32 columns of one pair), one
//     wave per SIMD holding up to eight units, all of their loads issued before the first update, so that across the
//     grid the state reads run ahead of the writes;
//   * the per-token k-side vectors (decay, a, b, k, r) are computed by lane i for channel i and broadcast through
//     a per-wave LDS slab; v is read per lane; sa = a^T S and y = S^T r are lane-local sums over the lane's 8 rows
//     followed by a butterfly over the 8 row groups, in the same order in both kernels.  Every lane ends with
//     bitwise identical sums (fp add is commutative), so all lanes hold the same update.  State traffic is streamed
//     with non-temporal loads and stores (each state is touched once per call).
// Decode is HBM-bound: 16 KB state read + 16 KB written per pair, plus 896 B of operands and output.
//
// The per-token arithmetic is one fixed instruction sequence with explicit fmaf (the file is built with
// -ffp-contract=off), shared by both kernels: a snapshot taken after token t is bit-identical to a re-run over the
// first t+1 tokens, by either kernel (t + 1 single-token decode steps included).
#include <algorithm>

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
    const int g = lane >> 3, c = lane & 7;
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

// Dense single-token rows (decode) without snapshots: half-pair units.  Unit u is pair u >> 1, columns
// 32 (u & 1) .. + 31.  The recurrence is column-local (sa_j = a^T S[:, j] and y_j = r^T S[:, j] read column j only),
// so the two halves of a pair are independent.  One wavefront per SIMD holds G units, u = w, w + nwaves, ..., so
// 2 B H units spread evenly over the SIMDs (B = 64, H = 40: five per SIMD, where whole pairs would leave some SIMDs
// three and some two), and all of a wave's state loads are in flight before its first update.  Measured per launch
// at B = 64 (pool slots, HIP graph of 32 layers): H = 64 24.7 us (whole pairs, four per wave: 25.3), H = 40 16.2 us
// (17.5), H = 8 5.3 us (5.9).
// Lane L = 8 g + c owns rows k = 8 i + g (i = 0..7) and columns 32 half + 4 c .. + 3: 32 fp32 per unit.  Load
// instruction i of a unit reads rows 8 i .. 8 i + 7, 128 contiguous bytes each.  sa and y are lane-local sums over
// 8 rows and a three-step butterfly over the row groups: the same arithmetic as wkv7_token.h's per-pair code, so a
// decode step lands on the same bits as that token run inside a verify (snapshots) or a rollback replay.
// State rows go through buffer resources that cover the 16 KB state or nothing (num_records = 0: loads return zeros,
// stores are dropped), so a zero initial state or an unstored final state needs no branch around the loads.
constexpr int kDecodeMaxUnits = 8;

struct HalfIn {  // one token's operands for a half-pair unit
    uint16_t w, a, b, k, r;
    uint2 v;  // 4 bf16: v[32 half + 4c .. + 3]
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t state_rsrc(const float* base, bool live) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, live ? HS2 * (int)sizeof(float) : 0,
                                             0x00020000 /* raw 32-bit buffer, gfx9 family */);
}

constexpr int kCachePolicyNT = 2;  // buffer-instruction cache policy: non-temporal
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int G>
__global__ __launch_bounds__(64 * kWaves, 1) void wkv7_decode_kernel(const Params p) {
    __shared__ __attribute__((aligned(16))) float slab[kWaves][5 * HS];  // decay, a, b, k, r (permuted)
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 3, c = lane & 7;
    const uint64_t nunits = 2ull * (uint64_t)p.num_seqs * (uint64_t)p.H;  // pair indices u >> 1 fit 31 bits
    const uint32_t nwaves = gridDim.x * kWaves;
    float* const dvec = slab[wv];
    float* const avec = dvec + HS;
    float* const bvec = dvec + 2 * HS;
    float* const kvec = dvec + 3 * HS;
    float* const rvec = dvec + 4 * HS;
    const int slot = slab_slot(lane);  // LDS position of channel `lane` (channel 8 i + g at 8 g + i)
    const int rowoff = g * HS + 4 * c;               // this lane's offset (floats) in rows 0 .. 7
    auto lane64 = [](int64_t x, int j) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, j);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)x >> 32), j);
        return (int64_t)(((uint64_t)hi << 32) | lo);
    };

    for (uint64_t base = blockIdx.x * kWaves + wv; base < nunits; base += (uint64_t)G * nwaves) {
        // Unit j's state rows and token count, gathered in lane j (j < G).  Dense single-token rows: the row of
        // sequence n is token n, its length min(1, max(n_keep[n], 0)).
        const uint64_t mu = base + (uint64_t)lane * nwaves;
        const bool mvalid = lane < G && mu < nunits;
        const uint32_t mpr = (uint32_t)((mvalid ? mu : 0) >> 1);
        const int mn = (int)(mpr / (uint32_t)p.H), mh = (int)(mpr % (uint32_t)p.H);
        int64_t nk = 1, hi = mn, ti = mn;
        uint8_t fr = 0;
        if (p.n_keep) nk = p.n_keep[mn];
        if (p.fresh) fr = p.fresh[mn];
        if (p.h0_idx) hi = p.h0_idx[mn];
        if (p.ht_idx) ti = p.ht_idx[mn];
        // The token operands depend on no index: their loads go out while the index loads are in flight (units past
        // nunits read token 0, which always exists).
        HalfIn x[G];
        int col0[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const uint64_t u = base + (uint64_t)j * nwaves;
            const uint32_t pr = (uint32_t)((u < nunits ? u : 0) >> 1);
            const int n = (int)(pr / (uint32_t)p.H), h = (int)(pr % (uint32_t)p.H);
            col0[j] = 32 * (int)(u & 1);
            const int64_t off = (int64_t)n * p.in_tok_stride + (int64_t)h * HS;
            x[j].w = uniform_ptr(p.w + off)[lane];
            x[j].a = uniform_ptr(p.a + off)[lane];
            x[j].b = uniform_ptr(p.b + off)[lane];
            x[j].k = uniform_ptr(p.k + off)[lane];
            x[j].r = uniform_ptr(p.r + off)[lane];
            x[j].v = uniform_ptr(reinterpret_cast<const uint2*>(p.v + off + col0[j]))[c];
        }
        __builtin_amdgcn_sched_barrier(0);  // the index values are first used below, after the token loads
        const int mlen = mvalid && nk >= 1 ? 1 : 0;
        const int64_t msrc = (mvalid && p.h0 && !fr && hi >= 0 && hi < p.h0_rows) ? (hi * p.H + mh) * (int64_t)HS2 : -1;
        const int64_t mdst = (mvalid && p.ht && ti >= 0 && ti < p.ht_rows) ? (ti * p.H + mh) * (int64_t)HS2 : -1;
        f4 S[G][8];
        int len[G];
        __amdgpu_buffer_rsrc_t dst[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const int64_t s = lane64(msrc, j), d = lane64(mdst, j);
            len[j] = __builtin_amdgcn_readlane(mlen, j);
            // a row another launch owns (rec_max_len) is neither read nor written here
            const bool mine = base + (uint64_t)j * nwaves < nunits && (p.rec_max_len < 0 || len[j] <= p.rec_max_len);
            const __amdgpu_buffer_rsrc_t src = state_rsrc(s >= 0 ? p.h0 + s : nullptr, mine && s >= 0);
            dst[j] = state_rsrc(d >= 0 ? p.ht + d : nullptr, mine && d >= 0);
            if (!mine) len[j] = -1;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                S[j][i] = __builtin_bit_cast(
                    f4, __builtin_amdgcn_raw_buffer_load_b128(
                            src, (int)((rowoff + 8 * i * HS + col0[j]) * sizeof(float)), 0, kCachePolicyNT));
        }

#pragma unroll
        for (int j = 0; j < G; ++j) {
            if (len[j] < 0) continue;  // wave-uniform
            if (len[j] == 1) {
                const HalfIn cur = x[j];
                dvec[slot] = decay(bf16_to_f32(cur.w));
                avec[slot] = bf16_to_f32(cur.a);
                bvec[slot] = bf16_to_f32(cur.b);
                kvec[slot] = bf16_to_f32(cur.k);
                rvec[slot] = bf16_to_f32(cur.r);
                float vj[4];
                bf16x2_to_f32(cur.v.x, vj[0], vj[1]);
                bf16x2_to_f32(cur.v.y, vj[2], vj[3]);
                wave_lds_sync();
                // sa[q] = sum_k a_k S[k][q] over the old state (wkv7.py:75)
                float sa[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i2 = 0; i2 < 2; ++i2) {
                    const f4 av = *reinterpret_cast<const f4*>(avec + 8 * g + 4 * i2);
#pragma unroll
                    for (int ii = 0; ii < 4; ++ii) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) sa[q] = fmaf(av[ii], S[j][4 * i2 + ii][q], sa[q]);
                    }
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) sa[q] = butterfly8(sa[q]);
                // S[k][q] = d_k S[k][q] + b_k sa[q] + k_k v_q;  y[q] = sum_k r_k S[k][q] (updated state, wkv7.py:75-77)
                float y[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i2 = 0; i2 < 2; ++i2) {
                    const f4 dv = *reinterpret_cast<const f4*>(dvec + 8 * g + 4 * i2);
                    const f4 bv = *reinterpret_cast<const f4*>(bvec + 8 * g + 4 * i2);
                    const f4 kv = *reinterpret_cast<const f4*>(kvec + 8 * g + 4 * i2);
                    const f4 rv = *reinterpret_cast<const f4*>(rvec + 8 * g + 4 * i2);
#pragma unroll
                    for (int ii = 0; ii < 4; ++ii) {
                        const int i = 4 * i2 + ii;
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            S[j][i][q] = fmaf(dv[ii], S[j][i][q], fmaf(bv[ii], sa[q], kv[ii] * vj[q]));
                            y[q] = fmaf(rv[ii], S[j][i][q], y[q]);
                        }
                    }
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) y[q] = butterfly8(y[q]);
                if (p.o && g == 0) {
                    const uint32_t pr = (uint32_t)((base + (uint64_t)j * nwaves) >> 1);
                    const int n = (int)(pr / (uint32_t)p.H), h = (int)(pr % (uint32_t)p.H);
                    uint2 pk;
                    pk.x = pack_bf16x2(y[0], y[1]);
                    pk.y = pack_bf16x2(y[2], y[3]);
                    uniform_ptr(reinterpret_cast<uint2*>(p.o + (int64_t)n * p.o_tok_stride + (int64_t)h * HS +
                                                         col0[j]))[c] = pk;
                }
                wave_lds_sync();  // this unit's LDS reads precede the next unit's writes
            }
            // the updated state, or for a row with no tokens the initial state passed through (dropped when not
            // stored)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, S[j][i]), dst[j],
                                                       (int)((rowoff + 8 * i * HS + col0[j]) * sizeof(float)), 0,
                                                       kCachePolicyNT);
        }
    }
}

// One decode token on a half-pair unit's state S (rows 8 i + g, columns col0 + 4 c .. + 3) and its output, u the unit
// index; dvec is the wave's LDS slab (decay, a, b, k, r, 64 floats each).  The same instruction sequence as the
// token step written out in wkv7_decode_kernel (kept inline there: its register allocation at eight units per wave
// is tuned), so both decode kernels produce the same bits; a GPU test compares them.
__device__ __forceinline__ void decode_token(const Params& p, const HalfIn& x, f4 (&S)[8], uint64_t u, int col0, int g,
                             int c, int slot, float* dvec, uint32_t nwaves) {
    float* const avec = dvec + HS;
    float* const bvec = dvec + 2 * HS;
    float* const kvec = dvec + 3 * HS;
    float* const rvec = dvec + 4 * HS;
    const HalfIn& cur = x;
    dvec[slot] = decay(bf16_to_f32(cur.w));
    avec[slot] = bf16_to_f32(cur.a);
    bvec[slot] = bf16_to_f32(cur.b);
    kvec[slot] = bf16_to_f32(cur.k);
    rvec[slot] = bf16_to_f32(cur.r);
    float vj[4];
    bf16x2_to_f32(cur.v.x, vj[0], vj[1]);
    bf16x2_to_f32(cur.v.y, vj[2], vj[3]);
    wave_lds_sync();
    // sa[q] = sum_k a_k S[k][q] over the old state (wkv7.py:75)
    float sa[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i2 = 0; i2 < 2; ++i2) {
        const f4 av = *reinterpret_cast<const f4*>(avec + 8 * g + 4 * i2);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
#pragma unroll
            for (int q = 0; q < 4; ++q) sa[q] = fmaf(av[ii], S[4 * i2 + ii][q], sa[q]);
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) sa[q] = butterfly8(sa[q]);
    // S[k][q] = d_k S[k][q] + b_k sa[q] + k_k v_q;  y[q] = sum_k r_k S[k][q] (updated state, wkv7.py:75-77)
    float y[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i2 = 0; i2 < 2; ++i2) {
        const f4 dv = *reinterpret_cast<const f4*>(dvec + 8 * g + 4 * i2);
        const f4 bv = *reinterpret_cast<const f4*>(bvec + 8 * g + 4 * i2);
        const f4 kv = *reinterpret_cast<const f4*>(kvec + 8 * g + 4 * i2);
        const f4 rv = *reinterpret_cast<const f4*>(rvec + 8 * g + 4 * i2);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const int i = 4 * i2 + ii;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                S[i][q] = fmaf(dv[ii], S[i][q], fmaf(bv[ii], sa[q], kv[ii] * vj[q]));
                y[q] = fmaf(rv[ii], S[i][q], y[q]);
            }
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) y[q] = butterfly8(y[q]);
    if (p.o && g == 0) {
        const uint32_t pr = (uint32_t)(u >> 1);
        const int n = (int)(pr / (uint32_t)p.H), h = (int)(pr % (uint32_t)p.H);
        uint2 pk;
        pk.x = pack_bf16x2(y[0], y[1]);
        pk.y = pack_bf16x2(y[2], y[3]);
        uniform_ptr(reinterpret_cast<uint2*>(p.o + (int64_t)n * p.o_tok_stride + (int64_t)h * HS +
                                             col0))[c] = pk;
    }
    wave_lds_sync();  // this unit's LDS reads precede the next unit's writes
}

// Wave-uniform loads through the constant address space compile to scalar loads (s_load), which put a unit's slot
// index into the SGPRs that address its state without a vector load and a readlane.  The caller's index arrays are
// not written during the launch.
template <typename T>
__device__ __forceinline__ T scalar_load(const T* ptr) {
    return *(const __attribute__((address_space(4))) T*)(ptr);
}
// One byte by a scalar load of the aligned dword that holds it (an aligned dword never crosses a page, so it is
// mapped wherever the byte is).
__device__ __forceinline__ int scalar_load_u8(const uint8_t* ptr) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(ptr);
    const uint32_t w = scalar_load(reinterpret_cast<const uint32_t*>(a & ~(uintptr_t)3));
    return (int)((w >> (8 * (a & 3))) & 0xffu);
}

// The decode kernel for launches with few units per wave (G <= kDecodeScalarMaxUnits: small B * H, e.g. one
// tensor-parallel rank's heads), where the launch is latency-bound: each unit's row metadata (n_keep, fresh, the
// two slot indices) comes by scalar loads issued before the token loads, so the state loads start one vector round
// trip earlier.  Same layout and arithmetic as wkv7_decode_kernel.  (For many units per wave the vector gather of
// wkv7_decode_kernel is faster: 2 G scalar loads and their SGPRs cost more than one vector round trip.)
constexpr int kDecodeScalarMaxUnits = 4;

template <int G>
__global__ __launch_bounds__(64 * kWaves, 1) void wkv7_decode_small_kernel(const Params p) {
    __shared__ __attribute__((aligned(16))) float slab[kWaves][5 * HS];  // decay, a, b, k, r (permuted)
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 3, c = lane & 7;
    const uint64_t nunits = 2ull * (uint64_t)p.num_seqs * (uint64_t)p.H;
    const uint32_t nwaves = gridDim.x * kWaves;
    float* const dvec = slab[wv];
    const int slot = slab_slot(lane);
    const int rowoff = g * HS + 4 * c;

    for (uint64_t base = blockIdx.x * kWaves + wv; base < nunits; base += (uint64_t)G * nwaves) {
        HalfIn x[G];
        int col0[G], hd[G], fr[G];
        int64_t nk[G], hi[G], ti[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const uint64_t u = base + (uint64_t)j * nwaves;
            const uint32_t pr = (uint32_t)((u < nunits ? u : 0) >> 1);
            const int n = (int)(pr / (uint32_t)p.H), h = (int)(pr % (uint32_t)p.H);
            hd[j] = h;
            nk[j] = p.n_keep ? scalar_load(p.n_keep + n) : 1;
            fr[j] = p.fresh ? scalar_load_u8(p.fresh + n) : 0;
            hi[j] = p.h0_idx ? scalar_load(p.h0_idx + n) : n;
            ti[j] = p.ht_idx ? scalar_load(p.ht_idx + n) : n;
            col0[j] = 32 * (int)(u & 1);
            const int64_t off = (int64_t)n * p.in_tok_stride + (int64_t)h * HS;
            x[j].w = uniform_ptr(p.w + off)[lane];
            x[j].a = uniform_ptr(p.a + off)[lane];
            x[j].b = uniform_ptr(p.b + off)[lane];
            x[j].k = uniform_ptr(p.k + off)[lane];
            x[j].r = uniform_ptr(p.r + off)[lane];
            x[j].v = uniform_ptr(reinterpret_cast<const uint2*>(p.v + off + col0[j]))[c];
        }
        __builtin_amdgcn_sched_barrier(0);
        f4 S[G][8];
        int len[G];
        __amdgpu_buffer_rsrc_t dst[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const bool valid = base + (uint64_t)j * nwaves < nunits;
            len[j] = valid && nk[j] >= 1 ? 1 : 0;
            const int64_t s = (valid && p.h0 && !fr[j] && hi[j] >= 0 && hi[j] < p.h0_rows)
                                  ? (hi[j] * p.H + hd[j]) * (int64_t)HS2 : -1;
            const int64_t d = (valid && p.ht && ti[j] >= 0 && ti[j] < p.ht_rows) ? (ti[j] * p.H + hd[j]) * (int64_t)HS2
                                                                               : -1;
            const bool mine = valid && (p.rec_max_len < 0 || len[j] <= p.rec_max_len);
            const __amdgpu_buffer_rsrc_t src = state_rsrc(s >= 0 ? p.h0 + s : nullptr, mine && s >= 0);
            dst[j] = state_rsrc(d >= 0 ? p.ht + d : nullptr, mine && d >= 0);
            if (!mine) len[j] = -1;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                S[j][i] = __builtin_bit_cast(
                    f4, __builtin_amdgcn_raw_buffer_load_b128(
                            src, (int)((rowoff + 8 * i * HS + col0[j]) * sizeof(float)), 0, kCachePolicyNT));
        }
#pragma unroll
        for (int j = 0; j < G; ++j) {
            if (len[j] == 1) decode_token(p, x[j], S[j], base + (uint64_t)j * nwaves, col0[j], g, c, slot, dvec, nwaves);
            if (len[j] < 0) continue;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, S[j][i]), dst[j],
                                                       (int)((rowoff + 8 * i * HS + col0[j]) * sizeof(float)), 0,
                                                       kCachePolicyNT);
        }
    }
}

}  // namespace

hipError_t launch_recurrent(const Params& p, hipStream_t stream) {
    const int64_t pairs = (int64_t)p.num_seqs * p.H;
    if (pairs == 0) return hipSuccess;
    const int cus = device_cu_count();
    const int64_t simds = (int64_t)cus * 4;
    // Dense single-token rows without snapshots: the decode kernel, one wavefront per SIMD (or one per unit when
    // there are fewer units than SIMDs), ceil(units / waves) units per wave up to eight, then further rounds.
    if (p.T == 1 && !p.cu && !p.snap) {
        const int64_t units = 2 * pairs;
        const int64_t waves = std::min<int64_t>(units, simds);
        const int G = (int)std::min<int64_t>((units + waves - 1) / waves, kDecodeMaxUnits);
        const dim3 grid((unsigned)((waves + kWaves - 1) / kWaves)), block(64 * kWaves);
        if (G <= kDecodeScalarMaxUnits) {
            switch (G) {
                case 1: hipLaunchKernelGGL(wkv7_decode_small_kernel<1>, grid, block, 0, stream, p); break;
                case 2: hipLaunchKernelGGL(wkv7_decode_small_kernel<2>, grid, block, 0, stream, p); break;
                case 3: hipLaunchKernelGGL(wkv7_decode_small_kernel<3>, grid, block, 0, stream, p); break;
                default: hipLaunchKernelGGL(wkv7_decode_small_kernel<4>, grid, block, 0, stream, p); break;
            }
            return hipGetLastError();
        }
        switch (G) {
            case 1: hipLaunchKernelGGL(wkv7_decode_kernel<1>, grid, block, 0, stream, p); break;
            case 2: hipLaunchKernelGGL(wkv7_decode_kernel<2>, grid, block, 0, stream, p); break;
            case 3: hipLaunchKernelGGL(wkv7_decode_kernel<3>, grid, block, 0, stream, p); break;
            case 4: hipLaunchKernelGGL(wkv7_decode_kernel<4>, grid, block, 0, stream, p); break;
            case 5: hipLaunchKernelGGL(wkv7_decode_kernel<5>, grid, block, 0, stream, p); break;
            case 6: hipLaunchKernelGGL(wkv7_decode_kernel<6>, grid, block, 0, stream, p); break;
            case 7: hipLaunchKernelGGL(wkv7_decode_kernel<7>, grid, block, 0, stream, p); break;
            default: hipLaunchKernelGGL(wkv7_decode_kernel<8>, grid, block, 0, stream, p); break;
        }
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
