// wkv7_token.h -- the token-serial recurrence on one (sequence, head) pair held in one wavefront's registers: the
// per-pair building blocks of wkv7_recurrent.hip's kernels, shared with the single-dispatch chain kernel
// (wkv7_chunked.hip), which runs a ragged batch's short rows with them.
//
// Lane L = 16 g + c of a wavefront owns state rows k = 4 i + g (i = 0..15) and columns v = 4 c .. 4 c + 3: 64 fp32
// in VGPRs; each of the 16 dwordx4 row loads of a wave reads 1 KB contiguous.  The k-side vectors (decay, a, b, k,
// r) are computed by lane i for channel i and broadcast through a per-wave LDS slab of 5 x 64 floats; sa = a^T S and
// y = S^T r are lane-local sums over 16 rows plus a two-step xor butterfly.  One fixed instruction sequence per token
// with explicit fmaf (the files are built with -ffp-contract=off), so a snapshot after token t is bit-identical to a
// re-run over t + 1 tokens (rwkv_next/kernels/wkv7.py:65-77).
#pragma once
#include "wkv7_device.h"

namespace wkv7 {

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

}  // namespace wkv7
