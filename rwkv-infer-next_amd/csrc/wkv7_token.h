// wkv7_token.h -- the token-serial recurrence on one (sequence, head) pair held in one wavefront's registers: the
// per-pair building blocks of wkv7_recurrent.hip's kernels, shared with the single-dispatch chain kernel
// (wkv7_chunked.hip), which runs a ragged batch's short rows with them.
//
// Lane L = 8 g + c of a wavefront owns state rows k = 8 i + g (i = 0..7) and, in two halves hh = 0, 1, columns
// v = 32 hh + 4 c .. + 3: 64 fp32 in VGPRs; each of the 16 dwordx4 row loads of a wave reads 8 rows x 128 contiguous
// bytes.  The k-side vectors (decay, a, b, k, r) are computed by lane i for channel i and broadcast through a per-wave
// LDS slab of 5 x 64 floats; sa = a^T S and y = S^T r are, per column, an fmaf chain over the lane's 8 rows in i order
// plus a three-step butterfly over the row groups g.  This is exactly the arithmetic of the decode kernel
// (wkv7_recurrent.hip), whose half-pair units hold the same rows and columns of one half: a state reached token by
// token here (verify snapshots, rollback replays, short ragged rows) is bit-identical to the same tokens run as
// single-token decode steps.  One fixed instruction sequence per token with explicit fmaf (the files are built with
// -ffp-contract=off), so a snapshot after token t is also bit-identical to a re-run over t + 1 tokens
// (rwkv_next/kernels/wkv7.py:65-77).
#pragma once
#include "wkv7_device.h"

namespace wkv7 {

struct TokenIn {
    uint16_t w, a, b, k, r;
    uint2 v[2];  // 4 bf16 per half: v[32 hh + 4c .. + 3]
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
    x.v[0] = uniform_ptr(reinterpret_cast<const uint2*>(p.v + off))[c];
    x.v[1] = uniform_ptr(reinterpret_cast<const uint2*>(p.v + off + 32))[c];
}

// Sum over the eight row groups g = lane >> 3 (lanes L, L ^ 8, L ^ 16, ... ^ 56), without LDS: DPP row_ror:8 pairs
// the halves of each 16-lane row, v_permlane16_swap pairs rows 0-1 and 2-3, v_permlane32_swap the wave's halves.
// Every lane adds the same partial sums in the same order, so all lanes end with the same float.  (Cross-lane reads
// need their source lanes active: every lane runs this.)
__device__ __forceinline__ float butterfly8(float x) {
    float r = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128 /* row_ror:8 */, 0xf, 0xf, false));
    x += r;
    const auto pr = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    float e = __uint_as_float(pr[0]), o = __uint_as_float(pr[1]);  // the even row's value, the odd row's
    x = e + o;
    const auto hv = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    float lo = __uint_as_float(hv[0]), hi = __uint_as_float(hv[1]);  // rows 0-1, rows 2-3
    return lo + hi;
}

// LDS slab position of channel `lane`: channel 8 i + g at 8 g + i, so lane group g reads its rows' values as two f4
__device__ __forceinline__ int slab_slot(int lane) { return (lane & 7) * 8 + (lane >> 3); }

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

// state element offset (floats) of row 8 i + g, half hh, for lane (g, c)
__device__ __forceinline__ int state_off(int i, int hh, int g, int c) { return (8 * i + g) * HS + 32 * hh + 4 * c; }

// Issue the loads of a pair's initial state and of its first token's operands.  S[8 hh + i] holds row 8 i + g,
// columns 32 hh + 4 c .. + 3.
__device__ __forceinline__ void prefetch_pair(const Params& p, const Pair& q, int lane, int g, int c, f4 (&S)[16],
                                              TokenIn& x) {
    if (!q.run) return;
    if (const float* src = state_src(p, q.n, q.h)) {
        const float* s = uniform_ptr(src);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int i = 0; i < 8; ++i) S[8 * hh + i] = load_nt(s + state_off(i, hh, g, c));
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) S[i] = f4{0.f, 0.f, 0.f, 0.f};
    }
    if (q.L > 0) load_token(p, q.bos, q.h, lane, c, x);
}

// The recurrence over one pair's tokens, state in S (as prefetch_pair leaves it).
__device__ __forceinline__ void run_pair(const Params& p, const Pair& q, int lane, int g, int c, f4 (&S)[16],
                                         TokenIn cur, float* slab) {
    if (!q.run) return;
    float* const dvec = slab;
    float* const avec = slab + HS;
    float* const bvec = slab + 2 * HS;
    float* const kvec = slab + 3 * HS;
    float* const rvec = slab + 4 * HS;
    const int slot = slab_slot(lane);
    float* const dst = state_dst(p, q.n, q.h);
    float* const dst_u = dst ? uniform_ptr(dst) : nullptr;
    TokenIn nxt = cur;
    for (int t = 0; t < q.L; ++t) {
        dvec[slot] = decay(bf16_to_f32(cur.w));
        avec[slot] = bf16_to_f32(cur.a);
        bvec[slot] = bf16_to_f32(cur.b);
        kvec[slot] = bf16_to_f32(cur.k);
        rvec[slot] = bf16_to_f32(cur.r);
        float vj[2][4];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            bf16x2_to_f32(cur.v[hh].x, vj[hh][0], vj[hh][1]);
            bf16x2_to_f32(cur.v[hh].y, vj[hh][2], vj[hh][3]);
        }
        if (t + 1 < q.L) load_token(p, q.bos + t + 1, q.h, lane, c, nxt);  // in flight during this token's math
        wave_lds_sync();

        // sa[j] = sum_k a_k S[k][j] over the old state (wkv7.py:75)
        float sa[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
            const f4 av = *reinterpret_cast<const f4*>(avec + 8 * g + 4 * i2);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int j = 0; j < 4; ++j) sa[hh][j] = fmaf(av[ii], S[8 * hh + 4 * i2 + ii][j], sa[hh][j]);
            }
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int j = 0; j < 4; ++j) sa[hh][j] = butterfly8(sa[hh][j]);

        // S[k][j] = d_k S[k][j] + b_k sa[j] + k_k v_j;  y[j] = sum_k r_k S[k][j] (updated state, wkv7.py:75-77)
        const bool last = t + 1 == q.L;
        float* const snap = (p.snap && t < p.T)
                                ? uniform_ptr(p.snap + (((int64_t)q.n * p.T + t) * p.H + q.h) * (int64_t)HS2)
                                : nullptr;
        float y[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
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
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        S[8 * hh + i][j] = fmaf(dv[ii], S[8 * hh + i][j], fmaf(bv[ii], sa[hh][j], kv[ii] * vj[hh][j]));
                        y[hh][j] = fmaf(rv[ii], S[8 * hh + i][j], y[hh][j]);
                    }
            }
            if (snap) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii)
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
                        store_nt(snap + state_off(4 * i2 + ii, hh, g, c), S[8 * hh + 4 * i2 + ii]);
            }
            if (last && dst_u) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii)
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
                        store_nt(dst_u + state_off(4 * i2 + ii, hh, g, c), S[8 * hh + 4 * i2 + ii]);
            }
            // keeps the scheduler from hoisting all the broadcast reads above the FMAs (VGPR budget)
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int j = 0; j < 4; ++j) y[hh][j] = butterfly8(y[hh][j]);

        if (p.o && g == 0) {
            uint2* const orow = uniform_ptr(reinterpret_cast<uint2*>(p.o + (q.bos + t) * p.o_tok_stride + (int64_t)q.h * HS));
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                uint2 pk;
                pk.x = pack_bf16x2(y[hh][0], y[hh][1]);
                pk.y = pack_bf16x2(y[hh][2], y[hh][3]);
                orow[8 * hh + c] = pk;
            }
        }
        cur = nxt;
        wave_lds_sync();  // this token's LDS reads precede the next token's writes
    }
    if (q.L == 0 && dst_u) {  // no tokens: the state passes through (wkv7.py:65-79 with L = 0)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int i = 0; i < 8; ++i) store_nt(dst_u + state_off(i, hh, g, c), S[8 * hh + i]);
    }
}

}  // namespace wkv7
