// wkv7_recurrent.hip -- token-serial WKV7 kernel: decode (T = 1), speculative verify (short T) with per-token
// state snapshots, in-place rollback replay (n_keep), and the short rows of a ragged batch.
//
// Replaces the reference's fused recurrent Triton program _wkv7_raw (rwkv_next/kernels/wkv7.py:38-79) for
// these cases.  Work decomposition (MI355X, wave64):
//   * one wavefront per (sequence, head); a 256-thread workgroup holds 4 independent pairs;
//   * lane L = 16 g + c owns state rows k = 16 g .. 16 g + 15 and columns v = 4 c .. 4 c + 3, i.e. 64 fp32 in
//     VGPRs.  Each of the 16 row loads is one dwordx4 per lane, and one load instruction of the wave reads four
//     full 256-byte state rows, so the 16 KB state arrives in 16 coalesced instructions;
//   * the per-token k-side vectors (decay, a, b, k, r) are computed by lane i for channel i and broadcast
//     through a 1.25 KB per-wave LDS slab; v is read per lane;
//   * sa = a^T S and y = S^T r are lane-local sums over the lane's 16 rows followed by a two-step xor butterfly
//     over the four row groups.  Every lane ends with bitwise identical sums (fp add is commutative), so all
//     lanes hold the same update.
// Decode is HBM-bound: 16 KB state read + 16 KB written per pair, plus 896 B of operands and output.
//
// The per-token arithmetic is one fixed instruction sequence with explicit fmaf (the file is built with
// -ffp-contract=off), so a snapshot taken after token t is bit-identical to a re-run over the first t+1 tokens.
#include "wkv7_device.h"
#include "wkv7_launch.h"

namespace wkv7 {

namespace {

constexpr int kWaves = 4;

struct TokenIn {
    uint16_t w, a, b, k, r;
    uint2 v;  // 4 bf16: v[4c .. 4c+3]
};

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

__global__ __launch_bounds__(256, 4) void wkv7_recurrent_kernel(const Params p) {
    __shared__ __attribute__((aligned(16))) float vec[kWaves][5][HS];  // decay, a, b, k, r
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: indices stay in SGPRs
    const int64_t pair = (int64_t)blockIdx.x * kWaves + wv;
    if (pair >= (int64_t)p.num_seqs * p.H) return;  // no workgroup barriers below: waves are independent
    const int n = (int)(pair / p.H), h = (int)(pair % p.H);
    int64_t bos;
    int L;
    seq_extent(p, n, bos, L);
    if (p.rec_max_len >= 0 && L > p.rec_max_len) return;  // a chunked launch owns this row

    const int g = lane >> 4, c = lane & 15;
    float S[16][4];
    if (const float* src = state_src(p, n, h)) {
        const float* s = src + (16 * g) * HS + 4 * c;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const f4 x = *reinterpret_cast<const f4*>(s + i * HS);
            S[i][0] = x[0]; S[i][1] = x[1]; S[i][2] = x[2]; S[i][3] = x[3];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) S[i][0] = S[i][1] = S[i][2] = S[i][3] = 0.f;
    }

    float* const dvec = vec[wv][0];
    float* const avec = vec[wv][1];
    float* const bvec = vec[wv][2];
    float* const kvec = vec[wv][3];
    float* const rvec = vec[wv][4];

    TokenIn cur{}, nxt{};
    if (L > 0) load_token(p, bos, h, lane, c, cur);
    for (int t = 0; t < L; ++t) {
        dvec[lane] = decay(bf16_to_f32(cur.w));
        avec[lane] = bf16_to_f32(cur.a);
        bvec[lane] = bf16_to_f32(cur.b);
        kvec[lane] = bf16_to_f32(cur.k);
        rvec[lane] = bf16_to_f32(cur.r);
        float vj[4];
        bf16x2_to_f32(cur.v.x, vj[0], vj[1]);
        bf16x2_to_f32(cur.v.y, vj[2], vj[3]);
        if (t + 1 < L) load_token(p, bos + t + 1, h, lane, c, nxt);  // in flight during this token's math
        wave_lds_sync();

        // sa[j] = sum_k a_k S[k][j] over the old state (wkv7.py:75)
        float sa[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            const f4 av = *reinterpret_cast<const f4*>(avec + 16 * g + 4 * i4);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const int i = 4 * i4 + ii;
#pragma unroll
                for (int j = 0; j < 4; ++j) sa[j] = fmaf(av[ii], S[i][j], sa[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) sa[j] = butterfly4(sa[j]);

        // S[k][j] = d_k S[k][j] + b_k sa[j] + k_k v_j;  y[j] = sum_k r_k S[k][j] (updated state, wkv7.py:75-77)
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
            // keeps the scheduler from hoisting all 64 broadcast reads above the FMAs (VGPR budget: 4 waves/SIMD)
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) y[j] = butterfly4(y[j]);

        if (p.o && g == 0) {
            uint2 pk;
            pk.x = pack_bf16x2(y[0], y[1]);
            pk.y = pack_bf16x2(y[2], y[3]);
            uniform_ptr(reinterpret_cast<uint2*>(p.o + (bos + t) * p.o_tok_stride + (int64_t)h * HS))[c] = pk;
        }
        if (p.snap && t < p.T) {
            f4* sp = uniform_ptr(reinterpret_cast<f4*>(p.snap + (((int64_t)n * p.T + t) * p.H + h) * (int64_t)HS2));
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                f4 x;
                x[0] = S[i][0]; x[1] = S[i][1]; x[2] = S[i][2]; x[3] = S[i][3];
                sp[(16 * g + i) * (HS / 4) + c] = x;
            }
        }
        cur = nxt;
        wave_lds_sync();  // this token's LDS reads precede the next token's writes
    }

    if (float* dst = state_dst(p, n, h)) {
        float* s = dst + (16 * g) * HS + 4 * c;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            f4 x;
            x[0] = S[i][0]; x[1] = S[i][1]; x[2] = S[i][2]; x[3] = S[i][3];
            *reinterpret_cast<f4*>(s + i * HS) = x;
        }
    }
}

}  // namespace

hipError_t launch_recurrent(const Params& p, hipStream_t stream) {
    const int64_t pairs = (int64_t)p.num_seqs * p.H;
    if (pairs == 0) return hipSuccess;
    const int64_t blocks = (pairs + kWaves - 1) / kWaves;
    hipLaunchKernelGGL(wkv7_recurrent_kernel, dim3((unsigned)blocks), dim3(64 * kWaves), 0, stream, p);
    return hipGetLastError();
}

}  // namespace wkv7
