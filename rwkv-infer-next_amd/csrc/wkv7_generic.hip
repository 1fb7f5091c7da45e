// wkv7_generic.hip -- the token-serial WKV7 recurrence for head sizes other than 64 (1 <= K <= 256).
//
// The reference's kernel takes any head size: it pads K to BK = next_power_of_2(K) and masks the padding
// (rwkv_next/kernels/wkv7.py:35-79, 96).  Every RWKV-7 model uses K = 64, which the specialised kernels serve; this
// kernel serves every other size with the same interface and features (dense or ragged rows, pool slots, fresh rows,
// n_keep, per-token snapshots, optional output), so a caller with another head size gets the same results through
// the same entry points.
//
// One wavefront per (sequence, head, block of 16 state columns).  Lane L = 4 c + g holds column 16 cb + c of the
// state and rows k = g + 4 j (j < KP / 4, KP = K rounded up to a power of two, at least 4) in registers; rows and
// columns past K stay zero.  Per token the wavefront stages the k-side vectors (decay, a, b, k, r) in its own LDS slab,
// channel k at slot (k & 3) * KP / 4 + (k >> 2) so that each row group reads its rows contiguously;
// sa = a^T S and y = S^T r are, per column, an fmaf chain over the lane's rows in j order plus a sum over the four
// row groups (two quad DPP steps).  The next token's operands are loaded during the current token's arithmetic.
//   S_t = diag(d_t) S_{t-1} + b_t (a_t^T S_{t-1}) + k_t v_t^T,   d_t = exp(-exp(w_t)),   o_t = S_t^T r_t.
#include <stdint.h>

#include "wkv7.h"
#include "wkv7_device.h"
#include "wkv7_launch.h"
#include "wkv7_token.h"

namespace wkv7 {

namespace {

constexpr int kGCols = 16;   // state columns per wavefront
constexpr int kGWaves = 4;   // wavefronts per workgroup (independent: no workgroup barrier)

// Sum over the four lanes of a quad (the row groups of one column); every lane ends with the same float.
__device__ __forceinline__ float quad_sum(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1 /* quad_perm 1,0,3,2 */, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E /* quad_perm 2,3,0,1 */, 0xf, 0xf, false));
    return x;
}

// State row block of (sequence n, head h) for head size K: K x K floats, or nullptr (see state_src / state_dst).
__device__ __forceinline__ const float* gsrc(const Params& p, int n, int h) {
    if (!p.h0 || (p.fresh && p.fresh[n])) return nullptr;
    const int64_t s = p.h0_idx ? p.h0_idx[n] : n;
    if (s < 0 || s >= p.h0_rows) return nullptr;
    return p.h0 + (s * p.H + h) * (int64_t)p.K * p.K;
}
__device__ __forceinline__ float* gdst(const Params& p, int n, int h) {
    if (!p.ht) return nullptr;
    const int64_t s = p.ht_idx ? p.ht_idx[n] : n;
    if (s < 0 || s >= p.ht_rows) return nullptr;
    return p.ht + (s * p.H + h) * (int64_t)p.K * p.K;
}

// One token's operands for a lane: k-side channels lane + 64 m (m < NCH) and the lane's state column of v.
template <int NCH>
struct GTok {
    float d[NCH], a[NCH], b[NCH], k[NCH], r[NCH];
    float v;
};

template <int NCH>
__device__ __forceinline__ void gload(const Params& p, int64_t tok, int h, int lane, int col, GTok<NCH>& x) {
    const int K = p.K;
    const int64_t off = tok * p.in_tok_stride + (int64_t)h * K;
#pragma unroll
    for (int m = 0; m < NCH; ++m) {
        const int ch = lane + 64 * m;
        const bool in = ch < K;
        x.d[m] = in ? bf16_to_f32(p.w[off + ch]) : 0.f;  // raw w here; the decay is taken when staged
        x.a[m] = in ? bf16_to_f32(p.a[off + ch]) : 0.f;
        x.b[m] = in ? bf16_to_f32(p.b[off + ch]) : 0.f;
        x.k[m] = in ? bf16_to_f32(p.k[off + ch]) : 0.f;
        x.r[m] = in ? bf16_to_f32(p.r[off + ch]) : 0.f;
    }
    x.v = col < K ? bf16_to_f32(p.v[off + col]) : 0.f;
}

template <int RPL>
__global__ __launch_bounds__(64 * kGWaves) void wkv7_generic_kernel(const Params p) {
    constexpr int KP = 4 * RPL;                // padded head size
    constexpr int NCH = (KP + 63) / 64;        // k-side channels staged per lane
    __shared__ float slab_all[kGWaves][5 * KP];  // per wavefront: decay, a, b, k, r
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = lane >> 2, g = lane & 3;
    const int K = p.K, ncb = (K + kGCols - 1) / kGCols;
    const int64_t unit = (int64_t)blockIdx.x * kGWaves + wv;
    if (unit >= (int64_t)p.num_seqs * p.H * ncb) return;  // the whole wavefront: no barrier follows
    const int cb = (int)(unit % ncb);
    const int64_t pair = unit / ncb;
    const int n = (int)(pair / p.H), h = (int)(pair % p.H);
    int64_t bos;
    int L;
    seq_extent(p, n, bos, L);
    const int col = cb * kGCols + c;
    const bool colv = col < K;
    float* const slab = slab_all[wv];
    // padded channels (K .. KP - 1) read zeros for every token: their rows stay zero
#pragma unroll
    for (int m = 0; m < (5 * KP + 63) / 64; ++m) {
        const int x = lane + 64 * m;
        if (x < 5 * KP) slab[x] = 0.f;
    }
    float S[RPL];
    {
        const float* const src = gsrc(p, n, h);
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            const int kr = g + 4 * j;
            S[j] = (src && colv && kr < K) ? src[(int64_t)kr * K + col] : 0.f;
        }
    }
    GTok<NCH> cur, nxt;
    if (L > 0) gload(p, bos, h, lane, col, cur);
    const int64_t KK = (int64_t)K * K;
    for (int t = 0; t < L; ++t) {
        wave_lds_sync();  // the previous token's slab reads precede these writes
#pragma unroll
        for (int m = 0; m < NCH; ++m) {
            const int ch = lane + 64 * m;
            if (ch < K) {
                const int sl = (ch & 3) * RPL + (ch >> 2);
                slab[sl] = decay(cur.d[m]);
                slab[KP + sl] = cur.a[m];
                slab[2 * KP + sl] = cur.b[m];
                slab[3 * KP + sl] = cur.k[m];
                slab[4 * KP + sl] = cur.r[m];
            }
        }
        const float vv = cur.v;
        if (t + 1 < L) gload(p, bos + t + 1, h, lane, col, nxt);  // in flight during this token's arithmetic
        wave_lds_sync();
        const float* const dv = slab + g * RPL;
        // sa = sum_k a_k S[k][col] over the old state (wkv7.py:75)
        float sa = 0.f;
#pragma unroll
        for (int j = 0; j < RPL; ++j) sa = fmaf(dv[KP + j], S[j], sa);
        sa = quad_sum(sa);
        // S[k][col] = d_k S[k][col] + b_k sa + k_k v_col;  y = sum_k r_k S[k][col] (updated state, wkv7.py:75-77)
        float y = 0.f;
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            S[j] = fmaf(dv[j], S[j], fmaf(dv[2 * KP + j], sa, dv[3 * KP + j] * vv));
            y = fmaf(dv[4 * KP + j], S[j], y);
        }
        y = quad_sum(y);
        if (p.o && g == 0 && colv) p.o[(bos + t) * p.o_tok_stride + (int64_t)h * K + col] = f32_to_bf16(y);
        if (p.snap && t < p.T && colv) {
            float* const sp = p.snap + (((int64_t)n * p.T + t) * p.H + h) * KK + col;
#pragma unroll
            for (int j = 0; j < RPL; ++j) {
                const int kr = g + 4 * j;
                if (kr < K) sp[(int64_t)kr * K] = S[j];
            }
        }
        cur = nxt;
    }
    if (float* const dst = gdst(p, n, h)) {
        if (colv) {
#pragma unroll
            for (int j = 0; j < RPL; ++j) {
                const int kr = g + 4 * j;
                if (kr < K) dst[(int64_t)kr * K + col] = S[j];
            }
        }
    }
}

// Head sizes that are multiples of 32, with 16-byte aligned state buffers: the K = 64 decode kernel's layout
// (wkv7_token.h) stretched to K rows.  One wavefront per (sequence, head, block of 32 state columns); lane
// L = 8 g + c holds rows k = g + 8 j (j < K / 8) and columns 32 cb + 4 c .. + 3 as float4s, so every state load or
// store instruction moves 8 rows x 128 contiguous bytes; the k-side vectors are staged in a per-wave LDS slab
// (channel k at slot (k & 7) * K / 8 + (k >> 3)); sa and y are per-lane fmaf chains over the lane's rows plus the
// three-step butterfly over the row groups g.  Operands and outputs keep 2-byte accesses (the generic path's operand
// alignment).
constexpr int kVCols = 32;

// (K = 64 never comes here: the specialised kernels serve it)
inline bool vec_ok(const Params& p) {
    auto al = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    return p.K % kVCols == 0 && p.K != 64 && p.K <= kGenericMaxK && al(p.h0) && al(p.ht) && al(p.snap);
}

template <int RPL>
__global__ __launch_bounds__(64 * kGWaves) void wkv7_generic_vec_kernel(const Params p) {
    constexpr int K = 8 * RPL;
    constexpr int NCH = (K + 63) / 64;  // k-side channels staged per lane
    constexpr int ncb = K / kVCols;
    __shared__ float slab_all[kGWaves][5 * K];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g = lane >> 3, c = lane & 7;
    const int64_t unit = (int64_t)blockIdx.x * kGWaves + wv;
    if (unit >= (int64_t)p.num_seqs * p.H * ncb) return;  // the whole wavefront: no barrier follows
    const int cb = (int)(unit % ncb);
    const int64_t pair = unit / ncb;
    const int n = (int)(pair / p.H), h = (int)(pair % p.H);
    int64_t bos;
    int L;
    seq_extent(p, n, bos, L);
    const int col0 = cb * kVCols + 4 * c;
    float* const slab = slab_all[wv];
    f4 S[RPL];
    {
        const float* const src = gsrc(p, n, h);
#pragma unroll
        for (int j = 0; j < RPL; ++j)
            S[j] = src ? *reinterpret_cast<const f4*>(src + (int64_t)(g + 8 * j) * K + col0) : f4{0.f, 0.f, 0.f, 0.f};
    }
    GTok<NCH> cur{}, nxt{};
    float vc[4] = {0.f, 0.f, 0.f, 0.f}, vn[4] = {0.f, 0.f, 0.f, 0.f};
    auto vload = [&](int64_t tok, float (&v)[4]) {
        const uint16_t* const vp = p.v + tok * p.in_tok_stride + (int64_t)h * K + col0;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = bf16_to_f32(vp[e]);
    };
    if (L > 0) {
        gload(p, bos, h, lane, 0, cur);
        vload(bos, vc);
    }
    const int64_t KK = (int64_t)K * K;
    for (int t = 0; t < L; ++t) {
        wave_lds_sync();  // the previous token's slab reads precede these writes
#pragma unroll
        for (int m = 0; m < NCH; ++m) {
            const int ch = lane + 64 * m;
            if (ch < K) {
                const int sl = (ch & 7) * RPL + (ch >> 3);
                slab[sl] = decay(cur.d[m]);
                slab[K + sl] = cur.a[m];
                slab[2 * K + sl] = cur.b[m];
                slab[3 * K + sl] = cur.k[m];
                slab[4 * K + sl] = cur.r[m];
            }
        }
        if (t + 1 < L) {  // in flight during this token's arithmetic
            gload(p, bos + t + 1, h, lane, 0, nxt);
            vload(bos + t + 1, vn);
        }
        wave_lds_sync();
        const float* const dv = slab + g * RPL;
        // sa = a^T S over the old state, per column (wkv7.py:75)
        float sa[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < RPL; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) sa[e] = fmaf(dv[K + j], S[j][e], sa[e]);
#pragma unroll
        for (int e = 0; e < 4; ++e) sa[e] = butterfly8(sa[e]);
        // S = d S + b sa + k v;  y = r^T S over the updated state (wkv7.py:75-77)
        float y[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            const float d = dv[j], b = dv[2 * K + j], k = dv[3 * K + j], r = dv[4 * K + j];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                S[j][e] = fmaf(d, S[j][e], fmaf(b, sa[e], k * vc[e]));
                y[e] = fmaf(r, S[j][e], y[e]);
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = butterfly8(y[e]);
        if (p.o && g == 0) {
            uint16_t* const op = p.o + (bos + t) * p.o_tok_stride + (int64_t)h * K + col0;
#pragma unroll
            for (int e = 0; e < 4; ++e) op[e] = f32_to_bf16(y[e]);
        }
        if (p.snap && t < p.T) {
            float* const sp = p.snap + (((int64_t)n * p.T + t) * p.H + h) * KK + col0;
#pragma unroll
            for (int j = 0; j < RPL; ++j) *reinterpret_cast<f4*>(sp + (int64_t)(g + 8 * j) * K) = S[j];
        }
        cur = nxt;
#pragma unroll
        for (int e = 0; e < 4; ++e) vc[e] = vn[e];
    }
    if (float* const dst = gdst(p, n, h)) {
#pragma unroll
        for (int j = 0; j < RPL; ++j) *reinterpret_cast<f4*>(dst + (int64_t)(g + 8 * j) * K + col0) = S[j];
    }
}

}  // namespace

int64_t generic_grid(const Params& p) {
    const int cols = vec_ok(p) ? kVCols : kGCols;
    const int64_t units = (int64_t)p.num_seqs * p.H * ((p.K + cols - 1) / cols);
    return (units + kGWaves - 1) / kGWaves;
}

hipError_t launch_generic(const Params& p, hipStream_t stream) {
    const int64_t blocks = generic_grid(p);
    if (blocks == 0) return hipSuccess;
    const dim3 grid((unsigned)blocks), block(64 * kGWaves);
    if (vec_ok(p)) {
        switch (p.K) {
            case 32: hipLaunchKernelGGL(wkv7_generic_vec_kernel<4>, grid, block, 0, stream, p); break;
            case 96: hipLaunchKernelGGL(wkv7_generic_vec_kernel<12>, grid, block, 0, stream, p); break;
            case 128: hipLaunchKernelGGL(wkv7_generic_vec_kernel<16>, grid, block, 0, stream, p); break;
            case 160: hipLaunchKernelGGL(wkv7_generic_vec_kernel<20>, grid, block, 0, stream, p); break;
            case 192: hipLaunchKernelGGL(wkv7_generic_vec_kernel<24>, grid, block, 0, stream, p); break;
            case 224: hipLaunchKernelGGL(wkv7_generic_vec_kernel<28>, grid, block, 0, stream, p); break;
            default: hipLaunchKernelGGL(wkv7_generic_vec_kernel<32>, grid, block, 0, stream, p); break;  // 256
        }
        return hipGetLastError();
    }
    int kp = 4;
    while (kp < p.K) kp *= 2;
    switch (kp) {
        case 4: hipLaunchKernelGGL(wkv7_generic_kernel<1>, grid, block, 0, stream, p); break;
        case 8: hipLaunchKernelGGL(wkv7_generic_kernel<2>, grid, block, 0, stream, p); break;
        case 16: hipLaunchKernelGGL(wkv7_generic_kernel<4>, grid, block, 0, stream, p); break;
        case 32: hipLaunchKernelGGL(wkv7_generic_kernel<8>, grid, block, 0, stream, p); break;
        case 64: hipLaunchKernelGGL(wkv7_generic_kernel<16>, grid, block, 0, stream, p); break;
        case 128: hipLaunchKernelGGL(wkv7_generic_kernel<32>, grid, block, 0, stream, p); break;
        default: hipLaunchKernelGGL(wkv7_generic_kernel<64>, grid, block, 0, stream, p); break;
    }
    return hipGetLastError();
}

}  // namespace wkv7
