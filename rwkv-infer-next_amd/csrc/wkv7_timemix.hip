// wkv7_timemix.hip -- the time-mix work on either side of the WKV7 recurrence, fused: the operand prologue that
// turns the projections into the six WKV operands, and the epilogue that turns the recurrence output into the
// input of the output projection.
//
// Reference (rwkv_next/model.py, Layer.part_att), per token and head of N = 64 channels, all tensors bf16:
//   prologue (model.py:142-152)
//     w  = -softplus(-(b_w + o_w)) - 0.5
//     a  = sigmoid(b_a + o_a)
//     v' = v                                   (first layer: v_first := v)
//        = v + (v_first - v) sigmoid(b_v + o_v)  (other layers)
//     kk = normalize(k * kk_mul) over the head's channels (L2, eps 1e-12)
//     k' = k * (1 + (a - 1) * ka_mul)
//     WKV operands: (r, w, k', v', -kk, kk * a)
//   epilogue (model.py:156-158, up to the output projection)
//     out = (group_norm(y; one group per head, lnx_w, lnx_b, eps) + sum_c(r k' r_k) v') * g
// The reference runs these as about ten elementwise torch kernels, each a full pass over (tokens, channels) in
// HBM; here each is one pass, HBM-bound.  Layout of the work: a lane owns 8 consecutive channels (one 16-byte
// load per operand row), 8 lanes cover a head and a wavefront covers a group of 8 heads of one token.  Each
// wavefront stays on one head group and strides over tokens, so the per-channel parameters are loaded once into
// registers; the per-head sums are 8-lane butterflies.  All arithmetic is fp32 with one bf16 rounding per output
// (the reference rounds after every torch op).
#include <stdint.h>

#include "wkv7.h"
#include "wkv7_device.h"
#include "wkv7_launch.h"

namespace wkv7 {
namespace {

constexpr int kWaves = 4;                 // wavefronts per workgroup
constexpr int kVec = 8;                   // channels per lane
constexpr int kHeadLanes = HS / kVec;     // lanes per head (8)
constexpr int kGroupHeads = 64 / kHeadLanes;  // heads per wavefront (8)

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void load8(const uint16_t* p, float (&x)[kVec]) {
    const u4 u = *reinterpret_cast<const u4*>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) bf16x2_to_f32(u[j], x[2 * j], x[2 * j + 1]);
}

__device__ __forceinline__ void store8(uint16_t* p, const float (&x)[kVec]) {
    u4 u;
#pragma unroll
    for (int j = 0; j < 4; ++j) u[j] = pack_bf16x2(x[2 * j], x[2 * j + 1]);
    *reinterpret_cast<u4*>(p) = u;
}

__device__ __forceinline__ void zero8(float (&x)[kVec]) {
#pragma unroll
    for (int j = 0; j < kVec; ++j) x[j] = 0.f;
}

// Sum over the 8 lanes of one head.
__device__ __forceinline__ float head_sum(float x) {
#pragma unroll
    for (int m = 1; m < kHeadLanes; m <<= 1) x += __shfl_xor(x, m);
    return x;
}

// Transcendentals on the hardware's base-2 exp/log and reciprocal (about 1 ulp of fp32; every output is rounded
// to bf16, 2^-9 relative).
constexpr float kLog2e = 1.44269504088896341f;
constexpr float kLn2 = 0.693147180559945309f;

__device__ __forceinline__ float sigmoid(float x) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * kLog2e));  // exp2 -> inf gives 0
}

// softplus(x) = log(1 + e^x) = max(x, 0) + log(1 + e^-|x|), which neither overflows nor loses the small tail
__device__ __forceinline__ float softplus(float x) {
    return fmaxf(x, 0.f) + kLn2 * __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(-fabsf(x) * kLog2e));
}

// Work split shared by both kernels: wavefront gw owns head group gw % groups and tokens gw / groups, + stride.
struct Lanes {
    int64_t t0, tstride;
    int c;        // first channel of this lane within a token row
    bool active;  // the wavefront has work and the lane's head exists
};

__device__ __forceinline__ Lanes lanes(int H) {
    const int lane = threadIdx.x & 63;
    const int groups = (H + kGroupHeads - 1) / kGroupHeads;
    const int64_t gw = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int64_t per = (int64_t)gridDim.x * kWaves / groups;  // >= 1 by the launch (grid_for)
    Lanes l;
    const int h = (int)(gw % groups) * kGroupHeads + lane / kHeadLanes;
    l.t0 = gw / groups;
    l.tstride = per;
    l.c = h * HS + (lane % kHeadLanes) * kVec;
    l.active = h < H && l.t0 < per;  // waves past per * groups would repeat another wave's tokens
    return l;
}

// Token rows of one lane, raw (8 bf16 per operand).  Two of these alternate in the token loops below, so the
// loads of the next token are in flight while the current one is computed; the row index is clamped to the last
// token so that the look-ahead loads are unconditional and in bounds.
struct ProRows {
    u4 k, v, ow, oa, vf, ov;
};

template <bool MIX>
__device__ __forceinline__ void load_rows(const wkv7_prologue_args& a, int64_t t, int c, ProRows& x) {
    const int64_t ii = (t < a.tokens ? t : a.tokens - 1) * a.in_stride + c;
    x.k = *reinterpret_cast<const u4*>(a.k + ii);
    x.v = *reinterpret_cast<const u4*>(a.v + ii);
    x.ow = *reinterpret_cast<const u4*>(a.o_w + ii);
    x.oa = *reinterpret_cast<const u4*>(a.o_a + ii);
    if constexpr (MIX) {
        x.vf = *reinterpret_cast<const u4*>(a.v_first + ii);
        x.ov = *reinterpret_cast<const u4*>(a.o_v + ii);
    }
}

__device__ __forceinline__ void unpack8(u4 u, float (&x)[kVec]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) bf16x2_to_f32(u[j], x[2 * j], x[2 * j + 1]);
}

struct ProParams {
    float bw[kVec], ba[kVec], bv[kVec], km[kVec], ka[kVec];
};

template <bool MIX>
__device__ __forceinline__ void prologue_token(const wkv7_prologue_args& a, const ProParams& p, const ProRows& x,
                                               int64_t t, int c) {
    float k[kVec], v[kVec], ow[kVec], oa[kVec], vf[kVec], ov[kVec];
    unpack8(x.k, k);
    unpack8(x.v, v);
    unpack8(x.ow, ow);
    unpack8(x.oa, oa);
    if constexpr (MIX) {
        unpack8(x.vf, vf);
        unpack8(x.ov, ov);
    }
    float w[kVec], ag[kVec], kk[kVec], kp[kVec], ss = 0.f;
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
        w[j] = -softplus(-(p.bw[j] + ow[j])) - 0.5f;
        ag[j] = sigmoid(p.ba[j] + oa[j]);
        if constexpr (MIX) v[j] = v[j] + (vf[j] - v[j]) * sigmoid(p.bv[j] + ov[j]);
        kk[j] = k[j] * p.km[j];
        ss += kk[j] * kk[j];
        kp[j] = k[j] * (1.f + (ag[j] - 1.f) * p.ka[j]);
    }
    const float inv = 1.f / fmaxf(sqrtf(head_sum(ss)), 1e-12f);
    float na[kVec], nb[kVec];
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
        const float kn = kk[j] * inv;
        na[j] = -kn;
        nb[j] = kn * ag[j];
    }
    const int64_t oo = t * a.out_stride + c;
    store8(a.w_out + oo, w);
    store8(a.k_out + oo, kp);
    store8(a.v_out + oo, v);
    store8(a.a_out + oo, na);
    store8(a.b_out + oo, nb);
}

template <bool MIX>
__global__ __launch_bounds__(64 * kWaves) void timemix_prologue_kernel(const wkv7_prologue_args a) {
    const Lanes l = lanes(a.H);
    if (!l.active) return;
    ProParams p;
    load8(a.b_w + l.c, p.bw);
    load8(a.b_a + l.c, p.ba);
    load8(a.kk_mul + l.c, p.km);
    load8(a.ka_mul + l.c, p.ka);
    if constexpr (MIX) load8(a.b_v + l.c, p.bv);
    ProRows x0, x1;
    int64_t t = l.t0;
    load_rows<MIX>(a, t, l.c, x0);
    while (t < a.tokens) {
        load_rows<MIX>(a, t + l.tstride, l.c, x1);
        prologue_token<MIX>(a, p, x0, t, l.c);
        t += l.tstride;
        if (t >= a.tokens) break;
        load_rows<MIX>(a, t + l.tstride, l.c, x0);
        prologue_token<MIX>(a, p, x1, t, l.c);
        t += l.tstride;
    }
}

struct EpiRows {
    u4 y, r, k, v, g;
};

__device__ __forceinline__ void load_rows(const wkv7_epilogue_args& a, int64_t t, int c, EpiRows& x) {
    const int64_t ii = (t < a.tokens ? t : a.tokens - 1) * a.in_stride + c;
    x.y = *reinterpret_cast<const u4*>(a.y + ii);
    x.r = *reinterpret_cast<const u4*>(a.r + ii);
    x.k = *reinterpret_cast<const u4*>(a.k + ii);
    x.v = *reinterpret_cast<const u4*>(a.v + ii);
    x.g = *reinterpret_cast<const u4*>(a.g + ii);
}

struct EpiParams {
    float lw[kVec], lb[kVec], rk[kVec];
};

__device__ __forceinline__ void epilogue_token(const wkv7_epilogue_args& a, const EpiParams& p, const EpiRows& x,
                                               int64_t t, int c) {
    float y[kVec], r[kVec], k[kVec], v[kVec], g[kVec];
    unpack8(x.y, y);
    unpack8(x.r, r);
    unpack8(x.k, k);
    unpack8(x.v, v);
    unpack8(x.g, g);
    float s = 0.f, rkk = 0.f;
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
        s += y[j];
        rkk += r[j] * k[j] * p.rk[j];
    }
    const float mean = head_sum(s) * (1.f / HS);
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
        y[j] -= mean;
        q += y[j] * y[j];
    }
    const float rs = rsqrtf(head_sum(q) * (1.f / HS) + a.eps);
    const float bonus = head_sum(rkk);
    float out[kVec];
#pragma unroll
    for (int j = 0; j < kVec; ++j) out[j] = (y[j] * rs * p.lw[j] + p.lb[j] + bonus * v[j]) * g[j];
    store8(a.out + t * a.out_stride + c, out);
}

__global__ __launch_bounds__(64 * kWaves) void timemix_epilogue_kernel(const wkv7_epilogue_args a) {
    const Lanes l = lanes(a.H);
    if (!l.active) return;
    EpiParams p;
    load8(a.lnx_w + l.c, p.lw);
    load8(a.lnx_b + l.c, p.lb);
    load8(a.r_k + l.c, p.rk);  // r_k is [H][64]: the same offset as the channel
    EpiRows x0, x1;
    int64_t t = l.t0;
    load_rows(a, t, l.c, x0);
    while (t < a.tokens) {
        load_rows(a, t + l.tstride, l.c, x1);
        epilogue_token(a, p, x0, t, l.c);
        t += l.tstride;
        if (t >= a.tokens) break;
        load_rows(a, t + l.tstride, l.c, x0);
        epilogue_token(a, p, x1, t, l.c);
        t += l.tstride;
    }
}

// Workgroups for `tokens` tokens of H heads: enough wavefronts in flight to stream HBM (8 workgroups per CU),
// and at least one wavefront per head group.
int grid_for(int64_t tokens, int H) {
    const int cus = device_cu_count();
    const int64_t groups = (H + kGroupHeads - 1) / kGroupHeads;
    const int64_t need = (tokens * groups + kWaves - 1) / kWaves;
    const int64_t cap = (int64_t)cus * 8;
    const int64_t floor = (groups + kWaves - 1) / kWaves;
    int64_t b = need < cap ? need : cap;
    if (b < floor) b = floor;
    return (int)b;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace wkv7

// Head count bound of the time-mix entry points (keeps the launch's head-group floor small).
constexpr int kMaxTimemixHeads = 1 << 16;

extern "C" {

int wkv7_timemix_prologue(const wkv7_prologue_args* a, void* stream) {
    if (!a) return WKV7_ERR_NULL;
    if (a->head_size != wkv7::HS || a->H < 1 || a->tokens < 0) return WKV7_ERR_SHAPE;
    if (a->H > kMaxTimemixHeads) return WKV7_ERR_SHAPE;
    if (a->in_stride < (int64_t)a->H * wkv7::HS || a->out_stride < (int64_t)a->H * wkv7::HS) return WKV7_ERR_SHAPE;
    if (a->tokens == 0) return WKV7_OK;
    const void* req[] = {a->k, a->v, a->o_w, a->o_a, a->b_w, a->b_a, a->kk_mul, a->ka_mul,
                         a->w_out, a->k_out, a->v_out, a->a_out, a->b_out};
    for (const void* q : req)
        if (!q) return WKV7_ERR_NULL;
    if (a->v_first && (!a->o_v || !a->b_v)) return WKV7_ERR_NULL;
    for (const void* q : req)
        if (!wkv7::aligned16(q)) return WKV7_ERR_ALIGN;
    if (a->v_first && (!wkv7::aligned16(a->v_first) || !wkv7::aligned16(a->o_v) || !wkv7::aligned16(a->b_v)))
        return WKV7_ERR_ALIGN;
    if (a->in_stride % 8 || a->out_stride % 8) return WKV7_ERR_ALIGN;
    const dim3 grid(wkv7::grid_for(a->tokens, a->H)), block(64 * wkv7::kWaves);
    if (a->v_first)
        hipLaunchKernelGGL(wkv7::timemix_prologue_kernel<true>, grid, block, 0, static_cast<hipStream_t>(stream), *a);
    else
        hipLaunchKernelGGL(wkv7::timemix_prologue_kernel<false>, grid, block, 0, static_cast<hipStream_t>(stream), *a);
    return static_cast<int>(hipGetLastError());
}

int wkv7_timemix_epilogue(const wkv7_epilogue_args* a, void* stream) {
    if (!a) return WKV7_ERR_NULL;
    if (a->head_size != wkv7::HS || a->H < 1 || a->tokens < 0) return WKV7_ERR_SHAPE;
    if (a->H > kMaxTimemixHeads) return WKV7_ERR_SHAPE;
    if (a->in_stride < (int64_t)a->H * wkv7::HS || a->out_stride < (int64_t)a->H * wkv7::HS) return WKV7_ERR_SHAPE;
    if (!(a->eps > 0.f)) return WKV7_ERR_ARG;
    if (a->tokens == 0) return WKV7_OK;
    const void* req[] = {a->y, a->r, a->k, a->v, a->g, a->lnx_w, a->lnx_b, a->r_k, a->out};
    for (const void* q : req)
        if (!q) return WKV7_ERR_NULL;
    for (const void* q : req)
        if (!wkv7::aligned16(q)) return WKV7_ERR_ALIGN;
    if (a->in_stride % 8 || a->out_stride % 8) return WKV7_ERR_ALIGN;
    hipLaunchKernelGGL(wkv7::timemix_epilogue_kernel, dim3(wkv7::grid_for(a->tokens, a->H)),
                       dim3(64 * wkv7::kWaves), 0, static_cast<hipStream_t>(stream), *a);
    return static_cast<int>(hipGetLastError());
}

}  // extern "C"
