// w6a16.hip -- weight-only 6-bit GEMM / GEMV (W6A16) on gfx950, reading the reference's bit-plane format directly.
//
// Format (rwkv_next/kernels/int6_gemm.py:14-38, 73-112): a (K, N) weight, N contiguous, quantised symmetrically to
// q in [-32, 31] per (group of group_k rows, column) with an fp16 scale s, w ~ s q.  Stored as u = q + 32 in [0, 63]
// split over two byte planes per 64-row chunk c:
//     lo[c*32 + j][n] = (u[c*64 + j] & 15) | (u[c*64 + j + 32] & 15) << 4                         j < 32
//     hi[c*16 + j][n] = u[c*64 + j] >> 4 | (u[.. + j + 16] >> 4) << 2 | (u[.. + j + 32] >> 4) << 4
//                       | (u[.. + j + 48] >> 4) << 6                                                 j < 16
// C[b][m][n] = sum_k A[b][m][k] s[k / group_k][n] q[k][n] with fp32 accumulation (int6_gemm.py:156-215).
//
// Narrow kernel (M <= 32, the decode GEMV): a workgroup of four wavefronts covers four adjacent 128-column strips
// (512 columns: neighbouring strips share DRAM pages, which the four wavefronts read at about the same time) for one
// range of 64-row chunks (split-K over chunk ranges) and one 16-row tile of A.  Each wavefront computes a 16 (M) x
// 128 (N) tile:
//   * the chunk's 48 plane rows x 128 columns (6 KB) are loaded coalesced (16 bytes per lane, 8 lanes per row), with
//     the next chunk's loads in flight, and written to the wave's own LDS buffer (no workgroup barrier: a wave's LDS
//     operations execute in order);
//   * ds_read_b64_tr_b8 hands each lane 8 consecutive plane rows of one column -- within each 16-lane group, lane
//     L receives byte L & 7 of the 8-byte reads of lanes (L & 15) / 8 + 2 e, so lane s of group q reading
//     row base + s / 2, columns 8 (s & 1) .. gives lane (i, q) rows base + e of column i -- which is exactly the
//     B operand of v_mfma_f32_16x16x32_bf16 (8 consecutive k of one column).  One read of the lo plane covers both
//     32-row halves of the chunk (low and high nibbles), one read of the hi plane supplies the top 2 bits;
//   * the 6-bit code u becomes a bf16 operand without conversion instructions: 0x4300 | u is the bf16 of 128 + u,
//     exact, assembled for two values with one v_perm_b32 against a register of 0x43 bytes.  One extra MFMA pair
//     per chunk against a constant B of -160 removes the bias (128 + u - 160 = q) exactly;
//   * each chunk's fp32 tile is scaled by s (fp16) and accumulated.
// Split-K partials are reduced inside the kernel: every split stores its tile (fp32) and the workgroup increments its
// tiles' arrival counters after one agent-scope release; the split that arrives last sums the partials in split
// order (a fixed order: the result does not depend on which split arrives last), stores the result and resets the
// counter to zero.  The wide kernel (M > 32) is described where it is defined.
// Rows m >= M and columns n >= N are clamped on load (they only feed outputs that are not stored).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>
#include <utility>

#include "w6a16.h"
#include "wkv7_launch.h"

namespace w6 {
namespace {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i lds_v2i;

constexpr int kTileN = 128;          // columns per wavefront
constexpr int kTiles = kTileN / 16;  // 16x16 MFMA tiles per wavefront and M tile
constexpr int kStrips = 4;           // adjacent 128-column strips per workgroup
constexpr int kPitch = 136;          // LDS row pitch in bytes (128 + 8: the 8 rows of one transposing read differ in bank)
constexpr int kRows = 48;            // plane rows per chunk: 32 lo + 16 hi
constexpr int kScaleOff = kRows * kPitch;    // the chunk's 128 fp16 scales follow the plane rows
constexpr int kBuf = kScaleOff + 2 * kTileN;
constexpr int kCounterAlign = 256;   // bytes: workspace alignment
// The arrival counters occupy a fixed region at the start of the workspace, the partials follow it.  Calls with
// different tile counts can share one workspace: the partials of one call never overlap the counters of another,
// and every call leaves the counters it used at zero.
constexpr size_t kCounterRegion = size_t(1) << 20;

struct Args {
    const uint16_t* a;
    int64_t sa_b, sa_m;
    const uint8_t *lo, *hi;
    int64_t sl_b, sh_b;
    const uint16_t* sc;
    int64_t ss_b;
    void* out;
    int64_t so_b, so_m;
    uint32_t* cnt;  // split_k > 1: arrival counters, one per (batch, M group, column strip); zero between calls
    float* part;    // split_k > 1: partial tiles [tile][split][16 MT rows][128 columns]
    float* rsum;    // wide kernel: row-sum bias per chain of 64 CG k, [batch][chain][mpad]
    int32_t B, M, N, K, group_k, split_k, out_dtype, m_groups, n_strips, chunks_per_split;
    int32_t mpad, chain_k, nchains, chains_per_split;  // wide kernel
    int32_t out_vec;  // large-M kernel: the output takes 8-byte (16-byte for fp32) stores of 4 adjacent columns
};

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

__device__ __forceinline__ f4 mfma(bf8 a, bf8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));

// Activation element types.  The 6-bit code u becomes an exact MFMA operand 2^e + u with no conversion instruction
// (the code byte beside a constant high byte), and one MFMA pair per chunk against the constant -(2^e + 32) takes the
// offset out again: 2^e + u - (2^e + 32) = q exactly.  bf16 (the model's activations): 128 + u, high bytes 0x43,
// offset 160.  fp16 (the reference op casts its codes to a.dtype, rwkv_next/kernels/int6_gemm.py:144-147): 1024 + u,
// high bytes 0x64, offset 1056; the products stay exact in the fp32 accumulators.
struct ActBF16 {
    static constexpr uint32_t kCodeHi = 0x43434343u;
    static constexpr uint32_t kBias = 0xC320C320u;  // (-160, -160)
    static constexpr uint32_t kOnes = 0x3F803F80u;  // (1, 1)
    static constexpr float kOffset = 160.f;
    __device__ static f4 mma(u4 a, u4 b, f4 c) { return mfma(__builtin_bit_cast(bf8, a), __builtin_bit_cast(bf8, b), c); }
    __device__ static float dot2(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a), __builtin_bit_cast(bf2, b), c, false);
    }
};
struct ActF16 {
    static constexpr uint32_t kCodeHi = 0x64646464u;
    static constexpr uint32_t kBias = 0xE420E420u;  // (-1056, -1056)
    static constexpr uint32_t kOnes = 0x3C003C00u;  // (1, 1)
    static constexpr float kOffset = 1056.f;
    __device__ static f4 mma(u4 a, u4 b, f4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
    }
    __device__ static float dot2(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
    }
};

// Orders LDS traffic between the lanes of one wavefront (its LDS instructions execute in issue order).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// 4 codes u (one per byte) -> 4 operand values 2^e + u as two dwords.
template <class A>
__device__ __forceinline__ void codes_to_op(uint32_t u, uint32_t& lo2, uint32_t& hi2) {
    lo2 = __builtin_amdgcn_perm(A::kCodeHi, u, 0x04010400u);  // bytes: u0, hi, u1, hi
    hi2 = __builtin_amdgcn_perm(A::kCodeHi, u, 0x04030402u);  // bytes: u2, hi, u3, hi
}

__device__ __forceinline__ void store8(__bf16* dst, const float (&v)[8]) {
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
        o[e] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v[2 * e]) |
               (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v[2 * e + 1]) << 16;
    *reinterpret_cast<u4*>(dst) = u4{o[0], o[1], o[2], o[3]};
}

__device__ __forceinline__ void store8(_Float16* dst, const float (&v)[8]) {
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
        o[e] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * e]) |
               (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * e + 1]) << 16;
    *reinterpret_cast<u4*>(dst) = u4{o[0], o[1], o[2], o[3]};
}

__device__ __forceinline__ void store8(float* dst, const float (&v)[8]) {
    *reinterpret_cast<f4*>(dst) = f4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f4*>(dst + 4) = f4{v[4], v[5], v[6], v[7]};
}

// Output element o of the call as its out_dtype, in kernels instantiated apart for fp16 outputs (F16) and for bf16 /
// fp32 ones.
template <bool F16>
__device__ __forceinline__ void put_out(const Args& p, int64_t o, float v) {
    if constexpr (F16)
        reinterpret_cast<_Float16*>(p.out)[o] = (_Float16)v;
    else if (p.out_dtype == W6A16_OUT_F32)
        reinterpret_cast<float*>(p.out)[o] = v;
    else
        reinterpret_cast<__bf16*>(p.out)[o] = (__bf16)v;
}

// Device-coherent accesses to the split-K partials: relaxed atomics at agent scope, which the compiler emits as
// plain stores / loads that bypass the caches that are not coherent across the chip (sc1).
__device__ __forceinline__ void coherent_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float2 coherent_load2(const float* p) {
    const uint64_t u = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __builtin_bit_cast(float2, u);
}

// One chunk's operands, held in registers between its load and its use.
template <int MT>
struct Stage {
    u4 plane[6];   // plane rows 8 k + lane / 8 of the chunk (0..31 lo, 32..47 hi), 16 columns each
    u4 a[MT][2];   // A[m0 + 16 mt + i][chunk * 64 + 32 h + 8 q .. + 7]
    uint32_t sc;   // scales of columns n0 + 2 lane, n0 + 2 lane + 1 for the chunk's group
};

// Loads never branch: a column or row outside the matrix is clamped to one inside it.  Output columns depend only
// on their own weight columns and scales, output rows only on their own A rows, so the clamped values land in
// outputs that are never stored.
template <int MT>
__device__ __forceinline__ void load_stage(const Args& p, int b, int m0, int n0, int c, Stage<MT>& s) {
    const int lane = threadIdx.x & 63;
    const int seg = lane & 7, rr = lane >> 3;
    const int n = min(n0 + 16 * seg, p.N - 16);
    const uint8_t* const lo = p.lo + (int64_t)b * p.sl_b + ((int64_t)c * 32 + rr) * p.N + n;
    const uint8_t* const hi = p.hi + (int64_t)b * p.sh_b + ((int64_t)c * 16 + rr) * p.N + n;
#pragma unroll
    for (int k = 0; k < 4; ++k) s.plane[k] = *reinterpret_cast<const u4*>(lo + (int64_t)(8 * k) * p.N);
#pragma unroll
    for (int k = 0; k < 2; ++k) s.plane[4 + k] = *reinterpret_cast<const u4*>(hi + (int64_t)(8 * k) * p.N);
    const int i = lane & 15, q = lane >> 4;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = min(m0 + 16 * mt + i, p.M - 1);
        const uint16_t* const arow = p.a + (int64_t)b * p.sa_b + (int64_t)m * p.sa_m + (int64_t)c * 64 + 8 * q;
        s.a[mt][0] = *reinterpret_cast<const u4*>(arow);
        s.a[mt][1] = *reinterpret_cast<const u4*>(arow + 32);
    }
    const int g = (c * 64) / p.group_k;
    const int col = min(n0 + 2 * lane, p.N - 2);
    s.sc = *reinterpret_cast<const uint32_t*>(p.sc + (int64_t)b * p.ss_b + (int64_t)g * p.N + col);
}

// Contract one chunk into acc: stage it in the wave's LDS buffer, read it back transposed, dequantise, MFMA.
template <class A, int MT>
__device__ __forceinline__ void process_stage(const Stage<MT>& s, uint8_t* buf, f4 (&acc)[MT][kTiles]) {
    const int lane = threadIdx.x & 63, q = lane >> 4, i = lane & 15;
    const int seg = lane & 7, rr = lane >> 3;
    wave_lds_sync();  // the previous chunk's reads of buf are issued before these writes
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        uint8_t* dst = buf + (8 * k + rr) * kPitch + 16 * seg;
        *reinterpret_cast<uint2*>(dst) = uint2{s.plane[k][0], s.plane[k][1]};
        *reinterpret_cast<uint2*>(dst + 8) = uint2{s.plane[k][2], s.plane[k][3]};
    }
    *reinterpret_cast<uint32_t*>(buf + kScaleOff + 4 * lane) = s.sc;
    wave_lds_sync();
    const u4 bias = u4{A::kBias, A::kBias, A::kBias, A::kBias};  // -(2^e + 32)
    f4 corr[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        corr[mt] = A::mma(s.a[mt][0], bias, f4{0.f, 0.f, 0.f, 0.f});
        corr[mt] = A::mma(s.a[mt][1], bias, corr[mt]);
    }
    const int sel = 2 * (q >> 1);  // hi-plane field of rows 8 q .. (first half); the second half's is 4 bits up
    const int r = lane & 15;
    const int off = (r >> 1) * kPitch + 8 * (r & 1);
    // every transposing read of the chunk is issued before the first use (one LDS latency per chunk)
    v2i lo_t[kTiles], hi_t[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        lo_t[t] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(buf + (8 * q) * kPitch + off + 16 * t));
        hi_t[t] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(buf + (32 + 8 * (q & 1)) * kPitch + off + 16 * t));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        const v2i lov = lo_t[t], hiv = hi_t[t];
        const float sv = h2f(*reinterpret_cast<const uint16_t*>(buf + kScaleOff + 2 * (16 * t + i)));
        // lov: lo-plane rows 8 q + e of column i (e = 0..7, one byte each); hiv: hi-plane rows 8 (q & 1) + e
        uint32_t o0[4], o1[4];
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            const uint32_t L = (uint32_t)lov[d], Hs = (uint32_t)hiv[d] >> sel;
            const uint32_t u0 = (L & 0x0F0F0F0Fu) | ((Hs & 0x03030303u) << 4);          // rows 8 q + e
            const uint32_t u1 = ((L >> 4) & 0x0F0F0F0Fu) | (Hs & 0x30303030u);          // rows 32 + 8 q + e
            codes_to_op<A>(u0, o0[2 * d], o0[2 * d + 1]);
            codes_to_op<A>(u1, o1[2 * d], o1[2 * d + 1]);
        }
        const u4 w0 = u4{o0[0], o0[1], o0[2], o0[3]};
        const u4 w1 = u4{o1[0], o1[1], o1[2], o1[3]};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            f4 tc = A::mma(s.a[mt][0], w0, corr[mt]);
            tc = A::mma(s.a[mt][1], w1, tc);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[mt][t][v] += tc[v] * sv;
        }
    }
}

template <int MT, bool F16>
__device__ __forceinline__ void store_tile_as(const Args& p, int b, int m0, int n0, const f4 (&acc)[MT][kTiles]) {
    const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    // lane (i, q) holds C[m0 + 16 mt + 4 q + v][n0 + 16 t + i]
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            const int n = n0 + 16 * t + i;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int m = m0 + 16 * mt + 4 * q + v;
                if (n >= p.N || m >= p.M) continue;
                put_out<F16>(p, (int64_t)b * p.so_b + (int64_t)m * p.so_m + n, acc[mt][t][v]);
            }
        }
}
template <int MT>
__device__ __forceinline__ void store_tile(const Args& p, int b, int m0, int n0, const f4 (&acc)[MT][kTiles]) {
    if (p.out_dtype == W6A16_OUT_F16)
        store_tile_as<MT, true>(p, b, m0, n0, acc);
    else
        store_tile_as<MT, false>(p, b, m0, n0, acc);
}

// Split-K reduction of rows r0 .. r0 + R - 1 (those below `rows`) of a tile whose partials lie at `part`: lane l sums
// columns 2 l, 2 l + 1 split by split in order 0, 1, ... and stores the result.  The loads of R rows x 8 splits are
// issued together (each batch waits about one memory latency); rows past `rows` and splits past split_k re-read
// valid entries whose values are not used.
template <int R, bool F16>
__device__ __forceinline__ void reduce_rows(const Args& p, const float* part, int tile_floats, int r0, int rows,
                                            int b, int m0, int n0) {
    const int lane = threadIdx.x & 63;
    const int n = n0 + 2 * lane;
    const float* src[R];
#pragma unroll
    for (int j = 0; j < R; ++j) src[j] = part + min(r0 + j, rows - 1) * kTileN + 2 * lane;
    float2 s[R];
#pragma unroll
    for (int j = 0; j < R; ++j) s[j] = float2{0.f, 0.f};
    for (int sp = 0; sp < p.split_k; sp += 8) {
        float2 x[R][8];
#pragma unroll
        for (int j = 0; j < R; ++j)
#pragma unroll
            for (int k = 0; k < 8; ++k)
                x[j][k] = coherent_load2(src[j] + (int64_t)min(sp + k, p.split_k - 1) * tile_floats);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (sp + k >= p.split_k) break;
#pragma unroll
            for (int j = 0; j < R; ++j) {
                s[j].x += x[j][k].x;
                s[j].y += x[j][k].y;
            }
        }
    }
    const int64_t ob = (int64_t)b * p.so_b;
#pragma unroll
    for (int j = 0; j < R; ++j) {
        if (r0 + j >= rows || n >= p.N) continue;
        const int64_t o = ob + (int64_t)(m0 + r0 + j) * p.so_m + n;
        put_out<F16>(p, o, s[j].x);
        put_out<F16>(p, o + 1, s[j].y);
    }
}

// Split-K: this split's partial tile of `tile`, row-major [16 MT rows][128 columns] fp32 per (tile, split); rows >= M
// are not written.
template <int MT>
__device__ __forceinline__ void publish_partials(const Args& p, int64_t tile, int split, int m0,
                                                 const f4 (&acc)[MT][kTiles]) {
    const int lane = threadIdx.x & 63, q = lane >> 4;
    constexpr int kTileFloats = 16 * MT * kTileN;
    const int rows = min(16 * MT, p.M - m0);  // valid rows of this tile
    float* const mine = p.part + (tile * p.split_k + split) * kTileFloats + (lane & 15);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < kTiles; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int r = 16 * mt + 4 * q + v;
                if (r < rows) coherent_store(mine + r * kTileN + 16 * t, acc[mt][t][v]);
            }
}

// Split-K, in the split that completed `tile`: sum the partials in split order (a fixed order: the result does not
// depend on which split arrived last), store the result, reset the tile's counter.
template <int MT>
__device__ __forceinline__ void reduce_tile(const Args& p, int64_t tile, int b, int m0, int n0) {
    const int lane = threadIdx.x & 63;
    constexpr int kTileFloats = 16 * MT * kTileN;
    const float* const part = p.part + tile * p.split_k * kTileFloats;
    const int rows = min(16 * MT, p.M - m0);
    const bool f16 = p.out_dtype == W6A16_OUT_F16;
    if (rows == 1) {
        if (f16)
            reduce_rows<1, true>(p, part, kTileFloats, 0, 1, b, m0, n0);
        else
            reduce_rows<1, false>(p, part, kTileFloats, 0, 1, b, m0, n0);
    } else {
        for (int r0 = 0; r0 < rows; r0 += 4)
            if (f16)
                reduce_rows<4, true>(p, part, kTileFloats, r0, rows, b, m0, n0);
            else
                reduce_rows<4, false>(p, part, kTileFloats, r0, rows, b, m0, n0);
    }
    if (lane == 0) __hip_atomic_store(p.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------------------------------
// Packed layout: the same 6 bits per weight and fp16 scales, re-laid out once (w6a16_pack) so that each wavefront's
// 64-row chunk of a 128-column strip is one contiguous 6 KB block already in MFMA operand order.  Block (b, strip,
// chunk) lies at ((b * strips + strip) * chunks + chunk) * 6144; load instruction k (0..5) of lane l reads bytes
// k * 1024 + 16 l .. + 15, i.e. dwords 4 k .. 4 k + 3 of lane l's 24-dword record R.  For lane (i, q) = (l & 15,
// l >> 4) and tile t (column n = 128 strip + 16 t + i):
//   R[2 t], R[2 t + 1]  bytes e = 0..7: lo plane row chunk * 32 + 8 q + e (low nibble: row 8 q + e of the chunk,
//                       high nibble: row 32 + 8 q + e)
//   R[16 + t]           byte e' = 0..3: the top 2 bits of rows 8 q + e', 32 + 8 q + e', 8 q + 4 + e',
//                       32 + 8 q + 4 + e' at bits 0-1, 2-3, 4-5, 6-7
// Scales: block (b, strip, group) of 128 fp16 at ((b * strips + strip) * groups + group) * 128, ordered [i][t], so
// lane (i, q) reads its eight columns' scales as one 16-byte load.  Columns past N hold zero codes and scales.
constexpr int kPackBytes = 6144;

template <int MT>
struct PStage {
    u4 w[6];       // the lane's 24-dword record
    u4 a[MT][2];   // A[m0 + 16 mt + i][chunk * 64 + 32 h + 8 q .. + 7]
    u4 sc;         // scales of columns n0 + 16 t + i, t = 0..7 (fp16)
};

template <int MT>
__device__ __forceinline__ void load_pstage(const Args& p, int b, int m0, int strip, int c, PStage<MT>& s) {
    const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    const int nchunks = p.K / 64;
    const uint8_t* const blk =
        p.lo + (int64_t)b * p.sl_b + ((int64_t)strip * nchunks + c) * kPackBytes + 16 * lane;
#pragma unroll
    for (int k = 0; k < 6; ++k) s.w[k] = *reinterpret_cast<const u4*>(blk + 1024 * k);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = min(m0 + 16 * mt + i, p.M - 1);
        const uint16_t* const arow = p.a + (int64_t)b * p.sa_b + (int64_t)m * p.sa_m + (int64_t)c * 64 + 8 * q;
        s.a[mt][0] = *reinterpret_cast<const u4*>(arow);
        s.a[mt][1] = *reinterpret_cast<const u4*>(arow + 32);
    }
    const int g = (c * 64) / p.group_k, groups = p.K / p.group_k;
    s.sc = *reinterpret_cast<const u4*>(p.sc + (int64_t)b * p.ss_b + ((int64_t)strip * groups + g) * kTileN + 8 * i);
}

template <class A, int MT>
__device__ __forceinline__ void process_pstage(const PStage<MT>& s, f4 (&acc)[MT][kTiles]) {
    const u4 bias = u4{A::kBias, A::kBias, A::kBias, A::kBias};  // -(2^e + 32)
    f4 corr[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        corr[mt] = A::mma(s.a[mt][0], bias, f4{0.f, 0.f, 0.f, 0.f});
        corr[mt] = A::mma(s.a[mt][1], bias, corr[mt]);
    }
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        const uint32_t L0 = s.w[t >> 1][2 * (t & 1)], L1 = s.w[t >> 1][2 * (t & 1) + 1];
        const uint32_t Hd = s.w[4 + (t >> 2)][t & 3];
        const uint32_t u0a = (L0 & 0x0F0F0F0Fu) | ((Hd & 0x03030303u) << 4);         // rows 8 q + 0..3
        const uint32_t u0b = (L1 & 0x0F0F0F0Fu) | (Hd & 0x30303030u);                // rows 8 q + 4..7
        const uint32_t u1a = ((L0 >> 4) & 0x0F0F0F0Fu) | ((Hd & 0x0C0C0C0Cu) << 2);  // rows 32 + 8 q + 0..3
        const uint32_t u1b = ((L1 >> 4) & 0x0F0F0F0Fu) | ((Hd >> 2) & 0x30303030u);  // rows 32 + 8 q + 4..7
        uint32_t o0[4], o1[4];
        codes_to_op<A>(u0a, o0[0], o0[1]);
        codes_to_op<A>(u0b, o0[2], o0[3]);
        codes_to_op<A>(u1a, o1[0], o1[1]);
        codes_to_op<A>(u1b, o1[2], o1[3]);
        const u4 w0 = u4{o0[0], o0[1], o0[2], o0[3]};
        const u4 w1 = u4{o1[0], o1[1], o1[2], o1[3]};
        const float sv = h2f((uint16_t)(s.sc[t >> 1] >> (16 * (t & 1))));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            f4 tc = A::mma(s.a[mt][0], w0, corr[mt]);
            tc = A::mma(s.a[mt][1], w1, tc);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[mt][t][v] += tc[v] * sv;
        }
    }
}

// Narrow kernel (M <= 32), both weight formats: a workgroup of four wavefronts, one per 128-column strip.
template <class A, int MT, int D, bool PACKED>
__global__ __launch_bounds__(64 * kStrips) void w6a16_kernel(const Args p) {
    constexpr int kStage = PACKED ? 16 : kStrips * kBuf;  // planes: each wavefront's staging buffer
    __shared__ __attribute__((aligned(16))) uint8_t lds[kStage];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int sw = wv;
    const int strip = blockIdx.x * kStrips + sw;
    const bool live = strip < p.n_strips;
    const int n0 = strip * kTileN;
    const int split = blockIdx.y;
    const int b = blockIdx.z / p.m_groups, mg = blockIdx.z % p.m_groups;
    const int m0 = mg * 16 * MT;
    const int nchunks = p.K / 64;
    const int c0 = split * p.chunks_per_split, c1 = min(nchunks, c0 + p.chunks_per_split);
    uint8_t* const buf = lds + (PACKED ? 0 : wv * kBuf);

    f4 acc[MT][kTiles];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < kTiles; ++t) acc[mt][t] = f4{0.f, 0.f, 0.f, 0.f};

    if (live && c0 < c1) {
        // D chunks in flight.  Chunks past the range re-load the last one (a cache hit), so every load is
        // unconditional.  Packed: whole groups of D chunks run unconditionally (a use of a stage under a condition
        // let the compiler sink that stage's loads to the use, leaving no load in flight) and a scheduling barrier
        // keeps each stage's loads where they are issued; the remainder (fewer than D chunks, already loaded)
        // follows.
        typedef typename std::conditional<PACKED, PStage<MT>, Stage<MT>>::type S;
        S st[D];
        auto load = [&](int c, S& x) {
            if constexpr (PACKED) load_pstage<MT>(p, b, m0, strip, c, x);
            else load_stage<MT>(p, b, m0, n0, c, x);
        };
        auto work = [&](const S& x) {
            if constexpr (PACKED) process_pstage<A, MT>(x, acc);
            else process_stage<A, MT>(x, buf, acc);
        };
#pragma unroll
        for (int j = 0; j < D; ++j) load(min(c0 + j, c1 - 1), st[j]);
        if constexpr (PACKED) {
            const int full = c0 + (c1 - c0) / D * D;
            for (int c = c0; c < full; c += D) {
#pragma unroll
                for (int j = 0; j < D; ++j) {
                    work(st[j]);
                    load(min(c + j + D, c1 - 1), st[j]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
#pragma unroll
            for (int j = 0; j + 1 < D; ++j)
                if (full + j < c1) work(st[j]);
        } else {
            // the planes' stages are consumed by LDS stores: here the compiler keeps the loads in place on its own
            // (measured 1 us faster per call than the form above)
            for (int c = c0; c < c1; c += D) {
#pragma unroll
                for (int j = 0; j < D; ++j) {
                    if (c + j < c1) work(st[j]);
                    load(min(c + j + D, c1 - 1), st[j]);
                }
            }
        }
    }

    const bool owner = live;  // this wavefront finishes its strip's tile
    if (p.split_k == 1) {  // uniform over the grid
        if (owner) store_tile<MT>(p, b, m0, n0, acc);
        return;
    }
    // Split-K hand-off, one agent-scope release per workgroup.  An agent-scope release fence writes back the XCD's L2
    // (a walk whose cost grows with the number of releases, not with the dirty data): issued by every wavefront it
    // cost 6 us per call at M = 1 and 42 us at M = 128.  Here every wavefront stores its strip's partials and waits
    // for them; the workgroup barrier orders those stores before wavefront 0's release fence, which then counts all
    // of the workgroup's strips in with relaxed atomic increments; if a strip completed, wavefront 0's acquire fence
    // follows, and the second barrier orders it before the reducing wavefronts' reads.
    const int64_t tile0 = ((int64_t)b * p.m_groups + mg) * p.n_strips;
    if (owner) publish_partials<MT>(p, tile0 + strip, split, m0, acc);
    __builtin_amdgcn_s_waitcnt(0);  // this wavefront's partial stores have completed
    __shared__ uint32_t completed[kStrips];
    __syncthreads();
    if (wv == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        bool done = false;
        if (lane < kStrips) {
            const int st = blockIdx.x * kStrips + lane;
            if (st < p.n_strips)
                done = __hip_atomic_fetch_add(p.cnt + tile0 + st, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                       (uint32_t)p.split_k - 1;
            completed[lane] = done ? 1u : 0u;
        }
        if (__builtin_amdgcn_ballot_w64(done)) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    if (owner && completed[sw]) reduce_tile<MT>(p, tile0 + strip, b, m0, n0);
}

// Half a strip of the packed layout (tiles 4 h .. 4 h + 3 of the 128-column strip, one 16-row tile of A): load
// instructions 2 h, 2 h + 1 (the low bits) and 4 + h (the top bits) of the chunk's 6 KB block, scale dwords 2 h and
// 2 h + 1.  Tile t of the half computes exactly what process_pstage computes for tile 4 h + t.
struct PHalf {
    u4 w[3];
    u4 a[2];
    uint2 sc;
};

__device__ __forceinline__ void load_phalf(const Args& p, int b, int m0, int strip, int h, int c, PHalf& s) {
    const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    const int nchunks = p.K / 64;
    const uint8_t* const blk =
        p.lo + (int64_t)b * p.sl_b + ((int64_t)strip * nchunks + c) * kPackBytes + 16 * lane;
    s.w[0] = *reinterpret_cast<const u4*>(blk + 1024 * (2 * h));
    s.w[1] = *reinterpret_cast<const u4*>(blk + 1024 * (2 * h + 1));
    s.w[2] = *reinterpret_cast<const u4*>(blk + 1024 * (4 + h));
    const int m = min(m0 + i, p.M - 1);
    const uint16_t* const arow = p.a + (int64_t)b * p.sa_b + (int64_t)m * p.sa_m + (int64_t)c * 64 + 8 * q;
    s.a[0] = *reinterpret_cast<const u4*>(arow);
    s.a[1] = *reinterpret_cast<const u4*>(arow + 32);
    const int g = (c * 64) / p.group_k, groups = p.K / p.group_k;
    s.sc = *reinterpret_cast<const uint2*>(p.sc + (int64_t)b * p.ss_b + ((int64_t)strip * groups + g) * kTileN + 8 * i +
                                           4 * h);
}

template <class A>
__device__ __forceinline__ void process_phalf(const PHalf& s, f4 (&acc)[1][4]) {
    const u4 bias = u4{A::kBias, A::kBias, A::kBias, A::kBias};  // -(2^e + 32)
    f4 corr = A::mma(s.a[0], bias, f4{0.f, 0.f, 0.f, 0.f});
    corr = A::mma(s.a[1], bias, corr);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t L0 = s.w[t >> 1][2 * (t & 1)], L1 = s.w[t >> 1][2 * (t & 1) + 1];
        const uint32_t Hd = s.w[2][t];
        const uint32_t u0a = (L0 & 0x0F0F0F0Fu) | ((Hd & 0x03030303u) << 4);
        const uint32_t u0b = (L1 & 0x0F0F0F0Fu) | (Hd & 0x30303030u);
        const uint32_t u1a = ((L0 >> 4) & 0x0F0F0F0Fu) | ((Hd & 0x0C0C0C0Cu) << 2);
        const uint32_t u1b = ((L1 >> 4) & 0x0F0F0F0Fu) | ((Hd >> 2) & 0x30303030u);
        uint32_t o0[4], o1[4];
        codes_to_op<A>(u0a, o0[0], o0[1]);
        codes_to_op<A>(u0b, o0[2], o0[3]);
        codes_to_op<A>(u1a, o1[0], o1[1]);
        codes_to_op<A>(u1b, o1[2], o1[3]);
        const u4 w0 = u4{o0[0], o0[1], o0[2], o0[3]};
        const u4 w1 = u4{o1[0], o1[1], o1[2], o1[3]};
        const float sv = h2f((uint16_t)((t >> 1 ? s.sc.y : s.sc.x) >> (16 * (t & 1))));
        f4 tc = A::mma(s.a[0], w0, corr);
        tc = A::mma(s.a[1], w1, tc);
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[0][t][v] += tc[v] * sv;
    }
}

// In-workgroup split-K (M <= 32, 2 <= split_k <= kGemvMaxSplit): the split_k ranges of one 128-column strip run as
// the wavefronts of one workgroup -- wavefront w takes exactly the chunks split w of w6a16_kernel takes -- and their
// partial tiles are summed through LDS in split order 0, 1, ..., the same fp32 sums as w6a16_kernel's hand-off
// (bit-identical results) with no cross-workgroup hand-off, counter or workspace traffic.  One workgroup per strip
// and 16-row M group, or (NT = 4, packed layout) per half strip, which doubles the workgroups where strips are fewer
// than CUs.
constexpr int kGemvMaxSplit = 8;
constexpr int kGemvPart = kGemvMaxSplit * 16 * kTileN * 4;  // fp32 partial tiles [split][16 rows][128 columns]
constexpr int kGemvLds = kGemvMaxSplit * kBuf > kGemvPart ? kGemvMaxSplit * kBuf : kGemvPart;

// The gemv epilogue: output element (r, col) of the tile is the sum of the ks wavefront partials in `part`.
template <int NC, bool F16>
__device__ __forceinline__ void gemv_sum_store(const Args& p, const float* part, int rows, int ks, int b, int m0,
                                               int n0) {
    for (int e = threadIdx.x; e < rows * NC; e += blockDim.x) {
        const int r = e / NC, col = e % NC, n = n0 + col;
        float sum = 0.f;
        for (int w = 0; w < ks; ++w) sum += part[(w * 16 + r) * NC + col];
        if (n >= p.N) continue;
        put_out<F16>(p, (int64_t)b * p.so_b + (int64_t)(m0 + r) * p.so_m + n, sum);
    }
}

template <class A, int D, bool PACKED, int NT>
__global__ __launch_bounds__(64 * kGemvMaxSplit) void w6a16_gemv_kernel(const Args p) {
    static_assert(NT == kTiles || (NT == 4 && PACKED), "half strips: packed layout only");
    constexpr int MT = 1, NC = 16 * NT;  // NC: columns per workgroup
    __shared__ __attribute__((aligned(16))) uint8_t lds[kGemvLds];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int strip = blockIdx.x / (kTiles / NT), h = blockIdx.x % (kTiles / NT);
    const int n0 = strip * kTileN + h * NC;
    const int b = blockIdx.z / p.m_groups, mg = blockIdx.z % p.m_groups;
    const int m0 = mg * 16;
    const int nchunks = p.K / 64;
    const int c0 = wv * p.chunks_per_split, c1 = min(nchunks, c0 + p.chunks_per_split);
    uint8_t* const buf = lds + (PACKED ? 0 : wv * kBuf);

    f4 acc[MT][NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[0][t] = f4{0.f, 0.f, 0.f, 0.f};

    if (c0 < c1) {  // the loop of w6a16_kernel, for this wavefront's range
        typedef typename std::conditional<PACKED, typename std::conditional<NT == 4, PHalf, PStage<MT>>::type,
                                          Stage<MT>>::type S;
        S st[D];
        auto load = [&](int c, S& x) {
            if constexpr (PACKED && NT == 4) load_phalf(p, b, m0, strip, h, c, x);
            else if constexpr (PACKED) load_pstage<MT>(p, b, m0, strip, c, x);
            else load_stage<MT>(p, b, m0, n0, c, x);
        };
        auto work = [&](const S& x) {
            if constexpr (PACKED && NT == 4) process_phalf<A>(x, acc);
            else if constexpr (PACKED) process_pstage<A, MT>(x, acc);
            else process_stage<A, MT>(x, buf, acc);
        };
#pragma unroll
        for (int j = 0; j < D; ++j) load(min(c0 + j, c1 - 1), st[j]);
        if constexpr (PACKED) {
            const int full = c0 + (c1 - c0) / D * D;
            for (int c = c0; c < full; c += D) {
#pragma unroll
                for (int j = 0; j < D; ++j) {
                    work(st[j]);
                    load(min(c + j + D, c1 - 1), st[j]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
#pragma unroll
            for (int j = 0; j + 1 < D; ++j)
                if (full + j < c1) work(st[j]);
        } else {
            for (int c = c0; c < c1; c += D) {
#pragma unroll
                for (int j = 0; j < D; ++j) {
                    if (c + j < c1) work(st[j]);
                    load(min(c + j + D, c1 - 1), st[j]);
                }
            }
        }
    }
    __syncthreads();  // the staging buffers are dead: the partial tiles reuse the LDS
    float* const part = reinterpret_cast<float*>(lds);
    {
        const int i = lane & 15, q = lane >> 4;  // lane (i, q) holds rows 4 q + v of column 16 t + i
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v) part[(wv * 16 + 4 * q + v) * NC + 16 * t + i] = acc[0][t][v];
    }
    __syncthreads();
    const int rows = min(16, p.M - m0), ks = p.split_k;
    if (p.out_dtype == W6A16_OUT_F16)
        gemv_sum_store<NC, true>(p, part, rows, ks, b, m0, n0);
    else
        gemv_sum_store<NC, false>(p, part, rows, ks, b, m0, n0);
}

// ---------------------------------------------------------------------------------------------------------------
// Wide kernel (M > 32).  A workgroup of 4 KP wavefronts covers one 128-column strip for 16 MTW rows of A: wavefront
// w owns column tiles 2 (w & 3) and 2 (w & 3) + 1 for all the workgroup's rows, over K part w >> 2 (the workgroup's
// chunk range cut into KP contiguous parts, summed through LDS at the end).  Each dequantised weight operand serves
// MTW M tiles, each A operand two column tiles.  The M groups of one strip are 8 blocks apart in dispatch order (the
// same XCD, one after the other), so the weight bytes come from HBM once per strip and hit that XCD's L2 for the
// other groups.
//   * A's chunk of every part ([16 MTW rows][64 k] bf16) is staged in LDS, double-buffered, one workgroup barrier
//     per step.  16-byte piece j of row r sits at slot 8 r + (j ^ ((r >> 1) & 7)): the 16 lanes of an MFMA operand
//     read (rows r0 .. r0 + 15, one j) touch all 64 banks once, and so do the writes.
//   * Chains: the products of CG consecutive chunks (CG = 2 when the quantisation group holds two chunks, else 1)
//     accumulate in one MFMA chain whose accumulator starts at the chain's bias -160 sum_k A[m][k] (the row sums of
//     w6a16_rowsum_kernel, computed once per call instead of once per strip), then are scaled once: acc += s * chain.
//     (Measured against row sums taken by the staging threads with per-chunk scaling, which saves that launch: M = 64
//     1 us faster, M = 128 3 us and M = 256 18 us slower per call -- the per-step VALU work decides at four M tiles.)
//   * Packed weights are loaded straight into registers (16 + 8 bytes per lane and chunk: the lane's records of its
//     two tiles), D steps ahead; planes are staged in LDS with A (48 rows x 128 columns) and read back transposed as
//     in the narrow kernel.
// Split-K (when used): one partial tile per (tile, split) in the accumulators' register layout, one release per
// workgroup; the last split adds the others to its own registers in split order.
constexpr int kCachePolicySC1 = 16;  // buffer instructions' cache-policy bit sc1: device-scope write-through
constexpr int kPlaneBytes = kBuf;    // planes: the chunk's 48 plane rows and 128 scales, as in the narrow kernel

template <int MTW>
constexpr int part_a_bytes() { return 16 * MTW * 128; }

// One K part's share of an LDS stage: A slots, the chain's row sums (16 MTW fp32), then (planes) the plane rows.
template <int MTW, bool PACKED>
constexpr int part_bytes() { return part_a_bytes<MTW>() + 16 * MTW * 4 + (PACKED ? 0 : kPlaneBytes); }

__device__ __forceinline__ int a_slot(int r, int j) { return 8 * r + (j ^ ((r >> 1) & 7)); }

using wkv7::unroll;  // f(integral_constant<0>), .., f(integral_constant<N - 1>)

// (1, 1) as an activation pair held in a register (an empty asm keeps the compiler from folding the pair into an
// inline constant, which the packed dot product would read differently).
template <class A>
__device__ __forceinline__ uint32_t ones_x2() {
    uint32_t bits = A::kOnes;
    asm("" : "+v"(bits));
    return bits;
}

template <class A>
__device__ __forceinline__ float sum8(const u4 v, uint32_t one) {
    float x = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        // the element is copied out first: bit-casting a vector element in place (v[d]) compiled to a read of
        // element 0 for every d
        const uint32_t word = v[d];
        x = A::dot2(word, one, x);
    }
    return x;
}

template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {  // x + x of the lane DPP control CTRL selects (all lanes active)
    return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Row sums of A per chain of 64 CG k: rsum[b][chain][m] = -(2^e + 32) sum A[b][m][chain 64 CG .. + 64 CG - 1], zero for
// rows M <= m < mpad.  One wavefront per (row, 512-element segment of K; 8 bf16 per lane, coalesced); the 8 CG lanes
// of a chain add their sums with DPP in a fixed order.
template <class A>
__global__ __launch_bounds__(256) void w6a16_rowsum_kernel(const Args p) {
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6), k = blockIdx.y * 512 + 8 * lane, b = blockIdx.z;
    if (m >= p.mpad) return;  // uniform over the wavefront
    const int lanes_per_chain = 8 * p.chain_k / 64;  // 8 or 16
    const uint16_t* const row = p.a + (int64_t)b * p.sa_b + (int64_t)min(m, p.M - 1) * p.sa_m;
    // K is a multiple of 64 CG: a chain's lanes are all inside K or all past it
    float x = (m < p.M && k < p.K) ? sum8<A>(*reinterpret_cast<const u4*>(row + k), ones_x2<A>()) : 0.f;
    x = dpp_add<0xB1>(x);   // lanes ^ 1
    x = dpp_add<0x4E>(x);   // lanes ^ 2: each lane holds its quad's sum
    x = dpp_add<0x141>(x);  // half-row mirror: lane 7 - l of the 8-lane group, in the other quad
    if (lanes_per_chain == 16) x = dpp_add<0x140>(x);  // row mirror: lane 15 - l, in the other half
    if ((lane & (lanes_per_chain - 1)) == 0 && k < p.K)
        p.rsum[((int64_t)b * p.nchains + k / p.chain_k) * p.mpad + m] = -A::kOffset * x;
}

// The chunk schedule of one workgroup: its split's range of chains, cut into KP contiguous parts.
struct Sched {
    int cg, c_s, per, n_s, nchunks;  // chunks per chain, first chunk of the split, chunks per part, split's chunks
    __device__ __forceinline__ int part_n(int kq) const { return max(0, min(per, n_s - kq * per)); }
    // chunk of part kq at step s, clamped into the part and the matrix (steps past a part's end re-load its last
    // chunk; a part with no chunk loads a valid one)
    __device__ __forceinline__ int chunk(int kq, int s) const {
        return min(c_s + kq * per + max(0, min(s, part_n(kq) - 1)), nchunks - 1);
    }
};

// What one thread loads per step into the LDS stage: MTW / 2 pieces of A, four row sums (threads 0 .. 4 MTW - 1
// of each part's 256) and (planes) 16 bytes of a lo-plane row, 16 bytes of a hi-plane row (threads 0..127 of each
// part's 256) or two scales (threads 128..191).
template <int MTW, bool PACKED>
struct WideLds {
    u4 a[MTW / 2];
    u4 rs;
    u4 pl[2];
    uint32_t sc;
};

// The packed weights of one chunk in one lane's registers: R[4 cp .. 4 cp + 3] (lo plane bytes of tiles 2 cp and
// 2 cp + 1), R[16 + 2 cp], R[17 + 2 cp] (their top bits) and the two tiles' scales of column i.
struct WideW {
    u4 lo;
    uint2 hd;
    uint32_t sc;
};

// Buffer resources and per-lane offsets of the wide kernel's loads, fixed for the whole call: inside the loop only
// the chunk-dependent part changes, and it is the same for a whole wavefront (its K part's chunk), so it goes into the
// instructions' scalar offset and the loop's address arithmetic runs on the scalar unit.
// A raw buffer over [base, base + bytes) (capped at 2 GB; the validation keeps every range the kernel addresses below
// it).  The base and size are passed through readfirstlane so that the descriptor is provably wave-uniform: a
// descriptor the compiler cannot prove uniform is used through a per-lane loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(uint64_t base, int64_t bytes) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
    const int n = __builtin_amdgcn_readfirstlane(bytes < 0x7FFFFFFF ? (int)bytes : 0x7FFFFFFF);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0, n,
                                             0x00020000 /* raw 32-bit buffer, gfx9 family */);
}

// A wave-uniform scalar offset (held in an SGPR, as buffer instructions need it).
__device__ __forceinline__ int soff(int x) { return __builtin_amdgcn_readfirstlane(x); }

template <int MTW>
struct WideSrc {
    uint64_t a, rs, lo, hi, sc;                 // buffer bases (wave-uniform)
    int64_t na, nrs, nlo, nhi, nsc;             // and sizes in bytes
    uint32_t va[MTW / 2], vrs, vlo, vhi, vsc;  // per-lane byte offsets
    int kq[MTW / 2], kq_t, kp;                 // wave-uniform K parts: of each A piece, of the row-sum / plane loads,
                                               // of this wavefront
};

template <int MTW, int KP, bool PACKED>
__device__ __forceinline__ void wide_src(const Args& p, int b, int m0, int strip, WideSrc<MTW>& x) {
    const int tid = threadIdx.x, lane = tid & 63, t = tid & 255, i = lane & 15, cp = (tid >> 6) & 3;
    const int n0 = strip * kTileN;
    x.a = reinterpret_cast<uint64_t>(p.a + (int64_t)b * p.sa_b);
    x.na = ((int64_t)(p.M - 1) * p.sa_m + p.K) * 2;
#pragma unroll
    for (int e = 0; e < MTW / 2; ++e) {
        const int piece = tid + 256 * KP * e, w = piece % (128 * MTW);
        x.kq[e] = __builtin_amdgcn_readfirstlane(piece / (128 * MTW));  // one K part per wavefront and e
        const int m = min(m0 + (w >> 3), p.M - 1);
        x.va[e] = (uint32_t)(((int64_t)m * p.sa_m + 8 * (w & 7)) * 2);
    }
    x.kq_t = __builtin_amdgcn_readfirstlane(tid >> 8);
    x.kp = __builtin_amdgcn_readfirstlane(tid >> 8);
    x.rs = reinterpret_cast<uint64_t>(p.rsum + (int64_t)b * p.nchains * p.mpad);
    x.nrs = (int64_t)p.nchains * p.mpad * 4;
    x.vrs = (m0 + 4 * min(t, 4 * MTW - 1)) * 4;
    if constexpr (PACKED) {
        const int nchunks = p.K / 64, groups = p.K / p.group_k;
        x.lo = reinterpret_cast<uint64_t>(p.lo + (int64_t)b * p.sl_b + (int64_t)strip * nchunks * kPackBytes);
        x.nlo = (int64_t)nchunks * kPackBytes;
        x.vlo = 16 * lane + 1024 * cp;
        x.vhi = 4096 + 1024 * (cp >> 1) + 8 * (cp & 1) + 16 * lane;
        x.sc = reinterpret_cast<uint64_t>(p.sc + (int64_t)b * p.ss_b + (int64_t)strip * groups * kTileN);
        x.nsc = (int64_t)groups * kTileN * 2;
        x.vsc = (8 * i + 2 * cp) * 2;
    } else {
        const int row = t >> 3, n = min(n0 + 16 * (t & 7), p.N - 16);  // lo row 0..31; hi row (row & 15)
        x.lo = reinterpret_cast<uint64_t>(p.lo + (int64_t)b * p.sl_b);
        x.nlo = (int64_t)(p.K / 2) * p.N;
        x.vlo = row * p.N + n;
        x.hi = reinterpret_cast<uint64_t>(p.hi + (int64_t)b * p.sh_b);
        x.nhi = (int64_t)(p.K / 4) * p.N;
        x.vhi = (row & 15) * p.N + n;
        x.sc = reinterpret_cast<uint64_t>(p.sc + (int64_t)b * p.ss_b);
        x.nsc = (int64_t)(p.K / p.group_k) * p.N * 2;
        x.vsc = min(n0 + 2 * (t & 63), p.N - 2) * 2;
    }
}

template <int MTW, int KP, bool PACKED>
__device__ __forceinline__ void wide_load_lds(const Args& p, const Sched& S, const WideSrc<MTW>& src, int s,
                                              WideLds<MTW, PACKED>& x) {
#pragma unroll
    for (int e = 0; e < MTW / 2; ++e)
        x.a[e] = __builtin_amdgcn_raw_buffer_load_b128(rsrc(src.a, src.na), src.va[e], soff(S.chunk(src.kq[e], s) * 128), 0);
    const int c = soff(S.chunk(src.kq_t, s));
    x.rs = __builtin_amdgcn_raw_buffer_load_b128(rsrc(src.rs, src.nrs), src.vrs, soff((c / S.cg) * p.mpad * 4), 0);
    if constexpr (!PACKED) {
        x.pl[0] = __builtin_amdgcn_raw_buffer_load_b128(rsrc(src.lo, src.nlo), src.vlo, soff(c * 32 * p.N), 0);
        x.pl[1] = __builtin_amdgcn_raw_buffer_load_b128(rsrc(src.hi, src.nhi), src.vhi, soff(c * 16 * p.N), 0);
        x.sc = __builtin_amdgcn_raw_buffer_load_b32(rsrc(src.sc, src.nsc), src.vsc, soff((c * 64 / p.group_k) * p.N * 2), 0);
    }
}

template <int MTW, int KP, bool PACKED>
__device__ __forceinline__ void wide_store_lds(const WideLds<MTW, PACKED>& x, uint8_t* st) {
    constexpr int PB = part_bytes<MTW, PACKED>();
    const int tid = threadIdx.x;
#pragma unroll
    for (int e = 0; e < MTW / 2; ++e) {
        const int piece = tid + 256 * KP * e, kq = piece / (128 * MTW), w = piece % (128 * MTW);
        *reinterpret_cast<u4*>(st + kq * PB + 16 * a_slot(w >> 3, w & 7)) = x.a[e];
    }
    const int kq = tid >> 8, t = tid & 255;
    uint8_t* const ps = st + kq * PB;
    if (t < 4 * MTW) *reinterpret_cast<u4*>(ps + part_a_bytes<MTW>() + 16 * t) = x.rs;
    if constexpr (!PACKED) {
        uint8_t* const pl = ps + part_a_bytes<MTW>() + 16 * MTW * 4;
        uint8_t* dst = pl + (t >> 3) * kPitch + 16 * (t & 7);
        *reinterpret_cast<uint2*>(dst) = uint2{x.pl[0][0], x.pl[0][1]};
        *reinterpret_cast<uint2*>(dst + 8) = uint2{x.pl[0][2], x.pl[0][3]};
        if (t < 128) {
            dst += 32 * kPitch;
            *reinterpret_cast<uint2*>(dst) = uint2{x.pl[1][0], x.pl[1][1]};
            *reinterpret_cast<uint2*>(dst + 8) = uint2{x.pl[1][2], x.pl[1][3]};
        } else if (t < 192) {
            *reinterpret_cast<uint32_t*>(pl + kScaleOff + 4 * (t & 63)) = x.sc;
        }
    }
}

template <int MTW>
__device__ __forceinline__ void wide_load_w(const Args& p, const WideSrc<MTW>& src, int c, WideW& w) {
    const __amdgpu_buffer_rsrc_t lo = rsrc(src.lo, src.nlo);
    const int off = soff(c * kPackBytes);
    w.lo = __builtin_amdgcn_raw_buffer_load_b128(lo, src.vlo, off, 0);
    w.hd = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(lo, src.vhi, off, 0));
    w.sc = __builtin_amdgcn_raw_buffer_load_b32(rsrc(src.sc, src.nsc), src.vsc, soff((c * 64 / p.group_k) * kTileN * 2), 0);
}

// x s + a per element, written as a whole vector (stores into the components of an accumulator passed by reference
// kept the accumulators in scratch memory)
__device__ __forceinline__ f4 fma4(const f4 x, float s, const f4 a) {
    return f4{fmaf(x[0], s, a[0]), fmaf(x[1], s, a[1]), fmaf(x[2], s, a[2]), fmaf(x[3], s, a[3])};
}

// Dequantise the wavefront's two column tiles of one chunk into B operands w0 (rows 0..31 of the chunk) and w1
// (rows 32..63), and their scales.
template <class A, int MTW, bool PACKED>
__device__ __forceinline__ void wide_dequant(const uint8_t* ps, const WideW& w, u4 (&w0)[2], u4 (&w1)[2],
                                             float (&sv)[2]) {
    const int lane = threadIdx.x & 63, cp = (threadIdx.x >> 6) & 3;
    const int i = lane & 15, q = lane >> 4;
    if constexpr (PACKED) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const uint32_t L0 = w.lo[2 * tt], L1 = w.lo[2 * tt + 1], Hd = tt ? w.hd.y : w.hd.x;
            const uint32_t u0a = (L0 & 0x0F0F0F0Fu) | ((Hd & 0x03030303u) << 4);         // rows 8 q + 0..3
            const uint32_t u0b = (L1 & 0x0F0F0F0Fu) | (Hd & 0x30303030u);                // rows 8 q + 4..7
            const uint32_t u1a = ((L0 >> 4) & 0x0F0F0F0Fu) | ((Hd & 0x0C0C0C0Cu) << 2);  // rows 32 + 8 q + 0..3
            const uint32_t u1b = ((L1 >> 4) & 0x0F0F0F0Fu) | ((Hd >> 2) & 0x30303030u);  // rows 32 + 8 q + 4..7
            uint32_t o0[4], o1[4];
            codes_to_op<A>(u0a, o0[0], o0[1]);
            codes_to_op<A>(u0b, o0[2], o0[3]);
            codes_to_op<A>(u1a, o1[0], o1[1]);
            codes_to_op<A>(u1b, o1[2], o1[3]);
            w0[tt] = u4{o0[0], o0[1], o0[2], o0[3]};
            w1[tt] = u4{o1[0], o1[1], o1[2], o1[3]};
            sv[tt] = h2f((uint16_t)(w.sc >> (16 * tt)));
        }
    } else {
        const uint8_t* const pl = ps + part_a_bytes<MTW>() + 16 * MTW * 4;
        const int sel = 2 * (q >> 1), r = lane & 15;
        const int off = (r >> 1) * kPitch + 8 * (r & 1);
        v2i lo_t[2], hi_t[2];
        uint16_t sh[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int t = 2 * cp + tt;
            lo_t[tt] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(pl + (8 * q) * kPitch + off + 16 * t));
            hi_t[tt] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(pl + (32 + 8 * (q & 1)) * kPitch + off + 16 * t));
            sh[tt] = *reinterpret_cast<const uint16_t*>(pl + kScaleOff + 2 * (16 * t + i));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            uint32_t o0[4], o1[4];
#pragma unroll
            for (int d = 0; d < 2; ++d) {
                const uint32_t L = (uint32_t)lo_t[tt][d], Hs = (uint32_t)hi_t[tt][d] >> sel;
                const uint32_t u0 = (L & 0x0F0F0F0Fu) | ((Hs & 0x03030303u) << 4);   // rows 8 q + e
                const uint32_t u1 = ((L >> 4) & 0x0F0F0F0Fu) | (Hs & 0x30303030u);   // rows 32 + 8 q + e
                codes_to_op<A>(u0, o0[2 * d], o0[2 * d + 1]);
                codes_to_op<A>(u1, o1[2 * d], o1[2 * d + 1]);
            }
            w0[tt] = u4{o0[0], o0[1], o0[2], o0[3]};
            w1[tt] = u4{o1[0], o1[1], o1[2], o1[3]};
            sv[tt] = h2f(sh[tt]);
        }
    }
}

// One chunk of the wavefront's part: two MFMAs per (M tile, column tile) into the chain accumulators tc; FIRST starts
// the chain at the row sums' bias, LAST scales it into acc.  The LDS reads are issued in batches of up to four M tiles
// ahead of the work that hides them (the first batch ahead of the dequantisation, each further batch ahead of the
// previous batch's MFMAs), with scheduling barriers keeping that order: left to itself the compiler reused a few
// operand registers and waited on the LDS once per M tile.
template <class A, int MTW, bool PACKED, bool FIRST, bool LAST>
__device__ __forceinline__ void wide_compute(const uint8_t* ps, const WideW& w, f4 (&tc)[MTW][2], f4 (&acc)[MTW][2]) {
    constexpr int MB = MTW < 4 ? MTW : 4;  // M tiles per batch of LDS reads
    const int lane = threadIdx.x & 63;
    const int i = lane & 15, q = lane >> 4;
    const float* const rsum = reinterpret_cast<const float*>(ps + part_a_bytes<MTW>());
    u4 a0[MB], a1[MB], w0[2], w1[2];
    f4 nc[MB];
    float sv[2];
    auto read = [&](int mb) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < MB; ++k) {
            const int mt = mb + k;
            a0[k] = *reinterpret_cast<const u4*>(ps + 16 * a_slot(16 * mt + i, q));
            a1[k] = *reinterpret_cast<const u4*>(ps + 16 * a_slot(16 * mt + i, 4 + q));
            if constexpr (FIRST) nc[k] = *reinterpret_cast<const f4*>(rsum + 16 * mt + 4 * q);  // rows 16 mt + 4 q + v
        }
    };
    read(0);
    wide_dequant<A, MTW, PACKED>(ps, w, w0, w1, sv);
#pragma unroll
    for (int mb = 0; mb < MTW; mb += MB) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < MB; ++k)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const f4 c = A::mma(a0[k], w0[tt], FIRST ? nc[k] : tc[mb + k][tt]);
                tc[mb + k][tt] = A::mma(a1[k], w1[tt], c);
            }
        if (mb + MB < MTW) read(mb + MB);
    }
    if constexpr (LAST) {
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) acc[mt][tt] = fma4(tc[mt][tt], sv[tt], acc[mt][tt]);
    }
}

// lane (i, q) of wavefront cp holds C[m0 + 16 mt + 4 q + v][n0 + 16 (2 cp + tt) + i]
template <int MTW, bool F16>
__device__ __forceinline__ void wide_store_as(const Args& p, int b, int m0, int n0, const f4 (&acc)[MTW][2]) {
    const int lane = threadIdx.x & 63, cp = (threadIdx.x >> 6) & 3;
    const int i = lane & 15, q = lane >> 4;
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int n = n0 + 16 * (2 * cp + tt) + i;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int m = m0 + 16 * mt + 4 * q + v;
                if (n >= p.N || m >= p.M) continue;
                put_out<F16>(p, (int64_t)b * p.so_b + (int64_t)m * p.so_m + n, acc[mt][tt][v]);
            }
        }
}
template <int MTW>
__device__ __forceinline__ void wide_store(const Args& p, int b, int m0, int n0, const f4 (&acc)[MTW][2]) {
    if (p.out_dtype == W6A16_OUT_F16)
        wide_store_as<MTW, true>(p, b, m0, n0, acc);
    else
        wide_store_as<MTW, false>(p, b, m0, n0, acc);
}

template <class A, int MTW, int KP, int CG, int D, int NL, bool PACKED>
__global__ __launch_bounds__(256 * KP) void w6a16_wide_kernel(const Args p) {
    constexpr int PB = part_bytes<MTW, PACKED>(), kStage = KP * PB;
    constexpr int kRed = (KP - 1) * 4 * MTW * 2 * 64 * 16;  // K-part partials in LDS
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kStage > kRed ? 2 * kStage : kRed];
    __shared__ uint32_t completed;
    static_assert(D % CG == 0 && D % 2 == 0 && D % NL == 0, "a group of D steps holds whole chains, buffer pairs and rings");
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, kp = wv >> 2;
    // XCD-aware order: the M groups of one strip are 8 blocks apart (same XCD, consecutive in its dispatch order)
    const int bx = blockIdx.x, rest = bx >> 3;
    const int mg = rest % p.m_groups, strip = (rest / p.m_groups) * 8 + (bx & 7);
    if (strip >= p.n_strips) return;  // uniform over the workgroup
    const int n0 = strip * kTileN;
    const int split = blockIdx.y, b = blockIdx.z;
    const int m0 = mg * 16 * MTW;
    Sched S;
    S.cg = CG;
    S.nchunks = p.K / 64;
    {
        const int nch = p.K / (64 * CG);  // chains
        const int h0 = split * p.chains_per_split, h1 = min(nch, h0 + p.chains_per_split);
        const int nh = max(0, h1 - h0);
        S.c_s = h0 * CG;
        S.n_s = nh * CG;
        S.per = (nh + KP - 1) / KP * CG;
    }
    const int steps = S.per;        // uniform over the workgroup
    WideSrc<MTW> src;
    wide_src<MTW, KP, PACKED>(p, b, m0, strip, src);
    const int mine_n = S.part_n(src.kp);  // this wavefront's chunks (uniform over the wavefront)

    f4 acc[MTW][2], tc[MTW][2];
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt) acc[mt][0] = acc[mt][1] = f4{0.f, 0.f, 0.f, 0.f};

    if (steps > 0) {
        // The LDS stage of step s is written in step s - 1 (after its reads of the other buffer have passed that
        // step's barrier) from a ring of NL register stages loaded NL - 1 steps earlier; packed weights are loaded D
        // steps ahead of their use.  Loads past a part's range re-load its last chunk (a cache hit), so every load is
        // unconditional; whole groups of D steps run unconditionally with a scheduling barrier after each step's
        // loads, and the remainder (fewer than D steps, already loaded, whole chains) follows.
        WideLds<MTW, PACKED> ls[NL];
        WideW ws[D];
#pragma unroll
        for (int j = 0; j < NL; ++j) wide_load_lds<MTW, KP, PACKED>(p, S, src, j, ls[j]);
        if constexpr (PACKED) {
#pragma unroll
            for (int j = 0; j < D; ++j) wide_load_w(p, src, S.chunk(src.kp, j), ws[j]);
        }
        wide_store_lds<MTW, KP, PACKED>(ls[0], lds);
        wide_load_lds<MTW, KP, PACKED>(p, S, src, NL, ls[0]);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        // step s = base + j (base a multiple of D, so s = j modulo 2 and NL): compute from buffer j & 1, write step
        // s + 1 into buffer (j + 1) & 1 from ls[(j + 1) % NL], refill that register stage with step s + 1 + NL, and
        // (packed) ws[j] with step s + D.  Every register index is a compile-time constant (a run-time one put the
        // stages in scratch memory).
        auto step = [&](int base, auto J) __attribute__((always_inline)) {
            constexpr int j = decltype(J)::value;
            const int s = base + j;
            const uint8_t* const ps = lds + (j & 1) * kStage + kp * PB;
            if (s < mine_n) wide_compute<A, MTW, PACKED, j % CG == 0, j % CG == CG - 1>(ps, ws[j], tc, acc);
            if constexpr (PACKED) wide_load_w(p, src, S.chunk(src.kp, s + D), ws[j]);
            wide_store_lds<MTW, KP, PACKED>(ls[(j + 1) % NL], lds + ((j + 1) & 1) * kStage);
            wide_load_lds<MTW, KP, PACKED>(p, S, src, s + 1 + NL, ls[(j + 1) % NL]);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
        };
        const int full = steps / D * D;
        for (int base = 0; base < full; base += D) unroll<D>([&](auto J) __attribute__((always_inline)) { step(base, J); });
        unroll<D - 1>([&](auto J) __attribute__((always_inline)) {
            if (full + decltype(J)::value < steps) step(full, J);
        });
    }

    if constexpr (KP > 1) {  // sum the K parts through LDS in part order 0, 1, ..
        f4* const red = reinterpret_cast<f4*>(lds) + (wv & 3) * MTW * 2 * 64 + lane;
        constexpr int kPartF4 = 4 * MTW * 2 * 64;
        __syncthreads();  // the last step's LDS reads are done
        if (kp > 0) {
#pragma unroll
            for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) red[(kp - 1) * kPartF4 + (mt * 2 + tt) * 64] = acc[mt][tt];
        }
        __syncthreads();
        if (kp == 0) {
#pragma unroll
            for (int k = 1; k < KP; ++k)
#pragma unroll
                for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) acc[mt][tt] += red[(k - 1) * kPartF4 + (mt * 2 + tt) * 64];
        }
    }

    if (p.split_k == 1) {  // uniform over the grid
        if (kp == 0) wide_store<MTW>(p, b, m0, n0, acc);
        return;
    }
    // Split-K hand-off, one release per workgroup.  Partials are kept in the accumulators' own layout
    // ([wavefront][mt][tt][lane] f4, 16 bytes per lane and store) and written through the L2 (sc1 stores: written
    // back, the release fence's L2 walk has nothing of theirs left to write; with plain stores it cost 10 us per call
    // at M = 128); the release fence orders them before the arrival count, and the last split's acquire fence orders
    // its loads after it.  The last split keeps its own tile in registers and adds the others' in split order 0, 1, ..
    // (a fixed order: the result does not depend on which split arrives last).
    const int64_t tile = ((int64_t)b * p.m_groups + mg) * p.n_strips + strip;
    constexpr int kTileF4 = 4 * MTW * 2 * 64;  // f4 per partial tile
    f4* const tbase = reinterpret_cast<f4*>(p.part) + tile * p.split_k * kTileF4;
    const int cp = wv & 3;
    if (kp == 0) {
        const __amdgpu_buffer_rsrc_t prs =
            __builtin_amdgcn_make_buffer_rsrc(tbase, 0, p.split_k * kTileF4 * 16, 0x00020000);
        const int mine = split * kTileF4 + cp * MTW * 2 * 64 + lane;
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, acc[mt][tt]), prs,
                                                       (mine + (mt * 2 + tt) * 64) * 16, 0, kCachePolicySC1);
    }
    // Each wavefront waits for its own stores (wavefront 0's release fence waits only for wavefront 0's), then the
    // barrier puts all of them before that fence.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (wv == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        bool done = false;
        if (lane == 0) {
            done = __hip_atomic_fetch_add(p.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   (uint32_t)p.split_k - 1;
            completed = done ? 1u : 0u;
        }
        if (__builtin_amdgcn_ballot_w64(done)) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            if (lane == 0) __hip_atomic_store(p.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __syncthreads();  // wavefront 0's acquire precedes every wavefront's loads
    if (!completed || kp != 0) return;
    const f4* const part = tbase + cp * MTW * 2 * 64 + lane;
    f4 tot[MTW][2];
    for (int sp = 0; sp < p.split_k; ++sp) {
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const f4 x = sp == split ? acc[mt][tt] : part[sp * kTileF4 + (mt * 2 + tt) * 64];
                tot[mt][tt] = sp == 0 ? x : tot[mt][tt] + x;
            }
    }
    wide_store<MTW>(p, b, m0, n0, tot);
}

// Dequantise the packed layout: one thread per (b, strip, chunk, lane) writes its 16 rows x 8 columns (rows
// 8 q + e and 32 + 8 q + e, columns 128 strip + 16 t + i); for each (row, tile) the 16 lanes of a row group store
// 16 consecutive columns.
template <typename OutT>
__global__ __launch_bounds__(256) void w6a16_dequant_packed_kernel(const uint8_t* pk, const uint16_t* psc, OutT* w,
                                                                   int32_t K, int32_t N, int32_t group_k,
                                                                   int32_t strips, int64_t sw_b) {
    const int nchunks = K / 64, groups = K / group_k;
    const int64_t x = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int b = blockIdx.y;
    if (x >= (int64_t)strips * nchunks * 64) return;
    const int lane = (int)(x & 63);
    const int64_t sc = x >> 6;
    const int c = (int)(sc % nchunks), strip = (int)(sc / nchunks);
    const int i = lane & 15, q = lane >> 4;
    const uint8_t* const blk = pk + ((int64_t)b * strips * nchunks + sc) * kPackBytes + 16 * lane;
    uint32_t R[24];
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        const u4 v = *reinterpret_cast<const u4*>(blk + 1024 * k);
        R[4 * k] = v[0];
        R[4 * k + 1] = v[1];
        R[4 * k + 2] = v[2];
        R[4 * k + 3] = v[3];
    }
    const int g = (c * 64) / group_k;
    const u4 sv = *reinterpret_cast<const u4*>(psc + ((int64_t)b * strips * groups + (int64_t)strip * groups + g) * kTileN + 8 * i);
    OutT* const wb = w + b * sw_b;
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        const int n = strip * kTileN + 16 * t + i;
        if (n >= N) continue;
        const float s = h2f((uint16_t)(sv[t >> 1] >> (16 * (t & 1))));
        const uint32_t Lw[2] = {R[2 * t], R[2 * t + 1]}, Hd = R[16 + t];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t lb = (Lw[e >> 2] >> (8 * (e & 3))) & 0xFF;
            const uint32_t hb = (Hd >> (8 * (e & 3) + 4 * (e >> 2))) & 0xF;  // bits 0-1: row 8 q + e, 2-3: row 32 + ..
            const int q0 = (int)((lb & 15) | ((hb & 3) << 4)) - 32;
            const int q1 = (int)((lb >> 4) | ((hb >> 2) << 4)) - 32;
            const int64_t r0 = (int64_t)c * 64 + 8 * q + e;
            wb[r0 * N + n] = (OutT)(s * (float)q0);
            wb[(r0 + 32) * N + n] = (OutT)(s * (float)q1);
        }
    }
}

// Repack: one thread per (b, strip, chunk, lane) writes the lane's 24-dword record.
__global__ __launch_bounds__(256) void w6a16_pack_kernel(const uint8_t* lo, const uint8_t* hi, uint8_t* out, int32_t K,
                                                         int32_t N, int32_t strips, int64_t sl_b, int64_t sh_b) {
    const int nchunks = K / 64;
    const int64_t x = (int64_t)blockIdx.x * 256 + threadIdx.x;  // ((strip * nchunks + c) * 64 + lane) within batch
    const int b = blockIdx.y;
    if (x >= (int64_t)strips * nchunks * 64) return;
    const int lane = (int)(x & 63);
    const int64_t sc = x >> 6;
    const int c = (int)(sc % nchunks), strip = (int)(sc / nchunks);
    const int i = lane & 15, q = lane >> 4;
    const uint8_t* const L = lo + b * sl_b;
    const uint8_t* const H = hi + b * sh_b;
    uint32_t R[24];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        const int n = strip * kTileN + 16 * t + i;
        uint32_t l0 = 0, l1 = 0, hd = 0;
        if (n < N) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                l0 |= (uint32_t)L[((int64_t)c * 32 + 8 * q + e) * N + n] << (8 * e);
                l1 |= (uint32_t)L[((int64_t)c * 32 + 8 * q + 4 + e) * N + n] << (8 * e);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int rows[4] = {8 * q + e, 32 + 8 * q + e, 8 * q + 4 + e, 32 + 8 * q + 4 + e};
                uint32_t byte = 0;
#pragma unroll
                for (int f = 0; f < 4; ++f) {
                    const int r = rows[f];
                    const uint32_t top = (H[((int64_t)c * 16 + (r & 15)) * N + n] >> (2 * (r >> 4))) & 3u;
                    byte |= top << (2 * f);
                }
                hd |= byte << (8 * e);
            }
        }
        R[2 * t] = l0;
        R[2 * t + 1] = l1;
        R[16 + t] = hd;
    }
    uint8_t* const blk = out + ((int64_t)b * strips * nchunks + sc) * kPackBytes + 16 * lane;
#pragma unroll
    for (int k = 0; k < 6; ++k) *reinterpret_cast<u4*>(blk + 1024 * k) = u4{R[4 * k], R[4 * k + 1], R[4 * k + 2], R[4 * k + 3]};
}

// Repack the scales: one thread per (b, strip, group, i) writes the eight scales of columns 128 strip + 16 t + i.
__global__ __launch_bounds__(256) void w6a16_pack_scales_kernel(const uint16_t* sc, uint16_t* out, int32_t groups,
                                                                int32_t N, int32_t strips, int64_t ss_b) {
    const int64_t x = (int64_t)blockIdx.x * 256 + threadIdx.x;  // ((strip * groups + g) * 16 + i) within batch
    const int b = blockIdx.y;
    if (x >= (int64_t)strips * groups * 16) return;
    const int i = (int)(x & 15);
    const int64_t sg = x >> 4;
    const int g = (int)(sg % groups), strip = (int)(sg / groups);
    uint32_t o[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        uint32_t v[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int n = strip * kTileN + 16 * (2 * h + u) + i;
            v[u] = n < N ? sc[b * ss_b + (int64_t)g * N + n] : 0u;
        }
        o[h] = v[0] | v[1] << 16;
    }
    *reinterpret_cast<u4*>(out + ((int64_t)b * strips * groups + sg) * kTileN + 8 * i) = u4{o[0], o[1], o[2], o[3]};
}

// Dequantise: w[b][k][n] = s q as bf16 or fp32 (the large-M path hands the result to a library GEMM).  Grid
// (ceil(N / 4096), K / 2, B): one thread per (lo row c * 32 + j, 16 columns); it writes rows c * 64 + j and
// c * 64 + j + 32 of those columns.
template <typename OutT>
__global__ __launch_bounds__(256) void w6a16_dequant_kernel(const uint8_t* lo, const uint8_t* hi, const uint16_t* sc,
                                                            OutT* w, int32_t K, int32_t N, int32_t group_k,
                                                            int64_t sl_b, int64_t sh_b, int64_t ss_b, int64_t sw_b) {
    const int n = (blockIdx.x * 256 + threadIdx.x) * 16;
    if (n >= N) return;
    const int lrow = blockIdx.y, b = blockIdx.z;
    const int c = lrow >> 5, j = lrow & 31;
    const u4 L = *reinterpret_cast<const u4*>(lo + b * sl_b + (int64_t)lrow * N + n);
    const u4 H = *reinterpret_cast<const u4*>(hi + b * sh_b + ((int64_t)c * 16 + (j & 15)) * N + n);
    const int sh0 = 2 * (j >> 4), sh1 = sh0 + 4;  // 2-bit fields of rows j and j + 32
    const int r0 = c * 64 + j, r1 = r0 + 32;
    const uint16_t* const s0 = sc + b * ss_b + (int64_t)(r0 / group_k) * N + n;
    const uint16_t* const s1 = sc + b * ss_b + (int64_t)(r1 / group_k) * N + n;
    OutT* const w0 = w + b * sw_b + (int64_t)r0 * N + n;
    OutT* const w1 = w + b * sw_b + (int64_t)r1 * N + n;
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // columns n + 8 h .. + 7
        const u4 sa = *reinterpret_cast<const u4*>(s0 + 8 * h), sb = *reinterpret_cast<const u4*>(s1 + 8 * h);
        float va[8], vb[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int col = 8 * h + e, wd = col >> 2, by = 8 * (col & 3);
            const uint32_t l = (L[wd] >> by) & 0xFF, hh = (H[wd] >> by) & 0xFF;
            const int q0 = (int)((l & 15) | (((hh >> sh0) & 3) << 4)) - 32;
            const int q1 = (int)((l >> 4) | (((hh >> sh1) & 3) << 4)) - 32;
            va[e] = h2f((uint16_t)(sa[e >> 1] >> (16 * (e & 1)))) * (float)q0;  // exact: 11 x 6 bit product
            vb[e] = h2f((uint16_t)(sb[e >> 1] >> (16 * (e & 1)))) * (float)q1;
        }
        store8(w0 + 8 * h, va);
        store8(w1 + 8 * h, vb);
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Large-M kernel (M > kBigMinM, prefill-sized M, packed weights): C = A W~ with W~ = s q rounded to A's type -- the
// values w6a16_dequantize writes, so the result is that of dequantising and multiplying, in one kernel with no
// workspace.  A workgroup of eight wavefronts (two per SIMD) computes a 256 x 256 tile of C.  Per 64-row chunk of K it
// stages A's 256 x 64 slice and W~'s 64 x 256 slice (dequantised once per workgroup and stored transposed: LDS row n
// holds the 64 k of column n) in LDS, double-buffered with one barrier per chunk.  Wavefront (wm, wn) multiplies a
// 128 x 64 eighth: 32 MFMA tiles, 128 fp32 accumulators a lane, in 16 blocks (k half, 16-row tile) whose A operand is
// read one block ahead.  In the MFMAs' shadow, a quarter of the next chunk's weight share (loaded one chunk earlier)
// is dequantised and stored after every fourth block, A's next chunk (loaded at the chunk's start) is stored at its
// end, and the weight bytes of the chunk after that are loaded; scheduler fences keep this order.  The MFMA's A
// operand is a W~^T tile (rows n), its B operand an A^T tile (columns m), so lane (i, q) of tile (mt, nt) ends
// holding C[m0 + 16 mt + i][n0 + 16 nt + 4 q .. + 3]: four adjacent outputs, stored together.
constexpr int kBigTile = 256;                  // rows of A and columns of W per workgroup
constexpr int kBigStage = 2 * kBigTile * 128;  // bytes per stage: A rows, then W~^T rows, 64 elements each

// 16-byte piece p (k = 8 p .. 8 p + 7) of LDS row r (128-byte rows): piece slots XOR-swizzled by (r >> 1) & 7, so the
// 16 rows of one operand read (one p) fall in 16 different 16-byte bank groups.
__device__ __forceinline__ int big_slot(int r, int p) { return r * 128 + 16 * (p ^ ((r >> 1) & 7)); }

// Two values as a pair of A's element type (round to nearest even).
template <class A>
__device__ __forceinline__ uint32_t pack_act(float x, float y) {
    if constexpr (std::is_same_v<A, ActF16>)
        return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x) |
               (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)y) << 16;
    else
        return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x) | (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)y)
                                                                      << 16;
}

// s (u - 32) of the four codes u in the bytes of `u`, as A's type: the fp32 product of an 11-bit scale and a 6-bit
// integer is exact, so the one rounding is the conversion (the dequantisation kernel's values, bit for bit).
template <class A>
__device__ __forceinline__ void dequant4(uint32_t u, float s, float s32, uint32_t& d0, uint32_t& d1) {
    const float v0 = __builtin_fmaf((float)(u & 0xFF), s, s32), v1 = __builtin_fmaf((float)((u >> 8) & 0xFF), s, s32);
    const float v2 = __builtin_fmaf((float)((u >> 16) & 0xFF), s, s32), v3 = __builtin_fmaf((float)(u >> 24), s, s32);
    d0 = pack_act<A>(v0, v1);
    d1 = pack_act<A>(v2, v3);
}

// One chunk's weight bytes, per thread: the packed weight's share of wavefront w (strip w >> 2 of the tile, tiles
// 2 (w & 3) and 2 (w & 3) + 1 -- their lo dwords, one 16-byte lane load of the block, their two hi dwords and their
// two scales).  A's rows go from memory straight into LDS (big_copy_a).
struct BigW {
    u4 w;
    uint2 h;
    uint32_t sc;
};

// Where a thread's loads go, fixed for the call: raw buffers over A's batch slice, the packed weight's and its scales
// (wave-uniform descriptors), the lane's 32-bit offsets, and the wavefront's strip offsets; per chunk only a scalar
// offset changes.  (With 64-bit per-lane addresses the compiler placed the next chunk's address registers where the
// previous chunk's weight bytes were still arriving and waited for those loads first.)
struct BigSrc {
    __amdgpu_buffer_rsrc_t ra, rw, rs;
    int va[4];        // A row 8 w + 64 j + (lane >> 3) of the tile, the piece its LDS slot lane & 7 holds (+ 128
                      // bytes per chunk)
    int vw, vh, vs;   // the lane's offsets into a weight block (lo dwords, hi dwords) and a scale block
    int sw, ss;       // the wavefront's strip: byte offsets of its first weight block and first scale block
};

__device__ __forceinline__ BigSrc big_src(const Args& p, int b, int m0, int n0) {
    BigSrc d;
    const int t = threadIdx.x, wv = t >> 6, lane = t & 63, i = lane & 15, w4 = wv & 3;
    const int nchunks = p.K / 64, groups = p.K / p.group_k;
    d.ra = rsrc((uint64_t)(p.a + (int64_t)b * p.sa_b), ((int64_t)(p.M - 1) * p.sa_m + p.K) * 2);
    d.rw = rsrc((uint64_t)(p.lo + (int64_t)b * p.sl_b), (int64_t)p.n_strips * nchunks * kPackBytes);
    d.rs = rsrc((uint64_t)(p.sc + (int64_t)b * p.ss_b), (int64_t)p.n_strips * groups * kTileN * 2);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = 8 * wv + 64 * j + (lane >> 3), piece = (lane & 7) ^ ((r >> 1) & 7);  // big_slot's swizzle
        d.va[j] = min(m0 + r, p.M - 1) * (int)p.sa_m * 2 + 16 * piece;
    }
    const int strip = min(n0 / kTileN + (wv >> 2), p.n_strips - 1);
    d.vw = 1024 * w4 + 16 * lane;                                  // R[4 w4 .. 4 w4 + 3]
    d.vh = 1024 * (4 + (w4 >> 1)) + 8 * (w4 & 1) + 16 * lane;     // R[16 + 2 w4], R[17 + 2 w4]
    d.vs = (8 * i + 2 * w4) * 2;
    d.sw = strip * nchunks * kPackBytes;
    d.ss = strip * groups * kTileN * 2;
    return d;
}

__device__ __forceinline__ void vmem_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// A's 256 x 64 slice of chunk c into a stage, straight from memory (buffer_load ... lds): wavefront w's load j fills
// the stage's 1 KB of rows 8 w + 64 j .. + 7, lane l the 16-byte slot l & 7 of row 8 w + 64 j + (l >> 3), with the
// piece big_slot places there.  The two stages are separate LDS arrays, so the compiler sees that these writes do
// not alias the current stage's operand reads and waits for them only at the barrier.
__device__ __forceinline__ void big_copy_a(const BigSrc& d, int c, uint8_t* stage) {
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(d.ra, (__attribute__((address_space(3))) void*)(stage + (8 * wv + 64 * j) * 128),
                                                 16, d.va[j], soff(128 * c), 0, 0);
}

__device__ __forceinline__ void big_load_w(const Args& p, const BigSrc& d, int c, BigW& g) {
    const int blk = soff(d.sw + c * kPackBytes);
    g.w = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(d.rw, d.vw, blk, 0));
    g.h = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(d.rw, d.vh, blk, 0));
    g.sc = __builtin_amdgcn_raw_buffer_load_b32(d.rs, d.vs, soff(d.ss + ((c * 64) / p.group_k) * kTileN * 2), 0);
}

// Piece e (0..3) of the wavefront's weight share, dequantised into the stage: tile t = 2 (w & 3) + (e >> 1), rows
// 8 q .. + 7 (e even) or 32 + 8 q .. + 7 (e odd) of column 128 (w >> 2) + 16 t + i.
template <class A>
__device__ __forceinline__ void big_store_w(uint8_t* stage, const BigW& g, int e) {
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4, w4 = wv & 3;
    const int tt = e >> 1;
    const uint32_t L0 = g.w[2 * tt], L1 = g.w[2 * tt + 1], Hd = tt ? g.h.y : g.h.x;
    uint32_t ua, ub;
    if (e & 1) {
        ua = ((L0 >> 4) & 0x0F0F0F0Fu) | ((Hd & 0x0C0C0C0Cu) << 2);  // rows 32 + 8 q + 0..3
        ub = ((L1 >> 4) & 0x0F0F0F0Fu) | ((Hd >> 2) & 0x30303030u);  // rows 32 + 8 q + 4..7
    } else {
        ua = (L0 & 0x0F0F0F0Fu) | ((Hd & 0x03030303u) << 4);  // rows 8 q + 0..3
        ub = (L1 & 0x0F0F0F0Fu) | (Hd & 0x30303030u);         // rows 8 q + 4..7
    }
    const float s = h2f((uint16_t)(g.sc >> (16 * tt))), s32 = -32.f * s;
    uint32_t d[4];
    dequant4<A>(ua, s, s32, d[0], d[1]);
    dequant4<A>(ub, s, s32, d[2], d[3]);
    const int r = kBigTile + 128 * (wv >> 2) + 16 * (2 * w4 + tt) + i;
    *reinterpret_cast<u4*>(stage + big_slot(r, (e & 1) * 4 + q)) = u4{d[0], d[1], d[2], d[3]};
}

// Tile index -> (M tile, N tile).  Workgroup x runs on XCD x % 8; when the tiles divide evenly, XCD x takes the x-th
// eighth of the tiles in bands of 8 N tiles, M tile by M tile, so the workgroups resident on one XCD at a time share
// A's rows and W's columns in that XCD's L2.
__device__ __forceinline__ void big_tile(int tiles_m, int tiles_n, int& tm, int& tn) {
    const int T = tiles_m * tiles_n, x = blockIdx.x;
    const int L = (T % 8 == 0) ? (x % 8) * (T / 8) + x / 8 : x;
    constexpr int kBand = 8;
    const int band = L / (tiles_m * kBand), idx = L - band * tiles_m * kBand;
    const int width = min(kBand, tiles_n - band * kBand);
    tm = idx / width;
    tn = band * kBand + idx % width;
}

// The wavefront's 128 x 64 outputs, lane row m0 + 16 mt, columns n0 + 16 nt .. + 3: ES = 4 (fp32) or 2 (bf16 / fp16,
// out_dtype) bytes an element in one vector store, or (VEC false) element by element as out_dtype.
template <int ES, bool VEC>
__device__ __forceinline__ void big_store_out(const Args& p, int b, int m0, int n0, const f4 (&acc)[8][4]) {
    const bool f16 = p.out_dtype == W6A16_OUT_F16;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
        const int m = m0 + 16 * mt;
        if (m >= p.M) continue;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            const int n = n0 + 16 * nt;
            if (n >= p.N) continue;
            const int64_t o = (int64_t)b * p.so_b + (int64_t)m * p.so_m + n;
            const f4 v = acc[mt][nt];
            if constexpr (VEC && ES == 4) {
                *reinterpret_cast<f4*>(reinterpret_cast<float*>(p.out) + o) = v;
            } else if constexpr (VEC) {
                *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.out) + o) =
                    f16 ? uint2{pack_act<ActF16>(v[0], v[1]), pack_act<ActF16>(v[2], v[3])}
                        : uint2{pack_act<ActBF16>(v[0], v[1]), pack_act<ActBF16>(v[2], v[3])};
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (p.out_dtype == W6A16_OUT_F32)
                        reinterpret_cast<float*>(p.out)[o + e] = v[e];
                    else if (f16)
                        reinterpret_cast<_Float16*>(p.out)[o + e] = (_Float16)v[e];
                    else
                        reinterpret_cast<__bf16*>(p.out)[o + e] = (__bf16)v[e];
                }
            }
        }
    }
}

// One chunk of the large-M kernel: the MFMAs over stage `cur`; the next chunk's weights dequantised into the other
// stage's weight rows (`nxt_w`) during the first two MFMA blocks, then A's next chunk copied into its A rows (`nxt_a`,
// the same stage base: the two touch disjoint bytes).  The stages come in as restrict pointers, so that after
// inlining their accesses carry alias scopes and the compiler's wait insertion sees that the copies do not alias the
// operand reads of `cur`; no LDS store follows the copies within the step (the compiler would wait for them before
// one), so the only wait for them is at the barrier.
template <class A>
__device__ __forceinline__ void big_step(const Args& p, const BigSrc& src, int c, int nch,
                                         const uint8_t* __restrict__ cur, uint8_t* __restrict__ nxt_a,
                                         uint8_t* __restrict__ nxt_w, const BigW& ws, BigW& wl, f4 (&acc)[8][4]) {
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    const int wm = wv & 1, wn = wv >> 1;
    big_load_w(p, src, min(c + 2, nch - 1), wl);
    u4 wo[4], ao[2];
    ao[0] = *reinterpret_cast<const u4*>(cur + big_slot(128 * wm + i, q));
#pragma unroll
    for (int blk = 0; blk < 16; ++blk) {
        const int kh = blk >> 3, mt = blk & 7;
        if (mt == 0) {
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
                wo[nt] = *reinterpret_cast<const u4*>(cur + kBigTile * 128 + big_slot(64 * wn + 16 * nt + i, 4 * kh + q));
        }
        if (blk + 1 < 16) {
            const int kn = (blk + 1) >> 3, mn = (blk + 1) & 7;
            ao[(blk + 1) & 1] = *reinterpret_cast<const u4*>(cur + big_slot(128 * wm + 16 * mn + i, 4 * kn + q));
        }
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = A::mma(wo[nt], ao[blk & 1], acc[mt][nt]);
        if (blk < 2) {
#pragma unroll
            for (int e = 2 * blk; e < 2 * blk + 2; ++e) big_store_w<A>(nxt_w, ws, e);
        }
        if (blk == 1) big_copy_a(src, min(c + 1, nch - 1), nxt_a);  // after the last weight store (the last steps
                                                                       // copy the last chunk again, unused)
        __builtin_amdgcn_sched_barrier(0);
    }
    vmem_wait();
    __syncthreads();
}

template <class A>
__global__ __launch_bounds__(512, 1) void w6a16_big_kernel(const Args p) {
    __shared__ __attribute__((aligned(16))) uint8_t lds0[kBigStage];
    __shared__ __attribute__((aligned(16))) uint8_t lds1[kBigStage];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    const int wm = wv & 1, wn = wv >> 1;  // rows 128 wm .., columns 64 wn ..
    const int tiles_m = (p.M + kBigTile - 1) / kBigTile, tiles_n = (p.N + kBigTile - 1) / kBigTile;
    int tm, tn;
    big_tile(tiles_m, tiles_n, tm, tn);
    const int b = blockIdx.z, m0 = tm * kBigTile, n0 = tn * kBigTile;
    const int nch = p.K / 64;
    f4 acc[8][4];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};
    const BigSrc src = big_src(p, b, m0, n0);
    BigW w0, w1;
    big_copy_a(src, 0, lds0);
    big_load_w(p, src, 0, w0);
    big_load_w(p, src, min(1, nch - 1), w1);
#pragma unroll
    for (int e = 0; e < 4; ++e) big_store_w<A>(lds0, w0, e);
    vmem_wait();  // this wavefront's copies into the stage have landed (the barrier does not wait for them)
    __syncthreads();
    // chunk c: its stage is c & 1 (lds0 / lds1, fixed per unrolled step); ws holds chunk c + 1's weight bytes, wl
    // receives chunk c + 2's
    auto step = [&](auto odd, int c, const BigW& ws, BigW& wl) {
        if constexpr (decltype(odd)::value)
            big_step<A>(p, src, c, nch, lds1, lds0, lds0, ws, wl, acc);
        else
            big_step<A>(p, src, c, nch, lds0, lds1, lds1, ws, wl, acc);
    };
    for (int c = 0; c < nch; c += 2) {
        step(std::false_type{}, c, w1, w0);
        if (c + 1 < nch) step(std::true_type{}, c + 1, w0, w1);
    }
    // lane (i, q) of tile (mt, nt): C[m0 + 128 wm + 16 mt + i][n0 + 64 wn + 16 nt + 4 q .. + 3] (N % 16 == 0: the
    // four columns are all inside or all outside)
    if (p.out_vec && p.out_dtype == W6A16_OUT_F32)
        big_store_out<4, true>(p, b, m0 + 128 * wm + i, n0 + 64 * wn + 4 * q, acc);
    else if (p.out_vec)
        big_store_out<2, true>(p, b, m0 + 128 * wm + i, n0 + 64 * wn + 4 * q, acc);
    else
        big_store_out<0, false>(p, b, m0 + 128 * wm + i, n0 + 64 * wn + 4 * q, acc);
}

int cu_count() { return wkv7::device_cu_count(); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Narrow kernel (M <= 32 rows): one 16-row tile per wavefront, one M group per 16 rows (measured at K = 4096,
// N = 16384: M = 32 is faster with one tile per wavefront and two M groups).  Wide kernel (M > 32): MTW 16-row tiles
// per wavefront, KP K parts per workgroup, chains of CG chunks.
bool wide_rows(int M) { return M > 32; }

struct WideCfg {
    int mtw, kp;
};
// Measured at K = 4096, N = 16384 (us per call, packed / planes): M = 64 (2, 2) 27.2 / 33.0, (4, 2) 31.3 / 32.4,
// (2, 1) 32.8 / 44.9; M = 128 (4, 2) 36.2 / 40.9, (2, 2) 46.2 / 54.8, (4, 1) 43.7 / 53.5; M = 256 (4, 1) 54.1 / 71.9,
// (8, 2) 57.5 / 72.8, (8, 1) 94.4 / 103.5, (4, 2) 64.1 / 73.2.
WideCfg wide_cfg(int M) {
    if (M <= 64) return {2, 2};
    if (M <= 128) return {4, 2};
    return {4, 1};
}

// Large-M kernel: M above this, packed weights (no workspace, no split-K).
constexpr int kBigMinM = 256;
// (its loads go through raw buffers: A's batch slice and the packed weight's below 2 GB)
bool big_rows(const w6a16_args* a) {
    if (a->M <= kBigMinM || a->format != W6A16_FORMAT_PACKED || a->K < 64) return false;
    const int64_t a_bytes = ((int64_t)(a->M - 1) * a->a_row_stride + a->K) * 2;
    const int64_t w_bytes = (int64_t)((a->N + kTileN - 1) / kTileN) * (a->K / 64) * kPackBytes;
    return a_bytes < 0x7FFFFFFF && w_bytes < 0x7FFFFFFF;
}

struct Layout {
    bool big;                    // the large-M kernel
    bool wide, gemv, gemv_half;  // gemv: the in-workgroup split-K kernel (no workspace); gemv_half: per half strip
    int mt, kp, cg, m_groups, n_strips, mpad, nchains;
    size_t tiles, counter_bytes, partial_bytes, rsum_offset, rsum_bytes;
};

Layout layout(const w6a16_args* a) {
    Layout l{};
    l.big = big_rows(a);
    l.wide = !l.big && wide_rows(a->M);
    l.n_strips = (a->N + kTileN - 1) / kTileN;
    if (l.big) return l;  // no workspace
    if (l.wide) {
        const WideCfg c = wide_cfg(a->M);
        l.mt = c.mtw;
        l.kp = c.kp;
        l.cg = (a->group_k % 128 == 0) ? 2 : 1;
        l.nchains = a->K / (64 * l.cg);
    } else {
        l.mt = 1;
        l.kp = 1;
    }
    const int rows_per_group = 16 * l.mt;  // A rows per workgroup (wide) or per wavefront (narrow)
    l.m_groups = (a->M + rows_per_group - 1) / rows_per_group;
    l.mpad = l.m_groups * rows_per_group;
    // In-workgroup split-K for the packed layout, and for the planes once its grid (one workgroup per strip and M
    // group) fills the chip.  Measured at K = 4096, N = 16384 (us per call, planes / packed, split 8): M = 1 split-K
    // across workgroups 17.2 / 16.4, in-workgroup 20.6 / 16.1; M = 16 22.4 / 23.1 against 22.6 / 18.6; M = 32 (split 4
    // across workgroups) 30.1 / 26.5 against 22.0 / 18.6.
    l.gemv = !l.wide && a->split_k >= 2 && a->split_k <= kGemvMaxSplit &&
             (a->format == W6A16_FORMAT_PACKED || (int64_t)a->B * l.m_groups * l.n_strips >= cu_count());
    l.gemv_half = l.gemv && a->format == W6A16_FORMAT_PACKED && (int64_t)a->B * l.m_groups * l.n_strips < cu_count();
    if ((a->split_k > 1 && !l.gemv) || l.wide) {
        l.tiles = (size_t)a->B * l.m_groups * l.n_strips;
        l.counter_bytes = kCounterRegion;
        l.partial_bytes = a->split_k > 1 ? l.tiles * a->split_k * (size_t)rows_per_group * kTileN * 4 : 0;
        l.rsum_offset = l.counter_bytes + l.partial_bytes;
        l.rsum_bytes = l.wide ? (size_t)a->B * l.nchains * l.mpad * 4 : 0;
    }
    return l;
}

int validate(const w6a16_args* a) {
    if (!a) return WKV7_ERR_NULL;
    if (a->B < 1 || a->M < 0 || a->N < 1 || a->K < 64 || a->K % 64 || a->N % 16) return WKV7_ERR_SHAPE;
    if (a->group_k < 64 || a->group_k % 64 || a->K % a->group_k) return WKV7_ERR_SHAPE;
    if (a->split_k < 1 || a->split_k > 256) return WKV7_ERR_ARG;
    if (a->out_dtype != W6A16_OUT_BF16 && a->out_dtype != W6A16_OUT_F16 && a->out_dtype != W6A16_OUT_F32)
        return WKV7_ERR_ARG;
    if (a->a_dtype != W6A16_IN_BF16 && a->a_dtype != W6A16_IN_F16) return WKV7_ERR_ARG;
    if (a->M == 0) return WKV7_OK;
    if (a->format != W6A16_FORMAT_PLANES && a->format != W6A16_FORMAT_PACKED) return WKV7_ERR_ARG;
    const bool packed = a->format == W6A16_FORMAT_PACKED;
    if (!a->a || !a->lo || (!packed && !a->hi) || !a->scales || !a->out) return WKV7_ERR_NULL;
    if (!aligned16(a->a) || !aligned16(a->lo) || a->a_row_stride % 8 || a->a_batch_stride % 8 ||
        a->lo_batch_stride % 16)
        return WKV7_ERR_ALIGN;
    if (packed ? (!aligned16(a->scales) || a->scales_batch_stride % 8)
               : (!aligned16(a->hi) || (reinterpret_cast<uintptr_t>(a->scales) & 3) || a->hi_batch_stride % 16 ||
                  a->scales_batch_stride % 2))
        return WKV7_ERR_ALIGN;
    if (a->a_row_stride < a->K || a->out_row_stride < a->N) return WKV7_ERR_SHAPE;
    const Layout l = layout(a);
    if (l.big) {  // grid (tiles, 1, B)
        const int64_t tiles = (int64_t)((a->M + kBigTile - 1) / kBigTile) * ((a->N + kBigTile - 1) / kBigTile);
        return (a->B > 65535 || tiles > 0x7FFFFFFF) ? WKV7_ERR_SHAPE : WKV7_OK;
    }
    if ((int64_t)a->B * (l.wide ? 1 : l.m_groups) > 65535) return WKV7_ERR_SHAPE;  // grid z: batch (x M groups)
    if (l.wide && (int64_t)l.m_groups * ((l.n_strips + 7) / 8) * 8 > 0x7FFFFFFF) return WKV7_ERR_SHAPE;
    if (a->split_k > 1 && l.tiles * 4 > kCounterRegion) return WKV7_ERR_SHAPE;  // more tiles than counters (0: gemv)
    if ((a->split_k > 1 && !l.gemv) || l.wide) {
        if (!a->workspace || a->workspace_bytes < l.rsum_offset + l.rsum_bytes) return WKV7_ERR_WORKSPACE;
        if (reinterpret_cast<uintptr_t>(a->workspace) % kCounterAlign) return WKV7_ERR_ALIGN;
    }
    return WKV7_OK;
}

template <class A, int D, int DH>
void launch_gemv(const Args& p, const Layout& l, bool packed, hipStream_t s) {
    const dim3 block(64 * p.split_k);
    if (packed && l.gemv_half)
        hipLaunchKernelGGL((w6a16_gemv_kernel<A, DH, true, 4>), dim3(2 * l.n_strips, 1, p.B * l.m_groups), block, 0, s,
                           p);
    else if (packed)
        hipLaunchKernelGGL((w6a16_gemv_kernel<A, D, true, kTiles>), dim3(l.n_strips, 1, p.B * l.m_groups), block, 0, s,
                           p);
    else
        hipLaunchKernelGGL((w6a16_gemv_kernel<A, D, false, kTiles>), dim3(l.n_strips, 1, p.B * l.m_groups), block, 0, s,
                           p);
}

template <class A, int MT, int D>
void launch(const Args& p, const Layout& l, bool packed, hipStream_t s) {
    const dim3 grid((l.n_strips + kStrips - 1) / kStrips, p.split_k, p.B * l.m_groups);
    if (packed)
        hipLaunchKernelGGL((w6a16_kernel<A, MT, D, true>), grid, dim3(64 * kStrips), 0, s, p);
    else
        hipLaunchKernelGGL((w6a16_kernel<A, MT, D, false>), grid, dim3(64 * kStrips), 0, s, p);
}

template <class A, int MTW, int KP, int CG>
void launch_wide(const Args& p, const Layout& l, bool packed, hipStream_t s) {
    constexpr int D = 4, NL = 4;  // packed weights D steps ahead; NL register stages of the LDS ring
    hipLaunchKernelGGL(w6a16_rowsum_kernel<A>, dim3(l.mpad / 4, (p.K + 511) / 512, p.B), dim3(256), 0, s, p);
    const dim3 grid(8 * l.m_groups * ((l.n_strips + 7) / 8), p.split_k, p.B);
    if (packed)
        hipLaunchKernelGGL((w6a16_wide_kernel<A, MTW, KP, CG, D, NL, true>), grid, dim3(256 * KP), 0, s, p);
    else
        hipLaunchKernelGGL((w6a16_wide_kernel<A, MTW, KP, CG, D, NL, false>), grid, dim3(256 * KP), 0, s, p);
}

template <class A, int MTW, int KP>
void launch_wide_cg(const Args& p, const Layout& l, bool packed, hipStream_t s) {
    if (l.cg == 2)
        launch_wide<A, MTW, KP, 2>(p, l, packed, s);
    else
        launch_wide<A, MTW, KP, 1>(p, l, packed, s);
}

// The kernel for the call's shape and layout, with activations of type A.
template <class A>
void launch_matmul(const Args& p, const Layout& l, bool packed, hipStream_t s) {
    if (l.big) {
        const int tiles = ((p.M + kBigTile - 1) / kBigTile) * ((p.N + kBigTile - 1) / kBigTile);
        hipLaunchKernelGGL(w6a16_big_kernel<A>, dim3(tiles, 1, p.B), dim3(512), 0, s, p);
    } else if (l.gemv && l.gemv_half && p.split_k <= 4)  // half strips, split <= 4: three chunks in flight
        launch_gemv<A, 2, 3>(p, l, packed, s);
    else if (l.gemv)
        launch_gemv<A, 2, 2>(p, l, packed, s);
    else if (!l.wide)
        launch<A, 1, 2>(p, l, packed, s);
    else if (l.mt == 2)
        launch_wide_cg<A, 2, 2>(p, l, packed, s);
    else if (l.kp == 2)
        launch_wide_cg<A, 4, 2>(p, l, packed, s);
    else
        launch_wide_cg<A, 4, 1>(p, l, packed, s);
}

}  // namespace
}  // namespace w6

extern "C" {

size_t w6a16_args_size(void) { return sizeof(w6a16_args); }

int w6a16_workspace_size(const w6a16_args* a, size_t* bytes) {
    if (!a || !bytes) return WKV7_ERR_NULL;
    if (a->M <= 0 || a->B < 1 || a->N < 1 || a->K < 64 || a->group_k < 64 ||
        (a->split_k <= 1 && !w6::wide_rows(a->M)) || w6::big_rows(a)) {
        *bytes = 0;
        return WKV7_OK;
    }
    const w6::Layout l = w6::layout(a);
    *bytes = l.rsum_offset + l.rsum_bytes;
    return WKV7_OK;
}

int w6a16_plan_split(int32_t B, int32_t M, int32_t N, int32_t K) {
    if (B < 1 || M < 1 || N < 1 || K < 64) return 1;
    w6a16_args shape{};
    shape.B = B;
    shape.M = M;
    shape.N = N;
    shape.K = K;
    shape.group_k = K % 128 == 0 ? 128 : 64;  // chains of two chunks where K allows them
    const w6::Layout l = w6::layout(&shape);
    // workgroups per split: narrow, four strips per workgroup; wide, one strip per workgroup
    const int64_t groups = (int64_t)B * l.m_groups * (l.wide ? l.n_strips : (l.n_strips + w6::kStrips - 1) / w6::kStrips);
    const int chunks = l.wide ? l.nchains : K / 64;  // the units a split range holds
    // narrow: one workgroup per CU; wide (4 KP wavefronts per workgroup): eight wavefronts per CU
    const int64_t cus = l.wide ? w6::cu_count() * 2 / l.kp : w6::cu_count();
    // The smallest power of two that gives every CU a workgroup (every range keeps at least one chunk); then doubled
    // while ranges keep at least 16 chunks and the launch stays within one workgroup per CU (each workgroup's
    // split-K hand-off costs one agent-scope release).  Measured at K = 4096, N = 16384 (us, planes / packed): M = 128
    // split 2 63.5 / 53.9, split 4 64.0 / 60.6; M = 64 split 4 41.7 / 37.1, split 8 51.3 / 49.1; M = 16 split 8
    // 23.6 / 23.4, split 4 29.1 / 25.3.
    int sk = 1;
    while (groups * sk < cus && sk * 2 <= 64 && chunks / (sk * 2) >= 1) sk *= 2;
    while (chunks / (sk * 2) >= 16 && groups * sk * 2 <= cus && sk * 2 <= 64) sk *= 2;
    // Narrow, split, and one workgroup per (strip, M group) fills the chip: the in-workgroup split-K kernel takes the
    // split, and its deepest split is the fastest (M = 32 above: split 4 24.1 / 19.5 us, split 8 22.0 / 18.6).
    if (!l.wide && sk >= 2 && (int64_t)B * l.m_groups * l.n_strips >= cus)
        while (sk * 2 <= w6::kGemvMaxSplit && chunks / (sk * 2) >= 1) sk *= 2;
    return sk;
}

int w6a16_plan_split_packed(int32_t B, int32_t M, int32_t N, int32_t K) {
    const int sk = w6a16_plan_split(B, M, N, K);
    if (sk != 8) return sk;
    w6a16_args shape{};
    shape.B = B;
    shape.M = M;
    shape.N = N;
    shape.K = K;
    shape.group_k = K % 128 == 0 ? 128 : 64;
    shape.split_k = sk;
    shape.format = W6A16_FORMAT_PACKED;
    const w6::Layout l = w6::layout(&shape);
    // Half strips (the in-workgroup kernel where strips are fewer than CUs) run fastest at split 4 with three chunks
    // in flight, given at least 8 chunks per range.  Measured at K = 4096, N = 16384 (us per call): M = 1 split 4
    // 11.9, split 8 12.4; M = 16 14.1 / 14.7.
    if (l.gemv_half && K / 64 / 4 >= 8) return 4;
    return sk;
}

int w6a16_matmul(const w6a16_args* a, void* stream) {
    const int rc = w6::validate(a);
    if (rc != WKV7_OK || a->M == 0) return rc;
    const w6::Layout l = w6::layout(a);
    w6::Args p{};
    p.a = a->a;
    p.sa_b = a->a_batch_stride;
    p.sa_m = a->a_row_stride;
    p.lo = a->lo;
    p.hi = a->hi;
    p.sl_b = a->lo_batch_stride;
    p.sh_b = a->hi_batch_stride;
    p.sc = a->scales;
    p.ss_b = a->scales_batch_stride;
    p.out = a->out;
    p.so_b = a->out_batch_stride;
    p.so_m = a->out_row_stride;
    if ((a->split_k > 1 && !l.gemv) || l.wide) {
        p.cnt = static_cast<uint32_t*>(a->workspace);
        p.part = reinterpret_cast<float*>(static_cast<char*>(a->workspace) + l.counter_bytes);
        p.rsum = reinterpret_cast<float*>(static_cast<char*>(a->workspace) + l.rsum_offset);
    }
    p.B = a->B;
    p.M = a->M;
    p.N = a->N;
    p.K = a->K;
    p.group_k = a->group_k;
    p.split_k = a->split_k;
    p.out_dtype = a->out_dtype;
    p.m_groups = l.m_groups;
    p.n_strips = l.n_strips;
    const int chunks = a->K / 64;
    p.chunks_per_split = (chunks + a->split_k - 1) / a->split_k;
    if (l.wide) {
        p.mpad = l.mpad;
        p.chain_k = 64 * l.cg;
        p.nchains = l.nchains;
        p.chains_per_split = (l.nchains + a->split_k - 1) / a->split_k;
    }
    p.out_vec = w6::aligned16(a->out) && a->out_row_stride % 8 == 0 && a->out_batch_stride % 8 == 0;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const bool packed = a->format == W6A16_FORMAT_PACKED;
    if (a->a_dtype == W6A16_IN_F16)
        w6::launch_matmul<w6::ActF16>(p, l, packed, s);
    else
        w6::launch_matmul<w6::ActBF16>(p, l, packed, s);
    return static_cast<int>(hipGetLastError());
}

int w6a16_dequantize_packed(const void* packed, const uint16_t* packed_scales, void* w, int32_t B, int32_t K,
                            int32_t N, int32_t group_k, int64_t w_batch_stride, int32_t out_dtype, void* stream) {
    if (!packed || !packed_scales || !w) return WKV7_ERR_NULL;
    if (B < 1 || N < 16 || N % 16 || K < 64 || K % 64 || group_k < 64 || group_k % 64 || K % group_k)
        return WKV7_ERR_SHAPE;
    if (out_dtype != W6A16_OUT_BF16 && out_dtype != W6A16_OUT_F16 && out_dtype != W6A16_OUT_F32) return WKV7_ERR_ARG;
    if (!w6::aligned16(packed) || !w6::aligned16(packed_scales)) return WKV7_ERR_ALIGN;
    if (B > 65535) return WKV7_ERR_SHAPE;
    const int strips = (N + w6::kTileN - 1) / w6::kTileN;
    const int64_t nw = (int64_t)strips * (K / 64) * 64;
    const dim3 grid((unsigned)((nw + 255) / 256), B);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t* pk = static_cast<const uint8_t*>(packed);
    if (out_dtype == W6A16_OUT_F32)
        hipLaunchKernelGGL(w6::w6a16_dequant_packed_kernel<float>, grid, dim3(256), 0, s, pk, packed_scales,
                           static_cast<float*>(w), K, N, group_k, strips, w_batch_stride);
    else if (out_dtype == W6A16_OUT_F16)
        hipLaunchKernelGGL(w6::w6a16_dequant_packed_kernel<_Float16>, grid, dim3(256), 0, s, pk, packed_scales,
                           static_cast<_Float16*>(w), K, N, group_k, strips, w_batch_stride);
    else
        hipLaunchKernelGGL(w6::w6a16_dequant_packed_kernel<__bf16>, grid, dim3(256), 0, s, pk, packed_scales,
                           static_cast<__bf16*>(w), K, N, group_k, strips, w_batch_stride);
    return static_cast<int>(hipGetLastError());
}

int w6a16_packed_size(int32_t B, int32_t K, int32_t N, int32_t group_k, size_t* weight_bytes, size_t* scale_bytes) {
    if (!weight_bytes || !scale_bytes) return WKV7_ERR_NULL;
    if (B < 1 || N < 16 || N % 16 || K < 64 || K % 64 || group_k < 64 || group_k % 64 || K % group_k)
        return WKV7_ERR_SHAPE;
    const size_t strips = (N + w6::kTileN - 1) / w6::kTileN;
    *weight_bytes = (size_t)B * strips * (K / 64) * w6::kPackBytes;
    *scale_bytes = (size_t)B * strips * (K / group_k) * w6::kTileN * 2;
    return WKV7_OK;
}

int w6a16_pack(const uint8_t* lo, const uint8_t* hi, const uint16_t* scales, int32_t B, int32_t K, int32_t N,
               int32_t group_k, int64_t lo_batch_stride, int64_t hi_batch_stride, int64_t scales_batch_stride,
               void* packed, uint16_t* packed_scales, void* stream) {
    size_t wb = 0, sb = 0;
    const int rc = w6a16_packed_size(B, K, N, group_k, &wb, &sb);
    if (rc != WKV7_OK) return rc;
    if (!lo || !hi || !scales || !packed || !packed_scales) return WKV7_ERR_NULL;
    if (!w6::aligned16(packed) || !w6::aligned16(packed_scales)) return WKV7_ERR_ALIGN;
    if (B > 65535) return WKV7_ERR_SHAPE;
    const int strips = (N + w6::kTileN - 1) / w6::kTileN, groups = K / group_k;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t nw = (int64_t)strips * (K / 64) * 64, ns = (int64_t)strips * groups * 16;
    hipLaunchKernelGGL(w6::w6a16_pack_kernel, dim3((unsigned)((nw + 255) / 256), B), dim3(256), 0, s, lo, hi,
                       static_cast<uint8_t*>(packed), K, N, strips, lo_batch_stride, hi_batch_stride);
    hipLaunchKernelGGL(w6::w6a16_pack_scales_kernel, dim3((unsigned)((ns + 255) / 256), B), dim3(256), 0, s, scales,
                       packed_scales, groups, N, strips, scales_batch_stride);
    return static_cast<int>(hipGetLastError());
}

int w6a16_dequantize(const uint8_t* lo, const uint8_t* hi, const uint16_t* scales, void* w, int32_t B, int32_t K,
                     int32_t N, int32_t group_k, int64_t lo_batch_stride, int64_t hi_batch_stride,
                     int64_t scales_batch_stride, int64_t w_batch_stride, int32_t out_dtype, void* stream) {
    if (!lo || !hi || !scales || !w) return WKV7_ERR_NULL;
    if (B < 1 || N < 16 || N % 16 || K < 64 || K % 64 || group_k < 64 || group_k % 64 || K % group_k)
        return WKV7_ERR_SHAPE;
    if (out_dtype != W6A16_OUT_BF16 && out_dtype != W6A16_OUT_F16 && out_dtype != W6A16_OUT_F32) return WKV7_ERR_ARG;
    if (!w6::aligned16(lo) || !w6::aligned16(hi) || !w6::aligned16(scales) || !w6::aligned16(w) ||
        lo_batch_stride % 16 || hi_batch_stride % 16 || scales_batch_stride % 8 || w_batch_stride % 8)
        return WKV7_ERR_ALIGN;
    if (K / 2 > 65535 || B > 65535) return WKV7_ERR_SHAPE;  // grid y and z
    const dim3 grid((N / 16 + 255) / 256, K / 2, B);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (out_dtype == W6A16_OUT_F32)
        hipLaunchKernelGGL(w6::w6a16_dequant_kernel<float>, grid, dim3(256), 0, s, lo, hi, scales,
                           static_cast<float*>(w), K, N, group_k, lo_batch_stride, hi_batch_stride,
                           scales_batch_stride, w_batch_stride);
    else if (out_dtype == W6A16_OUT_F16)
        hipLaunchKernelGGL(w6::w6a16_dequant_kernel<_Float16>, grid, dim3(256), 0, s, lo, hi, scales,
                           static_cast<_Float16*>(w), K, N, group_k, lo_batch_stride, hi_batch_stride,
                           scales_batch_stride, w_batch_stride);
    else
        hipLaunchKernelGGL(w6::w6a16_dequant_kernel<__bf16>, grid, dim3(256), 0, s, lo, hi, scales,
                           static_cast<__bf16*>(w), K, N, group_k, lo_batch_stride, hi_batch_stride,
                           scales_batch_stride, w_batch_stride);
    return static_cast<int>(hipGetLastError());
}

}  // extern "C"
