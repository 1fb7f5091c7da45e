// wkv7_device.h -- device-side building blocks shared by the WKV7 kernels (gfx950, wave64).
//
// Conventions (the reference's, rwkv_next/kernels/wkv7.py:4-7, 20):
//   per (sequence, head) the state S is K x V = 64 x 64 fp32 stored row-major [k][v] (v contiguous);
//   S_t = diag(d_t) S_{t-1} + b_t (a_t^T S_{t-1}) + k_t v_t^T,   d_t = exp(-exp(w_t)),   o_t = S_t^T r_t.
//   Operands r, w, k, v, a, b and the output o are bf16 rows [token][head][64].
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace wkv7 {

constexpr int HS = 64;          // head size, K == V
constexpr int HS2 = HS * HS;    // state elements per (sequence, head)

// f(std::integral_constant<int, 0>{}), .., f(std::integral_constant<int, N - 1>{}): straight-line copies of a step
// whose register-array indices must be compile-time constants.
template <typename F, int... J>
__device__ __forceinline__ void unroll_seq(F&& f, std::integer_sequence<int, J...>) {
    (f(std::integral_constant<int, J>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void unroll(F&& f) { unroll_seq(f, std::make_integer_sequence<int, N>{}); }

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN); gfx950 converts in hardware (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Unpack two bf16 held in one 32-bit word (low half first).
__device__ __forceinline__ void bf16x2_to_f32(uint32_t x, float& lo, float& hi) {
    lo = __uint_as_float(x << 16);
    hi = __uint_as_float(x & 0xffff0000u);
}

// Two fp32 -> two bf16 in one word (lo in the low half), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f2_t x = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2_t));
}

// Hi/lo split of two fp32 values into bf16 pairs: hw = (bf16(x0), bf16(x1)) rounded to nearest even, lw = the bf16 of
// the remainders x - hi.  Each remainder is exact in fp32 (hi holds x's top 8 significant bits) and is formed by one
// v_dot2c_f32_bf16 (x + hi . (-1, 0)) instead of unpacking hi and subtracting.  x ~ hi + lo to about 2^-17 relative.
// The selector pairs are kept in registers (an empty non-volatile asm, which the compiler may still hoist and share):
// folded into an inline constant, the bf16 pair (-1, 0) is emitted as the operand "-1.0", which the hardware reads
// as the pair (0, -1) -- measured on gfx950: every remainder wrong that way, all exact from a register.
__device__ __forceinline__ bf16x2_t bf16_pair_in_register(uint32_t bits) {
    asm("" : "+v"(bits));
    return __builtin_bit_cast(bf16x2_t, bits);
}

__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t& hw, uint32_t& lw) {
    const f2_t x = {x0, x1};
    const bf16x2_t h = __builtin_convertvector(x, bf16x2_t);
    const bf16x2_t m0 = bf16_pair_in_register(0x0000BF80u), m1 = bf16_pair_in_register(0xBF800000u);
    const float l0 = __builtin_amdgcn_fdot2_f32_bf16(h, m0, x0, false);
    const float l1 = __builtin_amdgcn_fdot2_f32_bf16(h, m1, x1, false);
    hw = __builtin_bit_cast(uint32_t, h);
    lw = pack_bf16x2(l0, l1);
}

// Decay d = exp(-exp(w)) of the raw w (rwkv_next/kernels/wkv7.py:74), with the device library's full-precision
// expf.
__device__ __forceinline__ float decay(float w) { return expf(-expf(w)); }

// Orders LDS traffic between the lanes of one wavefront: a wave's LDS instructions execute in issue order, so
// only compiler reordering has to be prevented.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Returns p (a pointer to global memory) as a wave-uniform (SGPR) value.  Loads through the result use a scalar
// base plus a 32-bit per-lane offset; without it LLVM hoists `base + lane` out of token loops as one 64-bit VGPR
// pair per pointer.  The value is rebuilt as a global-address-space pointer: rebuilt as a generic pointer the
// accesses would compile to flat instructions, which also count on lgkmcnt, so every LDS wait would then wait
// for outstanding global loads as well.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
    typedef __attribute__((address_space(1))) T GT;
    const uint64_t x = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
    GT* const g = (GT*)(((uint64_t)hi << 32) | lo);
    return (T*)g;
}

// Kernel-side view of one call (filled by the C-ABI layer from wkv7_args after validation).
struct Params {
    const uint16_t *r, *w, *k, *v, *a, *b;
    int64_t in_tok_stride;          // elements between tokens of the operands (head stride is 64)
    uint16_t* o;                    // nullable output
    int64_t o_tok_stride;
    const float* h0;                // nullable initial states [h0_rows, H, 64, 64]
    const int64_t* h0_idx;          // nullable: sequence n reads h0[h0_idx[n]]
    float* ht;                      // nullable final states [ht_rows, H, 64, 64]
    const int64_t* ht_idx;          // nullable: sequence n writes ht[ht_idx[n]]
    int64_t h0_rows, ht_rows;       // state rows addressable through h0 / ht (indices outside are ignored)
    const uint8_t* fresh;           // nullable: nonzero = sequence n starts from zeros
    const int32_t* cu;              // nullable cu_seqlens [num_seqs + 1]
    const int64_t* n_keep;          // nullable
    float* snap;                    // nullable [num_seqs][T][H][64][64]
    int64_t total_tokens;           // packed token count; ragged extents are clamped to it
    int32_t num_seqs;
    int32_t T;                      // dense tokens per sequence; snapshot time stride
    int32_t H;
    int32_t rec_max_len;            // chunked launches: rows this short run the recurrent path instead
    int32_t* status;                // nullable device status word (WKV7_STATUS_* bits)
    int32_t K;                      // head size: 64 for every kernel but the generic one (wkv7_generic.hip)
};

// Extent of sequence n (rwkv_next/kernels/wkv7.py:46-54).
__device__ __forceinline__ void seq_extent(const Params& p, int n, int64_t& bos, int& len) {
    if (p.cu) {
        // clamped to [0, total_tokens] so that a malformed cu_seqlens cannot index past the operands, and to the
        // caller's length bound T when one is given (it sizes the workspaces and the snapshot rows)
        int64_t s = p.cu[n], e = p.cu[n + 1];
        s = s < 0 ? 0 : (s > p.total_tokens ? p.total_tokens : s);
        e = e < s ? s : (e > p.total_tokens ? p.total_tokens : e);
        if (p.T > 0 && e - s > p.T) e = s + p.T;
        bos = s;
        len = (int)(e - s);
    } else {
        bos = (int64_t)n * p.T;
        len = p.T;
    }
    if (p.n_keep) {
        const int64_t nk = p.n_keep[n];
        if (nk < len) len = (int)(nk < 0 ? 0 : nk);
    }
    if (len < 0) len = 0;
}

// Initial state of (sequence n, head h), or nullptr for a zero state (no h0, a fresh row, or a slot index
// outside [0, h0_rows): such rows start from zeros instead of reading out of bounds; wkv7_status_kernel reports
// such indices when the caller asks for it).
__device__ __forceinline__ const float* state_src(const Params& p, int n, int h) {
    if (!p.h0 || (p.fresh && p.fresh[n])) return nullptr;
    const int64_t s = p.h0_idx ? p.h0_idx[n] : n;
    if (s < 0 || s >= p.h0_rows) return nullptr;
    return p.h0 + (s * p.H + h) * (int64_t)HS2;
}

// Final-state destination, or nullptr when not stored (no ht, or a slot index outside [0, ht_rows)).
__device__ __forceinline__ float* state_dst(const Params& p, int n, int h) {
    if (!p.ht) return nullptr;
    const int64_t s = p.ht_idx ? p.ht_idx[n] : n;
    if (s < 0 || s >= p.ht_rows) return nullptr;
    return p.ht + (s * p.H + h) * (int64_t)HS2;
}

}  // namespace wkv7
