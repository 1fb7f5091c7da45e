// wkv7_seg.hip -- chunked WKV7 prefill in one dispatch, with no chunk records in HBM (gfx950, bf16 MFMA).
//
// Replaces the reference's token-serial Triton program (rwkv_next/kernels/wkv7.py:65-77) for rows longer than the
// token-serial threshold, dense or varlen (wkv7.py:46-54).  The reference walks every token of a row in one program,
// so a B=1, T=4096, H=64 prefill has (64/BV)*64 programs and no parallelism over T.
//
// Decomposition.  A row is cut into chunks of C = 32 tokens and its chunks into segments of at most `seg` chunks.
// One workgroup (a "unit") takes one (row, head, segment):
//   * four prep wavefronts each build the transition of one chunk at a time, alone (no barrier inside a chunk), in
//     factored form (below), and hand the chunk's record (44 KB) to the state wavefronts through a three-slot LDS
//     ring;
//   * four state wavefronts each own 16 columns of the state (columns of S evolve independently) and apply the
//     records in chunk order: U = W S + U0, y, then S <- Gamma S + Bt^T U + Kt^T V.
//   A segment after the first starts from zeros and also accumulates P = A_n .. A_1 (A_c = Gamma + Bt^T W, the
//   chunk's linear part), the map from its true initial state S_in to its end state: S_end = S_local + P S_in, and
//   every output of chunk c gets (R0 + rho W)_c P_{c-1} S_in added.  S_in is
//   the previous segment's S_end, handed over through global memory (one flag per unit; the waiting unit always has
//   the higher workgroup index, so the earliest unfinished unit never waits and every wait ends).
//
// Algebra of one chunk (per head; S is K x V, the reference's orientation, wkv7.py:4-7, 62-79).  With
// g_t = sum_{u<=t} log2 d_u per channel (padding tokens count log2 d = 0), m = g_15 and c = g_31:
//   Ah_t = a_t 2^{g_{t-1} - m},  Rh_t = r_t 2^{g_t - m},  Bp_t = b_t 2^{m - g_t},  Kp_t = k_t 2^{m - g_t}
//   alpha[t][s] = Ah_t . Bp_s (s < t),  beta = Ah_t . Kp_s (s < t),  rho = Rh_t . Bp_s (s <= t),  sigma = Rh_t . Kp_s
//   T = (I - alpha)^{-1},  W = T Ah diag(2^m),  U0 = T beta V,  Bt = Bp diag(2^{c-m}),  Kt = Kp diag(2^{c-m}),
//   R0 = Rh diag(2^m),  Gamma = diag(2^c):
//   U = W S_0 + U0 (U_t = a_t^T S_{t-1}, from (I - alpha) U = Ah 2^m S_0 + beta V),
//   S_C = Gamma S_0 + Bt^T U + Kt^T V,   y^T = S_0^T R0^T + U^T rho^T + V^T sigma^T.
// Every decay factor is one v_exp_f32 of a difference of the same partial sums, and |g_t - m| <= 16 max|log2 d|
// (<= 63 for w <= WKV7_CHUNK_W_MAX), inside fp32 and bf16 range.
//
// Precision.  Products feeding the state (alpha, beta, T, W, U0, U, the state update and P) run as three bf16
// MFMAs on hi/lo splits (x = hi + lo, relative error ~2^-17 per operand), two where one operand is exact bf16 (V);
// products feeding only y (rho, sigma, R0, y, the P terms of y, the correction) run as one.  fp32 accumulation.
//
// Register layouts (lane l: i = l & 15, q = l >> 4).
//   N layout of a token x channel matrix M, token tile tau (16 rows), channel block kb (32): lane holds
//     M[16 tau + i][32 kb + 8 q + e], e = 0..7 -- one 16-byte global load.  Two N fragments as the A and B operands
//     of v_mfma_f32_16x16x32_bf16 give the Gram tile M1 M2^T.
//   RL layout of a 16 x 16 tile of X (the MFMA result layout): lane holds X[x0 + 4 q + v][y0 + i], v = 0..3.
//     With RL(X) as the A operand and RL(Y) as the B operand, v_mfma_f32_16x16x16bf16_1k accumulates RL(X^T Y)
//     (contraction over the 16 rows); two RL tiles stacked (rows 0-15 in elements 0-3, rows 16-31 in 4-7) are the
//     16x16x32 operand of a 32-row contraction (the contraction order is permuted alike in both operands).
//   An identity operand turns an N fragment into the RL tile of M or of M^T (one exact MFMA per tile).
// The state S is held as RL tiles (k tile m, column tile j); a state wavefront j holds tiles (0..3, j).
#include <algorithm>
#include <cstdint>

#include "wkv7.h"
#include "wkv7_device.h"
#include "wkv7_launch.h"
#include "wkv7_token.h"

namespace wkv7 {

namespace {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2v __attribute__((ext_vector_type(2)));

constexpr int SC = kSegChunk;          // 32 tokens per chunk
constexpr int NREC = 3;                // LDS ring slots
constexpr float kL2E = 1.4426950408889634f;
constexpr int kSpinLimit = 1 << 22;    // LDS ring waits (s_sleep 1 each: a few hundred ms at most)
constexpr int kFlagSpinLimit = 1 << 20;  // segment hand-off waits (s_sleep 8 each)

// Record of one chunk in the LDS ring (byte offsets).  Pieces are lane-contiguous 16-byte words.
// The chunk transition is kept in factored form (W = W' diag(2^m), R0 = Rh diag(2^m), and Bp, Kp with their row
// factor 2^{c-m} kept apart): the state wavefronts apply
//   U = W S + U0,   S <- Gamma S + diag(2^{c-m}) (Bp^T U + Kp^T V),   y^T = S^T R0^T + U^T rho^T + V^T sigma^T
// per 16-column tile, which costs them about as many MFMAs as a dense A S + H would and saves the prep wavefront
// forming A, H and O (its critical path; the state wavefronts have slack).  Bp and Kp go into the record as exact
// transposes of the prep's own hi/lo splits, so the prep wavefront does not rescale and split them again.
constexpr int REC_W = 0;                       // W^T hi/lo as 16x16x32 A operands: [token tile][kb][hl][lane]
constexpr int REC_B = REC_W + 8 * 1024;        // Bp hi/lo as 16x16x32 A operands: [k tile m][hl][lane]
constexpr int REC_K = REC_B + 8 * 1024;        // Kp hi/lo, same
constexpr int REC_R = REC_K + 8 * 1024;        // R0^T hi as 16x16x32 B operands: [token tile][kb][lane]
constexpr int REC_U = REC_R + 4 * 1024;        // U0, RL fp32: [column tile j][token tile][lane]
constexpr int REC_V = REC_U + 8 * 1024;        // V (exact), RL tiles (0, j), (1, j) stacked: [column tile j][lane]
constexpr int REC_RHO = REC_V + 4 * 1024;      // rho^T hi: tile (0,0) (low 8 bytes), then tiles (0,1), (1,1) stacked
constexpr int REC_SIG = REC_RHO + 2 * 1024;    // sigma^T hi, same
constexpr int REC_G = REC_SIG + 2 * 1024;      // Gamma = 2^c per channel, fp32 [64]
constexpr int REC_F = REC_G + 256;             // 2^{c-m} per channel, fp32 [64]
constexpr int REC_BYTES = REC_F + 256;         // 45568

struct SegSmem {
    char ring[NREC][REC_BYTES];
    float fac[4][4][HS];   // per prep wavefront: 2^m, 2^{c-m}, 2^c, 2^{-m} per channel of its current chunk
    int ready[NREC];       // chunk index + 1 of the record a slot holds
    int done[NREC][4];     // per state wavefront: uses of the slot it has finished reading
    int fail;
    int scan[8];
    int rows[kSegMaxRows + 1];  // ragged and n_keep calls: first stream chunk of each row
};

__device__ __forceinline__ f4 z4() { return f4{0.f, 0.f, 0.f, 0.f}; }
__device__ __forceinline__ f4 mma32(bf8 a, bf8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
__device__ __forceinline__ f4 mma16(s4 a, s4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0); }

struct T4 { s4 h, l; };   // hi/lo bf16 of an RL tile
struct T8 { bf8 h, l; };  // hi/lo bf16 16x16x32 operand

__device__ __forceinline__ T4 split_t(f4 x) {
    uint32_t hw[2], lw[2];
    split_pair(x[0], x[1], hw[0], lw[0]);
    split_pair(x[2], x[3], hw[1], lw[1]);
    return T4{__builtin_bit_cast(s4, hw), __builtin_bit_cast(s4, lw)};
}
__device__ __forceinline__ s4 hi_t(f4 x) {
    const uint32_t hw[2] = {pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
    return __builtin_bit_cast(s4, hw);
}
__device__ __forceinline__ bf8 cat(s4 a, s4 b) {
    return __builtin_bit_cast(bf8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}
__device__ __forceinline__ T8 cat(T4 a, T4 b) { return T8{cat(a.h, b.h), cat(a.l, b.l)}; }
// RL(X^T Y) += ..., 16 contraction rows (small terms first)
__device__ __forceinline__ f4 p16x3(T4 x, T4 y, f4 c) {
    c = mma16(x.h, y.l, c);
    c = mma16(x.l, y.h, c);
    return mma16(x.h, y.h, c);
}
__device__ __forceinline__ f4 p16x2(T4 x, s4 y, f4 c) {  // y exact in bf16
    c = mma16(x.l, y, c);
    return mma16(x.h, y, c);
}
// 32 contraction rows
__device__ __forceinline__ f4 p32x3(T8 x, T8 y, f4 c) {
    c = mma32(x.h, y.l, c);
    c = mma32(x.l, y.h, c);
    return mma32(x.h, y.h, c);
}
__device__ __forceinline__ f4 p32x2(T8 x, bf8 y, f4 c) {
    c = mma32(x.l, y, c);
    return mma32(x.h, y, c);
}

// x + I for an RL tile on the diagonal
__device__ __forceinline__ f4 plus_i(f4 x, int lane) {
    const int i = lane & 15, q = lane >> 4;
#pragma unroll
    for (int v = 0; v < 4; ++v) x[v] += (4 * q + v == i) ? 1.f : 0.f;
    return x;
}
// RL(I) as a bf16 operand
__device__ __forceinline__ s4 ident16(int lane) {
    const int i = lane & 15, q = lane >> 4;
    s4 r;
#pragma unroll
    for (int v = 0; v < 4; ++v) r[v] = (4 * q + v == i) ? (short)0x3F80 : (short)0;
    return r;
}
// Column selector of a 16x16x32 operand: element e of lane (i, q) is 1 iff 8 q + e == i + 16 par.  As the B operand
// after an N fragment of block kb it yields the RL tile of columns 32 kb + 16 par ..; as the A operand before one, the
// RL tile of the transpose.
__device__ __forceinline__ bf8 isel(int par, int lane) {
    const int i = lane & 15, q = lane >> 4;
    s4 a, b;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        a[e] = (8 * q + e == i + 16 * par) ? (short)0x3F80 : (short)0;
        b[e] = (8 * q + 4 + e == i + 16 * par) ? (short)0x3F80 : (short)0;
    }
    return cat(a, b);
}

// mask of an RL tile on the diagonal: keep row < column (strict) or row <= column
__device__ __forceinline__ f4 keep_upper(f4 x, int lane, bool strict) {
    const int i = lane & 15, q = lane >> 4;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int r = 4 * q + v;
        if (strict ? !(r < i) : !(r <= i)) x[v] = 0.f;
    }
    return x;
}

// Cross-lane moves.  prep_chunk runs them in straight-line code with every lane active (its lane-dependent choices
// are bit selects, never branches), so no move can read a lane that is switched off.
template <int CTRL, bool BC>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, BC));
}
// a where mask is all ones, b where it is zero (v_bfi_b32)
__device__ __forceinline__ float bitsel(uint32_t mask, float a, float b) {
    return __uint_as_float((__float_as_uint(a) & mask) | (__float_as_uint(b) & ~mask));
}
// inclusive prefix sums over the 16 lanes of each row of N values (Hillis-Steele on row_shr; lanes before the start
// read 0), in lockstep: each step runs over all N values, so the dependent adds of one value are N instructions apart
// (no DPP read-after-write waits, N chains in flight)
template <int N>
__device__ __forceinline__ void row_scan16(float* x) {
#pragma unroll
    for (int n = 0; n < N; ++n) x[n] = x[n] + dpp<0x111, true>(x[n]);
#pragma unroll
    for (int n = 0; n < N; ++n) x[n] = x[n] + dpp<0x112, true>(x[n]);
#pragma unroll
    for (int n = 0; n < N; ++n) x[n] = x[n] + dpp<0x114, true>(x[n]);
#pragma unroll
    for (int n = 0; n < N; ++n) x[n] = x[n] + dpp<0x118, true>(x[n]);
}
__device__ __forceinline__ float bcast15(float x) { return dpp<0x15F, false>(x); }  // row_newbcast:15
__device__ __forceinline__ float shr1(float x) { return dpp<0x111, true>(x); }

__device__ __forceinline__ void lds_wait_all() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Ring flags, read and written as LDS accesses (ds_read / ds_write).  Through a generic volatile pointer they would
// compile to flat accesses that also count on vmcnt, so every flag store would wait for the wavefront's outstanding
// global stores.
typedef __attribute__((address_space(3))) volatile int lds_vint;
__device__ __forceinline__ int lds_load(const int* p) { return *(const lds_vint*)(p); }
__device__ __forceinline__ void lds_store(int* p, int v) { *(lds_vint*)(p) = v; }
__device__ __forceinline__ void vmem_wait_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Exchange between workgroups.  Every word of an exchange entry is written and read as a relaxed agent-scope atomic,
// which is coherent across the device by itself (no cache maintenance); a writer waits for its stores to complete
// before its flag store, and a reader issues its loads only after its flag load returned.  Agent-scope fences would
// write back / invalidate a whole L2 per call and cost microseconds each.
__device__ __forceinline__ void xstore(f4* dst, f4 x) {
    uint64_t* d = reinterpret_cast<uint64_t*>(dst);
    const uint64_t a = __builtin_bit_cast(uint64_t, f2_t{x[0], x[1]}), b = __builtin_bit_cast(uint64_t, f2_t{x[2], x[3]});
    __hip_atomic_store(d, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(d + 1, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f4 xload(const f4* src) {
    const uint64_t* s = reinterpret_cast<const uint64_t*>(src);
    const f2_t a = __builtin_bit_cast(f2_t, __hip_atomic_load(s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const f2_t b = __builtin_bit_cast(f2_t, __hip_atomic_load(s + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    return f4{a[0], a[1], b[0], b[1]};
}

__device__ __forceinline__ bf8 as_bf8(uint4 x) { return __builtin_bit_cast(bf8, x); }
__device__ __forceinline__ uint4 as_u4(bf8 x) { return __builtin_bit_cast(uint4, x); }

// ------------------------------------------------------------------------------------------------------------------
// Units.  Each head's owned rows, in row order, form a stream of chunks: a row of L tokens has max(1, ceil(L / 32))
// of them (an empty row's one chunk holds no token and passes its state through).  A unit (one workgroup) takes one
// head's stream chunks [c0, c1):
//   * dense calls (every row T tokens, no n_keep): the segments of one row, seg_start's split;
//   * ragged and n_keep calls: equal shares of the stream, ceil(chunks / units per head) each (at least
//     kSegMinChunks), which may cross rows, so that every CU gets the same work whatever the row lengths.
// The unit's first piece (the chunks of its first row) continues a row an earlier unit started when c0 is inside
// that row ("P mode": it starts from zeros, carries P, and its outputs are corrected once the row's state at c0 is
// known); every later row of the unit starts inside it, from the row's initial state.  A row spanning the units
// k0 < .. < km of a head is handed on through their exchange entries: k0 publishes its true end state, k0+1 .. km-1
// their local end states and P; unit k reads the entries of k0 .. k-1 (lower workgroup indices: dispatched first).
// ------------------------------------------------------------------------------------------------------------------

// Rows this launch owns: every row when p.rec_max_len < 0, else rows longer than it (the token-serial kernel takes
// the others).
__device__ __forceinline__ bool owns(const Params& p, int L) { return p.rec_max_len < 0 || L > p.rec_max_len; }
__device__ __forceinline__ int row_chunks(int L) { return L > 0 ? (L + SC - 1) / SC : 1; }

struct Row {   // an owned row: stream chunks [first, first + nch), tokens [bos, bos + L)
    int n, nch, L;
    int64_t first, bos;
};

struct Unit {
    bool ok;
    bool dense;
    int h;
    int64_t k;              // unit index within the head; exchange slot and workgroup index k * H + h
    int64_t c0, c1;         // stream chunks of the unit
    int nch, nseg, first;   // dense: chunks per row, segments per row, chunks of a row's first segment
    int64_t seg;            // ragged: stream chunks per unit
    int N;                  // ragged: rows of the call (the LDS table's length)
};

__device__ __forceinline__ Row row_dense(const Params& p, const Unit& U, int64_t c) {
    Row r;
    r.n = (int)(c / U.nch);
    r.nch = U.nch;
    r.first = (int64_t)r.n * U.nch;
    r.bos = (int64_t)r.n * p.T;
    r.L = p.T;
    return r;
}
__device__ __forceinline__ Row row_ragged(const Params& p, const int* rows, int n) {
    Row r;
    r.n = n;
    r.first = rows[n];
    r.nch = rows[n + 1] - rows[n];
    seq_extent(p, n, r.bos, r.L);
    return r;
}
// the owned row holding stream chunk c
__device__ Row row_at(const Params& p, const Unit& U, const int* rows, int64_t c) {
    if (U.dense) return row_dense(p, U, c);
    int lo = 0, hi = U.N - 1;  // the last n with rows[n] <= c (then rows[n + 1] > c: row n owns chunks)
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (rows[mid] <= c) lo = mid; else hi = mid - 1;
    }
    return row_ragged(p, rows, lo);
}
// the owned row after r (called only while r ends before the unit's last chunk, so one exists)
__device__ Row next_row(const Params& p, const Unit& U, const int* rows, const Row& r) {
    if (U.dense) return row_dense(p, U, r.first + r.nch);
    int n = r.n + 1;
    while (rows[n + 1] == rows[n]) ++n;  // rows without chunks (not owned)
    return row_ragged(p, rows, n);
}
// the units of the head holding row r's first and last chunks
__device__ __forceinline__ int64_t first_unit(const Unit& U, const Row& r) {
    return U.dense ? (int64_t)r.n * U.nseg : r.first / U.seg;
}
__device__ __forceinline__ int64_t last_unit(const Unit& U, const Row& r) {
    return U.dense ? (int64_t)r.n * U.nseg + U.nseg - 1 : (r.first + r.nch - 1) / U.seg;
}

// Exclusive prefix sum of x over the workgroup's 512 threads (tmp: 8 ints of LDS); *total gets the sum.
__device__ int block_excl_scan(int x, int* tmp, int* total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int incl = x;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(incl, d);
        if (lane >= d) incl += y;
    }
    if (lane == 63) tmp[wv] = incl;
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        const int t = tmp[w];
        off += w < wv ? t : 0;
        tot += t;
    }
    __syncthreads();
    *total = tot;
    return off + incl - x;
}

// The unit of workgroup blk.  Ragged and n_keep calls first build the row table in LDS with every thread:
// rows[n] = the first stream chunk of row n (rows[N] = the stream's length), N <= kSegMaxRows.
__device__ Unit find_unit(const Params& p, int seg, int64_t blk, int* rows, int* tmp) {
    Unit U{};
    const int H = p.H;
    U.k = blk / H;
    U.h = (int)(blk - U.k * H);
    if (!p.cu && !p.n_keep) {
        U.dense = true;
        if (!owns(p, p.T)) return U;
        U.nch = row_chunks(p.T);
        U.nseg = std::max(1, (U.nch + seg - 1) / seg);
        U.first = seg_start(U.nch, U.nseg, 1);
        const int64_t n = U.k / U.nseg;
        if (n >= p.num_seqs) return U;
        const int s = (int)(U.k - n * U.nseg);
        U.c0 = n * U.nch + seg_start(U.nch, U.nseg, s);
        U.c1 = n * U.nch + seg_start(U.nch, U.nseg, s + 1);
    } else {
        const int N = p.num_seqs, tid = threadIdx.x;
        const int per = (N + 511) / 512;
        const int r0 = min(N, tid * per), r1 = min(N, r0 + per);
        int a = 0;
        for (int n = r0; n < r1; ++n) {
            int64_t bos;
            int L;
            seq_extent(p, n, bos, L);
            rows[n] = owns(p, L) ? row_chunks(L) : 0;
            a += rows[n];
        }
        int total;
        int off = block_excl_scan(a, tmp, &total);
        for (int n = r0; n < r1; ++n) {
            const int x = rows[n];
            rows[n] = off;
            off += x;
        }
        if (tid == 0) rows[N] = total;
        __syncthreads();
        U.N = N;
        const int64_t per_head = std::max<int64_t>(1, (int64_t)gridDim.x / H);
        U.seg = std::max<int64_t>(kSegMinChunks, (total + per_head - 1) / per_head);
        U.c0 = U.k * U.seg;
        U.c1 = std::min<int64_t>(U.c0 + U.seg, total);
    }
    U.ok = U.c0 < U.c1;
    return U;
}

// ------------------------------------------------------------------------------------------------------------------
// Prep wavefront: one chunk -> record
// ------------------------------------------------------------------------------------------------------------------

struct Raw {
    uint4 w[2][2], a[2][2], b[2][2], k[2][2], r[2][2], v[2][2];  // N layout [token tile][channel block]
};

// A wave-uniform raw buffer over [base, base + bytes) for the chunk operand loads and output stores: accesses past
// `bytes` read zeros and drop their writes.  readfirstlane returns int: each half goes through uint32_t, so that the
// low one is not sign-extended.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(uint64_t base, int bytes) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0,
                                             __builtin_amdgcn_readfirstlane(bytes), 0x00020000 /* raw 32-bit buffer */);
}

// The chunk's operands, token rows 16 tau + i, head h, channels 32 kb + 8 q ..: each through a buffer that ends after
// the chunk's last valid token, so rows t >= Lc (and every row of an empty row's chunk) read zeros.  Offsets are
// 32-bit: the launch requires in_tok_stride <= kSegMaxTokStride.
__device__ __forceinline__ void load_raw(Raw& x, const Params& p, int64_t tok0, int Lc, int h, int lane) {
    const int i = lane & 15, q = lane >> 4;
    const int64_t e0 = tok0 * p.in_tok_stride + (int64_t)h * HS;
    const int bytes = Lc > 0 ? (Lc - 1) * (int)p.in_tok_stride * 2 + HS * 2 : 0;
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc((uint64_t)(p.w + e0), bytes), ra = buf_rsrc((uint64_t)(p.a + e0), bytes),
                                 rb = buf_rsrc((uint64_t)(p.b + e0), bytes), rk = buf_rsrc((uint64_t)(p.k + e0), bytes),
                                 rr = buf_rsrc((uint64_t)(p.r + e0), bytes), rv = buf_rsrc((uint64_t)(p.v + e0), bytes);
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int off = ((16 * tau + i) * (int)p.in_tok_stride + 8 * q + 32 * kb) * 2;
            x.w[tau][kb] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 0));
            x.a[tau][kb] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0));
            x.b[tau][kb] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0));
            x.k[tau][kb] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
            x.r[tau][kb] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rr, off, 0, 0));
            x.v[tau][kb] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
        }
    }
}

__device__ __forceinline__ void unpack8(uint4 x, float (&f)[8]) {
    bf16x2_to_f32(x.x, f[0], f[1]);
    bf16x2_to_f32(x.y, f[2], f[3]);
    bf16x2_to_f32(x.z, f[4], f[5]);
    bf16x2_to_f32(x.w, f[6], f[7]);
}
// fp32 x 8 -> hi / lo bf16 x 8
__device__ __forceinline__ void split8(const float (&f)[8], bf8& h, bf8& l) {
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) split_pair(f[2 * e], f[2 * e + 1], hw[e], lw[e]);
    h = __builtin_bit_cast(bf8, hw);
    l = __builtin_bit_cast(bf8, lw);
}
__device__ __forceinline__ bf8 hi8(const float (&f)[8]) {
    uint32_t hw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) hw[e] = pack_bf16x2(f[2 * e], f[2 * e + 1]);
    return __builtin_bit_cast(bf8, hw);
}

// 2^m etc. of channel ch, this wavefront's chunk
struct Fac {
    const float* em;   // 2^m
    const float* ecm;  // 2^{c-m}
    const float* ec;   // 2^c
};

// The transition of one chunk into `rec` (an LDS ring slot), after waiting for that slot to be free.
__device__ __forceinline__ void prep_chunk(const Raw& raw, int Lc, char* rec, float (*fac)[HS], int lane,
                                           const int* done4, int use, int* fail) {
    const int i = lane & 15, q = lane >> 4;

    // ---- 1. log2-decays lam = log2 d = -e^w log2(e) and their running sums over the chunk's tokens.  Lanes i of
    //         a row hold tokens 16 tau + i of the row's 8 channels; every sum is a fixed sequence of row_shr adds, so
    //         the midpoint m (token 15) and the total c (token 31) equal the g of those tokens bit for bit.
    float g[2][2][8];
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) {
        const bool valid = 16 * tau + i < Lc;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            float w8[8];
            unpack8(raw.w[tau][kb], w8);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float lam = -__builtin_amdgcn_exp2f(w8[e] * kL2E) * kL2E;
                g[tau][kb][e] = valid ? lam : 0.f;
            }
        }
    }
    row_scan16<32>(&g[0][0][0]);
    float m[2][8], c[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            m[kb][e] = bcast15(g[0][kb][e]);
            g[1][kb][e] += m[kb][e];
            c[kb][e] = bcast15(g[1][kb][e]);
        }
    // per-channel factors for the products' row/column scalings: the lanes i == 0, which hold every channel's m and c
    // once, park them in fac[0] and fac[1]; lane l then turns channel l's into 2^m, 2^{c-m}, 2^c and 2^{-m} (four
    // quarter-rate exponentials a lane instead of 48 on every lane, most of them masked off)
    if (i == 0) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int h4 = 0; h4 < 2; ++h4) {
                const int ch = 32 * kb + 8 * q + 4 * h4;
                *reinterpret_cast<f4*>(&fac[0][ch]) = f4{m[kb][4 * h4], m[kb][4 * h4 + 1], m[kb][4 * h4 + 2], m[kb][4 * h4 + 3]};
                *reinterpret_cast<f4*>(&fac[1][ch]) = f4{c[kb][4 * h4], c[kb][4 * h4 + 1], c[kb][4 * h4 + 2], c[kb][4 * h4 + 3]};
            }
    }
    wave_lds_sync();
    {
        const float ml = fac[0][lane], cl = fac[1][lane];
        fac[0][lane] = __builtin_amdgcn_exp2f(ml);
        fac[1][lane] = __builtin_amdgcn_exp2f(cl - ml);
        fac[2][lane] = __builtin_amdgcn_exp2f(cl);
        fac[3][lane] = __builtin_amdgcn_exp2f(-ml);
    }
    wave_lds_sync();

    // ---- 2. operands referenced to the midpoint (N layout), split hi/lo
    bf8 Ah[2][2], Al[2][2], Bh[2][2], Bl[2][2], Kh[2][2], Kl[2][2], Rh[2][2], Vn[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        float fr0[8], fm[8];  // (tau = 1) token 15's 2^{g-m}; 2^{-m} of the lane's 8 channels
        {
            const f4 f0 = *reinterpret_cast<const f4*>(&fac[3][32 * kb + 8 * q]);
            const f4 f1 = *reinterpret_cast<const f4*>(&fac[3][32 * kb + 8 * q + 4]);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                fm[v] = f0[v];
                fm[4 + v] = f1[v];
            }
        }
#pragma unroll
        for (int tau = 0; tau < 2; ++tau) {
            float a8[8], b8[8], k8[8], r8[8];  // zero past the chunk's valid tokens (load_raw)
            unpack8(raw.a[tau][kb], a8);
            unpack8(raw.b[tau][kb], b8);
            unpack8(raw.k[tau][kb], k8);
            unpack8(raw.r[tau][kb], r8);
            float fa[8], fr[8], fb[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float d = g[tau][kb][e] - m[kb][e];
                fr[e] = __builtin_amdgcn_exp2f(d);
                fb[e] = __builtin_amdgcn_exp2f(-d);
                const float prev = shr1(fr[e]);  // token t - 1 of the row (lane 0 reads 0)
                const float first = tau == 0 ? fm[e] : bcast15(fr0[e]);
                fa[e] = bitsel(i == 0 ? 0xffffffffu : 0u, first, prev);
            }
            if (tau == 0)
#pragma unroll
                for (int e = 0; e < 8; ++e) fr0[e] = fr[e];
            float x8[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x8[e] = a8[e] * fa[e];
            split8(x8, Ah[tau][kb], Al[tau][kb]);
#pragma unroll
            for (int e = 0; e < 8; ++e) x8[e] = b8[e] * fb[e];
            split8(x8, Bh[tau][kb], Bl[tau][kb]);
#pragma unroll
            for (int e = 0; e < 8; ++e) x8[e] = k8[e] * fb[e];
            split8(x8, Kh[tau][kb], Kl[tau][kb]);
#pragma unroll
            for (int e = 0; e < 8; ++e) x8[e] = r8[e] * fr[e];
            Rh[tau][kb] = hi8(x8);
            Vn[tau][kb] = as_bf8(raw.v[tau][kb]);
        }
    }

    // ---- 3. Grams (RL tiles, rows s, columns t): alphaT = Bp Ah^T, betaT = Kp Ah^T (s < t), rhoT = Bp Rh^T,
    //         sigmaT = Kp Rh^T (s <= t).  Tiles (s tile, t tile) = (0,0), (0,1), (1,1); (1,0) is zero.
    f4 aT[3], bT[3], rT[3], sT[3];
    {
        const int st[3] = {0, 0, 1}, tt[3] = {0, 1, 1};
#pragma unroll
        for (int x = 0; x < 3; ++x) {
            f4 a = z4(), b = z4(), r = z4(), s = z4();
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const bf8 bh = Bh[st[x]][kb], bl = Bl[st[x]][kb], kh = Kh[st[x]][kb], kl = Kl[st[x]][kb];
                const bf8 ah = Ah[tt[x]][kb], al = Al[tt[x]][kb], rh = Rh[tt[x]][kb];
                a = mma32(bh, al, a);
                a = mma32(bl, ah, a);
                a = mma32(bh, ah, a);
                b = mma32(kh, al, b);
                b = mma32(kl, ah, b);
                b = mma32(kh, ah, b);
                r = mma32(bh, rh, r);
                s = mma32(kh, rh, s);
            }
            if (st[x] == tt[x]) {
                a = keep_upper(a, lane, true);
                b = keep_upper(b, lane, true);
                r = keep_upper(r, lane, false);
                s = keep_upper(s, lane, false);
            }
            aT[x] = a;
            bT[x] = b;
            rT[x] = r;
            sT[x] = s;
        }
    }

    // ---- 4. T^T = (I - alpha^T)^{-1} by 16 x 16 blocks: T_dd = (I + L)(I + L^2)(I + L^4)(I + L^8) with L = alpha_dd
    //         strictly lower (L^16 = 0); products in the RL form X^T Y, so powers of L and L^T feed each other.
    //         T10 = T11 alpha10 T00, so (T^T)_01 = T10^T = (alpha10 T00)^T T11^T.
    const s4 Id = ident16(lane);
    T4 tt00, tt01, tt11;
    {
        T4 TT[2], T00;
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            const f4 LTf = aT[d == 0 ? 0 : 2];                                 // RL(L^T)
            const T4 LT = split_t(LTf);
            const f4 LLf = mma16(LT.l, Id, mma16(LT.h, Id, z4()));            // RL(L): transpose, exact
            const T4 LL = split_t(LLf);
            const f4 L2f = p16x3(LT, LL, z4()), L2tf = p16x3(LL, LT, z4());
            const T4 L2 = split_t(L2f), L2t = split_t(L2tf);
            const f4 L4f = p16x3(L2t, L2, z4()), L4tf = p16x3(L2, L2t, z4());
            const T4 L4 = split_t(L4f), L4t = split_t(L4tf);
            const f4 L8f = p16x3(L4t, L4, z4());
            // T^T = (I + L^T)(I + L^2T)(I + L^4T)(I + L^8T) as X^T Y products with X = I + L^{2^k}; the diagonals of
            // the powers are zero, so adding I is exact
            T4 acc = split_t(p16x3(split_t(plus_i(LLf, lane)), split_t(plus_i(L2tf, lane)), z4()));
            acc = split_t(p16x3(split_t(plus_i(L4f, lane)), acc, z4()));
            TT[d] = split_t(p16x3(split_t(plus_i(L8f, lane)), acc, z4()));
            if (d == 0)  // T00 itself, for the off-diagonal block: the transpose of T00^T (hi and lo, exact)
                T00 = split_t(mma16(TT[0].l, Id, mma16(TT[0].h, Id, z4())));
        }
        const T4 Z = split_t(p16x3(split_t(aT[1]), T00, z4()));  // alpha10 T00
        tt00 = TT[0];
        tt11 = TT[1];
        tt01 = split_t(p16x3(Z, TT[1], z4()));
    }
    const T8 ttp = cat(tt01, tt11);  // rows s 0-31 of (T^T)'s token tile 1

    // ---- 5. token-row RL tiles (token tile tau, channel tile j) through identity MFMAs (exact): V now, the others
    //         on the fly below.
    const bf8 I0 = isel(0, lane), I1 = isel(1, lane);
    s4 rV[2][4];
#pragma unroll
    for (int tau = 0; tau < 2; ++tau)
#pragma unroll
        for (int j = 0; j < 4; ++j) rV[tau][j] = hi_t(mma32(Vn[tau][j >> 1], (j & 1) ? I1 : I0, z4()));
    auto rl = [&](const bf8 (&H8)[2][2], const bf8 (&L8)[2][2], int tau, int j) {
        const bf8 I = (j & 1) ? I1 : I0;
        return T4{hi_t(mma32(H8[tau][j >> 1], I, z4())), hi_t(mma32(L8[tau][j >> 1], I, z4()))};
    };

    // ---- 6. wait for the ring slot
    {
        bool ok = false;
        for (int it = 0; it < kSpinLimit; ++it) {
            const int d0 = lds_load(done4 + 0), d1 = lds_load(done4 + 1), d2 = lds_load(done4 + 2), d3 = lds_load(done4 + 3);
            if (min(min(d0, d1), min(d2, d3)) >= use) {
                ok = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (!ok) *fail = 1;
        asm volatile("" ::: "memory");
    }
    uint4* const R = reinterpret_cast<uint4*>(rec);

    // ---- 7. per channel tile j: W^T = diag(2^m) (T Ah)^T (RL tiles (j, token tile): the record's X = W S operand),
    //         U0 = T (beta V) and V (RL tiles (token tile, j)), R0^T = diag(2^m) Rh^T (tiles (j, token tile)), all
    //         stored
    f4 emr[4];  // 2^m of rows 16 j + 4 q + v, read in one batch ahead of the record stores
#pragma unroll
    for (int j = 0; j < 4; ++j) emr[j] = *reinterpret_cast<const f4*>(&fac[0][16 * j + 4 * q]);
    {
        const T4 b00 = split_t(bT[0]);
        const T8 bp = cat(split_t(bT[1]), split_t(bT[2]));
        const s4 r00 = hi_t(rT[0]), s00 = hi_t(sT[0]);
        const bf8 rp = cat(hi_t(rT[1]), hi_t(rT[2])), sp = cat(hi_t(sT[1]), hi_t(sT[2]));
        T4 Wtt[4][2];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const T4 a0 = rl(Ah, Al, 0, j), a1 = rl(Ah, Al, 1, j);
            f4 w0 = p16x3(a0, tt00, z4()), w1 = p32x3(cat(a0, a1), ttp, z4());
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                w0[v] *= emr[j][v];
                w1[v] *= emr[j][v];
            }
            Wtt[j][0] = split_t(w0);
            Wtt[j][1] = split_t(w1);
            const T4 bv0 = split_t(p16x2(b00, rV[0][j], z4()));
            const T4 bv1 = split_t(p32x2(bp, cat(rV[0][j], rV[1][j]), z4()));
            const f4 u0f = p16x3(tt00, bv0, z4()), u1f = p32x3(ttp, cat(bv0, bv1), z4());
            const bf8 I = (j & 1) ? I1 : I0;
            f4 q0 = mma32(I, Rh[0][j >> 1], z4()), q1 = mma32(I, Rh[1][j >> 1], z4());
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                q0[v] *= emr[j][v];
                q1[v] *= emr[j][v];
            }
            // R0^T pieces [token tile][kb]: k tiles j = 2 kb, 2 kb + 1 in the low / high 8 bytes
            reinterpret_cast<uint2*>(R + (REC_R / 16) + (0 * 2 + (j >> 1)) * 64 + lane)[j & 1] = __builtin_bit_cast(uint2, hi_t(q0));
            reinterpret_cast<uint2*>(R + (REC_R / 16) + (1 * 2 + (j >> 1)) * 64 + lane)[j & 1] = __builtin_bit_cast(uint2, hi_t(q1));
            R[(REC_U / 16) + (j * 2 + 0) * 64 + lane] = __builtin_bit_cast(uint4, u0f);
            R[(REC_U / 16) + (j * 2 + 1) * 64 + lane] = __builtin_bit_cast(uint4, u1f);
            R[(REC_V / 16) + j * 64 + lane] = as_u4(cat(rV[0][j], rV[1][j]));
        }
        // W^T pieces [token tile][kb][hl]: k tiles 2 kb, 2 kb + 1 stacked
#pragma unroll
        for (int tau = 0; tau < 2; ++tau)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const T8 pc = cat(Wtt[2 * kb][tau], Wtt[2 * kb + 1][tau]);
                R[(REC_W / 16) + ((tau * 2 + kb) * 2 + 0) * 64 + lane] = as_u4(pc.h);
                R[(REC_W / 16) + ((tau * 2 + kb) * 2 + 1) * 64 + lane] = as_u4(pc.l);
            }
        // rho^T and sigma^T pieces for y's U^T rho^T and V^T sigma^T terms
        R[(REC_RHO / 16) + lane] = as_u4(cat(r00, s4{0, 0, 0, 0}));
        R[(REC_RHO / 16) + 64 + lane] = as_u4(rp);
        R[(REC_SIG / 16) + lane] = as_u4(cat(s00, s4{0, 0, 0, 0}));
        R[(REC_SIG / 16) + 64 + lane] = as_u4(sp);
        // Gamma per channel
        if (lane < 16)
            reinterpret_cast<f4*>(rec + REC_G)[lane] = *reinterpret_cast<const f4*>(&fac[2][4 * lane]);
    }

    // ---- 8. per k tile m: Bp and Kp as token-row RL tiles (the transposes of their hi and lo parts, each exact),
    //         stored with the row factors 2^{c-m}
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const T8 bpm = cat(rl(Bh, Bl, 0, m), rl(Bh, Bl, 1, m));
        R[(REC_B / 16) + (m * 2 + 0) * 64 + lane] = as_u4(bpm.h);
        R[(REC_B / 16) + (m * 2 + 1) * 64 + lane] = as_u4(bpm.l);
        const T8 kpm = cat(rl(Kh, Kl, 0, m), rl(Kh, Kl, 1, m));
        R[(REC_K / 16) + (m * 2 + 0) * 64 + lane] = as_u4(kpm.h);
        R[(REC_K / 16) + (m * 2 + 1) * 64 + lane] = as_u4(kpm.l);
    }
    if (lane < 16) reinterpret_cast<f4*>(rec + REC_F)[lane] = *reinterpret_cast<const f4*>(&fac[1][4 * lane]);
}

// ------------------------------------------------------------------------------------------------------------------
// State wavefront
// ------------------------------------------------------------------------------------------------------------------

// the state's 16x16x32 operands: contraction block kb stacks k tiles 2 kb and 2 kb + 1 of column tile j
__device__ __forceinline__ void state_ops(const f4 (&S)[4], T8 (&o)[2]) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) o[kb] = cat(split_t(S[2 * kb]), split_t(S[2 * kb + 1]));
}

// y^T tiles (column tile j, token tiles 0, 1) of a chunk's first Lc tokens as bf16, through a raw buffer that covers
// exactly those tokens' rows (head h, columns 16 j ..): the stores of rows t >= Lc fall outside it and are dropped,
// and so are all of them without an output (an empty range), so no branch splits the caller's code.  Offsets are
// 32-bit: the launch requires o_tok_stride <= kSegMaxTokStride.
__device__ __forceinline__ void store_y(const Params& p, int64_t tok0, int Lc, int h, int j, int lane, const f4 (&y)[2]) {
    const int i = lane & 15, q = lane >> 4;
    const int stride2 = (int)p.o_tok_stride * 2;
    const uint64_t base = p.o ? (uint64_t)(p.o + tok0 * p.o_tok_stride + (int64_t)h * HS + 16 * j) : 0;
    const int bytes = (p.o && Lc > 0) ? (Lc - 1) * stride2 + 32 : 0;
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(base, bytes);
#pragma unroll
    for (int tau = 0; tau < 2; ++tau) {
        uint2 pk;
        pk.x = pack_bf16x2(y[tau][0], y[tau][1]);
        pk.y = pack_bf16x2(y[tau][2], y[tau][3]);
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2v, pk), rs, (16 * tau + i) * stride2 + 8 * q, 0, 0);
    }
}

}  // namespace

// One unit: its chunks' main loop (prep and state wavefronts) and the end phase (hand-off, correction).
__device__ __forceinline__ void run_unit(const Params& p, const Unit& U, int32_t* __restrict__ flags,
                                         float* __restrict__ xbuf, char* __restrict__ qpbuf, SegSmem& sm) {
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15, q = lane >> 4;
    const int H = p.H, h = U.h;
    const int64_t uid = blockIdx.x;
    if (tid < NREC) sm.ready[tid] = 0;
    if (tid < NREC * 4) (&sm.done[0][0])[tid] = 0;
    if (tid == 0) sm.fail = 0;
    __syncthreads();
    const int nloc = (int)(U.c1 - U.c0);  // chunks of this unit
    const Row A = row_at(p, U, sm.rows, U.c0);  // the unit's first row
    const bool pmodeA = U.c0 > A.first;       // ... continued from an earlier unit
    // Q P record of stream chunk c of the first row (P mode only): dense calls number a row's chunks after its
    // first segment, ragged calls the stream's chunks
    auto qp_slot = [&](int64_t c) -> uint4* {
        const int64_t slot = U.dense ? (int64_t)A.n * (U.nch - U.first) + (c - A.first - U.first) : c;
        return reinterpret_cast<uint4*>(qpbuf + (slot * H + h) * (int64_t)(4 * 1024));
    };
    // exchange entry e: its local end state [m][j][lane], then (P mode) its P^T [j][m][lane]
    auto xs_of = [&](int64_t e) { return reinterpret_cast<f4*>(xbuf + e * (int64_t)(2 * HS2)); };

    f4 S[4], P[4];  // state wavefronts: column tile j of S and of P
    if (wv < 4) {
        // ---------------- prep wavefronts: chunks cl = wv, wv + 4, ..
        Row r = A;
        for (int cl = wv; cl < nloc; cl += 4) {
            const int64_t c = U.c0 + cl;
            while (c >= r.first + r.nch) r = next_row(p, U, sm.rows, r);
            const int ci = (int)(c - r.first);
            const int64_t tok0 = r.bos + (int64_t)ci * SC;
            const int Lc = (int)std::max<int64_t>(0, std::min<int64_t>(SC, r.L - (int64_t)ci * SC));
            Raw raw;
            load_raw(raw, p, tok0, Lc, h, lane);
            const int slot = cl % NREC;
            prep_chunk(raw, Lc, sm.ring[slot], sm.fac[wv], lane, sm.done[slot], cl / NREC, &sm.fail);
            lds_wait_all();
            if (lane == 0) lds_store(&sm.ready[slot], cl + 1);
        }
    } else {
        // ---------------- state wavefronts: columns 16 j .. 16 j + 15
        const int j = wv - 4;
        // a row's initial / final state (true mode): RL tiles (m, j), element (16 m + 4 q + v, 16 j + i), addressed
        // from one per-lane pointer (precomputed 64-bit element offsets would spill)
        const int lane_off = 4 * q * HS + 16 * j + i;
        auto load_state = [&](const Row& rr) {
            const float* src = state_src(p, rr.n, h);
            if (src) {
                const float* s0 = src + lane_off;
#pragma unroll
                for (int m = 0; m < 4; ++m)
#pragma unroll
                    for (int v = 0; v < 4; ++v) S[m][v] = s0[(16 * m + v) * HS];
            } else {
#pragma unroll
                for (int m = 0; m < 4; ++m) S[m] = z4();
            }
        };
        auto store_state = [&](const Row& rr) {
            float* const dst = state_dst(p, rr.n, h);
            if (dst) {
                float* const d0 = dst + lane_off;
#pragma unroll
                for (int m = 0; m < 4; ++m)
#pragma unroll
                    for (int v = 0; v < 4; ++v) d0[(16 * m + v) * HS] = S[m][v];
            }
        };
        Row r = A;
        // chunk cl of row r.  PM: P mode (S starts at zero, P = A_c .. A_1 accumulates, (Q P)^T goes out for the
        // output correction).  After the record wait the step is one basic block (the output stores are masked by
        // their buffer range, not by branches), so the S and P chains of a P-mode chunk schedule together.
        auto chunk = [&](auto pm, const int cl) {
            constexpr bool PM = decltype(pm)::value;
            const int64_t c = U.c0 + cl;
            const int slot = cl % NREC;
            {
                bool ok = false;
                for (int it = 0; it < kSpinLimit; ++it) {
                    if (lds_load(&sm.ready[slot]) == cl + 1) {
                        ok = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                if (!ok) sm.fail = 1;
                asm volatile("" ::: "memory");
            }
            const uint4* const R = reinterpret_cast<const uint4*>(sm.ring[slot]);
            uint4 rw[2][2][2], rb[4][2], rk[4][2], rr[2][2], rho[2], sig[2], rv;
            f4 ru[2], gm[4], cf[4];
#pragma unroll
            for (int tau = 0; tau < 2; ++tau)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int hl = 0; hl < 2; ++hl) rw[tau][kb][hl] = R[(REC_W / 16) + ((tau * 2 + kb) * 2 + hl) * 64 + lane];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
#pragma unroll
                for (int hl = 0; hl < 2; ++hl) {
                    rb[m][hl] = R[(REC_B / 16) + (m * 2 + hl) * 64 + lane];
                    rk[m][hl] = R[(REC_K / 16) + (m * 2 + hl) * 64 + lane];
                }
                gm[m] = reinterpret_cast<const f4*>(sm.ring[slot] + REC_G)[4 * m + q];  // 2^c of rows 16 m + 4 q + v
                cf[m] = reinterpret_cast<const f4*>(sm.ring[slot] + REC_F)[4 * m + q];  // 2^{c-m}, same rows
            }
#pragma unroll
            for (int tau = 0; tau < 2; ++tau) {
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) rr[tau][kb] = R[(REC_R / 16) + (tau * 2 + kb) * 64 + lane];
                ru[tau] = __builtin_bit_cast(f4, R[(REC_U / 16) + (j * 2 + tau) * 64 + lane]);
                rho[tau] = R[(REC_RHO / 16) + tau * 64 + lane];
                sig[tau] = R[(REC_SIG / 16) + tau * 64 + lane];
            }
            rv = R[(REC_V / 16) + j * 64 + lane];
            lds_wait_all();
            if (lane == 0) lds_store(&sm.done[slot][j], cl / NREC + 1);

            const int ci = (int)(c - r.first);
            const int64_t tok0 = r.bos + (int64_t)ci * SC;
            const int Lc = (int)std::max<int64_t>(0, std::min<int64_t>(SC, r.L - (int64_t)ci * SC));
            // X = W M (token tiles 0, 1; columns 16 j ..) for M = S or P
            auto wmul = [&](const T8 (&mo)[2], f4 (&X)[2]) {
#pragma unroll
                for (int tau = 0; tau < 2; ++tau) {
                    f4 x = z4();
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
                        x = p32x3(T8{as_bf8(rw[tau][kb][0]), as_bf8(rw[tau][kb][1])}, mo[kb], x);
                    X[tau] = x;
                }
            };
            // M <- Gamma M + diag(2^{c-m}) (Bp^T X (+ Kp^T V for the state))
            auto apply = [&](f4 (&M)[4], const f4 (&X)[2], bool state) {
                const T8 xo = cat(split_t(X[0]), split_t(X[1]));
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    f4 x = z4();
                    if (state) x = p32x2(T8{as_bf8(rk[m][0]), as_bf8(rk[m][1])}, as_bf8(rv), x);
                    x = p32x3(T8{as_bf8(rb[m][0]), as_bf8(rb[m][1])}, xo, x);
#pragma unroll
                    for (int v = 0; v < 4; ++v) M[m][v] = fmaf(cf[m][v], x[v], gm[m][v] * M[m][v]);
                }
            };
            // (R0 M + rho X)^T tiles (column tile j, token tile): y^T for M = S, X = U, (Q P)^T for M = P, X = W P
            auto qmul = [&](const T8 (&mo)[2], const f4 (&X)[2], f4 (&Y)[2]) {
                const s4 x0 = hi_t(X[0]), x1 = hi_t(X[1]);
                Y[0] = mma16(x0, __builtin_bit_cast(s4, uint2{rho[0].x, rho[0].y}), Y[0]);  // tile (0, 0): low 8 bytes
                Y[1] = mma32(cat(x0, x1), as_bf8(rho[1]), Y[1]);
#pragma unroll
                for (int tau = 0; tau < 2; ++tau)
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb) Y[tau] = mma32(mo[kb].h, as_bf8(rr[tau][kb]), Y[tau]);
            };
            T8 so[2];
            state_ops(S, so);
            f4 X[2];
            wmul(so, X);
#pragma unroll
            for (int tau = 0; tau < 2; ++tau) X[tau] += ru[tau];  // U = W S + U0
            f4 y[2] = {z4(), z4()};
            {  // V^T sigma^T
                const bf8 vp = as_bf8(rv);
                const s4 v0 = __builtin_bit_cast(s4, uint2{rv.x, rv.y});
                y[0] = mma16(v0, __builtin_bit_cast(s4, uint2{sig[0].x, sig[0].y}), y[0]);
                y[1] = mma32(vp, as_bf8(sig[1]), y[1]);
            }
            qmul(so, X, y);
            store_y(p, tok0, Lc, h, j, lane, y);
            if constexpr (PM) {
                T8 po[2];
                state_ops(P, po);
                f4 XP[2];
                wmul(po, XP);
                // (Q P)^T rows k' in column tile j, for the correction once S_in is known
                f4 qp[2] = {z4(), z4()};
                qmul(po, XP, qp);
                uint4* const dst = qp_slot(c);
#pragma unroll
                for (int tau = 0; tau < 2; ++tau) {
                    // piece [tau][kb = j >> 1], half j & 1
                    uint2* d2 = reinterpret_cast<uint2*>(dst + (tau * 2 + (j >> 1)) * 64 + lane) + (j & 1);
                    *d2 = __builtin_bit_cast(uint2, hi_t(qp[tau]));
                }
                apply(P, XP, false);
            }
            apply(S, X, true);
        };
        int cl = 0;
        if (pmodeA) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                S[m] = z4();
                P[m] = (m == j) ? plus_i(z4(), lane) : z4();
            }
            const int nA = (int)(std::min<int64_t>(U.c1, A.first + A.nch) - U.c0);
            for (; cl < nA; ++cl) chunk(std::true_type{}, cl);
            if (nA < nloc) {
                // row A ends here: park its local end state and P^T for the end phase
                f4* const xd = xs_of((int64_t)gridDim.x + uid);
                const s4 Id = ident16(lane);
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    xstore(xd + (m * 4 + j) * 64 + lane, S[m]);
                    const T4 x = split_t(P[m]);
                    xstore(xd + 16 * 64 + (j * 4 + m) * 64 + lane, mma16(x.l, Id, mma16(x.h, Id, z4())));
                }
                r = next_row(p, U, sm.rows, r);
                load_state(r);
            }
        } else {
            load_state(r);
        }
        for (; cl < nloc; ++cl) {
            if (U.c0 + cl >= r.first + r.nch) {  // row r ends here: its final state; the next starts from its initial
                store_state(r);
                r = next_row(p, U, sm.rows, r);
                load_state(r);
            }
            chunk(std::false_type{}, cl);
        }
        // the last row, if it ends here in true mode: its final state (P mode and rows continuing in later units are
        // finished in the end phase)
        if (U.c1 == r.first + r.nch && !(pmodeA && r.n == A.n)) store_state(r);
    }
    __syncthreads();  // every main loop done: the ring is free
    // ---------------- end phase: all eight wavefronts.  LDS (ring space): the first row's local end state and P^T,
    // then its S_in.  Row A (first) in P mode needs S_in; row Z (last) continuing past the unit is published.
    f4* const Sx = reinterpret_cast<f4*>(sm.ring[0]);  // S_local, [column tile j][k tile m][lane]
    f4* const Ptx = Sx + 16 * 64;                      // P^T, RL tiles [k' tile][k tile][lane]
    f4* const Sin = Ptx + 16 * 64;                     // S_in, [k tile m][column tile j][lane]
    const Row Z = row_at(p, U, sm.rows, U.c1 - 1);
    const bool cont = U.c1 < Z.first + Z.nch;  // row Z goes on in later units
    const bool one_row = A.n == Z.n;           // (then S and P in registers are row A's)
    if (wv >= 4) {
        const int j = wv - 4;
        const s4 Id = ident16(lane);
        if (pmodeA) {
            if (one_row) {
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    Sx[(j * 4 + m) * 64 + lane] = S[m];
                    const T4 x = split_t(P[m]);
                    Ptx[(j * 4 + m) * 64 + lane] = mma16(x.l, Id, mma16(x.h, Id, z4()));  // RL(P^T) tile (j, m)
                }
            } else {  // parked by this wavefront at the row switch
                vmem_wait_all();
                const f4* const st = xs_of((int64_t)gridDim.x + uid);
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    Sx[(j * 4 + m) * 64 + lane] = xload(st + (m * 4 + j) * 64 + lane);
                    Ptx[(j * 4 + m) * 64 + lane] = xload(st + 16 * 64 + (j * 4 + m) * 64 + lane);
                }
            }
        }
        if (cont) {  // publish row Z's entry: its end state here, and P^T when that is P-mode row A
            f4* const xd = xs_of(uid);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                xstore(xd + (m * 4 + j) * 64 + lane, S[m]);
                if (pmodeA && one_row) xstore(xd + 16 * 64 + (j * 4 + m) * 64 + lane, Ptx[(j * 4 + m) * 64 + lane]);
            }
            vmem_wait_all();
        }
    }
    __syncthreads();
    // every later unit holding row Z reads this entry once: the flag counts its readers down to zero
    if (cont && tid == 0)
        __hip_atomic_store(flags + uid, (int)(last_unit(U, Z) - U.k), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    if (pmodeA) {
        // S_in = row A's state at c0, by Horner over the entries of its earlier units k0 .. k - 1: X = S_end(k0);
        // X <- P X + S_local of each later one
        const int64_t k0 = first_unit(U, A);
        const int ns = (int)(U.k - k0);
        auto entry = [&](int jj) { return xs_of((k0 + jj) * H + h); };
        if (tid < ns) {
            int* const f = flags + (k0 + tid) * H + h;
            bool ok = false;
            for (int it = 0; it < kFlagSpinLimit; ++it) {
                if (__hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) > 0) {
                    ok = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            if (!ok) sm.fail = 1;
        }
        __syncthreads();
        if (wv >= 4) {
            const int j = wv - 4;
            f4 X[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) X[m] = xload(entry(0) + (m * 4 + j) * 64 + lane);
            // entries two at a time, both loaded before either is applied (one memory round trip per pair)
            for (int jj = 1; jj < ns; jj += 2) {
                f4 es[2][4], ep[2][4][4];
#pragma unroll
                for (int x = 0; x < 2; ++x) {
                    const f4* const e = entry(min(jj + x, ns - 1));
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        es[x][m] = xload(e + (m * 4 + j) * 64 + lane);
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) ep[x][m][kk] = xload(e + 16 * 64 + (kk * 4 + m) * 64 + lane);
                    }
                }
#pragma unroll
                for (int x = 0; x < 2; ++x) {
                    if (jj + x >= ns) break;
                    T8 xo[2];
                    state_ops(X, xo);
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        f4 acc = es[x][m];
#pragma unroll
                        for (int kb = 0; kb < 2; ++kb)
                            acc = p32x3(cat(split_t(ep[x][m][2 * kb]), split_t(ep[x][m][2 * kb + 1])), xo[kb], acc);
                        X[m] = acc;
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < 4; ++m) Sin[(m * 4 + j) * 64 + lane] = X[m];
            if (!(cont && one_row)) {  // row A ends in this unit: its final state S_end = P S_in + S_local
                T8 xo[2];
                state_ops(X, xo);
                float* const dst = state_dst(p, A.n, h);
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    f4 x = Sx[(j * 4 + m) * 64 + lane];
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
                        x = p32x3(cat(split_t(Ptx[((2 * kb) * 4 + m) * 64 + lane]),
                                      split_t(Ptx[((2 * kb + 1) * 4 + m) * 64 + lane])), xo[kb], x);
                    if (dst)
#pragma unroll
                        for (int v = 0; v < 4; ++v) dst[(16 * m + 4 * q + v) * HS + 16 * j + i] = x[v];
                }
            }
        }
        __syncthreads();
        // the earlier units' entries are read: count this unit out of their flags
        if (tid < ns)
            __hip_atomic_fetch_add(flags + (k0 + tid) * H + h, -1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // correction of row A's outputs here (its first nA chunks): y_c^T += S_in^T (Q_c P_{c-1})^T.  Wavefront w
        // takes the chunks cl = w, w + 8, .. whole (all four column tiles: one Q P read per chunk, full 128-byte rows
        // of y), RB chunks per round with their loads issued together
        const int nA = (int)(std::min<int64_t>(U.c1, A.first + A.nch) - U.c0);
        if (p.o) {
            bf8 sh[4][2];  // S_in hi, [column tile j][k block]
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
                    sh[j][kb] = cat(hi_t(Sin[((2 * kb) * 4 + j) * 64 + lane]), hi_t(Sin[((2 * kb + 1) * 4 + j) * 64 + lane]));
            constexpr int RB = 4;
            for (int cl0 = wv; cl0 < nA; cl0 += 8 * RB) {
                uint4 qp[RB][4];
                uint2 old[RB][4][2];
                int64_t tok0[RB];
                int Lc[RB];
#pragma unroll
                for (int r = 0; r < RB; ++r) {
                    const int cl = min(cl0 + 8 * r, nA - 1);  // a duplicate of the last chunk is not stored
                    const int64_t c = U.c0 + cl;
                    const int ci = (int)(c - A.first);
                    tok0[r] = A.bos + (int64_t)ci * SC;
                    Lc[r] = (cl0 + 8 * r < nA) ? (int)std::max<int64_t>(0, std::min<int64_t>(SC, A.L - (int64_t)ci * SC))
                                               : 0;
                    const uint4* const src = qp_slot(c);
#pragma unroll
                    for (int x = 0; x < 4; ++x) qp[r][x] = src[x * 64 + lane];
#pragma unroll
                    for (int tau = 0; tau < 2; ++tau) {
                        const int t = 16 * tau + i;
                        const uint16_t* const row =
                            p.o + (tok0[r] + (t < Lc[r] ? t : 0)) * p.o_tok_stride + (int64_t)h * HS + 4 * q;
#pragma unroll
                        for (int j = 0; j < 4; ++j) old[r][j][tau] = *reinterpret_cast<const uint2*>(row + 16 * j);
                    }
                }
#pragma unroll
                for (int r = 0; r < RB; ++r) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        f4 y[2];
#pragma unroll
                        for (int tau = 0; tau < 2; ++tau) {
                            float y0, y1, y2, y3;
                            bf16x2_to_f32(old[r][j][tau].x, y0, y1);
                            bf16x2_to_f32(old[r][j][tau].y, y2, y3);
                            y[tau] = f4{y0, y1, y2, y3};
#pragma unroll
                            for (int kb = 0; kb < 2; ++kb)
                                y[tau] = mma32(sh[j][kb], as_bf8(qp[r][tau * 2 + kb]), y[tau]);
                        }
                        store_y(p, tok0[r], Lc[r], h, j, lane, y);
                    }
                }
            }
        }
    }
}

// Short rows (p.rec_max_len >= 0: rows of at most that many tokens, which no unit owns), token-serial with the
// recurrent kernel's per-pair code (wkv7_token.h), after the workgroup's own unit: every workgroup builds the list of
// short rows in the freed ring, and its wavefronts take the (row, head) pairs blockIdx * 8 + wave, + 8 * gridDim, ..
__device__ __forceinline__ void run_short_rows(const Params& p, SegSmem& sm) {
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    __syncthreads();  // the ring is free
    int* const list = reinterpret_cast<int*>(sm.ring[0]);                          // <= kSegMaxRows rows
    float* const slab = reinterpret_cast<float*>(sm.ring[1]) + wv * 5 * HS;       // per wavefront: d, a, b, k, r
    const int N = p.num_seqs;
    const int per = (N + 511) / 512;
    const int r0 = min(N, tid * per), r1 = min(N, r0 + per);
    int cnt = 0;
    for (int n = r0; n < r1; ++n) {
        int64_t bos;
        int L;
        seq_extent(p, n, bos, L);
        cnt += owns(p, L) ? 0 : 1;
    }
    int total;
    int off = block_excl_scan(cnt, sm.scan, &total);
    for (int n = r0; n < r1; ++n) {
        int64_t bos;
        int L;
        seq_extent(p, n, bos, L);
        if (!owns(p, L)) list[off++] = n;
    }
    __syncthreads();
    const int g = lane >> 3, c = lane & 7;
    const int64_t npairs = (int64_t)total * p.H, nwaves = (int64_t)gridDim.x * 8;
    f4 S[16];
    for (int64_t pa = (int64_t)blockIdx.x * 8 + wv; pa < npairs; pa += nwaves) {
        const int64_t k = pa / p.H;
        Pair pr;
        pr.n = list[k];
        pr.h = (int)(pa - k * p.H);
        seq_extent(p, pr.n, pr.bos, pr.L);
        pr.run = true;
        TokenIn x{};
        prefetch_pair(p, pr, lane, g, c, S, x);
        run_pair(p, pr, lane, g, c, S, x, slab);
    }
}

// xbuf: 32 KB exchange entries (a local end state, then its P^T, RL tiles): entry b for workgroup b's published row,
// and for ragged calls entry gridDim.x + b, where workgroup b parks its first row's local end state and P when that
// row ends inside it.  flags: one per workgroup, set to the number of later units that read its entry and counted
// down by them.  seg: dense calls' chunks per segment.
__global__ __launch_bounds__(512) void wkv7_seg_kernel(const Params p, int seg, int32_t* __restrict__ flags,
                                                       float* __restrict__ xbuf, char* __restrict__ qpbuf,
                                                       bool short_rows) {
    __shared__ SegSmem sm;
    const int tid = threadIdx.x;
    if (tid == 0) sm.fail = 0;
    const Unit U = find_unit(p, seg, (int64_t)blockIdx.x, sm.rows, sm.scan);
    if (U.ok) run_unit(p, U, flags, xbuf, qpbuf, sm);
    if (short_rows) run_short_rows(p, sm);
    if (tid == 0 && sm.fail && p.status)
        __hip_atomic_fetch_or(p.status, WKV7_STATUS_SEGMENT_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

SegWorkspace seg_workspace(int num_seqs, int H, int64_t total_tokens, int64_t max_len_bound, bool varlen,
                           int rec_max_len, int cus) {
    SegWorkspace ws{};
    int64_t entries, qp_chunks;
    if (!varlen) {
        // dense: each row cut into segments, about one unit per CU over the call
        const int nch = (int)std::max<int64_t>(1, (max_len_bound + SC - 1) / SC);
        const int64_t chunks = (int64_t)num_seqs * nch;
        ws.seg = (int)std::max<int64_t>(kSegMinChunks, (chunks * H + cus - 1) / std::max(1, cus));
        const int nseg = std::max(1, (nch + ws.seg - 1) / ws.seg);
        ws.units = (int64_t)num_seqs * nseg * H;
        entries = ws.units;  // a dense unit never crosses a row: nothing to park
        qp_chunks = (int64_t)num_seqs * (nch - seg_start(nch, nseg, 1));
    } else {
        // ragged / n_keep: CUs / H units per head share each head's chunk stream; the stream has ceil(L / 32) chunks
        // per owned row (1 for an empty one), at most ceil(total / 32) + the owned rows
        const int64_t long_rows = rec_max_len < 0 ? num_seqs
                                                  : std::min<int64_t>(num_seqs, total_tokens / ((int64_t)rec_max_len + 1));
        const int64_t chunks = std::min<int64_t>((int64_t)num_seqs * std::max<int64_t>(1, (max_len_bound + SC - 1) / SC),
                                                 (total_tokens + SC - 1) / SC + long_rows);
        ws.seg = 0;  // the kernel sizes the shares from the stream's length
        ws.units = std::max(1, cus / std::max(1, H)) * (int64_t)H;
        if (chunks > 0x7fffffff) ws.units = INT64_MAX;  // stream offsets are int32 in LDS: refused by the callers
        entries = 2 * ws.units;  // published, and parked
        qp_chunks = chunks;
    }
    if (ws.units == INT64_MAX) return ws;
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    ws.flag_bytes = al(sizeof(int32_t) * (size_t)ws.units);
    ws.x_bytes = al((size_t)entries * 2 * HS2 * sizeof(float));  // local end state + P^T per entry
    ws.qp_bytes = al((size_t)qp_chunks * H * 4096);
    ws.total_bytes = kSegFlagRegion + ws.x_bytes + ws.qp_bytes;
    return ws;
}

hipError_t launch_seg(const Params& p, const SegWorkspace& ws, void* workspace, bool short_rows, hipStream_t stream) {
    if (p.num_seqs == 0 || ws.units == 0) return hipSuccess;
    char* base = static_cast<char*>(workspace);
    int32_t* flags = reinterpret_cast<int32_t*>(base);
    float* xbuf = reinterpret_cast<float*>(base + kSegFlagRegion);
    char* qp = base + kSegFlagRegion + ws.x_bytes;
    hipLaunchKernelGGL(wkv7_seg_kernel, dim3((unsigned)ws.units), dim3(512), 0, stream, p, ws.seg, flags, xbuf, qp,
                       short_rows);
    return hipGetLastError();
}

}  // namespace wkv7
