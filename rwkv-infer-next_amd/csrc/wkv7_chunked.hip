// wkv7_chunked.hip -- chunked WKV7 prefill on bf16 MFMA (gfx950, v_mfma_f32_16x16x32_bf16).
//
// Replaces the reference's token-serial Triton program (rwkv_next/kernels/wkv7.py:65-77) for long rows: the
// reference walks every token of a row in one program, so a B=1, T=4096, H=64 prefill has only
// (64/BV)*64 programs and no parallelism over T.  Here the row is cut into chunks of C = 64 tokens.
//
// Algebra (per head; S is K x V, reference orientation).  Inside a chunk with initial state S0, write
// g_t = sum_{u<=t} log d_u (per channel), u_s = a_s^T S_{s-1} (the a^T S term of step s).  Then
//   U = W S0 + G V,                         W = T A0,  G = T beta,  T = (I - alpha)^{-1}
//   O = R0 S0 + rho U + sigma V = Q S0 + E V,          Q = R0 + rho W,  E = sigma + rho G
//   S_C = Gamma S0 + Bh^T U + Kh^T V = A S0 + F V,     A = Gamma + Bh^T W,  F = Bh^T G + Kh^T
// with (rows = tokens, columns = channels)
//   A0[t] = a_t e^{g_{t-1}},  R0[t] = r_t e^{g_t},  Bh[s] = b_s e^{g_C - g_s},  Kh[s] = k_s e^{g_C - g_s},
//   Gamma = diag(e^{g_C}),
//   alpha[t][s] = sum_k a_t b_s e^{g_{t-1} - g_s} (s < t),   beta  = same with k_s,
//   rho[t][s]   = sum_k r_t b_s e^{g_t - g_s}     (s <= t),  sigma = same with k_s.
// Every exponent above is <= 0.  The four Gram matrices are matmuls of operands referenced to the chunk
// midpoint m: alpha = (a e^{g_{t-1}-m}) (b e^{m-g_s})^T etc.; for the model's decays (|log d| < 0.61 per token)
// those factors stay below e^{20}.
//
// Precision.  Products feeding the state (alpha, beta, W, G, A, F, H and the scan's A S) run as three bf16 MFMAs
// on a hi/lo split of each fp32 operand (x = hi + lo, hi = bf16(x), lo = bf16(x - hi); x*y ~ hi*hi + hi*lo +
// lo*hi, relative error ~2^-16); products feeding only the output y (rho, sigma, Q, E, O_intra, the scan's Q S)
// run as one bf16 MFMA.  T = (I - alpha)^{-1} is formed in fp32 (fp32 MFMA).  Accumulation is fp32 throughout.
//
// Kernels:
//   plan  (ragged calls only): chunk table of the rows this launch owns;
//   prep  one 512-thread workgroup per (chunk, head): everything above that does not depend on S0, written to
//         the workspace as A (hi/lo bf16), H = F V (fp32, transposed), Q (bf16), O_intra = E V (bf16);
//   scan  one workgroup per (row, head, 16-column block): S <- A S + H, y <- Q S + O_intra, chunk after
//         chunk.  The chunks of a head and its 4 column blocks run on one XCD (block id = head mod 8 when H is a
//         multiple of 8), so the scan reads the prep's records from that XCD's L2 / the Infinity Cache.
#include <algorithm>

#include "wkv7_device.h"
#include "wkv7_launch.h"
#include "wkv7_token.h"

namespace wkv7 {

namespace {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf4 __attribute__((ext_vector_type(4)));

constexpr int C = kChunk;        // 64
constexpr int PB = 72;           // LDS row pitch in bf16 (144 B: 16 rows of a ds_read_b128 hit distinct banks)
constexpr int PF = 72;           // LDS row pitch in fp32 for the fp32 matrices (same bytes as a hi/lo pair)
constexpr int SLOT = 64 * PB;    // bf16 elements of one 64 x 64 LDS matrix (9216 B)
constexpr int NSLOT = 17;

// Workspace record of one (chunk, head), byte offsets.  Every part is stored in the fragment order of the scan's
// MFMAs, so that each scan lane reads its operands as contiguous 16-byte pieces.  A and Q are 16x16x32 operands:
// for row tile a and contraction block c (32 wide), lane (i, q) holds row 16 a + i, columns 32 c + 8 q .. + 7.  H^T
// and O_intra are 16x16 results: lane (i, q) holds rows 4 q .. 4 q + 3 of column i (H), or row i, columns
// 4 q .. 4 q + 3 (O_intra, two token tiles per 16-byte piece).
constexpr int REC_AH = 0;                  // A hi, bf16: [k1 tile r][k2 block c][lane][8]
constexpr int REC_AL = REC_AH + 2 * HS2;   // A lo, same
constexpr int REC_HT = REC_AL + 2 * HS2;   // H^T fp32: [v tile vg][k tile r][lane][4]  (H[16 r + 4 q + e][16 vg + i])
constexpr int REC_Q = REC_HT + 4 * HS2;    // Q bf16: [token tile t][k block c][lane][8]
constexpr int REC_OT = REC_Q + 2 * HS2;    // O_intra bf16: [v tile vg][token tile pair][lane][8]
static_assert(REC_OT + 2 * HS2 == kChunkBytes, "workspace record size");

// Byte offset of tile (row tile a, contraction tile b) of a 64 x 64 bf16 record part, for this lane: tiles b = 2 c and
// 2 c + 1 share a 16-byte piece per lane.
__device__ __forceinline__ int frag_off_bf16(int a, int b, int lane) { return ((a * 2 + (b >> 1)) * 64 + lane) * 16 + (b & 1) * 8; }

// Where a 16x16 result tile (row tile a, column tile b; lane (li, lq) holding row 16 a + li, columns 16 b + 4 lq ..
// + 3) lands in the 16x16x32 operand order of a record part: scan lane li + 16 (2 (b & 1) + (lq >> 1)) of block
// (a, b >> 1), values 4 (lq & 1) .. + 3 of its 8.
__device__ __forceinline__ int frag32_off(int a, int b, int lane) {
    const int li = lane & 15, lq = lane >> 4;
    return ((a * 2 + (b >> 1)) * 64 + li + 16 * (2 * (b & 1) + (lq >> 1))) * 16 + 8 * (lq & 1);
}

__device__ __forceinline__ f4 zero4() { return f4{0.f, 0.f, 0.f, 0.f}; }

// Makes the compiler complete the loads that produced `x` here (an empty asm reading the registers).  Used after a
// loop's prologue loads: with nothing in flight from the prologue, the loop header's wait bookkeeping only carries
// the loop's own prefetches, which it counts exactly, instead of falling back to waiting for every memory operation.
template <typename T>
__device__ __forceinline__ void settle(const T& x) {
    static_assert(sizeof(T) % 4 == 0, "settle: 32-bit words");
    const uint32_t* w = reinterpret_cast<const uint32_t*>(&x);
#pragma unroll
    for (int e = 0; e < (int)(sizeof(T) / 4); ++e) asm volatile("" ::"v"(w[e]));
}

__device__ __forceinline__ f4 mfma_bf16(bf8 a, bf8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma_f32(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

typedef short s4 __attribute__((ext_vector_type(4)));  // 4 bf16 bit patterns, the 16x16x16 MFMA operand

// 16x16x16 bf16 MFMA.  Lane (i = lane & 15, q = lane >> 4) feeds A[i][4q .. 4q+3] and B[4q .. 4q+3][i] and receives
// D[4q + v][i] in acc[v]: a result tile is already laid out as a B operand.
__device__ __forceinline__ f4 mfma16(s4 a, s4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// An LDS matrix stored as bf16 rows of pitch PB: the high part and (for split fp32 values) the low part.
struct BM {
    __bf16* h;
    __bf16* l;
};

__device__ __forceinline__ bf8 ld8(const __bf16* p) { return *reinterpret_cast<const bf8*>(p); }

// One 16 x 16 tile of P[x][y] = sum_kappa X[x][kappa] Y[y][kappa], both operands stored with kappa contiguous.
// Lane (i = lane & 15, q = lane >> 4) feeds X[x0 + i][32 kb + 8 q .. + 7] and Y[y0 + i][32 kb + 8 q .. + 7] to
// MFMA block kb, so the 16 x 32 A operand and the 32 x 16 B operand share one contraction index per element.
// On return lane (i, q) holds P[x0 + 4 q + v][y0 + i] in acc[v].
// TERMS: 1 = X.h Y.h;  2 = X.h Y.h + X.l Y.h (Y exact in bf16);  3 = X.h Y.h + X.h Y.l + X.l Y.h.
template <int TERMS>
__device__ __forceinline__ f4 mma(f4 acc, BM X, int x0, BM Y, int y0, int kb0, int kb1) {
    const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    for (int kb = kb0; kb < kb1; ++kb) {
        const int xo = (x0 + i) * PB + 32 * kb + 8 * q;
        const int yo = (y0 + i) * PB + 32 * kb + 8 * q;
        const bf8 xh = ld8(X.h + xo), yh = ld8(Y.h + yo);
        if constexpr (TERMS == 3) acc = mfma_bf16(xh, ld8(Y.l + yo), acc);
        if constexpr (TERMS >= 2) acc = mfma_bf16(ld8(X.l + xo), yh, acc);
        acc = mfma_bf16(xh, yh, acc);
    }
    return acc;
}

// Four fp32 values as hi/lo bf16 operands of mfma16 (split_pair on each half).
__device__ __forceinline__ void split4(f4 x, s4& h, s4& l) {
    uint32_t hw[2], lw[2];
    split_pair(x[0], x[1], hw[0], lw[0]);
    split_pair(x[2], x[3], hw[1], lw[1]);
    h = __builtin_bit_cast(s4, hw);
    l = __builtin_bit_cast(s4, lw);
}

// LDS transposing read (ds_read_b64_tr_b16).  Within each 16-lane group, lane s reads 4 consecutive 16-bit values at
// its own address; lane L then receives value (L & 3) of the reads of lanes (L & 15) / 4 + 4 e, e = 0..3.  With lane
// L of group q addressing M[k0 + 4 q + ((L & 15) >> 2)][n0 + 4 (L & 3)] of a row-major matrix, lane L receives
// M[k0 + 4 q + e][n0 + (L & 15)]: an MFMA operand whose contraction runs down the rows of M.
typedef __attribute__((address_space(3))) s4 lds_s4;
__device__ __forceinline__ s4 ld_tr4(const __bf16* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p));
}

// Operand of the 16x16x32 MFMA for contraction block kb (rows 32 kb .. of M) and column block n0 of a row-major
// bf16 LDS matrix M[kappa][n]: lane (i, q) gets M[32 kb + 8 q + j][n0 + i], j = 0..7.
__device__ __forceinline__ bf8 ld8_tr(const __bf16* M, int kb, int n0) {
    const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    const __bf16* const p = M + (32 * kb + 8 * q + (i >> 2)) * PB + n0 + 4 * (i & 3);
    const s4 a = ld_tr4(p), b = ld_tr4(p + 4 * PB);
    return __builtin_bit_cast(bf8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Natural stores of a tile (element (x0 + 4q + v, y0 + i) at M[(y0 + i) * pitch + x0 + 4q + v]): 4 consecutive
// elements per lane.
__device__ __forceinline__ void st_hi(__bf16* M, int pitch, int x0, int y0, f4 acc) {
    const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    bf4 hv;
#pragma unroll
    for (int v = 0; v < 4; ++v) hv[v] = (__bf16)acc[v];
    *reinterpret_cast<bf4*>(M + (y0 + i) * pitch + x0 + 4 * q) = hv;
}
__device__ __forceinline__ void st_split(BM M, int pitch, int x0, int y0, f4 acc) {
    const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    s4 hv, lv;
    split4(acc, hv, lv);
    *reinterpret_cast<s4*>(M.h + (y0 + i) * pitch + x0 + 4 * q) = hv;
    *reinterpret_cast<s4*>(M.l + (y0 + i) * pitch + x0 + 4 * q) = lv;
}
__device__ __forceinline__ void st_f32(float* M, int pitch, int x0, int y0, f4 acc) {
    const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    *reinterpret_cast<f4*>(M + (y0 + i) * pitch + x0 + 4 * q) = acc;
}

// mask: 1 keeps x < y, 2 keeps x <= y, 3 keeps y < x (others become 0)
__device__ __forceinline__ f4 mask_tile(f4 acc, int x0, int y0, int mode) {
    const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    const int y = y0 + i;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int x = x0 + 4 * q + v;
        const bool keep = mode == 1 ? x < y : (mode == 2 ? x <= y : y < x);
        if (!keep) acc[v] = 0.f;
    }
    return acc;
}

// Position of a prep work item: item = j * H + h (chunk slot j, head h) and, for dense calls, j = n * ncps + c (row
// n, chunk c).  Divided out once per workgroup, then advanced by the grid stride with adds and a rare carry: the
// CU's waves share one scalar unit, and a 64-bit division per item per wave cost more than a thousand cycles.
struct ItemPos {
    int64_t item, j;
    int h, n, c;
};

__device__ __forceinline__ ItemPos item_pos(const Params& p, int ncps, int64_t item) {
    ItemPos q;
    q.item = item;
    q.j = item / p.H;
    q.h = (int)(item % p.H);
    q.n = (int)(q.j / ncps);
    q.c = (int)(q.j % ncps);
    return q;
}

// q += stride, where stride = sj * H + sh (0 <= sh < H)
__device__ __forceinline__ void advance(ItemPos& q, const Params& p, int ncps, int64_t stride, int64_t sj, int sh) {
    q.item += stride;
    int64_t dj = sj;
    q.h += sh;
    if (q.h >= p.H) {
        q.h -= p.H;
        ++dj;
    }
    q.j += dj;
    int64_t c = q.c + dj;
    if (c >= ncps) {
        q.n += (int)(c / ncps);
        c %= ncps;
    }
    q.c = (int)c;
}

// Chunk slot -> (row, chunk index) of the rows this launch owns.  Returns false if the slot has no chunk.
__device__ __forceinline__ bool chunk_of(const Params& p, const int32_t* plan, int64_t max_chunks, const ItemPos& q,
                                         int& n, int& c) {
    if (p.cu) {
        const int32_t total = plan[2 * max_chunks + p.num_seqs + 1];
        if (q.j >= total) return false;
        n = plan[q.j];
        c = plan[max_chunks + q.j];
    } else {
        n = q.n;
        c = q.c;
    }
    return true;
}

__device__ __forceinline__ bool owns_row(const Params& p, int L) { return p.rec_max_len < 0 || L > p.rec_max_len; }

// fp32 16 x 16 tile product on MFMA 16x16x4: acc += sum_{kappa < K} X(x0 + i, kappa) Y(y0 + i, kappa) with
// X(x, kappa) = Xp[x * xs + kappa * xk] and Y(y, kappa) = Yp[y * ys + kappa * yk] (Xp, Yp already offset to the
// tile).  Lane (i, q) feeds contraction index m + q to step m and ends with P[4 q + v][i] in acc[v].
__device__ __forceinline__ f4 mm_f32(f4 acc, const float* Xp, int xs, int xk, const float* Yp, int ys, int yk, int K) {
    const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    for (int m = 0; m < K; m += 4) acc = mfma_f32(Xp[i * xs + (m + q) * xk], Yp[i * ys + (m + q) * yk], acc);
    return acc;
}
// Row-major store of such a tile: D[(4 q + v) * pd + i] = acc[v].
__device__ __forceinline__ void st_rows_f32(float* D, int pd, f4 acc) {
    const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
#pragma unroll
    for (int v = 0; v < 4; ++v) D[(4 * q + v) * pd + i] = acc[v];
}

// B operand of a scaled identity, built in registers: Y[y][kappa] = (kappa == y) ? s : 0 for lane row y and the
// lane's 8 contraction indices 32 kb + 8 q .. + 7.  P = X diag(s) stored naturally ([y][x]) is the transpose of
// X with its columns scaled: the LDS transposes below cost a few MFMAs instead of scattered 2-byte stores.
__device__ __forceinline__ bf8 diag_operand(int y, int kb, __bf16 s) {
    const int lane = threadIdx.x & 63, q = lane >> 4;
    bf8 d;
#pragma unroll
    for (int e = 0; e < 8; ++e) d[e] = (32 * kb + 8 * q + e == y) ? s : (__bf16)0.f;
    return d;
}

// Inclusive scan over the 8 tokens of a wave for one channel, tokens in lanes 8 t + channel group: each 16-lane row
// holds two tokens (DPP row_ror:8 swaps its halves), v_permlane16_swap pairs rows and v_permlane32_swap pairs the
// wave's halves.  Returns g(t) and sets prev to g(t - 1) (0 for the first token); both are built from the same
// partial sums, so g(t - 1) here and g(t - 1) returned to that token's lanes are the same float.
// Cross-lane reads need every source lane active, so each is evaluated in all lanes before any select, and the empty
// asm keeps the compiler from sinking it into the branch of a later select.
__device__ __forceinline__ float dpp_ror8(float x) {
    float r = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));
    asm volatile("" : "+v"(r));
    return r;
}
__device__ __forceinline__ float wave_scan8(float v, int lane, float& prev) {
    const bool upper = (lane & 8) != 0;
    const int rowi = lane >> 4;
    const float vo = dpp_ror8(v);
    const float y = upper ? vo + v : v;                  // inclusive within the row
    const float yr = dpp_ror8(y);
    const float t = upper ? y : yr;                      // the row's total, in both halves
    const auto pr = __builtin_amdgcn_permlane16_swap(__float_as_uint(t), __float_as_uint(t), false, false);
    float te = __uint_as_float(pr[0]), to = __uint_as_float(pr[1]);  // totals of the pair's even / odd row
    asm volatile("" : "+v"(te), "+v"(to));
    const float u = te + to;                                                // the pair's total
    const auto hv = __builtin_amdgcn_permlane32_swap(__float_as_uint(u), __float_as_uint(u), false, false);
    float p0 = __uint_as_float(hv[0]);                                      // rows 0-1 total
    asm volatile("" : "+v"(p0));
    const float before = (rowi & 1 ? te : 0.f) + (rowi >= 2 ? p0 : 0.f);  // tokens of the earlier rows
    const float g = y + before;
    const float gr = dpp_ror8(g);
    prev = upper ? gr : before;
    return g;
}

struct PrepSmem {
    __bf16 slot[NSLOT][SLOT];
    float m[HS], em[HS], eglm[HS], gam[HS];  // m, em, eglm, gam: base-2 midpoint and decay factors per channel
    float bsum[8][HS];
};

// Raw operands of one chunk for one thread (token row `row`, channels cb .. cb + 7), bf16 x 8 each.
struct RawIn {
    uint4 w, a, b, k, r, v;
};

// One work item (chunk, head) of the prep kernel.
struct Item {
    bool ok;
    int h, Lc;        // Lc = 0 for items without a chunk
    int64_t j, tok0;  // chunk slot, first token of the chunk
    int64_t rec;      // workspace record: (j, h), or the trash record after the last one for items without a chunk
};

__device__ __forceinline__ Item describe_item(const Params& p, const int32_t* plan, int64_t max_chunks,
                                             const ItemPos& q) {
    Item it{};
    it.j = q.j;
    it.h = q.h;
    it.rec = max_chunks * p.H;  // trash
    int n, c;
    if (!chunk_of(p, plan, max_chunks, q, n, c)) return it;
    int64_t bos;
    int L;
    seq_extent(p, n, bos, L);
    if (!owns_row(p, L) || c * C >= L) return it;
    it.ok = true;
    it.Lc = min(C, L - c * C);
    it.tok0 = bos + (int64_t)c * C;
    it.rec = it.j * p.H + it.h;
    return it;
}

// The six loads are issued for every thread and item: rows outside the chunk (and items without a chunk) read token
// 0, which always exists, and prep_item zeroes them.  A fixed number of loads per item lets the compiler count the
// outstanding prefetch exactly; with conditional loads it falls back to waiting for all of them at first use.
__device__ __forceinline__ RawIn load_item(const Params& p, const Item& it, int row, int cb) {
    const bool valid = row < it.Lc;
    const int64_t off = valid ? (it.tok0 + row) * p.in_tok_stride + (int64_t)it.h * HS + cb : (int64_t)cb;
    RawIn x;
    x.w = *reinterpret_cast<const uint4*>(p.w + off);
    x.a = *reinterpret_cast<const uint4*>(p.a + off);
    x.b = *reinterpret_cast<const uint4*>(p.b + off);
    x.k = *reinterpret_cast<const uint4*>(p.k + off);
    x.r = *reinterpret_cast<const uint4*>(p.r + off);
    x.v = *reinterpret_cast<const uint4*>(p.v + off);
    return x;
}

// Element offset of this thread's operand row of an item (token 0 for rows outside the chunk, see load_item).
__device__ __forceinline__ int64_t item_offset(const Params& p, const Item& it, int row, int cb) {
    return row < it.Lc ? (it.tok0 + row) * p.in_tok_stride + (int64_t)it.h * HS + cb : (int64_t)cb;
}

constexpr float kLog2e = 1.4426950408889634f;

// Slots (each 64 x 72 bf16 = 9 KB; an fp32 64 x 72 matrix takes two):
//   0-1   alpha (fp32, diagonal blocks replaced by their inverses T_ii) -> W hi/lo
//   2-3   Aq hi/lo -> F hi/lo
//   4-5   Bk hi/lo                  6-7   Kk hi/lo
//   8     Rq hi
//   10-11 beta hi/lo -> G hi/lo     12 rho    13 sigma    14 E
//   15    V^T ([v][s], exact)
// The products that contract over tokens (W = T A0, A = Bh^T W, F = Kh^T + Bh^T G, H = F V, O_intra = E V) read Aq,
// Bk, Kk and V where they lie, through transposing LDS reads, and apply the per-channel decay factors that separate
// A0, Bh, Kh from Aq, Bk, Kk (2^m, 2^{g_C - m}) to their fp32 results.
// Decays are handled in base 2 (g = cumulative log2 d), so every decay factor is one v_exp_f32.
// The next item's operands (element offset noff) are loaded into `next` one operand per phase, spread over the item
// so that their issue does not queue behind one another.
// Where the record of an item goes: the workspace (the two-kernel path: prep writes, the scan kernel reads), or the
// LDS slots kRecSlot.. (the chain kernel, which applies the record to the state itself).  In LDS the record reuses
// operand slots that step 8 still reads, so step 8's A and Q tiles are held in registers and stored in step 9.
constexpr int kRecSlot = 4;  // LDS record: slots 4 .. 9 (48 KB of the 6 x 9 KB)

template <bool LDS_REC>
__device__ __forceinline__ void prep_item(const Params& p, const Item& it, const RawIn& raw, char* wsc,
                                          PrepSmem& sm, int64_t noff, RawIn& next) {
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15, lq = lane >> 4;
    float* const F32 = reinterpret_cast<float*>(sm.slot[0]);   // slots 0-1 as fp32 [64][PF]
    const BM Aq{sm.slot[2], sm.slot[3]};
    const BM Bk{sm.slot[4], sm.slot[5]};
    const BM Kk{sm.slot[6], sm.slot[7]};
    const BM Rq{sm.slot[8], nullptr};
    const BM Be{sm.slot[10], sm.slot[11]};
    const BM Rho{sm.slot[12], nullptr};
    const BM Sig{sm.slot[13], nullptr};
    const BM Em{sm.slot[14], nullptr};
    const BM Vt{sm.slot[15], nullptr};  // V transposed: [v][s]
    const BM Wm{sm.slot[0], sm.slot[1]}, Gm = Be;   // after step 7: W^T [k][t], G^T [s'][t]
    const BM Fm{sm.slot[2], sm.slot[3]};            // step 8 (Aq is dead after step 7)
    char* const rec = LDS_REC ? reinterpret_cast<char*>(sm.slot[kRecSlot]) : wsc + it.rec * (int64_t)kChunkBytes;
    const int row = tid >> 3, cb = (tid & 7) * 8;
    const bool valid = row < it.Lc;

    // ---- 1. log2-decay lam = log2 d = -e^w log2(e) = -2^{w log2(e)} log2(e) of this thread's row and 8 channels,
    //         and its inclusive cumulative sum over the rows: first within the wave (rows 8 wv .. 8 wv + 7 live in
    //         lanes 8 r + channel group, so a scan over lanes with stride 8), then across waves through the wave
    //         totals.  Every g below is (in-wave scan) + (sum of the earlier waves' totals, in wave order), so the
    //         previous row's g, the midpoint (row 31) and the chunk total (row 63) are the same floats wherever
    //         they are formed.  V (exact) -> Vt transposed, [v][s]: both of its products (step 9) contract over
    //         tokens, so stored this way they read it with ordinary row reads instead of transposing ones.
    float lam[8], gin[8], gprev[8];
    {
        const uint32_t ww[4] = {raw.w.x, raw.w.y, raw.w.z, raw.w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float lo, hi;
            bf16x2_to_f32(ww[e], lo, hi);
            lam[2 * e] = valid ? -__builtin_amdgcn_exp2f(lo * kLog2e) * kLog2e : 0.f;
            lam[2 * e + 1] = valid ? -__builtin_amdgcn_exp2f(hi * kLog2e) * kLog2e : 0.f;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) gin[e] = wave_scan8(lam[e], lane, gprev[e]);
        if (lane >= 56) {  // the wave's last row: its totals per channel
            *reinterpret_cast<f4*>(&sm.bsum[wv][cb]) = f4{gin[0], gin[1], gin[2], gin[3]};
            *reinterpret_cast<f4*>(&sm.bsum[wv][cb + 4]) = f4{gin[4], gin[5], gin[6], gin[7]};
        }
        const uint4 vv = valid ? raw.v : make_uint4(0u, 0u, 0u, 0u);
        const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
        uint16_t* const vt = reinterpret_cast<uint16_t*>(Vt.h) + row;
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
            vt[(cb + 2 * e2) * PB] = (uint16_t)(vw[e2] & 0xffffu);
            vt[(cb + 2 * e2 + 1) * PB] = (uint16_t)(vw[e2] >> 16);
        }
    }
    __syncthreads();
    next.w = *reinterpret_cast<const uint4*>(p.w + noff);

    // ---- 2. per channel (one lane each): the waves' prefix offsets in wave order, the midpoint m = g_31 (waves
    //         0-3) and the chunk total g_63, then the decay factors of the midpoint; every thread then forms g
    //         (inclusive) and g of the previous row from its in-wave scan plus its wave's offset.  Every sum is
    //         taken in wave order, so the midpoint and total here equal the g of rows 31 and 63 bit for bit.
    if (tid < HS) {
        float acc = 0.f, mid = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < 8; ++w2) {
            const float t = sm.bsum[w2][tid];
            sm.bsum[w2][tid] = acc;  // offset of wave w2: the sum of the earlier waves' totals
            if (w2 == 4) mid = acc;
            acc += t;
        }
        sm.m[tid] = mid;
        sm.em[tid] = __builtin_amdgcn_exp2f(mid);
        sm.eglm[tid] = __builtin_amdgcn_exp2f(acc - mid);
        sm.gam[tid] = __builtin_amdgcn_exp2f(acc);
    }
    __syncthreads();
    float gi[8], ge[8], mk[8];
    {
        const f4 o0 = *reinterpret_cast<const f4*>(&sm.bsum[wv][cb]);
        const f4 o1 = *reinterpret_cast<const f4*>(&sm.bsum[wv][cb + 4]);
        const f4 m0 = *reinterpret_cast<const f4*>(&sm.m[cb]);
        const f4 m1 = *reinterpret_cast<const f4*>(&sm.m[cb + 4]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float off = e < 4 ? o0[e] : o1[e - 4];
            mk[e] = e < 4 ? m0[e] : m1[e - 4];
            gi[e] = gin[e] + off;
            ge[e] = gprev[e] + off;
        }
    }

    // ---- 3. Gram operands referenced to the chunk midpoint: Aq = a 2^{g_{t-1}-m}, Rq = r 2^{g_t-m},
    //         Bk = b 2^{m-g_t}, Kk = k 2^{m-g_t} (split hi/lo)
    {
        // rows outside the chunk read token 0 (see load_item): their raw operands are zeroed once, word by word
        const uint32_t vm = valid ? 0xffffffffu : 0u;
        const uint32_t aw[4] = {raw.a.x & vm, raw.a.y & vm, raw.a.z & vm, raw.a.w & vm};
        const uint32_t bw[4] = {raw.b.x & vm, raw.b.y & vm, raw.b.z & vm, raw.b.w & vm};
        const uint32_t kw[4] = {raw.k.x & vm, raw.k.y & vm, raw.k.z & vm, raw.k.w & vm};
        const uint32_t rw[4] = {raw.r.x & vm, raw.r.y & vm, raw.r.z & vm, raw.r.w & vm};
        uint32_t aqh[4], aql[4], bkh[4], bkl[4], kkh[4], kkl[4], rqh[4];
        // hi/lo split of a channel pair straight into packed words
        auto split2 = [](float x0, float x1, uint32_t& hw, uint32_t& lw) { split_pair(x0, x1, hw, lw); };
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
            float a2[2], b2[2], k2[2], r2[2], fa[2], fr[2], fb[2];
            bf16x2_to_f32(aw[e2], a2[0], a2[1]);
            bf16x2_to_f32(bw[e2], b2[0], b2[1]);
            bf16x2_to_f32(kw[e2], k2[0], k2[1]);
            bf16x2_to_f32(rw[e2], r2[0], r2[1]);
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int e = 2 * e2 + u;
                fa[u] = __builtin_amdgcn_exp2f(ge[e] - mk[e]);
                fr[u] = __builtin_amdgcn_exp2f(gi[e] - mk[e]);
                fb[u] = __builtin_amdgcn_exp2f(mk[e] - gi[e]);
            }
            split2(a2[0] * fa[0], a2[1] * fa[1], aqh[e2], aql[e2]);
            split2(b2[0] * fb[0], b2[1] * fb[1], bkh[e2], bkl[e2]);
            split2(k2[0] * fb[0], k2[1] * fb[1], kkh[e2], kkl[e2]);
            rqh[e2] = pack_bf16x2(r2[0] * fr[0], r2[1] * fr[1]);
        }
        const int o = row * PB + cb;
        auto st = [&](__bf16* dst, const uint32_t (&w)[4]) {
            *reinterpret_cast<uint4*>(dst + o) = make_uint4(w[0], w[1], w[2], w[3]);
        };
        st(Aq.h, aqh);
        st(Aq.l, aql);
        st(Bk.h, bkh);
        st(Bk.l, bkl);
        st(Kk.h, kkh);
        st(Kk.l, kkl);
        st(Rq.h, rqh);
    }
    __syncthreads();
    next.a = *reinterpret_cast<const uint4*>(p.a + noff);

    // ---- 4. Grams (natural store of P(x, y) is [y][x]):
    //   alpha: x = s, y = t  (X = Bk, Y = Aq, 3 terms), keep s < t, fp32 -> F32 as alpha[t][s]
    //   beta : x = s, y = s' (X = Aq, Y = Kk, 3 terms), keep s' < s, hi/lo -> Be as beta[s][s'] at [s'][s]
    //   rho  : x = s, y = t  (X = Bk, Y = Rq),            keep s <= t, -> Rho as rho[t][s]
    //   sigma: x = s', y = t (X = Kk, Y = Rq),            keep s' <= t, -> Sig as sigma[t][s']
    // Wave wv owns tiles (bx, by) = (wv / 4 + 2 u, wv % 4), u = 0, 1 (the two waves on a SIMD cover one column of
    // tiles).  All four products of a tile are formed together, each operand fragment loaded once; tiles a causal
    // mask zeroes entirely skip their MFMAs and store zeros (later products contract over the full ranges).
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int bx = (wv >> 2) + 2 * u, by = wv & 3;
        const int x0 = 16 * bx, y0 = 16 * by;
        f4 aa = zero4(), bb = zero4(), rr = zero4(), ss = zero4();
        if (bx <= by) {  // alpha, rho, sigma (lower part)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int xo = (x0 + li) * PB + 32 * kb + 8 * lq, yo = (y0 + li) * PB + 32 * kb + 8 * lq;
                const bf8 bkh = ld8(Bk.h + xo), bkl = ld8(Bk.l + xo), kkh = ld8(Kk.h + xo);
                const bf8 aqh = ld8(Aq.h + yo), aql = ld8(Aq.l + yo), rq = ld8(Rq.h + yo);
                aa = mfma_bf16(bkh, aql, aa);
                aa = mfma_bf16(bkl, aqh, aa);
                aa = mfma_bf16(bkh, aqh, aa);
                rr = mfma_bf16(bkh, rq, rr);
                ss = mfma_bf16(kkh, rq, ss);
            }
        }
        if (bx >= by) {  // beta (upper part)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int xo = (x0 + li) * PB + 32 * kb + 8 * lq, yo = (y0 + li) * PB + 32 * kb + 8 * lq;
                const bf8 aqh = ld8(Aq.h + xo), aql = ld8(Aq.l + xo);
                const bf8 kkh = ld8(Kk.h + yo), kkl = ld8(Kk.l + yo);
                bb = mfma_bf16(aqh, kkl, bb);
                bb = mfma_bf16(aql, kkh, bb);
                bb = mfma_bf16(aqh, kkh, bb);
            }
        }
        if (bx == by) {  // only diagonal tiles straddle the causal boundary (bx, by are wave-uniform)
            aa = mask_tile(aa, x0, y0, 1);
            bb = mask_tile(bb, x0, y0, 3);
            rr = mask_tile(rr, x0, y0, 2);
            ss = mask_tile(ss, x0, y0, 2);
        }
        st_f32(F32, PF, x0, y0, aa);
        st_split(Be, PB, x0, y0, bb);
        st_hi(Rho.h, PB, x0, y0, rr);
        st_hi(Sig.h, PB, x0, y0, ss);
    }
    __syncthreads();
    next.b = *reinterpret_cast<const uint4*>(p.b + noff);

    // ---- 5. waves 0-3: inverse T_ii = (I - L)^{-1} of diagonal block i = wv (L = alpha_ii, strictly lower, so
    //         L^16 = 0 and T = (I + L)(I + L^2)(I + L^4)(I + L^8), the factors commuting).  With Bl(M) the 16x16x16
    //         MFMA's B / result layout (lane (c, q) holds M[4 q + v][c]) and Al(M) = Bl(M^T) its A layout, the
    //         powers P_k = L^(2^k) and Q_k = (L^T)^(2^k) feed each other: Bl(P_k) = mfma(Bl(Q_{k-1}), Bl(P_{k-1})),
    //         Bl(Q_k) = mfma(Bl(P_{k-1}), Bl(Q_{k-1})), and Bl(T^T) = prod (I + Q_k) accumulates as
    //         Z_k = mfma(Bl(I + P_k), Z_{k-1}).  Lane (c, q) then holds T[c][4 q + v], the row segment the
    //         substitution below reads as its A operand; 3-term hi/lo products throughout (state path).
    //         waves 4-7: the six blocks alpha_ij, i > j.
    //         Both leave their block split hi/lo in place, as the A operand of step 7: each 64-byte row segment of
    //         a 16 x 16 fp32 block becomes 16 bf16 hi followed by 16 bf16 lo.
    if (wv < 4) {
        float* const Lb = F32 + (16 * wv) * PF + 16 * wv;
        f4 P, Q;
#pragma unroll
        for (int v = 0; v < 4; ++v) P[v] = Lb[(4 * lq + v) * PF + li];  // Bl(L)
        Q = *reinterpret_cast<const f4*>(Lb + li * PF + 4 * lq);        // Bl(L^T)
        auto plus_i = [&](f4 x) {
#pragma unroll
            for (int v = 0; v < 4; ++v) x[v] += (4 * lq + v == li) ? 1.f : 0.f;
            return x;
        };
        auto mul3 = [](f4 a, f4 b) {  // Bl(A B) from Bl(A^T) and Bl(B), hi/lo
            s4 ah, al, bh, bl;
            split4(a, ah, al);
            split4(b, bh, bl);
            f4 acc = mfma16(ah, bl, zero4());
            acc = mfma16(al, bh, acc);
            return mfma16(ah, bh, acc);
        };
        f4 Z = plus_i(Q);  // Bl(I + Q_0)
#pragma unroll
        for (int k = 1; k < 4; ++k) {
            const f4 Pn = mul3(Q, P);
            if (k < 3) Q = mul3(P, Q);
            P = Pn;
            Z = mul3(plus_i(P), Z);
        }
        s4 zh, zl;
        split4(Z, zh, zl);
        char* const seg = reinterpret_cast<char*>(Lb + li * PF);  // row li: hi at bytes 0..31, lo at 32..63
        *reinterpret_cast<s4*>(seg + 8 * lq) = zh;
        *reinterpret_cast<s4*>(seg + 32 + 8 * lq) = zl;
    } else {
        const int r = lane >> 2, qq = lane & 3;  // one row segment per 4 lanes of one wave
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int blk = (wv - 4) + 4 * u;  // blocks 0..5: (1,0) (2,0) (2,1) (3,0) (3,1) (3,2)
            if (blk < 6) {
                const int bi = blk < 1 ? 1 : (blk < 3 ? 2 : 3), bj = blk < 1 ? 0 : (blk < 3 ? blk - 1 : blk - 3);
                float* const segf = F32 + (16 * bi + r) * PF + 16 * bj;
                const f4 x = *reinterpret_cast<const f4*>(segf + 4 * qq);
                s4 h4, l4;
                split4(x, h4, l4);
                char* const seg = reinterpret_cast<char*>(segf);
                *reinterpret_cast<s4*>(seg + 8 * qq) = h4;  // the segment's reads all precede these writes (one wave)
                *reinterpret_cast<s4*>(seg + 32 + 8 * qq) = l4;
            }
        }
    }
    __syncthreads();
    next.k = *reinterpret_cast<const uint4*>(p.k + noff);

    // ---- 7. W = T A0 and G = T beta without forming T: block forward substitution of (I - alpha) X = [A0 | beta]
    //         over the four 16-row blocks, X_i = T_ii (B_i + sum_{j<i} alpha_ij X_j), with the diagonal-block
    //         inverses T_ii and the blocks alpha_ij already split hi/lo by step 5.  Wave w owns one 16-column tile of X (w < 4: W columns 16 w ..; w >= 4: G
    //         columns 16 (w - 4) ..) and keeps its X_j in registers: the 16x16x16 MFMA returns a tile in exactly the
    //         layout it takes as its B operand.  3-term hi/lo products throughout (state path).
    {
        const bool is_w = wv < 4;
        const int col0 = 16 * (wv & 3);
        // right-hand side in the B layout, rows t = 16 bi + 4 lq + v, column col0 + li: A0 = Aq diag(2^m) read down
        // Aq's rows (transposing read), beta from its [s'][s] store
        const float sc = is_w ? sm.em[col0 + li] : 1.f;
        f4 X[4];
        s4 Xh[4], Xl[4];
#pragma unroll
        for (int bi = 0; bi < 4; ++bi) {
            s4 bh, bl;
            if (is_w) {
                const int o = (16 * bi + 4 * lq + (li >> 2)) * PB + col0 + 4 * (li & 3);
                bh = ld_tr4(Aq.h + o);
                bl = ld_tr4(Aq.l + o);
            } else {
                const int o = (col0 + li) * PB + 16 * bi + 4 * lq;
                bh = *reinterpret_cast<const s4*>(Be.h + o);
                bl = *reinterpret_cast<const s4*>(Be.l + o);
            }
            f4 acc;
#pragma unroll
            for (int v = 0; v < 4; ++v)
                acc[v] = (bf16_to_f32((uint16_t)bh[v]) + bf16_to_f32((uint16_t)bl[v])) * sc;
#pragma unroll
            for (int bj = 0; bj < bi; ++bj) {
                const char* const seg = reinterpret_cast<const char*>(F32 + (16 * bi + li) * PF + 16 * bj);
                const s4 ah4 = *reinterpret_cast<const s4*>(seg + 8 * lq), al4 = *reinterpret_cast<const s4*>(seg + 32 + 8 * lq);
                acc = mfma16(ah4, Xl[bj], acc);
                acc = mfma16(al4, Xh[bj], acc);
                acc = mfma16(ah4, Xh[bj], acc);
            }
            const char* const tseg = reinterpret_cast<const char*>(F32 + (16 * bi + li) * PF + 16 * bi);
            const s4 th4 = *reinterpret_cast<const s4*>(tseg + 8 * lq), tl4 = *reinterpret_cast<const s4*>(tseg + 32 + 8 * lq);
            s4 ch4, cl4;
            split4(acc, ch4, cl4);
            f4 x = mfma16(th4, cl4, zero4());
            x = mfma16(tl4, ch4, x);
            X[bi] = mfma16(th4, ch4, x);
            split4(X[bi], Xh[bi], Xl[bi]);
        }
        __syncthreads();  // alpha / T_ii (slots 0-1) and beta are read above; W and G are written over them
        next.r = *reinterpret_cast<const uint4*>(p.r + noff);
#pragma unroll
        for (int bi = 0; bi < 4; ++bi) st_split(is_w ? Wm : Gm, PB, 16 * bi, col0, X[bi]);
    }
    __syncthreads();

    next.v = *reinterpret_cast<const uint4*>(p.v + noff);

    // ---- 8. Q = R0 + rho W  (x = k, y = t; bf16 -> workspace [t][k])
    //          E = sigma + rho G (x = s', y = t; bf16 -> Em [t][s'], keep s' <= t)
    //          A = Gamma + Bh^T W (x = k2, y = k1; 3 terms -> workspace hi/lo)
    //          F = Kh^T + Bh^T G (x = s', y = k; 3 terms -> slots 2-3 as F[k][s'])
    //          (Bh = Bk diag(2^{g_C - m}), Kh likewise: Bk and Kk read down their rows, the factor applied to the
    //          fp32 result rows)
    // Wave wv owns tiles (bx, by) = (wv / 4 + 2 u, wv % 4).  The four products of a tile share their operands (W and
    // G as X, rho and the transposed Bk as Y), each fragment loaded once per contraction block.  rho is zero for
    // s > t, so for token tiles by < 2 the second contraction block of Q and E is skipped.
    bf4 q_keep[2];
    s4 ah_keep[2], al_keep[2];
    {
        // both tiles of this wave (same by) are accumulated together, so the Y operands (rho's row tile and the
        // transposed Bk tile, by) are read once per contraction block for the two
        const int by = wv & 3, y0 = 16 * by;
        f4 aqs[2], aes[2], aas[2], afs[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int x0 = 16 * ((wv >> 2) + 2 * u);
            const bf4 r4 = *reinterpret_cast<const bf4*>(Rq.h + (y0 + li) * PB + x0 + 4 * lq);
            const bf4 s4v = *reinterpret_cast<const bf4*>(Sig.h + (y0 + li) * PB + x0 + 4 * lq);
            const int o = (x0 + 4 * lq + (li >> 2)) * PB + y0 + 4 * (li & 3);
            const s4 kh4 = ld_tr4(Kk.h + o), kl4 = ld_tr4(Kk.l + o);  // Kk[x0 + 4 lq + v][y0 + li]
            aas[u] = zero4();
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                aqs[u][v] = (float)r4[v] * sm.em[x0 + 4 * lq + v];
                aes[u][v] = (float)s4v[v];
                afs[u][v] = bf16_to_f32((uint16_t)kh4[v]) + bf16_to_f32((uint16_t)kl4[v]);
            }
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const bf8 bh = ld8_tr(Bk.h, kb, y0), bl = ld8_tr(Bk.l, kb, y0);
            const bool use_rho = kb == 0 || by >= 2;
            bf8 rh;
            if (use_rho) rh = ld8(Rho.h + (y0 + li) * PB + 32 * kb + 8 * lq);
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int xo = (16 * ((wv >> 2) + 2 * u) + li) * PB + 32 * kb + 8 * lq;
                const bf8 wh = ld8(Wm.h + xo), wl = ld8(Wm.l + xo), gh = ld8(Gm.h + xo), gl = ld8(Gm.l + xo);
                if (use_rho) {
                    aqs[u] = mfma_bf16(wh, rh, aqs[u]);
                    aes[u] = mfma_bf16(gh, rh, aes[u]);
                }
                aas[u] = mfma_bf16(wh, bl, aas[u]);
                aas[u] = mfma_bf16(wl, bh, aas[u]);
                aas[u] = mfma_bf16(wh, bh, aas[u]);
                afs[u] = mfma_bf16(gh, bl, afs[u]);
                afs[u] = mfma_bf16(gl, bh, afs[u]);
                afs[u] = mfma_bf16(gh, bh, afs[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int bx = (wv >> 2) + 2 * u;
            const int x0 = 16 * bx;
            f4 aq = aqs[u], ae = aes[u], aa = aas[u], af = afs[u];
            // Q -> record (Q[t][k]: t tile by)
            bf4 qv;
#pragma unroll
            for (int v = 0; v < 4; ++v) qv[v] = (__bf16)aq[v];
            if constexpr (LDS_REC) q_keep[u] = qv;
            else *reinterpret_cast<bf4*>(rec + REC_Q + frag32_off(by, bx, lane)) = qv;
            // E -> Em, keep s' <= t
            // E = sigma + rho G is exactly zero above the diagonal (sigma is stored masked, rho and G are exactly
            // zero where the causal mask is), so only diagonal tiles are masked, as a guard
            if (bx == by) ae = mask_tile(ae, x0, y0, 2);
            st_hi(Em.h, PB, x0, y0, ae);
            // A[k1][k2] = gamma delta + 2^{g_C - m}[k1] sum_t W[t][k2] Bk[t][k1] -> record (k1 tile by)
            // F[k][s'] = 2^{g_C - m}[k] (Kk[s'][k] + sum_t G[t][s'] Bk[t][k]) -> Fm
            const float e1 = sm.eglm[y0 + li];
            f4 av;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                av[v] = aa[v] * e1;
                af[v] *= e1;
            }
            if (bx == by) {  // Gamma on the diagonal (bx, by are wave-uniform)
#pragma unroll
                for (int v = 0; v < 4; ++v) av[v] += (4 * lq + v == li) ? sm.gam[y0 + li] : 0.f;
            }
            s4 hv, lv;
            split4(av, hv, lv);
            if constexpr (LDS_REC) {
                ah_keep[u] = hv;
                al_keep[u] = lv;
            } else {
                *reinterpret_cast<s4*>(rec + REC_AH + frag32_off(by, bx, lane)) = hv;
                *reinterpret_cast<s4*>(rec + REC_AL + frag32_off(by, bx, lane)) = lv;
            }
            st_split(Fm, PB, x0, y0, af);
        }
    }
    __syncthreads();

    // ---- 9. H = F V (x = k, y = v; X split, V exact -> workspace fp32, H^T tiles);
    //          O_intra = E V (x = v, y = t -> workspace bf16, tiles of O_intra[t][v]); V read down its rows
    if constexpr (LDS_REC) {  // step 8's tiles of Q and A, now that their slots are free
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int bx = (wv >> 2) + 2 * u, by = wv & 3;
            *reinterpret_cast<bf4*>(rec + REC_Q + frag32_off(by, bx, lane)) = q_keep[u];
            *reinterpret_cast<s4*>(rec + REC_AH + frag32_off(by, bx, lane)) = ah_keep[u];
            *reinterpret_cast<s4*>(rec + REC_AL + frag32_off(by, bx, lane)) = al_keep[u];
        }
    }
    {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int prod = u >> 1, tile = wv + 8 * (u & 1), bx = tile >> 2, by = tile & 3;
            const int x0 = 16 * bx, y0 = 16 * by;
            if (prod == 0) {
                *reinterpret_cast<f4*>(rec + REC_HT + ((by * 4 + bx) * 64 + lane) * 16) =
                    mma<2>(zero4(), Fm, x0, Vt, y0, 0, 2);  // H^T[v][k]: v tile by, k tile bx
            } else {
                const f4 acc = mma<1>(zero4(), Vt, x0, Em, y0, 0, 2);  // O[t][v] = sum_s' Vt[v][s'] E[t][s']
                bf4 hv;
#pragma unroll
                for (int v = 0; v < 4; ++v) hv[v] = (__bf16)acc[v];
                *reinterpret_cast<bf4*>(rec + REC_OT + frag_off_bf16(bx, by, lane)) = hv;  // O[t][v]: v tile bx
            }
        }
    }
    __syncthreads();  // LDS is reused by the next item
}

// Persistent: a grid of about one workgroup per CU walks the (chunk, head) items item = blockIdx.x + k gridDim.x
// (chunk-major, head fastest, so with 8 | H and 8 | gridDim.x a head stays on one XCD) and prefetches the next
// item's operands into registers while the current one is processed.
__global__ __launch_bounds__(512) void wkv7_chunk_prep_kernel(const Params p, char* __restrict__ wsc,
                                                              const int32_t* __restrict__ plan, int64_t max_chunks,
                                                              int ncps) {
    __shared__ __attribute__((aligned(16))) PrepSmem sm;
    const int tid = threadIdx.x;
    const int row = tid >> 3, cb = (tid & 7) * 8;
    // ragged calls: only the chunk slots the plan filled (the table size is an upper bound); items without a chunk
    // would all write the one trash record at the same time
    int64_t nitems = max_chunks * p.H;
    if (p.cu) {
        const int64_t used = plan[2 * max_chunks + p.num_seqs + 1];
        nitems = std::max<int64_t>(0, std::min<int64_t>(used, max_chunks)) * p.H;
    }
    if ((int64_t)blockIdx.x >= nitems) return;
    const int64_t stride = gridDim.x, sj = stride / p.H;
    const int sh = (int)(stride % p.H);
    ItemPos pos = item_pos(p, ncps, blockIdx.x);
    Item cur = describe_item(p, plan, max_chunks, pos);
    RawIn rc = load_item(p, cur, row, cb);
    settle(rc);
    while (pos.item < nitems) {
        ItemPos np = pos;
        advance(np, p, ncps, stride, sj, sh);
        Item nxt{};
        nxt.rec = max_chunks * p.H;
        if (np.item < nitems) nxt = describe_item(p, plan, max_chunks, np);
        // the next item's operands are loaded during `cur`; every item runs the same instruction stream (an item
        // without a chunk computes on zeros and writes the trash record), so the number of vector memory operations
        // between a prefetch and its use is fixed
        RawIn rn;
        prep_item<false>(p, cur, rc, wsc, sm, item_offset(p, nxt, row, cb), rn);
        cur = nxt;
        rc = rn;
        pos = np;
    }
}

typedef short s8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ s4 half4(s8 x, int hi) {
    return hi ? __builtin_shufflevector(x, x, 4, 5, 6, 7) : __builtin_shufflevector(x, x, 0, 1, 2, 3);
}

// One half of a record as one of the two wavefronts of a column group uses it: row tiles (of A, H) and token tiles
// (of Q, O_intra) 2 hf and 2 hf + 1.
struct ScanRecH {
    s8 ah[2][2], al[2][2];  // [row tile 2 hf + x][k block c]
    s8 q[2][2];             // [token tile 2 hf + x][k block c]
    f4 h[2];                // [k tile 2 hf + x]
    s8 o;                   // token tile pair hf
};

template <bool LDS_REC = false>
__device__ __forceinline__ void scan_load_half(ScanRecH& r, const char* rec, int vg, int hf, int lane) {
    const char* const b = LDS_REC ? rec : uniform_ptr(rec);
    const int lo = lane * 16;
#pragma unroll
    for (int x = 0; x < 2; ++x) {
        const int X = 2 * hf + x;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            r.ah[x][c] = *reinterpret_cast<const s8*>(b + REC_AH + (X * 2 + c) * 1024 + lo);
            r.al[x][c] = *reinterpret_cast<const s8*>(b + REC_AL + (X * 2 + c) * 1024 + lo);
            r.q[x][c] = *reinterpret_cast<const s8*>(b + REC_Q + (X * 2 + c) * 1024 + lo);
        }
        r.h[x] = *reinterpret_cast<const f4*>(b + REC_HT + (vg * 4 + X) * 1024 + lo);
    }
    r.o = *reinterpret_cast<const s8*>(b + REC_OT + (vg * 2 + hf) * 1024 + lo);
}

// The state as 16x16x32 operands, one contraction block c at a time (X = S[2 c], Y = S[2 c + 1]).  Lane (i, q)
// holds S[16 r + 4 q + e][col] (e = 0..3) of the k tiles r; the operand of contraction block c needs
// S[32 c + 8 q + j][col], j = 0..7, which lanes 2 (q & 1) and 2 (q & 1) + 1 of tile 2 c + (q >> 1) hold.  With X = tile 2 c, Y = tile 2 c + 1 and rows of 16 lanes: v_permlane32_swap(X, Y) gives
// P = (X0, X1, Y0, Y1), Q = (X2, X3, Y2, Y3), and v_permlane16_swap(P, Q) gives (X0, X2, Y0, Y2) -- values j = 0..3
// for every row q -- and (X1, X3, Y1, Y3) -- values j = 4..7.  The same vector is the A operand of S^T.
__device__ __forceinline__ void state_operand_block(const f4& X, const f4& Y, bf8& Bh, bf8& Bl) {
    uint32_t h[2][2], l[2][2];
    const f4 xs[2] = {X, Y};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int w = 0; w < 2; ++w) split_pair(xs[u][2 * w], xs[u][2 * w + 1], h[u][w], l[u][w]);
    }
    uint32_t oh[4], ol[4];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
        const auto ph = __builtin_amdgcn_permlane32_swap(h[0][w], h[1][w], false, false);
        const auto rh = __builtin_amdgcn_permlane16_swap(ph[0], ph[1], false, false);
        oh[w] = rh[0];
        oh[2 + w] = rh[1];
        const auto pl = __builtin_amdgcn_permlane32_swap(l[0][w], l[1][w], false, false);
        const auto rl = __builtin_amdgcn_permlane16_swap(pl[0], pl[1], false, false);
        ol[w] = rl[0];
        ol[2 + w] = rl[1];
    }
    Bh = __builtin_bit_cast(bf8, oh);
    Bl = __builtin_bit_cast(bf8, ol);
}

constexpr int kPlanSortRows = 4096;    // ragged calls: longest-first ordering of up to this many chunked rows
constexpr int kScanRaggedGrid = 2048;  // ragged calls: scan workgroups (four rounds of residency at two per CU)
constexpr int kScanDepth = 4;  // chunk record register sets per lane (three in flight, one in use)
// Chunks per pass of the scan's main loop, fully unrolled: the compiler counts outstanding loads exactly only within
// straight-line code and drains them all at a loop header, so a long body keeps the record loads in flight across
// most chunks (the remaining chunks run in passes of kScanDepth).
constexpr int kScanUnroll = 16;

// The shares of a chunk record in the scan: state wavefront r (row tile r) reads A's row tile r (hi, lo, both
// contraction blocks) and H^T's k tile r; output wavefront t reads Q's token tile t and the O_intra pair holding it.
struct ScanRecS {
    s8 ah[2], al[2];  // [k block c]
    f4 h;
};
struct ScanRecY {
    s8 q[2];  // [k block c]
    s4 o;     // token tile t's half of the O_intra piece of pair t / 2
};

// The record loads go through a buffer resource at the record (wave-uniform) with the lane's 16-byte slot as the
// vector offset and the share's offset as the scalar one, so a refill costs no vector address arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rec_rsrc(const char* rec) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(uniform_ptr(rec)), 0, kChunkBytes,
                                             0x00020000 /* raw 32-bit buffer, gfx9 family */);
}
__device__ __forceinline__ s8 rec_s8(__amdgpu_buffer_rsrc_t r, int lo, int off) {
    return __builtin_bit_cast(s8, __builtin_amdgcn_raw_buffer_load_b128(r, lo, off, 0));
}

__device__ __forceinline__ void scan_load_s(ScanRecS& r, const char* rec, int vg, int t, int lane) {
    const __amdgpu_buffer_rsrc_t rs = rec_rsrc(rec);
    const int lo = lane * 16;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        r.ah[c] = rec_s8(rs, lo, REC_AH + (t * 2 + c) * 1024);
        r.al[c] = rec_s8(rs, lo, REC_AL + (t * 2 + c) * 1024);
    }
    r.h = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, lo, REC_HT + (vg * 4 + t) * 1024, 0));
}

__device__ __forceinline__ void scan_load_y(ScanRecY& r, const char* rec, int vg, int t, int lane) {
    const __amdgpu_buffer_rsrc_t rs = rec_rsrc(rec);
    const int lo = lane * 16;
#pragma unroll
    for (int c = 0; c < 2; ++c) r.q[c] = rec_s8(rs, lo, REC_Q + (t * 2 + c) * 1024);
    r.o = __builtin_bit_cast(s4, __builtin_amdgcn_raw_buffer_load_b64(rs, lo + 8 * (t & 1), REC_OT + (vg * 2 + (t >> 1)) * 1024, 0));
}

// The state of one column group as published each chunk for the 16x16x32 operands: [row tile][column][row in tile]
// bf16, hi and lo (column-major within a tile, so that the 8 consecutive rows an operand lane needs are 16 contiguous
// bytes, and the 4 rows a result lane holds are 8).
struct ScanEx {
    __bf16 v[2][2][4][16][16];  // [buffer][hi, lo][row tile][column][row]
};

// A workgroup of eight wavefronts owns one (row, head, 16-column group vg); block b -> XCD b % 8, and the 4 groups
// of a (row, head) share an XCD, so 3 of the 4 reads of a chunk's A and Q hit that XCD's L2.
//   * State wavefront r = 0..3 holds row tile r of the state in the 16x16 MFMA result layout -- lane (i, q) holds
//     S[16 r + 4 q + e][16 vg + i], e = 0..3 -- so the state stays in registers from chunk to chunk.  Each chunk it
//     runs  S_r <- A_r S + H_r  (6 MFMAs: 2 contraction blocks, 3 terms on the hi/lo split), splits the new tile hi/lo
//     and publishes it in LDS (one 8-byte store per lane and part; double-buffered, one workgroup barrier per chunk);
//     after the barrier every wavefront reads the operand of contraction block c (rows 32 c + 8 q .. + 7 of column
//     i) as one 16-byte load per part.
//   * Output wavefront 4 + t computes  y_t^T = S^T Q_t^T + O_intra,t^T  for token tile t (2 MFMAs on S hi) from the
//     same published operands, off the state's dependency chain.
// Chunk records stream through a ring of kScanDepth register sets per wavefront (each loads only its share).  Every
// step issues the same memory operations (the refill index is clamped to the last chunk; stores that must not land
// go to the workspace's trash record), so within a pass the compiler counts the outstanding loads exactly and waits
// only for the record about to be used.
// Measured for one row of T = 4096, H = 64 (cycle stamps per phase in an instrumented copy): a chunk step is bound by
// the CU's vector-memory pipeline, not by the MFMA chain -- each workgroup streams about 30 KB of record per chunk
// (all of A and Q, its slices of H and O_intra), and issuing a 16-byte-per-lane load waits about 110 cycles for the
// pipeline.  This layout takes 50 us; two wavefronts each holding two row tiles, re-forming operands with lane swaps
// and computing y themselves, 56 us; one wavefront holding all four row tiles, 61 us.
// One work item b of the scan: (row, head) pair (b >> 5) * 8 + (b & 7) of the rows the call chunks, column group
// (b >> 3) & 3 -- numbered so that, with a grid (or grid stride) that is a multiple of 8, the 4 column groups of a
// pair run on one XCD and share its L2.  `rows` is the number of chunked rows; `row_of` lists them (ragged calls) or
// is null (dense calls: every row).  `buf` is the exchange buffer index, carried across a workgroup's items.
constexpr int kScanWaves = 8;
__device__ __forceinline__ void scan_item(const Params& p, char* __restrict__ wsc, const int32_t* __restrict__ plan,
                                          int64_t max_chunks, int ncps, int64_t b, int64_t rows,
                                          const int32_t* row_of, ScanEx& ex, int& buf) {
    const int xcd = (int)(b & 7), rsl = (int)(b >> 3), vg = rsl & 3;
    const int64_t pair = (int64_t)(rsl >> 2) * 8 + xcd;
    if (pair >= rows * p.H) return;  // uniform over the workgroup, as are the returns below
    const int k = (int)(pair / p.H), h = (int)(pair % p.H);
    const int n = row_of ? row_of[k] : k;
    int64_t bos;
    int L;
    seq_extent(p, n, bos, L);
    if (!owns_row(p, L)) return;

    const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = wv & 3;        // row tile (state wavefronts) or token tile (output wavefronts)
    const bool ywave = wv >= 4;  // wave-uniform role
    const int64_t j0 = p.cu ? (int64_t)plan[2 * max_chunks + n] : (int64_t)n * ncps;
    // the chunk table never exceeds max_chunks for valid cu_seqlens; the clamp keeps invalid ones in bounds
    const int nch = (int)std::max<int64_t>(0, std::min<int64_t>((L + C - 1) / C, max_chunks - j0));
    const float* src = state_src(p, n, h);
    float* dst = state_dst(p, n, h);
    const int col = 16 * vg + i;  // the state column this lane holds

    f4 S;  // state wavefronts: row tile t
    if (!ywave) {
#pragma unroll
        for (int e = 0; e < 4; ++e) S[e] = src ? src[(16 * t + 4 * q + e) * HS + col] : 0.f;
        if (nch == 0 && dst) {  // no chunks (length 0): the state passes through
#pragma unroll
            for (int e = 0; e < 4; ++e) dst[(16 * t + 4 * q + e) * HS + col] = S[e];
        }
    }
    if (nch == 0) return;
    // state operands of the chunk about to run, as 16x16x32 blocks c = 0, 1 (the output wavefronts use only hi)
    bf8 Bh[2], Bl[2];
    auto publish = [&]() {  // state wavefronts: rows 4 q .. 4 q + 3 of column i of tile t, hi and lo
        s4 hv, lv;
        split4(S, hv, lv);
        *reinterpret_cast<s4*>(&ex.v[buf][0][t][i][4 * q]) = hv;
        *reinterpret_cast<s4*>(&ex.v[buf][1][t][i][4 * q]) = lv;
    };
    auto collect = [&]() {  // after the barrier: rows 32 c + 8 q .. + 7 (tile 2 c + q / 2, rows 8 (q & 1) ..) of column i
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            Bh[c] = *reinterpret_cast<const bf8*>(&ex.v[buf][0][2 * c + (q >> 1)][i][8 * (q & 1)]);
            if (!ywave) Bl[c] = *reinterpret_cast<const bf8*>(&ex.v[buf][1][2 * c + (q >> 1)][i][8 * (q & 1)]);
        }
        buf ^= 1;  // the next writes go to the other buffer: every wavefront reads this one before the next barrier
    };
    if (!ywave) publish();
    __syncthreads();
    collect();

    const char* const rec0 = wsc + (j0 * p.H + h) * (int64_t)kChunkBytes;
    const int64_t rec_stride = (int64_t)p.H * kChunkBytes;
    if (!ywave) {
        ScanRecS ring[kScanDepth];
#pragma unroll
        for (int d = 0; d < kScanDepth - 1; ++d) scan_load_s(ring[d], rec0 + std::min(d, nch - 1) * rec_stride, vg, t, lane);
        // chunk cc (ring set d = cc % kScanDepth, a compile-time index in every unrolled copy)
        auto step = [&](int cc, auto D) __attribute__((always_inline)) {
            constexpr int d = decltype(D)::value;
            // the set used one chunk ago takes the record kScanDepth - 1 chunks ahead; its loads issue while the
            // exchange's LDS reads are in flight
            scan_load_s(ring[(d + kScanDepth - 1) % kScanDepth],
                        rec0 + std::min(cc + kScanDepth - 1, nch - 1) * rec_stride, vg, t, lane);
            const ScanRecS& R = ring[d];
            // two accumulators (one per contraction block), interleaved so that no MFMA waits on the one before
            f4 n0 = R.h, n1 = zero4();
            const bf8 ah0 = __builtin_bit_cast(bf8, R.ah[0]), al0 = __builtin_bit_cast(bf8, R.al[0]);
            const bf8 ah1 = __builtin_bit_cast(bf8, R.ah[1]), al1 = __builtin_bit_cast(bf8, R.al[1]);
            n0 = mfma_bf16(ah0, Bl[0], n0);
            n1 = mfma_bf16(ah1, Bl[1], n1);
            n0 = mfma_bf16(al0, Bh[0], n0);
            n1 = mfma_bf16(al1, Bh[1], n1);
            n0 = mfma_bf16(ah0, Bh[0], n0);
            n1 = mfma_bf16(ah1, Bh[1], n1);
            if (cc < nch) {  // wave-uniform
#pragma unroll
                for (int e = 0; e < 4; ++e) S[e] = n0[e] + n1[e];
            }
            publish();
            __syncthreads();
            collect();
        };
        int c0 = 0;
        for (; c0 + kScanUnroll <= nch; c0 += kScanUnroll)
            unroll<kScanUnroll>([&](auto J) __attribute__((always_inline)) {
                step(c0 + decltype(J)::value, std::integral_constant<int, decltype(J)::value % kScanDepth>{});
            });
        for (; c0 < nch; c0 += kScanDepth)
            unroll<kScanDepth>([&](auto J) __attribute__((always_inline)) { step(c0 + decltype(J)::value, J); });
        if (dst) {
#pragma unroll
            for (int e = 0; e < 4; ++e) dst[(16 * t + 4 * q + e) * HS + col] = S[e];
        }
    } else {
        // stores that must not land go to the trash record, 2 KB per block slot (24 slots) so that blocks do not all
        // hit the same lines
        char* const trash = wsc + max_chunks * p.H * (int64_t)kChunkBytes + (int)(b % 24) * 2048 + lane * 8;
        uint16_t* const obase = p.o ? p.o + bos * p.o_tok_stride + (int64_t)h * HS + 16 * vg + 4 * q : nullptr;
        ScanRecY ring[kScanDepth];
#pragma unroll
        for (int d = 0; d < kScanDepth - 1; ++d) scan_load_y(ring[d], rec0 + std::min(d, nch - 1) * rec_stride, vg, t, lane);
        auto step = [&](int cc, auto D) __attribute__((always_inline)) {
            constexpr int d = decltype(D)::value;
            scan_load_y(ring[(d + kScanDepth - 1) % kScanDepth],
                        rec0 + std::min(cc + kScanDepth - 1, nch - 1) * rec_stride, vg, t, lane);
            const ScanRecY& R = ring[d];
            f4 y;
            const s4 o4 = R.o;
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = bf16_to_f32((uint16_t)o4[e]);
#pragma unroll
            for (int c = 0; c < 2; ++c) y = mfma_bf16(Bh[c], __builtin_bit_cast(bf8, R.q[c]), y);
            // lane (i, q) holds y[token 16 t + i][columns 16 vg + 4 q .. + 3]
            const int tok = cc * C + 16 * t + i;
            uint2 pk;
            pk.x = pack_bf16x2(y[0], y[1]);
            pk.y = pack_bf16x2(y[2], y[3]);
            char* const out = (cc < nch && tok < L && obase)
                                  ? reinterpret_cast<char*>(obase + (int64_t)tok * p.o_tok_stride)
                                  : trash + t * 512;
            *reinterpret_cast<uint2*>(out) = pk;
            __syncthreads();  // the state wavefronts have published the next chunk's operands
            collect();
        };
        int c0 = 0;
        for (; c0 + kScanUnroll <= nch; c0 += kScanUnroll)
            unroll<kScanUnroll>([&](auto J) __attribute__((always_inline)) {
                step(c0 + decltype(J)::value, std::integral_constant<int, decltype(J)::value % kScanDepth>{});
            });
        for (; c0 < nch; c0 += kScanDepth)
            unroll<kScanDepth>([&](auto J) __attribute__((always_inline)) { step(c0 + decltype(J)::value, J); });
    }
}

// Dense calls: one item per workgroup.  Ragged calls: a bounded grid walks the items of the rows the plan marked as
// chunked (a grid over every row would be almost all empty workgroups when decode rows dominate, and their dispatch
// costs more than the work).
__global__ __launch_bounds__(64 * kScanWaves) void wkv7_chunk_scan_kernel(const Params p, char* __restrict__ wsc,
                                                                          const int32_t* __restrict__ plan,
                                                                          int64_t max_chunks, int ncps) {
    __shared__ __attribute__((aligned(16))) ScanEx ex;
    int buf = 0;
    if (!p.cu) {
        scan_item(p, wsc, plan, max_chunks, ncps, blockIdx.x, p.num_seqs, nullptr, ex, buf);
        return;
    }
    const int32_t* const rows_list = plan + 2 * max_chunks + p.num_seqs + 2;
    const int64_t rows = std::min<int64_t>(std::max<int32_t>(rows_list[p.num_seqs], 0), p.num_seqs);
    const int64_t items = ((rows * p.H + 7) / 8) * 8 * 4;
    for (int64_t it = blockIdx.x; it < items; it += gridDim.x)
        scan_item(p, wsc, plan, max_chunks, ncps, it, rows, rows_list, ex, buf);
}

// Chunk table of a ragged call: rows owned by the chunked path get ceil(len / C) consecutive chunk slots.
__global__ __launch_bounds__(1024) void wkv7_chunk_plan_kernel(const Params p, int32_t* __restrict__ plan,
                                                               int64_t max_chunks) {
    __shared__ int32_t scan[1024], fscan[1024];
    __shared__ int32_t base, fbase;
    const int tid = threadIdx.x;
    int32_t* const chunk_seq = plan;
    int32_t* const chunk_idx = plan + max_chunks;
    int32_t* const seq_off = plan + 2 * max_chunks;
    int32_t* const rows_list = seq_off + p.num_seqs + 2;  // the rows the chunked path owns, in order, then their count
    if (tid == 0) base = fbase = 0;
    __syncthreads();
    for (int n0 = 0; n0 < p.num_seqs; n0 += 1024) {
        const int n = n0 + tid;
        int32_t cnt = 0, flag = 0;  // flag: the chunked path owns the row (an empty owned row passes its state)
        if (n < p.num_seqs) {
            int64_t bos;
            int L;
            seq_extent(p, n, bos, L);
            flag = owns_row(p, L) ? 1 : 0;
            cnt = flag ? (L + C - 1) / C : 0;
        }
        scan[tid] = cnt;
        fscan[tid] = flag;
        __syncthreads();
        for (int off = 1; off < 1024; off <<= 1) {
            const int32_t add = tid >= off ? scan[tid - off] : 0;
            const int32_t fadd = tid >= off ? fscan[tid - off] : 0;
            __syncthreads();
            scan[tid] += add;
            fscan[tid] += fadd;
            __syncthreads();
        }
        const int32_t excl = base + scan[tid] - cnt;
        if (n < p.num_seqs) {
            seq_off[n] = excl;
            for (int32_t c = 0; c < cnt; ++c) {
                if (excl + c < max_chunks) {
                    chunk_seq[excl + c] = n;
                    chunk_idx[excl + c] = c;
                }
            }
            if (flag) rows_list[fbase + fscan[tid] - 1] = n;
        }
        __syncthreads();
        if (tid == 1023) {
            base += scan[1023];
            fbase += fscan[1023];
        }
        __syncthreads();
    }
    if (tid == 0) {
        seq_off[p.num_seqs] = base;
        seq_off[p.num_seqs + 1] = (int32_t)min((int64_t)base, max_chunks);
        rows_list[p.num_seqs] = fbase;
    }
    // Longest rows first: the scan walks rows_list in order with a bounded grid, so a long row that started last
    // would set the call's length.  Rows are grouped by floor(log2(chunks)), descending (the order inside a group and
    // the order itself do not change any result, only when each row's scan starts).  Lists longer than the LDS copy
    // keep the natural order.
    __syncthreads();
    const int32_t count = fbase;
    if (count > 1 && count <= kPlanSortRows) {
        __shared__ int32_t rows_copy[kPlanSortRows];
        __shared__ int32_t hist[33], cursor[33];
        if (tid < 33) hist[tid] = 0;
        for (int k = tid; k < count; k += 1024) rows_copy[k] = rows_list[k];
        __syncthreads();
        auto bucket = [&](int n) {
            const int32_t cnt = seq_off[n + 1 < p.num_seqs ? n + 1 : p.num_seqs] - seq_off[n];  // chunks of row n
            return cnt > 0 ? 32 - __builtin_clz((uint32_t)cnt) : 0;                            // 0 .. 32
        };
        for (int k = tid; k < count; k += 1024) atomicAdd(&hist[bucket(rows_copy[k])], 1);
        __syncthreads();
        if (tid == 0) {
            int32_t acc = 0;
            for (int b2 = 32; b2 >= 0; --b2) {
                cursor[b2] = acc;
                acc += hist[b2];
            }
        }
        __syncthreads();
        for (int k = tid; k < count; k += 1024) {
            const int n = rows_copy[k];
            rows_list[atomicAdd(&cursor[bucket(n)], 1)] = n;
        }
    }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }


// ---------------------------------------------------------------------------------------------------------------
// Chain kernel: a whole ragged step (token-serial rows and chunked rows) in one dispatch, with no workspace.
// Each workgroup takes whole (row, head) chains of chunked rows and walks their chunks in order: prep_item builds
// the chunk's record in LDS and chain_step applies it at once to the state, which stays in the registers of the
// eight wavefronts (wavefront wv: column group wv >> 1, row tiles 2 (wv & 1), 2 (wv & 1) + 1).  So the 48 KB record
// never leaves the CU, and no second kernel, plan kernel or cross-workgroup synchronisation is needed.  The price is
// that a chain's chunks are serial on one CU: the launcher picks this kernel when the rows are short enough for that
// not to set the call's length (many chains, few chunks each -- a continuous-batching step of prefill rows and
// decode rows), and the two-kernel path for long rows.
// ---------------------------------------------------------------------------------------------------------------

// One chunk of a chain on the LDS record `rec`: y <- Q S + O_intra for this wavefront's token tiles 2 hf, 2 hf + 1
// (column group vg), S <- A S + H for its row tiles, then the new state's operand halves are exchanged through
// `ex` (one barrier).  (Bh, Bl) hold the state at the chunk start as the 16x16x32 operands of contraction blocks 0, 1.
__device__ __forceinline__ void chain_step(const Params& p, const char* rec, f4 (&S)[2], bf8 (&Bh)[2], bf8 (&Bl)[2],
                                           bf8 (*ex)[2][64], int vg, int hf, int lane, int64_t bos, int c, int L,
                                           int h) {
    const int i = lane & 15, q = lane >> 4;
    ScanRecH R;
    scan_load_half<true>(R, rec, vg, hf, lane);
    f4 nS[2];
#pragma unroll
    for (int x = 0; x < 2; ++x) nS[x] = R.h[x];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
        for (int x = 0; x < 2; ++x) {
            const bf8 ah = __builtin_bit_cast(bf8, R.ah[x][cb]), al = __builtin_bit_cast(bf8, R.al[x][cb]);
            nS[x] = mfma_bf16(ah, Bl[cb], nS[x]);
            nS[x] = mfma_bf16(al, Bh[cb], nS[x]);
            nS[x] = mfma_bf16(ah, Bh[cb], nS[x]);
        }
    }
    f4 y[2];
#pragma unroll
    for (int x = 0; x < 2; ++x) {
        const s4 o4 = half4(R.o, x);
#pragma unroll
        for (int e = 0; e < 4; ++e) y[x][e] = bf16_to_f32((uint16_t)o4[e]);
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) y[x] = mfma_bf16(Bh[cb], __builtin_bit_cast(bf8, R.q[x][cb]), y[x]);
    }
    if (p.o) {
        uint16_t* const obase = p.o + bos * p.o_tok_stride + (int64_t)h * HS + 16 * vg + 4 * q;
#pragma unroll
        for (int x = 0; x < 2; ++x) {
            // lane (i, q) holds y[token 16 t + i][columns 16 vg + 4 q .. + 3], t = 2 hf + x
            const int tok = c * C + 16 * (2 * hf + x) + i;
            if (tok < L) {
                uint2 pk;
                pk.x = pack_bf16x2(y[x][0], y[x][1]);
                pk.y = pack_bf16x2(y[x][2], y[x][3]);
                *reinterpret_cast<uint2*>(obase + (int64_t)tok * p.o_tok_stride) = pk;
            }
        }
    }
#pragma unroll
    for (int x = 0; x < 2; ++x) S[x] = nS[x];
}

// The state's operand halves, exchanged between the two wavefronts of a column group (one barrier).
__device__ __forceinline__ void chain_exchange(const f4 (&S)[2], bf8 (&Bh)[2], bf8 (&Bl)[2], bf8 (*ex)[2][64], int hf,
                                               int lane) {
    bf8 oh, ol;
    state_operand_block(S[0], S[1], oh, ol);
    ex[hf][0][lane] = oh;
    ex[hf][1][lane] = ol;
    __syncthreads();
    const bf8 th = ex[1 - hf][0][lane], tl = ex[1 - hf][1][lane];
    Bh[0] = hf ? th : oh;
    Bl[0] = hf ? tl : ol;
    Bh[1] = hf ? oh : th;
    Bl[1] = hf ? ol : tl;
}

// Chain (row, head) -> Item of its chunk c (the chain's rows are longer than rec_max_len, so c < chunks exists).
__device__ __forceinline__ Item chain_item(int h, int64_t bos, int L, int c) {
    Item it{};
    it.ok = true;
    it.h = h;
    it.Lc = min(C, L - c * C);
    it.tok0 = bos + (int64_t)c * C;
    return it;
}

// Token-serial pairs per chunk-item of chain work, for balancing: a pair moves 33.7 KB (HBM-bound), a chunk-item
// keeps a CU busy for about 10 us; with a few workgroups on the token-serial rows at a time, the eight wavefronts of
// one take about as long for 48 pairs as for a chunk-item (measured on the mixed step: 24, 48, 96 gave 365, 362 and
// 362-368 us).
constexpr int kPairsPerItem = 48;
// Chain assignment: when the workgroups come in whole groups of H (G % H == 0, at most kChainLptGroups groups) and
// there are at most kChainLptRows chained rows, longest row first, each row's H chains to the group with the least
// chain work so far; otherwise the snake.  For the mixed step's eight prefill rows (28, 22, 19, 16, 10, 10, 9, 7
// chunks over 4 groups of 64) that is 28 | 22 + 9 | 19 + 10 | 16 + 10 + 7, the busiest workgroup 33 chunk-items
// against 35 for the snake's pairs.
constexpr int kChainLptRows = 64;    // the list of one workgroup's chains holds at most this many
constexpr int kChainLptGroups = 64;

__global__ __launch_bounds__(512) void wkv7_chain_kernel(const Params p) {
    __shared__ __attribute__((aligned(16))) PrepSmem sm;
    __shared__ int32_t wave_count[8], wave_count2[8];
    __shared__ int32_t max_load, list_len;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = (int)gridDim.x, b = (int)blockIdx.x;

    // ---- 1. plan, the same in every workgroup (num_seqs <= kChainMaxSeqs = the workgroup size, gridDim.x <=
    //         kChainMaxSeqs: both checked by the launcher; one row / one workgroup per thread):
    //   crow / cnch: the chain rows (longer than rec_max_len), longest first (rank = rows with more chunks, or as
    //   many and an earlier index); srow: the token-serial rows in row order; start: each workgroup's range of
    //   token-serial pairs, proportional to how far its chain work (snake assignment below) falls short of the
    //   longest, plus an even share.
    int32_t* const crow = reinterpret_cast<int32_t*>(sm.slot[16]);  // kept to the end of the kernel
    int32_t* const cnch = crow + kChainMaxSeqs;
    int32_t* const srow = cnch + kChainMaxSeqs;
    int32_t* const start = srow + kChainMaxSeqs;                     // [G + 1]
    int32_t* const list = start + kChainMaxSeqs + 1;                 // [kChainLptRows]: chains j (lpt)
    int nrows, nshort;
    bool lpt;
    {
        int32_t* const tmp_row = reinterpret_cast<int32_t*>(sm.slot[0]);
        int32_t* const tmp_nch = tmp_row + kChainMaxSeqs;
        int64_t bos = 0;
        int L = 0;
        bool chain = false, shrt = false;
        if (tid < p.num_seqs) {
            seq_extent(p, tid, bos, L);
            chain = owns_row(p, L);
            shrt = !chain;
        }
        const uint64_t bal = __ballot(chain), bal2 = __ballot(shrt);
        if (lane == 0) {
            wave_count[wv] = __popcll(bal);
            wave_count2[wv] = __popcll(bal2);
        }
        __syncthreads();
        int off = 0, off2 = 0;
        nrows = nshort = 0;
#pragma unroll
        for (int w2 = 0; w2 < 8; ++w2) {
            off += w2 < wv ? wave_count[w2] : 0;
            off2 += w2 < wv ? wave_count2[w2] : 0;
            nrows += wave_count[w2];
            nshort += wave_count2[w2];
        }
        const uint64_t below = (1ull << lane) - 1;
        if (chain) {
            const int k = off + __popcll(bal & below);
            tmp_row[k] = tid;
            tmp_nch[k] = (L + C - 1) / C;
        }
        if (shrt) srow[off2 + __popcll(bal2 & below)] = tid;
        __syncthreads();
        if (tid < nrows) {
            const int mine = tmp_nch[tid];
            int rank = 0;
            for (int j = 0; j < nrows; ++j) {
                const int o = tmp_nch[j];
                rank += (o > mine || (o == mine && j < tid)) ? 1 : 0;
            }
            crow[rank] = tmp_row[tid];
            cnch[rank] = mine;
        }
        if (tid == 0) {
            max_load = 0;
            list_len = 0;
        }
        __syncthreads();
        // chain load (chunk-items) of workgroup tid; with lpt, this workgroup's chains are listed in `list`
        const int64_t nchains = (int64_t)nrows * p.H;
        lpt = nrows > 0 && nrows <= kChainLptRows && G % p.H == 0 && G / p.H <= kChainLptGroups;
        int load = 0;
        if (lpt) {
            // Workgroups g H .. g H + H - 1 form group g.  Each row's H chains go to the least-loaded group (the
            // lowest index on ties), workgroup g H + h taking head h, so a group's workgroups always carry equal work
            // and this is exactly the assignment that gives each chain to a least-loaded workgroup.  One thread
            // deals the rows (rows x groups steps), then every workgroup reads its group's rows.
            const int groups = G / p.H, gb = b / p.H;
            int32_t* const gl = reinterpret_cast<int32_t*>(sm.slot[1]);  // [groups] chain work per group, scratch
            if (tid == 0) {
                for (int g = 0; g < groups; ++g) gl[g] = 0;
                for (int r = 0; r < nrows; ++r) {
                    int best = 0;
                    for (int g = 1; g < groups; ++g) best = gl[g] < gl[best] ? g : best;
                    gl[best] += cnch[r];
                    if (best == gb) list[list_len++] = r * p.H + (b - gb * p.H);
                }
            }
            __syncthreads();
            if (tid < G) {
                load = gl[tid / p.H];
                atomicMax(&max_load, load);
            }
        } else if (tid < G) {  // snake
            for (int64_t k = 0;; ++k) {
                const int64_t j = k * G + ((k & 1) ? G - 1 - tid : tid);
                if (j >= nchains) break;
                load += cnch[j / p.H];
            }
            atomicMax(&max_load, load);
        }
        __syncthreads();
        // token-serial pairs: weight = deficit + even share (in pairs), then an exclusive prefix over workgroups
        const int64_t npairs = (int64_t)nshort * p.H;
        const int64_t even = (npairs + G - 1) / G;
        int64_t* const wgt = reinterpret_cast<int64_t*>(tmp_row);  // [G + 1], reusing the scratch
        if (tid < G) wgt[tid] = (int64_t)(max_load - load) * kPairsPerItem + even;
        __syncthreads();
        if (tid == 0) {
            int64_t acc = 0;
            for (int w2 = 0; w2 < G; ++w2) {
                const int64_t x = wgt[w2];
                wgt[w2] = acc;
                acc += x;
            }
            wgt[G] = acc;
        }
        __syncthreads();
        if (tid <= G) start[tid] = (int32_t)(wgt[G] > 0 ? npairs * wgt[tid] / wgt[G] : 0);
        __syncthreads();
    }

    // ---- 2. chains j = rank * H + h: this workgroup's list (lpt), or snake-assigned: pass k covers chains
    //         [k G, (k + 1) G); workgroup b takes k G + b on even passes and k G + G - 1 - b on odd ones (the
    //         longest chains are spread over all workgroups, and a workgroup with a long chain in one pass gets a
    //         short one in the next)
    const int64_t nchains = (int64_t)nrows * p.H;
    const int vg = wv >> 1, hf = wv & 1;
    bf8 (*const ex)[2][64] = reinterpret_cast<bf8 (*)[2][64]>(sm.slot[12]) + 2 * vg;  // [hf][hi, lo][lane]
    const int trow = tid >> 3, cb = (tid & 7) * 8;
    const int i = lane & 15, q = lane >> 4, col = 16 * vg + i;
    const int nlist = list_len;
    auto chain_at = [&](int64_t k, int& n, int& h) {
        int64_t j;
        if (lpt) {
            if (k >= nlist) return false;
            j = list[k];
        } else {
            j = k * G + ((k & 1) ? G - 1 - b : b);
            if (j >= nchains) return false;
        }
        n = crow[j / p.H];
        h = (int)(j % p.H);
        return true;
    };
    int n, h;
    if (chain_at(0, n, h)) {  // uniform over the workgroup
        int64_t bos;
        int L;
        seq_extent(p, n, bos, L);
        RawIn raw = load_item(p, chain_item(h, bos, L, 0), trow, cb);
        for (int64_t k = 0;; ++k) {
            const int nch = (L + C - 1) / C;
            const float* src = state_src(p, n, h);
            float* dst = state_dst(p, n, h);
            f4 S[2];
#pragma unroll
            for (int x = 0; x < 2; ++x) {
#pragma unroll
                for (int e = 0; e < 4; ++e) S[x][e] = src ? src[(16 * (2 * hf + x) + 4 * q + e) * HS + col] : 0.f;
            }
            // the next chain (for the look-ahead load of its first chunk)
            int n2 = 0, h2 = 0, L2 = 0;
            int64_t bos2 = 0;
            const bool more = chain_at(k + 1, n2, h2);
            if (more) seq_extent(p, n2, bos2, L2);
            bf8 Bh[2], Bl[2];
            __syncthreads();  // the previous chain's last exchange has been read
            chain_exchange(S, Bh, Bl, ex, hf, lane);
            for (int c = 0; c < nch; ++c) {
                const Item it = chain_item(h, bos, L, c);
                Item nx{};
                if (c + 1 < nch) nx = chain_item(h, bos, L, c + 1);
                else if (more) nx = chain_item(h2, bos2, L2, 0);
                RawIn rn;
                prep_item<true>(p, it, raw, nullptr, sm, item_offset(p, nx, trow, cb), rn);
                chain_step(p, reinterpret_cast<const char*>(sm.slot[kRecSlot]), S, Bh, Bl, ex, vg, hf, lane, bos, c,
                           L, h);
                if (c + 1 < nch) chain_exchange(S, Bh, Bl, ex, hf, lane);
                raw = rn;
            }
            if (dst) {
#pragma unroll
                for (int x = 0; x < 2; ++x) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) dst[(16 * (2 * hf + x) + 4 * q + e) * HS + col] = S[x][e];
                }
            }
            if (!more) break;
            n = n2;
            h = h2;
            bos = bos2;
            L = L2;
        }
    }
    __syncthreads();  // the chain state of LDS is dead; the token-serial slabs reuse slots 14-15

    // ---- 3. this workgroup's token-serial pairs (rows of at most rec_max_len tokens: decode rows, short prefills),
    //         one pair per wavefront at a time, with the token-serial kernel's code
    {
        float* const slab = reinterpret_cast<float*>(sm.slot[14]) + wv * 5 * HS;
        const int g = lane >> 3, c = lane & 7;
        for (int64_t u = start[b] + wv; u < start[b + 1]; u += 8) {
            const uint32_t pa = (uint32_t)srow[u / p.H] * (uint32_t)p.H + (uint32_t)(u % p.H);
            const Pair qp = pair_of(p, pa);
            f4 S[16];
            TokenIn x{};
            prefetch_pair(p, qp, lane, g, c, S, x);
            run_pair(p, qp, lane, g, c, S, x, slab);
        }
    }
}

}  // namespace

ChunkWorkspace chunk_workspace(int num_seqs, int H, int64_t total_tokens, int64_t max_len_bound, bool varlen,
                               int rec_max_len) {
    ChunkWorkspace ws{};
    const int64_t per_row = (max_len_bound + C - 1) / C;
    int64_t maxc = (int64_t)num_seqs * per_row;
    if (varlen) {
        const int64_t lb = rec_max_len >= 0 ? (int64_t)rec_max_len + 1 : 1;
        const int64_t long_rows = std::min<int64_t>(num_seqs, total_tokens / lb);
        maxc = std::min<int64_t>(maxc, (total_tokens + C - 1) / C + long_rows);
    }
    ws.max_chunks = maxc;
    // chunk table (row, chunk index), row offsets + totals, the list of chunked rows + its length
    ws.plan_bytes = varlen ? align256(sizeof(int32_t) * (size_t)(2 * maxc + 2 * (int64_t)num_seqs + 3)) : 0;
    ws.chunk_bytes = align256(((size_t)maxc * (size_t)H + 1) * kChunkBytes);  // + the trash record
    ws.total_bytes = ws.plan_bytes + ws.chunk_bytes;
    return ws;
}

hipError_t launch_chain(const Params& p, hipStream_t stream) {
    if (p.num_seqs == 0) return hipSuccess;
    if (p.num_seqs > kChainMaxSeqs) return hipErrorInvalidValue;  // the C-ABI layer never routes such calls here
    const int grid = std::min(device_cu_count(), kChainMaxSeqs);   // one workgroup per CU (LDS-bound)
    hipLaunchKernelGGL(wkv7_chain_kernel, dim3((unsigned)grid), dim3(512), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_chunked(const Params& p, const ChunkWorkspace& ws, void* workspace, hipStream_t stream) {
    if (p.num_seqs == 0) return hipSuccess;
    int32_t* plan = reinterpret_cast<int32_t*>(workspace);
    char* wsc = static_cast<char*>(workspace) + ws.plan_bytes;
    const int ncps = (int)std::max<int64_t>(1, (p.T + C - 1) / C);
    if (p.cu) hipLaunchKernelGGL(wkv7_chunk_plan_kernel, dim3(1), dim3(1024), 0, stream, p, plan, ws.max_chunks);
    if (ws.max_chunks > 0) {
        const int cus = device_cu_count();
        const int64_t items = ws.max_chunks * p.H;
        const int64_t grid = std::min<int64_t>(items, cus);  // one 157 KB-LDS workgroup per CU
        hipLaunchKernelGGL(wkv7_chunk_prep_kernel, dim3((unsigned)grid), dim3(512), 0, stream, p, wsc, plan,
                           ws.max_chunks, ncps);
    }
    const int64_t pairs = (int64_t)p.num_seqs * p.H;
    int64_t blocks = ((pairs + 7) / 8) * 8 * 4;
    if (p.cu) blocks = std::min<int64_t>(blocks, kScanRaggedGrid);  // a multiple of 8: see scan_item
    hipLaunchKernelGGL(wkv7_chunk_scan_kernel, dim3((unsigned)blocks), dim3(64 * kScanWaves), 0, stream, p, wsc, plan,
                       ws.max_chunks, ncps);
    return hipGetLastError();
}

}  // namespace wkv7
