"""CPU oracle for the W6A16 weight format and GEMM -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/ and bench.py's cpu_baseline leg, as the checker.  The product package never imports it.

Restates, in numpy:
  * pack_codes / unpack_codes -- the bit-plane packing of 6-bit codes u = q + 32 in 64-row chunks
    (rwkv_next/kernels/int6_gemm.py:14-38 format, packing at 105-107, unpacking at 124-128 and 185-188);
  * dequantize_ref            -- w = s q with one fp16 scale per (group of group_k rows, column)  (int6_gemm.py:115-131);
  * int6_matmul_ref           -- C = A @ w in float64: what `_w6a16` computes with fp32 accumulation
                                 (int6_gemm.py:156-215), the exact sum of which the kernel's result approximates.
  * pack_packed / unpack_packed -- this build's load-time re-layout of the same codes (include/w6a16.h,
                                   w6a16_pack), restated from its definition.
Pinned by tests/test_int6_oracle.py: hand-computed known-answer planes and packed records, the packings'
bijectivity, agreement of the two unpacking forms the reference uses (dequantize_int6's and the kernel's sub-tile
form), and numpy's matmul.
"""
from __future__ import annotations

import numpy as np

CHUNK = 64


def pack_codes(u: np.ndarray):
    """u uint8 [..., K, N] in [0, 63] -> (lo [..., K/2, N], hi [..., K/4, N]) uint8."""
    u = np.asarray(u, dtype=np.uint8)
    *lead, K, N = u.shape
    if K % CHUNK:
        raise ValueError("K must be a multiple of 64")
    c = u.reshape(*lead, K // CHUNK, CHUNK, N)
    lo = (c[..., :32, :] & 15) | ((c[..., 32:, :] & 15) << 4)
    h = c >> 4
    hi = h[..., 0:16, :] | (h[..., 16:32, :] << 2) | (h[..., 32:48, :] << 4) | (h[..., 48:64, :] << 6)
    return lo.reshape(*lead, K // 2, N).astype(np.uint8), hi.reshape(*lead, K // 4, N).astype(np.uint8)


def unpack_codes(lo: np.ndarray, hi: np.ndarray) -> np.ndarray:
    """(lo, hi) -> u uint8 [..., K, N]: rows j < 32 of a chunk take lo's low nibble, rows 32 + j its high nibble; the
    top two bits of row r come from hi row r % 16, field r // 16 (dequantize_int6's form, int6_gemm.py:124-128)."""
    lo = np.asarray(lo, dtype=np.uint8)
    hi = np.asarray(hi, dtype=np.uint8)
    *lead, K2, N = lo.shape
    K = 2 * K2
    L = lo.reshape(*lead, K // CHUNK, 32, N)
    H = hi.reshape(*lead, K // CHUNK, 16, N)
    low = np.concatenate([L & 15, L >> 4], axis=-2)                                     # rows 0..63
    top = np.concatenate([(H >> (2 * f)) & 3 for f in range(4)], axis=-2)               # rows 0..63
    return (low | (top << 4)).reshape(*lead, K, N).astype(np.uint8)


def dequantize_ref(lo, hi, sc, group_k: int) -> np.ndarray:
    """w [..., K, N] float64 = s q, s the fp16 scale of (row // group_k, column), q = u - 32."""
    q = unpack_codes(lo, hi).astype(np.float64) - 32.0
    s = np.asarray(sc, dtype=np.float16).astype(np.float64)
    K = q.shape[-2]
    rows = np.arange(K) // group_k
    return q * s[..., rows, :]


def int6_matmul_ref(a, lo, hi, sc, group_k: int) -> np.ndarray:
    """C [..., M, N] float64 = a [..., M, K] @ dequant(lo, hi, sc) (a shared (K, N) weight broadcasts over batch)."""
    w = dequantize_ref(lo, hi, sc, group_k)
    return np.matmul(np.asarray(a, dtype=np.float64), w)


def abs_bound(a, lo, hi, sc, group_k: int) -> np.ndarray:
    """|a| @ |w|: the scale of the rounding errors of any fp32 evaluation of the product, element by element."""
    w = dequantize_ref(lo, hi, sc, group_k)
    return np.matmul(np.abs(np.asarray(a, dtype=np.float64)), np.abs(w))


# ----------------------------------------------------------------------------------------------------------------
# packed layout: per (batch, 128-column strip, 64-row chunk) a 6144-byte block; lane l = 16 q + i owns the 24-dword
# record R whose dwords 4 k .. 4 k + 3 sit at bytes 1024 k + 16 l.  For tile t (column 128 strip + 16 t + i):
#   R[2 t], R[2 t + 1]: bytes e = 0..7 = lo plane row 32 chunk + 8 q + e
#   R[16 + t]: byte e' = 0..3 = hi2(8 q + e') | hi2(32 + 8 q + e') << 2 | hi2(8 q + 4 + e') << 4
#                               | hi2(32 + 8 q + 4 + e') << 6          (rows within the chunk)
# Scales: per (batch, strip, group) 128 fp16 ordered [i][t].  Columns past N: zero bytes, zero scales.
# ----------------------------------------------------------------------------------------------------------------
def _records(u, N):
    """u uint8 [K, Npad] codes (Npad = 128 * strips) -> records uint32 [strips, K/64, 64 lanes, 24]."""
    K, Npad = u.shape
    S, Cn = Npad // 128, K // CHUNK
    lo, _ = pack_codes(u)
    top = (u >> 4).astype(np.uint32)                                  # [K, Npad]
    R = np.zeros((S, Cn, 64, 24), np.uint32)
    for q in range(4):
        for i in range(16):
            lane = 16 * q + i
            for t in range(8):
                n = np.arange(S) * 128 + 16 * t + i                   # [S]
                for c in range(Cn):
                    lb = lo[c * 32 + 8 * q: c * 32 + 8 * q + 8][:, n].astype(np.uint32)     # [8, S]
                    R[:, c, lane, 2 * t] = lb[0] | lb[1] << 8 | lb[2] << 16 | lb[3] << 24
                    R[:, c, lane, 2 * t + 1] = lb[4] | lb[5] << 8 | lb[6] << 16 | lb[7] << 24
                    hd = np.zeros(S, np.uint32)
                    for e in range(4):
                        rows = (8 * q + e, 32 + 8 * q + e, 8 * q + 4 + e, 32 + 8 * q + 4 + e)
                        byte = np.zeros(S, np.uint32)
                        for f, r in enumerate(rows):
                            byte |= top[c * 64 + r, n] << (2 * f)
                        hd |= byte << (8 * e)
                    R[:, c, lane, 16 + t] = hd
    return R


def pack_packed(lo, hi, sc, group_k):
    """Planes ([K/2, N], [K/4, N], [G, N] or with a leading batch) -> (weight uint8 [B, bytes], scales fp16 [B, n])."""
    lo, hi, sc = np.asarray(lo), np.asarray(hi), np.asarray(sc, dtype=np.float16)
    if lo.ndim == 2:
        lo, hi, sc = lo[None], hi[None], sc[None]
    B, K2, N = lo.shape
    K = 2 * K2
    S = (N + 127) // 128
    G = K // group_k
    ws, ss = [], []
    for b in range(B):
        u = np.zeros((K, 128 * S), np.uint8)
        u[:, :N] = unpack_codes(lo[b], hi[b])
        R = _records(u, N)                                            # [S, C, 64, 24]
        # bytes: block (s, c) = 6 instructions x 64 lanes x 4 dwords
        blk = R.reshape(S, K // CHUNK, 64, 6, 4).transpose(0, 1, 3, 2, 4)      # [S, C, k, lane, 4]
        ws.append(np.frombuffer(blk.astype("<u4").tobytes(), np.uint8).copy())  # padding columns: code 0, zero bytes
        scp = np.zeros((G, 128 * S), np.float16)
        scp[:, :N] = sc[b]
        ss.append(scp.reshape(G, S, 8, 16).transpose(1, 0, 3, 2).reshape(-1))  # [S][G][i][t]
    return np.stack(ws), np.stack(ss)


def unpack_packed(weight, scales, K, N, group_k):
    """(weight [B, bytes], scales [B, n]) -> (codes uint8 [B, K, N], scales fp16 [B, G, N])."""
    weight, scales = np.asarray(weight, np.uint8), np.asarray(scales, np.float16)
    B = weight.shape[0]
    S, Cn, G = (N + 127) // 128, K // CHUNK, K // group_k
    us, scs = [], []
    for b in range(B):
        R = np.frombuffer(weight[b].tobytes(), "<u4").reshape(S, Cn, 6, 64, 4).transpose(0, 1, 3, 2, 4)
        R = R.reshape(S, Cn, 64, 24)
        u = np.zeros((K, 128 * S), np.uint8)
        for q in range(4):
            for i in range(16):
                lane = 16 * q + i
                for t in range(8):
                    n = np.arange(S) * 128 + 16 * t + i
                    for c in range(Cn):
                        lw = (R[:, c, lane, 2 * t], R[:, c, lane, 2 * t + 1])
                        hd = R[:, c, lane, 16 + t]
                        for e in range(8):
                            lb = (lw[e >> 2] >> (8 * (e & 3))) & 0xFF
                            hb = (hd >> (8 * (e & 3) + 4 * (e >> 2))) & 0xF
                            u[c * 64 + 8 * q + e, n] = (lb & 15) | ((hb & 3) << 4)
                            u[c * 64 + 32 + 8 * q + e, n] = (lb >> 4) | ((hb >> 2) << 4)
        us.append(u[:, :N])
        scs.append(scales[b].reshape(S, G, 16, 8).transpose(1, 0, 3, 2).reshape(G, 128 * S)[:, :N])
    return np.stack(us), np.stack(scs)
