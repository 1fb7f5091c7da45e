"""CPU oracle for the W6A16 weight format and GEMM -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/ and bench.py's cpu_baseline leg, as the checker.  The product package never imports it.

Restates, in numpy:
  * pack_codes / unpack_codes -- the bit-plane packing of 6-bit codes u = q + 32 in 64-row chunks
    (rwkv_next/kernels/int6_gemm.py:14-38 format, packing at 105-107, unpacking at 124-128 and 185-188);
  * dequantize_ref            -- w = s q with one fp16 scale per (group of group_k rows, column)  (int6_gemm.py:115-131);
  * int6_matmul_ref           -- C = A @ w in float64: what `_w6a16` computes with fp32 accumulation
                                 (int6_gemm.py:156-215), the exact sum of which the kernel's result approximates.
Pinned by tests/test_int6_oracle.py: hand-computed known-answer planes, the packing's bijectivity, agreement of the
two unpacking forms the reference uses (dequantize_int6's and the kernel's sub-tile form), and numpy's matmul.
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
