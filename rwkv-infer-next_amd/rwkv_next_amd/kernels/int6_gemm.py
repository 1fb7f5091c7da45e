"""Weight-only 6-bit GEMM / GEMV (W6A16) on the HIP kernels of include/w6a16.h.

Same calls, arguments and weight format as the reference module rwkv_next/kernels/int6_gemm.py, so weights
quantised there load unchanged:

    quantize_int6(w, group_k=128, clip_search=True) -> (lo, hi, scales, group_k)       (int6_gemm.py:73-112)
    dequantize_int6(lo, hi, sc, group_k, dtype)     -> w                               (int6_gemm.py:115-131)
    plan_int6(M, N, K, n_batch, device)             -> (split_k, use_dot)              (int6_gemm.py:239-250)
    int6_matmul(a, lo, hi, s, group_k, split_k=None, use_dot=None)                    (int6_gemm.py:296-308)
    int6_matmul_op(a, lo, hi, s, group_k, split_k, use_dot)  op rwkv_next_amd::int6_matmul   (int6_gemm.py:316-323)
plus a load-time re-layout with no counterpart in the reference:
    prepack_int6(lo, hi, s, group_k) -> Int6Packed      accepted by int6_matmul in place of lo, and by
    int6_matmul_packed_op(a, weight, scales, batches, K, N, group_k, split_k)   op rwkv_next_amd::int6_matmul_packed
    plan_int6_packed(M, N, K, n_batch, device)      -> split_k for a packed weight

Format: a (K, N) weight (N contiguous) is quantised to q in [-32, 31] per (group of group_k rows, column) with an
fp16 scale, w ~ s q; the code u = q + 32 is split into bit planes per 64-row chunk c:
    lo[c*32 + j] = lo4(row j) | lo4(row j + 32) << 4                                        j < 32
    hi[c*16 + j] = hi2(row j) | hi2(row j + 16) << 2 | hi2(row j + 32) << 4 | hi2(row j + 48) << 6   j < 16

Compute: one MFMA kernel for every M up to MAX_M (the reference's reduction form for M = 1 has no counterpart:
an MFMA with M padded to 16 rows costs the CDNA4 matrix core less than a VALU reduction costs the vector units, and
the weight bytes, not the arithmetic, bound both).  `use_dot` is accepted for the reference's signature and does
not change the computation.  Above MAX_M the weight is dequantised once to the activations' type and the product
goes to the library GEMM (hipBLASLt through torch.matmul), which is compute-bound there.  The C ABI has its own kernel
for that range (packed weights, M > 256: dequantisation in LDS fused with the product, the same values); at K = 4096,
N = 16384 it is level with dequantise + hipBLASLt at M = 1024 and slower from M = 2048 (585 against 465 us at
M = 4096), so MAX_M (env RWKV_INT6_MAX_M) keeps the library GEMM by default.

Activations are bf16 (the model's) or fp16 (the reference op takes any a.dtype its dot accepts); the result is
a.dtype, or out_dtype (fp32 accumulation).  Every call runs on the current stream, no host sync.
"""
from __future__ import annotations

import ctypes
import os
from typing import NamedTuple

import torch

from .. import _lib
from ._workspace import stream_workspace

CHUNK = 64
QMIN, QMAX = -32, 31
# Largest M that the W6A16 kernel serves; larger M dequantises once and runs the library GEMM.
MAX_M = int(os.environ.get("RWKV_INT6_MAX_M", "256"))
_RATIOS = (1.0, 0.97, 0.94, 0.91, 0.88, 0.85)


# ----------------------------------------------------------------------------------------------------------------
# quantisation / packing (host-side preparation of the weights, run once at load time on the weight's device)
# ----------------------------------------------------------------------------------------------------------------
@torch.no_grad()
def quantize_int6(w, group_k=128, clip_search=True):
    """(K, N) or (B, K, N) float -> (lo uint8 (.., K/2, N), hi uint8 (.., K/4, N), scales fp16 (.., K/group_k, N),
    group_k).  group_k outside (0, K) means one group of K rows; it must be a multiple of 64 dividing K.

    The scale of each (group, column) is fp16(absmax * r / 31.5) for the clip ratio r in
    (1, .97, .94, .91, .88, .85) (only 1 without clip_search) whose rounded weights have the least squared error,
    the first such r on ties; q = clamp(round(w / s), -32, 31) with the stored fp16 scale (int6_gemm.py:92-104).
    """
    squeeze = w.dim() == 2
    if squeeze:
        w = w.unsqueeze(0)
    B, K, N = w.shape
    g = group_k if group_k and 0 < group_k < K else K
    if K % CHUNK or g % CHUNK or K % g:
        raise ValueError(f"int6 needs K % 64 == 0 and group_k % 64 == 0 dividing K (K={K}, group_k={g})")
    G, C = K // g, K // CHUNK
    lo = torch.empty((B, K // 2, N), dtype=torch.uint8, device=w.device)
    hi = torch.empty((B, K // 4, N), dtype=torch.uint8, device=w.device)
    sc = torch.empty((B, G, N), dtype=torch.float16, device=w.device)
    cols = max(256, (1 << 23) // K)  # column blocks keep the fp32 temporaries to ~32 MB
    ratios = _RATIOS if clip_search else _RATIOS[:1]
    for b in range(B):
        for n0 in range(0, N, cols):
            n1 = min(N, n0 + cols)
            x = w[b, :, n0:n1].float().view(G, g, n1 - n0)
            amax = x.abs().amax(dim=1, keepdim=True).clamp_min(1e-10)
            best_s = best_err = None
            for r in ratios:
                s = (amax * r / 31.5).half().float()
                err = (torch.round(x / s).clamp(QMIN, QMAX) * s - x).square().sum(dim=1, keepdim=True)
                if best_s is None:
                    best_s, best_err = s, err
                else:
                    better = err < best_err
                    best_s = torch.where(better, s, best_s)
                    best_err = torch.where(better, err, best_err)
            u = (torch.round(x / best_s).clamp(QMIN, QMAX) + 32).to(torch.uint8).view(C, CHUNK, n1 - n0)
            sc[b, :, n0:n1] = best_s.view(G, n1 - n0).half()
            lo[b, :, n0:n1] = ((u[:, :32] & 15) | ((u[:, 32:] & 15) << 4)).view(K // 2, n1 - n0)
            h2 = u >> 4
            hi[b, :, n0:n1] = (h2[:, :16] | (h2[:, 16:32] << 2) | (h2[:, 32:48] << 4) | (h2[:, 48:] << 6)).view(
                K // 4, n1 - n0)
    if squeeze:
        lo, hi, sc = lo[0], hi[0], sc[0]
    return lo.contiguous(), hi.contiguous(), sc.contiguous(), g


def _weights3(lo, hi, s):
    L = lo if lo.dim() == 3 else lo.unsqueeze(0)
    H = hi if hi.dim() == 3 else hi.unsqueeze(0)
    S = s if s.dim() == 3 else s.unsqueeze(0)
    if L.dtype != torch.uint8 or H.dtype != torch.uint8 or S.dtype != torch.float16:
        raise TypeError("int6 weights are (lo uint8, hi uint8, scales float16)")
    for t, name in ((L, "lo"), (H, "hi"), (S, "scales")):
        if t.device.type != "cuda":
            raise ValueError(f"{name} must be on a GPU (got {t.device})")
    Bq, K2, N = L.shape
    K = 2 * K2
    if H.shape != (Bq, K // 4, N) or S.shape[0] != Bq or S.shape[2] != N:
        raise ValueError(f"int6 planes do not match: lo {tuple(L.shape)}, hi {tuple(H.shape)}, s {tuple(S.shape)}")
    return _aligned(L), _aligned(H), _aligned(S), Bq, K, N


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """t contiguous at a 16-byte aligned address (the kernels load 16 bytes per lane)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _group_k(group_k, K, n_groups):
    g = group_k if group_k and 0 < group_k < K else K
    if g % CHUNK or K % g or K // g != n_groups:
        raise ValueError(f"group_k {group_k} does not match K = {K} with {n_groups} scale rows")
    return g


_OUT_CODES = {torch.bfloat16: _lib.W6A16_OUT_BF16, torch.float16: _lib.W6A16_OUT_F16,
              torch.float32: _lib.W6A16_OUT_F32}
_IN_CODES = {torch.bfloat16: _lib.W6A16_IN_BF16, torch.float16: _lib.W6A16_IN_F16}


@torch.no_grad()
def dequantize_int6(lo, hi, sc, group_k, dtype=torch.float32):
    """w = s q, (K, N) or (B, K, N) in `dtype` (bfloat16, float16 or float32; float32 is exact), on the device."""
    squeeze = lo.dim() == 2
    L, H, S, Bq, K, N = _weights3(lo, hi, sc)
    g = _group_k(group_k, K, S.shape[1])
    if dtype not in _OUT_CODES:
        raise TypeError(f"dequantize_int6 writes bfloat16, float16 or float32 (got {dtype})")
    w = torch.empty((Bq, K, N), dtype=dtype, device=L.device)
    with torch.cuda.device(L.device):
        _lib.check(_lib.load().w6a16_dequantize(
            L.data_ptr(), H.data_ptr(), S.data_ptr(), w.data_ptr(), Bq, K, N, g, L.stride(0), H.stride(0),
            S.stride(0), w.stride(0), _OUT_CODES[dtype], torch.cuda.current_stream(L.device).cuda_stream))
    return w[0] if squeeze else w


# ----------------------------------------------------------------------------------------------------------------
# dispatch
# ----------------------------------------------------------------------------------------------------------------
def plan_int6(M, N, K, n_batch, device=None):
    """(split_k, use_dot) for one shape.  split_k is the kernel's rule (w6a16_plan_split: the smallest power of two
    that gives every CU a workgroup, doubled while ranges keep 16 chunks within two workgroups per CU); use_dot is M > 1 as in the reference and does not change the computation."""
    if device is not None and torch.device(device).type == "cuda":
        with torch.cuda.device(device):
            sk = _lib.load().w6a16_plan_split(n_batch, M, N, K)
    else:
        sk = _lib.load().w6a16_plan_split(n_batch, M, N, K)
    return int(sk), M > 1


def plan_int6_packed(M, N, K, n_batch, device=None):
    """split_k for a packed weight (w6a16_plan_split_packed; no counterpart in the reference): plan_int6's split, made
    shallower where the packed kernel runs half strips.  A packed call equals the planes' bit for bit only at the same
    split_k."""
    lib = _lib.load()
    if device is not None and torch.device(device).type == "cuda":
        with torch.cuda.device(device):
            return int(lib.w6a16_plan_split_packed(n_batch, M, N, K))
    return int(lib.w6a16_plan_split_packed(n_batch, M, N, K))


class Int6Packed(NamedTuple):
    """A W6A16 weight in the packed layout (include/w6a16.h, w6a16_pack): the same 6-bit codes and fp16 scales,
    re-laid out once so that each wavefront streams one contiguous 6 KB block per 64-row chunk and needs no LDS
    transposition.  Made by prepack_int6; accepted by int6_matmul / int6_matmul_packed_op in place of (lo, hi, s)."""
    weight: torch.Tensor   # uint8 [batches or 1][strips][K / 64][6144], flattened per batch
    scales: torch.Tensor   # float16 [batches or 1][strips][K / group_k][128]
    batches: int           # 0: one (K, N) weight; else the number of (K, N) weights
    K: int
    N: int
    group_k: int


@torch.no_grad()
def prepack_int6(lo, hi, s, group_k) -> Int6Packed:
    """Re-lay out a quantised weight (quantize_int6's planes, (K, N) or (B, K, N)) into the packed layout, on its
    device.  The codes and scales are unchanged, so results equal int6_matmul on the planes bit for bit."""
    L, H, S, Bq, K, N = _weights3(lo, hi, s)
    g = _group_k(group_k, K, S.shape[1])
    lib = _lib.load()
    wb, sb = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _lib.check(lib.w6a16_packed_size(Bq, K, N, g, ctypes.byref(wb), ctypes.byref(sb)))
    weight = torch.empty(int(wb.value), dtype=torch.uint8, device=L.device)
    scales = torch.empty(int(sb.value) // 2, dtype=torch.float16, device=L.device)
    with torch.cuda.device(L.device):
        _lib.check(lib.w6a16_pack(L.data_ptr(), H.data_ptr(), S.data_ptr(), Bq, K, N, g, L.stride(0), H.stride(0),
                                  S.stride(0), weight.data_ptr(), scales.data_ptr(),
                                  torch.cuda.current_stream(L.device).cuda_stream))
    return Int6Packed(weight.view(Bq, -1), scales.view(Bq, -1), 0 if lo.dim() == 2 else Bq, K, N, g)


@torch.no_grad()
def dequantize_int6_packed(pk: Int6Packed, dtype=torch.float32):
    """dequantize_int6 for a packed weight: (K, N) or (B, K, N) in bfloat16, float16 or float32."""
    if dtype not in _OUT_CODES:
        raise TypeError(f"dequantize_int6_packed writes bfloat16, float16 or float32 (got {dtype})")
    Bq = pk.weight.shape[0]
    w = torch.empty((Bq, pk.K, pk.N), dtype=dtype, device=pk.weight.device)
    with torch.cuda.device(w.device):
        _lib.check(_lib.load().w6a16_dequantize_packed(
            pk.weight.data_ptr(), pk.scales.data_ptr(), w.data_ptr(), Bq, pk.K, pk.N, pk.group_k, w.stride(0),
            _OUT_CODES[dtype], torch.cuda.current_stream(w.device).cuda_stream))
    return w if pk.batches else w[0]


class _W(NamedTuple):
    """A weight as the kernel sees it: format, the base pointers' tensors and batch strides."""
    fmt: int
    w0: torch.Tensor       # lo plane, or the packed weight
    w1: torch.Tensor       # hi plane, or None
    sc: torch.Tensor       # scales (planes [Bq][G][N] or packed [Bq][...])
    Bq: int
    K: int
    N: int
    g: int


def _planes(lo, hi, s, group_k) -> _W:
    L, H, S, Bq, K, N = _weights3(lo, hi, s)
    return _W(_lib.W6A16_FORMAT_PLANES, L, H, S, Bq, K, N, _group_k(group_k, K, S.shape[1]))


def _packed(pk: Int6Packed) -> _W:
    for t, name, dt in ((pk.weight, "weight", torch.uint8), (pk.scales, "scales", torch.float16)):
        if t.dtype != dt or t.device.type != "cuda" or t.dim() != 2:
            raise ValueError(f"packed {name} must be a 2-D {dt} GPU tensor (from prepack_int6)")
    return _W(_lib.W6A16_FORMAT_PACKED, _aligned(pk.weight), None, _aligned(pk.scales), pk.weight.shape[0], pk.K,
              pk.N, pk.group_k)


def _dequant(w: _W, dtype):
    if w.fmt == _lib.W6A16_FORMAT_PACKED:
        return dequantize_int6_packed(Int6Packed(w.w0, w.sc, w.Bq, w.K, w.N, w.g), dtype=dtype)
    return dequantize_int6(w.w0, w.w1, w.sc, w.g, dtype=dtype)


def _impl(a, w: _W, split_k, out_dtype=None):
    batched = a.dim() == 3
    A = a if batched else a.unsqueeze(0)
    if A.dtype not in _IN_CODES:
        raise TypeError(f"int6_matmul takes bfloat16 or float16 activations (got {A.dtype})")
    if A.device.type != "cuda":
        raise ValueError(f"a must be on a GPU (got {A.device})")
    B, M, Ka = A.shape
    Bq, K, N = w.Bq, w.K, w.N
    if Ka != K:
        raise ValueError(f"K mismatch: a has {Ka}, int6 weight has {K}")
    if Bq not in (1, B):
        raise ValueError(f"weight batch {Bq} does not match activation batch {B}")
    odt = A.dtype if out_dtype is None else out_dtype
    if odt not in _OUT_CODES:
        raise TypeError(f"int6_matmul writes bfloat16, float16 or float32 (got {odt})")
    if M > MAX_M:  # prefill: compute-bound, dequantise once (to the activations' type) and use the library GEMM
        wd = _dequant(w, A.dtype)
        if wd.dim() == 2:
            wd = wd.unsqueeze(0)
        C = torch.matmul(A, wd[0] if Bq == 1 else wd)
        C = C.to(odt)
        return C if batched else C[0]
    out = torch.empty((B, M, N), dtype=odt, device=A.device)
    if M == 0:
        return out if batched else out[0]
    if A.stride(2) != 1 or A.stride(1) % 8 or A.stride(0) % 8 or A.data_ptr() % 16:
        A = _aligned(A)
    args = _lib.W6a16Args()
    args.a, args.a_batch_stride, args.a_row_stride = A.data_ptr(), A.stride(0), A.stride(1)
    shared = Bq == 1 and B > 1
    args.format = w.fmt
    args.lo, args.scales = w.w0.data_ptr(), w.sc.data_ptr()
    args.lo_batch_stride = 0 if shared else w.w0.stride(0)
    args.scales_batch_stride = 0 if shared else w.sc.stride(0)
    if w.w1 is not None:
        args.hi, args.hi_batch_stride = w.w1.data_ptr(), 0 if shared else w.w1.stride(0)
    args.out, args.out_batch_stride, args.out_row_stride = out.data_ptr(), out.stride(0), out.stride(1)
    args.B, args.M, args.N, args.K, args.group_k = B, M, N, K, w.g
    args.split_k = max(1, int(split_k))
    args.out_dtype = _OUT_CODES[odt]
    args.a_dtype = _IN_CODES[A.dtype]
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    _lib.check(lib.w6a16_workspace_size(args, ctypes.byref(n)))
    if n.value:  # split-K counters and partials, and the wide kernel's row sums (M > 32)
        ws = _workspace(A.device, int(n.value))
        args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(lib.w6a16_matmul(args, torch.cuda.current_stream(A.device).cuda_stream))
    return out if batched else out[0]


_COUNTER_BYTES = 1 << 20   # the workspace's arrival-counter region (include/w6a16.h, w6a16_workspace_size)
_WORKSPACES: dict = {}     # (device index, stream handle) -> [buffer, counters zeroed in stream order, capture id]


def _workspace(device, nbytes):
    """The workspace (a fixed counter region, then split-K partials and row sums) of the current stream on `device`;
    see `_workspace.stream_workspace`."""
    return stream_workspace(_WORKSPACES, device, nbytes, _COUNTER_BYTES)


def int6_matmul(a, lo, hi=None, s=None, group_k=None, split_k=None, use_dot=None, *, out_dtype=None):
    """a (M, K) | (B, M, K) bf16 or fp16 @ dequant(int6 weight (K, N) | (B, K, N)) -> (M, N) | (B, M, N) in a.dtype
    (or out_dtype: bfloat16 / float16 / float32), as the reference casts the codes to a.dtype.  The weight is the planes (lo, hi, s, group_k) or an Int6Packed passed as `lo`
    (hi, s, group_k then unused).  A single weight (K, N) is shared by every batch row.  Eager entry point; the
    model-facing functional ops are int6_matmul_op and int6_matmul_packed_op."""
    packed = isinstance(lo, Int6Packed)
    w = _packed(lo) if packed else _planes(lo, hi, s, group_k)
    B = a.shape[0] if a.dim() == 3 else 1
    M = a.shape[-2]
    if split_k is None:
        split_k = plan_int6_packed(M, w.N, w.K, B, a.device) if packed else plan_int6(M, w.N, w.K, B, a.device)[0]
    with torch.cuda.device(a.device):
        return _impl(a, w, split_k, out_dtype)


@torch.library.custom_op("rwkv_next_amd::int6_matmul", mutates_args=())
def int6_matmul_op(a: torch.Tensor, lo: torch.Tensor, hi: torch.Tensor, s: torch.Tensor, group_k: int, split_k: int,
                   use_dot: bool) -> torch.Tensor:
    """Functional op with the schema of the reference's rwkv_next::int6_matmul (int6_gemm.py:316-323); the plan
    (split_k, use_dot) comes from plan_int6, resolved by the caller."""
    with torch.cuda.device(a.device):
        return _impl(a, _planes(lo, hi, s, group_k), split_k)


@torch.library.custom_op("rwkv_next_amd::int6_matmul_packed", mutates_args=())
def int6_matmul_packed_op(a: torch.Tensor, weight: torch.Tensor, scales: torch.Tensor, batches: int, K: int, N: int,
                          group_k: int, split_k: int) -> torch.Tensor:
    """int6_matmul_op for a packed weight (the fields of an Int6Packed); no counterpart in the reference."""
    with torch.cuda.device(a.device):
        return _impl(a, _packed(Int6Packed(weight, scales, batches, K, N, group_k)), split_k)


@int6_matmul_packed_op.register_fake
def _(a, weight, scales, batches, K, N, group_k, split_k):
    return a.new_empty((*a.shape[:-1], N))


@int6_matmul_op.register_fake
def _(a, lo, hi, s, group_k, split_k, use_dot):
    return a.new_empty((*a.shape[:-1], lo.shape[-1]))
