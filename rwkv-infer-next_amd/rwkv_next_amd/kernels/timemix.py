"""Fused time-mix prologue and epilogue around the WKV7 recurrence (HIP kernels of include/wkv7.h).

Same arguments and results as the reference's inline code in Layer.part_att (rwkv_next/model.py):

    timemix_prologue(r, k, v, o, v_first, b_w, b_a, b_v, kk_mul, ka_mul, H, N, first_layer)
        -> (ins, v_first)       ins = (r, w, k', v', -kk, kk * a), the WKV operands    (model.py:142-152)
    timemix_epilogue(y, r, k, v, g, lnx_w, lnx_b, r_k, H, N, eps)
        -> (group_norm(y) + bonus) * g, the input of the output projection             (model.py:156-158)

Tensors are bf16 with rows of H*N channels ((M, C) or (B, T, C)); o is the (3, M, C) LoRA output stack; the
per-channel parameters are (1, C) or (C,), r_k is (H, N).  One pass per call on the current stream, no host sync.
"""
from __future__ import annotations

import torch

from .. import _lib

HEAD_SIZE = 64


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """t contiguous at a 16-byte aligned address (the kernels load 8 channels per lane)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _rows(t: torch.Tensor, C: int, name: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16 (got {t.dtype})")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a GPU (got {t.device})")
    if t.shape[-1] != C:
        raise ValueError(f"{name} has {t.shape[-1]} channels, expected {C}")
    return _aligned(t).view(-1, C)


def _param(t: torch.Tensor, n: int, name: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16 or t.numel() != n:
        raise ValueError(f"{name} must be a bfloat16 tensor of {n} elements")
    return _aligned(t)


def timemix_prologue(r, k, v, o, v_first, b_w, b_a, b_v, kk_mul, ka_mul, H, N, first_layer):
    """The six WKV operands from the projections (model.py:142-152).  On the first layer v_first is ignored and
    returned as v; elsewhere v is mixed towards v_first.  Returns ((r, w, k', v', -kk, kk * a), v_first)."""
    if N != HEAD_SIZE:
        raise ValueError(f"head size {N} is not supported (N = {HEAD_SIZE})")
    C = H * N
    shape = k.shape
    kk2, vv2, rr2 = _rows(k, C, "k"), _rows(v, C, "v"), _rows(r, C, "r")
    M = kk2.shape[0]
    if o.shape[0] != 3:
        raise ValueError("o must stack the three LoRA outputs (v, w, a) on its first axis")
    oo = [_rows(o[j], C, f"o[{j}]") for j in range(3)]
    for t in oo:
        if t.shape[0] != M:
            raise ValueError("o rows do not match k")
    vf = None if first_layer else _rows(v_first, C, "v_first")
    prm = [_param(x, C, n) for x, n in ((b_w, "b_w"), (b_a, "b_a"), (b_v, "b_v"), (kk_mul, "kk_mul"), (ka_mul, "ka_mul"))]
    outs = [torch.empty(M, C, device=k.device, dtype=torch.bfloat16) for _ in range(5)]
    a = _lib.PrologueArgs()
    a.k, a.v = kk2.data_ptr(), vv2.data_ptr()
    a.o_v, a.o_w, a.o_a = (t.data_ptr() for t in oo)
    a.v_first = None if vf is None else vf.data_ptr()
    a.b_w, a.b_a, a.b_v, a.kk_mul, a.ka_mul = (t.data_ptr() for t in prm)
    a.w_out, a.k_out, a.v_out, a.a_out, a.b_out = (t.data_ptr() for t in outs)
    a.tokens, a.in_stride, a.out_stride, a.H, a.head_size = M, C, C, H, N
    with torch.cuda.device(k.device):
        _lib.check(_lib.load().wkv7_timemix_prologue(a, torch.cuda.current_stream(k.device).cuda_stream))
    w, k2, v2, aa, bb = (t.view(shape) for t in outs)
    ins = (r, w, k2, v2, aa, bb)
    return ins, (v if first_layer else v_first)


def timemix_epilogue(y, r, k, v, g, lnx_w, lnx_b, r_k, H, N, eps):
    """(group_norm(y, one group per head, lnx_w, lnx_b, eps) + sum_c(r k r_k) v) * g  (model.py:156-158), where k and
    v are the WKV operands k' and v'.  Returns (M, C) bf16, the input of the output projection."""
    if N != HEAD_SIZE:
        raise ValueError(f"head size {N} is not supported (N = {HEAD_SIZE})")
    C = H * N
    yy, rr, kk, vv, gg = (_rows(t, C, n) for t, n in ((y, "y"), (r, "r"), (k, "k"), (v, "v"), (g, "g")))
    M = yy.shape[0]
    for t in (rr, kk, vv, gg):
        if t.shape[0] != M:
            raise ValueError("epilogue inputs must have the same number of rows")
    lw, lb, rk = _param(lnx_w, C, "lnx_w"), _param(lnx_b, C, "lnx_b"), _param(r_k, C, "r_k")
    out = torch.empty(M, C, device=y.device, dtype=torch.bfloat16)
    a = _lib.EpilogueArgs()
    a.y, a.r, a.k, a.v, a.g = (t.data_ptr() for t in (yy, rr, kk, vv, gg))
    a.lnx_w, a.lnx_b, a.r_k, a.out = lw.data_ptr(), lb.data_ptr(), rk.data_ptr(), out.data_ptr()
    a.tokens, a.in_stride, a.out_stride, a.eps, a.H, a.head_size = M, C, C, float(eps), H, N
    with torch.cuda.device(y.device):
        _lib.check(_lib.load().wkv7_timemix_epilogue(a, torch.cuda.current_stream(y.device).cuda_stream))
    return out
