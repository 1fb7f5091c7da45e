"""W6A16 without a GPU: the numpy oracle of the bit-plane format pinned by known answers and invariants, the
host-side quantiser's contract (it runs in torch on any device), and the C ABI of include/w6a16.h (exports,
struct layout, host-side validation; no launch is reached)."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from conftest import REPO

from oracle import int6_ref as R
from rwkv_next_amd import _lib
from rwkv_next_amd.kernels import int6_gemm as I6

HEADER = os.path.join(REPO, "include", "w6a16.h")


# ----------------------------------------------------------------------------------------------------------------
# oracle pins
# ----------------------------------------------------------------------------------------------------------------
def test_known_answer_planes_of_a_ramp():
    """Codes u[r] = r (r = 0..63) in one column.  By the format (int6_gemm.py:20-24) lo row j holds rows j and j+32,
    whose low nibbles are both j & 15, and every hi row holds the top bits 0, 1, 2, 3 of rows j, j+16, j+32, j+48:
    0b11_10_01_00 = 0xE4."""
    u = np.arange(64, dtype=np.uint8).reshape(64, 1)
    lo, hi = R.pack_codes(u)
    assert lo[:, 0].tolist() == [0x00, 0x11, 0x22, 0x33, 0x44, 0x55, 0x66, 0x77, 0x88, 0x99, 0xAA, 0xBB, 0xCC, 0xDD,
                                 0xEE, 0xFF] * 2
    assert hi[:, 0].tolist() == [0xE4] * 16
    np.testing.assert_array_equal(R.unpack_codes(lo, hi), u)


def test_known_answer_planes_of_single_codes():
    """One non-zero code at a time lands in exactly one nibble / bit pair."""
    for r, val, lo_row, lo_byte, hi_row, hi_byte in [
            (0, 63, 0, 0x0F, 0, 0x03),      # row 0: lo nibble 0, hi field 0
            (37, 0x2A, 5, 0xA0, 5, 0x20),   # row 37 = 32 + 5: lo high nibble of row 5; 37 // 16 = 2 -> bits 4-5
            (50, 0x15, 18, 0x50, 2, 0x40),  # row 50 = 32 + 18: lo row 18 high nibble; hi row 50 % 16 = 2, field 3
            (16, 0x30, 16, 0x00, 0, 0x0C),  # row 16: lo row 16 low nibble 0; hi row 0 field 1
            (127, 0x3F, 63, 0xF0, 31, 0xC0)]:  # second chunk, row 63 of it: lo row 32+31, hi row 16+15, field 3
        u = np.zeros((128, 1), np.uint8)
        u[r, 0] = val
        lo, hi = R.pack_codes(u)
        expect_lo = np.zeros(64, np.uint8)
        expect_hi = np.zeros(32, np.uint8)
        expect_lo[lo_row] = lo_byte
        expect_hi[hi_row] = hi_byte
        np.testing.assert_array_equal(lo[:, 0], expect_lo, err_msg=f"row {r}")
        np.testing.assert_array_equal(hi[:, 0], expect_hi, err_msg=f"row {r}")


def test_packing_is_a_bijection():
    rng = np.random.default_rng(3)
    u = rng.integers(0, 64, size=(2, 256, 48), dtype=np.uint8)
    lo, hi = R.pack_codes(u)
    assert lo.shape == (2, 128, 48) and hi.shape == (2, 64, 48)
    np.testing.assert_array_equal(R.unpack_codes(lo, hi), u)
    # every plane byte pattern is reachable: unpack(random planes) packs back to the same planes
    lo2 = rng.integers(0, 256, size=(128, 48), dtype=np.uint8)
    hi2 = rng.integers(0, 256, size=(64, 48), dtype=np.uint8)
    l3, h3 = R.pack_codes(R.unpack_codes(lo2, hi2))
    np.testing.assert_array_equal(l3, lo2)
    np.testing.assert_array_equal(h3, hi2)


def test_unpack_agrees_with_the_kernel_sub_tile_form():
    """The reference kernel decodes a chunk as four 16-row sub-tiles from lo rows [0,16) and [16,32) and hi rows
    [0,16) (int6_gemm.py:185-188); the oracle's unpacking must give the same codes."""
    rng = np.random.default_rng(4)
    lo = rng.integers(0, 256, size=(64, 40), dtype=np.uint8).astype(np.int32)
    hi = rng.integers(0, 256, size=(32, 40), dtype=np.int32)
    u = R.unpack_codes(lo.astype(np.uint8), hi.astype(np.uint8)).astype(np.int32)
    for c in range(2):
        la, lb = lo[c * 32:c * 32 + 16], lo[c * 32 + 16:c * 32 + 32]
        hh = hi[c * 16:c * 16 + 16]
        w0 = (la & 15) | ((hh & 3) << 4)
        w1 = (lb & 15) | ((hh & 12) << 2)
        w2 = (la >> 4) | (hh & 48)
        w3 = (lb >> 4) | ((hh >> 2) & 48)
        np.testing.assert_array_equal(np.concatenate([w0, w1, w2, w3]), u[c * 64:(c + 1) * 64])


def test_dequant_and_matmul_oracle():
    """w = s q with the scale of row // group_k; C is numpy's product of a with that w (a shared weight broadcasts)."""
    rng = np.random.default_rng(5)
    K, N, g = 256, 32, 128
    u = rng.integers(0, 64, size=(K, N), dtype=np.uint8)
    lo, hi = R.pack_codes(u)
    sc = rng.uniform(0.01, 0.1, size=(K // g, N)).astype(np.float16)
    w = R.dequantize_ref(lo, hi, sc, g)
    assert w[0, 3] == (int(u[0, 3]) - 32) * float(sc[0, 3])
    assert w[200, 7] == (int(u[200, 7]) - 32) * float(sc[1, 7])
    a = rng.standard_normal((3, 5, K))
    C = R.int6_matmul_ref(a, lo, hi, sc, g)
    np.testing.assert_allclose(C[2], a[2] @ w, rtol=1e-12, atol=1e-12)
    # brute force on one element
    i, j = 4, 9
    assert abs(C[1, i, j] - sum(a[1, i, k] * w[k, j] for k in range(K))) < 1e-10


def test_known_answer_packed_records():
    """Single codes land at the byte the packed layout's definition gives (include/w6a16.h, w6a16_pack):
    record dword d of lane l sits at byte 1024 (d // 4) + 16 l + 4 (d % 4) of its 6144-byte block."""
    K, N, g = 64, 256, 64
    # row 5, column 35 = 16 * 2 + 3 (strip 0, tile 2, lane i = 3, q = 0, e = 5): lo byte row 5 -> dword 2 t + 1 = 5,
    # byte 1; top bits -> dword 16 + t = 18, byte e' = 1, bits 4-5
    # row 40 = 32 + 8, column 130 = 128 + 2 (strip 1, tile 0, i = 2, q = 1, e = 0): high nibble of lo row 8 ->
    # dword 0, byte 0, bits 4-7; top bits -> dword 16, byte 0, bits 2-3
    u = np.zeros((K, N), np.uint8)
    u[5, 35] = 0x3F
    u[40, 130] = 0x3F
    lo, hi = R.pack_codes(u)
    sc = np.ones((1, N), np.float16)
    w, _ = R.pack_packed(lo, hi, sc, g)
    w = w[0]
    expect = np.zeros(2 * 6144, np.uint8)
    lane = 3
    expect[1024 * 1 + 16 * lane + 4 * 1 + 1] = 0x0F        # dword 5 = 0x00000F00
    expect[1024 * 4 + 16 * lane + 4 * 2 + 1] = 0x30        # dword 18 = 0x00003000
    lane = 16 + 2
    expect[6144 + 16 * lane] = 0xF0                        # dword 0 = 0x000000F0
    expect[6144 + 1024 * 4 + 16 * lane] = 0x0C             # dword 16 = 0x0000000C
    np.testing.assert_array_equal(w, expect)


def test_packed_layout_round_trip():
    rng = np.random.default_rng(8)
    for B, K, N, g in [(1, 128, 144, 64), (2, 192, 256, 192)]:
        u = rng.integers(0, 64, size=(B, K, N), dtype=np.uint8)
        lo, hi = R.pack_codes(u)
        sc = rng.uniform(0.01, 0.1, size=(B, K // g, N)).astype(np.float16)
        w, s = R.pack_packed(lo, hi, sc, g)
        strips = (N + 127) // 128
        assert w.shape == (B, strips * (K // 64) * 6144) and s.shape == (B, strips * (K // g) * 128)
        u2, s2 = R.unpack_packed(w, s, K, N, g)
        np.testing.assert_array_equal(u2, u)
        np.testing.assert_array_equal(s2, sc)


# ----------------------------------------------------------------------------------------------------------------
# the product's quantiser (host code in torch; CPU here)
# ----------------------------------------------------------------------------------------------------------------
def _codes_and_scales(w, g, clip=True):
    lo, hi, sc, gg = I6.quantize_int6(torch.from_numpy(w), g, clip_search=clip)
    return lo.numpy(), hi.numpy(), sc.numpy(), gg


@pytest.mark.parametrize("clip", [True, False])
def test_quantiser_contract(clip):
    rng = np.random.default_rng(6)
    K, N, g = 256, 48, 128
    w = (rng.standard_normal((K, N)) * rng.uniform(0.01, 1.0, size=(1, N))).astype(np.float32)
    w[:, 5] *= 0
    w[:, 5] += 0.25                                  # a constant column
    w[3, 7] = 40.0                                   # an outlier
    lo, hi, sc, gg = _codes_and_scales(w, g, clip)
    assert gg == g and lo.shape == (K // 2, N) and hi.shape == (K // 4, N) and sc.shape == (K // g, N)
    assert sc.dtype == np.float16
    u = R.unpack_codes(lo, hi).astype(np.int64)
    q = u - 32
    s = sc.astype(np.float32)[np.arange(K) // g]
    # the codes are the rounding of w by the stored scale, clamped to the int6 range
    expect_q = np.clip(np.round(w / s), -32, 31)
    np.testing.assert_array_equal(q, expect_q)
    ratios = (1.0, 0.97, 0.94, 0.91, 0.88, 0.85) if clip else (1.0,)
    wg = w.reshape(K // g, g, N)
    amax = np.maximum(np.abs(wg).max(axis=1), 1e-10)
    for gi in range(K // g):
        for n in range(N):
            cands = [np.float32(np.float16(np.float32(amax[gi, n]) * np.float32(r) / np.float32(31.5)))
                     for r in ratios]
            assert np.float32(sc[gi, n]) in cands, (gi, n)
            x = wg[gi, :, n]
            errs = [((np.clip(np.round(x / c), -32, 31) * c - x) ** 2).sum() for c in cands]
            chosen = float(((q.reshape(K // g, g, N)[gi, :, n] * np.float32(sc[gi, n]) - x) ** 2).sum())
            assert chosen <= min(errs) * (1 + 1e-5) + 1e-12, (gi, n)
    # unclipped weights round to within half a step
    err = np.abs(q * s - w)
    inside = np.abs(w / s) <= 31.0
    assert (err[inside] <= 0.5 * s[inside] * (1 + 1e-6)).all()


def test_quantiser_batched_group_and_layout():
    rng = np.random.default_rng(7)
    w = rng.standard_normal((2, 128, 16)).astype(np.float32)
    lo, hi, sc, g = I6.quantize_int6(torch.from_numpy(w), group_k=0, clip_search=False)  # 0 -> one group
    assert g == 128 and lo.shape == (2, 64, 16) and hi.shape == (2, 32, 16) and sc.shape == (2, 1, 16)
    w1 = R.dequantize_ref(lo[1].numpy(), hi[1].numpy(), sc[1].numpy(), g)
    # absmax / 31.5 scales clip nothing but the rounding of s to fp16 (relative 2^-11, times up to 32 steps):
    # every weight is within 0.5 + 32 * 2^-11 < 0.52 steps
    assert (np.abs(w1 - w[1]) <= 0.52 * sc[1].float().numpy()).all()
    with pytest.raises(ValueError):
        I6.quantize_int6(torch.zeros(96, 16), 64)       # K % 64
    with pytest.raises(ValueError):
        I6.quantize_int6(torch.zeros(256, 16), 96)      # group_k % 64


# ----------------------------------------------------------------------------------------------------------------
# C ABI (no launch)
# ----------------------------------------------------------------------------------------------------------------
def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    return sorted(set(re.findall(r"^[A-Za-z_][\w \*]*?\b(w6a16_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_w6a16_function():
    lib = _lib.load()
    names = declared_functions()
    assert set(names) == set(_lib.W6A16_EXPORTED), names
    for n in names:
        assert hasattr(lib, n), n
    assert lib.w6a16_args_size() == ctypes.sizeof(_lib.W6a16Args)


def base_args(**kw):
    a = _lib.W6a16Args()
    fake = 0x10000
    a.a, a.lo, a.hi, a.scales, a.out = fake, fake, fake, fake, fake
    a.B, a.M, a.N, a.K, a.group_k, a.split_k = 1, 4, 256, 512, 128, 1
    a.a_batch_stride, a.a_row_stride = 4 * 512, 512
    a.lo_batch_stride, a.hi_batch_stride, a.scales_batch_stride = 256 * 256, 128 * 256, 4 * 256
    a.out_batch_stride, a.out_row_stride = 4 * 256, 256
    a.out_dtype = _lib.W6A16_OUT_BF16
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("field,value,code", [
    ("K", 500, _lib.WKV7_ERR_SHAPE),
    ("N", 250, _lib.WKV7_ERR_SHAPE),
    ("group_k", 96, _lib.WKV7_ERR_SHAPE),
    ("group_k", 1024, _lib.WKV7_ERR_SHAPE),
    ("B", 0, _lib.WKV7_ERR_SHAPE),
    ("B", 65536, _lib.WKV7_ERR_SHAPE),                # grid z = batch (x 16-row groups for M <= 32)
    ("a_row_stride", 256, _lib.WKV7_ERR_SHAPE),       # < K
    ("out_row_stride", 128, _lib.WKV7_ERR_SHAPE),     # < N
    ("split_k", 0, _lib.WKV7_ERR_ARG),
    ("split_k", 257, _lib.WKV7_ERR_ARG),
    ("out_dtype", 3, _lib.WKV7_ERR_ARG),
    ("a_dtype", 2, _lib.WKV7_ERR_ARG),
    ("lo", None, _lib.WKV7_ERR_NULL),
    ("out", None, _lib.WKV7_ERR_NULL),
    ("a", 0x10008, _lib.WKV7_ERR_ALIGN),
    ("hi", 0x10004, _lib.WKV7_ERR_ALIGN),
    ("scales", 0x10002, _lib.WKV7_ERR_ALIGN),
    ("a_row_stride", 516, _lib.WKV7_ERR_ALIGN),
    ("lo_batch_stride", 8, _lib.WKV7_ERR_ALIGN),
    ("split_k", 4, _lib.WKV7_ERR_WORKSPACE),          # partials needed, none given
])
def test_matmul_validates_before_launch(field, value, code):
    a = base_args(**{field: value})
    assert _lib.load().w6a16_matmul(ctypes.byref(a), None) == code


def test_matmul_empty_and_workspace_size():
    lib = _lib.load()
    assert lib.w6a16_matmul(ctypes.byref(base_args(M=0, a=None, out=None)), None) == _lib.WKV7_OK
    n = ctypes.c_size_t(1)
    assert lib.w6a16_workspace_size(ctypes.byref(base_args()), ctypes.byref(n)) == 0 and n.value == 0
    assert lib.w6a16_workspace_size(ctypes.byref(base_args(split_k=8, B=2, M=3)), ctypes.byref(n)) == 0
    # the fixed 1 MiB counter region, then per tile (B x M groups x 128-column strips = 2 x 1 x 2) and split a
    # 16 x 128 fp32 partial tile
    tiles = 2 * 1 * 2
    assert n.value == (1 << 20) + tiles * 8 * 16 * 128 * 4
    # M > 32 runs the wide kernel: after the counters and partials, the row sums of A per chain of two 64-row chunks
    # (group_k = 128), [B][K / 128][rows padded to the M groups]
    # M = 40: two 16-row tiles per wavefront, two M groups of 32 rows, two strips (N = 256): four tiles
    assert lib.w6a16_workspace_size(ctypes.byref(base_args(split_k=2, M=40)), ctypes.byref(n)) == 0
    assert n.value == (1 << 20) + 4 * 2 * 32 * 128 * 4 + 4 * 64 * 4
    # M = 100: four 16-row tiles per wavefront, two M groups of 64 rows, two strips
    assert lib.w6a16_workspace_size(ctypes.byref(base_args(split_k=2, M=100)), ctypes.byref(n)) == 0
    assert n.value == (1 << 20) + 4 * 2 * 64 * 128 * 4 + 4 * 128 * 4
    # M = 200: four M groups of 64 rows
    assert lib.w6a16_workspace_size(ctypes.byref(base_args(split_k=2, M=200)), ctypes.byref(n)) == 0
    assert n.value == (1 << 20) + 8 * 2 * 64 * 128 * 4 + 4 * 256 * 4
    # without split-K the wide kernel still needs the counter region's place and the row sums
    assert lib.w6a16_workspace_size(ctypes.byref(base_args(M=40)), ctypes.byref(n)) == 0
    assert n.value == (1 << 20) + 4 * 64 * 4
    wide = base_args(M=40, a_batch_stride=40 * 512, out_batch_stride=40 * 256)
    assert lib.w6a16_matmul(ctypes.byref(wide), None) == _lib.WKV7_ERR_WORKSPACE
    small = base_args(split_k=8, B=2, M=3, workspace=0x10000, workspace_bytes=(1 << 20) + tiles * 8 * 16 * 128 * 4 - 4)
    assert lib.w6a16_matmul(ctypes.byref(small), None) == _lib.WKV7_ERR_WORKSPACE
    # the in-workgroup split-K kernel (packed layout, split 2..8; or planes once one workgroup per strip and M group
    # fills the chip) sums its partials in LDS: no workspace
    packed = dict(format=_lib.W6A16_FORMAT_PACKED, split_k=8, B=2, M=3)
    assert lib.w6a16_workspace_size(ctypes.byref(base_args(**packed)), ctypes.byref(n)) == 0 and n.value == 0
    assert lib.w6a16_workspace_size(ctypes.byref(base_args(**dict(packed, split_k=16))), ctypes.byref(n)) == 0
    assert n.value == (1 << 20) + tiles * 16 * 16 * 128 * 4
    # at most 262144 tiles (the counter region's u32 counters): 40000 x 1 x 8 tiles are refused, 30000 x 1 x 8 reach
    # the workspace check (split 16: the cross-workgroup hand-off)
    many = dict(split_k=16, N=1024, out_row_stride=1024, out_batch_stride=4 * 1024, workspace=0x10000, workspace_bytes=1)
    assert lib.w6a16_matmul(ctypes.byref(base_args(B=40000, **many)), None) == _lib.WKV7_ERR_SHAPE
    assert lib.w6a16_matmul(ctypes.byref(base_args(B=30000, **many)), None) == _lib.WKV7_ERR_WORKSPACE
    odd = base_args(split_k=8, B=2, M=3, workspace=0x10080, workspace_bytes=1 << 24)
    assert lib.w6a16_matmul(ctypes.byref(odd), None) == _lib.WKV7_ERR_ALIGN


def test_packed_entry_points_validate_before_launch():
    lib = _lib.load()
    f = 0x10000
    wb, sb = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert lib.w6a16_packed_size(2, 256, 144, 64, ctypes.byref(wb), ctypes.byref(sb)) == 0
    assert wb.value == 2 * 2 * 4 * 6144 and sb.value == 2 * 2 * 4 * 128 * 2
    assert lib.w6a16_packed_size(1, 256, 140, 64, ctypes.byref(wb), ctypes.byref(sb)) == _lib.WKV7_ERR_SHAPE
    assert lib.w6a16_pack(f, f, f, 1, 256, 144, 96, 0, 0, 0, f, f, None) == _lib.WKV7_ERR_SHAPE
    assert lib.w6a16_pack(f, None, f, 1, 256, 144, 64, 0, 0, 0, f, f, None) == _lib.WKV7_ERR_NULL
    assert lib.w6a16_pack(f, f, f, 1, 256, 144, 64, 0, 0, 0, f + 8, f, None) == _lib.WKV7_ERR_ALIGN
    assert lib.w6a16_dequantize_packed(f, None, f, 1, 256, 144, 64, 0, 0, None) == _lib.WKV7_ERR_NULL
    assert lib.w6a16_dequantize_packed(f, f, f, 1, 256, 144, 64, 0, 3, None) == _lib.WKV7_ERR_ARG
    # the matmul's format field: packed needs no hi plane but 16-byte aligned packed scales
    a = base_args(format=_lib.W6A16_FORMAT_PACKED, hi=None)
    assert lib.w6a16_matmul(ctypes.byref(base_args(format=2)), None) == _lib.WKV7_ERR_ARG
    assert lib.w6a16_matmul(ctypes.byref(base_args(format=_lib.W6A16_FORMAT_PACKED, hi=None, scales=0x10004)),
                            None) == _lib.WKV7_ERR_ALIGN
    assert lib.w6a16_matmul(ctypes.byref(base_args(format=_lib.W6A16_FORMAT_PLANES, hi=None)), None) == \
        _lib.WKV7_ERR_NULL
    assert a.format == _lib.W6A16_FORMAT_PACKED


def test_dequantize_validates_before_launch():
    lib = _lib.load()
    f = 0x10000
    ok = dict(lo=f, hi=f, sc=f, w=f, B=1, K=256, N=64, g=128, sl=0, sh=0, ss=0, sw=0, dt=_lib.W6A16_OUT_BF16)

    def call(**kw):
        d = dict(ok, **kw)
        return lib.w6a16_dequantize(d["lo"], d["hi"], d["sc"], d["w"], d["B"], d["K"], d["N"], d["g"], d["sl"],
                                    d["sh"], d["ss"], d["sw"], d["dt"], None)
    assert call(lo=None) == _lib.WKV7_ERR_NULL
    assert call(N=40) == _lib.WKV7_ERR_SHAPE
    assert call(K=200) == _lib.WKV7_ERR_SHAPE
    assert call(g=192) == _lib.WKV7_ERR_SHAPE
    assert call(dt=5) == _lib.WKV7_ERR_ARG
    assert call(w=f + 2) == _lib.WKV7_ERR_ALIGN
    assert call(sw=4) == _lib.WKV7_ERR_ALIGN


def test_split_rule():
    lib = _lib.load()
    for B, M, N, K in [(1, 1, 16384, 4096), (1, 16, 16384, 4096), (1, 64, 4096, 4096), (4, 1, 2048, 2048),
                       (1, 1, 256, 128), (1, 200, 65536, 8192)]:
        sk = lib.w6a16_plan_split(B, M, N, K)
        assert 1 <= sk <= 64 and sk & (sk - 1) == 0
        assert (K // 64) // sk >= 1
    # without a GPU the CU count is taken as 256: K = 4096, N = 16384 has 32 groups of four 128-column strips
    assert lib.w6a16_plan_split(1, 1, 16384, 4096) == 8
    # M > 32: the wide kernel, one 128-column strip per workgroup; two M groups of eight wavefronts (M = 64, 128) or
    # four M groups of four (M = 256) put eight wavefronts on every CU without split-K
    assert lib.w6a16_plan_split(1, 64, 16384, 4096) == 1
    assert lib.w6a16_plan_split(1, 128, 16384, 4096) == 1
    assert lib.w6a16_plan_split(1, 256, 16384, 4096) == 1
    assert lib.w6a16_plan_split(1, 128, 4096, 4096) == 4        # 32 strips x 2 M groups: split 4 fills the chip
    assert lib.w6a16_plan_split(1, 1, 1024, 16384) == 64        # 2 groups, 256 chunks: capped at 64
    assert lib.w6a16_plan_split(1, 1, 4096, 16384) == 32
    assert I6.plan_int6(1, 4096, 4096, 1) == (lib.w6a16_plan_split(1, 1, 4096, 4096), False)
    assert I6.plan_int6(8, 4096, 4096, 1)[1] is True
    # M = 32: two M groups x 128 strips = 256 in-workgroup blocks fill the chip, so the deepest split
    assert lib.w6a16_plan_split(1, 32, 16384, 4096) == 8


def test_split_rule_packed():
    """The packed layout takes split 4 instead of 8 where its kernel runs half strips (fewer strips x M groups than
    CUs) and the ranges keep at least 8 chunks; everywhere else it takes the planes' split."""
    lib = _lib.load()
    assert lib.w6a16_plan_split_packed(1, 1, 16384, 4096) == 4
    assert lib.w6a16_plan_split_packed(1, 16, 16384, 4096) == 4
    assert lib.w6a16_plan_split_packed(1, 32, 16384, 4096) == 8      # 256 blocks: whole strips
    assert lib.w6a16_plan_split_packed(1, 1, 16384, 1024) == 8       # 16 chunks: 4 per range at split 4
    for B, M, N, K in [(1, 64, 16384, 4096), (1, 1, 1024, 16384), (4, 1, 2048, 2048), (1, 1, 256, 128)]:
        assert lib.w6a16_plan_split_packed(B, M, N, K) == lib.w6a16_plan_split(B, M, N, K), (B, M, N, K)
    assert I6.plan_int6_packed(1, 16384, 4096, 1) == 4
