"""W6A16 on the GPU through the C ABI (include/w6a16.h), against the numpy oracle on the same weights.

Tolerances (stated per test):
  * dequantisation: exact (s q is exact in fp32; bf16 is its round-to-nearest-even);
  * the W6A16 kernel, fp32 result: |C - C_ref| <= 2e-5 (|a| @ |w|) element-wise (fp32 accumulation of exact
    bf16 x int6 products, scaled per 64-row chunk);
  * bf16 result: that plus one bf16 rounding, 2^-8 |C_ref|;
  * the dequantise-then-library-GEMM path (M > MAX_M): 8e-3 (|a| @ |w|) (the weight is rounded to bf16 first);
  * fp16 activations (the reference casts its codes to a.dtype): the kernels' fp32 result within 3e-4 (|a| @ |w|)
    (exact fp16 x int6 products; the offset 1024 + u, taken out once per chunk, leaves about 2^-24 x 1056 of the
    row's |a| sum per fp32 accumulation), fp16 outputs one fp16 rounding (2^-11 |C_ref|) more; the GEMM path 2e-3
    (|a| @ |w|) (the weight rounded to fp16 first).
"""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import say

from oracle import int6_ref as R

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
KERNEL_TOL = 2e-5
GEMM_TOL = 8e-3
F16_KERNEL_TOL = 3e-4
F16_GEMM_TOL = 2e-3


def _weights(rng, Bq, K, N, g):
    u = rng.integers(0, 64, size=(Bq, K, N), dtype=np.uint8)
    lo, hi = R.pack_codes(u)
    sc = rng.uniform(0.002, 0.05, size=(Bq, K // g, N)).astype(np.float16)
    return lo, hi, sc


def _act(rng, B, M, K):
    a = torch.from_numpy(rng.standard_normal((B, M, K)).astype(np.float32)).to(torch.bfloat16)
    return a


def _dev(*xs):
    return [torch.from_numpy(np.ascontiguousarray(x)).to(DEV) for x in xs]


def _split(split, B, M, N, K):
    """The split_k a planes-vs-packed comparison uses for both calls: the given one, else plan_int6's."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    return split if split is not None else I6.plan_int6(M, N, K, B, torch.device(DEV))[0]


def _check(C, a_bf, lo, hi, sc, g, tol, bf16_out=False, shared=False, f16_out=False):
    a64 = a_bf.float().numpy().astype(np.float64)
    L, H, S = (lo[0], hi[0], sc[0]) if shared else (lo, hi, sc)
    ref = R.int6_matmul_ref(a64, L, H, S, g)
    bound = R.abs_bound(a64, L, H, S, g)
    got = C.float().cpu().numpy().astype(np.float64)
    lim = tol * bound + (2.0 ** -8 * np.abs(ref) if bf16_out else 0.0) + (2.0 ** -11 * np.abs(ref) if f16_out else 0.0)
    lim = lim + 1e-30
    err = np.abs(got - ref)
    worst = np.unravel_index(np.argmax(err / lim), err.shape)
    assert (err <= lim).all(), f"worst at {worst}: got {got[worst]}, ref {ref[worst]}, limit {lim[worst]}"


@pytest.mark.parametrize("B,M,N,K,g,split", [
    (1, 1, 256, 512, 128, None),
    (1, 1, 4096, 4096, 128, None),
    (1, 2, 1024, 2048, 128, None),
    (1, 16, 2048, 1024, 64, None),
    (1, 37, 640, 1024, 128, None),
    (1, 64, 1024, 4096, 128, None),
    (1, 1, 16, 128, 128, None),       # narrowest N: one 16-column tile
    (1, 5, 144, 256, 256, None),      # N not a multiple of the 128-column wave tile; one group of K rows
    (1, 3, 512, 1024, 128, 1),
    (1, 3, 512, 1024, 128, 3),        # uneven split ranges
    (1, 1, 512, 640, 64, 7),          # 10 chunks over 7 splits: one empty range
    (1, 1, 256, 4096, 128, 64),
    (1, 17, 2048, 1024, 64, None),    # two M groups of one 16-row tile
    (1, 48, 144, 512, 256, 2),        # two 16-row tiles per wavefront; N not a multiple of 128
    (1, 100, 640, 1024, 128, 4),      # four M groups of 32 rows, the last one partly past M
    (1, 128, 1024, 2048, 128, None),
])
def test_matmul_matches_oracle(B, M, N, K, g, split):
    from rwkv_next_amd.kernels import int6_gemm as I6
    say("int6_matmul", dict(B=B, M=M, N=N, K=K, g=g, split=split))
    rng = np.random.default_rng(100 + M + N + K)
    lo, hi, sc = _weights(rng, 1, K, N, g)
    a = _act(rng, B, M, K)
    Ld, Hd, Sd = _dev(lo[0], hi[0], sc[0])
    C = I6.int6_matmul(a[0].to(DEV), Ld, Hd, Sd, g, split_k=split, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert C.shape == (M, N) and C.dtype == torch.float32
    _check(C[None], a, lo, hi, sc, g, KERNEL_TOL)
    Cb = I6.int6_matmul(a[0].to(DEV), Ld, Hd, Sd, g, split_k=split)
    torch.cuda.synchronize()
    assert Cb.dtype == torch.bfloat16
    _check(Cb[None], a, lo, hi, sc, g, KERNEL_TOL, bf16_out=True)


@pytest.mark.parametrize("B,M,N,K,g,shared,split", [
    (1, 80, 384, 640, 64, True, None),      # chains of one chunk (group_k = 64), two M groups of 64 rows
    (3, 70, 272, 512, 128, True, None),     # a batch sharing one weight; N not a multiple of 128
    (2, 150, 640, 1024, 256, False, None),  # four 16-row tiles per wavefront, one K part, three M groups
    (1, 96, 1024, 2048, 128, True, 3),      # split-K with uneven ranges of chains
])
def test_wide_kernel_matches_oracle(B, M, N, K, g, shared, split):
    """M > 32 runs the wide kernel (row-sum pre-pass, K parts, chains per quantisation group); planes and packed give
    the same bits."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    say("int6_matmul wide kernel", dict(B=B, M=M, N=N, K=K, g=g, shared=shared, split=split))
    rng = np.random.default_rng(300 + M + N + K)
    lo, hi, sc = _weights(rng, 1 if shared else B, K, N, g)
    a = _act(rng, B, M, K)
    Ld, Hd, Sd = _dev(lo, hi, sc)
    if shared:
        Ld, Hd, Sd = Ld[0], Hd[0], Sd[0]
    split = _split(split, B, M, N, K)
    C = I6.int6_matmul(a.to(DEV), Ld, Hd, Sd, g, split_k=split, out_dtype=torch.float32)
    pk = I6.prepack_int6(Ld, Hd, Sd, g)
    Cp = I6.int6_matmul(a.to(DEV), pk, split_k=split, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(C, Cp)
    _check(C, a, lo, hi, sc, g, KERNEL_TOL, shared=shared)


@pytest.mark.parametrize("seed", range(8))
def test_random_shapes_match_oracle(seed):
    """Seeded random shapes across both kernels: M in [1, 256] (weighted to the 16/32/64/128 tile edges), N a
    multiple of 16 up to 1280, K a multiple of 64 up to 2560, group_k in {64, 128, 256} dividing K, one or two
    batches with a shared or per-batch weight, automatic or forced split-K; planes and packed weights give the same
    bits, and the fp32 result is within KERNEL_TOL of the oracle."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    rng = np.random.default_rng(7000 + seed)
    M = int(rng.choice([1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 200, 256])) if rng.random() < 0.6 \
        else int(rng.integers(1, 257))
    N = 16 * int(rng.integers(1, 81))
    g = int(rng.choice([64, 128, 256]))
    K = g * int(rng.integers(1, 2560 // g + 1))
    B = int(rng.integers(1, 3))
    shared = bool(rng.random() < 0.5)
    split = None if rng.random() < 0.5 else int(rng.integers(1, 9))
    say("int6_matmul random", dict(seed=seed, B=B, M=M, N=N, K=K, g=g, shared=shared, split=split))
    lo, hi, sc = _weights(rng, 1 if shared else B, K, N, g)
    a = _act(rng, B, M, K)
    Ld, Hd, Sd = _dev(lo, hi, sc)
    if shared:
        Ld, Hd, Sd = Ld[0], Hd[0], Sd[0]
    split = _split(split, B, M, N, K)
    C = I6.int6_matmul(a.to(DEV), Ld, Hd, Sd, g, split_k=split, out_dtype=torch.float32)
    Cp = I6.int6_matmul(a.to(DEV), I6.prepack_int6(Ld, Hd, Sd, g), split_k=split, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert C.shape == (B, M, N)
    assert torch.equal(C, Cp)
    _check(C, a, lo, hi, sc, g, KERNEL_TOL, shared=shared)


@pytest.mark.parametrize("split", [2, 4, 8, 16])
def test_in_workgroup_split_on_planes(split):
    """B x ceil(M / 16) x N / 128 = 4 x 2 x 32 = 256 workgroups fill the chip, so split 2..8 runs the in-workgroup
    split-K kernel on the planes as well as on the packed layout (split 16: the cross-workgroup hand-off on both);
    the two layouts give the same bits, within KERNEL_TOL of the oracle."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    B, M, N, K, g = 4, 20, 4096, 1024, 128
    say("int6_matmul in-workgroup split", dict(B=B, M=M, N=N, K=K, split=split))
    rng = np.random.default_rng(60 + split)
    lo, hi, sc = _weights(rng, B, K, N, g)
    a = _act(rng, B, M, K)
    Ld, Hd, Sd = _dev(lo, hi, sc)
    C = I6.int6_matmul(a.to(DEV), Ld, Hd, Sd, g, split_k=split, out_dtype=torch.float32)
    Cp = I6.int6_matmul(a.to(DEV), I6.prepack_int6(Ld, Hd, Sd, g), split_k=split, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(C, Cp)
    _check(C, a, lo, hi, sc, g, KERNEL_TOL)


@pytest.mark.parametrize("N,M,split", [(80, 1, 4), (80, 17, 3), (208, 5, 2), (16, 32, 4), (208, 2, 8)])
def test_half_strips_ragged_n(N, M, split):
    """Packed layout, few strips: each workgroup takes half a 128-column strip (three chunks in flight at split <= 4,
    two at 8), so at N = 80 the second half (columns 64..127) holds 16 valid columns, at N = 16 none; split 3 leaves
    uneven ranges; planes (the cross-workgroup kernel) give the same bits."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    K, g = 768, 64
    say("int6_matmul half strips", dict(M=M, N=N, K=K, split=split))
    rng = np.random.default_rng(90 + N + M)
    lo, hi, sc = _weights(rng, 1, K, N, g)
    a = _act(rng, 1, M, K)
    Ld, Hd, Sd = _dev(lo, hi, sc)
    C = I6.int6_matmul(a.to(DEV), Ld[0], Hd[0], Sd[0], g, split_k=split, out_dtype=torch.float32)
    Cp = I6.int6_matmul(a.to(DEV), I6.prepack_int6(Ld[0], Hd[0], Sd[0], g), split_k=split, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(C, Cp)
    _check(C, a, lo, hi, sc, g, KERNEL_TOL, shared=True)


@pytest.mark.parametrize("shared,split", [(False, 3), (True, 4), (False, 8)])
def test_half_strips_batched(shared, split):
    """Half strips over a batch (grid z = batch x M groups; per-batch or shared packed weights and scales): same bits
    as the planes, within KERNEL_TOL of the oracle."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    B, M, N, K, g = 3, 21, 208, 768, 64
    say("int6_matmul half strips batched", dict(B=B, M=M, N=N, K=K, shared=shared, split=split))
    rng = np.random.default_rng(70 + split + shared)
    lo, hi, sc = _weights(rng, 1 if shared else B, K, N, g)
    a = _act(rng, B, M, K)
    Ld, Hd, Sd = _dev(lo, hi, sc)
    if shared:
        Ld, Hd, Sd = Ld[0], Hd[0], Sd[0]
    C = I6.int6_matmul(a.to(DEV), Ld, Hd, Sd, g, split_k=split, out_dtype=torch.float32)
    Cp = I6.int6_matmul(a.to(DEV), I6.prepack_int6(Ld, Hd, Sd, g), split_k=split, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(C, Cp)
    _check(C, a, lo, hi, sc, g, KERNEL_TOL, shared=shared)


@pytest.mark.parametrize("shared", [True, False])
def test_batched(shared):
    from rwkv_next_amd.kernels import int6_gemm as I6
    B, M, N, K, g = 3, 7, 384, 1024, 128
    say("int6_matmul batched", dict(B=B, M=M, shared=shared))
    rng = np.random.default_rng(11)
    lo, hi, sc = _weights(rng, 1 if shared else B, K, N, g)
    a = _act(rng, B, M, K)
    Ld, Hd, Sd = _dev(lo, hi, sc)
    if shared:
        Ld, Hd, Sd = Ld[0], Hd[0], Sd[0]
    C = I6.int6_matmul(a.to(DEV), Ld, Hd, Sd, g, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert C.shape == (B, M, N)
    _check(C, a, lo, hi, sc, g, KERNEL_TOL, shared=shared)


def test_strided_and_misaligned_activations():
    from rwkv_next_amd.kernels import int6_gemm as I6
    M, N, K, g = 9, 256, 512, 128
    say("int6_matmul strided", dict(M=M, N=N, K=K))
    rng = np.random.default_rng(12)
    lo, hi, sc = _weights(rng, 1, K, N, g)
    a = _act(rng, 1, M, K)
    Ld, Hd, Sd = _dev(lo[0], hi[0], sc[0])
    wide = torch.zeros(M, K + 64, dtype=torch.bfloat16, device=DEV)
    wide[:, 8:8 + K] = a[0].to(DEV)
    view = wide[:, 8:8 + K]                       # row stride K + 64, 16-byte aligned start
    C = I6.int6_matmul(view, Ld, Hd, Sd, g, out_dtype=torch.float32)
    flat = torch.zeros(M * K + 1, dtype=torch.bfloat16, device=DEV)
    flat[1:] = a[0].to(DEV).reshape(-1)
    mis = flat[1:].view(M, K)                     # 2-byte offset: the wrapper re-aligns it
    C2 = I6.int6_matmul(mis, Ld, Hd, Sd, g, out_dtype=torch.float32)
    torch.cuda.synchronize()
    _check(C[None], a, lo, hi, sc, g, KERNEL_TOL)
    assert torch.equal(C, C2)


def test_split_k_is_deterministic_and_consistent():
    """Every split gives the oracle's result within tolerance, and the same call twice gives identical bits."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    M, N, K, g = 4, 1024, 4096, 128
    say("int6_matmul split sweep", dict(M=M, N=N, K=K))
    rng = np.random.default_rng(13)
    lo, hi, sc = _weights(rng, 1, K, N, g)
    a = _act(rng, 1, M, K)
    Ld, Hd, Sd = _dev(lo[0], hi[0], sc[0])
    ad = a[0].to(DEV)
    for sk in (1, 2, 4, 8, 16, 32, 64):
        C = I6.int6_matmul(ad, Ld, Hd, Sd, g, split_k=sk, out_dtype=torch.float32)
        C2 = I6.int6_matmul(ad, Ld, Hd, Sd, g, split_k=sk, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(C, C2), sk
        _check(C[None], a, lo, hi, sc, g, KERNEL_TOL)


@pytest.mark.parametrize("B,M,N,K,g,split,packed", [
    (1, 1, 4096, 4096, 128, None, False),   # GEMV, split-K across workgroups or in the workgroup
    (1, 1, 4096, 4096, 128, None, True),    # packed: half strips
    (1, 5, 144, 256, 256, 3, False),        # narrow kernel, uneven split ranges, N past the last full strip
    (1, 16, 2048, 1024, 64, None, True),
    (2, 48, 272, 512, 128, None, False),    # wide kernel (row-sum pre-pass), batched weights
    (1, 150, 640, 1024, 256, 2, True),      # wide kernel, split-K
])
def test_fp16_activations(B, M, N, K, g, split, packed):
    """fp16 activations, as the reference takes them (its dot casts the codes to a.dtype, int6_gemm.py:144-147): the
    result is fp16 by default (a.dtype) or fp32; every kernel form is checked against the oracle on the same fp16
    values, and planes and packed weights give the same bits."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    say("int6_matmul fp16", dict(B=B, M=M, N=N, K=K, g=g, split=split, packed=packed))
    rng = np.random.default_rng(700 + M + N + K)
    lo, hi, sc = _weights(rng, B, K, N, g)
    a = torch.from_numpy(rng.standard_normal((B, M, K)).astype(np.float32)).to(torch.float16)
    Ld, Hd, Sd = _dev(lo, hi, sc)
    split = _split(split, B, M, N, K)
    w = I6.prepack_int6(Ld, Hd, Sd, g) if packed else None
    call = (lambda **kw: I6.int6_matmul(a.to(DEV), w, split_k=split, **kw)) if packed else \
        (lambda **kw: I6.int6_matmul(a.to(DEV), Ld, Hd, Sd, g, split_k=split, **kw))
    C = call(out_dtype=torch.float32)
    Ch = call()
    Cp = I6.int6_matmul(a.to(DEV), Ld, Hd, Sd, g, split_k=split, out_dtype=torch.float32) if packed else C
    torch.cuda.synchronize()
    assert C.dtype == torch.float32 and Ch.dtype == torch.float16 and Ch.shape == (B, M, N)
    assert torch.equal(C, Cp)
    _check(C, a, lo, hi, sc, g, F16_KERNEL_TOL)
    _check(Ch, a, lo, hi, sc, g, F16_KERNEL_TOL, f16_out=True)


def test_fp16_large_m_dequantises_to_fp16():
    from rwkv_next_amd.kernels import int6_gemm as I6
    M, N, K, g = I6.MAX_M + 44, 512, 1024, 128
    say("int6_matmul fp16 large M", dict(M=M, N=N, K=K))
    rng = np.random.default_rng(17)
    lo, hi, sc = _weights(rng, 1, K, N, g)
    a = torch.from_numpy(rng.standard_normal((1, M, K)).astype(np.float32)).to(torch.float16)
    Ld, Hd, Sd = _dev(lo[0], hi[0], sc[0])
    C = I6.int6_matmul(a[0].to(DEV), Ld, Hd, Sd, g)
    torch.cuda.synchronize()
    assert C.shape == (M, N) and C.dtype == torch.float16
    _check(C[None], a, lo, hi, sc, g, F16_GEMM_TOL, f16_out=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_dequantize_is_exact(dtype):
    from rwkv_next_amd.kernels import int6_gemm as I6
    K, N, g = 512, 272, 128
    say("dequantize_int6", dict(K=K, N=N, dtype=str(dtype)))
    rng = np.random.default_rng(14)
    lo, hi, sc = _weights(rng, 2, K, N, g)
    Ld, Hd, Sd = _dev(lo, hi, sc)
    w = I6.dequantize_int6(Ld, Hd, Sd, g, dtype=dtype)
    w0 = I6.dequantize_int6(Ld[1], Hd[1], Sd[1], g, dtype=dtype)
    torch.cuda.synchronize()
    ref = torch.from_numpy(R.dequantize_ref(lo, hi, sc, g).astype(np.float32)).to(dtype)
    assert w.shape == (2, K, N) and w0.shape == (K, N)
    assert torch.equal(w.cpu(), ref)
    assert torch.equal(w0.cpu(), ref[1])


def test_large_m_dequantises_then_library_gemm():
    from rwkv_next_amd.kernels import int6_gemm as I6
    M, N, K, g = I6.MAX_M + 44, 512, 1024, 128
    say("int6_matmul large M", dict(M=M, N=N, K=K))
    rng = np.random.default_rng(15)
    lo, hi, sc = _weights(rng, 1, K, N, g)
    a = _act(rng, 1, M, K)
    Ld, Hd, Sd = _dev(lo[0], hi[0], sc[0])
    C = I6.int6_matmul(a[0].to(DEV), Ld, Hd, Sd, g)
    torch.cuda.synchronize()
    assert C.shape == (M, N) and C.dtype == torch.bfloat16
    _check(C[None], a, lo, hi, sc, g, GEMM_TOL, bf16_out=True)


def test_quantise_on_device_then_matmul():
    """The reference's load-time flow: quantize_int6 on the GPU, then the op with plan_int6's plan."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    M, N, K = 4, 768, 2048
    say("quantize_int6 + op", dict(M=M, N=N, K=K))
    torch.manual_seed(16)
    w = (torch.randn(K, N) * 0.02).to(DEV)
    lo, hi, sc, g = I6.quantize_int6(w, 128)
    assert g == 128 and lo.shape == (K // 2, N) and hi.shape == (K // 4, N) and sc.shape == (K // g, N)
    # the codes are the rounding of w by the stored scales, clamped to [-32, 31]
    q = R.unpack_codes(lo.cpu().numpy(), hi.cpu().numpy()).astype(np.float32) - 32
    s = sc.cpu().float().numpy()[np.arange(K) // g]
    mism = q != np.clip(np.round(w.cpu().numpy() / s), -32, 31)
    assert mism.mean() < 1e-4, mism.sum()          # exact but for last-ulp divisions landing on a .5 boundary
    a = torch.randn(M, K).to(torch.bfloat16)
    sk, ud = I6.plan_int6(M, N, K, 1, torch.device(DEV))
    C = I6.int6_matmul_op(a.to(DEV), lo, hi, sc, g, sk, ud)
    Ce = I6.int6_matmul(a.to(DEV), lo, hi, sc, g)
    torch.cuda.synchronize()
    assert torch.equal(C, Ce)
    _check(C[None], a[None], lo.cpu().numpy(), hi.cpu().numpy(), sc.cpu().numpy(), g, KERNEL_TOL, bf16_out=True)
    # quantisation error against the float weight stays at the int6 level
    wq = I6.dequantize_int6(lo, hi, sc, g).cpu()
    rel = ((wq - w.cpu()).norm() / w.cpu().norm()).item()
    assert rel < 0.03, rel


# ----------------------------------------------------------------------------------------------------------------
# packed layout (prepack_int6): same codes, re-laid out; results must equal the planes' bit for bit
# ----------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("B,K,N,g", [(1, 512, 384, 128), (1, 256, 144, 256), (2, 192, 272, 64)])
def test_prepack_matches_oracle_layout(B, K, N, g):
    from rwkv_next_amd.kernels import int6_gemm as I6
    say("prepack_int6", dict(B=B, K=K, N=N, g=g))
    rng = np.random.default_rng(20 + K + N)
    lo, hi, sc = _weights(rng, B, K, N, g)
    Ld, Hd, Sd = _dev(lo, hi, sc)
    if B == 1:
        Ld, Hd, Sd = Ld[0], Hd[0], Sd[0]
    pk = I6.prepack_int6(Ld, Hd, Sd, g)
    torch.cuda.synchronize()
    w_ref, s_ref = R.pack_packed(lo, hi, sc, g)
    assert pk.batches == (0 if B == 1 else B) and (pk.K, pk.N, pk.group_k) == (K, N, g)
    np.testing.assert_array_equal(pk.weight.cpu().numpy(), w_ref)
    np.testing.assert_array_equal(pk.scales.cpu().view(torch.int16).numpy(), s_ref.view(np.int16))
    # dequantising the packed weight gives the planes' weight exactly
    for dt in (torch.float32, torch.bfloat16):
        wp = I6.dequantize_int6_packed(pk, dtype=dt)
        wq = I6.dequantize_int6(Ld, Hd, Sd, g, dtype=dt)
        torch.cuda.synchronize()
        assert torch.equal(wp, wq), dt


@pytest.mark.parametrize("B,M,N,K,g,split,shared", [
    (1, 1, 4096, 4096, 128, None, True),
    (1, 3, 512, 1024, 128, 3, True),
    (1, 16, 2048, 1024, 64, None, True),
    (1, 40, 640, 1024, 128, None, True),      # two 16-row tiles per wavefront
    (1, 5, 144, 256, 256, None, True),        # N not a multiple of 128
    (1, 1, 512, 640, 64, 7, True),            # an empty split range
    (3, 7, 384, 1024, 128, None, True),       # one weight shared by the batch
    (3, 7, 384, 1024, 128, None, False),      # one weight per batch row
])
def test_packed_matmul_equals_planes(B, M, N, K, g, split, shared):
    from rwkv_next_amd.kernels import int6_gemm as I6
    say("int6_matmul packed", dict(B=B, M=M, N=N, K=K, split=split, shared=shared))
    rng = np.random.default_rng(30 + M + N + K)
    Bq = 1 if shared else B
    lo, hi, sc = _weights(rng, Bq, K, N, g)
    a = _act(rng, B, M, K)
    Ld, Hd, Sd = _dev(lo, hi, sc)
    if shared:
        Ld, Hd, Sd = Ld[0], Hd[0], Sd[0]
    pk = I6.prepack_int6(Ld, Hd, Sd, g)
    ad = a.to(DEV) if B > 1 else a[0].to(DEV)
    if split is None:  # the packed default plan, given to the planes too (results depend on split_k)
        split = I6.plan_int6_packed(M, N, K, B, torch.device(DEV))
        Cd = I6.int6_matmul(ad, pk, out_dtype=torch.float32)
        assert torch.equal(Cd, I6.int6_matmul(ad, pk, split_k=split, out_dtype=torch.float32))
    for odt in (torch.float32, torch.bfloat16):
        Cp = I6.int6_matmul(ad, pk, split_k=split, out_dtype=odt)
        Cq = I6.int6_matmul(ad, Ld, Hd, Sd, g, split_k=split, out_dtype=odt)
        torch.cuda.synchronize()
        assert torch.equal(Cp, Cq), odt
    _check(Cp.float() if B > 1 else Cp.float()[None], a, lo, hi, sc, g, KERNEL_TOL, bf16_out=True, shared=shared)
    # the functional op
    Co = I6.int6_matmul_packed_op(ad, pk.weight, pk.scales, pk.batches, K, N, g, split)
    torch.cuda.synchronize()
    assert torch.equal(Co, Cp)


def test_packed_large_m_path():
    from rwkv_next_amd.kernels import int6_gemm as I6
    M, N, K, g = I6.MAX_M + 9, 384, 512, 128
    say("int6_matmul packed large M", dict(M=M, N=N, K=K))
    rng = np.random.default_rng(41)
    lo, hi, sc = _weights(rng, 1, K, N, g)
    a = _act(rng, 1, M, K)
    Ld, Hd, Sd = _dev(lo[0], hi[0], sc[0])
    pk = I6.prepack_int6(Ld, Hd, Sd, g)
    Cp = I6.int6_matmul(a[0].to(DEV), pk)
    Cq = I6.int6_matmul(a[0].to(DEV), Ld, Hd, Sd, g)
    torch.cuda.synchronize()
    assert torch.equal(Cp, Cq)


@pytest.mark.parametrize("packed", [False, True])
def test_kernel_beyond_128_rows(monkeypatch, packed):
    """The kernel itself takes any M (the module hands M > MAX_M to dequantise + library GEMM by default): 200 rows
    are seven M groups of 32 rows, batched with a per-batch weight."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    monkeypatch.setattr(I6, "MAX_M", 1 << 20)
    B, M, N, K, g = 2, 200, 384, 512, 128
    say("int6_matmul kernel M > 128", dict(B=B, M=M, N=N, K=K, packed=packed))
    rng = np.random.default_rng(63)
    lo, hi, sc = _weights(rng, B, K, N, g)
    a = _act(rng, B, M, K)
    Ld, Hd, Sd = _dev(lo, hi, sc)
    w = (I6.prepack_int6(Ld, Hd, Sd, g),) if packed else (Ld, Hd, Sd, g)
    for split in (1, 2):
        C = I6.int6_matmul(a.to(DEV), *w, split_k=split, out_dtype=torch.float32)
        torch.cuda.synchronize()
        _check(C, a, lo, hi, sc, g, KERNEL_TOL)


def _dequant_as(lo, hi, sc, g, dtype):
    """s q rounded to `dtype` (what w6a16_dequantize writes), as float64."""
    w = torch.from_numpy(R.dequantize_ref(lo, hi, sc, g).astype(np.float32)).to(dtype)
    return w.double().numpy()


@pytest.mark.parametrize("B,M,N,K,g,adt,shared", [
    (1, 257, 272, 192, 64, torch.bfloat16, False),    # a second M tile of one row; a last N tile of 16 columns
    (2, 300, 512, 512, 128, torch.bfloat16, False),   # batched weights
    (3, 300, 400, 256, 128, torch.bfloat16, True),    # one weight for the batch; N not a multiple of 128
    (1, 520, 1024, 1024, 128, torch.float16, False),  # fp16 activations
    (1, 2304, 768, 256, 256, torch.bfloat16, False),  # 9 x 3 tiles: the XCD-banded tile order
])
def test_large_m_kernel(monkeypatch, B, M, N, K, g, adt, shared):
    """M > 256 on packed weights runs the large-M kernel (the weight dequantised in LDS to A's type, then the
    product): its result is A times the dequantised weight (the values w6a16_dequantize writes) with fp32
    accumulation, |C - C_ref| <= 2e-5 (|a| @ |w~|), plus one rounding of the output type."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    monkeypatch.setattr(I6, "MAX_M", 1 << 20)
    say("int6_matmul large-M kernel", dict(B=B, M=M, N=N, K=K, g=g, adt=str(adt), shared=shared))
    rng = np.random.default_rng(900 + M + N + K)
    Bq = 1 if shared else B
    lo, hi, sc = _weights(rng, Bq, K, N, g)
    a = torch.from_numpy(rng.standard_normal((B, M, K)).astype(np.float32)).to(adt)
    Ld, Hd, Sd = _dev(lo, hi, sc)
    pk = I6.prepack_int6(Ld[0], Hd[0], Sd[0], g) if shared else I6.prepack_int6(Ld, Hd, Sd, g)
    a_dev = a.to(DEV)
    C = I6.int6_matmul(a_dev, pk, out_dtype=torch.float32)
    Co = I6.int6_matmul(a_dev, pk)
    torch.cuda.synchronize()
    assert C.shape == (B, M, N) and Co.dtype == adt
    w = _dequant_as(lo, hi, sc, g, adt)
    a64 = a.double().numpy()
    wb = [w[0 if shared else bi] for bi in range(B)]
    ref = np.stack([a64[bi] @ wb[bi] for bi in range(B)])
    bound = np.stack([np.abs(a64[bi]) @ np.abs(wb[bi]) for bi in range(B)]) + 1e-30
    got = C.cpu().double().numpy()
    err = np.abs(got - ref)
    assert (err <= 2e-5 * bound).all(), f"max err / bound {(err / bound).max():.3g}"
    rnd = 2.0 ** -8 if adt == torch.bfloat16 else 2.0 ** -11
    got_o = Co.cpu().double().numpy()
    assert (np.abs(got_o - ref) <= 2e-5 * bound + rnd * np.abs(ref)).all()


def test_large_m_kernel_unaligned_output(monkeypatch):
    """An output whose rows are not 16-byte aligned takes element stores; the result equals the aligned call's."""
    from rwkv_next_amd import _lib
    from rwkv_next_amd.kernels import int6_gemm as I6
    monkeypatch.setattr(I6, "MAX_M", 1 << 20)
    M, N, K, g = 300, 272, 256, 128
    say("int6 large-M kernel, strided output", dict(M=M, N=N, K=K))
    rng = np.random.default_rng(933)
    lo, hi, sc = _weights(rng, 1, K, N, g)
    a = _act(rng, 1, M, K)[0].to(DEV)
    Ld, Hd, Sd = _dev(lo[0], hi[0], sc[0])
    pk = I6.prepack_int6(Ld, Hd, Sd, g)
    C = I6.int6_matmul(a, pk)
    big = torch.full((M, N + 3), 7.0, dtype=torch.bfloat16, device=DEV)
    out = big[:, 1:N + 1]  # rows N + 3 elements apart, first element 2 bytes past a 16-byte boundary
    args = _lib.W6a16Args()
    args.a, args.a_batch_stride, args.a_row_stride = a.data_ptr(), 0, a.stride(0)
    args.format, args.lo, args.scales = _lib.W6A16_FORMAT_PACKED, pk.weight.data_ptr(), pk.scales.data_ptr()
    args.out, args.out_batch_stride, args.out_row_stride = out.data_ptr(), 0, out.stride(0)
    args.B, args.M, args.N, args.K, args.group_k, args.split_k = 1, M, N, K, g, 1
    args.out_dtype, args.a_dtype = _lib.W6A16_OUT_BF16, _lib.W6A16_IN_BF16
    lib = _lib.load()
    nb = ctypes.c_size_t(0)
    _lib.check(lib.w6a16_workspace_size(args, ctypes.byref(nb)))
    assert nb.value == 0  # the large-M kernel takes no workspace
    _lib.check(lib.w6a16_matmul(args, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(out, C)
    assert (big[:, 0] == 7).all() and (big[:, N + 1:] == 7).all()


def test_workspace_shared_across_shapes():
    """One stream's workspace serves calls whose tile counts differ, in an order where a call with few tiles (and
    large partials) precedes one with many: the counters live in a region the partials never reach."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    N, K, g = 2048, 1024, 128
    rng = np.random.default_rng(61)
    lo, hi, sc = _weights(rng, 1, K, N, g)
    Ld, Hd, Sd = _dev(lo[0], hi[0], sc[0])
    for M, split in [(1, 16), (128, 4), (3, 16), (64, 2), (128, 8), (17, 4), (1, 8)]:
        say("int6_matmul workspace sequence", dict(M=M, N=N, K=K, split=split))
        a = _act(rng, 1, M, K)
        C = I6.int6_matmul(a[0].to(DEV), Ld, Hd, Sd, g, split_k=split, out_dtype=torch.float32)
        torch.cuda.synchronize()
        _check(C[None], a, lo, hi, sc, g, KERNEL_TOL)


def test_workspace_created_during_graph_capture():
    """A workspace first created inside a HIP graph capture is zero-filled by that graph only; a second graph
    captured on the same stream starts with its own fill of the counters, so either graph may be replayed first.
    Each graph is replayed several times, with eager calls between the replays, and every replay is checked."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    M, N, K, g = 64, 1024, 2048, 128
    say("int6_matmul graph capture workspace", dict(M=M, N=N, K=K))
    rng = np.random.default_rng(62)
    lo, hi, sc = _weights(rng, 1, K, N, g)
    Ld, Hd, Sd = _dev(lo[0], hi[0], sc[0])
    acts = [_act(rng, 1, M, K) for _ in range(2)]
    xs = [x[0].to(DEV) for x in acts]
    cs = torch.cuda.Stream()
    I6._WORKSPACES.pop((torch.device(DEV).index or 0, cs.cuda_stream), None)   # force creation inside the capture
    graphs, outs = [], []
    torch.cuda.synchronize()
    for x in xs:
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=cs):
            outs.append(I6.int6_matmul_op(x, Ld, Hd, Sd, g, 4, True))
        graphs.append(gr)
    for rep in range(3):
        for j in (1, 0):                      # the graph that did not create the workspace first
            graphs[j].replay()
            torch.cuda.synchronize()
            _check(outs[j][None], acts[j], lo, hi, sc, g, KERNEL_TOL, bf16_out=True)
        with torch.cuda.stream(cs):           # eager calls on the capture stream between replays
            C = I6.int6_matmul(xs[rep % 2], Ld, Hd, Sd, g, split_k=4, out_dtype=torch.float32)
        torch.cuda.synchronize()
        _check(C[None], acts[rep % 2], lo, hi, sc, g, KERNEL_TOL)


def test_two_streams_use_separate_workspaces():
    """Split-K calls issued on two streams without synchronisation between them (they may run at the same time):
    each stream has its own arrival counters, so every result equals the single-stream one bit for bit."""
    from rwkv_next_amd.kernels import int6_gemm as I6
    M, N, K, g = 2, 2048, 4096, 128
    say("int6_matmul two streams", dict(M=M, N=N, K=K))
    rng = np.random.default_rng(51)
    lo, hi, sc = _weights(rng, 1, K, N, g)
    Ld, Hd, Sd = _dev(lo[0], hi[0], sc[0])
    acts = [_act(rng, 1, M, K)[0].to(DEV) for _ in range(8)]
    ref = [I6.int6_matmul(x, Ld, Hd, Sd, g, split_k=8, out_dtype=torch.float32) for x in acts]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = []
    for j, x in enumerate(acts):
        with torch.cuda.stream(streams[j % 2]):
            outs.append(I6.int6_matmul(x, Ld, Hd, Sd, g, split_k=8, out_dtype=torch.float32))
    torch.cuda.synchronize()
    for j in range(len(acts)):
        assert torch.equal(outs[j], ref[j]), j
