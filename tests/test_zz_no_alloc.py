"""wkv7_run_noalloc (the allocation-free variant of wkv7_run, include/wkv7_noalloc.h, in librwkv7_noalloc.so) through
the C ABI: two chunked calls
in a row (the second smaller), a ragged call, a decode call and the headline prefill (configuration 2), each
bit-identical to wkv7_run with a
caller-allocated workspace on the same inputs; a call that needs more than WKV7_NOALLOC_SCRATCH_BYTES is refused
before anything is launched."""
import ctypes
import types

import numpy as np
import pytest

from gpu_util import operands, say, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def lib():
    """wkv7_run from librwkv7_hip.so and wkv7_run_noalloc from librwkv7_noalloc.so (which links the former)."""
    from rwkv_next_amd import _lib
    main, noalloc = _lib.load(), _lib.load_noalloc()
    return types.SimpleNamespace(wkv7_run=main.wkv7_run, wkv7_run_noalloc=noalloc.wkv7_run_noalloc)


def make_args(x, H, N, T, total, o, h0=None, ht=None, cu=None, algo=0):
    from rwkv_next_amd import _lib
    a = _lib.Wkv7Args()
    for name, t in zip(("r", "w", "k", "v", "a", "b"), x):
        setattr(a, name, t.data_ptr())
    a.in_tok_stride = a.o_tok_stride = H * 64
    a.o = o.data_ptr()
    if h0 is not None:
        a.h0, a.h0_rows = h0.data_ptr(), N
    if ht is not None:
        a.ht, a.ht_rows = ht.data_ptr(), N
    if cu is not None:
        a.cu_seqlens = cu.data_ptr()
    a.num_seqs, a.T, a.total_tokens, a.H, a.head_size, a.algo, a.rec_max_len = N, T, total, H, 64, algo, -1
    return a


def run_both(lib, dev, x, H, N, T, total, h0=None, cu=None, algo=0):
    """wkv7_run with a torch-allocated workspace, then wkv7_run_noalloc, on the same inputs."""
    from rwkv_next_amd import _lib
    stream = torch.cuda.current_stream(dev).cuda_stream
    outs = []
    for noalloc in (False, True):
        o = torch.full_like(x[3], float("nan"))
        ht = torch.full((N, H, 64, 64), float("nan"), device=dev)
        a = make_args(x, H, N, T, total, o, h0, ht, cu, algo)
        if noalloc:
            rc = lib.wkv7_run_noalloc(ctypes.byref(a), ctypes.c_void_p(stream))
        else:
            nbytes = _lib.workspace_size(a)
            # zeroed: the first WKV7_SEG_FLAG_BYTES are the segmented kernel's hand-off flags
            ws = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=dev)
            a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
            rc = lib.wkv7_run(ctypes.byref(a), ctypes.c_void_p(stream))
        assert rc == 0, _lib.strerror(rc)
        torch.cuda.synchronize()
        outs.append((o, ht))
    (o0, s0), (o1, s1) = outs
    assert torch.equal(o0, o1) and torch.equal(s0, s1)
    assert not torch.isnan(o1.float()).any() and not torch.isnan(s1).any()


@pytest.mark.parametrize("algo,sizes", [(2, ((2, 300, 1), (1, 100, 2))), (4, ((1, 3000, 1), (2, 700, 2)))])
def test_two_chunked_calls_in_a_row_second_smaller(dev, lib, algo, sizes):
    """The two-kernel chunked path (algo 2) and the segmented kernel (algo 4: rows cut into several segments that
    hand their states on through flags in the scratch's first 256 KB, which every call must leave zero)."""
    H = 8
    for B, T, seed in sizes:
        say("noalloc chunked", algo, B, T)
        x = to_dev(operands(B, T, H, seed=seed), dev)
        h0 = torch.from_numpy((0.3 * np.random.default_rng(seed).standard_normal((B, H, 64, 64))).astype(np.float32)).to(dev)
        run_both(lib, dev, x, H, B, T, B * T, h0=h0, algo=algo)


def test_ragged_and_decode_calls(dev, lib):
    H = 8
    lens = [5, 1, 130, 0, 64, 33]
    say("noalloc ragged", lens)
    total = sum(lens)
    x = to_dev(operands(1, total, H, seed=3), dev)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=dev)
    h0 = torch.from_numpy((0.3 * np.random.default_rng(4).standard_normal((len(lens), H, 64, 64))).astype(np.float32)).to(dev)
    run_both(lib, dev, x, H, len(lens), 0, total, h0=h0, cu=cu)
    say("noalloc decode")
    x = to_dev(operands(16, 1, H, seed=5), dev)
    h0 = torch.from_numpy((0.3 * np.random.default_rng(6).standard_normal((16, H, 64, 64))).astype(np.float32)).to(dev)
    run_both(lib, dev, x, H, 16, 1, 16, h0=h0)


def test_headline_prefill_fits(dev, lib):
    """Configuration 2 (B = 1, T = 4096, H = 64), AUTO: the segmented kernel's workspace (hand-off flags and entries,
    the later segments' Q P records: about 33 MB) fits the scratch, and the result equals wkv7_run's."""
    from rwkv_next_amd import _lib
    H, B, T = 64, 1, 4096
    say("noalloc configuration 2", B, T, H)
    x = to_dev(operands(B, T, H, seed=12), dev)
    a = make_args(x, H, B, T, B * T, torch.empty_like(x[3]))
    assert 0 < _lib.workspace_size(a) <= _lib.WKV7_NOALLOC_SCRATCH_BYTES
    run_both(lib, dev, x, H, B, T, B * T)


def test_too_large_is_refused_before_launch(dev, lib):
    from rwkv_next_amd import _lib
    H, T = 64, 8192
    say("noalloc over the limit")
    x = [torch.zeros(1, T, H * 64, dtype=torch.bfloat16, device=dev) for _ in range(6)]
    o = torch.full_like(x[3], 7.0)
    a = make_args(x, H, 1, T, T, o, algo=2)
    assert _lib.workspace_size(a) > _lib.WKV7_NOALLOC_SCRATCH_BYTES
    rc = lib.wkv7_run_noalloc(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    assert rc == _lib.WKV7_ERR_SCRATCH_LIMIT
    torch.cuda.synchronize()
    assert bool((o == 7.0).all())


def test_noalloc_call_captured_in_a_graph(dev, lib):
    """For code under HIP graph capture: after one eager wkv7_run_noalloc call on the device (which looks up the
    scratch array's device address), a captured call replays bit-equal to the eager wkv7_run result, three times with
    eager work between the replays.  The segmented kernel, so the replays also use the scratch's hand-off flags."""
    from rwkv_next_amd import _lib
    H, B, T = 8, 1, 1500
    say("noalloc under graph capture", B, T)
    x = to_dev(operands(B, T, H, seed=9), dev)
    h0 = torch.from_numpy((0.3 * np.random.default_rng(10).standard_normal((B, H, 64, 64))).astype(np.float32)).to(dev)
    # eager reference through wkv7_run with a zeroed workspace
    o_ref = torch.full_like(x[3], float("nan"))
    s_ref = torch.full((B, H, 64, 64), float("nan"), device=dev)
    a = make_args(x, H, B, T, B * T, o_ref, h0, s_ref, None, 4)
    nbytes = _lib.workspace_size(a)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    assert lib.wkv7_run(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)) == 0
    torch.cuda.synchronize()
    o = torch.full_like(x[3], float("nan"))
    ht = torch.full((B, H, 64, 64), float("nan"), device=dev)
    g_args = make_args(x, H, B, T, B * T, o, h0, ht, None, 4)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # the eager call before capture
        assert lib.wkv7_run_noalloc(ctypes.byref(g_args), ctypes.c_void_p(side.cuda_stream)) == 0
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = lib.wkv7_run_noalloc(ctypes.byref(g_args), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    for rep in range(3):
        o.fill_(float("nan"))
        ht.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref) and torch.equal(ht, s_ref), f"replay {rep}"
        # eager work on the device between replays (another noalloc call on the same scratch)
        assert lib.wkv7_run_noalloc(ctypes.byref(g_args), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
        torch.cuda.synchronize()
