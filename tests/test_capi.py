"""The C ABI (include/wkv7.h) without a GPU: the library loads, exports every function the header declares, its
struct layout matches the ctypes binding, and invalid arguments are rejected on the host before any launch.
No compute call is made here (wkv7_run only reaches a launch after validation succeeds)."""
import ctypes
import os
import re

import pytest

from conftest import REPO

from rwkv_next_amd import _lib

HEADER = os.path.join(REPO, "include", "wkv7.h")
NOALLOC_HEADER = os.path.join(REPO, "include", "wkv7_noalloc.h")


def declared_functions(header=HEADER):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^[A-Za-z_][\w \*]*?\b(wkv7_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_function():
    lib = _lib.load()
    names = declared_functions()
    assert set(names) == set(_lib.EXPORTED), names
    for n in names:
        assert hasattr(lib, n), n


def dynamic_symbols(path):
    """Names the shared object defines in its dynamic symbol table (nm -D --defined-only)."""
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_noalloc_library_is_separate():
    """wkv7_run_noalloc and its static scratch array live in librwkv7_noalloc.so, which links librwkv7_hip.so: the
    main library neither defines the entry nor carries the array, so loading it alone holds no scratch."""
    names = declared_functions(NOALLOC_HEADER)
    assert set(names) == set(_lib.NOALLOC_EXPORTED), names
    main_syms, na_syms = dynamic_symbols(_lib.LIB_PATH), dynamic_symbols(_lib.NOALLOC_LIB_PATH)
    assert "wkv7_run_noalloc" not in main_syms
    assert set(_lib.NOALLOC_EXPORTED) <= na_syms
    assert "wkv7_run" not in na_syms  # resolved from librwkv7_hip.so at load time
    lib = _lib.load_noalloc()
    for n in names:
        assert hasattr(lib, n), n
    # the array's host-side shadow symbol exists in the no-alloc library only
    import subprocess
    syms = lambda p: subprocess.run(["nm", p], capture_output=True, text=True, check=True).stdout
    assert "7scratchE" in syms(_lib.NOALLOC_LIB_PATH) and "7scratchE" not in syms(_lib.LIB_PATH)


def test_abi_version_and_struct_layout():
    lib = _lib.load()
    assert lib.wkv7_abi_version() == _lib.WKV7_ABI_VERSION
    assert lib.wkv7_args_size() == ctypes.sizeof(_lib.Wkv7Args)


def base_args(**kw):
    a = _lib.Wkv7Args()
    fake = 0x10000  # 64 KiB-aligned non-null "device" address: never dereferenced by the host-side checks below
    for n in ("r", "w", "k", "v", "a", "b"):
        setattr(a, n, fake)
    a.in_tok_stride = 2 * 64
    a.o, a.o_tok_stride = fake, 2 * 64
    a.num_seqs, a.T, a.total_tokens, a.H, a.head_size = 3, 5, 15, 2, 64
    a.algo, a.rec_max_len = _lib.ALGO_AUTO, -1
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("field,value,code", [
    ("head_size", 257, _lib.WKV7_ERR_SHAPE),            # 1..256: 64 and the generic kernel's other sizes
    ("head_size", 0, _lib.WKV7_ERR_SHAPE),
    ("H", 0, _lib.WKV7_ERR_SHAPE),
    ("num_seqs", -1, _lib.WKV7_ERR_SHAPE),
    ("total_tokens", 14, _lib.WKV7_ERR_SHAPE),        # dense rows need num_seqs * T operand rows
    ("algo", 7, _lib.WKV7_ERR_ARG),
    ("rec_max_len", -2, _lib.WKV7_ERR_ARG),
    ("r", None, _lib.WKV7_ERR_NULL),
    ("w", 0x10002, _lib.WKV7_ERR_ALIGN),
    ("in_tok_stride", 2 * 64 + 4, _lib.WKV7_ERR_ALIGN),
    ("in_tok_stride", 64, _lib.WKV7_ERR_ALIGN),        # smaller than H * 64
    ("o_tok_stride", 2 * 64 + 2, _lib.WKV7_ERR_ALIGN),
    ("h0_idx", 0x10000, _lib.WKV7_ERR_ARG),            # an index without a state array
])
def test_validation_rejects_before_launch(field, value, code):
    a = base_args(**{field: value})
    n = ctypes.c_size_t(0)
    lib = _lib.load()
    assert lib.wkv7_workspace_size(ctypes.byref(a), ctypes.byref(n)) == code
    assert lib.wkv7_run(ctypes.byref(a), None) == code
    assert _lib.strerror(code) not in ("", "unknown error")


@pytest.mark.parametrize("K,kw,code", [
    (32, dict(algo=_lib.ALGO_CHUNKED), _lib.WKV7_ERR_ARG),     # the chunked, chain and segmented forms are K = 64
    (32, dict(algo=_lib.ALGO_SEGMENTED), _lib.WKV7_ERR_ARG),
    (100, dict(), _lib.WKV7_ERR_ALIGN),                        # in_tok_stride 128 < H * K = 200
    (100, dict(in_tok_stride=200, o_tok_stride=199), _lib.WKV7_ERR_ALIGN),
    (24, dict(w=0x10001), _lib.WKV7_ERR_ALIGN),                # bf16 operands need 2-byte alignment
    (24, dict(h0=0x10002, h0_rows=3), _lib.WKV7_ERR_ALIGN),    # fp32 states 4-byte
])
def test_other_head_sizes_validate(K, kw, code):
    """Head sizes other than 64 run the generic token-serial kernel (no workspace) with scalar accesses."""
    a = base_args(head_size=K, **kw)
    n = ctypes.c_size_t(0)
    lib = _lib.load()
    assert lib.wkv7_workspace_size(ctypes.byref(a), ctypes.byref(n)) == code
    assert lib.wkv7_run(ctypes.byref(a), None) == code
    ok = base_args(head_size=24, T=4000, total_tokens=12000)   # long rows: still no workspace at K != 64
    assert lib.wkv7_workspace_size(ctypes.byref(ok), ctypes.byref(n)) == 0 and n.value == 0


def test_snapshots_force_the_token_serial_kernel():
    a = base_args(snapshots=0x10000, T=40, total_tokens=120)
    assert _lib.workspace_size(a) == 0                     # token-serial: no workspace
    a.algo = _lib.ALGO_CHUNKED
    with pytest.raises(_lib.Wkv7Error) as e:
        _lib.workspace_size(a)
    assert e.value.code == _lib.WKV7_ERR_ARG


def test_workspace_sizing_follows_the_dispatch_rule():
    # dense short rows: token-serial, no workspace
    assert _lib.workspace_size(base_args(T=32, total_tokens=96)) == 0
    # dense long rows: chunked; 3 rows x ceil(100/64) chunks x H=2 records of 48 KB
    # (A hi/lo bf16, H^T fp32, Q bf16, O_intra^T bf16: 64 x 64 each)
    n = _lib.workspace_size(base_args(T=100, total_tokens=300))
    assert n >= 3 * 2 * 2 * (2 * 2 + 4 + 2 + 2) * 64 * 64
    # a dense call of at least 8 x CUs 32-token chunk-heads takes the segmented kernel (256 CUs assumed without a
    # GPU): B = 1, T = 4096, H = 64 is 4 segments of the row per head (36 + 31 + 31 + 30 chunks), 256 units with a
    # 32 KB hand-off entry each, a 4 KB Q P record per chunk after the first segment, after the flag region
    seg = _lib.workspace_size(base_args(num_seqs=1, T=4096, total_tokens=4096, H=64, in_tok_stride=64 * 64,
                                           o_tok_stride=64 * 64))
    assert seg == _lib.WKV7_FLAG_REGION_BYTES + 256 * 2 * 64 * 64 * 4 + (128 - 36) * 64 * 4096
    # the segmented kernel addresses a chunk's operand and output rows with 32-bit offsets: beyond 2^24 elements per
    # token AUTO takes the chunked path (another workspace) and SEGMENTED is refused
    dense = dict(num_seqs=1, T=4096, total_tokens=4096, H=64, in_tok_stride=64 * 64, o_tok_stride=64 * 64)
    for field in ("in_tok_stride", "o_tok_stride"):
        wide = dict(dense, **{field: (1 << 24) + 8})
        assert _lib.workspace_size(base_args(**wide)) != seg
        assert _lib.workspace_size(base_args(**dict(wide, **{field: 1 << 24}))) == seg
        with pytest.raises(_lib.Wkv7Error) as e:
            _lib.workspace_size(base_args(algo=_lib.ALGO_SEGMENTED, **wide))
        assert e.value.code == _lib.WKV7_ERR_SHAPE
    # ragged: short rows token-serial, long rows segmented (bounded by total_tokens); the flag region leads
    r = _lib.workspace_size(base_args(cu_seqlens=0x10000, T=0, total_tokens=1000))
    assert r > _lib.WKV7_FLAG_REGION_BYTES
    # a missing workspace is refused before launch
    a = base_args(T=100, total_tokens=300)
    assert _lib.load().wkv7_run(ctypes.byref(a), None) == _lib.WKV7_ERR_WORKSPACE


def test_zero_sequences_is_a_no_op():
    a = base_args(num_seqs=0, total_tokens=0)
    assert _lib.load().wkv7_run(ctypes.byref(a), None) == _lib.WKV7_OK


def test_pool_entry_points_validate_before_launch():
    """The slot-pool entry points reject bad sizes, NULL pointers and misalignment on the host; empty work is a
    no-op (nothing is launched, so no GPU is needed)."""
    lib = _lib.load()
    fake = 0x10000
    E = _lib
    # reset: pool, layers, rows, H, idx, n, stream
    assert lib.wkv7_pool_reset(fake, 2, 4, 0, fake, 1, None) == E.WKV7_ERR_SHAPE
    assert lib.wkv7_pool_reset(fake, 2, 4, 2, fake, -1, None) == E.WKV7_ERR_SHAPE
    assert lib.wkv7_pool_reset(None, 2, 4, 2, fake, 1, None) == E.WKV7_ERR_NULL
    assert lib.wkv7_pool_reset(fake, 2, 4, 2, None, 1, None) == E.WKV7_ERR_NULL
    assert lib.wkv7_pool_reset(fake + 4, 2, 4, 2, fake, 1, None) == E.WKV7_ERR_ALIGN
    assert lib.wkv7_pool_reset(None, 2, 4, 2, None, 0, None) == E.WKV7_OK
    # move: pool, layers, rows, H, src, dst, n, stream
    assert lib.wkv7_pool_move(fake, 1, 4, 2, fake, None, 1, None) == E.WKV7_ERR_NULL
    assert lib.wkv7_pool_move(fake, 1, 4, 2, fake, fake, E.MAX_MOVES + 1, None) == E.WKV7_ERR_SHAPE
    assert lib.wkv7_pool_move(fake + 8, 1, 4, 2, fake, fake, 1, None) == E.WKV7_ERR_ALIGN
    assert lib.wkv7_pool_move(None, 1, 4, 2, None, None, 0, None) == E.WKV7_OK
    # restore: pool, rows, H, slots, snapshots, T, n_accepted, num_seqs, stream
    assert lib.wkv7_snapshot_restore(fake, 4, 2, fake, fake, 0, fake, 1, None) == E.WKV7_ERR_SHAPE
    assert lib.wkv7_snapshot_restore(fake, 4, 2, fake, None, 5, fake, 1, None) == E.WKV7_ERR_NULL
    assert lib.wkv7_snapshot_restore(fake, 4, 2, fake, fake + 4, 5, fake, 1, None) == E.WKV7_ERR_ALIGN
    assert lib.wkv7_snapshot_restore(None, 4, 2, None, None, 5, None, 0, None) == E.WKV7_OK


def test_timemix_entry_points_validate_before_launch():
    """Prologue / epilogue reject bad sizes and NULL or misaligned pointers on the host; zero tokens is a no-op."""
    lib = _lib.load()
    fake = 0x10000
    p = _lib.PrologueArgs()
    for n in ("k", "v", "o_v", "o_w", "o_a", "b_w", "b_a", "b_v", "kk_mul", "ka_mul", "w_out", "k_out", "v_out",
              "a_out", "b_out"):
        setattr(p, n, fake)
    p.tokens, p.in_stride, p.out_stride, p.H, p.head_size = 3, 128, 128, 2, 64
    for field, value, code in [("head_size", 32, _lib.WKV7_ERR_SHAPE), ("in_stride", 64, _lib.WKV7_ERR_SHAPE),
                               ("H", 1 << 17, _lib.WKV7_ERR_SHAPE), ("kk_mul", None, _lib.WKV7_ERR_NULL),
                               ("w_out", fake + 8, _lib.WKV7_ERR_ALIGN), ("out_stride", 130, _lib.WKV7_ERR_ALIGN)]:
        q = _lib.PrologueArgs.from_buffer_copy(p)
        setattr(q, field, value)
        assert lib.wkv7_timemix_prologue(ctypes.byref(q), None) == code, field
    q = _lib.PrologueArgs.from_buffer_copy(p)
    q.v_first, q.o_v = fake, None                       # mixing towards v_first needs o_v
    assert lib.wkv7_timemix_prologue(ctypes.byref(q), None) == _lib.WKV7_ERR_NULL
    q = _lib.PrologueArgs.from_buffer_copy(p)
    q.tokens = 0
    assert lib.wkv7_timemix_prologue(ctypes.byref(q), None) == _lib.WKV7_OK
    e = _lib.EpilogueArgs()
    for n in ("y", "r", "k", "v", "g", "lnx_w", "lnx_b", "r_k", "out"):
        setattr(e, n, fake)
    e.tokens, e.in_stride, e.out_stride, e.eps, e.H, e.head_size = 3, 128, 128, 6.4e-4, 2, 64
    for field, value, code in [("eps", 0.0, _lib.WKV7_ERR_ARG), ("H", 0, _lib.WKV7_ERR_SHAPE),
                               ("r_k", None, _lib.WKV7_ERR_NULL), ("g", fake + 2, _lib.WKV7_ERR_ALIGN),
                               ("in_stride", 132, _lib.WKV7_ERR_ALIGN)]:
        q = _lib.EpilogueArgs.from_buffer_copy(e)
        setattr(q, field, value)
        assert lib.wkv7_timemix_epilogue(ctypes.byref(q), None) == code, field
    assert ctypes.sizeof(_lib.PrologueArgs) == 16 * 8 + 3 * 8 + 2 * 4
    assert ctypes.sizeof(_lib.EpilogueArgs) == 9 * 8 + 3 * 8 + 3 * 4 + 4  # trailing padding to 8 bytes
