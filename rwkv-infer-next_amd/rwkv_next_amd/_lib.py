"""ctypes binding of librwkv7_hip.so (the C ABI declared in include/wkv7.h and include/w6a16.h) and of
librwkv7_noalloc.so (include/wkv7_noalloc.h, loaded only on request by load_noalloc).

The library must have been built (rwkv_next_amd._build / __graft_entry__.build()).  There is no fallback: if the
shared object is missing or does not match this binding, importing the kernels raises.
"""
from __future__ import annotations

import ctypes
import os

from ._build import LIB_PATH, NOALLOC_LIB_PATH

WKV7_ABI_VERSION = 2
WKV7_OK = 0
WKV7_ERR_NULL = -1
WKV7_ERR_SHAPE = -2
WKV7_ERR_ALIGN = -3
WKV7_ERR_WORKSPACE = -4
WKV7_ERR_ARG = -5
WKV7_ERR_SCRATCH_LIMIT = -6
WKV7_NOALLOC_SCRATCH_BYTES = 128 << 20  # include/wkv7_noalloc.h
NOALLOC_EXPORTED = ("wkv7_run_noalloc",)

WKV7_STATUS_H0_SLOT = 1
WKV7_STATUS_HT_SLOT = 2
WKV7_STATUS_SEQLENS = 4
WKV7_STATUS_NKEEP = 8
WKV7_STATUS_DECAY = 16
WKV7_STATUS_SLOT_CLASH = 32
WKV7_STATUS_SEGMENT_WAIT = 64
WKV7_STATUS_CLASH_MAX_SEQS = 1024
WKV7_CHUNK_W_MAX = 1.0

ALGO_AUTO = 0
ALGO_RECURRENT = 1
ALGO_CHUNKED = 2
ALGO_CHAIN = 3
ALGO_SEGMENTED = 4
WKV7_FLAG_REGION_BYTES = 256 << 10  # leading workspace region of hand-off flags (zero between calls)

EXPORTED = ("wkv7_run", "wkv7_workspace_size", "wkv7_strerror", "wkv7_abi_version", "wkv7_args_size",
            "wkv7_args_layout",
            "wkv7_pool_reset", "wkv7_pool_move", "wkv7_snapshot_restore", "wkv7_timemix_prologue",
            "wkv7_timemix_epilogue")
W6A16_EXPORTED = ("w6a16_args_size", "w6a16_workspace_size", "w6a16_plan_split", "w6a16_plan_split_packed",
                  "w6a16_matmul",
                  "w6a16_dequantize", "w6a16_packed_size", "w6a16_pack", "w6a16_dequantize_packed")
W6A16_FORMAT_PLANES = 0
W6A16_FORMAT_PACKED = 1
W6A16_OUT_BF16 = 0
W6A16_OUT_F16 = 1
W6A16_OUT_F32 = 2
W6A16_IN_BF16 = 0
W6A16_IN_F16 = 1
MAX_MOVES = 1024

_vp = ctypes.c_void_p


class Wkv7Args(ctypes.Structure):
    """Mirror of `wkv7_args` (include/wkv7.h); field order and types must match the header exactly."""
    _fields_ = [
        ("r", _vp), ("w", _vp), ("k", _vp), ("v", _vp), ("a", _vp), ("b", _vp),
        ("in_tok_stride", ctypes.c_int64),
        ("o", _vp),
        ("o_tok_stride", ctypes.c_int64),
        ("h0", _vp),
        ("h0_idx", _vp),
        ("h0_rows", ctypes.c_int64),
        ("ht", _vp),
        ("ht_idx", _vp),
        ("ht_rows", ctypes.c_int64),
        ("fresh", _vp),
        ("cu_seqlens", _vp),
        ("n_keep", _vp),
        ("snapshots", _vp),
        ("workspace", _vp),
        ("workspace_bytes", ctypes.c_size_t),
        ("num_seqs", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("total_tokens", ctypes.c_int64),
        ("H", ctypes.c_int32),
        ("head_size", ctypes.c_int32),
        ("algo", ctypes.c_int32),
        ("rec_max_len", ctypes.c_int32),
        ("status", _vp),
    ]


class PrologueArgs(ctypes.Structure):
    """Mirror of `wkv7_prologue_args` (include/wkv7.h)."""
    _fields_ = [(n, _vp) for n in ("k", "v", "o_v", "o_w", "o_a", "v_first", "b_w", "b_a", "b_v", "kk_mul", "ka_mul",
                                   "w_out", "k_out", "v_out", "a_out", "b_out")] + [
        ("tokens", ctypes.c_int64), ("in_stride", ctypes.c_int64), ("out_stride", ctypes.c_int64),
        ("H", ctypes.c_int32), ("head_size", ctypes.c_int32)]


class EpilogueArgs(ctypes.Structure):
    """Mirror of `wkv7_epilogue_args` (include/wkv7.h)."""
    _fields_ = [(n, _vp) for n in ("y", "r", "k", "v", "g", "lnx_w", "lnx_b", "r_k", "out")] + [
        ("tokens", ctypes.c_int64), ("in_stride", ctypes.c_int64), ("out_stride", ctypes.c_int64),
        ("eps", ctypes.c_float), ("H", ctypes.c_int32), ("head_size", ctypes.c_int32)]


class W6a16Args(ctypes.Structure):
    """Mirror of `w6a16_args` (include/w6a16.h)."""
    _fields_ = [
        ("a", _vp), ("a_batch_stride", ctypes.c_int64), ("a_row_stride", ctypes.c_int64),
        ("lo", _vp), ("hi", _vp), ("lo_batch_stride", ctypes.c_int64), ("hi_batch_stride", ctypes.c_int64),
        ("scales", _vp), ("scales_batch_stride", ctypes.c_int64),
        ("out", _vp), ("out_batch_stride", ctypes.c_int64), ("out_row_stride", ctypes.c_int64),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("B", ctypes.c_int32), ("M", ctypes.c_int32), ("N", ctypes.c_int32), ("K", ctypes.c_int32),
        ("group_k", ctypes.c_int32), ("split_k", ctypes.c_int32), ("out_dtype", ctypes.c_int32),
        ("format", ctypes.c_int32), ("a_dtype", ctypes.c_int32),
    ]


class Wkv7Error(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"wkv7 error {code}: {msg}")
        self.code = code


_lib = None
_noalloc = None


def load(path: str = LIB_PATH):
    """Load the library (after torch, so that it binds to the HIP runtime torch loaded) and check its ABI."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with `python -m rwkv_next_amd._build` "
                          "(or __graft_entry__.build()); there is no fallback implementation")
    try:
        import torch  # noqa: F401  -- load torch's libamdhip64 first
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    lib.wkv7_run.restype = ctypes.c_int
    lib.wkv7_run.argtypes = [ctypes.POINTER(Wkv7Args), _vp]
    lib.wkv7_workspace_size.restype = ctypes.c_int
    lib.wkv7_workspace_size.argtypes = [ctypes.POINTER(Wkv7Args), ctypes.POINTER(ctypes.c_size_t)]
    lib.wkv7_strerror.restype = ctypes.c_char_p
    lib.wkv7_strerror.argtypes = [ctypes.c_int]
    lib.wkv7_abi_version.restype = ctypes.c_int
    lib.wkv7_args_size.restype = ctypes.c_size_t
    lib.wkv7_args_layout.restype = ctypes.c_int
    lib.wkv7_args_layout.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.c_int]
    i32, i64 = ctypes.c_int32, ctypes.c_int64
    lib.wkv7_pool_reset.restype = ctypes.c_int
    lib.wkv7_pool_reset.argtypes = [_vp, i32, i64, i32, _vp, i32, _vp]
    lib.wkv7_pool_move.restype = ctypes.c_int
    lib.wkv7_pool_move.argtypes = [_vp, i32, i64, i32, _vp, _vp, i32, _vp]
    lib.wkv7_snapshot_restore.restype = ctypes.c_int
    lib.wkv7_snapshot_restore.argtypes = [_vp, i64, i32, _vp, _vp, i32, _vp, i32, _vp]
    lib.wkv7_timemix_prologue.restype = ctypes.c_int
    lib.wkv7_timemix_prologue.argtypes = [ctypes.POINTER(PrologueArgs), _vp]
    lib.wkv7_timemix_epilogue.restype = ctypes.c_int
    lib.wkv7_timemix_epilogue.argtypes = [ctypes.POINTER(EpilogueArgs), _vp]
    lib.w6a16_args_size.restype = ctypes.c_size_t
    lib.w6a16_workspace_size.restype = ctypes.c_int
    lib.w6a16_workspace_size.argtypes = [ctypes.POINTER(W6a16Args), ctypes.POINTER(ctypes.c_size_t)]
    lib.w6a16_plan_split.restype = ctypes.c_int
    lib.w6a16_plan_split.argtypes = [i32, i32, i32, i32]
    lib.w6a16_plan_split_packed.restype = ctypes.c_int
    lib.w6a16_plan_split_packed.argtypes = [i32, i32, i32, i32]
    lib.w6a16_matmul.restype = ctypes.c_int
    lib.w6a16_matmul.argtypes = [ctypes.POINTER(W6a16Args), _vp]
    lib.w6a16_dequantize.restype = ctypes.c_int
    lib.w6a16_dequantize.argtypes = [_vp, _vp, _vp, _vp, i32, i32, i32, i32, i64, i64, i64, i64, i32, _vp]
    lib.w6a16_packed_size.restype = ctypes.c_int
    lib.w6a16_packed_size.argtypes = [i32, i32, i32, i32, ctypes.POINTER(ctypes.c_size_t),
                                      ctypes.POINTER(ctypes.c_size_t)]
    lib.w6a16_pack.restype = ctypes.c_int
    lib.w6a16_pack.argtypes = [_vp, _vp, _vp, i32, i32, i32, i32, i64, i64, i64, _vp, _vp, _vp]
    lib.w6a16_dequantize_packed.restype = ctypes.c_int
    lib.w6a16_dequantize_packed.argtypes = [_vp, _vp, _vp, i32, i32, i32, i32, i64, i32, _vp]
    if lib.wkv7_abi_version() != WKV7_ABI_VERSION:
        raise ImportError(f"{path}: ABI version {lib.wkv7_abi_version()} != {WKV7_ABI_VERSION}")
    if lib.wkv7_args_size() != ctypes.sizeof(Wkv7Args):
        raise ImportError(f"{path}: sizeof(wkv7_args) {lib.wkv7_args_size()} != binding {ctypes.sizeof(Wkv7Args)}")
    if args_layout(lib) != binding_layout():
        raise ImportError(f"{path}: wkv7_args field offsets {args_layout(lib)} != binding {binding_layout()}")
    if lib.w6a16_args_size() != ctypes.sizeof(W6a16Args):
        raise ImportError(f"{path}: sizeof(w6a16_args) {lib.w6a16_args_size()} != binding {ctypes.sizeof(W6a16Args)}")
    _lib = lib
    return lib


def load_noalloc(path: str = NOALLOC_LIB_PATH):
    """Load librwkv7_noalloc.so (wkv7_run_noalloc, include/wkv7_noalloc.h), after librwkv7_hip.so, which it links
    and shares with this process.  Loading it makes every GPU the process uses hold its static scratch array."""
    global _noalloc
    if _noalloc is not None:
        return _noalloc
    load()
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with `python -m rwkv_next_amd._build`")
    lib = ctypes.CDLL(path)
    lib.wkv7_run_noalloc.restype = ctypes.c_int
    lib.wkv7_run_noalloc.argtypes = [ctypes.POINTER(Wkv7Args), _vp]
    _noalloc = lib
    return lib


def args_layout(lib=None):
    """Field offsets of wkv7_args as compiled into the library (declaration order)."""
    lib = lib or load()
    n = lib.wkv7_args_layout(None, 0)
    buf = (ctypes.c_size_t * n)()
    lib.wkv7_args_layout(buf, n)
    return list(buf)


def binding_layout():
    """Field offsets of the ctypes mirror, in the same order."""
    return [getattr(Wkv7Args, name).offset for name, _ in Wkv7Args._fields_]


def strerror(code: int) -> str:
    return load().wkv7_strerror(code).decode()


def workspace_size(args: Wkv7Args) -> int:
    n = ctypes.c_size_t(0)
    rc = load().wkv7_workspace_size(ctypes.byref(args), ctypes.byref(n))
    if rc != WKV7_OK:
        raise Wkv7Error(rc, strerror(rc))
    return int(n.value)


def run(args: Wkv7Args, stream: int) -> None:
    rc = load().wkv7_run(ctypes.byref(args), _vp(stream))
    if rc != WKV7_OK:
        raise Wkv7Error(rc, strerror(rc))


def check(rc: int) -> None:
    """Raise Wkv7Error for a non-zero return code of the library."""
    if rc != WKV7_OK:
        raise Wkv7Error(rc, strerror(rc))
