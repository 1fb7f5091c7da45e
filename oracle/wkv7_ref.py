"""CPU oracle for the WKV7 recurrence -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, as the checker (or as
the timed CPU baseline).  The product path (rwkv_next_amd) never imports it and has no CPU fallback.

Two restatements of the reference recurrence (rwkv_next/kernels/wkv7.py:38-79; tools/test_wkv7.py:13-23):
  * wkv7_ref(...)        -- the C++ loop in wkv7_oracle.cpp through ctypes, fp64 or fp32, OpenMP over pairs;
  * wkv7_ref_numpy(...)  -- a vectorised numpy fp64 loop over tokens (small cases; an independent transcription
                            used to cross-check the C++ one).
and the reference's error metrics (tools/test_wkv7.py:37-38) plus the max-relative metric of the build's
tolerances.

Array conventions: operands r, w, k, v, a, b are float32 arrays [B, T, H, K] (dense) or [1, sumT, H, K] (varlen,
with cu_seqlens), holding bf16-rounded values; w is RAW (decay = exp(-exp(w))).  States are [N, H, K, K] (k rows,
v columns), or a pool [S, H, K, K] addressed through `state_idx`.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libwkv7_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile wkv7_oracle.cpp into libwkv7_oracle.so (make, in this directory)."""
    if force or not os.path.exists(_LIB_PATH) or (
            os.path.getmtime(_LIB_PATH) < os.path.getmtime(os.path.join(_HERE, "wkv7_oracle.cpp"))):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        vp = ctypes.c_void_p
        for name in ("wkv7_oracle_f64", "wkv7_oracle_f32"):
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [vp] * 13 + [ctypes.c_int] * 5
        lib.wkv7_oracle_max_threads.restype = ctypes.c_int
        _lib = lib
    return _lib


def max_threads() -> int:
    return _load().wkv7_oracle_max_threads()


def _ptr(x):
    return None if x is None else ctypes.c_void_p(x.ctypes.data)


def _f32(x):
    return None if x is None else np.ascontiguousarray(x, dtype=np.float32)


def wkv7_ref(r, w, k, v, a, b, h0=None, *, cu_seqlens=None, n_keep=None, state_idx=None, store_o=True,
             snapshots=False, precision="f64", threads=None, num_slots=None):
    """Run the recurrence on the CPU.

    Returns (o, states, snap):
      o       [B, T, H, K] (same leading shape as the operands) in the oracle's precision, or None;
      states  [N, H, K, K] final state per sequence, or -- when `state_idx` is given -- the whole updated pool
              [S, H, K, K] (untouched slots keep h0's values; h0 is then required and is the pool);
      snap    [N, T, H, K, K] state after every token (None unless snapshots=True; rows past a sequence's end are
              left as NaN).
    """
    r, w, k, v, a, b = (_f32(x) for x in (r, w, k, v, a, b))
    B, T, H, K = r.shape
    if cu_seqlens is not None:
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        N = cu.size - 1
        assert B == 1, "cu_seqlens requires B == 1 (rwkv_next/kernels/wkv7.py:128)"
        Tn = int(np.max(np.diff(cu))) if N else 0
    else:
        cu, N, Tn = None, B, T
    real = np.float64 if precision == "f64" else np.float32
    fn = _load().wkv7_oracle_f64 if precision == "f64" else _load().wkv7_oracle_f32
    h0c = _f32(h0)
    sidx = None if state_idx is None else np.ascontiguousarray(state_idx, dtype=np.int64)
    if sidx is not None:
        assert h0c is not None, "pool mode needs the pool as h0"
        states = h0c.astype(real)  # the pool, updated in place below
    else:
        states = np.zeros((N, H, K, K), dtype=real)
    o = np.zeros((B, T, H, K), dtype=real) if store_o else None
    nk = None if n_keep is None else np.ascontiguousarray(n_keep, dtype=np.int64)
    snap = np.full((N, Tn, H, K, K), np.nan, dtype=real) if snapshots else None
    nthreads = threads if threads is not None else max_threads()
    rc = fn(_ptr(r), _ptr(w), _ptr(k), _ptr(v), _ptr(a), _ptr(b), _ptr(o), _ptr(h0c), _ptr(sidx), _ptr(states),
            _ptr(cu), _ptr(nk), _ptr(snap), N, Tn, H, K, nthreads)
    if rc != 0:
        raise ValueError(f"oracle rejected the arguments (rc={rc})")
    return o, states, snap


def wkv7_ref_numpy(r, w, k, v, a, b, h0=None):
    """Independent vectorised fp64 transcription of tools/test_wkv7.py:13-23 (dense shapes only).
    inputs [B, T, H, K]; h0 [B, H, K, K] or None -> (o [B, T, H, K], S [B, H, K, K])."""
    r, w, k, v, a, b = (np.asarray(x, dtype=np.float64) for x in (r, w, k, v, a, b))
    B, T, H, K = r.shape
    S = np.zeros((B, H, K, K)) if h0 is None else np.array(h0, dtype=np.float64)
    o = np.empty((B, T, H, K))
    for t in range(T):
        d = np.exp(-np.exp(w[:, t]))                                            # [B, H, K]
        sa = np.einsum("bhk,bhkv->bhv", a[:, t], S)                              # a^T S (old S)
        S = d[..., None] * S + b[:, t][..., None] * sa[:, :, None, :] + k[:, t][..., None] * v[:, t][:, :, None, :]
        o[:, t] = np.einsum("bhkv,bhk->bhv", S, r[:, t])                         # S^T r (updated S)
    return o, S


def rel_fro(x, y) -> float:
    """Normwise relative error ||x - y||_F / ||y||_F (tools/test_wkv7.py:37-38)."""
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    return float(np.linalg.norm((x - y).ravel()) / max(np.linalg.norm(y.ravel()), 1e-12))


def rel_max(x, y) -> float:
    """Max-relative error max|x - y| / max|y| (the build's tolerance metric)."""
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    return float(np.max(np.abs(x - y)) / max(np.max(np.abs(y)), 1e-30))
