"""rwkv_next_amd -- MI355X-native (gfx950) WKV7 recurrence for RWKV-Infer-Next.

A drop-in for the reference's WKV7 hot path (rwkv_next/kernels/wkv7.py): the same Python-facing calls
(`wkv7`, `wkv7_replay`, the functional torch op) plus an in-place slot-pool entry (`wkv7_pool_`) with per-token
state snapshots, all backed by hand-written HIP kernels in librwkv7_hip.so (C ABI: include/wkv7.h).
"""
from . import _lib  # noqa: F401

__version__ = "0.1.0"
