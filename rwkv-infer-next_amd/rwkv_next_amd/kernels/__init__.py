"""HIP kernels of rwkv_next_amd (mirrors the reference package rwkv_next.kernels)."""
from .timemix import timemix_epilogue, timemix_prologue  # noqa: F401
from .wkv7 import (StatePool, check_distinct_slots, model_wkv7, restore_snapshots_, wkv7, wkv7_fwd,  # noqa: F401
                   wkv7_pool_, wkv7_replay)
