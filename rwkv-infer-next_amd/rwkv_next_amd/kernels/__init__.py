"""HIP kernels of rwkv_next_amd (mirrors the reference package rwkv_next.kernels)."""
from .wkv7 import (check_distinct_slots, restore_snapshots_, wkv7, wkv7_fwd, wkv7_pool_,  # noqa: F401
                   wkv7_replay)
