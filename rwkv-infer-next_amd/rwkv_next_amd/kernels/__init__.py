"""HIP kernels of rwkv_next_amd (mirrors the reference package rwkv_next.kernels)."""
from .int6_gemm import (dequantize_int6, int6_matmul, int6_matmul_op, plan_int6,  # noqa: F401
                        quantize_int6)
from .timemix import timemix_epilogue, timemix_prologue  # noqa: F401
from .wkv7 import (StatePool, check_distinct_slots, model_wkv7, restore_snapshots_, wkv7, wkv7_fwd,  # noqa: F401
                   wkv7_pool_, wkv7_replay)
