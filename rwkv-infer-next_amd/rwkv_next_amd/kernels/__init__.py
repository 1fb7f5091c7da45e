"""HIP kernels of rwkv_next_amd (mirrors the reference package rwkv_next.kernels)."""
from .int6_gemm import (Int6Packed, dequantize_int6, dequantize_int6_packed, int6_matmul,  # noqa: F401
                        int6_matmul_op, int6_matmul_packed_op, plan_int6, prepack_int6, quantize_int6)
from .timemix import timemix_epilogue, timemix_prologue  # noqa: F401
from .wkv7 import (StatePool, check_distinct_slots, check_status, model_wkv7, new_status,  # noqa: F401
                   restore_snapshots_, wkv7, wkv7_fwd, wkv7_pool_, wkv7_pool_op, wkv7_replay, wkv7_replay_)
