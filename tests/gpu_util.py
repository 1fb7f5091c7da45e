"""Helpers shared by the GPU parity tests: seeded operands on the device, and the oracle on the same values."""
import sys

import numpy as np

import rwkv_next_amd.synth as synth

# Tolerances (the parity bar: y <= 2e-2, final state <= 1e-4, both max|x - y| / max|y| against the fp64 recurrence on
# the same bf16-rounded inputs).
Y_TOL = 2e-2
S_TOL = 1e-4


def say(*a):
    """Names the case before a GPU step, flushed, so a failing run's log shows what was running."""
    print("[gpu-test]", *a, flush=True)
    sys.stdout.flush()


def operands(B, T, H, seed, K=64):
    """numpy float32 [B, T, H, K] dict (bf16-representable values)."""
    return synth.operands_np((B, T, H, K), seed)


def to_dev(ops, dev, flat=True):
    """numpy operands -> list of bf16 device tensors (B, T, H*K) in r, w, k, v, a, b order (exact conversion)."""
    import torch
    out = []
    for n in synth.OPERAND_NAMES:
        x = torch.from_numpy(np.ascontiguousarray(ops[n])).to(dev).to(torch.bfloat16)
        out.append(x.reshape(x.shape[0], x.shape[1], -1) if flat else x)
    return out


def np_list(ops):
    return [ops[n] for n in synth.OPERAND_NAMES]


def as_np(t):
    import torch
    return t.detach().to(torch.float32).cpu().numpy()
