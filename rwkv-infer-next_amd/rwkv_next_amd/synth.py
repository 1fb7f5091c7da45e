"""Seeded synthetic WKV7 operands, the measurement inputs of the build.

Distributions (the reference's operand producer, rwkv_next/model.py:142-152, with the spreads the benchmark
configurations fix):
  r, k, v ~ N(0, 1)
  w = -softplus(-x) - 0.5 with x ~ N(0, 2^2)       (RAW log-log decay; the kernel applies exp(-exp(w)),
                                                    so the decay lies in (0.545, 1))
  kappa = L2-normalised N(0, 1) over the head's 64 channels
  a = -kappa,  b = kappa * sigmoid(N(0, 1))
Everything is rounded to bf16 (round-to-nearest-even) because the kernel consumes bf16 operands.

`operands_np` is the reproducible generator (numpy PCG64): parity tests feed the same values to the GPU kernel
and to the CPU oracle.  `operands_torch` draws the same distributions on a torch device; the benchmark uses it
for full-size inputs, which are generated on the GPU.
"""
from __future__ import annotations

import numpy as np

OPERAND_NAMES = ("r", "w", "k", "v", "a", "b")


def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even); returns float32 holding bf16 values."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = ((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return rounded.view(np.float32)


def bf16_bits(x) -> np.ndarray:
    """bf16 bit patterns (uint16) of float32 values that are already bf16-representable."""
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _softplus(x):
    return np.logaddexp(0.0, x)


def operands_np(shape, seed: int):
    """dict name -> float32 array of `shape` (..., K): bf16-rounded r, w (raw), k, v, a, b."""
    rng = np.random.Generator(np.random.PCG64(seed))
    K = shape[-1]
    n = lambda: rng.standard_normal(shape, dtype=np.float32)
    r, k, v = n(), n(), n()
    x = 2.0 * n()
    w = -_softplus(-x) - 0.5
    kap = n()
    kap = kap / np.maximum(np.linalg.norm(kap, axis=-1, keepdims=True), 1e-12)
    gate = 1.0 / (1.0 + np.exp(-n()))
    a, b = -kap, kap * gate
    assert K > 0
    return {name: bf16_round(t.astype(np.float32)) for name, t in zip(OPERAND_NAMES, (r, w, k, v, a, b))}


def state_np(shape, seed: int, std: float = 0.1):
    """fp32 state (pool) seeded from N(0, std^2)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return (std * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)


def operands_torch(shape, seed: int, device, dtype=None):
    """Same distributions drawn with torch on `device`; returns dict name -> bf16 tensor of `shape`."""
    import torch
    dtype = dtype or torch.bfloat16
    g = torch.Generator(device=device).manual_seed(seed)
    n = lambda: torch.randn(*shape, device=device, generator=g, dtype=torch.float32)
    r, k, v = n(), n(), n()
    w = -torch.nn.functional.softplus(-2.0 * n()) - 0.5
    kap = torch.nn.functional.normalize(n(), dim=-1)
    a, b = -kap, kap * torch.sigmoid(n())
    return {name: t.to(dtype) for name, t in zip(OPERAND_NAMES, (r, w, k, v, a, b))}
