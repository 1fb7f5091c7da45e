#!/usr/bin/env python3
"""Writes the golden fixtures in this directory: seeded operands (bf16 bit patterns) and the fp64 oracle's outputs.

The reference holds no golden vectors for the WKV7 path (its test draws fresh inputs on a CUDA generator,
tools/test_wkv7.py:26-34), so the fixtures come from the build's own fp64 restatement (oracle/), whose semantics
tests/test_oracle.py pins against closed forms and invariants.  Cases follow the reference's test layout:
dense with h0, varlen with per-sequence h0 (including an empty row), replay with n_keep, and a multi-chunk row
(130 tokens: chunks of 64, 64 and 2) for the chunked kernels.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.join(REPO, "rwkv-infer-next_amd"))

import oracle  # noqa: E402
import rwkv_next_amd.synth as synth  # noqa: E402

CASES = {
    "dense": dict(B=2, T=24, H=1, seed=501, s0=True),
    "varlen": dict(lens=[3, 0, 17, 1, 40], H=1, seed=502, s0=True),
    "replay": dict(B=3, T=4, H=1, seed=503, s0=True, n_keep=[1, 4, 2]),
    "chunks": dict(B=1, T=130, H=1, seed=504, s0=True),
}


def make(name, spec):
    H = spec["H"]
    if "lens" in spec:
        T = int(sum(spec["lens"]))
        ops = synth.operands_np((1, T, H, 64), spec["seed"])
        cu = np.concatenate([[0], np.cumsum(spec["lens"])]).astype(np.int32)
        N = len(spec["lens"])
    else:
        ops = synth.operands_np((spec["B"], spec["T"], H, 64), spec["seed"])
        cu, N = None, spec["B"]
    s0 = synth.state_np((N, H, 64, 64), spec["seed"] + 1, std=0.3) if spec.get("s0") else None
    nk = np.array(spec["n_keep"], np.int64) if "n_keep" in spec else None
    ins = [ops[n] for n in synth.OPERAND_NAMES]
    o, S, _ = oracle.wkv7_ref(*ins, s0, cu_seqlens=cu, n_keep=nk, store_o=nk is None)
    out = {f"in_{n}": synth.bf16_bits(ops[n]) for n in synth.OPERAND_NAMES}
    out["seed"] = np.int64(spec["seed"])
    out["H"] = np.int64(H)
    if s0 is not None:
        out["s0"] = s0
    if cu is not None:
        out["cu_seqlens"] = cu
    if nk is not None:
        out["n_keep"] = nk
    # float32 outputs: their rounding (~6e-8 relative) is far below every tolerance they are checked at
    if o is not None:
        out["o"] = o.astype(np.float32)
    out["state"] = S.astype(np.float32)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)
    return out


def load(name):
    """dict of arrays; operands come back as float32 (from their bf16 bits)."""
    z = dict(np.load(os.path.join(HERE, f"{name}.npz")))
    for n in synth.OPERAND_NAMES:
        z[n] = (z.pop(f"in_{n}").astype(np.uint32) << 16).view(np.float32)
    return z


if __name__ == "__main__":
    oracle.build()
    for name, spec in CASES.items():
        make(name, spec)
        print("wrote", name)
