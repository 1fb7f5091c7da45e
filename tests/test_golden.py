"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the seeded generator reproduces the stored operand bits, and the oracle reproduces the stored outputs
(a regression pin on both).  GPU: the HIP kernels, through every algorithm choice, match the stored outputs
within the parity tolerances (y <= 2e-2, state <= 1e-4, max-relative)."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden  # noqa: E402

import oracle  # noqa: E402
import rwkv_next_amd.synth as synth  # noqa: E402

NAMES = list(make_golden.CASES)


def fixture_inputs(z):
    return [z[n] for n in synth.OPERAND_NAMES]


@pytest.mark.parametrize("name", NAMES)
def test_generator_reproduces_fixture_operands(name):
    z = make_golden.load(name)
    spec = make_golden.CASES[name]
    shape = (1, int(sum(spec["lens"])), spec["H"], 64) if "lens" in spec else (spec["B"], spec["T"], spec["H"], 64)
    ops = synth.operands_np(shape, spec["seed"])
    for n in synth.OPERAND_NAMES:
        assert np.array_equal(synth.bf16_bits(ops[n]), synth.bf16_bits(z[n])), n


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture_outputs(name):
    z = make_golden.load(name)
    o, S, _ = oracle.wkv7_ref(*fixture_inputs(z), z.get("s0"), cu_seqlens=z.get("cu_seqlens"),
                              n_keep=z.get("n_keep"), store_o="o" in z)
    assert oracle.rel_max(S, z["state"]) < 1e-6
    if "o" in z:
        assert oracle.rel_max(o, z["o"]) < 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("algo", [0, 1, 2, 3])
@pytest.mark.parametrize("name", NAMES)
def test_gpu_matches_fixture(name, algo):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from gpu_util import say
    from rwkv_next_amd import kernels
    say("golden", name, algo)
    dev = torch.device("cuda:0")
    z = make_golden.load(name)
    H = int(z["H"])
    x = [torch.from_numpy(a).to(dev).to(torch.bfloat16).reshape(a.shape[0], a.shape[1], -1) for a in fixture_inputs(z)]
    s0 = torch.from_numpy(z["s0"]).to(dev) if "s0" in z else None
    if "n_keep" in z:
        if algo in (2, 3):
            pytest.skip("replay runs on the token-serial kernel")
        kernels.wkv7_replay(*x, s0, torch.from_numpy(z["n_keep"]).to(dev), H, 64)
        torch.cuda.synchronize()
        assert oracle.rel_max(s0.cpu().numpy(), z["state"]) <= 1e-4
        return
    cu = torch.from_numpy(z["cu_seqlens"]).to(dev) if "cu_seqlens" in z else None
    o, S = kernels.wkv7(*x, s0, H, 64, cu_seqlens=cu, algo=algo)
    torch.cuda.synchronize()
    assert oracle.rel_max(S.cpu().numpy(), z["state"]) <= 1e-4
    assert oracle.rel_max(o.float().cpu().numpy().reshape(z["o"].shape), z["o"]) <= 2e-2
