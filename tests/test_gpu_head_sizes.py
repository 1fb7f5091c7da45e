"""Head sizes other than 64 (the reference takes any K, padding it to a power of two with masks,
rwkv_next/kernels/wkv7.py:55-59, 96): the generic token-serial kernels (float4 rows for multiples of 32 with 16-byte
aligned states -- K = 32, 96, 128, 256 here -- scalar rows otherwise) through every entry point -- the functional
wkv7 (dense and varlen), the in-place replay (n_keep), and the slot pool with fresh rows and per-token snapshots --
against the fp64 oracle on the same bf16-rounded inputs.  Tolerances as for K = 64: y max-relative <= 2e-2 (bf16
output), states max-relative <= 1e-4."""
import numpy as np
import pytest

from gpu_util import S_TOL, Y_TOL, as_np, np_list, operands, say, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

SIZES = [1, 8, 24, 32, 48, 100, 128, 256]


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from rwkv_next_amd import _lib
    _lib.load()
    return torch.device("cuda:0")


def _check(got, ref, tol, what):
    from oracle import rel_max
    e = rel_max(as_np(got).reshape(ref.shape), ref)
    assert e <= tol, f"{what} max-rel {e:.3e}"


@pytest.mark.parametrize("K", SIZES)
def test_dense_matches_oracle(dev, K):
    from oracle import wkv7_ref
    from rwkv_next_amd import kernels
    B, T, H = 2, (9 if K > 128 else 33), 3
    say("head size dense", K, B, T, H)
    ops = operands(B, T, H, seed=500 + K, K=K)
    s0 = (0.3 * np.random.default_rng(K).standard_normal((B, H, K, K))).astype(np.float32)
    o_ref, S_ref, _ = wkv7_ref(*np_list(ops), s0)
    for algo in (0, 1):  # AUTO and RECURRENT both run the generic kernel
        o, S = kernels.wkv7(*to_dev(ops, dev), torch.from_numpy(s0).to(dev), H, K, algo=algo)
        torch.cuda.synchronize()
        assert o.shape == (B, T, H * K) and S.shape == (B, H, K, K)
        _check(o, o_ref, Y_TOL, "y")
        _check(S, S_ref, S_TOL, "state")


@pytest.mark.parametrize("K", [16, 96])
def test_varlen_and_no_state(dev, K):
    from oracle import wkv7_ref
    from rwkv_next_amd import kernels
    H, lens = 2, [5, 0, 40, 1, 17]
    say("head size varlen", K, lens)
    total = sum(lens)
    ops = operands(1, total, H, seed=600 + K, K=K)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    o_ref, S_ref, _ = wkv7_ref(*np_list(ops), None, cu_seqlens=cu)
    o, S = kernels.wkv7(*to_dev(ops, dev), None, H, K, cu_seqlens=torch.from_numpy(cu).to(dev))
    torch.cuda.synchronize()
    _check(o, o_ref, Y_TOL, "y")
    _check(S, S_ref, S_TOL, "state")


@pytest.mark.parametrize("K", [32, 128])
def test_replay_in_place(dev, K):
    from oracle import wkv7_ref
    from rwkv_next_amd import kernels
    B, T, H = 3, 6, 2
    say("head size replay", K)
    ops = operands(B, T, H, seed=700 + K, K=K)
    s0 = (0.3 * np.random.default_rng(K + 1).standard_normal((B, H, K, K))).astype(np.float32)
    n_keep = np.array([0, 4, 6], dtype=np.int64)
    _, S_ref, _ = wkv7_ref(*np_list(ops), s0, n_keep=n_keep)
    st = torch.from_numpy(s0).to(dev)
    kernels.wkv7_replay(*to_dev(ops, dev), st, torch.from_numpy(n_keep).to(dev), H, K)
    torch.cuda.synchronize()
    _check(st, S_ref, S_TOL, "state")
    assert torch.equal(st[0].cpu(), torch.from_numpy(s0[0]))  # n_keep = 0 keeps the state bit for bit


@pytest.mark.parametrize("K", [24, 64 + 16, 96])  # 96: the float4 kernel for multiples of 32
def test_pool_with_fresh_rows_and_snapshots(dev, K):
    """Slots in a pool, one row fresh (starts from zeros), snapshots after every token: each snapshot equals the
    oracle's state after that token, and the pool's untouched slots keep their values."""
    from oracle import wkv7_ref
    from rwkv_next_amd import kernels
    N, T, H, S_rows = 3, 5, 2, 6
    say("head size pool", K)
    ops = operands(N, T, H, seed=800 + K, K=K)
    pool0 = (0.3 * np.random.default_rng(K + 2).standard_normal((S_rows, H, K, K))).astype(np.float32)
    slots = np.array([4, 1, 2], dtype=np.int64)
    fresh = np.array([False, True, False])
    h0 = pool0.copy()
    h0[slots[1]] = 0.0  # the fresh row's starting state
    _, pool_ref, snap_ref = wkv7_ref(*np_list(ops), h0, state_idx=slots, snapshots=True)
    pool_ref[[0, 3, 5]] = pool0[[0, 3, 5]]
    pool = torch.from_numpy(pool0).to(dev)
    snaps = torch.full((N, T, H, K, K), float("nan"), device=dev)
    o = kernels.wkv7_pool_(*to_dev(ops, dev), pool, torch.from_numpy(slots).to(dev), H, K,
                           fresh=torch.from_numpy(fresh).to(dev), snapshots=snaps)
    torch.cuda.synchronize()
    assert o.shape == (N, T, H * K)
    _check(pool, pool_ref, S_TOL, "pool")
    _check(snaps, snap_ref, S_TOL, "snapshots")
    assert torch.equal(pool[[0, 3, 5]].cpu(), torch.from_numpy(pool0[[0, 3, 5]]))
