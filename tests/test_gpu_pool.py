"""GPU tests of the slot-pool entry points (include/wkv7.h: wkv7_pool_reset, wkv7_pool_move, wkv7_snapshot_restore),
the StatePool wrapper (the WKV part of rwkv_next/model.py:298-316) and the model-level wrapper model_wkv7
(rwkv_next/model.py:77-83).  Byte copies, so every comparison is bit-exact (torch.equal) against torch indexing
with the reference's semantics."""
import numpy as np
import pytest

from gpu_util import S_TOL, Y_TOL, as_np, np_list, operands, say, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def K():
    from rwkv_next_amd import kernels
    return kernels


def random_pool(K, dev, L, S, H, seed):
    p = K.StatePool(L, S, H, dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    p.wkv.copy_(torch.randn(p.wkv.shape, device=dev, generator=g))
    return p


def test_reset_slots_zeroes_listed_slots_of_every_layer(dev, K):
    say("pool reset")
    p = random_pool(K, dev, 3, 10, 4, seed=1)
    ref = p.wkv.clone()
    idx = torch.tensor([2, 7, 0], device=dev)
    p.reset_slots(idx)
    ref[:, idx] = 0
    torch.cuda.synchronize()
    assert torch.equal(p.wkv, ref)
    assert p.state_bytes_per_slot() == 3 * 4 * 64 * 64 * 4


@pytest.mark.parametrize("case", ["swap_chain", "many"])
def test_move_slots_is_gather_then_scatter(dev, K, case):
    say("pool move", case)
    if case == "swap_chain":
        L, S, H = 2, 12, 3
        src = [1, 4, 5, 8, 9]
        dst = [4, 1, 9, 2, 11]          # 1 <-> 4 swap, 5 -> 9 while 9 -> 11 (chain), 8 -> 2
    else:
        L, S, H = 2, 400, 2
        rng = np.random.default_rng(7)
        src = rng.permutation(S)[:300].tolist()
        dst = rng.permutation(S)[:300].tolist()   # many moves: small staging ranges, overlapping sets
    p = random_pool(K, dev, L, S, H, seed=2)
    ref = p.wkv.clone()
    s = torch.tensor(src, device=dev)
    d = torch.tensor(dst, device=dev)
    ref[:, d] = ref[:, s]                 # the reference's move_slots (model.py:313-316)
    p.move_slots(s, d)
    torch.cuda.synchronize()
    assert torch.equal(p.wkv, ref)


def test_snapshot_restore_matches_indexing(dev, K):
    say("snapshot restore")
    N, T, H, S = 6, 5, 4, 9
    g = torch.Generator(device=dev).manual_seed(3)
    pool = torch.randn(S, H, 64, 64, device=dev, generator=g)
    snaps = torch.randn(N, T, H, 64, 64, device=dev, generator=g)
    slots = torch.tensor([8, 0, 3, 5, 1, 6], device=dev)
    n = torch.tensor([1, 0, 5, 3, 2, 4], device=dev)
    ref = pool.clone()
    for b in range(N):
        if int(n[b]) > 0:
            ref[int(slots[b])] = snaps[b, int(n[b]) - 1]
    K.restore_snapshots_(pool, slots, snaps, n)
    torch.cuda.synchronize()
    assert torch.equal(pool, ref)


def test_snapshot_restore_two_units_per_workgroup(dev, K):
    """Enough (sequence, head) units (257 x 5 = 1285, odd) for the two-units-per-workgroup launch, with accepted
    counts 0..T and a pool slot per sequence."""
    say("snapshot restore, two units per workgroup")
    N, T, H, S = 257, 3, 5, 300
    g = torch.Generator(device=dev).manual_seed(5)
    pool = torch.randn(S, H, 64, 64, device=dev, generator=g)
    snaps = torch.randn(N, T, H, 64, 64, device=dev, generator=g)
    slots = torch.randperm(S, device=dev, generator=g)[:N]
    n = torch.randint(0, T + 1, (N,), device=dev, generator=g)
    ref = pool.clone()
    for b in range(N):
        if int(n[b]) > 0:
            ref[int(slots[b])] = snaps[b, int(n[b]) - 1]
    K.restore_snapshots_(pool, slots, snaps, n)
    torch.cuda.synchronize()
    assert torch.equal(pool, ref)


def test_pool_ops_in_a_graph_replay_like_eager(dev, K):
    """reset + move + decode recorded into one HIP graph, replayed several times with eager work between the
    replays; every replay equals the same calls made eagerly."""
    say("pool graph")
    L, S, H, B = 2, 16, 4, 4
    pg = random_pool(K, dev, L, S, H, seed=4)
    pe = K.StatePool(L, S, H, dev)
    pe.wkv.copy_(pg.wkv)
    x = [t.clone() for t in to_dev(operands(B, 1, H, seed=5), dev)]
    slots = torch.tensor([3, 9, 0, 12], device=dev)
    ridx = torch.tensor([5], device=dev)
    src, dst = torch.tensor([3, 9], device=dev), torch.tensor([9, 3], device=dev)

    def step(p):
        p.reset_slots(ridx)
        p.move_slots(src, dst)
        return [K.wkv7_pool_(*x, p.layer(i), slots, H, 64) for i in range(L)]

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        scratch = K.StatePool(L, S, H, dev)
        step(scratch)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = step(pg)
    torch.cuda.synchronize()
    for it in range(3):
        g.replay()
        oe = step(pe)
        torch.cuda.synchronize()
        for a, b in zip(outs, oe):
            assert torch.equal(a, b), f"replay {it}"
        assert torch.equal(pg.wkv, pe.wkv), f"replay {it}"


def test_model_wrapper_casts_and_reshapes(dev, K):
    """model_wkv7 takes any float dtype, casts to bf16 (model.py:81) and returns o as (B, T, C)."""
    from oracle import rel_max, wkv7_ref
    say("model_wkv7")
    B, T, H = 2, 40, 4
    ops = operands(B, T, H, seed=9)
    x32 = [t.float() for t in to_dev(ops, dev)]
    s0 = torch.from_numpy((0.2 * np.random.default_rng(9).standard_normal((B, H, 64, 64))).astype(np.float32)).to(dev)
    o, S = K.model_wkv7(*x32, s0, H, 64)
    o_bf, S_bf = K.wkv7(*[t.bfloat16() for t in x32], s0, H, 64)
    torch.cuda.synchronize()
    assert o.shape == (B, T, H * 64) and o.dtype == torch.bfloat16
    assert torch.equal(o, o_bf.view(B, T, H * 64)) and torch.equal(S, S_bf)
    o_ref, S_ref, _ = wkv7_ref(*np_list(ops), s0.cpu().numpy())
    assert rel_max(as_np(o).reshape(o_ref.shape), o_ref) <= Y_TOL
    assert rel_max(as_np(S), S_ref) <= S_TOL


def test_speculative_verify_and_rollback_across_layers(dev, K):
    """Configuration 4 (speculative verify, B=64, T=5) wired through the pool: every layer verifies T tokens (pool untouched, snapshots taken),
    then rollback_ restores each row's accepted prefix in every layer.  The result equals, bit for bit, the
    reference's method -- wkv7_replay of the first n[b] tokens per layer from the incoming states (model.py:498-503)
    -- eagerly and inside one captured HIP graph replayed three times (the pool reset eagerly between replays)."""
    say("spec verify + rollback")
    L, S, H, B, T = 3, 16, 4, 6, 5
    pool = random_pool(K, dev, L, S, H, seed=41)
    pool0 = pool.wkv.clone()
    slots = torch.tensor([7, 2, 11, 0, 14, 5], device=dev)
    n = torch.tensor([1, 5, 3, 0, 2, 4], device=dev)
    xs = [[t.clone() for t in to_dev(operands(B, T, H, seed=42 + i), dev)] for i in range(L)]
    snaps = pool.snapshot_buffer(B, T)

    def spec_step():
        outs = [pool.verify_(i, *xs[i], slots, snaps) for i in range(L)]
        pool.rollback_(slots, n, snaps)
        return outs

    outs_e = spec_step()
    torch.cuda.synchronize()
    # the reference's rollback: replay the first n tokens of each row from the incoming states, per layer
    expect = pool0.clone()
    for i in range(L):
        st = expect[i][slots].contiguous()
        K.wkv7_replay(*xs[i], st, torch.clamp(n, min=1), H, 64)
        keep = (n > 0).view(-1, 1, 1, 1)
        expect[i][slots] = torch.where(keep, st, expect[i][slots])
        o_plain = K.wkv7_pool_(*xs[i], pool0[i].clone(), slots, H, 64, algo=1)
        assert torch.equal(outs_e[i], o_plain), f"layer {i}: verify output"
    torch.cuda.synchronize()
    assert torch.equal(pool.wkv, expect)
    untouched = [s for s in range(S) if s not in slots.tolist()]
    assert torch.equal(pool.wkv[:, untouched], pool0[:, untouched])
    # the replay form of the rollback (no snapshots) lands on the same bits, n = 0 rows included
    rp = K.StatePool(L, S, H, dev)
    rp.wkv.copy_(pool0)
    for i in range(L):
        K.wkv7_pool_(*xs[i], rp.layer(i), slots, H, 64, final=False)
        rp.replay_(i, *xs[i], slots, n)
    torch.cuda.synchronize()
    assert torch.equal(rp.wkv, expect)

    pool.wkv.copy_(pool0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        spec_step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    pool.wkv.copy_(pool0)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        outs_g = spec_step()
    for it in range(3):
        pool.wkv.copy_(pool0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(pool.wkv, expect), f"replay {it}"
        for i in range(L):
            assert torch.equal(outs_g[i], outs_e[i]), f"replay {it} layer {i}"
