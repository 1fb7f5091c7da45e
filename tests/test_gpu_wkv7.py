"""GPU parity of the HIP WKV7 kernels against the CPU oracle, on the reference's own test cases
(tools/test_wkv7.py:41-91: plain T = 1 / 4 / 300 with and without h0, varlen with per-sequence h0, replay of
the first n[b] of T = 4 steps in place) and on the slot-pool, snapshot and graph paths the build adds.

Every case runs the token-serial kernel, the chunked MFMA kernel and the automatic choice.  Tolerances: y
max-relative <= 2e-2 (bf16 output) and final state max-relative <= 1e-4, both against the fp64 recurrence
on the same bf16-rounded inputs."""
import numpy as np
import pytest

from gpu_util import S_TOL, Y_TOL, as_np, np_list, operands, say, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

H8 = 8
ALGOS = {"auto": 0, "recurrent": 1, "chunked": 2, "chain": 3, "seg": 4}


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from rwkv_next_amd import _lib
    _lib.load()
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def K():
    from rwkv_next_amd import kernels
    return kernels


def check(o_gpu, o_ref, S_gpu=None, S_ref=None, y_tol=Y_TOL, s_tol=S_TOL):
    from oracle import rel_fro, rel_max
    if o_gpu is not None:
        eo = rel_max(as_np(o_gpu).reshape(o_ref.shape), o_ref)
        assert eo <= y_tol, f"y max-rel {eo:.3e}"
        assert rel_fro(as_np(o_gpu).reshape(o_ref.shape), o_ref) < 2e-2
    if S_gpu is not None:
        es = rel_max(as_np(S_gpu).reshape(S_ref.shape), S_ref)
        assert es <= s_tol, f"state max-rel {es:.3e}"


@pytest.mark.parametrize("algo", list(ALGOS))
@pytest.mark.parametrize("B,T,use_s0", [(3, 1, True), (2, 4, True), (2, 300, False), (1, 300, True)])
def test_reference_cases_dense(dev, K, B, T, use_s0, algo):
    from oracle import wkv7_ref
    say("dense", B, T, use_s0, algo)
    ops = operands(B, T, H8, seed=B * 1000 + T)
    s0 = (0.3 * np.random.default_rng(B + T).standard_normal((B, H8, 64, 64))).astype(np.float32) if use_s0 else None
    o_ref, S_ref, _ = wkv7_ref(*np_list(ops), s0)
    st = torch.from_numpy(s0).to(dev) if use_s0 else None
    o, S = K.wkv7(*to_dev(ops, dev), st, H8, 64, algo=ALGOS[algo])
    torch.cuda.synchronize()
    check(o, o_ref, S, S_ref)
    if st is not None:
        assert torch.equal(st.cpu(), torch.from_numpy(s0))  # the functional form never mutates state


@pytest.mark.parametrize("algo", list(ALGOS))
def test_reference_case_varlen(dev, K, algo):
    from oracle import wkv7_ref
    lens = [5, 1, 37, 300, 0, 64, 65, 128]
    say("varlen", lens, algo)
    seqs = [operands(1, L, H8, seed=7 + L) for L in lens]
    s0 = (0.3 * np.random.default_rng(1).standard_normal((len(lens), H8, 64, 64))).astype(np.float32)
    cat = {n: np.concatenate([s[n] for s in seqs], axis=1) for n in seqs[0]}
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    o_ref, S_ref, _ = wkv7_ref(*np_list(cat), s0, cu_seqlens=cu)
    o, S = K.wkv7(*to_dev(cat, dev), torch.from_numpy(s0).to(dev), H8, 64,
                  cu_seqlens=torch.from_numpy(cu).to(dev), algo=ALGOS[algo])
    torch.cuda.synchronize()
    check(o, o_ref, S, S_ref)


def test_reference_case_replay(dev, K):
    from oracle import wkv7_ref
    B, T = 4, 4
    say("replay")
    ops = operands(B, T, H8, seed=99)
    s0 = (0.3 * np.random.default_rng(2).standard_normal((B, H8, 64, 64))).astype(np.float32)
    n = np.array([1, 2, 4, 3], np.int64)
    _, S_ref, _ = wkv7_ref(*np_list(ops), s0, n_keep=n, store_o=False)
    st = torch.from_numpy(s0).to(dev)
    out = K.wkv7_replay(*to_dev(ops, dev), st, torch.from_numpy(n).to(dev), H8, 64)
    torch.cuda.synchronize()
    assert out is st
    check(None, None, st, S_ref)


@pytest.mark.parametrize("algo", list(ALGOS))
def test_final_false_returns_no_state(dev, K, algo):
    from oracle import wkv7_ref
    say("final=False", algo)
    ops = operands(2, 70, H8, seed=5)
    o_ref, _, _ = wkv7_ref(*np_list(ops))
    o, S = K.wkv7(*to_dev(ops, dev), None, H8, 64, final=False, algo=ALGOS[algo])
    torch.cuda.synchronize()
    assert S is None
    check(o, o_ref)


# ---------------------------------------------------------------------------------------------------------------
# slot pool
# ---------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("algo", list(ALGOS))
@pytest.mark.parametrize("T", [1, 5, 100])
def test_pool_in_place_update(dev, K, T, algo):
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    S_slots, B, H = 16, 6, 4
    say("pool", T, algo)
    ops = operands(B, T, H, seed=11 + T)
    pool0 = synth.state_np((S_slots, H, 64, 64), seed=12)
    slots = np.array([9, 2, 15, 0, 7, 4], np.int64)
    fresh = np.array([0, 1, 0, 0, 1, 0], bool)
    pool_ref_in = pool0.copy()
    pool_ref_in[slots[fresh]] = 0.0
    o_ref, pool_ref, _ = wkv7_ref(*np_list(ops), pool_ref_in, state_idx=slots)
    pool = torch.from_numpy(pool0).to(dev)
    o = K.wkv7_pool_(*to_dev(ops, dev), pool, torch.from_numpy(slots).to(dev), H, 64,
                     fresh=torch.from_numpy(fresh).to(dev), algo=ALGOS[algo], check_slots=True)
    torch.cuda.synchronize()
    check(o, o_ref, pool, pool_ref)
    untouched = sorted(set(range(S_slots)) - set(slots.tolist()))
    assert torch.equal(pool[untouched].cpu(), torch.from_numpy(pool0[untouched]))


@pytest.mark.parametrize("algo", list(ALGOS))
def test_pool_ragged_mixed_rows(dev, K, algo):
    """Packed rows of very different lengths in one call (decode rows next to prefill rows)."""
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    H = 4
    lens = [1, 1, 200, 1, 33, 64, 1, 2]
    say("pool ragged", lens, algo)
    seqs = [operands(1, L, H, seed=40 + i) for i, L in enumerate(lens)]
    cat = {n: np.concatenate([s[n] for s in seqs], axis=1) for n in seqs[0]}
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pool0 = synth.state_np((20, H, 64, 64), seed=41)
    slots = np.array([3, 17, 5, 0, 19, 8, 11, 2], np.int64)
    o_ref, pool_ref, _ = wkv7_ref(*np_list(cat), pool0, cu_seqlens=cu, state_idx=slots)
    pool = torch.from_numpy(pool0).to(dev)
    o = K.wkv7_pool_(*to_dev(cat, dev), pool, torch.from_numpy(slots).to(dev), H, 64,
                     cu_seqlens=torch.from_numpy(cu).to(dev), algo=ALGOS[algo])
    torch.cuda.synchronize()
    check(o, o_ref, pool, pool_ref)


def test_chain_kernel_many_chains(dev, K):
    """The single-dispatch chain kernel with more (row, head) chains than workgroups and very uneven rows: packed rows
    of 0 .. 700 tokens (most above the 32-token token-serial bound, some below), distinct pool slots, fresh rows and
    n_keep limits; every state and output against the oracle, and slots outside the batch untouched."""
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    H, S_slots = 16, 64
    rng = np.random.default_rng(77)
    lens = [int(x) for x in rng.integers(0, 701, size=40)]
    lens[3], lens[7], lens[11] = 1, 0, 32
    say("chain kernel", len(lens), "rows", sum(lens), "tokens")
    seqs = [operands(1, L, H, seed=300 + i) for i, L in enumerate(lens)]
    cat = {n: np.concatenate([s[n] for s in seqs], axis=1) for n in seqs[0]}
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pool0 = synth.state_np((S_slots, H, 64, 64), seed=301)
    slots = rng.permutation(S_slots)[:len(lens)].astype(np.int64)
    fresh = rng.random(len(lens)) < 0.2
    n_keep = np.array([L if i % 5 else max(0, L - 17) for i, L in enumerate(lens)], np.int64)
    pool_in = pool0.copy()
    pool_in[slots[fresh]] = 0.0
    o_ref, pool_ref, _ = wkv7_ref(*np_list(cat), pool_in, cu_seqlens=cu, state_idx=slots, n_keep=n_keep)
    pool = torch.from_numpy(pool0).to(dev)
    status = K.new_status(dev)
    o = K.wkv7_pool_(*to_dev(cat, dev), pool, torch.from_numpy(slots).to(dev), H, 64,
                     cu_seqlens=torch.from_numpy(cu).to(dev), n_keep=torch.from_numpy(n_keep).to(dev),
                     fresh=torch.from_numpy(fresh).to(dev), max_len=700, algo=3, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    # outputs past a row's n_keep are not produced (the reference's STORE_O loop stops at L = min(len, n_keep))
    keep = np.zeros(sum(lens), bool)
    for i in range(len(lens)):
        keep[cu[i]:cu[i] + min(lens[i], n_keep[i])] = True
    from oracle import rel_max
    eo = rel_max(as_np(o).reshape(o_ref.shape)[:, keep], o_ref[:, keep])
    es = rel_max(as_np(pool), pool_ref)
    say(f"y max-rel {eo:.3e}  state max-rel {es:.3e}")
    assert eo <= Y_TOL and es <= S_TOL
    untouched = np.setdiff1d(np.arange(S_slots), slots)
    assert np.array_equal(as_np(pool)[untouched], pool0[untouched])


@pytest.mark.parametrize("algo", list(ALGOS))
@pytest.mark.parametrize("seed", [2, 4, 5, 6, 7, 10])
def test_random_ragged_batches(dev, K, algo, seed):
    """Seeded random ragged batches on every algorithm: 1 to 12 rows whose lengths are drawn with weight on the
    token-serial bound and the chunk edges (0, 1, 31, 32, 33, 63, 64, 65, 127, 128, 129) and otherwise uniform in
    [0, 300), 1 to 12 heads, distinct random pool slots, fresh rows, n_keep limits and a tight or absent max_len.
    Every kept output and every state against the oracle, the status word clean, other slots untouched."""
    from oracle import rel_max, wkv7_ref
    import rwkv_next_amd.synth as synth
    rng = np.random.default_rng(4000 + seed)
    H = int(rng.choice([1, 3, 8, 12]))
    B = int(rng.integers(1, 13))
    edges = [0, 1, 31, 32, 33, 63, 64, 65, 127, 128, 129]
    lens = [int(rng.choice(edges)) if rng.random() < 0.6 else int(rng.integers(0, 300)) for _ in range(B)]
    if sum(lens) == 0:
        lens[0] = 65
    S_slots = B + 5
    slots = rng.permutation(S_slots)[:B].astype(np.int64)
    fresh = rng.random(B) < 0.25
    n_keep = np.array([L if rng.random() < 0.7 else int(rng.integers(0, L + 1)) for L in lens], np.int64)
    max_len = max(lens) if seed % 2 else 0
    say("random ragged", seed, algo, "H", H, "lens", lens, "n_keep", n_keep.tolist(), "max_len", max_len)
    seqs = [operands(1, L, H, seed=500 + 13 * seed + i) for i, L in enumerate(lens)]
    cat = {n: np.concatenate([s[n] for s in seqs], axis=1) for n in seqs[0]}
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pool0 = synth.state_np((S_slots, H, 64, 64), seed=600 + seed)
    pool_in = pool0.copy()
    pool_in[slots[fresh]] = 0.0
    o_ref, pool_ref, _ = wkv7_ref(*np_list(cat), pool_in, cu_seqlens=cu, state_idx=slots, n_keep=n_keep)
    pool = torch.from_numpy(pool0).to(dev)
    status = K.new_status(dev)
    o = K.wkv7_pool_(*to_dev(cat, dev), pool, torch.from_numpy(slots).to(dev), H, 64,
                     cu_seqlens=torch.from_numpy(cu).to(dev), n_keep=torch.from_numpy(n_keep).to(dev),
                     fresh=torch.from_numpy(fresh).to(dev), max_len=max_len, algo=ALGOS[algo], status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    keep = np.zeros(sum(lens), bool)
    for i in range(B):
        keep[cu[i]:cu[i] + min(lens[i], n_keep[i])] = True
    if keep.any():
        eo = rel_max(as_np(o).reshape(o_ref.shape)[:, keep], o_ref[:, keep])
        assert eo <= Y_TOL, f"y max-rel {eo:.3e}"
    es = rel_max(as_np(pool), pool_ref)
    assert es <= S_TOL, f"state max-rel {es:.3e}"
    untouched = np.setdiff1d(np.arange(S_slots), slots)
    assert np.array_equal(as_np(pool)[untouched], pool0[untouched])


def test_chunked_rows_across_scan_passes(dev, K):
    """The chunked path's scan walks a row's chunks in unrolled passes of 16 and then passes of 4: rows of 17 to 63
    chunks use both.  Dense T = 1100 (18 chunks, the last partial) and a ragged batch on the chunked algorithm with
    rows of 1030, 2100, 64, 5 and 0 tokens (17, 33, 1, 1, 0 chunks), fresh rows and an n_keep limit, against the
    oracle."""
    from oracle import rel_max, wkv7_ref
    import rwkv_next_amd.synth as synth
    H = 4
    say("chunked scan passes: dense T=1100")
    ops = operands(2, 1100, H, seed=91)
    s0 = (0.3 * np.random.default_rng(92).standard_normal((2, H, 64, 64))).astype(np.float32)
    o_ref, S_ref, _ = wkv7_ref(*np_list(ops), s0)
    o, S = K.wkv7(*to_dev(ops, dev), torch.from_numpy(s0).to(dev), H, 64, algo=ALGOS["chunked"])
    torch.cuda.synchronize()
    check(o, o_ref, S, S_ref)

    lens = [1030, 2100, 64, 5, 0]
    say("chunked scan passes: ragged", lens)
    seqs = [operands(1, L, H, seed=93 + i) for i, L in enumerate(lens)]
    cat = {n: np.concatenate([s[n] for s in seqs], axis=1) for n in seqs[0]}
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pool0 = synth.state_np((8, H, 64, 64), seed=94)
    slots = np.array([6, 1, 3, 7, 0], np.int64)
    fresh = np.array([0, 1, 0, 0, 1], bool)
    n_keep = np.array([1030, 1500, 64, 5, 0], np.int64)
    pool_in = pool0.copy()
    pool_in[slots[fresh]] = 0.0
    o_ref, pool_ref, _ = wkv7_ref(*np_list(cat), pool_in, cu_seqlens=cu, state_idx=slots, n_keep=n_keep)
    pool = torch.from_numpy(pool0).to(dev)
    o = K.wkv7_pool_(*to_dev(cat, dev), pool, torch.from_numpy(slots).to(dev), H, 64,
                     cu_seqlens=torch.from_numpy(cu).to(dev), n_keep=torch.from_numpy(n_keep).to(dev),
                     fresh=torch.from_numpy(fresh).to(dev), max_len=2100, algo=ALGOS["chunked"])
    torch.cuda.synchronize()
    keep = np.zeros(sum(lens), bool)
    for i in range(len(lens)):
        keep[cu[i]:cu[i] + min(lens[i], n_keep[i])] = True
    eo = rel_max(as_np(o).reshape(o_ref.shape)[:, keep], o_ref[:, keep])
    es = rel_max(as_np(pool), pool_ref)
    say(f"y max-rel {eo:.3e}  state max-rel {es:.3e}")
    assert eo <= Y_TOL and es <= S_TOL


def test_pool_final_false_leaves_pool_untouched(dev, K):
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    say("pool final=False")
    H = 4
    ops = operands(3, 5, H, seed=21)
    pool0 = synth.state_np((5, H, 64, 64), seed=22)
    slots = np.array([4, 1, 2], np.int64)
    o_ref, _, _ = wkv7_ref(*np_list(ops), pool0, state_idx=slots)
    pool = torch.from_numpy(pool0).to(dev)
    o = K.wkv7_pool_(*to_dev(ops, dev), pool, torch.from_numpy(slots).to(dev), H, 64, final=False)
    torch.cuda.synchronize()
    check(o, o_ref)
    assert torch.equal(pool.cpu(), torch.from_numpy(pool0))


def test_snapshots_are_bit_identical_to_a_rerun(dev, K):
    """The speculative-verify contract (configuration 4) at a small size: after a verify of T tokens with snapshots, restoring the state
    after n accepted tokens equals, bit for bit, re-running the first n tokens."""
    import rwkv_next_amd.synth as synth
    say("snapshots")
    B, T, H = 8, 5, 4
    ops = operands(B, T, H, seed=31)
    pool0 = synth.state_np((12, H, 64, 64), seed=32)
    slots = torch.tensor([3, 0, 11, 7, 5, 1, 9, 2], device=dev)
    x = to_dev(ops, dev)
    pool = torch.from_numpy(pool0).to(dev)
    snaps = torch.empty(B, T, H, 64, 64, device=dev)
    o_verify = K.wkv7_pool_(*x, pool, slots, H, 64, final=False, snapshots=snaps)
    n = torch.tensor([1, 2, 3, 4, 5, 0, 5, 2], device=dev)
    K.restore_snapshots_(pool, slots, snaps, n)
    rerun = torch.from_numpy(pool0).to(dev)
    K.wkv7_pool_(*x, rerun, slots, H, 64, n_keep=n, store_o=False)
    torch.cuda.synchronize()
    assert torch.equal(pool, rerun)
    # the verify's outputs equal a plain run's outputs bit for bit as well
    o_plain = K.wkv7_pool_(*x, torch.from_numpy(pool0).to(dev), slots, H, 64, algo=1)
    torch.cuda.synchronize()
    assert torch.equal(o_verify, o_plain)


def test_ragged_snapshots_and_rollback(dev, K):
    """A ragged verify (rows of 0..5 tokens packed with cu_seqlens) with per-token snapshots (N, max_len, H, 64, 64):
    row n's entries t < its length hold the state after token t (the oracle within tolerance, and bit for bit a dense
    verify of that row alone), the entries past its length are untouched, and restoring n accepted tokens equals a
    ragged re-run of the first n tokens bit for bit."""
    from oracle import rel_max, wkv7_ref
    import rwkv_next_amd.synth as synth
    H, Tm = 4, 5
    lens = [5, 1, 0, 3, 5, 2]
    N = len(lens)
    say("ragged snapshots", lens)
    seqs = [operands(1, L, H, seed=600 + i) for i, L in enumerate(lens)]
    cat = {n: np.concatenate([s[n] for s in seqs], axis=1) for n in seqs[0]}
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pool0 = synth.state_np((10, H, 64, 64), seed=601)
    slots = np.array([7, 2, 9, 0, 4, 5], np.int64)
    _, _, snap_ref = wkv7_ref(*np_list(cat), pool0, cu_seqlens=cu, state_idx=slots, snapshots=True)
    x, sl, cu_d = to_dev(cat, dev), torch.from_numpy(slots).to(dev), torch.from_numpy(cu).to(dev)
    pool = torch.from_numpy(pool0).to(dev)
    snaps = torch.full((N, Tm, H, 64, 64), -7.0, device=dev)
    status = K.new_status(dev)
    K.wkv7_pool_(*x, pool, sl, H, 64, cu_seqlens=cu_d, final=False, snapshots=snaps, max_len=Tm, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    assert torch.equal(pool.cpu(), torch.from_numpy(pool0))  # final=False: the pool is only read
    got = as_np(snaps)
    for n, L in enumerate(lens):
        assert np.all(got[n, L:] == -7.0), n
        if L == 0:
            continue
        es = rel_max(got[n, :L], snap_ref[n, :L])
        say(f"row {n}: snapshot max-rel {es:.3e}")
        assert es <= S_TOL
        alone = torch.empty(1, L, H, 64, 64, device=dev)
        K.wkv7_pool_(*to_dev(seqs[n], dev), torch.from_numpy(pool0).to(dev), sl[n:n + 1], H, 64, final=False,
                     snapshots=alone)
        torch.cuda.synchronize()
        assert torch.equal(snaps[n, :L], alone[0]), n
    n_acc = torch.tensor([5, 1, 0, 2, 0, 1], device=dev)
    K.restore_snapshots_(pool, sl, snaps, n_acc)
    rerun = torch.from_numpy(pool0).to(dev)
    K.wkv7_pool_(*x, rerun, sl, H, 64, cu_seqlens=cu_d, n_keep=n_acc, store_o=False, max_len=Tm)
    torch.cuda.synchronize()
    assert torch.equal(pool, rerun)
    with pytest.raises(ValueError, match="max_len"):
        K.wkv7_pool_(*x, pool, sl, H, 64, cu_seqlens=cu_d, final=False, snapshots=snaps)


@pytest.mark.parametrize("algo", [0, 1, 2, 3, 4])
def test_ragged_rows_longer_than_max_len_are_cut(dev, K, algo):
    """max_len bounds a ragged call's rows (it sizes the chunked and segmented workspaces): a longer row runs on its
    first max_len tokens only, on every path, and the status word reports it."""
    from rwkv_next_amd import _lib
    from oracle import rel_max, wkv7_ref
    import rwkv_next_amd.synth as synth
    H, max_len = 4, 96
    lens = [300, 40, 0, 129, 7, 96]
    say("rows cut to max_len", algo, lens, max_len)
    seqs = [operands(1, L, H, seed=700 + i) for i, L in enumerate(lens)]
    cat = {n: np.concatenate([s[n] for s in seqs], axis=1) for n in seqs[0]}
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pool0 = synth.state_np((8, H, 64, 64), seed=701)
    slots = np.array([3, 6, 0, 1, 7, 4], np.int64)
    kept = np.minimum(lens, max_len)
    o_ref, pool_ref, _ = wkv7_ref(*np_list(cat), pool0, cu_seqlens=cu, state_idx=slots, n_keep=kept)
    pool = torch.from_numpy(pool0).to(dev)
    status = K.new_status(dev)
    o = K.wkv7_pool_(*to_dev(cat, dev), pool, torch.from_numpy(slots).to(dev), H, 64,
                     cu_seqlens=torch.from_numpy(cu).to(dev), max_len=max_len, algo=algo, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == _lib.WKV7_STATUS_SEQLENS
    keep = np.zeros(sum(lens), bool)
    for i in range(len(lens)):
        keep[cu[i]:cu[i] + kept[i]] = True
    eo = rel_max(as_np(o).reshape(o_ref.shape)[:, keep], o_ref[:, keep])
    es = rel_max(as_np(pool), pool_ref)
    say(f"y max-rel {eo:.3e}  state max-rel {es:.3e}")
    assert eo <= Y_TOL and es <= S_TOL


def test_check_distinct_slots(dev, K):
    with pytest.raises(ValueError):
        K.check_distinct_slots(torch.tensor([1, 2, 1], device=dev), 4)
    with pytest.raises(ValueError):
        K.check_distinct_slots(torch.tensor([1, 4], device=dev), 4)
    K.check_distinct_slots(torch.tensor([3, 0, 1], device=dev), 4)


def test_graph_capture_replays_match_eager(dev, K):
    """Decode step captured once in a CUDA (HIP) graph and replayed with new inputs and new slots; every replay
    is compared with an eager call on the same values (eager work and syncs between replays)."""
    import rwkv_next_amd.synth as synth
    say("graph")
    B, H, S_slots = 8, 4, 32
    pool_g = torch.from_numpy(synth.state_np((S_slots, H, 64, 64), seed=50)).to(dev)
    pool_e = pool_g.clone()
    static_in = [t.clone() for t in to_dev(operands(B, 1, H, seed=51), dev)]
    static_slots = torch.arange(B, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        K.wkv7_pool_(*static_in, pool_g.clone(), static_slots, H, 64)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_out = K.wkv7_pool_(*static_in, pool_g, static_slots, H, 64)
    torch.cuda.synchronize()
    pool_g.copy_(pool_e)  # capture does not execute, but reset anyway
    rng = np.random.default_rng(52)
    for it in range(4):
        new = to_dev(operands(B, 1, H, seed=60 + it), dev)
        sl = torch.from_numpy(rng.permutation(S_slots)[:B].astype(np.int64)).to(dev)
        for dst, src in zip(static_in, new):
            dst.copy_(src)
        static_slots.copy_(sl)
        g.replay()
        o_e = K.wkv7_pool_(*new, pool_e, sl, H, 64)
        torch.cuda.synchronize()
        assert torch.equal(static_out, o_e), f"replay {it}"
        assert torch.equal(pool_g, pool_e), f"replay {it}"


def test_graph_capture_chunked_prefill(dev, K):
    """The chunked path (workspace from the graph pool) captured and replayed with new inputs."""
    import rwkv_next_amd.synth as synth
    say("graph chunked")
    B, T, H = 1, 200, 4
    static_in = [t.clone() for t in to_dev(operands(B, T, H, seed=70), dev)]
    pool_g = torch.from_numpy(synth.state_np((2, H, 64, 64), seed=71)).to(dev)
    pool_e = pool_g.clone()
    slots = torch.tensor([1], device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        K.wkv7_pool_(*static_in, pool_g.clone(), slots, H, 64)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_out = K.wkv7_pool_(*static_in, pool_g, slots, H, 64)
    torch.cuda.synchronize()
    for it in range(3):
        new = to_dev(operands(B, T, H, seed=80 + it), dev)
        for dst, src in zip(static_in, new):
            dst.copy_(src)
        g.replay()
        o_e = K.wkv7_pool_(*new, pool_e, slots, H, 64)
        torch.cuda.synchronize()
        assert torch.equal(static_out, o_e), f"replay {it}"
        assert torch.equal(pool_g, pool_e), f"replay {it}"
