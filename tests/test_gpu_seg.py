"""GPU parity of the segmented chunked prefill (algo ALGO_SEGMENTED, rwkv-infer-next_amd/csrc/wkv7_seg.hip) in the
cases its design adds to the reference's single varlen launch (rwkv_next/kernels/wkv7.py:89-104, 126-138): rows cut
into several segments whose end states are handed over between workgroups (with and without an initial state), chunk
edges, ragged slot-pool calls with fresh rows and n_keep (units that start inside one row, run whole rows and hand
their last row on), calls without outputs, repeated calls on one workspace (the hand-off flags must come back to zero)
and replays of a captured HIP graph.  Tolerances as everywhere: y <= 2e-2 and
final state <= 1e-4 (max-relative) against the fp64 recurrence on the same bf16-rounded inputs."""
import numpy as np
import pytest

from gpu_util import S_TOL, Y_TOL, as_np, np_list, operands, say, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

SEG = 4  # _lib.ALGO_SEGMENTED


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from rwkv_next_amd import _lib
    _lib.load()
    assert _lib.ALGO_SEGMENTED == SEG
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def K():
    from rwkv_next_amd import kernels
    return kernels


def errs(o, o_ref, S, S_ref):
    from oracle import rel_max
    eo = rel_max(as_np(o).reshape(o_ref.shape), o_ref) if o is not None else 0.0
    es = rel_max(as_np(S).reshape(S_ref.shape), S_ref) if S is not None else 0.0
    say(f"y max-rel {eo:.3e}  state max-rel {es:.3e}")
    return eo, es


@pytest.mark.parametrize("B,T,H,use_s0", [(2, 2000, 4, True), (1, 1025, 2, True), (3, 511, 8, False),
                                          (1, 8 * 32 * 9 + 1, 1, True)])
def test_dense_rows_over_many_segments(dev, K, B, T, H, use_s0):
    """Few heads, so each row is cut into many segments (at least 8 chunks each) and every segment after the first
    takes its initial state from the previous one; lengths on and off the 32-token chunk edge."""
    from oracle import wkv7_ref
    say("seg dense", B, T, H, use_s0)
    ops = operands(B, T, H, seed=9000 + T + B)
    s0 = (0.3 * np.random.default_rng(T).standard_normal((B, H, 64, 64))).astype(np.float32) if use_s0 else None
    o_ref, S_ref, _ = wkv7_ref(*np_list(ops), s0)
    st = torch.from_numpy(s0).to(dev) if use_s0 else None
    o, S = K.wkv7(*to_dev(ops, dev), st, H, 64, algo=SEG)
    torch.cuda.synchronize()
    eo, es = errs(o, o_ref, S, S_ref)
    assert eo <= Y_TOL and es <= S_TOL


def test_repeated_calls_on_one_workspace(dev, K):
    """The same multi-segment call three times on one stream (one workspace): bit-identical results, so every call
    found the hand-off flags at zero and left them there."""
    B, T, H = 1, 3000, 2
    say("seg repeat", B, T, H)
    x = to_dev(operands(B, T, H, seed=77), dev)
    outs = [K.wkv7(*x, None, H, 64, algo=SEG) for _ in range(3)]
    torch.cuda.synchronize()
    for o, S in outs[1:]:
        assert torch.equal(o, outs[0][0]) and torch.equal(S, outs[0][1])


def test_ragged_pool_long_rows(dev, K):
    """A ragged slot-pool call whose long rows span several segments, next to short and empty rows, with fresh rows
    and n_keep limits; other slots untouched."""
    from oracle import rel_max, wkv7_ref
    import rwkv_next_amd.synth as synth
    H, S_slots = 4, 24
    lens = [1500, 0, 33, 1, 700, 2048, 64, 95, 1030]
    rng = np.random.default_rng(5)
    say("seg ragged pool", lens)
    seqs = [operands(1, L, H, seed=900 + i) for i, L in enumerate(lens)]
    cat = {n: np.concatenate([s[n] for s in seqs], axis=1) for n in seqs[0]}
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pool0 = synth.state_np((S_slots, H, 64, 64), seed=901)
    slots = rng.permutation(S_slots)[:len(lens)].astype(np.int64)
    fresh = np.array([0, 0, 1, 0, 0, 1, 0, 0, 0], bool)
    n_keep = np.array([L if i % 3 else max(0, L - 45) for i, L in enumerate(lens)], np.int64)
    pool_in = pool0.copy()
    pool_in[slots[fresh]] = 0.0
    o_ref, pool_ref, _ = wkv7_ref(*np_list(cat), pool_in, cu_seqlens=cu, state_idx=slots, n_keep=n_keep)
    pool = torch.from_numpy(pool0).to(dev)
    status = K.new_status(dev)
    o = K.wkv7_pool_(*to_dev(cat, dev), pool, torch.from_numpy(slots).to(dev), H, 64,
                     cu_seqlens=torch.from_numpy(cu).to(dev), n_keep=torch.from_numpy(n_keep).to(dev),
                     fresh=torch.from_numpy(fresh).to(dev), max_len=2048, algo=SEG, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    keep = np.zeros(sum(lens), bool)
    for i in range(len(lens)):
        keep[cu[i]:cu[i] + min(lens[i], n_keep[i])] = True
    eo = rel_max(as_np(o).reshape(o_ref.shape)[:, keep], o_ref[:, keep])
    es = rel_max(as_np(pool), pool_ref)
    say(f"y max-rel {eo:.3e}  state max-rel {es:.3e}")
    assert eo <= Y_TOL and es <= S_TOL
    untouched = np.setdiff1d(np.arange(S_slots), slots)
    assert np.array_equal(as_np(pool)[untouched], pool0[untouched])


def test_no_outputs_final_state_only(dev, K):
    """store_o = False: the segments skip the output correction but still combine their end states."""
    from oracle import rel_max, wkv7_ref
    import rwkv_next_amd.synth as synth
    H, T = 4, 1800
    say("seg store_o False", T, H)
    ops = operands(1, T, H, seed=31)
    pool0 = synth.state_np((3, H, 64, 64), seed=32)
    slots = np.array([2], np.int64)
    _, pool_ref, _ = wkv7_ref(*np_list(ops), pool0, state_idx=slots)
    pool = torch.from_numpy(pool0).to(dev)
    o = K.wkv7_pool_(*to_dev(ops, dev), pool, torch.from_numpy(slots).to(dev), H, 64, store_o=False, algo=SEG)
    torch.cuda.synchronize()
    assert o is None
    es = rel_max(as_np(pool), pool_ref)
    say(f"state max-rel {es:.3e}")
    assert es <= S_TOL


def test_graph_replays_match_eager(dev, K):
    """Captured in a HIP graph and replayed three times, with eager work in between: every replay bit-equal to the
    eager call (the hand-off flags are consumed within each replay)."""
    B, T, H = 1, 2600, 8
    say("seg graph", B, T, H)
    x = [t.clone() for t in to_dev(operands(B, T, H, seed=123), dev)]
    s0 = torch.from_numpy((0.2 * np.random.default_rng(3).standard_normal((B, H, 64, 64))).astype(np.float32)).to(dev)
    o_e, S_e = K.wkv7(*x, s0, H, 64, algo=SEG)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        K.wkv7(*x, s0, H, 64, algo=SEG)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        o_g, S_g = K.wkv7(*x, s0, H, 64, algo=SEG)
    for rep in range(3):
        o_g.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o_g, o_e) and torch.equal(S_g, S_e), f"replay {rep}"
        K.wkv7(*x, s0, H, 64, algo=SEG)  # eager work on the same stream between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("rec_max_len", [-1, 32])
def test_ragged_units_cross_many_rows(dev, K, rec_max_len):
    """H = 64 gives four units per head, each an equal share of the head's chunk stream, so a unit starts inside one
    row (P mode), finishes it, runs several whole rows (final states stored mid-loop) and hands its last row on.
    Empty and one-token rows sit between long ones.  rec_max_len = 32 sends the rows of at most 32 tokens to the
    token-serial kernel (two dispatches); -1 runs every row, empty ones included, through the segmented kernel."""
    from oracle import rel_max, wkv7_ref
    import rwkv_next_amd.synth as synth
    H, S_slots = 64, 48
    rng = np.random.default_rng(17)
    lens = [int(x) for x in rng.integers(1, 400, size=24)] + [0, 1, 31, 32, 33, 1100, 0, 2, 700, 64]
    lens = [lens[i] for i in rng.permutation(len(lens))]
    say("seg ragged cross rows", rec_max_len, len(lens), sum(lens))
    total = sum(lens)
    ops = operands(1, total, H, seed=4242)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pool0 = synth.state_np((S_slots, H, 64, 64), seed=4243)
    slots = rng.permutation(S_slots)[:len(lens)].astype(np.int64)
    o_ref, pool_ref, _ = wkv7_ref(*np_list(ops), pool0, cu_seqlens=cu, state_idx=slots)
    pool = torch.from_numpy(pool0).to(dev)
    status = K.new_status(dev)
    o = K.wkv7_pool_(*to_dev(ops, dev), pool, torch.from_numpy(slots).to(dev), H, 64,
                     cu_seqlens=torch.from_numpy(cu).to(dev), max_len=max(lens), algo=SEG, rec_max_len=rec_max_len,
                     status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    eo = rel_max(as_np(o).reshape(o_ref.shape), o_ref)
    es = rel_max(as_np(pool), pool_ref)
    say(f"y max-rel {eo:.3e}  state max-rel {es:.3e}")
    assert eo <= Y_TOL and es <= S_TOL
    untouched = np.setdiff1d(np.arange(S_slots), slots)
    assert np.array_equal(as_np(pool)[untouched], pool0[untouched])


def test_ragged_equal_rows_on_unit_edges_and_auto(dev, K):
    """Four 2048-token rows at H = 64: the four units of a head take one row each (no hand-off at all).  The same
    batch through AUTO (short rows token-serial, long rows segmented) gives the same bits."""
    from oracle import rel_max, wkv7_ref
    import rwkv_next_amd.synth as synth
    H, lens = 64, [2048] * 4
    say("seg ragged equal rows")
    total = sum(lens)
    ops = operands(1, total, H, seed=515)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pool0 = synth.state_np((8, H, 64, 64), seed=516)
    slots = np.array([6, 1, 3, 0], np.int64)
    o_ref, pool_ref, _ = wkv7_ref(*np_list(ops), pool0, cu_seqlens=cu, state_idx=slots)
    outs = []
    for algo in (SEG, 0):
        pool = torch.from_numpy(pool0).to(dev)
        o = K.wkv7_pool_(*to_dev(ops, dev), pool, torch.from_numpy(slots).to(dev), H, 64,
                         cu_seqlens=torch.from_numpy(cu).to(dev), max_len=2048, algo=algo)
        torch.cuda.synchronize()
        outs.append((o, pool))
    eo = rel_max(as_np(outs[0][0]).reshape(o_ref.shape), o_ref)
    es = rel_max(as_np(outs[0][1]), pool_ref)
    say(f"y max-rel {eo:.3e}  state max-rel {es:.3e}")
    assert eo <= Y_TOL and es <= S_TOL
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("nrows", [4096, 4097])
def test_ragged_row_table_limit(dev, K, nrows):
    """The segmented kernel keeps a ragged call's row table in LDS, at most 4096 rows.  4096 rows (mostly short, a
    few long, H = 2 so that each head's chunk stream is shared by many units) run as one segmented dispatch with the
    short rows in its tail; 4097 rows make AUTO take the two-kernel chunked path beside a token-serial launch, and an
    explicit SEGMENTED request is refused before any launch.  Both AUTO calls against the fp64 oracle."""
    from oracle import wkv7_ref
    from rwkv_next_amd import _lib
    import rwkv_next_amd.synth as synth
    H = 2
    rng = np.random.default_rng(nrows)
    lens = rng.integers(0, 48, size=nrows)
    lens[rng.choice(nrows, size=8, replace=False)] = rng.integers(300, 1500, size=8)
    lens = [int(x) for x in lens]
    say("seg row table limit", nrows, sum(lens))
    total = sum(lens)
    ops = operands(1, total, H, seed=nrows + 1)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    slots_n = nrows + 16
    pool0 = synth.state_np((slots_n, H, 64, 64), seed=nrows + 2)
    slots = rng.permutation(slots_n)[:nrows].astype(np.int64)
    o_ref, pool_ref, _ = wkv7_ref(*np_list(ops), pool0, cu_seqlens=cu, state_idx=slots)
    pool = torch.from_numpy(pool0).to(dev)
    status = K.new_status(dev)
    dev_ops, dslots, dcu = to_dev(ops, dev), torch.from_numpy(slots).to(dev), torch.from_numpy(cu).to(dev)
    o = K.wkv7_pool_(*dev_ops, pool, dslots, H, 64, cu_seqlens=dcu, max_len=max(lens), status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    eo, es = errs(o, o_ref, pool, pool_ref)
    assert eo <= Y_TOL and es <= S_TOL
    if nrows > 4096:
        with pytest.raises(_lib.Wkv7Error):
            K.wkv7_pool_(*dev_ops, torch.from_numpy(pool0).to(dev), dslots, H, 64, cu_seqlens=dcu,
                         max_len=max(lens), algo=SEG)
        torch.cuda.synchronize()
