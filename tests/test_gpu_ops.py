"""The torch-op half of the boundary on the GPU: the registered ops pass torch.library.opcheck, run under
torch.compile the way the reference's own test drives its op (tools/test_wkv7.py:50-54), and a compiled
part_att-shaped function (rwkv_next/model.py:334-342: operand views -> wkv -> output, slot pool updated in place)
traces with no graph break, matches eager bit for bit and replays inside a captured graph.  Also the device
status word: out-of-range slot indices and malformed lengths are reported without a fault or a host sync.

Tolerances as everywhere: y <= 2e-2 and state <= 1e-4 max-relative against the fp64 oracle on the same
bf16-rounded inputs; compiled against eager and graph against eager with torch.equal."""
import numpy as np
import pytest

from gpu_util import S_TOL, Y_TOL, as_np, np_list, operands, say, to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

H8 = 8


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def K():
    from rwkv_next_amd import kernels
    return kernels


def _np(x):
    return x if isinstance(x, np.ndarray) else as_np(x)


def check(o_gpu, o_ref, S_gpu=None, S_ref=None):
    from oracle import rel_max
    if o_gpu is not None:
        eo = rel_max(_np(o_gpu).reshape(o_ref.shape), o_ref)
        assert eo <= Y_TOL, f"y max-rel {eo:.3e}"
    if S_gpu is not None:
        es = rel_max(_np(S_gpu).reshape(S_ref.shape), S_ref)
        assert es <= S_TOL, f"state max-rel {es:.3e}"


def opcheck(op, args):
    # test_aot_dispatch_dynamic needs autograd support, which none of these inference ops registers
    torch.library.opcheck(op, args, test_utils=("test_schema", "test_autograd_registration", "test_faketensor"))


@pytest.mark.parametrize("final", [True, False])
@pytest.mark.parametrize("T", [1, 100])
def test_opcheck_wkv7_fwd(dev, K, T, final):
    say("opcheck wkv7_fwd", T, final)
    ops = operands(2, T, H8, seed=40 + T)
    h0 = torch.from_numpy((0.3 * np.random.default_rng(T).standard_normal((2, H8, 64, 64))).astype(np.float32)).to(dev)
    x = to_dev(ops, dev)
    opcheck(torch.ops.rwkv_next_amd.wkv7_fwd.default, (*x, h0, H8, 64, final))
    opcheck(torch.ops.rwkv_next.wkv7_fwd.default, (*x, h0[:0], H8, 64, final))


@pytest.mark.parametrize("case", ["decode", "ragged", "snapshots", "verify"])
def test_opcheck_wkv7_pool_(dev, K, case):
    import rwkv_next_amd.synth as synth
    say("opcheck wkv7_pool_", case)
    S_slots = 12
    pool = torch.from_numpy(synth.state_np((S_slots, H8, 64, 64), seed=50)).to(dev)
    cu = n_keep = fresh = snaps = None
    max_len, final = 0, True
    if case == "ragged":
        lens = [3, 1, 70, 0, 40]
        ops = operands(1, sum(lens), H8, seed=51)
        cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=dev)
        slots = torch.tensor([4, 0, 9, 2, 7], device=dev)
        fresh = torch.tensor([0, 1, 0, 0, 1], dtype=torch.uint8, device=dev)
        max_len = 70
    else:
        T = 1 if case == "decode" else 5
        ops = operands(3, T, H8, seed=52)
        slots = torch.tensor([5, 1, 10], device=dev)
        if case == "snapshots":
            snaps = torch.zeros(3, T, H8, 64, 64, device=dev)
            final = False
        if case == "verify":
            n_keep = torch.tensor([2, 5, 0], device=dev)
    args = (*to_dev(ops, dev), pool, slots, H8, 64, cu, n_keep, fresh, final, True, snaps, None, max_len, 0, -1)
    opcheck(torch.ops.rwkv_next_amd.wkv7_pool_.default, args)


def test_opcheck_wkv7_replay_(dev, K):
    say("opcheck wkv7_replay_")
    ops = operands(4, 4, H8, seed=99)
    st = torch.from_numpy((0.3 * np.random.default_rng(2).standard_normal((4, H8, 64, 64))).astype(np.float32)).to(dev)
    n = torch.tensor([1, 2, 4, 3], device=dev)
    opcheck(torch.ops.rwkv_next_amd.wkv7_replay_.default, (*to_dev(ops, dev), st, n, H8, 64))


def test_registered_ops_reject_strided_or_misshaped_buffers(dev, K):
    """The registered ops pass raw pointers to the C ABI, so they check their own buffers: a transposed state, a
    strided pool, a wrong-dtype slot index or a mis-shaped snapshot buffer raises ValueError before any launch, and
    the buffers are left untouched."""
    say("registered ops validate buffers")
    B, T = 3, 4
    x = to_dev(operands(B, T, H8, seed=71), dev)
    st = torch.randn(B, H8, 64, 64, device=dev)
    st_t = st.transpose(2, 3)  # same shape, not contiguous
    before = st.clone()
    nk = torch.tensor([1, 2, 4], device=dev)
    with pytest.raises(ValueError, match="state"):
        torch.ops.rwkv_next_amd.wkv7_replay_(*x, st_t, nk, H8, 64)
    with pytest.raises(ValueError, match="state"):
        torch.ops.rwkv_next_amd.wkv7_replay_(*x, st[:2], nk, H8, 64)
    with pytest.raises(ValueError, match="n_keep"):
        torch.ops.rwkv_next_amd.wkv7_replay_(*x, st, nk.to(torch.int32), H8, 64)
    pool = torch.randn(8, H8, 64, 64, device=dev)
    slots = torch.tensor([5, 1, 2], device=dev)
    common = (H8, 64, None, None, None, True, True)
    with pytest.raises(ValueError, match="pool"):
        torch.ops.rwkv_next_amd.wkv7_pool_(*x, pool.transpose(2, 3), slots, *common, None, None, T, 0, -1)
    with pytest.raises(ValueError, match="slots"):
        torch.ops.rwkv_next_amd.wkv7_pool_(*x, pool, slots.to(torch.int32), *common, None, None, T, 0, -1)
    snaps = torch.zeros(B, T, H8, 64, 64, device=dev).transpose(3, 4)
    with pytest.raises(ValueError, match="snapshots"):
        torch.ops.rwkv_next_amd.wkv7_pool_(*x, pool, slots, H8, 64, None, None, None, False, True, snaps, None, T,
                                           0, -1)
    torch.cuda.synchronize()
    assert torch.equal(st, before)


@pytest.mark.parametrize("B,T,use_s0", [(3, 1, True), (2, 4, True), (2, 300, False), (1, 300, True)])
def test_reference_cases_compiled(dev, K, B, T, use_s0):
    """tools/test_wkv7.py:50-54: every dense case also through torch.compile(lambda *x: wkv7(*x, s0, H, K))."""
    from oracle import wkv7_ref
    say("compiled", B, T, use_s0)
    ops = operands(B, T, H8, seed=B * 1000 + T)
    s0np = (0.3 * np.random.default_rng(B + T).standard_normal((B, H8, 64, 64))).astype(np.float32) if use_s0 else None
    o_ref, S_ref, _ = wkv7_ref(*np_list(ops), s0np)
    s0 = torch.from_numpy(s0np).to(dev) if use_s0 else None
    torch._dynamo.reset()
    fn = torch.compile(lambda *x: K.wkv7(*x, s0, H8, 64), dynamic=False)
    o, S = fn(*to_dev(ops, dev))
    torch.cuda.synchronize()
    check(o, o_ref, S, S_ref)
    o_e, S_e = K.wkv7(*to_dev(ops, dev), s0, H8, 64)
    torch.cuda.synchronize()
    assert torch.equal(o, o_e) and torch.equal(S, S_e)


def _part_att(K, H):
    """The WKV part of Layer.part_att (rwkv_next/model.py:142-158) reduced to what touches the state: operand
    views of one projection, the in-place pool recurrence, then an elementwise consumer of o."""
    def fn(xr, xw, xk, xv, xa, xb, pool, slots):
        # exact elementwise work on either side (a power-of-two scale), so compiled and eager agree bit for bit
        k = (xk.float() * 0.5).to(torch.bfloat16)
        o = K.wkv7_pool_(xr, xw, k, xv, xa, xb, pool, slots, H, 64)
        return o.float() * 2.0
    return fn


def test_compiled_part_att_no_graph_break_and_graph_replay(dev, K):
    import rwkv_next_amd.synth as synth
    say("compiled part_att")
    B, H, S_slots = 6, H8, 16
    ops = operands(B, 1, H, seed=61)
    x = to_dev(ops, dev)
    pool0 = torch.from_numpy(synth.state_np((S_slots, H, 64, 64), seed=62)).to(dev)
    slots = torch.tensor([3, 9, 0, 14, 7, 11], device=dev)
    fn = _part_att(K, H)
    torch._dynamo.reset()
    expl = torch._dynamo.explain(fn)(*x, pool0.clone(), slots)
    assert expl.graph_break_count == 0, expl.break_reasons
    assert expl.graph_count == 1
    torch._dynamo.reset()
    cfn = torch.compile(fn, dynamic=False)
    p_eager, p_comp = pool0.clone(), pool0.clone()
    y_eager = fn(*x, p_eager, slots)
    y_comp = cfn(*x, p_comp, slots)
    torch.cuda.synchronize()
    assert torch.equal(y_eager, y_comp) and torch.equal(p_eager, p_comp)
    # capture the compiled step in a graph (warm-up on a side stream first, as model.py:420-440 does)
    p_graph = pool0.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            cfn(*x, p_graph.clone(), slots)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y_static = cfn(*x, p_graph, slots)
    p_ref = pool0.clone()
    for rep in range(3):  # each replay advances the pool one step; eager work and syncs in between
        p_ref_y = fn(*x, p_ref, slots)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(p_graph, p_ref), rep
        assert torch.equal(y_static, p_ref_y), rep


def test_status_word_reports_bad_slots_without_fault(dev, K):
    """One slot index outside the pool: the kernels skip that state (zero initial state, no store), set the status
    bits, and every other row is exact; in-range calls leave the word at zero."""
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    from rwkv_next_amd import _lib
    B, T, S_slots = 4, 3, 8
    say("status word")
    ops = operands(B, T, H8, seed=71)
    pool0 = synth.state_np((S_slots, H8, 64, 64), seed=72)
    x = to_dev(ops, dev)
    status = K.new_status(dev)
    pool = torch.from_numpy(pool0).to(dev)
    K.wkv7_pool_(*x, pool, torch.tensor([1, 5, 2, 7], device=dev), H8, 64, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    K.check_status(status)
    bad = np.array([3, S_slots + 2, 0, 6], np.int64)   # row 1 points past the pool
    pool = torch.from_numpy(pool0).to(dev)
    o = K.wkv7_pool_(*x, pool, torch.from_numpy(bad).to(dev), H8, 64, status=status)
    torch.cuda.synchronize()
    bits = int(status.item())
    assert bits == (_lib.WKV7_STATUS_H0_SLOT | _lib.WKV7_STATUS_HT_SLOT), bits
    with pytest.raises(ValueError, match="outside the pool"):
        K.check_status(status)
    good = [0, 2, 3]
    o_ref, S_ref, _ = wkv7_ref(*[t[good] for t in np_list(ops)], pool0[bad[good]])
    check(as_np(o)[good], o_ref, as_np(pool)[bad[good]], S_ref)
    untouched = np.setdiff1d(np.arange(S_slots), bad[good])
    assert np.array_equal(as_np(pool)[untouched], pool0[untouched])
    # the bad row ran from a zero state (its output is the zero-state recurrence)
    o1_ref, _, _ = wkv7_ref(*[t[1:2] for t in np_list(ops)], None)
    check(as_np(o)[1:2], o1_ref)
    # a negative n_keep and a malformed cu_seqlens are reported the same way
    status.zero_()
    pool = torch.from_numpy(pool0).to(dev)
    K.wkv7_pool_(*x, pool, torch.tensor([1, 5, 2, 7], device=dev), H8, 64, n_keep=torch.tensor([3, -1, 2, 1], device=dev),
                 store_o=False, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == _lib.WKV7_STATUS_NKEEP
    status.zero_()
    lens_cu = torch.tensor([0, 2, 1, 3], dtype=torch.int32, device=dev)  # decreasing entry
    flat = [t.reshape(1, B * T, -1)[:, :3].contiguous() for t in x]
    K.wkv7_pool_(*flat, pool, torch.tensor([1, 5, 2], device=dev), H8, 64, cu_seqlens=lens_cu, max_len=3,
                 status=status)
    torch.cuda.synchronize()
    assert int(status.item()) & _lib.WKV7_STATUS_SEQLENS


def test_status_word_reports_slot_clashes(dev, K):
    """Two rows of an in-place pool call on one slot set WKV7_STATUS_SLOT_CLASH, and so does, with h0 and ht one
    pool, a row storing where another reads its initial state; distinct slots, a row reading and writing its own
    slot, and fresh rows reading nothing leave the word at zero.  Every kernel exits normally."""
    from rwkv_next_amd import _lib
    import rwkv_next_amd.synth as synth
    B, T, S_slots = 4, 2, 8
    say("status word, slot clashes")
    ops = operands(B, T, H8, seed=75)
    x = to_dev(ops, dev)
    pool0 = synth.state_np((S_slots, H8, 64, 64), seed=76)
    status = K.new_status(dev)
    K.wkv7_pool_(*x, torch.from_numpy(pool0).to(dev), torch.tensor([6, 1, 4, 3], device=dev), H8, 64, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    K.wkv7_pool_(*x, torch.from_numpy(pool0).to(dev), torch.tensor([6, 1, 6, 3], device=dev), H8, 64, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == _lib.WKV7_STATUS_SLOT_CLASH
    with pytest.raises(ValueError, match="share a state slot"):
        K.check_status(status)
    # the C ABI with separate index lists on one pool: row 2 stores into slot 5, which row 0 reads from (unless row 0
    # starts fresh)
    import importlib
    W = importlib.import_module("rwkv_next_amd.kernels.wkv7")  # the package re-exports the function of that name
    pool = torch.from_numpy(pool0).to(dev)
    h0_idx = torch.tensor([5, 1, 2, 3], device=dev)
    ht_idx = torch.tensor([0, 1, 5, 3], device=dev)
    ops_p, Bp, Tp = W._prep_operands(*x, H8, 64)
    for fresh0, expect in ((False, _lib.WKV7_STATUS_SLOT_CLASH), (True, 0)):
        status.zero_()
        fresh = torch.tensor([fresh0, False, False, False], device=dev, dtype=torch.uint8)
        W._launch(ops_p, H=H8, num_seqs=Bp, T=Tp, total=Bp * Tp, o=torch.empty_like(ops_p[3]), h0=pool,
                  h0_idx=h0_idx, h0_rows=S_slots, ht=pool, ht_idx=ht_idx, ht_rows=S_slots, fresh=fresh,
                  status=status)
        torch.cuda.synchronize()
        assert int(status.item()) == expect, (fresh0, int(status.item()))
    # more rows than the check covers: not checked (no bit), and the call still runs
    n = _lib.WKV7_STATUS_CLASH_MAX_SEQS + 1
    big = operands(n, 1, H8, seed=77)
    status.zero_()
    slots = torch.arange(n, device=dev)
    slots[7] = 3
    K.wkv7_pool_(*to_dev(big, dev), torch.zeros(n, H8, 64, 64, device=dev), slots, H8, 64, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0


def test_status_word_reports_w_outside_the_chunked_range(dev, K):
    """A dense T = 100 call runs the chunked kernels: with the model's w (<= -0.5) the word stays zero; one w above
    WKV7_CHUNK_W_MAX sets WKV7_STATUS_DECAY (every kernel still exits normally); a token-serial call with the same w
    does not, since those kernels take any w, and its rows match the oracle."""
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    from rwkv_next_amd import _lib
    B, T, S_slots = 2, 100, 4
    say("status word, w range")
    ops = operands(B, T, H8, seed=73)
    pool0 = synth.state_np((S_slots, H8, 64, 64), seed=74)
    slots = torch.tensor([3, 0], device=dev)
    status = K.new_status(dev)
    x = to_dev(ops, dev)
    K.wkv7_pool_(*x, torch.from_numpy(pool0).to(dev), slots, H8, 64, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    w_hi = x[1].clone()
    w_hi[1, 57, 5] = 1.25                                            # one channel of one token of row 1
    xs = [x[0], w_hi] + list(x[2:])
    K.wkv7_pool_(*xs, torch.from_numpy(pool0).to(dev), slots, H8, 64, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == _lib.WKV7_STATUS_DECAY
    with pytest.raises(ValueError, match="ALGO_RECURRENT"):
        K.check_status(status)
    status.zero_()
    pool = torch.from_numpy(pool0).to(dev)
    o = K.wkv7_pool_(*xs, pool, slots, H8, 64, algo=_lib.ALGO_RECURRENT, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    npo = np_list(ops)
    npo[1] = as_np(w_hi).reshape(npo[1].shape).astype(npo[1].dtype)
    o_ref, S_ref, _ = wkv7_ref(*npo, pool0[[3, 0]])
    check(o, o_ref, as_np(pool)[[3, 0]], S_ref)


def test_status_w_check_covers_only_chunked_rows(dev, K):
    """In a ragged AUTO call, rows of at most 32 tokens run token-serial (any w); only the longer rows, within
    n_keep, are checked against WKV7_CHUNK_W_MAX.  w = 1.25 in a short row, or past a long row's n_keep, leaves the
    word zero and every result exact; the same w inside a long row sets WKV7_STATUS_DECAY."""
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    from rwkv_next_amd import _lib
    lens = [40, 7, 100, 1]
    n_keep = np.array([40, 7, 60, 1], np.int64)
    say("status word, w check on chunked rows only", lens)
    total = sum(lens)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    ops = operands(1, total, H8, seed=75)
    pool0 = synth.state_np((6, H8, 64, 64), seed=76)
    slots = np.array([4, 1, 5, 0], np.int64)
    x = to_dev(ops, dev)
    args = dict(cu_seqlens=torch.from_numpy(cu).to(dev), n_keep=torch.from_numpy(n_keep).to(dev), max_len=100)
    for tok, expect in ((40 + 3, 0), (47 + 80, 0), (47 + 10, _lib.WKV7_STATUS_DECAY)):
        w_hi = x[1].clone()
        w_hi[0, tok, 5] = 1.25  # head 5 of: row 1 (7 tokens), past row 2's n_keep, inside row 2's kept tokens
        xs = [x[0], w_hi] + list(x[2:])
        status = K.new_status(dev)
        pool = torch.from_numpy(pool0).to(dev)
        o = K.wkv7_pool_(*xs, pool, torch.from_numpy(slots).to(dev), H8, 64, status=status, **args)
        torch.cuda.synchronize()
        assert int(status.item()) == expect, (tok, int(status.item()))
        if expect == 0:
            npo = np_list(ops)
            npo[1] = as_np(w_hi).reshape(npo[1].shape).astype(npo[1].dtype)
            o_ref, pool_ref, _ = wkv7_ref(*npo, pool0, cu_seqlens=cu, state_idx=slots, n_keep=n_keep)
            keep = np.zeros(total, bool)
            for i in range(len(lens)):
                keep[cu[i]:cu[i] + min(lens[i], n_keep[i])] = True
            check(as_np(o).reshape(o_ref.shape)[:, keep], o_ref[:, keep], as_np(pool), pool_ref)
