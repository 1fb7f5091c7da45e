"""Parity at the full sizes of the five benchmark configurations (seeded synthetic inputs, seed = 1000 +
config index):

  config 0  the reference's CPU-runnable case, B = 1, T = 512, H = 12 (fp32 on the CPU there; here the same
            operands rounded to bf16, the kernels' input type), on every algorithm
  config 1  batched decode: B = 64 of a 128-slot pool, H = 40, T = 1 (one layer slice)
  config 2  chunked prefill: B = 1, T = 4096, H = 64, chunk 64, fp32 state from zeros
  config 3  mixed step: 256-slot pool, H = 64, 8 prefill rows U[1, 2048] + 120 decode rows, packed varlen,
            captured in a HIP graph and replayed
  config 4  speculative verify: B = 64, T = 5, H = 64 with per-token snapshots [64, 5, 64, 64, 64]; rollback to a
            random accepted prefix must equal a re-run bit for bit
  TP share  one tensor-parallel rank's slice of the 7.2B model at TP 8 (H = 8 per GPU, rwkv_next/model.py:8-16,
            109-110): decode B = 64 (512 pairs, occupancy-limited) and the T = 5 verify with snapshots

Tolerances: y <= 2e-2 and state <= 1e-4 max-relative against the fp64 oracle on the same bf16-rounded inputs."""
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


def errs(o_gpu, o_ref, S_gpu, S_ref):
    from oracle import rel_max
    eo = rel_max(as_np(o_gpu).reshape(o_ref.shape), o_ref) if o_gpu is not None else 0.0
    es = rel_max(as_np(S_gpu).reshape(S_ref.shape), S_ref) if S_gpu is not None else 0.0
    say(f"y max-rel {eo:.3e}  state max-rel {es:.3e}")
    return eo, es


@pytest.mark.parametrize("algo", [0, 1, 2])
def test_config0_B1_T512_H12(dev, K, algo):
    from oracle import wkv7_ref
    say("config 0", "algo", algo)
    H, T = 12, 512
    ops = operands(1, T, H, seed=1000)
    o_ref, S_ref, _ = wkv7_ref(*np_list(ops))
    o, S = K.wkv7(*to_dev(ops, dev), None, H, 64, algo=algo)
    torch.cuda.synchronize()
    eo, es = errs(o, o_ref, S, S_ref)
    assert eo <= Y_TOL and es <= S_TOL


def test_config1_decode(dev, K):
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    say("config 1")
    H, S_slots, B = 40, 128, 64
    ops = operands(B, 1, H, seed=1001)
    pool0 = synth.state_np((S_slots, H, 64, 64), seed=1101)
    slots = np.random.default_rng(1201).permutation(S_slots)[:B].astype(np.int64)
    o_ref, pool_ref, _ = wkv7_ref(*np_list(ops), pool0, state_idx=slots)
    pool = torch.from_numpy(pool0).to(dev)
    o = K.wkv7_pool_(*to_dev(ops, dev), pool, torch.from_numpy(slots).to(dev), H, 64)
    torch.cuda.synchronize()
    eo, es = errs(o, o_ref, pool, pool_ref)
    assert eo <= Y_TOL and es <= S_TOL


@pytest.mark.parametrize("B,S_slots", [(64, 128), (56, 128), (128, 160)])
def test_headline_decode_grouped_kernel(dev, K, B, S_slots):
    """The metric's decode shape (H = 64, B = 64 of a 128-slot pool: 4096 pairs) and two others that take the
    grouped single-token kernel (at least three pairs per SIMD): a partial last group (3584 pairs) and two groups
    per wave (8192 pairs).  The whole pool is compared, so slots outside the batch must come back untouched."""
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    H = 64
    say("decode grouped", dict(B=B, S=S_slots, H=H))
    ops = operands(B, 1, H, seed=1001 + B)
    pool0 = synth.state_np((S_slots, H, 64, 64), seed=1101 + B)
    slots = np.random.default_rng(1201 + B).permutation(S_slots)[:B].astype(np.int64)
    o_ref, pool_ref, _ = wkv7_ref(*np_list(ops), pool0, state_idx=slots)
    pool = torch.from_numpy(pool0).to(dev)
    o = K.wkv7_pool_(*to_dev(ops, dev), pool, torch.from_numpy(slots).to(dev), H, 64)
    torch.cuda.synchronize()
    eo, es = errs(o, o_ref, pool, pool_ref)
    assert eo <= Y_TOL and es <= S_TOL
    untouched = np.setdiff1d(np.arange(S_slots), slots)
    assert np.array_equal(as_np(pool)[untouched], pool0[untouched])


def test_grouped_decode_fresh_rows_snapshots_and_no_write_back(dev, K):
    """The grouped single-token kernel (4096 pairs) with fresh rows (zero initial state), a T = 1 snapshot and
    final=False: outputs match the oracle, the snapshot equals the updated state, and the pool is not written."""
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    B, S_slots, H = 64, 128, 64
    say("decode grouped fresh/snapshot/final=False", dict(B=B, H=H))
    ops = operands(B, 1, H, seed=1301)
    pool0 = synth.state_np((S_slots, H, 64, 64), seed=1302)
    slots = np.random.default_rng(1303).permutation(S_slots)[:B].astype(np.int64)
    fresh = np.zeros(B, bool)
    fresh[::5] = True
    h0 = pool0[slots].copy()
    h0[fresh] = 0.0
    o_ref, S_ref, _ = wkv7_ref(*np_list(ops), h0)
    pool = torch.from_numpy(pool0).to(dev)
    snaps = torch.empty(B, 1, H, 64, 64, device=dev)
    o = K.wkv7_pool_(*to_dev(ops, dev), pool, torch.from_numpy(slots).to(dev), H, 64,
                     fresh=torch.from_numpy(fresh).to(dev), final=False, snapshots=snaps)
    torch.cuda.synchronize()
    eo, es = errs(o, o_ref, snaps[:, 0], S_ref)
    assert eo <= Y_TOL and es <= S_TOL
    assert np.array_equal(as_np(pool), pool0)


@pytest.mark.parametrize("algo", [4, 2, 1])
def test_config2_prefill_T4096(dev, K, algo):
    from oracle import wkv7_ref
    say("config 2", "algo", algo)
    H, T = 64, 4096
    ops = operands(1, T, H, seed=1002)
    o_ref, S_ref, _ = wkv7_ref(*np_list(ops))
    o, S = K.wkv7(*to_dev(ops, dev), None, H, 64, algo=algo)
    torch.cuda.synchronize()
    eo, es = errs(o, o_ref, S, S_ref)
    assert eo <= Y_TOL and es <= S_TOL


def config3_batch(seed=1003):
    rng = np.random.default_rng(seed)
    lens = [int(x) for x in rng.integers(1, 2049, size=8)] + [1] * 120
    order = rng.permutation(len(lens))
    lens = [lens[i] for i in order]
    slots = rng.permutation(256)[:len(lens)].astype(np.int64)
    return lens, slots


def test_config3_mixed_step_in_graph(dev, K):
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    say("config 3")
    H = 64
    lens, slots = config3_batch()
    total = int(sum(lens))
    ops = operands(1, total, H, seed=1003)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    pool0 = synth.state_np((256, H, 64, 64), seed=1103)
    o_ref, pool_ref, _ = wkv7_ref(*np_list(ops), pool0, cu_seqlens=cu, state_idx=slots)

    x = [t.clone() for t in to_dev(ops, dev)]
    cu_d = torch.from_numpy(cu).to(dev)
    sl_d = torch.from_numpy(slots).to(dev)
    pool = torch.from_numpy(pool0).to(dev)
    # warm-up on a scratch pool, capture, then replay on the real pool
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        K.wkv7_pool_(*x, pool.clone(), sl_d, H, 64, cu_seqlens=cu_d, max_len=2048)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    scratch = pool.clone()
    with torch.cuda.graph(g):
        o_static = K.wkv7_pool_(*x, scratch, sl_d, H, 64, cu_seqlens=cu_d, max_len=2048)
    torch.cuda.synchronize()
    scratch.copy_(pool)
    g.replay()
    torch.cuda.synchronize()
    eo, es = errs(o_static, o_ref, scratch, pool_ref)
    assert eo <= Y_TOL and es <= S_TOL


def test_config4_verify_snapshots_rollback(dev, K):
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    say("config 4")
    B, T, H = 64, 5, 64
    ops = operands(B, T, H, seed=1004)
    pool0 = synth.state_np((B, H, 64, 64), seed=1104)
    slots = torch.arange(B, device=dev)
    x = to_dev(ops, dev)
    pool = torch.from_numpy(pool0).to(dev)
    snaps = torch.empty(B, T, H, 64, 64, device=dev)
    o = K.wkv7_pool_(*x, pool, slots, H, 64, final=False, snapshots=snaps)
    n = torch.from_numpy(np.random.default_rng(1204).integers(0, 5, size=B) + 1).to(dev)  # accepted j in 0..4
    K.restore_snapshots_(pool, slots, snaps, n)
    rerun = torch.from_numpy(pool0).to(dev)
    K.wkv7_pool_(*x, rerun, slots, H, 64, n_keep=n, store_o=False)
    torch.cuda.synchronize()
    assert torch.equal(pool, rerun)
    o_ref, _, snap_ref = wkv7_ref(*np_list(ops), pool0, snapshots=True)
    eo, es = errs(o, o_ref, snaps, snap_ref)
    assert eo <= Y_TOL and es <= S_TOL


@pytest.mark.parametrize("H", [64, 8])
def test_config4_snapshots_equal_decode_steps(dev, K, H):
    """Rollback bit-identity does not depend on which kernel re-runs the accepted tokens: the verify's snapshot
    after token t (token-serial kernel) equals, bit for bit, the state after t + 1 dense single-token wkv7_pool_ calls
    (a decode kernel), and each decode step's output equals the verify's output of that token.  B = 64: H = 64 runs
    the decode kernel with eight units per wave, H = 8 the small-launch decode kernel (scalar index loads)."""
    import rwkv_next_amd.synth as synth
    say("config 4: snapshots vs decode steps", H)
    B, T = 64, 5
    ops = operands(B, T, H, seed=1014)
    pool0 = synth.state_np((B, H, 64, 64), seed=1114)
    slots = torch.arange(B, device=dev)
    x = to_dev(ops, dev)
    snaps = torch.empty(B, T, H, 64, 64, device=dev)
    o_verify = K.wkv7_pool_(*x, torch.from_numpy(pool0).to(dev), slots, H, 64, final=False, snapshots=snaps)
    step = torch.from_numpy(pool0).to(dev)
    for t in range(T):
        xt = [v[:, t:t + 1].contiguous() for v in x]
        o_t = K.wkv7_pool_(*xt, step, slots, H, 64)
        torch.cuda.synchronize()
        assert torch.equal(step, snaps[:, t]), f"state after decode step {t} differs from the verify snapshot"
        assert torch.equal(o_t[:, 0], o_verify[:, t]), f"decode step {t} output differs from the verify output"


def test_tp_share_H8_decode(dev, K):
    """One TP-8 rank of the 7.2B model: H = 8, B = 64 of a 128-slot pool, T = 1 (512 pairs); untouched slots stay
    bit-identical."""
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    H, S_slots, B = 8, 128, 64
    say("TP share decode", dict(B=B, H=H))
    ops = operands(B, 1, H, seed=1008)
    pool0 = synth.state_np((S_slots, H, 64, 64), seed=1108)
    slots = np.random.default_rng(1208).permutation(S_slots)[:B].astype(np.int64)
    o_ref, pool_ref, _ = wkv7_ref(*np_list(ops), pool0, state_idx=slots)
    pool = torch.from_numpy(pool0).to(dev)
    o = K.wkv7_pool_(*to_dev(ops, dev), pool, torch.from_numpy(slots).to(dev), H, 64)
    torch.cuda.synchronize()
    eo, es = errs(o, o_ref, pool, pool_ref)
    assert eo <= Y_TOL and es <= S_TOL
    untouched = np.setdiff1d(np.arange(S_slots), slots)
    assert np.array_equal(as_np(pool)[untouched], pool0[untouched])


def test_tp_share_H8_verify_rollback(dev, K):
    """The same rank's speculative verify (B = 64, T = 5, H = 8) with snapshots; rollback equals a re-run bit for
    bit."""
    from oracle import wkv7_ref
    import rwkv_next_amd.synth as synth
    B, T, H, S_slots = 64, 5, 8, 128
    say("TP share verify", dict(B=B, T=T, H=H))
    ops = operands(B, T, H, seed=1009)
    pool0 = synth.state_np((S_slots, H, 64, 64), seed=1109)
    slots_np = np.random.default_rng(1209).permutation(S_slots)[:B].astype(np.int64)
    slots = torch.from_numpy(slots_np).to(dev)
    x = to_dev(ops, dev)
    pool = torch.from_numpy(pool0).to(dev)
    snaps = torch.empty(B, T, H, 64, 64, device=dev)
    o = K.wkv7_pool_(*x, pool, slots, H, 64, final=False, snapshots=snaps)
    n = torch.from_numpy(np.random.default_rng(1210).integers(0, 5, size=B) + 1).to(dev)
    K.restore_snapshots_(pool, slots, snaps, n)
    rerun = torch.from_numpy(pool0).to(dev)
    K.wkv7_pool_(*x, rerun, slots, H, 64, n_keep=n, store_o=False)
    torch.cuda.synchronize()
    assert torch.equal(pool, rerun)
    o_ref, _, snap_ref = wkv7_ref(*np_list(ops), pool0[slots_np], snapshots=True)
    eo, es = errs(o, o_ref, snaps, snap_ref)
    assert eo <= Y_TOL and es <= S_TOL
