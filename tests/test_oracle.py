"""Pins the CPU oracle (oracle/wkv7_oracle.cpp) against what the mathematics fixes, independently of how the
oracle is written: closed forms evaluated with numpy matmuls, a textbook decay value, an asymmetric elementary
row operation, explicit transition-matrix products, exact rational arithmetic on tiny inputs, and the invariants the
reference relies on (varlen == per-sequence, chunked prefill continuation, n_keep == prefix, snapshots == prefix
states, slot relabelling, value-column independence).

Reference semantics: rwkv_next/kernels/wkv7.py:4-7, 46-79; tools/test_wkv7.py:13-23.
"""
import numpy as np
import pytest

import oracle
from oracle import rel_max, wkv7_ref, wkv7_ref_numpy


def rnd(rng, *shape, scale=1.0):
    return (scale * rng.standard_normal(shape)).astype(np.float32)


def model_like(rng, B, T, H, K):
    """Operands in the model's ranges (rwkv_next/model.py:142-152), float32 (not rounded)."""
    r, k, v = rnd(rng, B, T, H, K), rnd(rng, B, T, H, K), rnd(rng, B, T, H, K)
    w = (-np.logaddexp(0.0, -2.0 * rnd(rng, B, T, H, K)) - 0.5).astype(np.float32)
    kap = rnd(rng, B, T, H, K)
    kap /= np.linalg.norm(kap, axis=-1, keepdims=True)
    gate = 1.0 / (1.0 + np.exp(-rnd(rng, B, T, H, K)))
    return r, w, k, v, (-kap).astype(np.float32), (kap * gate).astype(np.float32)


# ---------------------------------------------------------------------------------------------------------------
# closed forms
# ---------------------------------------------------------------------------------------------------------------
def test_pure_accumulation_is_cumulative_outer_products():
    """a = b = 0, d = 1 (w = -inf): S_T = S0 + K^T V and Y = R S0 + tril(R K^T) V."""
    rng = np.random.default_rng(1)
    B, T, H, K = 2, 9, 3, 16
    r, k, v = rnd(rng, B, T, H, K), rnd(rng, B, T, H, K), rnd(rng, B, T, H, K)
    w = np.full((B, T, H, K), -np.inf, np.float32)
    z = np.zeros_like(r)
    s0 = rnd(rng, B, H, K, K)
    o, S, _ = wkv7_ref(r, w, k, v, z, z, s0)
    for bb in range(B):
        for h in range(H):
            Kt, Vt, Rt = (x[bb, :, h].astype(np.float64) for x in (k, v, r))
            S_exp = s0[bb, h] + Kt.T @ Vt
            Y_exp = Rt @ s0[bb, h] + np.tril(Rt @ Kt.T) @ Vt
            assert rel_max(S[bb, h], S_exp) < 1e-12
            assert rel_max(o[bb, :, h], Y_exp) < 1e-12


def test_decayed_linear_attention_is_masked_matmul():
    """a = b = 0: y_t = (r_t e^{G_t})^T S0 + sum_{s<=t} (sum_k r_t k_s e^{G_t - G_s}) v_s, G = cumsum(-exp(w))."""
    rng = np.random.default_rng(2)
    T, H, K = 11, 2, 8
    r, w, k, v, _, _ = model_like(rng, 1, T, H, K)
    z = np.zeros_like(r)
    s0 = rnd(rng, 1, H, K, K)
    o, S, _ = wkv7_ref(r, w, k, v, z, z, s0)
    for h in range(H):
        G = np.cumsum(-np.exp(w[0, :, h].astype(np.float64)), axis=0)          # [T, K]
        Rt, Kt, Vt = (x[0, :, h].astype(np.float64) for x in (r, k, v))
        M = np.einsum("tk,sk,tsk->ts", Rt, Kt, np.exp(G[:, None, :] - G[None, :, :])) * np.tri(T)
        Y_exp = (Rt * np.exp(G)) @ s0[0, h] + M @ Vt
        S_exp = np.exp(G[-1])[:, None] * s0[0, h] + (Kt * np.exp(G[-1] - G)).T @ Vt
        assert rel_max(o[0, :, h], Y_exp) < 1e-11
        assert rel_max(S[0, h], S_exp) < 1e-11


def test_decay_is_exp_of_minus_exp_w():
    """k = v = a = b = 0 and w = log(log 2): every step halves the state (d = exp(-exp(w)) = 1/2)."""
    rng = np.random.default_rng(3)
    T, H, K = 5, 2, 8
    w = np.full((1, T, H, K), np.log(np.log(2.0)), np.float32)
    z = np.zeros_like(w)
    s0 = rnd(rng, 1, H, K, K)
    _, S, snap = wkv7_ref(z, w, z, z, z, z, s0, snapshots=True)
    # the float32 input w carries its own rounding: compare against d computed from that exact value
    d = np.exp(-np.exp(np.float64(w[0, 0, 0, 0])))
    assert abs(d - 0.5) < 1e-7
    for t in range(T):
        assert rel_max(snap[0, t], s0[0] * d ** (t + 1)) < 1e-14


def test_transition_is_a_projector_for_unit_kappa():
    """d = 1, a = -kappa, b = kappa, |kappa| = 1, k = v = 0: S <- (I - kappa kappa^T) S.  Idempotent, kills kappa."""
    rng = np.random.default_rng(4)
    H, K = 3, 16
    kap = rnd(rng, 1, 1, H, K)
    kap /= np.linalg.norm(kap, axis=-1, keepdims=True)
    a, b = np.repeat(-kap, 2, axis=1), np.repeat(kap, 2, axis=1)              # the same token twice
    w = np.full_like(a, -np.inf)
    z = np.zeros_like(a)
    s0 = rnd(rng, 1, H, K, K)
    _, _, snap = wkv7_ref(z, w, z, z, a, b, s0, snapshots=True)
    for h in range(H):
        kv = kap[0, 0, h].astype(np.float64)
        P = np.eye(K) - np.outer(kv, kv)
        assert rel_max(snap[0, 0, h], P @ s0[0, h]) < 1e-6                     # kappa rounded to fp32
        assert rel_max(snap[0, 1, h], snap[0, 0, h]) < 1e-6                    # idempotent
        assert np.max(np.abs(kv @ snap[0, 0, h])) < 1e-6 * np.max(np.abs(s0[0, h]))


def test_low_rank_term_orientation_is_b_times_aTS():
    """d = 1, k = v = 0, a = e_i, b = c e_j: S <- S + c e_j (e_i^T S), i.e. row j += c * row i (and only row j).
    A transposed a/b pair would change row i instead."""
    rng = np.random.default_rng(5)
    K, i, j, c = 8, 2, 5, 0.75
    a = np.zeros((1, 1, 1, K), np.float32)
    b = np.zeros_like(a)
    a[..., i] = 1.0
    b[..., j] = c
    w = np.full_like(a, -np.inf)
    z = np.zeros_like(a)
    s0 = rnd(rng, 1, 1, K, K)
    _, S, _ = wkv7_ref(z, w, z, z, a, b, s0)
    exp = s0[0, 0].astype(np.float64).copy()
    exp[j] += c * exp[i]
    assert rel_max(S[0, 0], exp) < 1e-14


@pytest.mark.parametrize("K", [16, 3, 48, 128])
def test_matches_explicit_transition_matrices(K):
    """S_t = (diag(d_t) + b_t a_t^T) S_{t-1} + k_t v_t^T and y_t = S_t^T r_t, evaluated with dense K x K matrices
    (head sizes other than 64 as well: the reference takes any K)."""
    rng = np.random.default_rng(6)
    B, T, H = 2, 7, 2
    r, w, k, v, a, b = model_like(rng, B, T, H, K)
    s0 = rnd(rng, B, H, K, K, scale=0.3)
    o, S, _ = wkv7_ref(r, w, k, v, a, b, s0)
    for bb in range(B):
        for h in range(H):
            St = s0[bb, h].astype(np.float64)
            for t in range(T):
                rt, wt, kt, vt, at, bt = (x[bb, t, h].astype(np.float64) for x in (r, w, k, v, a, b))
                A = np.diag(np.exp(-np.exp(wt))) + np.outer(bt, at)
                St = A @ St + np.outer(kt, vt)
                assert rel_max(o[bb, t, h], St.T @ rt) < 1e-12
            assert rel_max(S[bb, h], St) < 1e-12


@pytest.mark.parametrize("K", [64, 1, 24, 128, 256])
def test_cpp_matches_independent_numpy_transcription(K):
    rng = np.random.default_rng(7)
    B, T, H = 2, 13, 3
    ins = model_like(rng, B, T, H, K)
    s0 = rnd(rng, B, H, K, K, scale=0.3)
    o1, S1, _ = wkv7_ref(*ins, s0)
    o2, S2 = wkv7_ref_numpy(*ins, s0)
    assert rel_max(o1, o2) < 1e-12 and rel_max(S1, S2) < 1e-12


# ---------------------------------------------------------------------------------------------------------------
# invariants of the reference's call patterns
# ---------------------------------------------------------------------------------------------------------------
def test_varlen_equals_per_sequence_calls():
    """tools/test_wkv7.py:66-78: packed varlen with per-sequence initial states == separate calls."""
    rng = np.random.default_rng(8)
    H, K = 2, 64
    lens = [5, 1, 0, 37, 12]
    seqs = [model_like(rng, 1, L, H, K) for L in lens]
    s0 = rnd(rng, len(lens), H, K, K, scale=0.3)
    cat = [np.concatenate([s[j] for s in seqs], axis=1) for j in range(6)]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    o, S, _ = wkv7_ref(*cat, s0, cu_seqlens=cu)
    for n, L in enumerate(lens):
        o_n, S_n, _ = wkv7_ref(*seqs[n], s0[n:n + 1])
        assert np.array_equal(S[n], S_n[0])
        assert np.array_equal(o[:, cu[n]:cu[n + 1]], o_n)
    assert np.array_equal(S[2], s0[2].astype(np.float64))                     # L = 0: state carried through


def test_chunked_prefill_continuation_is_associative():
    """A non-fresh row continues its slot's state (model.py:382-383): run(T1) then run(T2) == run(T1 + T2)."""
    rng = np.random.default_rng(9)
    T1, T2, H, K = 17, 23, 2, 64
    ins = model_like(rng, 1, T1 + T2, H, K)
    s0 = rnd(rng, 1, H, K, K, scale=0.3)
    o, S, _ = wkv7_ref(*ins, s0, precision="f32")
    o1, S1, _ = wkv7_ref(*(x[:, :T1] for x in ins), s0, precision="f32")
    o2, S2, _ = wkv7_ref(*(x[:, T1:] for x in ins), S1, precision="f32")
    assert np.array_equal(S, S2)
    assert np.array_equal(o, np.concatenate([o1, o2], axis=1))


def test_n_keep_is_a_prefix_run_and_snapshots_are_prefix_states():
    """wkv7_replay semantics (wkv7.py:53-54, 141-147; test_wkv7.py:79-89) and the snapshot contract."""
    rng = np.random.default_rng(10)
    B, T, H, K = 4, 5, 2, 64
    ins = model_like(rng, B, T, H, K)
    s0 = rnd(rng, B, H, K, K, scale=0.3)
    n = np.array([1, 2, 5, 3], np.int64)
    _, S, _ = wkv7_ref(*ins, s0, n_keep=n, store_o=False)
    _, _, snap = wkv7_ref(*ins, s0, snapshots=True)
    for bb in range(B):
        _, Sp, _ = wkv7_ref(*(x[bb:bb + 1, :n[bb]] for x in ins), s0[bb:bb + 1])
        assert np.array_equal(S[bb], Sp[0])
        assert np.array_equal(snap[bb, n[bb] - 1], Sp[0])


def test_pool_mode_updates_only_the_given_slots():
    rng = np.random.default_rng(11)
    S_slots, B, T, H, K = 6, 3, 4, 2, 64
    ins = model_like(rng, B, T, H, K)
    pool = rnd(rng, S_slots, H, K, K, scale=0.1)
    slots = np.array([4, 0, 2], np.int64)
    o, newpool, _ = wkv7_ref(*ins, pool, state_idx=slots)
    o2, S2, _ = wkv7_ref(*ins, pool[slots])
    for i, s in enumerate(slots):
        assert np.array_equal(newpool[s], S2[i])
    for s in set(range(S_slots)) - set(slots.tolist()):
        assert np.array_equal(newpool[s], pool[s].astype(np.float64))
    assert np.array_equal(o, o2)


def test_permuting_slots_permutes_the_results():
    """Relabelling the pool's slots (pool'[pi(s)] = pool[s], indices pi(slots)) relabels the updated pool the same
    way and leaves the outputs unchanged."""
    rng = np.random.default_rng(12)
    S_slots, B, T, H, K = 7, 3, 3, 2, 16
    ins = model_like(rng, B, T, H, K)
    pool = rnd(rng, S_slots, H, K, K, scale=0.1)
    slots = np.array([5, 1, 3], np.int64)
    pi = rng.permutation(S_slots)
    pool_p = np.empty_like(pool)
    pool_p[pi] = pool
    o, new, _ = wkv7_ref(*ins, pool, state_idx=slots)
    o_p, new_p, _ = wkv7_ref(*ins, pool_p, state_idx=pi[slots])
    assert np.array_equal(o, o_p)
    assert np.array_equal(new_p[pi], new)


def test_value_columns_are_independent():
    """Column j of the state and of y depends only on column j of S0 and on v[..., j]: changing one value column
    (in v and in S0) changes exactly that column of every output."""
    rng = np.random.default_rng(13)
    B, T, H, K, j = 1, 6, 2, 16, 5
    r, w, k, v, a, b = model_like(rng, B, T, H, K)
    s0 = rnd(rng, B, H, K, K, scale=0.1)
    o, S, _ = wkv7_ref(r, w, k, v, a, b, s0)
    v2, s02 = v.copy(), s0.copy()
    v2[..., j] = rnd(rng, B, T, H)
    s02[..., j] = rnd(rng, B, H, K, scale=0.1)
    o2, S2, _ = wkv7_ref(r, w, k, v2, a, b, s02)
    others = [c for c in range(K) if c != j]
    assert np.array_equal(o[..., others], o2[..., others])
    assert np.array_equal(S[..., others], S2[..., others])
    assert not np.allclose(o[..., j], o2[..., j]) and not np.allclose(S[..., j], S2[..., j])


def test_exact_rational_brute_force_on_tiny_inputs():
    """T = 3, K = 4: the recurrence in exact rational arithmetic (the decays d = exp(-exp(w)) taken as the exact
    values of their float64 roundings) against the fp64 oracle; they agree to fp64 rounding."""
    from fractions import Fraction
    rng = np.random.default_rng(14)
    B, T, H, K = 2, 3, 2, 4
    r, w, k, v, a, b = model_like(rng, B, T, H, K)
    s0 = rnd(rng, B, H, K, K, scale=0.5)
    o, S, _ = wkv7_ref(r, w, k, v, a, b, s0)
    Fr = np.vectorize(lambda x: Fraction(float(x)), otypes=[object])
    d = Fr(np.exp(-np.exp(w.astype(np.float64))))
    R, Kk, V, A, Bb, St = Fr(r), Fr(k), Fr(v), Fr(a), Fr(b), Fr(s0)
    for n in range(B):
        for h in range(H):
            M = St[n, h].copy()                                        # M[k][j]
            for t in range(T):
                sa = [sum(A[n, t, h, i] * M[i, jj] for i in range(K)) for jj in range(K)]
                M = np.array([[d[n, t, h, i] * M[i, jj] + Bb[n, t, h, i] * sa[jj] + Kk[n, t, h, i] * V[n, t, h, jj]
                               for jj in range(K)] for i in range(K)], dtype=object)
                y = [sum(R[n, t, h, i] * M[i, jj] for i in range(K)) for jj in range(K)]
                for jj in range(K):
                    assert abs(float(y[jj]) - o[n, t, h, jj]) <= 1e-13 * (1 + abs(float(y[jj])))
            for i in range(K):
                for jj in range(K):
                    assert abs(float(M[i, jj]) - S[n, h, i, jj]) <= 1e-13 * (1 + abs(float(M[i, jj])))


def test_fp32_vs_fp64_gap_on_config0():
    """Calibrates the tolerances: the fp32 recurrence's own distance from fp64 on configuration 0
    (B=1, T=512, H=12; synthetic distributions).  The GPU is held to y <= 2e-2 and state <= 1e-4 (max-relative)."""
    import rwkv_next_amd.synth as synth
    ops = synth.operands_np((1, 512, 12, 64), seed=1000)
    ins = [ops[n] for n in synth.OPERAND_NAMES]
    o64, S64, _ = wkv7_ref(*ins)
    o32, S32, _ = wkv7_ref(*ins, precision="f32")
    assert rel_max(S32, S64) < 1e-5
    assert rel_max(o32, o64) < 1e-5


def test_metrics():
    x = np.array([1.0, 2.0, -4.0])
    assert oracle.rel_max(x, x) == 0.0
    assert abs(oracle.rel_max(x + 0.04, x) - 0.01) < 1e-15
    assert abs(oracle.rel_fro(2 * x, x) - 1.0) < 1e-15


def test_oracle_rejects_bad_head_size():
    z = np.zeros((1, 1, 1, 257), np.float32)
    with pytest.raises(ValueError):
        wkv7_ref(z, z, z, z, z, z)
