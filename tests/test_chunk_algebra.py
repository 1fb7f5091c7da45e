"""The chunked form of the recurrence used by the HIP prefill kernels (rwkv-infer-next_amd/csrc/wkv7_chunked.hip),
evaluated in float64 numpy and checked against the CPU oracle.  This pins the algebra (which products, which
decay references, which masks, the blocked triangular inverse) independently of the GPU code: the GPU parity
tests then only have to show the HIP kernels compute these same products.

Per chunk (C tokens, initial state S0):  S_C = A S0 + F V,  O = Q S0 + E V  with
  A = Gamma + Bh^T W,  F = Bh^T G + Kh^T,  Q = R0 + rho W,  E = sigma + rho G,  [W | G] = (I - alpha)^{-1} [A0 | beta],
the last solved block by block (forward substitution with the inverses of the 16 x 16 diagonal blocks).
"""
import numpy as np

from oracle import rel_max, wkv7_ref

C = 64


def blocked_unit_lower_inverse(alpha):
    """(I - alpha)^{-1} for strictly lower alpha (64 x 64) the way the prep kernel computes it: 16 x 16 diagonal
    blocks by forward substitution, then block rows  T_ij = T_ii sum_{j<=k<i} alpha_ik T_kj."""
    n = alpha.shape[0]
    nb = n // 16
    T = np.zeros_like(alpha)
    for d in range(nb):
        D = alpha[16 * d:16 * d + 16, 16 * d:16 * d + 16]
        Td = np.eye(16)
        for r in range(16):
            for c in range(r):
                Td[r, c] = D[r, c] + sum(D[r, k] * Td[k, c] for k in range(c + 1, r))
        T[16 * d:16 * d + 16, 16 * d:16 * d + 16] = Td
    for bi in range(1, nb):
        for bj in range(bi):
            Z = sum(alpha[16 * bi:16 * bi + 16, 16 * k:16 * k + 16] @ T[16 * k:16 * k + 16, 16 * bj:16 * bj + 16]
                    for k in range(bj, bi))
            T[16 * bi:16 * bi + 16, 16 * bj:16 * bj + 16] = T[16 * bi:16 * bi + 16, 16 * bi:16 * bi + 16] @ Z
    return T


def block_forward_substitution(alpha, B):
    """X = (I - alpha)^{-1} B for strictly lower alpha (64 x 64) the way the prep kernel solves for W and G: 16-row
    blocks in order, X_i = T_ii (B_i + sum_{j<i} alpha_ij X_j), with T_ii the inverse of the diagonal block."""
    X = np.zeros_like(B)
    for bi in range(4):
        rows = slice(16 * bi, 16 * bi + 16)
        acc = B[rows].copy()
        for bj in range(bi):
            acc += alpha[rows, 16 * bj:16 * bj + 16] @ X[16 * bj:16 * bj + 16]
        X[rows] = np.linalg.inv(np.eye(16) - alpha[rows, rows]) @ acc
    return X


def chunk_prep(r, w, k, v, a, b):
    """One chunk of one head; inputs [L, 64] (L <= C) -> (A, H = F V, Q, O_intra = E V)."""
    L = r.shape[0]
    pad = lambda x: np.vstack([x, np.zeros((C - L, x.shape[1]))])
    r, k, v, a, b = (pad(x.astype(np.float64)) for x in (r, k, v, a, b))
    lam = pad(-np.exp(w.astype(np.float64)))                    # padded rows: identity steps
    g = np.cumsum(lam, axis=0)
    g_ex = np.vstack([np.zeros((1, g.shape[1])), g[:-1]])
    m, gL = g[31], g[-1]
    Aq, Rq = a * np.exp(g_ex - m), r * np.exp(g - m)
    Bk, Kk = b * np.exp(m - g), k * np.exp(m - g)
    alpha, beta = np.tril(Aq @ Bk.T, -1), np.tril(Aq @ Kk.T, -1)
    rho, sigma = np.tril(Rq @ Bk.T), np.tril(Rq @ Kk.T)
    A0, R0 = Aq * np.exp(m), Rq * np.exp(m)
    Bh, Kh = Bk * np.exp(gL - m), Kk * np.exp(gL - m)
    X = block_forward_substitution(alpha, np.hstack([A0, beta]))
    W, G = X[:, :64], X[:, 64:]
    Q, E = R0 + rho @ W, sigma + rho @ G
    A = np.diag(np.exp(gL)) + Bh.T @ W
    F = Bh.T @ G + Kh.T
    return A, F @ v, Q, E @ v


def chunked_run(r, w, k, v, a, b, s0):
    """One head: inputs [T, 64], s0 [64, 64] -> (o [T, 64], S [64, 64])."""
    T_ = r.shape[0]
    S = s0.astype(np.float64).copy()
    o = np.zeros((T_, 64))
    for c0 in range(0, T_, C):
        sl = slice(c0, min(T_, c0 + C))
        A, Hm, Q, Oi = chunk_prep(r[sl], w[sl], k[sl], v[sl], a[sl], b[sl])
        o[sl] = (Q @ S + Oi)[:sl.stop - sl.start]
        S = A @ S + Hm
    return o, S


def test_blocked_inverse_matches_dense_inverse():
    rng = np.random.default_rng(0)
    alpha = np.tril(0.3 * rng.standard_normal((64, 64)), -1)
    T = blocked_unit_lower_inverse(alpha)
    assert rel_max(T @ (np.eye(64) - alpha), np.eye(64)) < 1e-12


def test_block_forward_substitution_matches_dense_solve():
    rng = np.random.default_rng(1)
    alpha = np.tril(0.3 * rng.standard_normal((64, 64)), -1)
    B = rng.standard_normal((64, 128))
    X = block_forward_substitution(alpha, B)
    assert rel_max(X, np.linalg.solve(np.eye(64) - alpha, B)) < 1e-12
    assert rel_max(X, blocked_unit_lower_inverse(alpha) @ B) < 1e-12


def test_chunked_form_reproduces_the_recurrence():
    import rwkv_next_amd.synth as synth
    T_, H = 200, 2                                              # chunks of 64, 64, 64 and 8 tokens
    ops = synth.operands_np((1, T_, H, 64), seed=7)
    ins = [ops[n] for n in synth.OPERAND_NAMES]
    s0 = synth.state_np((1, H, 64, 64), seed=8, std=0.3)
    o_ref, S_ref, _ = wkv7_ref(*ins, s0)
    for h in range(H):
        o, S = chunked_run(*(x[0, :, h] for x in ins), s0[0, h])
        assert rel_max(S, S_ref[0, h]) < 1e-11
        assert rel_max(o, o_ref[0, :, h]) < 1e-11


def test_chunk_factors_stay_bounded_for_model_decays():
    """With |log d| < 0.61 per token (w < -0.5), the midpoint-referenced factors stay below e^{20}, far inside fp32."""
    w = np.full((C, 64), -0.5)
    g = np.cumsum(-np.exp(w), axis=0)
    m = g[31]
    assert np.max(np.abs(g - m)) < 20.0


def chunk_prep_fp32(r, w, k, v, a, b):
    """chunk_prep in float32 (the kernels' range: bf16 hi/lo splits carry fp32's exponent range); the triangular
    solve stays float64 (only the range of the midpoint-referenced factors is at stake here)."""
    f = np.float32
    L = r.shape[0]
    pad = lambda x: np.vstack([x.astype(f), np.zeros((C - L, x.shape[1]), f)])
    r, k, v, a, b = (pad(x) for x in (r, k, v, a, b))
    lam = pad(-np.exp(w.astype(f)))
    g = np.cumsum(lam, axis=0, dtype=f)
    g_ex = np.vstack([np.zeros((1, g.shape[1]), f), g[:-1]])
    m, gL = g[31], g[-1]
    with np.errstate(over="ignore", invalid="ignore"):
        Aq, Rq = a * np.exp(g_ex - m), r * np.exp(g - m)
        Bk, Kk = b * np.exp(m - g), k * np.exp(m - g)
        alpha, beta = np.tril(Aq @ Bk.T, -1), np.tril(Aq @ Kk.T, -1)
        rho, sigma = np.tril(Rq @ Bk.T), np.tril(Rq @ Kk.T)
        A0, R0 = Aq * np.exp(m), Rq * np.exp(m)
        Bh, Kh = Bk * np.exp(gL - m), Kk * np.exp(gL - m)
        X = block_forward_substitution(alpha.astype(np.float64), np.hstack([A0, beta]).astype(np.float64)).astype(f)
        W, G = X[:, :64], X[:, 64:]
        Q, E = R0 + rho @ W, sigma + rho @ G
        A = np.diag(np.exp(gL)) + Bh.T @ W
        F = Bh.T @ G + Kh.T
    return A, F @ v, Q, E @ v


def test_chunked_form_range_of_w():
    """WKV7_CHUNK_W_MAX = 1.0: with every w at the bound the fp32 chunk factors (up to exp(32 e^w) = e^87) stay finite
    and the chunked form matches the fp64 recurrence; just above it (w = 1.05: e^91 > FLT_MAX) they overflow."""
    import rwkv_next_amd.synth as synth
    from rwkv_next_amd import _lib
    assert 32 * np.exp(_lib.WKV7_CHUNK_W_MAX) < np.log(np.finfo(np.float32).max) < 32 * np.exp(1.05)
    T_ = 128
    ops = synth.operands_np((1, T_, 1, 64), seed=7)
    ins = [ops[n] for n in synth.OPERAND_NAMES]
    s0 = synth.state_np((1, 1, 64, 64), seed=8, std=0.3)
    for wv, ok in ((-0.5, True), (0.0, True), (0.5, True), (_lib.WKV7_CHUNK_W_MAX, True), (1.05, False)):
        x = list(ins)
        x[1] = np.full_like(ins[1], wv)
        o_ref, S_ref, _ = wkv7_ref(*x, s0)
        S = s0[0, 0].astype(np.float32)
        o = np.zeros((T_, 64), np.float32)
        for c0 in range(0, T_, C):
            sl = slice(c0, c0 + C)
            A, Hm, Q, Oi = chunk_prep_fp32(*(t[0, sl, 0] for t in x))
            o[sl] = Q @ S + Oi
            S = A @ S + Hm
        finite = bool(np.isfinite(S).all() and np.isfinite(o).all())
        assert finite == ok, wv
        if ok:
            assert rel_max(S, S_ref[0, 0]) < 1e-5 and rel_max(o, o_ref[0, :, 0]) < 1e-5, wv
