"""Pins of the CPU oracle (oracle/asa_oracle.c) against facts fixed outside it.

The reference ships no golden vectors or tests for this path, and its CUDA
source cannot be built here, so every function of the oracle is checked
against something independent of its own code:

  * top-k, mask, CSR   brute force (stable sort by (-score, index), numpy)
  * tau recurrence     hand-derived known answers: k = 1 and all-equal rows
                       (no step is ever taken), the single-real-key row whose
                       iteration is the closed-form map x -> x(x^2+7)/(5x^2+3)
                       for alpha = 1.5 (the reference's f'' coefficient; the
                       textbook Halley map would be x(2x^2+6)/(6x^2+2)), and
                       sparsemax / entmax-1.5 closed forms on converged rows
  * forward            a hand-computed row where a key outside the top-k but
                       inside an active block contributes; dense exact
                       alpha-entmax (bisection) when tau is exact and the
                       top-k holds the support
  * backward           central finite differences in fp64 of the map each
                       gradient claims to differentiate
Reference file: source/adasplashattention.cu (line numbers in the oracle).
"""
import numpy as np
import pytest

from oracle import dense as D
from oracle import oracle as orc


# ---------------------------------------------------------------- top-k / mask


def _brute_topk(S, vis, k):
    BH, NQ, NK = S.shape
    idx = np.full((BH, NQ, k), -1, np.int32)
    val = np.full((BH, NQ, k), -1e6, np.float64)
    for b in range(BH):
        for i in range(NQ):
            js = np.nonzero(vis[b, i])[0]
            order = np.lexsort((js, -S[b, i, js]))  # score desc, index asc
            js = js[order][:k]
            idx[b, i, :len(js)] = js
            val[b, i, :len(js)] = S[b, i, js]
    return idx, val


@pytest.mark.parametrize("kind", ["normal", "ties", "saturated", "sparse_visibility"])
def test_topk_matches_brute_force(kind):
    rng = np.random.default_rng({"normal": 1, "ties": 2, "saturated": 3, "sparse_visibility": 4}[kind])
    BH, NQ, NK, k = 2, 70, 150, 9
    if kind == "ties":
        S = np.round(rng.normal(size=(BH, NQ, NK)) * 2) / 2
    elif kind == "saturated":
        S = np.clip(rng.normal(size=(BH, NQ, NK)) * 30, -10, 10)
    else:
        S = rng.normal(size=(BH, NQ, NK))
    S = S.astype(np.float32)
    if kind == "sparse_visibility":
        vis = (rng.random((BH, NQ, NK)) < 0.03).astype(np.uint8)  # many rows with < k keys
    else:
        qi = np.broadcast_to(np.arange(NQ) + NK - NQ, (BH, NQ))
        vis = (np.arange(NK)[None, None, :] <= qi[:, :, None]).astype(np.uint8)
    sel = orc.select(S, vis, k, 1.5)
    idx, val = _brute_topk(S.astype(np.float64), vis, k)
    np.testing.assert_array_equal(sel.topk_idx, idx)
    np.testing.assert_array_equal(sel.topk_val.astype(np.float64), val)


@pytest.mark.parametrize("block_m", [64, 32])
def test_mask_and_csr_closed_form(block_m):
    """The mask is the union over each block_m rows of their top-k key
    blocks (adasplashattention.cu:210-216), the CSR its ascending lists."""
    rng = np.random.default_rng(5)
    BH, NQ, NK, k = 3, 200, 330, 5
    S = rng.normal(size=(BH, NQ, NK)).astype(np.float32)
    vis = np.ones((BH, NQ, NK), np.uint8)
    sel = orc.select(S, vis, k, 1.5, block_m=block_m)
    nQB, nKB = -(-NQ // block_m), -(-NK // 64)
    want = np.zeros((BH, nQB, nKB), np.uint8)
    for b in range(BH):
        for i in range(NQ):
            for j in sel.topk_idx[b, i]:
                if j >= 0:
                    want[b, i // block_m, j // 64] = 1
    np.testing.assert_array_equal(sel.mask, want)
    c = orc.csr(sel.mask)
    for b in range(BH):
        rows = [np.nonzero(want[b, i])[0] for i in range(nQB)]
        ptr = np.concatenate([[0], np.cumsum([len(r) for r in rows])])
        np.testing.assert_array_equal(c.q_ptr[b], ptr)
        lst = np.zeros(nQB * nKB, np.int32)
        lst[:ptr[-1]] = np.concatenate(rows)
        np.testing.assert_array_equal(c.q_list[b], lst)
        cols = [np.nonzero(want[b, :, j])[0] for j in range(nKB)]
        kptr = np.concatenate([[0], np.cumsum([len(r) for r in cols])])
        np.testing.assert_array_equal(c.k_ptr[b], kptr)
        klst = np.zeros(nQB * nKB, np.int32)
        klst[:kptr[-1]] = np.concatenate(cols)
        np.testing.assert_array_equal(c.k_list[b], klst)


# ---------------------------------------------------------------- tau


@pytest.mark.parametrize("alpha", [1.25, 1.5, 2.0, 2.7])
@pytest.mark.parametrize("prec", ["f32", "f64"])
def test_tau_no_step_cases(alpha, prec):
    """k = 1, or all kept values equal: the midpoint start puts tau at
    (alpha-1) s, every term has u = 0, f' = 0, so no step is taken."""
    am1 = np.float32(alpha) - np.float32(1) if prec == "f32" else alpha - 1
    for s in (3.0, -2.5, 0.0):
        assert orc.entmax_threshold([s], alpha, prec) == pytest.approx(float(am1 * s), abs=0)
        assert orc.entmax_threshold([s] * 6, alpha, prec) == pytest.approx(float(am1 * s), abs=0)


def _phi_quirk(x):
    return x * (x * x + 7.0) / (5.0 * x * x + 3.0)


def _phi_halley(x):
    return x * (2.0 * x * x + 6.0) / (6.0 * x * x + 2.0)


@pytest.mark.parametrize("s1", [0.0, 1.7, -3.2, 9.0])
def test_tau_single_real_key_follows_reference_f2_coefficient(s1):
    """One real key and k-1 empty slots (-1e6), alpha = 1.5.  Hand derivation:
    with x = z - tau, z = s1/2, only the real key contributes, f = x^2 - 1,
    f' = -2x, and the reference's f'' = a(a + 1 - alpha) = 3 (not 2), so each
    Halley step maps x to x(x^2 + 7)/(5x^2 + 3); the start is the bracket
    midpoint x0 = z/2 + 250000 and no step leaves the bracket."""
    z = 0.5 * s1
    x = z / 2 + 250000.0
    for _ in range(5):
        if abs(x * x - 1.0) < 1e-4:
            break
        x = _phi_quirk(x)
    want = z - x
    got = orc.entmax_threshold([s1] + [-1e6] * 7, 1.5, "f64")
    assert got == pytest.approx(want, rel=1e-12)
    # The textbook coefficient would land elsewhere (5 steps of x/5 vs x/3).
    xh = z / 2 + 250000.0
    for _ in range(5):
        xh = _phi_halley(xh)
    assert abs((z - xh) - got) > 100.0
    got32 = orc.entmax_threshold([s1] + [-1e6] * 7, 1.5, "f32")
    assert got32 == pytest.approx(want, rel=1e-5)


def test_tau_single_real_key_sparsemax():
    """alpha = 2: f'' coefficient is 0, Halley is Newton, one step lands on
    tau = s1 - 1 (sparsemax of one element)."""
    for s1 in (0.3, 4.0, -1.0):
        # the start is near -5e5, so rounding of that size is inherent
        assert orc.entmax_threshold([s1] + [-1e6] * 3, 2.0, "f64") == pytest.approx(s1 - 1.0, abs=1e-9)


def test_tau_known_answers_by_hand():
    # alpha = 2, s = [1, 0]: tau0 = 0.5, Newton to 0, f(0) = 0 -> exit.
    assert orc.entmax_threshold([1.0, 0.0], 2.0, "f64") == 0.0
    # alpha = 2, s = [1, 0.9]: tau0 = 0.95 -> 0 -> 0.45 (f = 0) -> exit.
    assert orc.entmax_threshold([1.0, 0.9], 2.0, "f64") == pytest.approx(0.45, abs=1e-15)


def test_tau_bisection_fallback_by_hand():
    """The step that leaves the bracket (cu:102-104).  s = [9, -2, -14],
    alpha = 1.5, so a = 2, z = s / 2 = (4.5, -1, -7), f = sum u^2 - 1 over
    u = z - tau > 0, f' = -2 sum u, and the reference's f'' = 3 per term.
    Bracket [lo, hi] = [-7 - 2, 4.5 + 2] = [-9, 6.5], start at its midpoint
    -1.25, where u = (5.75, 0.25): f = 32.125, f' = -12, f'' = 6, and the
    Halley step -1.25 + 2 * 32.125 * 12 / (2 * 144 - 6 * 32.125)
    = -1.25 + 3084/381 = 6.8445 lies above hi: the fallback takes the
    midpoint, -1.25 again; f > 0 there makes it lo.  The next round repeats
    the same step (same tau), which again leaves the bracket, and the
    fallback gives (-1.25 + 6.5) / 2 = 2.625, where one key is active,
    u = 15/8, f = 161/64 > 0 (lo).  The last three rounds are single-key
    Halley steps, the map x -> x (x^2 + 7) / (5 x^2 + 3) on u (pinned in
    test_tau_single_real_key_follows_reference_f2_coefficient), each inside
    the bracket, none with |f| < 1e-4: tau = 4.5 - phi(phi(phi(15/8)))."""
    from fractions import Fraction as Fr

    step0 = Fr(-5, 4) + Fr(3084, 381)
    assert step0 > Fr(13, 2)  # leaves the bracket: the fallback is taken
    x = Fr(15, 8)
    for _ in range(3):
        x = x * (x * x + 7) / (5 * x * x + 3)
    want = float(Fr(9, 2) - x)
    assert want == pytest.approx(3.5000000555768707, rel=1e-15)
    assert orc.entmax_threshold([9.0, -2.0, -14.0], 1.5, "f64") == pytest.approx(want, rel=1e-14)
    assert orc.entmax_threshold([9.0, -2.0, -14.0], 1.5, "f32") == pytest.approx(want, rel=1e-6)
    # Taking the step instead of the midpoint would leave no key active at
    # 6.8445 and the iteration would stop moving there.
    assert abs(float(step0) - want) > 3.0


@pytest.mark.parametrize("alpha,closed", [(2.0, D.tau_sparsemax), (1.5, D.tau_entmax15)])
def test_tau_converged_rows_match_closed_forms(alpha, closed):
    """When the recurrence stops on |f| < 1e-4 and the top-k holds the whole
    support, tau solves sum p = 1 up to that tolerance: compare with the
    sort-based closed form (and with bisection)."""
    rng = np.random.default_rng(11)
    checked = 0
    for _ in range(200):
        s = np.sort(rng.normal(size=16) * 1.5)[::-1]
        t = orc.entmax_threshold(s, alpha, "f64")
        p = np.maximum((alpha - 1) * s - t, 0) ** (1 / (alpha - 1))
        if abs(p.sum() - 1) >= 1e-4 or p[-1] > 0:
            continue  # not converged, or support reaches the last kept value
        checked += 1
        assert t == pytest.approx(closed(s), abs=2e-4)
        assert t == pytest.approx(D.tau_bisect(s, alpha), abs=2e-4)
    assert checked > 150


def test_tau_f32_and_f64_builds_agree():
    rng = np.random.default_rng(3)
    for alpha in (1.25, 1.5, 2.0, 1.7):
        for _ in range(50):
            s = np.sort(rng.normal(size=32))[::-1].astype(np.float32)
            a = orc.entmax_threshold(s, alpha, "f32")
            b = orc.entmax_threshold(s.astype(np.float64), alpha, "f64")
            assert a == pytest.approx(b, rel=2e-4, abs=2e-5)


# ---------------------------------------------------------------- forward


def test_forward_key_outside_topk_in_active_block_contributes():
    """alpha = 2, k = 2, one query, keys scoring 1.0, 0.9, 0.8 in one block.
    Top-2 = {1.0, 0.9}; by hand tau = 0.45 (see test above); the third key is
    not in the top-k but its block is active and u = 0.35 > 0, so
    out = (0.55 v0 + 0.45 v1 + 0.35 v2) / (1.35 + EPS) (adasplashattention.cu:297-328)."""
    d = 64
    Q = np.zeros((1, 1, d))
    Q[0, 0, 0] = 1.0
    K = np.zeros((1, 3, d))
    K[0, :, 0] = [1.0, 0.9, 0.8]
    V = np.random.default_rng(0).normal(size=(1, 3, d))
    qi = np.array([[2]], np.int32)
    ki = np.array([[0, 1, 2]], np.int32)
    fw = orc.forward(Q, K, V, qi, ki, 2.0, 1.0, 2, precision="f64")
    assert fw.taus[0, 0] == pytest.approx(0.45, abs=1e-12)
    w = np.array([0.55, 0.45, 0.35])
    want = (w[:, None] * V[0]).sum(0) / (w.sum() + 1e-8)  # EPS of :328
    np.testing.assert_allclose(fw.out[0, 0], want, rtol=1e-10, atol=1e-12)
    assert fw.norms[0, 0] == pytest.approx(1.35, abs=1e-12)


def _rand_problem(seed, BH=2, N=96, d=64, scale=0.3):
    rng = np.random.default_rng(seed)
    Q = rng.normal(size=(BH, N, d)) * scale
    K = rng.normal(size=(BH, N, d)) * scale
    V = rng.normal(size=(BH, N, d))
    dO = rng.normal(size=(BH, N, d))
    idx = np.broadcast_to(np.arange(N, dtype=np.int32), (BH, N)).copy()
    return Q, K, V, dO, idx


@pytest.mark.parametrize("alpha", [1.5, 2.0, 1.25])
def test_forward_with_exact_tau_is_dense_entmax(alpha):
    """With k >= N the top-k holds every visible key; feeding the exact tau
    (bisection) makes the oracle's forward the dense alpha-entmax attention."""
    Q, K, V, dO, idx = _rand_problem(0)
    vis = (idx[:, None, :] <= idx[:, :, None])
    out_d, P, taus = D.attention_forward(Q, K, V, vis, alpha, 1.0 / 8)
    fw = orc.forward(Q, K, V, idx, idx, alpha, 1.0 / 8, 128, taus_in=taus, precision="f64")
    # equal up to the EPS = 1e-8 the reference adds to the row sum (:328)
    np.testing.assert_allclose(fw.out, out_d, rtol=3e-8, atol=1e-11)
    np.testing.assert_allclose(fw.norms, P.sum(-1), rtol=1e-9)


def test_forward_output_in_convex_hull_of_visible_values():
    Q, K, V, dO, idx = _rand_problem(1, N=130)
    fw = orc.forward(Q, K, V, idx, idx, 1.5, 0.125, 8, precision="f64")
    for b in range(Q.shape[0]):
        for i in range(Q.shape[1]):
            if fw.norms[b, i] == 0:
                assert np.all(fw.out[b, i] == 0)
                continue
            # the EPS added to the row sum pulls the output towards 0 by a
            # factor N / (N + EPS); allow for that
            lo = V[b, :i + 1].min(0)
            hi = V[b, :i + 1].max(0)
            slack = 1e-12 + 2e-8 / fw.norms[b, i] * np.maximum(np.abs(lo), np.abs(hi))
            lo, hi = lo - slack, hi + slack
            assert np.all(fw.out[b, i] >= lo) and np.all(fw.out[b, i] <= hi)


def test_forward_block_m32_sums_over_the_rows_own_blocks():
    """With 32-row mask blocks a row weights the visible keys of the key
    blocks active for ITS 32-row block (adasplashattention.cu:278-297 with
    iQB = q / BLOCK_M), not those of its 64-row pair; restated in numpy
    from the top-k blocks (closed form above) and the oracle's tau."""
    rng = np.random.default_rng(3)
    BH, N, d = 2, 256, 64
    # 32-row half h of the queries has its top-2 keys ("magnets") in key
    # block h % 4, so the two halves of a 64-row block pick different key
    # blocks; every other key scores near 0, within the top-2 tau's reach
    # (u > 0), so a row weights every key of each block active for it
    Q = rng.normal(size=(BH, N, d)) * 0.1
    K = rng.normal(size=(BH, N, d)) * 0.1
    V = rng.normal(size=(BH, N, d))
    for h in range(N // 32):
        Q[:, 32 * h:32 * h + 32, h] += 1.0
        K[:, 64 * (h % 4) + h, h] = 5.0
        K[:, 64 * (h % 4) + 8 + h, h] = 4.0
    idx = np.broadcast_to(np.arange(N, dtype=np.int32), (BH, N)).copy()
    qi = np.full((BH, N), N - 1, np.int32)  # every key visible
    alpha, scale, k = 1.5, 0.125, 2
    fw = orc.forward(Q, K, V, qi, idx, alpha, scale, k, block_m=32, precision="f64")
    fw64 = orc.forward(Q, K, V, qi, idx, alpha, scale, k, block_m=64, precision="f64")
    assert fw.mask.shape == (2, 8, 4)
    for h in range(N // 32):
        np.testing.assert_array_equal(fw.mask[:, h], np.eye(4, dtype=np.uint8)[[h % 4] * BH])
    for b in range(BH):
        for i in range(N):
            blocks = set(j // 64 for r in range(i // 32 * 32, min(i // 32 * 32 + 32, N))
                         for j in fw.topk_idx[b, r] if j >= 0)
            keys = [j for j in range(N) if j // 64 in blocks]
            s = np.clip(Q[b, i] @ K[b, keys].T * scale, -10, 10)
            u = (alpha - 1) * s - fw.taus[b, i]
            p = np.where(u > 0, np.maximum(u, 1e-8) ** (1 / (alpha - 1)), 0.0)
            want = (p[:, None] * V[b, keys]).sum(0) / (p.sum() + 1e-8)
            np.testing.assert_allclose(fw.out[b, i], want, rtol=1e-10, atol=1e-12)
    # the 64-row blocks admit the other half's key block: every row differs
    assert (np.abs(fw.out - fw64.out).max(-1) > 1e-2).all()


# ---------------------------------------------------------------- backward


def _fd(fun, X, eps, picks):
    g = np.zeros(len(picks))
    for n, ix in enumerate(picks):
        Xp = X.copy()
        Xp[ix] += eps
        Xm = X.copy()
        Xm[ix] -= eps
        g[n] = (fun(Xp) - fun(Xm)) / (2 * eps)
    return g


def _picks(shape, rng, n=12):
    return [tuple(rng.integers(0, s) for s in shape) for _ in range(n)]


@pytest.mark.parametrize("alpha", [1.5, 2.0])
def test_reference_gradient_is_fixed_tau_gradient(alpha):
    """Mode 1 (adasplashattention.cu:343-535) differentiates the forward with
    tau held fixed: compare with central differences of <out, dO> where tau
    and the block mask are frozen."""
    Q, K, V, dO, idx = _rand_problem(2, BH=1, N=80)
    k, scale = 6, 0.125
    fw = orc.forward(Q, K, V, idx, idx, alpha, scale, k, precision="f64")
    taus = fw.taus

    def loss(Qx, Kx, Vx):
        f = orc.forward(Qx, Kx, Vx, idx, idx, alpha, scale, k, taus_in=taus, precision="f64")
        np.testing.assert_array_equal(f.mask, fw.mask)
        return float((f.out * dO).sum())

    dQ, dK, dV = orc.backward(Q, K, V, idx, idx, dO, alpha, scale, taus, fw.csr.q_ptr,
                              fw.csr.q_list, orc.GRAD_REFERENCE, precision="f64")
    rng = np.random.default_rng(0)
    for X, G, f in ((Q, dQ, lambda x: loss(x, K, V)), (K, dK, lambda x: loss(Q, x, V)),
                    (V, dV, lambda x: loss(Q, K, x))):
        pk = _picks(X.shape, rng)
        np.testing.assert_allclose(np.array([G[p] for p in pk]), _fd(f, X, 1e-6, pk),
                                   rtol=2e-5, atol=2e-7)


@pytest.mark.parametrize("alpha", [1.5, 2.0, 1.25, 2.5])
def test_entmax_gradient_is_dense_entmax_gradient(alpha):
    """Mode 0 with the exact tau and k >= N is the gradient of dense exact
    alpha-entmax attention (tau re-solved at every perturbed point).  At
    alpha = 2.5 the Jacobian weight P^(2-alpha) has a negative exponent:
    dense.attention_backward must keep it on the support only."""
    Q, K, V, dO, idx = _rand_problem(3, BH=1, N=72)
    scale = 0.125
    vis = (idx[:, None, :] <= idx[:, :, None])

    def loss(Qx, Kx, Vx):
        out, _, _ = D.attention_forward(Qx, Kx, Vx, vis, alpha, scale)
        return float((out * dO).sum())

    _, P, taus = D.attention_forward(Q, K, V, vis, alpha, scale)
    fw = orc.forward(Q, K, V, idx, idx, alpha, scale, 128, taus_in=taus, precision="f64")
    dQ, dK, dV = orc.backward(Q, K, V, idx, idx, dO, alpha, scale, taus, fw.csr.q_ptr,
                              fw.csr.q_list, orc.GRAD_ENTMAX, precision="f64")
    rng = np.random.default_rng(1)
    for X, G, f in ((Q, dQ, lambda x: loss(x, K, V)), (K, dK, lambda x: loss(Q, x, V)),
                    (V, dV, lambda x: loss(Q, K, x))):
        pk = _picks(X.shape, rng)
        np.testing.assert_allclose(np.array([G[p] for p in pk]), _fd(f, X, 1e-6, pk),
                                   rtol=5e-5, atol=5e-7)
    # and the dense closed-form Jacobian agrees everywhere
    gq, gk, gv = D.attention_backward(Q, K, V, P, dO, alpha, scale)
    np.testing.assert_allclose(dQ, gq, rtol=1e-7, atol=1e-9)
    np.testing.assert_allclose(dK, gk, rtol=1e-7, atol=1e-9)
    np.testing.assert_allclose(dV, gv, rtol=1e-7, atol=1e-9)


def test_sparsemax_gradient_centres_dp_on_support():
    """alpha = 2: g = 1 on the support, so ds = dp - mean_support(dp)."""
    Q, K, V, dO, idx = _rand_problem(4, BH=1, N=40)
    vis = (idx[:, None, :] <= idx[:, :, None])
    _, P, taus = D.attention_forward(Q, K, V, vis, 2.0, 0.125)
    dP = np.einsum("bid,bjd->bij", dO, V)
    supp = P > 0
    mean = (dP * supp).sum(-1, keepdims=True) / supp.sum(-1, keepdims=True)
    dS = np.where(supp, dP - mean, 0.0)
    fw = orc.forward(Q, K, V, idx, idx, 2.0, 0.125, 64, taus_in=taus, precision="f64")
    dQ, _, _ = orc.backward(Q, K, V, idx, idx, dO, 2.0, 0.125, taus, fw.csr.q_ptr,
                            fw.csr.q_list, orc.GRAD_ENTMAX, precision="f64")
    np.testing.assert_allclose(dQ, np.einsum("bij,bjd->bid", dS, K) * 0.125, rtol=1e-8, atol=1e-10)


# ---------------------------------------------------------------- key blocks


@pytest.mark.parametrize("mode", [orc.GRAD_ENTMAX, orc.GRAD_REFERENCE])
@pytest.mark.parametrize("alpha,causal,block_m", [(1.5, True, 64), (2.0, False, 64),
                                                  (1.25, True, 64), (1.5, True, 32)])
def test_key_block_grads_match_oracle_backward(mode, alpha, causal, block_m):
    """oracle/keyblock.py (the chunked restatement the full-size GPU tests
    use for sampled key blocks) equals asao_backward on whole heads."""
    from oracle import keyblock as KB

    rng = np.random.default_rng(21)
    BH, N, d, k, scale = 2, 320, 64, 6, 0.125
    Q, K, V, dO = (rng.normal(size=(BH, N, d)) for _ in range(4))
    ki = np.tile(np.arange(N, dtype=np.int32), (BH, 1))
    qi = ki.copy() if causal else np.full((BH, N), N - 1, np.int32)
    fw = orc.forward(Q, K, V, qi, ki, alpha, scale, k, block_m=block_m, precision="f64")
    gq, gk, gv = orc.backward(Q, K, V, qi, ki, dO, alpha, scale, fw.taus, fw.csr.q_ptr,
                              fw.csr.q_list, mode, block_m=block_m, precision="f64")
    blocks = [0, 2, 4]
    rows = np.concatenate([np.arange(b * 64, min(b * 64 + 64, N)) for b in blocks])
    for bh in range(BH):
        dK, dV = KB.key_block_grads(Q[bh], K[bh], V[bh], dO[bh], qi[bh], ki[bh], fw.taus[bh],
                                    fw.mask[bh], alpha, scale, blocks, mode, chunk=96,
                                    block_m=block_m)
        np.testing.assert_allclose(dK, gk[bh][rows], rtol=1e-9, atol=1e-12 * np.abs(gk).max())
        np.testing.assert_allclose(dV, gv[bh][rows], rtol=1e-9, atol=1e-12 * np.abs(gv).max())


def test_overflowed_key_sum_is_inf_and_host_fixup_clamps():
    """dV of a key is the sum over the rows that weight it of P * dO
    (cu:473-479).  Two rows that see only key 0 weight it with P = 1 (one
    visible key: p / (p + EPS) rounds to 1); with dO[:, 0] = 3e38 its sum
    6e38 is beyond the float range: +inf, as the reference's fp32 atomic
    sum gives; dQ and dK stay finite.  The host fix-up
    (cu:684-697) then clamps the whole dV to [-100, 100]."""
    d = 64
    rng = np.random.default_rng(0)
    Q = rng.normal(size=(1, 2, d)).astype(np.float32)
    K = rng.normal(size=(1, 1, d)).astype(np.float32)
    V = rng.normal(size=(1, 1, d)).astype(np.float32)
    dO = rng.normal(size=(1, 2, d)).astype(np.float32)
    dO[:, :, 0] = 3e38
    qi = np.zeros((1, 2), np.int32)
    ki = np.zeros((1, 1), np.int32)
    for mode in (orc.GRAD_ENTMAX, orc.GRAD_REFERENCE):
        _, (dQ, dK, dV) = orc.attention(Q, K, V, qi, ki, dO, 1.5, 0.125, 8, mode=mode)
        assert dV[0, 0, 0] == np.inf
        np.testing.assert_allclose(dV[0, 0, 1:], dO[0, 0, 1:] + dO[0, 1, 1:], rtol=1e-6)
        assert np.isfinite(dK).all() and np.isfinite(dQ).all()
        fixed, nan, inf = orc.host_fixup(dV)
        assert inf and not nan
        assert fixed[0, 0, 0] == 100.0
        np.testing.assert_array_equal(fixed[0, 0, 1:], np.clip(dV[0, 0, 1:], -100, 100))
