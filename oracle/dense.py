"""Dense exact alpha-entmax attention in float64 (test infrastructure only).

Used by the oracle's own pinning tests (exact tau, closed forms) and as the
dense baseline.  Nothing here is part of the product path.

Parameterisation (the one the reference kernel uses,
source/adasplashattention.cu:70-73, :311-312):
    p_j = [(alpha - 1) s_j - tau]_+ ** (1 / (alpha - 1)),  sum_j p_j = 1.
"""
from __future__ import annotations

import numpy as np


def tau_bisect(s, alpha: float, iters: int = 200) -> float:
    """Exact threshold of one row of scores s (float64 bisection)."""
    z = (alpha - 1.0) * np.asarray(s, np.float64)
    a = 1.0 / (alpha - 1.0)
    top = float(z.max())
    lo, hi = top - 1.0, top  # f(lo) >= 0, f(hi) = -1
    for _ in range(iters):
        mid = 0.5 * (lo + hi)
        if mid == lo or mid == hi:
            break
        f = np.sum(np.maximum(z - mid, 0.0) ** a) - 1.0
        if f > 0:
            lo = mid
        else:
            hi = mid
    return 0.5 * (lo + hi)


def tau_sparsemax(s) -> float:
    """alpha = 2 closed form: tau = (sum_{j<=rho} s_j - 1) / rho on the sorted row."""
    z = np.sort(np.asarray(s, np.float64))[::-1]
    cs = np.cumsum(z)
    rho = np.arange(1, z.size + 1)
    taus = (cs - 1.0) / rho
    support = z > taus
    r = int(np.nonzero(support)[0].max())
    return float(taus[r])


def tau_entmax15(s) -> float:
    """alpha = 1.5 closed form (sort-based): sum_{j<=rho} (z_j - tau)^2 = 1, z = s/2."""
    z = np.sort(0.5 * np.asarray(s, np.float64))[::-1]
    rho = np.arange(1, z.size + 1)
    mean = np.cumsum(z) / rho
    msq = np.cumsum(z * z) / rho
    delta = (1.0 - rho * (msq - mean * mean)) / rho
    taus = mean - np.sqrt(np.maximum(delta, 0.0))
    support = (z > taus) & (delta >= 0)
    r = int(np.nonzero(support)[0].max())
    return float(taus[r])


def entmax_probs(s, alpha: float, tau: float | None = None) -> np.ndarray:
    s = np.asarray(s, np.float64)
    if tau is None:
        tau = tau_bisect(s, alpha)
    return np.maximum((alpha - 1.0) * s - tau, 0.0) ** (1.0 / (alpha - 1.0))


def attention_forward(Q, K, V, vis, alpha: float, sm_scale: float, clamp: bool = True):
    """Exact dense alpha-entmax attention over the visible keys of each row.

    Returns (out [BH,NQ,d], P [BH,NQ,NK], taus [BH,NQ]).  With clamp=True the
    scores are clamped to [-10, 10] like the reference's score pass.
    """
    Q = np.asarray(Q, np.float64)
    K = np.asarray(K, np.float64)
    V = np.asarray(V, np.float64)
    S = np.einsum("bid,bjd->bij", Q, K) * sm_scale
    if clamp:
        S = np.clip(S, -10.0, 10.0)
    BH, NQ, NK = S.shape
    P = np.zeros_like(S)
    taus = np.zeros((BH, NQ))
    for b in range(BH):
        for i in range(NQ):
            m = np.asarray(vis[b, i], bool)
            if not m.any():
                continue
            t = tau_bisect(S[b, i, m], alpha)
            taus[b, i] = t
            P[b, i, m] = entmax_probs(S[b, i, m], alpha, t)
    out = np.einsum("bij,bjd->bid", P, V)
    return out, P, taus


def attention_backward(Q, K, V, P, dO, alpha: float, sm_scale: float):
    """Exact entmax-Jacobian gradients of the dense attention above.

    ds = g * (dp - sum(g dp)/sum(g)),  g = P^(2-alpha) on the support.
    (No clamp derivative: callers keep |s| < 10.)
    """
    Q = np.asarray(Q, np.float64)
    K = np.asarray(K, np.float64)
    V = np.asarray(V, np.float64)
    dO = np.asarray(dO, np.float64)
    dP = np.einsum("bid,bjd->bij", dO, V)
    # P^(2-alpha) on the support only (for alpha > 2, 0^(2-alpha) is inf)
    g = np.where(P > 0, np.where(P > 0, P, 1.0) ** (2.0 - alpha), 0.0)
    sg = g.sum(-1, keepdims=True)
    shift = np.where(sg > 0, (g * dP).sum(-1, keepdims=True) / np.where(sg > 0, sg, 1.0), 0.0)
    dS = g * (dP - shift)
    dQ = np.einsum("bij,bjd->bid", dS, K) * sm_scale
    dK = np.einsum("bij,bid->bjd", dS, Q) * sm_scale
    dV = np.einsum("bij,bid->bjd", P, dO)
    return dQ, dK, dV
