"""dK and dV of chosen 64-key blocks, for rows of any length (test
infrastructure only; nothing in the product path imports it).

The C oracle (asa_oracle.c, asao_backward) computes every gradient of a
head with scalar loops, which takes minutes at N = 16384-32768.  A key
block's dK and dV need every query row that sees it, and each row's
constants (sum of p, and for the entmax gradient sum w and sum w dp) need
the whole row, so this restatement runs over the rows in chunks with dense
float64 products and keeps only the chosen key columns.  It follows the
same steps as asao_backward, which restates the reference's
splash_backward_sparse (source/adasplashattention.cu:343-535) in the build's
two gradient modes:
  s  = clamp(scale * q.k, -10, 10)                      (cu:195-197)
  u  = (alpha - 1) s - tau,  p = u^(1/(alpha-1)) for u > 0   (cu:307-312)
  only visible keys (K_idx <= Q_idx, cu:189) of active blocks (mask, cu:244-341)
  N  = sum_j p_j,  P = p / (N + EPS)
  dV_j = sum_i P_ij dO_i
  w  = u^((2-alpha)/(alpha-1)) for u > 0 (entmax) or u > EPS (reference, cu:494)
  entmax:    ds = (N + EPS)^(alpha-2) w (dp - sum w dp / sum w)
  reference: ds = w (dp - out.dO) / (N + EPS)
  dK_j = scale sum_i ds_ij q_i,  dp_ij = dO_i . v_j
It is pinned against asao_backward on whole heads at small sizes
(tests/test_oracle_pins.py).
"""
from __future__ import annotations

import numpy as np

EPS = 1e-8
GRAD_ENTMAX = 0
GRAD_REFERENCE = 1


def key_block_grads(Q, K, V, dO, q_idx, k_idx, taus, mask, alpha: float, scale: float,
                    blocks, mode: int = GRAD_ENTMAX, block: int = 64, chunk: int = 256,
                    block_m: int | None = None):
    """dK, dV of one head's key blocks `blocks` (list of block indices).

    Q, dO [NQ, d]; K, V [NK, d]; q_idx [NQ], k_idx [NK]; taus [NQ];
    mask [nQB, nKB] (nonzero: active) with query blocks of block_m rows
    (default: `block`, the key-block width).  Returns (dK, dV), each
    [len(blocks) * block, d] float64 (rows past NK are zero)."""
    block_m = block if block_m is None else block_m
    Q, K, V, dO = (np.asarray(t, np.float64) for t in (Q, K, V, dO))
    q_idx = np.asarray(q_idx, np.int64)
    k_idx = np.asarray(k_idx, np.int64)
    taus = np.asarray(taus, np.float64)
    mask = np.asarray(mask) != 0
    alpha = max(1.05, min(float(alpha), 3.0))
    am1 = alpha - 1.0
    a = 1.0 / am1
    ew = (2.0 - alpha) / am1
    NQ, d = Q.shape
    NK = K.shape[0]
    cols = np.concatenate([np.arange(b * block, min((b + 1) * block, NK)) for b in blocks])
    pos = np.concatenate([np.arange(len(range(b * block, min((b + 1) * block, NK))))
                          + i * block for i, b in enumerate(blocks)])
    dK = np.zeros((len(blocks) * block, d))
    dV = np.zeros((len(blocks) * block, d))
    key_block = np.arange(NK) // block
    for r0 in range(0, NQ, chunk):
        r1 = min(r0 + chunk, NQ)
        rows = np.arange(r0, r1)
        s = np.clip((Q[r0:r1] @ K.T) * scale, -10.0, 10.0)
        live = (k_idx[None, :] <= q_idx[rows, None]) & mask[(rows // block_m)[:, None],
                                                            key_block[None, :]]
        u = am1 * s - taus[rows, None]
        pos_u = live & (u > 0)
        up = np.where(pos_u, np.maximum(u, EPS), 1.0)
        p = np.where(pos_u, up ** a, 0.0)
        p[~np.isfinite(p)] = 0.0
        n = p.sum(1)
        invn = 1.0 / (n + EPS)
        P = p * invn[:, None]
        dp = dO[r0:r1] @ V.T
        wlive = pos_u if mode == GRAD_ENTMAX else (live & (u > EPS))
        w = np.where(wlive, up ** ew, 0.0)
        w[~np.isfinite(w)] = 0.0
        if mode == GRAD_ENTMAX:
            sw = w.sum(1)
            shift = np.where(sw > 0, (w * dp).sum(1) / np.where(sw > 0, sw, 1.0), 0.0)
            cg = (n + EPS) ** (alpha - 2.0)
        else:
            shift = (p * dp).sum(1) * invn  # out . dO
            cg = invn
        ds = cg[:, None] * w[:, cols] * (dp[:, cols] - shift[:, None])
        ds[~np.isfinite(ds)] = 0.0
        dK[pos] += scale * (ds.T @ Q[r0:r1])
        dV[pos] += P[:, cols].T @ dO[r0:r1]
    return dK, dV
