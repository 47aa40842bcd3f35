"""Shared helpers for the test suite: seeded inputs and comparisons."""
from __future__ import annotations

import numpy as np
import torch


def make_inputs(B, H, NQ, NK, d, seed=0, dtype=torch.float32, scale=1.0):
    """Q, K, V, dO drawn from N(0,1) on the CPU in that order (seed for Q/K/V,
    seed+1 for dO), cast to `dtype`; returns torch CPU tensors."""
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(B, H, NQ, d, generator=g) * scale
    K = torch.randn(B, H, NK, d, generator=g) * scale
    V = torch.randn(B, H, NK, d, generator=g)
    g2 = torch.Generator().manual_seed(seed + 1)
    dO = torch.randn(B, H, NQ, d, generator=g2)
    return tuple(t.to(dtype) for t in (Q, K, V, dO))


def causal_idx(BH, N):
    return torch.arange(N, dtype=torch.int32).unsqueeze(0).expand(BH, N).contiguous()


def np32(t):
    """Flatten [B,H,N,d] -> [BH,N,d] float32 numpy (exact for bf16 inputs)."""
    t = t.detach().float().cpu()
    if t.dim() == 4:
        t = t.reshape(-1, t.shape[2], t.shape[3])
    return t.numpy()


def rel_err(a, b, floor: float = 1e-30) -> float:
    """max |a - b| / max(max |b|, floor) (a, b array-like)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = max(float(np.abs(b).max()) if b.size else 0.0, floor)
    return float(np.abs(a - b).max()) / den if a.size else 0.0


def assert_close(name, got, want, tol, floor: float = 1e-30):
    """Max-norm relative error within tol; `floor` bounds the denominator
    from below for tensors that are zero in exact arithmetic (e.g. dQ of a
    row with one visible key), where it is the tensor's natural scale."""
    e = rel_err(got, want, floor)
    assert e <= tol, f"{name}: max relative error {e:.3e} > {tol:.1e}"
    return e


def oracle_at_gpu_tau(Q, K, V, dO, qidx, kidx, alpha, scale, k, gpu_taus, mode=0, block_m=64):
    """Oracle forward/backward evaluated at the GPU's taus.

    The reference's tau recurrence stops as soon as |f| < 1e-4
    (adasplashattention.cu:92), so a last-bit difference between the GPU's
    MFMA scores and the oracle's double-precision scores can end the
    iteration one (small) step earlier or later on a few rows.  Selection and
    tau are checked bit-exactly on identical scores elsewhere
    (test_gpu_select.py); here tau is compared at the recurrence's own
    resolution and the attention passes are compared at equal tau.
    Returns (oracle Forward at its own tau, Forward at gpu tau, grads at gpu tau).
    """
    from oracle import oracle as orc

    own = orc.forward(Q, K, V, qidx, kidx, alpha, scale, k, block_m=block_m)
    at = orc.forward(Q, K, V, qidx, kidx, alpha, scale, k, block_m=block_m, taus_in=gpu_taus)
    grads = orc.backward(Q, K, V, qidx, kidx, dO, alpha, scale, at.taus, at.csr.q_ptr,
                         at.csr.q_list, mode, block_m=block_m)
    return own, at, grads


def assert_tau_close(gpu_taus, own_taus, alpha):
    """tau within the resolution of the recurrence's exit test: one Halley
    step taken at |f| < 1e-4 moves tau by about |f / f'|, far below 1e-3."""
    import numpy as np

    d = np.abs(np.asarray(gpu_taus, np.float64) - np.asarray(own_taus, np.float64))
    assert float(d.max()) <= 1e-3, f"tau differs by {float(d.max()):.2e}"
    # and most rows agree to float rounding
    assert float(np.mean(d <= 1e-5 * np.maximum(1.0, np.abs(own_taus)))) > 0.99
