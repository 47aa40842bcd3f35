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


def rel_err(a, b) -> float:
    """max |a - b| / max |b| (a, b array-like)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = max(float(np.abs(b).max()) if b.size else 0.0, 1e-30)
    return float(np.abs(a - b).max()) / den if a.size else 0.0


def assert_close(name, got, want, tol):
    e = rel_err(got, want)
    assert e <= tol, f"{name}: max relative error {e:.3e} > {tol:.1e}"
    return e
