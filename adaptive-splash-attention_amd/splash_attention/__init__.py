"""splash_attention: block-sparse alpha-entmax attention on AMD MI355X (gfx950).

Drop-in for mvideet/Adaptive-Splash-Attention:

* ``AdaptiveSplashAttention`` -- the module its README documents
  (README.md:102-124).
* ``forward`` / ``backward`` -- the two native entry points its extension
  binds (source/adasplashattention.cu:702-705), same argument order:
  ``forward(Q, K, V, Q_idx, K_idx, sm_scale, alpha) -> Out`` and
  ``backward(Q, K, V, Q_idx, K_idx, sm_scale, alpha, dOut) -> [dQ, dK, dV]``,
  with ``k_keep`` as an extra keyword (the reference fixes it at 8 when it
  is compiled, :17-19).  ``backward`` recomputes the selection like the
  reference does (:669-676) and returns the reference kernel's gradient.
* ``splash_attention`` -- functional form with autograd.

All compute runs in hand-written HIP kernels in ``lib/libadasplash.so``;
there is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import math

import torch

from . import ops
from ._lib import ASAError
from .function import SplashAttentionFunction, splash_attention
from .module import AdaptiveSplashAttention

__all__ = [
    "AdaptiveSplashAttention",
    "ASAError",
    "SplashAttentionFunction",
    "backward",
    "forward",
    "ops",
    "splash_attention",
]

__version__ = "0.1.0"


def forward(Q, K, V, Q_idx, K_idx, sm_scale: float, alpha: float, k_keep: int = 8,
            block_m: int = 64):
    """Reference-compatible native forward (adasplashattention.cu:537-609).
    ``sm_scale=None`` means 1/sqrt(d) of the caller's head dimension (before
    any zero padding).  block_m = 32 gives the reference's default mask blocks
    (BLOCK_M, :8-9)."""
    ops.check_shapes(Q, K, V)
    d, dtype = Q.size(-1), Q.dtype
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    Q, K, V, qi, ki = ops.check_inputs(Q, K, V, Q_idx, K_idx)
    out, _ = ops.splash_forward(Q, K, V, qi, ki, ops.clamp_alpha(alpha), k_keep, sm_scale,
                                with_support=False, block_m=block_m)
    return ops.from_kernel_layout(out, d, dtype)


def backward(Q, K, V, Q_idx, K_idx, sm_scale: float, alpha: float, dOut, k_keep: int = 8,
             grad_mode: str = "reference", block_m: int = 64):
    """Reference-compatible native backward (adasplashattention.cu:611-700):
    reruns the selection, then returns [dQ, dK, dV].  ``sm_scale=None`` as
    in ``forward``."""
    ops.check_shapes(Q, K, V)
    if not isinstance(dOut, torch.Tensor) or dOut.shape != Q.shape:
        raise ValueError(f"dOut shape {tuple(getattr(dOut, 'shape', ()))} must equal Q shape "
                         f"{tuple(Q.shape)}")
    d, dtype = Q.size(-1), Q.dtype
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    Q, K, V, qi, ki = ops.check_inputs(Q, K, V, Q_idx, K_idx)
    a = ops.clamp_alpha(alpha)
    out, st = ops.splash_forward(Q, K, V, qi, ki, a, k_keep, sm_scale, block_m=block_m)
    grads = ops.splash_backward(Q, K, V, qi, ki, out, dOut, st, a, k_keep, sm_scale, grad_mode)
    return [ops.from_kernel_layout(g, d, dtype) for g in grads]
