"""splash_attention: block-sparse alpha-entmax attention on AMD MI355X (gfx950).

Drop-in for mvideet/Adaptive-Splash-Attention:

* ``AdaptiveSplashAttention`` -- the module its README documents
  (README.md:102-124).
* ``forward`` / ``backward`` -- the two native entry points its extension
  binds (source/adasplashattention.cu:702-705), same argument order:
  ``forward(Q, K, V, Q_idx, K_idx, sm_scale, alpha) -> Out`` and
  ``backward(Q, K, V, Q_idx, K_idx, sm_scale, alpha, dOut) -> [dQ, dK, dV]``,
  with the compiled reference's defaults (``k_keep`` 8, :17-19; 32-row mask
  blocks, :8-9) as extra keywords, and its host fix-up of non-finite
  results (:599-606, :684-697).  ``backward`` recomputes the selection like
  the reference does (:669-676) and returns the reference kernel's
  gradient.
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
            block_m: int = 32, fix_nonfinite: bool = True):
    """Reference-compatible native forward (adasplashattention.cu:537-609).

    Defaults are the compiled reference's: ``k_keep`` 8 (K_KEEP, :17-19) and
    32-row mask blocks (BLOCK_M, :8-9); ``block_m=64`` gives the 64x64
    blocks of the module's default.  ``sm_scale=None`` means 1/sqrt(d) of
    the caller's head dimension (before any zero padding).
    ``fix_nonfinite`` applies the reference's host fix-up to the output
    (NaN -> 0, and any Inf clamps the whole tensor to [-100, 100], each with
    a warning, :599-606); it synchronises with the device, as the reference
    does.  Pass False to skip the check."""
    ops.check_shapes(Q, K, V)
    d, dtype = Q.size(-1), Q.dtype
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    Q, K, V, qi, ki = ops.check_inputs(Q, K, V, Q_idx, K_idx)
    out, _ = ops.splash_forward(Q, K, V, qi, ki, ops.clamp_alpha(alpha), k_keep, sm_scale,
                                with_support=False, block_m=block_m)
    out = ops.from_kernel_layout(out, d, dtype)
    if fix_nonfinite:
        out = ops.fix_nonfinite(out, "output")
    return out


def backward(Q, K, V, Q_idx, K_idx, sm_scale: float, alpha: float, dOut, k_keep: int = 8,
             grad_mode: str = "reference", block_m: int = 32, fix_nonfinite: bool = True,
             bwd_passes: str = "support"):
    """Reference-compatible native backward (adasplashattention.cu:611-700):
    reruns the selection, then returns [dQ, dK, dV].  Defaults, ``sm_scale``
    and ``fix_nonfinite`` as in ``forward`` (the gradients' fix-up is
    :684-697, with the names dQ, dK, dV in the warnings).  ``bwd_passes``
    as in ``splash_attention`` (no reference counterpart)."""
    ops.check_shapes(Q, K, V)
    if not isinstance(dOut, torch.Tensor) or dOut.shape != Q.shape:
        raise ValueError(f"dOut shape {tuple(getattr(dOut, 'shape', ()))} must equal Q shape "
                         f"{tuple(Q.shape)}")
    d, dtype = Q.size(-1), Q.dtype
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    Q, K, V, qi, ki = ops.check_inputs(Q, K, V, Q_idx, K_idx)
    a = ops.clamp_alpha(alpha)
    ops.check_bwd_passes(bwd_passes)
    out, st = ops.splash_forward(Q, K, V, qi, ki, a, k_keep, sm_scale, block_m=block_m,
                                 with_support=bwd_passes == "support")
    grads = ops.splash_backward(Q, K, V, qi, ki, out, dOut, st, a, k_keep, sm_scale, grad_mode)
    grads = [ops.from_kernel_layout(g, d, dtype) for g in grads]
    if fix_nonfinite:
        grads = [ops.fix_nonfinite(g, n) for g, n in zip(grads, ("dQ", "dK", "dV"))]
    return grads
