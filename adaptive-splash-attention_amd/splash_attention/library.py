"""The attention as ``torch.library`` custom operators.

``adasplash::forward`` and ``adasplash::backward`` wrap the two C-ABI entry
points (asa_forward / asa_backward; the reference's ``forward`` /
``backward``, adasplashattention.cu:702-705) as opaque operators with
shape-only fake implementations and an autograd formula, so that
``torch.compile`` can trace models that call ``splash_attention`` without a
graph break and without looking inside the kernels.

The forward returns the attention output and the selection state (tau, row
sums, block mask, both CSR lists, the rows' support masks); the autograd
formula saves that state for the backward, as the eager autograd function
does.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
from torch import Tensor

from . import ops

_NS = "adasplash"


def _nblocks(n: int, b: int) -> int:
    return (n + b - 1) // b


@torch.library.custom_op(f"{_NS}::forward", mutates_args=(), device_types="cuda")
def forward_op(Q: Tensor, K: Tensor, V: Tensor, Q_idx: Optional[Tensor], K_idx: Optional[Tensor],
               alpha: float, k_keep: int, sm_scale: float, grad_mode: str,
               tau_mode: str = "reference", block_m: int = 64, bwd_passes: str = "support"
               ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """out, taus, norms, mask, q_ptr, q_list, k_ptr, k_list and the support
    masks sup_mask (empty for bwd_passes "tiles"; grad_mode is recorded for
    the backward only).  out is in the kernels' layout
    (ops.to_kernel_layout: the head dimension a whole number of 16-byte
    chunks), contiguous."""
    q, k, v, qi, ki = ops.check_inputs(Q, K, V, Q_idx, K_idx)
    out, st = ops.splash_forward(q, k, v, qi, ki, alpha, k_keep, sm_scale,
                                 with_support=bwd_passes == "support", tau_mode=tau_mode,
                                 block_m=block_m)
    sup = st.sup_mask
    if sup is None:
        sup = torch.empty((st.taus.size(0), 0, 4, 64), dtype=torch.int16, device=Q.device)
    return (out, *st.tensors()[:7], sup)


@forward_op.register_fake
def _forward_fake(Q, K, V, Q_idx, K_idx, alpha, k_keep, sm_scale, grad_mode,
                  tau_mode="reference", block_m=64, bwd_passes="support"):
    B, H, NQ, d = Q.shape
    NK = K.shape[2]
    BH = B * H
    nQB, nKB = _nblocks(NQ, block_m), _nblocks(NK, ops.BLOCK_N)
    nQ64 = _nblocks(NQ, 64)
    f32 = dict(dtype=torch.float32, device=Q.device)
    i32 = dict(dtype=torch.int32, device=Q.device)
    odt = Q.dtype
    return (torch.empty((B, H, NQ, ops.kernel_head_dim(d, Q.dtype)), dtype=odt, device=Q.device),
            torch.empty((BH, NQ), **f32), torch.empty((BH, NQ), **f32),
            torch.empty((BH, nQB, nKB), dtype=torch.uint8, device=Q.device),
            torch.empty((BH, nQB + 1), **i32), torch.empty((BH, nQB * nKB), **i32),
            torch.empty((BH, nKB + 1), **i32), torch.empty((BH, nKB * nQB), **i32),
            torch.empty((BH, nQ64 * nKB if bwd_passes == "support" else 0, 4, 64),
                        dtype=torch.int16, device=Q.device))


@torch.library.custom_op(f"{_NS}::backward", mutates_args=(), device_types="cuda")
def backward_op(Q: Tensor, K: Tensor, V: Tensor, Q_idx: Optional[Tensor], K_idx: Optional[Tensor],
                out: Tensor, dout: Tensor, taus: Tensor, norms: Tensor, mask: Tensor,
                q_ptr: Tensor, q_list: Tensor, k_ptr: Tensor, k_list: Tensor, sup_mask: Tensor,
                alpha: float,
                k_keep: int, sm_scale: float, grad_mode: str) -> tuple[Tensor, Tensor, Tensor]:
    """dQ, dK, dV from the state a matching forward_op returned."""
    q, k, v, qi, ki = ops.check_inputs(Q, K, V, Q_idx, K_idx)
    st = ops.SplashState.from_tensors((taus, norms, mask, q_ptr, q_list, k_ptr, k_list, sup_mask))
    grads = ops.splash_backward(q, k, v, qi, ki, out, dout, st, alpha, k_keep, sm_scale, grad_mode)
    return tuple(ops.from_kernel_layout(g, t.size(-1), t.dtype) for g, t in zip(grads, (Q, K, V)))


@backward_op.register_fake
def _backward_fake(Q, K, V, Q_idx, K_idx, out, dout, taus, norms, mask, q_ptr, q_list, k_ptr,
                   k_list, sup_mask, alpha, k_keep, sm_scale, grad_mode):
    c = torch.contiguous_format
    return (torch.empty_like(Q, memory_format=c), torch.empty_like(K, memory_format=c),
            torch.empty_like(V, memory_format=c))


def _setup_context(ctx, inputs, output):
    Q, K, V, Q_idx, K_idx, alpha, k_keep, sm_scale, grad_mode, tau_mode, block_m, bwd_passes = inputs
    out, *state = output
    ctx.params = (alpha, k_keep, sm_scale, grad_mode)
    ctx.save_for_backward(Q, K, V, Q_idx, K_idx, out, *state)


def _backward(ctx, dout, *unused_state_grads):
    Q, K, V, Q_idx, K_idx, out, *state = ctx.saved_tensors
    alpha, k_keep, sm_scale, grad_mode = ctx.params
    dQ, dK, dV = backward_op(Q, K, V, Q_idx, K_idx, out, dout, *state, alpha, k_keep, sm_scale,
                             grad_mode)
    return dQ, dK, dV, None, None, None, None, None, None, None, None, None


forward_op.register_autograd(_backward, setup_context=_setup_context)


def attention(Q: Tensor, K: Tensor, V: Tensor, Q_idx: Optional[Tensor], K_idx: Optional[Tensor],
              alpha: float, k_keep: int, sm_scale: Optional[float], grad_mode: str,
              tau_mode: str = "reference", block_m: int = 64,
              bwd_passes: str = "support") -> Tensor:
    """Shape-checked call of ``adasplash::forward``; returns the output in
    the caller's head dimension and dtype."""
    ops.check_shapes(Q, K, V, k_keep)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(Q.size(-1))
    out = forward_op(Q, K, V, Q_idx, K_idx, float(alpha), int(k_keep), float(sm_scale),
                     grad_mode, tau_mode, int(block_m), bwd_passes)[0]
    return ops.from_kernel_layout(out, Q.size(-1), Q.dtype)
