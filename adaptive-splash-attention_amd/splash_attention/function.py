"""Autograd wiring and the functional form of splash attention.

Under ``torch.compile``, ``splash_attention`` calls the ``adasplash::forward``
custom operator (library.py), whose autograd formula runs
``adasplash::backward``; eagerly it uses ``SplashAttentionFunction``, the
same pairing as a plain autograd function, which skips the operator
dispatch.

The reference exposes only separate native forward/backward calls and no
autograd wrapper (adasplashattention.cu:702-705); its README promises an
``AdaptiveSplashAttention`` module (README.md:102-124).  Here the forward
saves its selection state (tau, row sums, block mask, CSR lists) so that the
backward does not recompute it (the reference backward rebuilds the mask,
adasplashattention.cu:669-676).
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from . import library, ops


class SplashAttentionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, Q, K, V, Q_idx, K_idx, alpha, k_keep, sm_scale, grad_mode,
                tau_mode="reference", block_m=64, bwd_passes="support"):
        # support masks only when a support-pair backward can follow
        out, st = ops.splash_forward(Q, K, V, Q_idx, K_idx, alpha, k_keep, sm_scale,
                                     with_support=(any(ctx.needs_input_grad[:3])
                                                   and bwd_passes == "support"),
                                     tau_mode=tau_mode, block_m=block_m)
        ctx.params = (alpha, k_keep, sm_scale, grad_mode)
        ctx.save_for_backward(Q, K, V, Q_idx, K_idx, out, *st.tensors())
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        Q, K, V, Q_idx, K_idx, out, *state = ctx.saved_tensors
        alpha, k_keep, sm_scale, grad_mode = ctx.params
        st = ops.SplashState.from_tensors(state)
        dQ, dK, dV = ops.splash_backward(Q, K, V, Q_idx, K_idx, out, dout, st, alpha, k_keep,
                                         sm_scale, grad_mode)
        return dQ, dK, dV, None, None, None, None, None, None, None, None, None


def splash_attention(Q, K, V, Q_idx=None, K_idx=None, alpha: float = 1.5, k_keep: int = 8,
                     sm_scale: float | None = None, grad_mode: str = "entmax",
                     tau_mode: str = "reference", block_m: int = 64,
                     bwd_passes: str = "support") -> torch.Tensor:
    """Block-sparse alpha-entmax attention, differentiable in Q, K and V.

    Q: [B, H, NQ, d]; K, V: [B, H, NK, d], d <= 128; float32, bfloat16 or
    float16 (16-bit inputs: fp32 arithmetic on 16-bit MFMA operands) on
    one GPU.
    Q_idx: [B*H, NQ] and K_idx: [B*H, NK] integer positions (None: arange);
    key j is visible to query i iff K_idx[j] <= Q_idx[i].
    grad_mode "entmax" (default) uses the alpha-entmax Jacobian; "reference"
    reproduces the reference kernel's gradient.
    tau_mode "reference" (default) takes the reference's threshold over each
    row's top-k scores; "exact" solves the alpha-entmax threshold over every
    visible key of the row and activates the key blocks of its support, so
    the output is dense alpha-entmax attention (no reference counterpart).
    block_m: query rows per mask block, 64 (default) or 32 (the reference's
    compile-time BLOCK_M, adasplashattention.cu:8-9; reference tau mode).
    bwd_passes: how the backward runs (no reference counterpart; the same
    gradients either way, to float rounding): "support" (default) over each
    row's (row, key) pairs with nonzero weight, fastest when rows' supports
    are small; "tiles" over whole active 64 x 64 tiles on MFMA, fastest
    when supports fill most of the active tiles (near-uniform scores).
    """
    if grad_mode not in ops.GRAD_MODES:
        raise ValueError(f"grad_mode must be one of {sorted(ops.GRAD_MODES)}")
    ops.check_tau_mode(tau_mode)
    ops.check_block_m(block_m)
    ops.check_bwd_passes(bwd_passes)
    if torch.compiler.is_compiling():
        return library.attention(Q, K, V, Q_idx, K_idx, alpha, k_keep, sm_scale, grad_mode,
                                 tau_mode, block_m, bwd_passes)
    # eager: the autograd function, without the custom-operator dispatch;
    # check_inputs' padding and widening are differentiable torch ops
    d, dtype = Q.size(-1), Q.dtype
    if sm_scale is None:
        sm_scale = d ** -0.5
    Q, K, V, qi, ki = ops.check_inputs(Q, K, V, Q_idx, K_idx)
    out = SplashAttentionFunction.apply(Q, K, V, qi, ki, float(alpha), int(k_keep),
                                        float(sm_scale), grad_mode, tau_mode, int(block_m),
                                        bwd_passes)
    return ops.from_kernel_layout(out, d, dtype)
