"""``AdaptiveSplashAttention``: the module the reference README documents
(README.md:102-124), with the same constructor and call convention."""
from __future__ import annotations

import torch
from torch import nn

from .function import splash_attention


class AdaptiveSplashAttention(nn.Module):
    """Block-sparse alpha-entmax attention.

    Args follow README.md:105-111 of the reference:
      head_dim: last dimension of Q, K, V (1..128, as the reference's
        D_MAX; the kernels run at 64 or 128 with zero-padded columns).
      alpha: entmax parameter, clamped to [1.05, 3] as the reference does.
      k_keep: top-k kept per query row (1..128).
      adaptive_threshold: accepted for compatibility.  The reference
        recomputes tau on every call and has no parameters; so does this
        module (it has no state_dict entries).
      sm_scale: score scale (default 1/sqrt(head_dim)).
      grad_mode: "entmax" (alpha-entmax Jacobian, default) or "reference"
        (the reference kernel's gradient).
      tau_mode: "reference" (default: the reference's threshold over each
        row's top-k) or "exact" (the alpha-entmax threshold over the whole
        visible row, i.e. dense alpha-entmax attention; no reference
        counterpart).
      block_m: query rows per mask block, 64 (default) or 32 (the
        reference's compile-time BLOCK_M; reference tau mode only).
      bwd_passes: "support" (default: the backward over each row's
        (row, key) pairs with nonzero weight) or "tiles" (over whole active
        tiles on MFMA, faster when supports fill most of the active tiles);
        no reference counterpart.

    forward(Q, K, V, Q_idx=None, K_idx=None): Q [B, H, NQ, d], K and V
    [B, H, NK, d]; Q_idx [B*H, NQ], K_idx [B*H, NK] positions (default
    arange, i.e. causal).  float32, bfloat16 or float16 (fp32 arithmetic;
    16-bit inputs use 16-bit MFMA operands).  Returns [B, H, NQ, d] in the
    input dtype.
    """

    def __init__(self, head_dim: int = 64, alpha: float = 1.5, k_keep: int = 8,
                 adaptive_threshold: bool = True, sm_scale: float | None = None,
                 grad_mode: str = "entmax", tau_mode: str = "reference", block_m: int = 64,
                 bwd_passes: str = "support"):
        super().__init__()
        if not 1 <= int(head_dim) <= 128:
            raise ValueError(f"head_dim {head_dim} out of range [1, 128]")
        if not 1 <= int(k_keep) <= 128:
            raise ValueError(f"k_keep {k_keep} out of range [1, 128]")
        if grad_mode not in ("entmax", "reference"):
            raise ValueError("grad_mode must be 'entmax' or 'reference'")
        if tau_mode not in ("reference", "exact"):
            raise ValueError("tau_mode must be 'reference' or 'exact'")
        if block_m not in (64, 32):
            raise ValueError("block_m must be 64 or 32")
        if block_m == 32 and tau_mode == "exact":
            raise ValueError("tau_mode 'exact' needs block_m = 64")
        if bwd_passes not in ("support", "tiles"):
            raise ValueError("bwd_passes must be 'support' or 'tiles'")
        self.head_dim = int(head_dim)
        self.alpha = float(alpha)
        self.k_keep = int(k_keep)
        self.adaptive_threshold = bool(adaptive_threshold)
        self.sm_scale = float(sm_scale) if sm_scale is not None else self.head_dim ** -0.5
        self.grad_mode = grad_mode
        self.tau_mode = tau_mode
        self.block_m = int(block_m)
        self.bwd_passes = bwd_passes

    def extra_repr(self) -> str:
        return (f"head_dim={self.head_dim}, alpha={self.alpha}, k_keep={self.k_keep}, "
                f"sm_scale={self.sm_scale}, grad_mode={self.grad_mode!r}, "
                f"tau_mode={self.tau_mode!r}, block_m={self.block_m}, "
                f"bwd_passes={self.bwd_passes!r}")

    def forward(self, Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor,
                Q_idx: torch.Tensor | None = None, K_idx: torch.Tensor | None = None) -> torch.Tensor:
        if Q.size(-1) != self.head_dim:
            raise ValueError(f"Q head dim {Q.size(-1)} != head_dim {self.head_dim}")
        return splash_attention(Q, K, V, Q_idx, K_idx, self.alpha, self.k_keep, self.sm_scale,
                                self.grad_mode, self.tau_mode, self.block_m, self.bwd_passes)
