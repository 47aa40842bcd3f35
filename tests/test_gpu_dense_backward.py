"""The dense backward passes (asa_backward with no support masks in the
state: dq_kernel, dkdv_kernel, and delta_kernel in reference mode) against
the CPU oracle, and against the support-pair passes on the same forward.

A caller that runs the forward without support masks (asa_state.sup_mask
NULL, ops.splash_forward(with_support=False)) gets these passes.  Ragged
NQ != NK (partial last tiles), fp32 and bf16, both gradient modes.
Tolerances: 1e-5 relative (fp32), 2e-2 relative (bf16).
"""
import numpy as np
import pytest
import torch

import splash_attention as sa
from oracle import oracle as orc
from tests._util import assert_close, causal_idx, make_inputs, np32, oracle_at_gpu_tau

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 4e-3}


@pytest.mark.parametrize("mode", ["entmax", "reference"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_dense_backward_matches_oracle_and_sparse(dev, dtype, mode):
    print(f"[dense-bwd] {dtype} {mode}", flush=True)
    B, H, NQ, NK, d = 1, 2, 300, 350, 64
    Q, K, V, dO = make_inputs(B, H, NQ, NK, d, seed=31, dtype=dtype)
    qi = causal_idx(B * H, NQ) + (NK - NQ)
    ki = causal_idx(B * H, NK)
    q, kk, v, qi_, ki_ = sa.ops.check_inputs(Q.to(dev), K.to(dev), V.to(dev), qi.to(dev),
                                             ki.to(dev))
    out_d, st_d = sa.ops.splash_forward(q, kk, v, qi_, ki_, 1.5, 16, 0.125, with_support=False)
    assert st_d.sup_mask is None
    g_dense = sa.ops.splash_backward(q, kk, v, qi_, ki_, out_d, dO.to(dev), st_d, 1.5, 16, 0.125,
                                     mode)
    out_s, st_s = sa.ops.splash_forward(q, kk, v, qi_, ki_, 1.5, 16, 0.125, with_support=True)
    g_sparse = sa.ops.splash_backward(q, kk, v, qi_, ki_, out_s, dO.to(dev), st_s, 1.5, 16, 0.125,
                                      mode)
    torch.cuda.synchronize()
    assert torch.equal(out_d, out_s), "forward output depends on the support masks"
    m = orc.GRAD_ENTMAX if mode == "entmax" else orc.GRAD_REFERENCE
    own, fw, og = oracle_at_gpu_tau(np32(Q), np32(K), np32(V), np32(dO), qi.numpy(), ki.numpy(),
                                    1.5, 0.125, 16, st_d.taus.cpu().numpy(), m)
    np.testing.assert_array_equal(st_d.mask.cpu().numpy(), own.mask)
    tol = TOL[dtype]
    assert_close("dense-bwd out", np32(out_d), fw.out, tol)
    for name, gd, gs, w in zip(("dQ", "dK", "dV"), g_dense, g_sparse, og):
        assert_close(f"dense {name}", np32(gd), w, tol)
        assert_close(f"dense vs support-pair {name}", np32(gd), np32(gs), 2 * tol)
