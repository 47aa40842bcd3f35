"""Support masks written by the forward (asa_state.sup_mask) against dense
fp32 scores computed with torch on the same inputs.

Bit 4f + r of mask[bh, e, w, 4c + g] marks row qb*64 + 16w + c and key
kb*64 + 16f + 4g + r of the tile at q_list position e when the forward
weighted it with u = (alpha-1) clamp(scale q.k) - tau > 0.  Every pair of an
active block with u > 1e-4 must be marked and every pair with u < -1e-4, or
outside the visible/active set, must not (pairs within 1e-4 of u = 0 may
fall either way: the MFMA and torch round the dot products differently);
masks of unused tile slots are not read.
"""
import numpy as np
import pytest
import torch

import splash_attention as sa
from tests._util import causal_idx, make_inputs

pytestmark = pytest.mark.gpu


def _support_check(dev, B, H, NQ, NK, d, alpha, k, scale, dtype, seed):
    Q, K, V, _ = make_inputs(B, H, NQ, NK, d, seed=seed, dtype=dtype)
    BH = B * H
    qi = causal_idx(BH, NQ) + max(NK - NQ, 0)
    ki = causal_idx(BH, NK)
    q, kk, v, qi_, ki_ = sa.ops.check_inputs(Q.to(dev), K.to(dev), V.to(dev), qi.to(dev), ki.to(dev))
    out, st = sa.ops.splash_forward(q, kk, v, qi_, ki_, alpha, k, scale, with_support=True)
    torch.cuda.synchronize()
    nQB, nKB = -(-NQ // 64), -(-NK // 64)
    masks = st.sup_mask.cpu().numpy().view(np.uint16)  # [BH, nQB*nKB, 4, 64]
    taus = st.taus.cpu().numpy().astype(np.float64)
    mask = st.mask.cpu().numpy()
    q_ptr = st.q_ptr.cpu().numpy()
    q_list = st.q_list.cpu().numpy()
    S = torch.matmul(q.float().reshape(BH, NQ, d), kk.float().reshape(BH, NK, d).transpose(1, 2)
                     .contiguous()).cpu().numpy().astype(np.float64) * scale
    S = np.clip(S, -10, 10)
    am1 = sa.ops.clamp_alpha(alpha) - 1
    marked = 0
    for bh in range(BH):
        u = am1 * S[bh] - taus[bh][:, None]
        vis = ki[bh].numpy()[None, :] <= qi[bh].numpy()[:, None]
        act = np.repeat(np.repeat(mask[bh], 64, 0)[:NQ], 64, 1)[:, :NK].astype(bool)
        got = np.zeros((NQ, NK), bool)
        for qb in range(nQB):
            for e in range(q_ptr[bh, qb], q_ptr[bh, qb + 1]):
                kb = q_list[bh, e]
                for w in range(4):
                    for c in range(16):
                        row = qb * 64 + 16 * w + c
                        for g in range(4):
                            m = int(masks[bh, e, w, 4 * c + g])
                            for f in range(4):
                                for r in range(4):
                                    if m >> (4 * f + r) & 1:
                                        key = kb * 64 + 16 * f + 4 * g + r
                                        assert row < NQ and key < NK, "bit outside the problem"
                                        got[row, key] = True
        want = (u > 0) & vis & act
        sure_in = want & (u > 1e-4)
        sure_out = ~(vis & act) | (u < -1e-4)
        assert not np.any(sure_in & ~got), f"head {bh}: supported pairs not marked"
        assert not np.any(sure_out & got), f"head {bh}: pairs marked outside the support"
        marked += int(got.sum())
    assert marked > 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_support_masks_match_dense_scores(dev, dtype):
    print(f"[support] 1x2x300x300 d64 {dtype}", flush=True)
    _support_check(dev, 1, 2, 300, 300, 64, 1.5, 16, 0.125, dtype, seed=31)


def test_support_masks_nq_ne_nk_alpha2(dev):
    print("[support] 2x1x130x257 d128 alpha 2", flush=True)
    _support_check(dev, 2, 1, 130, 257, 128, 2.0, 8, 128 ** -0.5, torch.bfloat16, seed=32)
