"""Support lists written by the forward (asa_state.sup_*) against dense
fp32 scores computed with torch on the same inputs.

Every (row, key) pair of an active block with u = (alpha-1) clamp(scale
q.k) - tau > 0 must be listed in its row's wave region, with v = max(u, 0),
in tile order (sup_off) and with keys inside the tile's key block; pairs
within 1e-4 of u = 0 may fall either way (the MFMA and torch round the dot
products differently).
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
    cap = st.sup_key.shape[1]
    key = st.sup_key.cpu().numpy().astype(np.uint32)
    val = st.sup_val.cpu().numpy()
    off = st.sup_off.cpu().numpy()
    cnt = st.sup_cnt.cpu().numpy()
    taus = st.taus.cpu().numpy()
    mask = st.mask.cpu().numpy()
    q_ptr = st.q_ptr.cpu().numpy()
    q_list = st.q_list.cpu().numpy()
    S = torch.matmul(q.float().reshape(BH, NQ, d), kk.float().reshape(BH, NK, d).transpose(1, 2)
                     .contiguous()).cpu().numpy().astype(np.float64) * scale
    S = np.clip(S, -10, 10)
    am1 = sa.ops.clamp_alpha(alpha) - 1
    checked = 0
    for bh in range(BH):
        u = am1 * S[bh] - taus[bh][:, None].astype(np.float64)
        vis = ki[bh].numpy()[None, :] <= qi[bh].numpy()[:, None]
        act = np.repeat(np.repeat(mask[bh], 64, 0)[:NQ], 64, 1)[:, :NK].astype(bool)
        for qb in range(nQB):
            for w in range(4):
                wr = (bh * nQB + qb) * 4 + w
                n = int(cnt[wr])
                assert n <= cap, f"region {wr} overflowed ({n} > {cap})"
                rows = np.arange(qb * 64 + 16 * w, min(qb * 64 + 16 * w + 16, NQ))
                got = {}
                e0, e1 = q_ptr[bh, qb], q_ptr[bh, qb + 1]
                for e in range(e0, e1):
                    lo = off[bh, e, w]
                    hi = off[bh, e + 1, w] if e + 1 < e1 else n
                    kb = q_list[bh, e]
                    for x in range(lo, hi):
                        kj = int(key[wr, x] & 0x0FFFFFFF)
                        r = qb * 64 + 16 * w + int(key[wr, x] >> 28)
                        assert kb * 64 <= kj < kb * 64 + 64, "entry outside its tile's key block"
                        assert (r, kj) not in got, "duplicate entry"
                        got[(r, kj)] = val[wr, x]
                if rows.size == 0:
                    assert n == 0
                    continue
                uu = u[rows]
                want = (uu > 0) & vis[rows] & act[rows]
                sure_in = want & (uu > 1e-4)
                sure_out = ~want | (uu < -1e-4)
                for (r, kj), vv in got.items():
                    i = r - rows[0]
                    assert not (sure_out[i, kj] and not want[i, kj]), f"({r},{kj}) listed, u={uu[i, kj]}"
                    assert abs(vv - max(uu[i, kj], 0.0)) <= 1e-4 * max(1.0, abs(uu[i, kj])), \
                        f"({r},{kj}) v {vv} vs {uu[i, kj]}"
                ii, jj = np.nonzero(sure_in)
                for i, kj in zip(ii, jj):
                    assert (int(rows[i]), int(kj)) in got, f"({rows[i]},{kj}) u={uu[i, kj]} missing"
                checked += len(got)
    assert checked > 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_support_lists_match_dense_scores(dev, dtype):
    print(f"[support] 1x2x300x300 d64 {dtype}", flush=True)
    _support_check(dev, 1, 2, 300, 300, 64, 1.5, 16, 0.125, dtype, seed=31)


def test_support_lists_nq_ne_nk_alpha2(dev):
    print("[support] 2x1x130x257 d128 alpha 2", flush=True)
    _support_check(dev, 2, 1, 130, 257, 128, 2.0, 8, 128 ** -0.5, torch.bfloat16, seed=32)
