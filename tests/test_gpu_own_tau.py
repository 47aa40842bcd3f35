"""configs[0] (c1) and configs[1] (c2), fp32, against the oracle at the
oracle's own tau (no GPU value fed back into it).

The reference's tau recurrence stops the first time |f| < 1e-4
(adasplashattention.cu:92); the GPU's MFMA scores and the oracle's
double-precision dot products differ in the last bit, which can end the
recurrence one step apart on a few rows.  So:
  - every row whose tau matches the oracle's to 1e-6 (relative, floor 1):
    out and dQ within 1e-5 of the oracle's, relative to the tensor's
    max-norm;
  - every key outside the supports of the rows that do not match: dK and
    dV within 1e-5 (a key's gradient sums over the rows that weight it);
  - the rows that do not match are counted and bounded: at most 2 (c1) or
    16 (c2) of them, tau within 1e-4, and their out / dQ, and the dK / dV
    of the keys they weight, within 1e-4.
Block masks are compared exactly.  Both gradient modes.
"""
import numpy as np
import pytest
import torch

import splash_attention as sa
from oracle import oracle as orc
from tests._util import causal_idx, make_inputs, np32

pytestmark = pytest.mark.gpu


def _gauss(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g)


def _c1():
    Q, K, V, dO = make_inputs(1, 2, 256, 256, 64, seed=0)
    return Q, K, V, dO, 8


def _c2():
    shape = (2, 8, 1024, 64)
    return _gauss(shape, 0), _gauss(shape, 1), _gauss(shape, 2), _gauss(shape, 3), 8


@pytest.mark.parametrize("mode", ["entmax", "reference"])
@pytest.mark.parametrize("cfg", ["c1", "c2"])
def test_parity_at_oracle_tau(dev, cfg, mode):
    Q, K, V, dO, k = _c1() if cfg == "c1" else _c2()
    B, H, N, d = Q.shape
    alpha, scale = 1.5, 0.125
    print(f"[own tau] {cfg} {B}x{H}x{N}x{d} fp32 k={k} {mode}", flush=True)
    idx = causal_idx(B * H, N)
    q, kk, v, qi, ki = sa.ops.check_inputs(Q.to(dev), K.to(dev), V.to(dev), idx.to(dev),
                                           idx.to(dev))
    out, st = sa.ops.splash_forward(q, kk, v, qi, ki, alpha, k, scale)
    grads = sa.ops.splash_backward(q, kk, v, qi, ki, out, dO.to(dev), st, alpha, k, scale, mode)
    torch.cuda.synchronize()
    m = orc.GRAD_ENTMAX if mode == "entmax" else orc.GRAD_REFERENCE
    Qn, Kn, Vn, dOn = np32(Q), np32(K), np32(V), np32(dO)
    fw = orc.forward(Qn, Kn, Vn, idx.numpy(), idx.numpy(), alpha, scale, k)
    og = orc.backward(Qn, Kn, Vn, idx.numpy(), idx.numpy(), dOn, alpha, scale, fw.taus,
                      fw.csr.q_ptr, fw.csr.q_list, m)
    np.testing.assert_array_equal(st.mask.cpu().numpy(), fw.mask)

    gt = st.taus.cpu().numpy().astype(np.float64)
    ot = fw.taus.astype(np.float64)
    match = np.abs(gt - ot) <= 1e-6 * np.maximum(1.0, np.abs(ot))  # [BH, N]
    nbad = int((~match).sum())

    def rowerr(got, want):  # per-row max error relative to the tensor's max-norm
        got = np.asarray(got, np.float64)
        want = np.asarray(want, np.float64)
        return np.abs(got - want).max(-1) / max(np.abs(want).max(), 1e-30)

    e_out = rowerr(np32(out), fw.out)
    e_dq = rowerr(np32(grads[0]), og[0])
    assert float(e_out[match].max()) <= 1e-5, f"out {float(e_out[match].max()):.2e}"
    assert float(e_dq[match].max()) <= 1e-5, f"dQ {float(e_dq[match].max()):.2e}"

    # keys that a non-matching row may weight: visible, active, and with
    # u > -1e-5 at the smaller of the two taus
    S, vis = orc.scores(Qn, Kn, idx.numpy(), idx.numpy(), scale)
    am1 = alpha - 1.0
    tmin = np.minimum(gt, ot)
    nQB, nKB = fw.mask.shape[1], fw.mask.shape[2]
    active = np.repeat(np.repeat(fw.mask.astype(bool), 64, 1), 64, 2)[:, :N, :N]
    near = vis.astype(bool) & active & (am1 * S - tmin[:, :, None] > -1e-5)
    tainted = (near & ~match[:, :, None]).any(1)  # [BH, NK]
    e_dk = rowerr(np32(grads[1]), og[1])
    e_dv = rowerr(np32(grads[2]), og[2])
    clean = ~tainted
    assert float(e_dk[clean].max()) <= 1e-5, f"dK {float(e_dk[clean].max()):.2e}"
    assert float(e_dv[clean].max()) <= 1e-5, f"dV {float(e_dv[clean].max()):.2e}"
    dtau = float(np.abs(gt - ot).max())
    msg = (f"[own tau] {cfg} {mode}: {nbad} of {match.size} rows with tau off by > 1e-6 "
           f"(max |dtau| {dtau:.2e}); {int(tainted.sum())} of "
           f"{tainted.size} keys in their supports")
    if nbad:
        msg += (f"; on those rows out err {float(e_out[~match].max()):.2e}, "
                f"dQ err {float(e_dq[~match].max()):.2e}; on those keys dK err "
                f"{float(e_dk[tainted].max()):.2e}, dV err {float(e_dv[tainted].max()):.2e}")
    print(msg, flush=True)
    # The non-matching rows are the recurrence's one-step discontinuity, not
    # a drift: few of them (observed 0 at c1, 7 at c2), tau one small Halley
    # step apart (observed 3.05e-5), and their outputs and gradients within
    # 1e-4 (observed 2.1e-5 out, 3.7e-5 dQ).  A regression that made the
    # discontinuity several times more common or larger fails here.
    assert nbad <= {"c1": 2, "c2": 16}[cfg], f"{nbad} rows off the oracle's tau"
    assert dtau <= 1e-4, f"max |dtau| {dtau:.2e}"
    if nbad:
        assert float(e_out[~match].max()) <= 1e-4, f"out on tau-mismatched rows"
        assert float(e_dq[~match].max()) <= 1e-4, f"dQ on tau-mismatched rows"
        assert float(e_dk[tainted].max()) <= 1e-4, f"dK on their support keys"
        assert float(e_dv[tainted].max()) <= 1e-4, f"dV on their support keys"
