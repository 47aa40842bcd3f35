"""alpha at the reference's clamp bounds (adasplashattention.cu:52, :547).

alpha = 1.05 (p = u^20, the general-pow path, the widest supports) and
alpha = 3.0 (p = u^0.5, a Jacobian weight P^(2-alpha) = P^-1 that grows
without bound at the support's edge), in both tau modes:
  - reference tau mode against the C oracle (masks, top-k and tau exact,
    attention 1e-5 fp32 / 2e-2 bf16) on inputs whose scores are exact in
    fp32 (see _grid_inputs);
  - exact tau mode against dense alpha-entmax attention in float64
    (tolerances of test_gpu_exact._run; at alpha = 3 tau is checked as a
    root and the passes at the GPU's tau, see the test);
and in every case the forward's status word must carry neither the score
pass's round-bound bit nor the exact mode's sweep-cap bit.  Values outside
[1.05, 3] are clamped by the reference-order entry points as the reference
does (:547).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests._util import assert_close, causal_idx, make_inputs, np32, oracle_at_gpu_tau

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}
BOUNDS = [(1.05, torch.float32), (1.05, torch.bfloat16), (3.0, torch.float32),
          (3.0, torch.bfloat16)]
IDS = [f"a{a}-{str(t).split('.')[-1]}" for a, t in BOUNDS]


def _grid_inputs(B, H, N, d, seed, dtype):
    """Q, K on a 1/16 grid within [-4, 4] (exact in bf16), V and dO ~ N(0,1).
    With sm_scale = 1/8 every product and partial sum of a score is exact in
    fp32, on MFMA and in the oracle's double dot alike, so the GPU and the
    oracle see bit-identical scores.  That matters at alpha = 3, where
    p = u^(1/2) is only Hölder-1/2 in u and its derivative u^(-1/2) (the
    gradients' weight p^(2-alpha) = 1/p) is unbounded at the support's edge:
    a last-bit score difference there moves a weight by ~sqrt(1e-7) and its
    gradient terms without bound, and the reference recurrence can stop
    with tau right next to such a key (its Halley steps shrink to nothing
    beside the kink), so random fp32 scores would test the rounding of the
    dot products rather than the kernels."""
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=seed)
    Q, K = ((torch.round(t * 16) / 16).clamp(-4, 4) for t in (Q, K))
    return tuple(t.to(dtype) for t in (Q, K, V)) + (dO,)


@pytest.mark.parametrize("mode", ["entmax", "reference"])
@pytest.mark.parametrize("alpha,dtype", BOUNDS, ids=IDS)
def test_reference_tau_mode_at_alpha_bounds(dev, alpha, dtype, mode):
    import splash_attention as sa

    B, H, N, d, k, scale = 1, 2, 256, 64, 16, 0.125
    print(f"[alpha] reference tau alpha={alpha} {dtype} {mode}", flush=True)
    Q, K, V, dO = _grid_inputs(B, H, N, d, 31, dtype)
    idx = causal_idx(B * H, N)
    q, kk, v, qi, ki = sa.ops.check_inputs(Q.to(dev), K.to(dev), V.to(dev), idx.to(dev),
                                           idx.to(dev))
    out, st = sa.ops.splash_forward(q, kk, v, qi, ki, alpha, k, scale, with_topk=True)
    grads = sa.ops.splash_backward(q, kk, v, qi, ki, out, dO.to(dev), st, alpha, k, scale, mode)
    torch.cuda.synchronize()
    st.check_status()
    m = orc.GRAD_ENTMAX if mode == "entmax" else orc.GRAD_REFERENCE
    own, fw, og = oracle_at_gpu_tau(np32(Q), np32(K), np32(V), np32(dO), idx.numpy(),
                                    idx.numpy(), alpha, scale, k, st.taus.cpu().numpy(), m)
    np.testing.assert_array_equal(st.mask.cpu().numpy(), own.mask)
    np.testing.assert_array_equal(st.topk_idx.cpu().numpy(), own.topk_idx)
    # identical scores: identical top-k values, so the recurrence agrees bit for bit
    np.testing.assert_array_equal(st.taus.cpu().numpy().view(np.uint32),
                                  own.taus.astype(np.float32).view(np.uint32))
    tol = TOL[dtype]
    errs = {"out": assert_close("out", np32(out), fw.out, tol)}
    for name, g, w in zip(("dQ", "dK", "dV"), grads, og):
        errs[name] = assert_close(name, np32(g), w, tol)
    print("  " + ", ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)


@pytest.mark.parametrize("alpha,dtype", BOUNDS, ids=IDS)
def test_exact_tau_mode_at_alpha_bounds(dev, alpha, dtype):
    from oracle import dense
    from tests.test_gpu_exact import _gpu, _run

    B, H, N, d, k, scale = 1, 2, 256, 64, 16, 0.125
    Q, K, V, dO = _grid_inputs(B, H, N, d, 32, dtype)
    if alpha <= 2.0:
        _, st, _, P, _ = _run(f"alpha{alpha}", B, H, N, N, d, alpha, k, scale, dtype, Q, K, V, dO)
        st.check_status()
        sup = (P > 0).sum(-1)
        print(f"  support size: mean {sup.mean():.1f}, max {sup.max()}", flush=True)
        return
    # alpha = 3: tau in fp32 resolves the root to an ulp, and p = u^(1/2)
    # turns an ulp of tau into ~sqrt(1e-7) at the support's edge (its
    # gradient weight 1/p into anything); the reference's weight rule
    # p = max(u, EPS)^(1/(alpha-1)) where u > 0 (cu:311-312) also makes
    # Sum p jump by EPS^(1/2) = 1e-4 wherever a key's u crosses 0, so the
    # root can sit on a jump.  So tau is checked as the root at fp32
    # resolution (Sum p - 1 changes sign within a few ulps of it, in float64
    # with the weight rule), and the passes at the GPU's tau against float64
    # dense attention with the same weights (P = p / (Sum p + EPS)).
    print(f"[alpha] exact tau alpha={alpha} {dtype}", flush=True)
    idx = causal_idx(B * H, N)
    out, st, grads = _gpu(dev, Q, K, V, dO, idx, idx, alpha, k, scale)
    st.check_status()
    q, kk, v, do = np32(Q), np32(K), np32(V), np32(dO)
    vis = idx.numpy()[:, None, :] <= idx.numpy()[:, :, None]
    S = np.clip(np.einsum("bid,bjd->bij", q.astype(np.float64), kk.astype(np.float64)) * scale,
                -10, 10)
    tg = st.taus.cpu().numpy().astype(np.float64)

    def weights(t):
        uu = (alpha - 1.0) * S - t[:, :, None]
        return np.where(vis & (uu > 0), np.maximum(uu, 1e-8), 0.0) ** (1.0 / (alpha - 1.0))

    w = weights(tg)
    ulp = np.spacing(np.abs(st.taus.cpu().numpy())).astype(np.float64)
    f_lo = weights(tg - 4 * ulp).sum(-1) - 1.0
    f_hi = weights(tg + 4 * ulp).sum(-1) - 1.0
    assert (f_lo >= -1e-6).all() and (f_hi <= 1e-6).all(), "tau does not bracket the root"
    resid = float(np.abs(w.sum(-1) - 1.0).max())
    td = np.array([[dense.tau_bisect(S[b, i, vis[b, i]], alpha) for i in range(N)]
                   for b in range(B * H)])
    dtau = float(np.abs(td - tg).max())
    P = w / (w.sum(-1, keepdims=True) + 1e-8)
    want = np.einsum("bij,bjd->bid", P, v.astype(np.float64))
    dq, dk, dv = dense.attention_backward(q, kk, v, P, do, alpha, scale)
    tol = TOL[dtype]
    errs = {"out": assert_close("out", np32(out), want, tol)}
    for name, g, ww in zip(("dQ", "dK", "dV"), grads, (dq, dk, dv)):
        errs[name] = assert_close(name, np32(g), ww, max(tol, 1e-4))
    print(f"  residual {resid:.1e}, |dtau| {dtau:.1e}; "
          + ", ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)


def test_reference_order_calls_clamp_alpha(dev):
    """alpha outside [1.05, 3] is clamped (adasplashattention.cu:547): the
    results equal those at the bounds bit for bit."""
    import splash_attention as sa

    B, H, N, d = 1, 2, 128, 64
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=33)
    idx = causal_idx(B * H, N).to(dev)
    args = (Q.to(dev), K.to(dev), V.to(dev), idx, idx, 0.125)
    for outside, bound in ((1.0, 1.05), (0.5, 1.05), (3.5, 3.0), (10.0, 3.0)):
        assert torch.equal(sa.forward(*args, outside), sa.forward(*args, bound))
        for a, b in zip(sa.backward(*args, outside, dO.to(dev)),
                        sa.backward(*args, bound, dO.to(dev))):
            assert torch.equal(a, b)
