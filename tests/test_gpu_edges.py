"""Edge cases of the reference's semantics on the GPU vs the CPU oracle.

Rows that see no key, one-row and one-key problems, non-finite values (the
reference zeroes non-finite outputs, adasplashattention.cu:335-337),
non-positive sm_scale (the score pass then filters on exact scores), many
tiny heads and a long sequence checked on sampled query blocks.
Tolerances: 1e-5 relative (fp32), 2e-2 relative (bf16); masks exact.
"""
import numpy as np
import pytest
import torch

import splash_attention as sa
from oracle import oracle as orc
from tests._util import (assert_close, assert_tau_close, causal_idx, make_inputs, np32,
                         oracle_at_gpu_tau)

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def _run(dev, Q, K, V, dO, qi, ki, alpha, k, scale, mode="entmax"):
    q, kk, v, qi_, ki_ = sa.ops.check_inputs(Q.to(dev), K.to(dev), V.to(dev), qi.to(dev),
                                             ki.to(dev))
    out, st = sa.ops.splash_forward(q, kk, v, qi_, ki_, alpha, k, scale)
    grads = None
    if dO is not None:
        grads = sa.ops.splash_backward(q, kk, v, qi_, ki_, out, dO.to(dev), st, alpha, k, scale,
                                       mode)
    torch.cuda.synchronize()
    return out, st, grads


def _check_all(name, dtype, Q, K, V, dO, qi, ki, alpha, k, scale, mode, out, st, grads,
               floor=1e-30):
    m = orc.GRAD_ENTMAX if mode == "entmax" else orc.GRAD_REFERENCE
    own, fw, og = oracle_at_gpu_tau(np32(Q), np32(K), np32(V), np32(dO), qi.numpy(), ki.numpy(),
                                    alpha, scale, k, st.taus.cpu().numpy(), m)
    np.testing.assert_array_equal(st.mask.cpu().numpy(), own.mask, err_msg=f"{name}: mask")
    assert_tau_close(st.taus.cpu().numpy(), own.taus, alpha)
    tol = TOL[dtype]
    assert_close(f"{name}: out", np32(out), fw.out, tol)
    for gname, gg, w in zip(("dQ", "dK", "dV"), grads, og):
        assert_close(f"{name}: {gname}", np32(gg), w, tol, floor)


@pytest.mark.parametrize("mode", ["entmax", "reference"])
def test_rows_without_visible_keys(dev, mode):
    """Rows whose position precedes every key see nothing: out = 0, zero
    gradients, tau from the all-empty top-k (sentinel bracket)."""
    print(f"[edge] rows without visible keys {mode}", flush=True)
    B, H, NQ, NK, d = 1, 2, 130, 150, 64
    Q, K, V, dO = make_inputs(B, H, NQ, NK, d, seed=21)
    qi = causal_idx(B * H, NQ) + 20
    qi[:, 5:9] = -1
    qi[1, 70:140] = -3
    ki = causal_idx(B * H, NK)
    out, st, grads = _run(dev, Q, K, V, dO, qi, ki, 1.5, 8, 0.125, mode)
    o = out.reshape(B * H, NQ, d).cpu()
    assert torch.all(o[:, 5:9] == 0) and torch.all(o[1, 70:] == 0)
    _check_all("no-keys", torch.float32, Q, K, V, dO, qi, ki, 1.5, 8, 0.125, mode, out, st, grads)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("NQ,NK", [(1, 1), (1, 65), (65, 1), (3, 200)])
def test_tiny_problems(dev, dtype, NQ, NK):
    print(f"[edge] tiny NQ={NQ} NK={NK} {dtype}", flush=True)
    B, H, d = 2, 1, 64
    Q, K, V, dO = make_inputs(B, H, NQ, NK, d, seed=22, dtype=dtype)
    qi = torch.full((B * H, NQ), NK - 1, dtype=torch.int32)  # every key visible
    ki = causal_idx(B * H, NK)
    out, st, grads = _run(dev, Q, K, V, dO, qi, ki, 1.5, 4, 0.125)
    # with one visible key dQ and dK are zero in exact arithmetic: compare
    # them on the scale of the unit-normal inputs
    _check_all(f"tiny{NQ}x{NK}", dtype, Q, K, V, dO, qi, ki, 1.5, 4, 0.125, "entmax", out, st,
               grads, floor=1.0)


def test_nonfinite_values_are_zeroed(dev):
    """inf / NaN in V: outputs stay finite (non-finite results are zeroed,
    as the reference does at adasplashattention.cu:335-337).  The reference
    zeroes the affected dimension in the rows that see the bad key; the MFMA
    product also multiplies the keys a row does not see by a zero weight,
    and 0 * NaN is NaN, so here that dimension can also come out zero in
    rows of the same query block that do not see the key.  Every other
    element matches the oracle."""
    print("[edge] non-finite V", flush=True)
    B, H, N, d = 1, 1, 128, 64
    Q, K, V, _ = make_inputs(B, H, N, N, d, seed=23)
    V[0, 0, 3, 7] = float("inf")
    V[0, 0, 40, 0] = float("nan")
    idx = causal_idx(1, N)
    out, st, _ = _run(dev, Q, K, V, None, idx, idx, 1.5, 8, 0.125)
    assert torch.isfinite(out).all()
    own = orc.forward(np32(Q), np32(K), np32(V), idx.numpy(), idx.numpy(), 1.5, 0.125, 8)
    at = orc.forward(np32(Q), np32(K), np32(V), idx.numpy(), idx.numpy(), 1.5, 0.125, 8,
                     taus_in=st.taus.cpu().numpy())
    np.testing.assert_array_equal(st.mask.cpu().numpy(), own.mask)
    got, want = np32(out)[0], at.out[0]
    clean = [t for t in range(d) if t not in (0, 7)]
    assert_close("non-finite: clean dims", got[:, clean], want[:, clean], 1e-5)
    for t in (0, 7):
        col_ok = (got[:, t] == 0) | (np.abs(got[:, t] - want[:, t]) <= 1e-5 * np.abs(want).max())
        assert col_ok.all(), f"dim {t}: neither zero nor the oracle's value"
        assert np.all(got[want[:, t] == 0, t] == 0), f"dim {t}: oracle-zeroed element kept"


@pytest.mark.parametrize("scale", [-0.125, 0.0])
def test_nonpositive_scale(dev, scale):
    """sm_scale <= 0: the score pass filters on exact clamped scores."""
    print(f"[edge] sm_scale {scale}", flush=True)
    B, H, N, d = 1, 2, 192, 64
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=24)
    idx = causal_idx(B * H, N)
    out, st, grads = _run(dev, Q, K, V, dO, idx, idx, 1.5, 8, scale)
    _check_all(f"scale{scale}", torch.float32, Q, K, V, dO, idx, idx, 1.5, 8, scale, "entmax",
               out, st, grads)


def test_many_tiny_heads(dev):
    print("[edge] 8x32 heads of 64 rows bf16", flush=True)
    B, H, N, d = 8, 32, 64, 64
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=25, dtype=torch.bfloat16)
    idx = causal_idx(B * H, N)
    out, st, grads = _run(dev, Q, K, V, dO, idx, idx, 2.0, 16, 0.125)
    _check_all("tiny-heads", torch.bfloat16, Q, K, V, dO, idx, idx, 2.0, 16, 0.125, "entmax",
               out, st, grads)


def test_long_sequence_sampled_blocks(dev):
    """N = 16384 fp32 causal: 64-row query blocks at the start, middle and
    end against the oracle (rows of different blocks are independent given
    all keys): tau, mask row, out and dQ."""
    print("[edge] long sequence fp32 1x2x16384x64", flush=True)
    B, H, N, d = 1, 2, 16384, 64
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=26)
    idx = causal_idx(B * H, N)
    out, st, grads = _run(dev, Q, K, V, dO, idx, idx, 1.5, 8, 0.125)
    assert torch.isfinite(out).all()
    for bh in (0, 1):
        for q0 in (0, 8192, N - 64):
            qs = slice(q0, q0 + 64)
            sl = lambda t: np32(t[0:1, bh:bh + 1, qs])
            own, fw, og = oracle_at_gpu_tau(sl(Q), np32(K[0:1, bh:bh + 1]),
                                            np32(V[0:1, bh:bh + 1]), sl(dO),
                                            idx[bh:bh + 1, qs].numpy(), idx[bh:bh + 1].numpy(),
                                            1.5, 0.125, 8, st.taus[bh:bh + 1, qs].cpu().numpy())
            assert_tau_close(st.taus[bh:bh + 1, qs].cpu().numpy(), own.taus, 1.5)
            np.testing.assert_array_equal(
                st.mask[bh:bh + 1, q0 // 64:q0 // 64 + 1].cpu().numpy(), own.mask)
            assert_close(f"long out[{bh},{q0}]", sl(out), fw.out, 1e-5)
            assert_close(f"long dQ[{bh},{q0}]", sl(grads[0]), og[0], 1e-5)
