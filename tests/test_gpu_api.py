"""GPU tests of the user-facing API against the CPU oracle.

Tolerances: max |gpu - oracle| / max |oracle| <= 1e-5 (fp32), 2e-2 (bf16).
"""
import os

import numpy as np
import pytest
import torch

import splash_attention as sa
from oracle import oracle as orc
from tests._util import assert_close, causal_idx, make_inputs, np32

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_module_autograd_matches_oracle(dev):
    print("[api] module autograd fp32 1x2x256x64", flush=True)
    B, H, N, d = 1, 2, 256, 64
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=3)
    attn = sa.AdaptiveSplashAttention(head_dim=64, alpha=1.5, k_keep=8, sm_scale=0.125)
    q, k, v = (t.to(dev).requires_grad_(True) for t in (Q, K, V))
    idx = causal_idx(B * H, N).to(dev)
    out = attn(q, k, v, idx, idx)
    out.backward(dO.to(dev))
    fw, (gq, gk, gv) = orc.attention(np32(Q), np32(K), np32(V), idx.cpu().numpy(),
                                     idx.cpu().numpy(), np32(dO), 1.5, 0.125, 8)
    assert_close("out", np32(out), fw.out, 1e-5)
    assert_close("dQ", np32(q.grad), gq, 1e-5)
    assert_close("dK", np32(k.grad), gk, 1e-5)
    assert_close("dV", np32(v.grad), gv, 1e-5)


def _magnets(BH, N, d, seed=3):
    """Half h of the queries (32 rows) has its top-2 keys in key block h % 4
    (every key visible), so the two 32-row halves of each 64-row block
    select different key blocks: 32-row and 64-row mask blocks then give
    outputs that differ by O(1)."""
    rng = np.random.default_rng(seed)
    Q = rng.normal(size=(BH, N, d)) * 0.1
    K = rng.normal(size=(BH, N, d)) * 0.1
    V = rng.normal(size=(BH, N, d))
    dO = rng.normal(size=(BH, N, d))
    for h in range(N // 32):
        Q[:, 32 * h:32 * h + 32, h] += 1.0
        K[:, 64 * (h % 4) + h, h] = 5.0
        K[:, 64 * (h % 4) + 8 + h, h] = 4.0
    t = [torch.from_numpy(x.astype(np.float32)).reshape(1, BH, N, d) for x in (Q, K, V, dO)]
    qi = torch.full((BH, N), N - 1, dtype=torch.int32)
    return (*t, qi, causal_idx(BH, N))


@pytest.mark.parametrize("case", ["c1", "magnets"])
def test_reference_style_entry_points(dev, case):
    """sa.forward / sa.backward take the reference's argument order
    (adasplashattention.cu:537-541, :611-616), default to its compiled
    BLOCK_M = 32 (:8-9), and return its gradient.  On the "magnets" inputs
    a 64-row default would be off by O(1) (checked against the oracle)."""
    print(f"[api] reference-style forward/backward {case}", flush=True)
    if case == "c1":
        B, H, N, d = 1, 2, 192, 64
        Q, K, V, dO = make_inputs(B, H, N, N, d, seed=4)
        qi = ki = causal_idx(B * H, N)
        kw, k = {}, 8          # the reference's compiled K_KEEP
    else:
        Q, K, V, dO, qi, ki = _magnets(2, 256, 64)
        kw, k = {"k_keep": 2}, 2
    args = (Q.to(dev), K.to(dev), V.to(dev), qi.to(dev), ki.to(dev), 0.125, 1.5)
    out = sa.forward(*args, **kw)
    dQ, dK, dV = sa.backward(*args, dO.to(dev), **kw)
    fw, (gq, gk, gv) = orc.attention(np32(Q), np32(K), np32(V), qi.numpy(), ki.numpy(),
                                     np32(dO), 1.5, 0.125, k, mode=orc.GRAD_REFERENCE,
                                     block_m=32)
    assert_close("out", np32(out), fw.out, 1e-5)
    assert_close("dQ", np32(dQ), gq, 1e-5)
    assert_close("dK", np32(dK), gk, 1e-5)
    assert_close("dV", np32(dV), gv, 1e-5)
    if case == "magnets":
        fw64 = orc.forward(np32(Q), np32(K), np32(V), qi.numpy(), ki.numpy(), 1.5, 0.125, k,
                           block_m=64)
        assert float(np.abs(fw64.out - fw.out).max()) > 1e-2


def test_reference_host_fixup_clamps_overflowed_dv(dev):
    """The reference's host fix-up (adasplashattention.cu:684-697): a dV sum
    that overflows (fp32 atomics there, fp32 registers here) is +inf, and
    any inf clamps the whole tensor to [-100, 100] with a warning.  Rows
    0-3 see only key 0 (weight 1 each), and dO's column 0 is 3e38, so
    dV[key 0, 0] = 4 * 3e38 overflows; V is scaled by 1e-6 so that
    dp = dO . v stays finite and dQ, dK are ordinary (large) numbers."""
    print("[api] host fix-up: overflowing dV", flush=True)
    B, H, N, d = 1, 1, 128, 64
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=11)
    V = V * 1e-6
    dO[..., 0] = 3e38
    qi = causal_idx(1, N)
    qi[:, :4] = 0
    ki = causal_idx(1, N)
    args = (Q.to(dev), K.to(dev), V.to(dev), qi.to(dev), ki.to(dev), 0.125, 1.5)
    with pytest.warns(RuntimeWarning, match="Inf values detected in dV, clamping"):
        dQ, dK, dV = sa.backward(*args, dO.to(dev))
    assert float(dV.abs().max()) <= 100.0 and torch.isfinite(dV).all()
    fw, (gq, gk, gv) = orc.attention(np32(Q), np32(K), np32(V), qi.numpy(), ki.numpy(),
                                     np32(dO), 1.5, 0.125, 8, mode=orc.GRAD_REFERENCE,
                                     block_m=32)
    assert np.isinf(gv).any()          # the oracle's sum overflows too
    want, nan, inf = orc.host_fixup(gv)
    assert inf and not nan
    assert_close("dV (fixed up)", np32(dV), want, 1e-5)
    assert_close("dQ", np32(dQ), gq, 1e-5)
    assert_close("dK", np32(dK), gk, 1e-5)
    # opting out returns the raw sums: the overflowed element is +inf
    raw = sa.backward(*args, dO.to(dev), fix_nonfinite=False)[2]
    assert bool(torch.isinf(raw).any())
    assert torch.equal(torch.clamp(raw, -100, 100), dV)


def test_reference_style_default_scale_uses_callers_head_dim(dev):
    """sm_scale=None in the reference-order entry points is 1/sqrt(d) of the
    caller's d (here 40, zero-padded to 64 inside), not of the padded d."""
    print("[api] reference-style sm_scale=None, d=40", flush=True)
    B, H, N, d = 1, 2, 160, 40
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=7)
    idx = causal_idx(B * H, N).to(dev)
    args = (Q.to(dev), K.to(dev), V.to(dev), idx, idx)
    a = sa.forward(*args, None, 1.5)
    b = sa.forward(*args, d ** -0.5, 1.5)
    assert torch.equal(a, b)
    ga = sa.backward(*args, None, 1.5, dO.to(dev))
    gb = sa.backward(*args, d ** -0.5, 1.5, dO.to(dev))
    for x, y in zip(ga, gb):
        assert torch.equal(x, y)
    fw, _ = orc.attention(np32(Q), np32(K), np32(V), idx.cpu().numpy(), idx.cpu().numpy(),
                          np32(dO), 1.5, d ** -0.5, 8, mode=orc.GRAD_REFERENCE, block_m=32)
    assert_close("out", np32(a), fw.out, 1e-5)


def test_default_int64_arange_indices_are_accepted(dev):
    """README.md:120-121 passes int64 arange indices (the reference would
    reject them, adasplashattention.cu:571); they are converted."""
    B, H, N, d = 1, 1, 128, 64
    Q, K, V, _ = make_inputs(B, H, N, N, d, seed=5)
    i64 = torch.arange(N, device=dev).expand(B * H, N).contiguous()
    a = sa.forward(Q.to(dev), K.to(dev), V.to(dev), i64, i64, 0.125, 1.5)
    b = sa.forward(Q.to(dev), K.to(dev), V.to(dev), i64.int(), i64.int(), 0.125, 1.5)
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_deterministic(dev, dtype):
    print(f"[api] determinism {dtype}", flush=True)
    B, H, N, d = 2, 2, 320, 64
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=6, dtype=dtype)
    res = []
    for _ in range(2):
        q, k, v = (t.to(dev).requires_grad_(True) for t in (Q, K, V))
        out = sa.splash_attention(q, k, v, None, None, 1.5, 16, 0.125)
        out.backward(dO.to(dev))
        res.append([x.detach().cpu() for x in (out, q.grad, k.grad, v.grad)])
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_golden_fixture_on_gpu(dev):
    g = dict(np.load(os.path.join(GOLDEN, "c1_head0.npz")))
    print("[api] golden c1_head0 fp32", flush=True)
    t = lambda a: torch.from_numpy(a).unsqueeze(0).to(dev)  # [1, 1, N, d]
    q, k, v = t(g["Q"]), t(g["K"]), t(g["V"])
    qi = torch.from_numpy(g["idx"]).to(dev)
    q, k, v, qi, ki = sa.ops.check_inputs(q, k, v, qi, qi)
    out, st = sa.ops.splash_forward(q, k, v, qi, ki, float(g["alpha"]), int(g["k"]),
                                    float(g["scale"]), with_topk=True)
    np.testing.assert_array_equal(st.mask.cpu().numpy(), g["mask"])
    np.testing.assert_array_equal(st.q_list.cpu().numpy(), g["q_list"])
    assert_close("taus", st.taus.cpu().numpy(), g["taus"], 1e-5)
    assert_close("out", np32(out), g["out"], 1e-5)
    for mode in ("entmax", "reference"):
        grads = sa.ops.splash_backward(q, k, v, qi, ki, out, t(g["dO"]), st, float(g["alpha"]),
                                       int(g["k"]), float(g["scale"]), mode)
        for name, x in zip(("dQ", "dK", "dV"), grads):
            assert_close(f"{name}/{mode}", np32(x), g[f"{name}_{mode}"], 1e-5)


def test_nan_scores_follow_reference_clamp(dev):
    """A NaN score clamps to -10 (fmaxf/fminf, adasplashattention.cu:196-197);
    the output stays finite and matches the oracle's identical rule."""
    B, H, N, d = 1, 1, 128, 64
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=8)
    Q[0, 0, 5, :] = float("nan")
    K[0, 0, 17, 3] = float("nan")
    idx = causal_idx(1, N)
    out = sa.forward(Q.to(dev), K.to(dev), V.to(dev), idx.to(dev), idx.to(dev), 0.125, 1.5)
    assert torch.isfinite(out).all()
    fw = orc.forward(np32(Q), np32(K), np32(V), idx.numpy(), idx.numpy(), 1.5, 0.125, 8,
                     block_m=32)
    assert_close("out", np32(out), fw.out, 1e-5)


def test_noncausal_positions_and_nq_ne_nk(dev):
    """Non-causal attention expressed by positions (Q_idx = NK-1), NQ != NK."""
    B, H, NQ, NK, d = 1, 2, 96, 200, 64
    Q, K, V, dO = make_inputs(B, H, NQ, NK, d, seed=9)
    qi = torch.full((B * H, NQ), NK - 1, dtype=torch.int32)
    ki = causal_idx(B * H, NK)
    q, k, v = (t.to(dev).requires_grad_(True) for t in (Q, K, V))
    out = sa.splash_attention(q, k, v, qi.to(dev), ki.to(dev), 2.0, 16, 0.125)
    out.backward(dO.to(dev))
    fw, (gq, gk, gv) = orc.attention(np32(Q), np32(K), np32(V), qi.numpy(), ki.numpy(),
                                     np32(dO), 2.0, 0.125, 16)
    assert_close("out", np32(out), fw.out, 1e-5)
    assert_close("dQ", np32(q.grad), gq, 1e-5)
    assert_close("dK", np32(k.grad), gk, 1e-5)
    assert_close("dV", np32(v.grad), gv, 1e-5)


def test_non_contiguous_inputs(dev):
    B, H, N, d = 1, 2, 128, 64
    Q, K, V, _ = make_inputs(B, H, N, N, d, seed=10)
    # [B, N, H, d] storage viewed as [B, H, N, d]
    qt, kt, vt = (t.transpose(1, 2).contiguous().transpose(1, 2).to(dev) for t in (Q, K, V))
    assert not qt.is_contiguous()
    idx = causal_idx(B * H, N).to(dev)
    a = sa.forward(qt, kt, vt, idx, idx, 0.125, 1.5)
    b = sa.forward(Q.to(dev), K.to(dev), V.to(dev), idx, idx, 0.125, 1.5)
    assert torch.equal(a, b)
