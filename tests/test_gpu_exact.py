"""Exact tau mode on the GPU vs dense alpha-entmax attention (float64).

tau_mode="exact" solves the alpha-entmax threshold over every visible key
of a row and activates the key blocks of its support, so the block-sparse
forward must equal dense alpha-entmax attention (oracle/dense.py: bisection
in float64, pinned by the sort-based closed forms in test_oracle_pins.py),
and the entmax-mode gradients must equal its exact Jacobian gradients.

Tolerances (max |gpu - oracle| / max |oracle| per tensor): 1e-5 for fp32,
2e-2 for bf16 (gradients at alpha > 2: 1e-4, see _run); tau to 1e-5
(absolute, tau is O(1)).  Block masks: the
reference's top-k union (the C oracle's mask) plus every key block that
holds a dense support key with p > 1e-7, and nothing outside the top-k
union whose best key has u <= -1e-5 at the dense threshold.
"""
import numpy as np
import pytest
import torch

from oracle import dense
from oracle import oracle as orc
from tests._util import assert_close, causal_idx, make_inputs, np32

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def _vis(qidx, kidx):
    return kidx.numpy()[:, None, :] <= qidx.numpy()[:, :, None]


def _gpu(dev, Q, K, V, dO, qidx, kidx, alpha, k, scale):
    import splash_attention as sa

    q, kk, v, qi, ki = sa.ops.check_inputs(*(t.to(dev) for t in (Q, K, V, qidx, kidx)))
    out, st = sa.ops.splash_forward(q, kk, v, qi, ki, alpha, k, scale, tau_mode="exact")
    grads = sa.ops.splash_backward(q, kk, v, qi, ki, out, dO.to(dev), st, alpha, k, scale,
                                   "entmax")
    torch.cuda.synchronize()
    return out, st, grads


def _block_any(m, bm=64, bn=64):
    """[BH, NQ, NK] bool -> [BH, nQB, nKB]: any element in the block."""
    BH, NQ, NK = m.shape
    nqb, nkb = -(-NQ // bm), -(-NK // bn)
    pad = np.zeros((BH, nqb * bm, nkb * bn), bool)
    pad[:, :NQ, :NK] = m
    return pad.reshape(BH, nqb, bm, nkb, bn).any(axis=(2, 4))


def _run(name, B, H, NQ, NK, d, alpha, k, scale, dtype, Q=None, K=None, V=None, dO=None,
         qidx=None, kidx=None, seed=0):
    dev = torch.device("cuda:0")
    if Q is None:
        Q, K, V, dO = make_inputs(B, H, NQ, NK, d, seed=seed, dtype=dtype)
    BH = B * H
    qidx = causal_idx(BH, NQ) if qidx is None else qidx
    kidx = causal_idx(BH, NK) if kidx is None else kidx
    print(f"exact {name}: B={B} H={H} NQ={NQ} NK={NK} d={d} alpha={alpha} k={k} {dtype}",
          flush=True)
    out, st, grads = _gpu(dev, Q, K, V, dO, qidx, kidx, alpha, k, scale)

    q, kk, v, do = np32(Q), np32(K), np32(V), np32(dO)
    vis = _vis(qidx, kidx)
    ref_out, P, taus = dense.attention_forward(q, kk, v, vis, alpha, scale)
    dq, dk, dv = dense.attention_backward(q, kk, v, P, do, alpha, scale)
    seen = vis.any(-1)
    tol = TOL[dtype]

    gt = st.taus.cpu().numpy()
    dt = float(np.abs(gt - taus)[seen].max()) if seen.any() else 0.0
    assert dt <= (1e-5 if dtype == torch.float32 else 2e-2), f"{name}: tau differs by {dt:.2e}"
    errs = {"tau": dt, "out": assert_close(f"{name}: out", np32(out), ref_out, tol)}
    # alpha > 2: the Jacobian weight g = P^(2-alpha) has a negative exponent
    # and grows without bound as P -> 0, so keys at the support boundary
    # amplify the last-bit rounding of tau; the gradients get 1e-4 there
    gtol = max(tol, 1e-4) if alpha > 2.0 else tol
    for gname, g, w in zip(("dQ", "dK", "dV"), grads, (dq, dk, dv)):
        errs[gname] = assert_close(f"{name}: {gname}", np32(g), w, gtol)

    # block mask: top-k union plus the dense support's blocks
    S = np.clip(np.einsum("bid,bjd->bij", q.astype(np.float64), kk.astype(np.float64)) * scale,
                -10, 10)
    u = (alpha - 1.0) * S - taus[:, :, None]
    topk = orc.forward(q, kk, v, qidx.numpy(), kidx.numpy(), alpha, scale, k).mask.astype(bool)
    gm = st.mask.cpu().numpy().astype(bool)
    if dtype == torch.float32:
        strict = topk | _block_any((P > 1e-7) & vis)
        loose = topk | _block_any((u > -1e-5) & vis)
        assert not (strict & ~gm).any(), f"{name}: a support block is missing from the mask"
        assert not (gm & ~loose).any(), f"{name}: a block without support is in the mask"
    extra = int((gm & ~topk).sum())
    print(f"  {name}: " + ", ".join(f"{n}={e:.2e}" for n, e in errs.items())
          + f", blocks added to the top-k mask: {extra}", flush=True)
    return out, st, grads, P, extra


CASES = [
    # name, B, H, NQ, NK, d, alpha, k, scale, dtype
    ("c1_fp32", 1, 2, 256, 256, 64, 1.5, 8, 0.125, torch.float32),
    ("fp32_sparsemax_d128", 1, 2, 192, 192, 128, 2.0, 16, 128 ** -0.5, torch.float32),
    ("fp32_a125", 1, 2, 256, 256, 64, 1.25, 8, 0.125, torch.float32),
    ("fp32_alpha_general", 1, 1, 128, 128, 64, 1.7, 8, 0.125, torch.float32),
    ("fp32_alpha_above_2", 1, 1, 128, 128, 64, 2.5, 8, 0.125, torch.float32),
    ("fp32_ragged_k1", 2, 1, 100, 150, 64, 1.5, 1, 0.125, torch.float32),
    ("bf16_k32", 1, 2, 512, 512, 64, 1.5, 32, 0.125, torch.bfloat16),
    ("bf16_d128_a125", 1, 2, 256, 256, 128, 1.25, 64, 128 ** -0.5, torch.bfloat16),
]


@pytest.mark.parametrize("name,B,H,NQ,NK,d,alpha,k,scale,dtype", CASES, ids=[c[0] for c in CASES])
def test_exact_mode_equals_dense_entmax(name, B, H, NQ, NK, d, alpha, k, scale, dtype):
    _run(name, B, H, NQ, NK, d, alpha, k, scale, dtype)


def test_exact_mode_clustered_noncausal():
    """BASELINE configs[3]'s input family (keys around cluster centres,
    queries near random centres, non-causal, sparsemax) at a small size:
    every row's support exceeds k, so every row takes full sweeps.

    Sparsemax over such near-tied scores passes any score rounding straight
    into the output (p = s - tau over ~15 keys), so Q and K are quantised to
    multiples of 1/16 within [-4, 4] and the scale is 1/8: every product and
    partial sum is then exact in float32, on MFMA and in the float64 oracle
    alike, and the comparison isolates the threshold and the passes."""
    B, H, N, d, k, alpha, scale = 1, 2, 256, 64, 8, 2.0, 0.125
    g = torch.Generator().manual_seed(3)
    C = torch.randn(B, H, 8, d, generator=g)
    kc = torch.randint(0, 8, (B, H, N), generator=g)
    K = torch.gather(C, 2, kc[..., None].expand(B, H, N, d)) + 0.1 * torch.randn(B, H, N, d, generator=g)
    qc = torch.randint(0, 8, (B, H, N), generator=g)
    Q = torch.gather(C, 2, qc[..., None].expand(B, H, N, d)) + 0.1 * torch.randn(B, H, N, d, generator=g)
    Q, K = ((torch.round(t * 16) / 16).clamp(-4, 4) for t in (Q, K))
    V = torch.randn(B, H, N, d, generator=g)
    dO = torch.randn(B, H, N, d, generator=g)
    BH = B * H
    qidx = torch.full((BH, N), N - 1, dtype=torch.int32)
    kidx = causal_idx(BH, N)
    _, _, _, P, _ = _run("clustered", B, H, N, N, d, alpha, k, scale, torch.float32, Q, K, V, dO,
                         qidx, kidx)
    assert ((P > 0).sum(-1) > k).mean() > 0.5  # the case exercises full sweeps


def test_exact_mode_adds_support_blocks():
    """A few rows over a long non-causal key range.  Rows 0-3 have flat
    scores: their supports (hundreds of keys) span every key block and
    overflow the per-row key lists of the refine pass's first sweep, so they
    take further sweeps; rows 4-7 have sharp scores and finish on their
    lists, in the same query block.  The rows' top-1 keys cover at most 8 of
    32 key blocks, so the support's blocks must be added to the mask."""
    B, H, NQ, NK, d = 1, 2, 8, 2048, 64
    BH = B * H
    Q, K, V, dO = make_inputs(B, H, NQ, NK, d, seed=11)
    Q[:, :, 4:] *= 20.0
    qidx = torch.full((BH, NQ), NK - 1, dtype=torch.int32)
    _, _, _, P, extra = _run("few_rows_wide", B, H, NQ, NK, d, 1.25, 1, 0.02, torch.float32,
                             Q, K, V, dO, qidx=qidx, kidx=causal_idx(BH, NK))
    sup = (P > 0).sum(-1)
    assert (sup[:, :4] > 256).all() and (sup[:, 4:] > 1).all()
    # keys listed by the first sweep (u > -1e-3 at the top-k root, which is
    # z_max - 1 at k = 1), against the lists used at k = 1 (32 keys per wave
    # and row, the row's key tiles dealt to the four waves): head 0 mixes
    # overflowing rows (0-3) and listed rows (4-7) in one block
    z = 0.25 * np.clip(np.einsum("bid,bjd->bij", np32(Q).astype(np.float64),
                                 np32(K).astype(np.float64)) * 0.02, -10, 10)
    listed = (z > z.max(-1, keepdims=True) - 1.0 - 1e-3).sum(-1)
    assert (listed[0, :4] > 64).all() and (listed[0, 4:] <= 64).all()
    assert extra >= BH * 16


def test_exact_mode_rows_without_keys_and_sinks():
    """Rows that see no key give zero output and gradients; a few heavy
    'sink' keys (BASELINE configs[4]'s pattern) pull most rows' supports."""
    B, H, N, d, k, alpha = 1, 2, 256, 64, 4, 1.25
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=5)
    K[:, :, :4] *= 4.0
    BH = B * H
    qidx = causal_idx(BH, N).clone()
    qidx[:, 10:20] = -1  # no key position is <= -1
    out, _, grads, _, _ = _run("sinks_empty_rows", B, H, N, N, d, alpha, k, 0.125, torch.float32,
                            Q, K, V, dO, qidx, causal_idx(BH, N))
    assert float(out[:, :, 10:20].abs().max()) == 0.0
    assert float(grads[0][:, :, 10:20].abs().max()) == 0.0


def test_exact_mode_through_module_and_custom_op():
    """The module and the torch.library operator take tau_mode and agree
    with the ops-level call bit for bit."""
    import splash_attention as sa
    from splash_attention import library

    dev = torch.device("cuda:0")
    B, H, N, d, k, alpha = 1, 2, 256, 64, 8, 1.5
    Q, K, V, dO = (t.to(dev) for t in make_inputs(B, H, N, N, d, seed=7))
    out_ops, st, _ = _gpu(dev, *(t.cpu() for t in (Q, K, V, dO)), causal_idx(B * H, N),
                          causal_idx(B * H, N), alpha, k, 0.125)
    m = sa.AdaptiveSplashAttention(head_dim=d, alpha=alpha, k_keep=k, sm_scale=0.125,
                                   tau_mode="exact")
    q, kk, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
    out = m(q, kk, v)
    out.backward(dO)
    op = library.forward_op(Q, K, V, None, None, alpha, k, 0.125, "entmax", "exact")
    torch.cuda.synchronize()
    assert torch.equal(out.detach(), out_ops)
    assert torch.equal(op[0], out_ops)
    assert torch.equal(op[1], st.taus)
    ref = sa.splash_attention(Q, K, V, None, None, alpha, k, 0.125)  # reference tau
    assert not torch.equal(ref, out_ops)  # c1-like rows: supports exceed k
