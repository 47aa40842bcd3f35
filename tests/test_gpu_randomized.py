"""Randomized end-to-end parity: many small problems drawn from a fixed seed,
each through the autograd function, against the CPU oracle at the GPU's tau.

Every draw picks the dtype (fp32, bf16, fp16), batch and heads, NQ and NK
(1 to 600, ragged and not multiples of 64), the head dimension (any whole
number of 16-byte chunks), alpha (1.25, 1.5, 2, 2.5 or one in (1.05, 2.9)),
k, 64- or 32-row mask blocks, the positions (causal, causal with an
offset, non-causal, or random positions, so that some rows see no key),
the gradient mode and the backward passes (support pairs or tiles).  A
second set of draws runs tau_mode="exact" against dense alpha-entmax
attention in float64, and a third reads the operands in place from random
layouts (transposed views, row slices, broadcast heads or batch), which
must give the same bits as contiguous copies.

Q and K lie on a 1/16 grid in [-4, 4] and sm_scale is a power of two, so
every score is exact in fp32 on the GPU and in the oracle.  Without that
the comparison would measure score rounding where the maths magnifies it:
for alpha > 1.5 the Jacobian weight u^((2-alpha)/(alpha-1)) has unbounded
slope at the support's edge, and with k = 1 the reference recurrence
(adasplashattention.cu:51-125) can stop with tau within an ulp of the top
value, where one rounding decides between p = 0 and p = 1.  k = 1 is left
out for that reason (its selection and tau are bit-exact on identical
scores in test_gpu_select.py).

Checked: the block mask exactly, tau to 1e-5 (relative, where |tau| > 1),
and out, dQ, dK, dV at the tolerances of the other parity tests (1e-5
fp32, 2e-2 bf16, 4e-3 fp16), each relative to the tensor's natural scale
(a row that sees one key has dQ = dK = 0 in exact arithmetic).
"""
import random

import numpy as np
import pytest
import torch

import splash_attention as sa
from oracle import oracle as orc
from tests._util import np32, oracle_at_gpu_tau, rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 4e-3}
N_CASES = 48


def _draw(rng):
    dt = rng.choice([torch.float32, torch.bfloat16, torch.float16])
    step = 4 if dt == torch.float32 else 8
    kind = rng.choice(["causal", "offset", "noncausal", "random"])
    NQ = rng.choice([1, 7, 63, 64, 65, 100, 129, 200, 256, 333, 513])
    return dict(
        dt=dt, d=rng.choice([64, 64, 128, rng.randrange(step, 129, step)]),
        B=rng.choice([1, 2]), H=rng.choice([1, 2, 3]), kind=kind, NQ=NQ,
        NK=NQ if kind == "causal" else rng.choice([1, 9, 64, 65, 128, 191, 300, 512, 600]),
        alpha=rng.choice([1.5, 1.5, 2.0, 1.25, 2.5, round(rng.uniform(1.05, 2.9), 3)]),
        k=rng.choice([2, 4, 8, 16, 32, 64, rng.randrange(2, 65)]), bm=rng.choice([64, 64, 32]),
        mode=rng.choice(["entmax", "reference"]), bwd=rng.choice(["support", "tiles"]),
        scale=rng.choice([0.125, 0.0625]), seed=rng.randrange(10 ** 6))


_rng = random.Random(20261202)
CASES = [_draw(_rng) for _ in range(N_CASES)]


def _positions(c, g):
    BH, NQ, NK = c["B"] * c["H"], c["NQ"], c["NK"]
    if c["kind"] == "causal":
        qi = torch.arange(NQ, dtype=torch.int32).expand(BH, NQ).contiguous()
        return qi, qi.clone()
    ki = torch.arange(NK, dtype=torch.int32).expand(BH, NK).contiguous()
    if c["kind"] == "offset":
        return (torch.arange(NQ, dtype=torch.int32) + (NK - NQ)).expand(BH, NQ).contiguous(), ki
    if c["kind"] == "noncausal":
        return torch.full((BH, NQ), NK - 1, dtype=torch.int32), ki
    return (torch.randint(0, NK + 5, (BH, NQ), generator=g).to(torch.int32),
            torch.randint(0, NK + 5, (BH, NK), generator=g).to(torch.int32))


@pytest.mark.parametrize("i", range(N_CASES))
def test_randomized_parity(dev, i):
    c = CASES[i]
    dt, B, H, NQ, NK, d = c["dt"], c["B"], c["H"], c["NQ"], c["NK"], c["d"]
    print(f"[random] case {i}: {str(dt)[6:]} B{B} H{H} NQ{NQ} NK{NK} d{d} alpha {c['alpha']} "
          f"k {c['k']} block_m {c['bm']} {c['kind']} {c['mode']} {c['bwd']} seed {c['seed']}",
          flush=True)
    g = torch.Generator().manual_seed(c["seed"])
    Q, K = ((torch.round(torch.randn(B, H, n, d, generator=g) * 16) / 16).clamp(-4, 4)
            for n in (NQ, NK))
    V = torch.randn(B, H, NK, d, generator=g)
    dO = torch.randn(B, H, NQ, d, generator=g)
    Q, K, V, dO = (t.to(dt) for t in (Q, K, V, dO))
    qi, ki = _positions(c, g)
    alpha, k, scale, bm = c["alpha"], c["k"], c["scale"], c["bm"]

    Qg, Kg, Vg = (t.to(dev).requires_grad_() for t in (Q, K, V))
    out = sa.splash_attention(Qg, Kg, Vg, qi.to(dev), ki.to(dev), alpha, k, scale, c["mode"],
                              block_m=bm, bwd_passes=c["bwd"])
    out.backward(dO.to(dev))
    q, kk, v, qi_, ki_ = sa.ops.check_inputs(Q.to(dev), K.to(dev), V.to(dev), qi.to(dev),
                                             ki.to(dev))
    _, st = sa.ops.splash_forward(q, kk, v, qi_, ki_, alpha, k, scale, with_support=False,
                                  block_m=bm)
    torch.cuda.synchronize()

    m = orc.GRAD_ENTMAX if c["mode"] == "entmax" else orc.GRAD_REFERENCE
    own, fw, og = oracle_at_gpu_tau(np32(Q), np32(K), np32(V), np32(dO), qi.numpy(), ki.numpy(),
                                    alpha, scale, k, st.taus.cpu().numpy(), m, block_m=bm)
    np.testing.assert_array_equal(st.mask.cpu().numpy().reshape(own.mask.shape), own.mask)
    gt = st.taus.cpu().numpy().reshape(own.taus.shape).astype(np.float64)
    dtau = np.abs(gt - own.taus) / np.maximum(1.0, np.abs(own.taus))
    assert float(dtau.max(initial=0.0)) <= 1e-5, f"tau differs by {float(dtau.max()):.2e}"

    def mx(t):
        return float(np.abs(np32(t)).max()) if t.numel() else 0.0

    floors = {"out": mx(V), "dQ": scale * mx(K) * mx(dO) * mx(V),
              "dK": scale * mx(Q) * mx(dO) * mx(V), "dV": mx(dO)}
    errs = []
    for name, got, want in (("out", out.detach(), fw.out), ("dQ", Qg.grad, og[0]),
                            ("dK", Kg.grad, og[1]), ("dV", Vg.grad, og[2])):
        gg = np32(got)
        assert np.all(np.isfinite(gg)), f"{name} not finite"
        e = rel_err(gg, want.reshape(gg.shape), max(floors[name], 1e-30))
        assert e <= TOL[dt], f"{name}: relative error {e:.3e} > {TOL[dt]:.0e}"
        errs.append(e)
    print("  errs " + " ".join(f"{e:.2e}" for e in errs), flush=True)


def _draw_exact(rng):
    c = _draw(rng)
    c["dt"] = rng.choice([torch.float32, torch.bfloat16])
    if c["dt"] == torch.float32 and c["d"] % 4:
        c["d"] = 64
    c["alpha"] = rng.choice([1.25, 1.5, 2.0, round(rng.uniform(1.05, 2.0), 3)])
    return c


_rng_exact = random.Random(20261203)
EXACT_CASES = [_draw_exact(_rng_exact) for _ in range(24)]


@pytest.mark.parametrize("i", range(len(EXACT_CASES)))
def test_randomized_exact_mode(dev, i):
    """tau_mode="exact" on drawn problems against dense alpha-entmax
    attention in float64 (oracle/dense.py) and its exact Jacobian
    gradients (entmax mode).  alpha <= 2: above 2 the Jacobian weight
    P^(2-alpha) is unbounded at the support's edge (the exact-mode tests
    give such gradients 1e-4).  Tolerances as above, relative to each
    tensor's natural scale; tau to 1e-5 (fp32) or 2e-2 (bf16) on rows that
    see a key; fp32 masks hold every block with a support key (p > 1e-7)."""
    from oracle import dense

    c = EXACT_CASES[i]
    dt, B, H, NQ, NK, d = c["dt"], c["B"], c["H"], c["NQ"], c["NK"], c["d"]
    alpha, k, scale = c["alpha"], c["k"], c["scale"]
    print(f"[random] exact case {i}: {str(dt)[6:]} B{B} H{H} NQ{NQ} NK{NK} d{d} alpha {alpha} "
          f"k {k} {c['kind']} seed {c['seed']}", flush=True)
    g = torch.Generator().manual_seed(c["seed"])
    Q, K = ((torch.round(torch.randn(B, H, n, d, generator=g) * 16) / 16).clamp(-4, 4)
            for n in (NQ, NK))
    V = torch.randn(B, H, NK, d, generator=g)
    dO = torch.randn(B, H, NQ, d, generator=g)
    Q, K, V, dO = (t.to(dt) for t in (Q, K, V, dO))
    qi, ki = _positions(c, g)

    q, kk, v, qi_, ki_ = sa.ops.check_inputs(*(t.to(dev) for t in (Q, K, V, qi, ki)))
    out, st = sa.ops.splash_forward(q, kk, v, qi_, ki_, alpha, k, scale, tau_mode="exact")
    grads = sa.ops.splash_backward(q, kk, v, qi_, ki_, out, dO.to(dev), st, alpha, k, scale,
                                   "entmax")
    torch.cuda.synchronize()

    vis = ki.numpy()[:, None, :] <= qi.numpy()[:, :, None]
    ref_out, P, taus = dense.attention_forward(np32(Q), np32(K), np32(V), vis, alpha, scale)
    dq, dk, dv = dense.attention_backward(np32(Q), np32(K), np32(V), P, np32(dO), alpha, scale)
    seen = vis.any(-1)
    gt = st.taus.cpu().numpy().reshape(taus.shape)
    dtau = float(np.abs(gt - taus)[seen].max()) if seen.any() else 0.0
    assert dtau <= (1e-5 if dt == torch.float32 else 2e-2), f"tau differs by {dtau:.2e}"
    if dt == torch.float32:
        nqb, nkb = -(-NQ // 64), -(-NK // 64)
        sup = np.zeros((B * H, nqb * 64, nkb * 64), bool)
        sup[:, :NQ, :NK] = (P > 1e-7) & vis
        need = sup.reshape(B * H, nqb, 64, nkb, 64).any(axis=(2, 4))
        assert not (need & ~st.mask.cpu().numpy().astype(bool)).any(), "support block missing"

    def mx(t):
        return float(np.abs(np32(t)).max()) if t.numel() else 0.0

    floors = {"out": mx(V), "dQ": scale * mx(K) * mx(dO) * mx(V),
              "dK": scale * mx(Q) * mx(dO) * mx(V), "dV": mx(dO)}
    for name, got, want in (("out", out, ref_out), ("dQ", grads[0], dq), ("dK", grads[1], dk),
                            ("dV", grads[2], dv)):
        gg = np32(got)[..., :d]  # the ops-level calls return a head dimension padded to a chunk
        assert np.all(np.isfinite(gg)), f"{name} not finite"
        e = rel_err(gg, np.asarray(want).reshape(gg.shape), max(floors[name], 1e-30))
        assert e <= TOL[dt], f"{name}: relative error {e:.3e} > {TOL[dt]:.0e}"


def _draw_layout(rng):
    c = _draw(rng)
    c["NK"] = c["NQ"] if c["kind"] == "causal" else c["NK"]
    c["kind"] = "offset" if c["kind"] == "random" else c["kind"]
    c["lay"] = (rng.choice("ctw"), rng.choice("ctwhb"), rng.choice("ctwhb"), rng.choice("ctw"))
    return c


_rng_layout = random.Random(20261204)
LAYOUT_CASES = [_draw_layout(_rng_layout) for _ in range(24)]


def _view(leaf, lay, B, H, strided):
    """The operand the call sees: leaf itself ('c'), a [B, N, H, d] buffer
    viewed as [B, H, N, d] ('t'), a row slice of a wider buffer ('w'), or a
    [B, 1, N, d] / [1, H, N, d] leaf broadcast over heads ('h') or batch
    ('b'); strided=False gives the same values contiguous."""
    if lay in "hb":
        v = leaf.expand(B, H, *leaf.shape[2:])
        return v if strided else v.contiguous()
    if not strided or lay == "c":
        return leaf
    if lay == "t":
        return leaf.transpose(1, 2).contiguous().transpose(1, 2)
    pad = 16 // leaf.element_size()
    buf = torch.zeros(*leaf.shape[:3], leaf.shape[3] + pad, dtype=leaf.dtype, device=leaf.device)
    return buf.index_copy(3, torch.arange(leaf.shape[3], device=leaf.device), leaf)[..., :leaf.shape[3]]


@pytest.mark.parametrize("i", range(len(LAYOUT_CASES)))
def test_randomized_layouts_bit_identical(dev, i):
    """Operands read in place (transposed views, row slices of wider
    buffers, K or V shared across heads or the batch with stride 0, dOut
    strided) give, through the autograd function, the same bits as the
    same values passed contiguous: out and the leaves' gradients."""
    c = LAYOUT_CASES[i]
    dt, B, H, NQ, NK, d = c["dt"], c["B"], c["H"], c["NQ"], c["NK"], c["d"]
    print(f"[random] layout case {i}: {str(dt)[6:]} B{B} H{H} NQ{NQ} NK{NK} d{d} "
          f"layouts {''.join(c['lay'])} {c['mode']} {c['bwd']} block_m {c['bm']}", flush=True)
    g = torch.Generator().manual_seed(c["seed"])
    shapes = [(B, H, NQ, d), (B, H, NK, d), (B, H, NK, d), (B, H, NQ, d)]
    base = []
    for (b_, h_, n_, d_), lay in zip(shapes, c["lay"]):
        shp = (b_, 1, n_, d_) if lay == "h" else (1, h_, n_, d_) if lay == "b" else (b_, h_, n_, d_)
        base.append(torch.randn(*shp, generator=g).to(dt).to(dev))
    qi, ki = (t.to(dev) for t in _positions(c, g))
    res = []
    for strided in (True, False):
        leaves = [t.detach().clone().requires_grad_() for t in base[:3]]
        ops_ = [_view(lf, lay, B, H, strided) for lf, lay in zip(leaves, c["lay"][:3])]
        dov = _view(base[3], c["lay"][3], B, H, strided)
        out = sa.splash_attention(*ops_, qi, ki, c["alpha"], c["k"], c["scale"], c["mode"],
                                  block_m=c["bm"], bwd_passes=c["bwd"])
        out.backward(dov)
        res.append([out.detach()] + [lf.grad for lf in leaves])
    torch.cuda.synchronize()
    for name, a, b in zip(("out", "dQ", "dK", "dV"), res[0], res[1]):
        assert torch.equal(a, b), f"{name} differs from the contiguous call"
