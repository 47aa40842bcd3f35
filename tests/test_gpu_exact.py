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
    ("fp32_negative_scale", 1, 1, 128, 128, 64, 1.5, 8, -0.125, torch.float32),
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


def _exact_full(name, Q, K, V, dO, qi, ki, alpha, k, scale, sample):
    """Exact mode at a full BASELINE shape (bf16), checked through
    size-independent properties and sampled rows:
      - every row has sum_j p_j = 1 (the exact threshold's defining
        equation), read from the forward's own row sums: to 1e-3, since each
        lane adds up to N/4 float32 terms in sequence (about 2.4e-4 at
        N = 16384), while a top-k threshold misses by far more wherever the
        support exceeds k (c4: about 216 keys tie at the +10 clamp against
        k = 64, so the reference threshold gives sum p ~ 3.4);
      - the full-gradient identities of the entmax Jacobian (sum_j dK_j = 0,
        sum_j dV_j = sum_i dO_i N_i / (N_i + EPS));
      - for the sampled (head, 64-row block) pairs, tau and the output rows
        against dense alpha-entmax in float64 over the same bf16 inputs
        (tau to 1e-4, output 2e-2)."""
    import time

    import splash_attention as sa
    from tests.test_gpu_configs import _identities

    dev = torch.device("cuda:0")
    B, H, N, d = Q.shape
    q, kk, v, qi_, ki_ = sa.ops.check_inputs(Q.to(dev), K.to(dev), V.to(dev), qi.to(dev), ki.to(dev))
    do = dO.to(dev)

    def step():
        out, st = sa.ops.splash_forward(q, kk, v, qi_, ki_, alpha, k, scale, tau_mode="exact")
        grads = sa.ops.splash_backward(q, kk, v, qi_, ki_, out, do, st, alpha, k, scale, "entmax")
        return out, st, grads

    out, st, grads = step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3
    assert torch.isfinite(out).all()
    norms = st.norms  # every row of these configs sees at least key 0
    e_norm = float((norms - 1.0).abs().max())
    assert e_norm <= 1e-3, f"{name}: max |sum p - 1| = {e_norm:.2e}"
    _identities(name, norms, grads, dO, 2e-2)
    e_tau = e_out = 0.0
    for bh, q0 in sample:
        b, h = divmod(bh, H)
        qs = slice(q0, q0 + 64)
        qr = Q[b, h, qs].double().numpy()
        kr = K[b, h].double().numpy()
        vr = V[b, h].double().numpy()
        vis = ki[bh].numpy()[None, :] <= qi[bh, qs].numpy()[:, None]
        ref_out, _, taus = dense.attention_forward(qr[None], kr[None], vr[None], vis[None], alpha,
                                                   scale)
        gt = st.taus[bh, qs].cpu().double().numpy()
        e_tau = max(e_tau, float(np.abs(gt - taus[0]).max()))
        e_out = max(e_out, assert_close(f"{name} out[{bh},{q0}]", np32(out[b:b + 1, h:h + 1, qs]),
                                        ref_out, 2e-2))
    assert e_tau <= 1e-4, f"{name}: tau differs by {e_tau:.2e}"
    print(f"  {name}: fwd+bwd {ms:.1f} ms, max |sum p - 1| {e_norm:.1e}, sampled tau {e_tau:.1e}, "
          f"out {e_out:.1e}", flush=True)


def test_exact_mode_c4_full():
    """configs[3] at full size in exact mode: B=1, H=32, N=16384, d=128 bf16,
    sparsemax, k 64, non-causal, clustered keys (most supports exceed k)."""
    from tests.test_gpu_configs import _clustered

    print("[exact] c4 bf16 1x32x16384x128 clustered", flush=True)
    B, H, N, d = 1, 32, 16384, 128
    Q, K, V, dO = _clustered(B, H, N, d, seed=0)
    qi = torch.full((B * H, N), N - 1, dtype=torch.int32)
    _exact_full("c4", Q, K, V, dO, qi, causal_idx(B * H, N), 2.0, 64, 128 ** -0.5,
                ((0, 0), (21, 8192)))


def test_exact_mode_c5_full():
    """configs[4] at full size in exact mode: B=1, H=8, N=32768, d=128 bf16,
    alpha 1.25, k 128, causal, keys 0..15 scaled x4 (sinks)."""
    from tests.test_gpu_configs import _gauss

    print("[exact] c5 bf16 1x8x32768x128 sinks", flush=True)
    B, H, N, d = 1, 8, 32768, 128
    Q, K, V = (_gauss((B, H, N, d), s, torch.float32) for s in (0, 1, 2))
    K[:, :, :16] *= 4
    Q, K, V = (t.to(torch.bfloat16) for t in (Q, K, V))
    dO = _gauss((B, H, N, d), 3, torch.bfloat16)
    idx = causal_idx(B * H, N)
    _exact_full("c5", Q, K, V, dO, idx, idx, 1.25, 128, 128 ** -0.5,
                ((3, 0), (3, 16384), (5, 32704)))


@pytest.mark.parametrize("grad_mode", ["reference", "entmax"])
def test_exact_mode_backward_vs_oracle_at_gpu_state(grad_mode):
    """Both gradient modes after an exact-mode forward against the C oracle's
    backward evaluated at the GPU's taus and CSR (the exact mode's mask,
    top-k union plus support blocks): 1e-5 (fp32).  Few rows over a long
    key range, so the mask holds blocks outside the top-k union."""
    import splash_attention as sa

    dev = torch.device("cuda:0")
    B, H, NQ, NK, d, k, alpha, scale = 1, 2, 72, 1024, 64, 2, 1.5, 0.05
    Q, K, V, dO = make_inputs(B, H, NQ, NK, d, seed=13)
    BH = B * H
    qidx = torch.full((BH, NQ), NK - 1, dtype=torch.int32)
    qidx[:, 40:] = torch.arange(600, 632, dtype=torch.int32)  # partly causal rows
    kidx = causal_idx(BH, NK)
    print(f"[exact] backward {grad_mode} vs oracle at GPU state", flush=True)
    q, kk, v, qi, ki = sa.ops.check_inputs(*(t.to(dev) for t in (Q, K, V, qidx, kidx)))
    out, st = sa.ops.splash_forward(q, kk, v, qi, ki, alpha, k, scale, tau_mode="exact")
    grads = sa.ops.splash_backward(q, kk, v, qi, ki, out, dO.to(dev), st, alpha, k, scale,
                                   grad_mode)
    torch.cuda.synchronize()
    topk = orc.forward(np32(Q), np32(K), np32(V), qidx.numpy(), kidx.numpy(), alpha, scale,
                       k).mask.astype(bool)
    assert (st.mask.cpu().numpy().astype(bool) & ~topk).sum() > 0  # support blocks were added
    want = orc.backward(np32(Q), np32(K), np32(V), qidx.numpy(), kidx.numpy(), np32(dO), alpha,
                        scale, st.taus.cpu().numpy(), st.q_ptr.cpu().numpy(),
                        st.q_list.cpu().numpy(), 1 if grad_mode == "reference" else 0)
    for gname, g, w in zip(("dQ", "dK", "dV"), grads, want):
        e = assert_close(f"{grad_mode}: {gname}", np32(g), w, 1e-5)
        print(f"  {gname} {e:.2e}", flush=True)
