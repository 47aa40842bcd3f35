"""The BASELINE.json configurations at their real shapes on the GPU.

Where the oracle can afford the whole problem it checks everything; at the
large shapes it checks sampled (batch, head) slices or 64-row query blocks
(rows of different query blocks are independent given all keys), and the
full gradients through size-independent identities of the entmax-Jacobian
gradient:
  sum_j dK_j = 0        (entmax weights are invariant to adding a constant to
                         all scores of a row, so each row's ds sums to zero)
  sum_j dV_j = sum_i N_i / (N_i + EPS) dO_i   (each row's weights sum to
                         N_i / (N_i + EPS))
Tolerances: 1e-5 relative (fp32), 2e-2 relative (bf16), max-norm.
"""
import numpy as np
import pytest
import torch

import splash_attention as sa
from oracle import oracle as orc
from tests._util import assert_close, assert_tau_close, causal_idx, np32, oracle_at_gpu_tau

pytestmark = pytest.mark.gpu


def _run(dev, Q, K, V, dO, qi, ki, alpha, k, scale, mode="entmax"):
    q, kk, v, qi_, ki_ = sa.ops.check_inputs(Q.to(dev), K.to(dev), V.to(dev), qi.to(dev), ki.to(dev))
    out, st = sa.ops.splash_forward(q, kk, v, qi_, ki_, alpha, k, scale)
    grads = sa.ops.splash_backward(q, kk, v, qi_, ki_, out, dO.to(dev), st, alpha, k, scale, mode)
    torch.cuda.synchronize()
    return out, st, grads


def _gauss(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def _identities(name, out_norms, grads, dO, tol):
    """Size-independent checks of a full (entmax-mode) backward.

    sum_j dK_j is compared with sum_j |dK_j| per (head, dimension): the
    stored dK_j each carry at most half an ulp of rounding (bf16: 2^-8
    relative; fp32 outputs: the kernels' fp32 sums), so |sum_j dK_j| stays
    below 2^-8 sum_j |dK_j| for bf16; a gradient whose rows' ds do not sum
    to zero gives a sum of the order of the terms themselves.  (A key
    permutation keeps both sums; the sampled key blocks compared with the
    oracle catch that.)"""
    dQ, dK, dV = (g.float() for g in grads)
    BH = dK.shape[0] * dK.shape[1]
    dKr = dK.reshape(BH, -1, dK.shape[-1]).double()
    bound = 2.0 ** -8 if grads[1].dtype == torch.bfloat16 else 1e-5
    e = float((dKr.sum(1).abs() / dKr.abs().sum(1).clamp_min(1e-30)).max())
    assert e < bound, f"{name}: sum_j dK_j not ~0 (|sum| / sum|.| = {e:.2e} >= {bound:.1e})"
    n = out_norms.double()
    wsum = (n / (n + 1e-8)).unsqueeze(-1)
    want = (wsum * dO.reshape(BH, -1, dO.shape[-1]).to(dV.device).double()).sum(1)
    got = dV.reshape(BH, -1, dV.shape[-1]).double().sum(1)
    e2 = float((got - want).abs().max() / want.abs().max())
    assert e2 < tol, f"{name}: sum_j dV_j mismatch (rel {e2:.2e})"
    for g in (dQ, dK, dV):
        assert torch.isfinite(g).all()


def test_c2_fp32_full(dev):
    """B=2, H=8, N=1024, d=64 fp32, alpha 1.5, k 8, causal."""
    print("[cfg] c2 fp32 2x8x1024x64", flush=True)
    B, H, N, d = 2, 8, 1024, 64
    Q, K, V = (_gauss((B, H, N, d), s, torch.float32) for s in (0, 1, 2))
    dO = _gauss((B, H, N, d), 3, torch.float32)
    idx = causal_idx(B * H, N)
    for mode, m in (("entmax", orc.GRAD_ENTMAX), ("reference", orc.GRAD_REFERENCE)):
        out, st, grads = _run(dev, Q, K, V, dO, idx, idx, 1.5, 8, 0.125, mode)
        own, fw, og = oracle_at_gpu_tau(np32(Q), np32(K), np32(V), np32(dO), idx.numpy(),
                                        idx.numpy(), 1.5, 0.125, 8, st.taus.cpu().numpy(), m)
        np.testing.assert_array_equal(st.mask.cpu().numpy(), own.mask)
        assert_tau_close(st.taus.cpu().numpy(), own.taus, 1.5)
        assert_close("out", np32(out), fw.out, 1e-5)
        for nm, g, w in zip(("dQ", "dK", "dV"), grads, og):
            assert_close(f"{nm}/{mode}", np32(g), w, 1e-5)
        if mode == "entmax":
            _identities("c2", st.norms, grads, dO, 1e-5)


def test_headline_bf16_sampled_heads(dev):
    """B=4, H=16, N=4096, d=64 bf16, alpha 1.5, k 32, causal."""
    print("[cfg] headline bf16 4x16x4096x64", flush=True)
    B, H, N, d = 4, 16, 4096, 64
    Q, K, V = (_gauss((B, H, N, d), s, torch.bfloat16) for s in (0, 1, 2))
    dO = _gauss((B, H, N, d), 3, torch.bfloat16)
    idx = causal_idx(B * H, N)
    out, st, grads = _run(dev, Q, K, V, dO, idx, idx, 1.5, 32, 0.125)
    assert torch.isfinite(out).all()
    _identities("headline", st.norms, grads, dO, 2e-2)
    for bh in (0, 37):
        b, h = divmod(bh, H)
        sl = lambda t: np32(t[b:b + 1, h:h + 1])
        own, fw, og = oracle_at_gpu_tau(sl(Q), sl(K), sl(V), sl(dO), idx[:1].numpy(),
                                        idx[:1].numpy(), 1.5, 0.125, 32,
                                        st.taus[bh:bh + 1].cpu().numpy())
        np.testing.assert_array_equal(st.mask[bh:bh + 1].cpu().numpy(), own.mask)
        assert_tau_close(st.taus[bh:bh + 1].cpu().numpy(), own.taus, 1.5)
        assert_close(f"out[{bh}]", sl(out), fw.out, 2e-2)
        for nm, g, w in zip(("dQ", "dK", "dV"), grads, og):
            assert_close(f"{nm}[{bh}]", sl(g), w, 2e-2)


def _clustered(B, H, N, d, seed):
    """configs[3] inputs: 64 Gaussian centres per head (sigma 1); keys are
    centres + N(0, 0.1); queries are noisy copies (sigma 0.1) of random
    centres; V ~ N(0, 1)."""
    g = torch.Generator().manual_seed(seed)
    C = torch.randn(B, H, 64, d, generator=g)
    kid = torch.randint(0, 64, (B, H, N), generator=g)
    qid = torch.randint(0, 64, (B, H, N), generator=g)
    K = torch.gather(C, 2, kid.unsqueeze(-1).expand(B, H, N, d)) + 0.1 * torch.randn(B, H, N, d, generator=g)
    Q = torch.gather(C, 2, qid.unsqueeze(-1).expand(B, H, N, d)) + 0.1 * torch.randn(B, H, N, d, generator=g)
    V = torch.randn(B, H, N, d, generator=g)
    dO = torch.randn(B, H, N, d, generator=g)
    return tuple(t.to(torch.bfloat16) for t in (Q, K, V, dO))


def _row_sample_check(name, out, taus, grads, Q, K, V, dO, qi, ki, alpha, k, scale, bh_list, q0s,
                      H):
    """Oracle on 64-row query blocks [q0, q0+64) of chosen heads: out and dQ."""
    for bh in bh_list:
        b, h = divmod(bh, H)
        for q0 in q0s:
            qs = slice(q0, q0 + 64)
            own, fw, og = oracle_at_gpu_tau(np32(Q[b:b + 1, h:h + 1, qs]),
                                            np32(K[b:b + 1, h:h + 1]), np32(V[b:b + 1, h:h + 1]),
                                            np32(dO[b:b + 1, h:h + 1, qs]),
                                            qi[bh:bh + 1, qs].numpy(), ki[bh:bh + 1].numpy(),
                                            alpha, scale, k, taus[bh:bh + 1, qs].cpu().numpy())
            assert_tau_close(taus[bh:bh + 1, qs].cpu().numpy(), own.taus, alpha)
            assert_close(f"{name} out[{bh},{q0}]", np32(out[b:b + 1, h:h + 1, qs]), fw.out, 2e-2)
            assert_close(f"{name} dQ[{bh},{q0}]", np32(grads[0][b:b + 1, h:h + 1, qs]), og[0], 2e-2)


def _key_block_check(name, st, grads, Q, K, V, dO, qi, ki, alpha, scale, bh, blocks, H,
                     mode=0, tol=2e-2):
    """dK and dV of whole 64-key blocks of one head against the oracle's
    key-block restatement (oracle/keyblock.py, pinned to asao_backward) at
    the GPU's tau and block mask: every query row that sees the blocks."""
    from oracle import keyblock as KB

    b, h = divmod(bh, H)
    NK = K.shape[2]
    nQB = st.mask.shape[1]
    want_k, want_v = KB.key_block_grads(
        np32(Q[b:b + 1, h:h + 1])[0], np32(K[b:b + 1, h:h + 1])[0], np32(V[b:b + 1, h:h + 1])[0],
        np32(dO[b:b + 1, h:h + 1])[0], qi[bh].numpy(), ki[bh].numpy(),
        st.taus[bh].cpu().numpy(), st.mask[bh].reshape(nQB, -1).cpu().numpy(), alpha, scale,
        blocks, mode)
    rows = np.concatenate([np.arange(kb * 64, min(kb * 64 + 64, NK)) for kb in blocks])
    got_k = np32(grads[1][b:b + 1, h:h + 1])[0][rows]
    got_v = np32(grads[2][b:b + 1, h:h + 1])[0][rows]
    ek = assert_close(f"{name} dK blocks {blocks} of head {bh}", got_k, want_k[:len(rows)], tol)
    ev = assert_close(f"{name} dV blocks {blocks} of head {bh}", got_v, want_v[:len(rows)], tol)
    print(f"[cfg] {name} head {bh} key blocks {blocks}: dK rel {ek:.2e}, dV rel {ev:.2e}",
          flush=True)


def test_c4_clustered_sparsemax_noncausal(dev):
    """B=1, H=32, N=16384, d=128 bf16, alpha 2, k 64, non-causal."""
    print("[cfg] c4 bf16 1x32x16384x128 clustered", flush=True)
    B, H, N, d = 1, 32, 16384, 128
    Q, K, V, dO = _clustered(B, H, N, d, seed=0)
    qi = torch.full((B * H, N), N - 1, dtype=torch.int32)
    ki = causal_idx(B * H, N)
    scale = 128 ** -0.5
    out, st, grads = _run(dev, Q, K, V, dO, qi, ki, 2.0, 64, scale)
    assert torch.isfinite(out).all()
    _identities("c4", st.norms, grads, dO, 2e-2)
    _row_sample_check("c4", out, st.taus, grads, Q, K, V, dO, qi, ki, 2.0, 64, scale, (0, 21),
                      (0, 8192), H)
    _key_block_check("c4", st, grads, Q, K, V, dO, qi, ki, 2.0, scale, 5, [0, 131, 255], H)


def test_c5_long_sinks(dev):
    """B=1, H=8, N=32768, d=128 bf16, alpha 1.25, k 128, causal,
    keys at positions 0..15 scaled x4 (attention sinks)."""
    print("[cfg] c5 bf16 1x8x32768x128 sinks", flush=True)
    B, H, N, d = 1, 8, 32768, 128
    Q, K, V = (_gauss((B, H, N, d), s, torch.float32) for s in (0, 1, 2))
    K[:, :, :16] *= 4
    Q, K, V = (t.to(torch.bfloat16) for t in (Q, K, V))
    dO = _gauss((B, H, N, d), 3, torch.bfloat16)
    idx = causal_idx(B * H, N)
    scale = 128 ** -0.5
    out, st, grads = _run(dev, Q, K, V, dO, idx, idx, 1.25, 128, scale)
    assert torch.isfinite(out).all()
    _identities("c5", st.norms, grads, dO, 2e-2)
    _row_sample_check("c5", out, st.taus, grads, Q, K, V, dO, idx, idx, 1.25, 128, scale, (3,),
                      (0, 16384, 32704), H)
    # block 0 holds the sink keys, which every row weighs
    _key_block_check("c5", st, grads, Q, K, V, dO, idx, idx, 1.25, scale, 3, [0, 300, 511], H)


@pytest.mark.parametrize("d,alpha,k,causal", [(128, 2.0, 64, False), (64, 1.5, 32, True)])
def test_clustered_full_gradients(dev, d, alpha, k, causal):
    """Clustered keys and queries (the configs[3] generator) at a size the
    oracle covers whole: every gradient, including dK, whose bf16 product
    takes ds rounded once.  With clustered keys the dQ sum cancels heavily
    (each row's ds sums to zero), which its hi/lo operand split absorbs."""
    print(f"[cfg] clustered 1x2x2048x{d} alpha {alpha} k {k} causal={causal}", flush=True)
    B, H, N = 1, 2, 2048
    Q, K, V, dO = _clustered(B, H, N, d, seed=5)
    ki = causal_idx(B * H, N)
    qi = ki.clone() if causal else torch.full((B * H, N), N - 1, dtype=torch.int32)
    scale = d ** -0.5
    out, st, grads = _run(dev, Q, K, V, dO, qi, ki, alpha, k, scale)
    own, fw, og = oracle_at_gpu_tau(np32(Q), np32(K), np32(V), np32(dO), qi.numpy(), ki.numpy(),
                                    alpha, scale, k, st.taus.cpu().numpy())
    np.testing.assert_array_equal(st.mask.cpu().numpy(), own.mask)
    assert_close("clustered out", np32(out), fw.out, 2e-2)
    for nm, g, w in zip(("dQ", "dK", "dV"), grads, og):
        assert_close(f"clustered {nm}", np32(g), w, 2e-2)
    _identities("clustered", st.norms, grads, dO, 2e-2)


def _wave_list_sizes(st, BH, nQB, nKB):
    """Keys each dQ wave (16 rows of one query block) lists: the popcounts
    of its support masks summed over the query block's active tiles."""
    m = st.sup_mask.reshape(BH, nQB * nKB, 4, 64).to(torch.int32) & 0xFFFF
    c = torch.zeros_like(m)
    for b in range(16):
        c += (m >> b) & 1
    c = c.sum(-1).cpu()  # [BH, tile, wave]
    qp = st.q_ptr.reshape(BH, nQB + 1).cpu().long()
    return torch.stack([c[bh, qp[bh, qb]:qp[bh, qb + 1]].sum(0)
                        for bh in range(BH) for qb in range(nQB)])


@pytest.mark.parametrize("mode", ["entmax", "reference"])
def test_dq_balanced_and_chunked_paths(dev, mode):
    """The dQ pass lists a wave's keys whole when they fit in 1024 slots
    (lane groups then take the rows in a balanced order) and in per-row
    chunks otherwise.  Causal keys with sinks at alpha 1.25, k 128 give
    waves of both kinds; every gradient against the oracle in fp32."""
    print(f"[cfg] dQ paths 1x2x1536x64 fp32 sinks {mode}", flush=True)
    B, H, N, d = 1, 2, 1536, 64
    Q, K, V, dO = (_gauss((B, H, N, d), s, torch.float32) for s in (10, 11, 12, 13))
    K[:, :, :16] *= 4
    idx = causal_idx(B * H, N)
    out, st, grads = _run(dev, Q, K, V, dO, idx, idx, 1.25, 128, 0.125, mode)
    sizes = _wave_list_sizes(st, B * H, N // 64, N // 64)
    assert (sizes > 1024).any() and (sizes <= 1024).any(), "need waves on both paths"
    m = orc.GRAD_ENTMAX if mode == "entmax" else orc.GRAD_REFERENCE
    own, fw, og = oracle_at_gpu_tau(np32(Q), np32(K), np32(V), np32(dO), idx.numpy(), idx.numpy(),
                                    1.25, 0.125, 128, st.taus.cpu().numpy(), m)
    np.testing.assert_array_equal(st.mask.cpu().numpy(), own.mask)
    assert_close("dq paths out", np32(out), fw.out, 1e-5)
    for nm, g, w in zip(("dQ", "dK", "dV"), grads, og):
        assert_close(f"dq paths {nm}", np32(g), w, 1e-5)


@pytest.mark.parametrize("tau_mode", ["reference", "exact"])
def test_headline_step_is_deterministic(dev, tau_mode):
    """The headline step (B4 H16 N4096 d64 bf16, alpha 1.5, k 32), twice on
    the same inputs: out, tau, the mask and all three gradients equal bit
    for bit.  At this size thousands of workgroups run at once, so the
    order-dependent steps (candidate appends by LDS atomics in the score
    pass, the compaction's counts, the support-pair lists) are exercised
    under real concurrency; every sum they feed is formed in a fixed order."""
    print(f"[cfg] headline determinism {tau_mode}", flush=True)
    B, H, N, d = 4, 16, 4096, 64
    Q, K, V, dO = (_gauss((B, H, N, d), s, torch.bfloat16).to(dev) for s in (11, 12, 13, 14))
    idx = causal_idx(B * H, N).to(dev)
    res = []
    for _ in range(2):
        out, st = sa.ops.splash_forward(Q, K, V, idx, idx, 1.5, 32, 0.125, tau_mode=tau_mode)
        grads = sa.ops.splash_backward(Q, K, V, idx, idx, out, dO, st, 1.5, 32, 0.125, "entmax")
        torch.cuda.synchronize()
        res.append([out, st.taus, st.mask, *grads])
    for name, a, b in zip(("out", "tau", "mask", "dQ", "dK", "dV"), *res):
        assert torch.equal(a, b), f"{name} differs between two identical steps"
