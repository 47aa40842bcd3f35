"""32-row mask blocks (block_m = 32, the reference's compile-time BLOCK_M,
adasplashattention.cu:8-9) on the GPU against the CPU oracle at the same
block_m.

The state's mask is [BH, ceil(NQ/32), nKB] and its CSR lists are over those
rows, as the reference's; the kernels run over 64-row tiles of the union of
each pair of rows and drop the tiles a half lacks.  Selection (mask, CSR,
top-k, tau) must be bit-exact on given scores; attention within 1e-5
(fp32) or 2e-2 (bf16) of the oracle at the GPU's tau, both gradient modes,
with the support-pair backward and with the dense backward (no support
masks recorded).  The "magnets" inputs make the two halves of every 64-row
block select different key blocks, so a kernel that ignored the halves
would be off by O(1).
"""
import numpy as np
import pytest
import torch

import splash_attention as sa
from oracle import oracle as orc
from tests._util import (assert_close, assert_tau_close, causal_idx, make_inputs, np32,
                         oracle_at_gpu_tau)

pytestmark = pytest.mark.gpu


SEL_CASES = [
    # (name, BH, NQ, NK, k, causal)
    ("causal_c1", 2, 256, 256, 8, True),
    ("ragged", 3, 100, 333, 8, True),
    ("three_halves", 2, 80, 200, 5, True),
    ("noncausal_k32", 1, 192, 320, 32, False),
]


@pytest.mark.parametrize("with_topk", [True, False], ids=["topk", "values"])
@pytest.mark.parametrize("name,BH,NQ,NK,k,causal", SEL_CASES, ids=[c[0] for c in SEL_CASES])
def test_select_block_m32_bit_exact(dev, name, BH, NQ, NK, k, causal, with_topk):
    print(f"[bm32] select {name} BH={BH} NQ={NQ} NK={NK} k={k} topk={with_topk}", flush=True)
    rng = np.random.default_rng(abs(hash(name)) % 2**32)
    S = rng.normal(size=(BH, NQ, NK)).astype(np.float32)
    if causal:
        qidx = causal_idx(BH, NQ) + (NK - NQ if NK > NQ else 0)
    else:
        qidx = torch.full((BH, NQ), NK, dtype=torch.int32)
    kidx = causal_idx(BH, NK)
    st = sa.ops.select_from_scores(torch.from_numpy(S).to(dev), qidx.to(dev), kidx.to(dev), 1.5,
                                   k, batch=1, heads=BH, with_topk=with_topk, block_m=32)
    torch.cuda.synchronize()
    vis = (kidx.numpy()[:, None, :] <= qidx.numpy()[:, :, None]).astype(np.uint8)
    sel = orc.select(np.clip(S, -10, 10), vis, k, 1.5, block_m=32)
    c = orc.csr(sel.mask)
    assert st.mask.shape == (BH, -(-NQ // 32), -(-NK // 64))
    np.testing.assert_array_equal(st.mask.cpu().numpy(), sel.mask)
    np.testing.assert_array_equal(st.q_ptr.cpu().numpy(), c.q_ptr)
    np.testing.assert_array_equal(st.q_list.cpu().numpy(), c.q_list)
    np.testing.assert_array_equal(st.k_ptr.cpu().numpy(), c.k_ptr)
    np.testing.assert_array_equal(st.k_list.cpu().numpy(), c.k_list)
    if with_topk:
        np.testing.assert_array_equal(st.topk_idx.cpu().numpy(), sel.topk_idx)
    np.testing.assert_array_equal(st.taus.cpu().numpy().view(np.uint32),
                                  sel.taus.astype(np.float32).view(np.uint32))


def _magnets(BH, N, d, seed=3):
    """Half h of the queries has its top-2 keys in key block h % 4 (every
    key visible); the other keys score near 0, inside the tau's reach."""
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


def _c1():
    Q, K, V, dO = make_inputs(1, 2, 256, 256, 64, seed=0)
    idx = causal_idx(2, 256)
    return Q, K, V, dO, idx, idx


def _ragged():
    Q, K, V, dO = make_inputs(1, 2, 80, 80, 64, seed=9)
    idx = causal_idx(2, 80)
    return Q, K, V, dO, idx, idx


CASES = {"c1": (_c1, 8), "magnets": (lambda: _magnets(2, 256, 64), 2), "ragged80": (_ragged, 4)}


@pytest.mark.parametrize("support", [True, False], ids=["support", "dense"])
@pytest.mark.parametrize("mode", ["entmax", "reference"])
@pytest.mark.parametrize("case", list(CASES))
def test_attention_block_m32_matches_oracle(dev, case, mode, support):
    make, k = CASES[case]
    Q, K, V, dO, qi, ki = make()
    alpha, scale = 1.5, 0.125
    print(f"[bm32] attention {case} {tuple(Q.shape)} k={k} {mode} support={support}", flush=True)
    q, kk, v, qd, kd = sa.ops.check_inputs(Q.to(dev), K.to(dev), V.to(dev), qi.to(dev),
                                           ki.to(dev))
    out, st = sa.ops.splash_forward(q, kk, v, qd, kd, alpha, k, scale, with_support=support,
                                    block_m=32)
    grads = sa.ops.splash_backward(q, kk, v, qd, kd, out, dO.to(dev), st, alpha, k, scale, mode)
    torch.cuda.synchronize()
    m = orc.GRAD_ENTMAX if mode == "entmax" else orc.GRAD_REFERENCE
    Qn, Kn, Vn, dOn = np32(Q), np32(K), np32(V), np32(dO)
    own, at, og = oracle_at_gpu_tau(Qn, Kn, Vn, dOn, qi.numpy(), ki.numpy(), alpha, scale, k,
                                    st.taus.cpu().numpy(), m, block_m=32)
    np.testing.assert_array_equal(st.mask.cpu().numpy(), own.mask)
    np.testing.assert_array_equal(st.q_ptr.cpu().numpy(), own.csr.q_ptr)
    np.testing.assert_array_equal(st.q_list.cpu().numpy(), own.csr.q_list)
    assert_tau_close(st.taus.cpu().numpy(), own.taus, alpha)
    assert_close("out", np32(out), at.out, 1e-5)
    assert_close("norms", st.norms.cpu().numpy(), at.norms, 1e-5)
    for name, g, w in zip(("dQ", "dK", "dV"), grads, og):
        assert_close(name, np32(g), w, 1e-5)
    if case == "magnets":
        # 64-row blocks give a different answer on these inputs
        out64, _ = sa.ops.splash_forward(q, kk, v, qd, kd, alpha, k, scale, with_support=False)
        assert float((out64 - out).abs().max()) > 1e-2


TOL16 = {torch.bfloat16: 2e-2, torch.float16: 4e-3}


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("mode", ["entmax", "reference"])
def test_attention_block_m32_16bit_magnets(dev, pairing, mode, dtype, d):
    """16-bit inputs through the paired forward (bf16, and fp16 with its P
    scaling, at d = 64 and 128); with 32-row masks a wave's half drops the
    union tiles its mask row lacks (its clip bounds set to -0 there).  The
    magnets make every pair of halves differ."""
    pairing("always")  # the paired forward's 32-row gating, as on large problems
    print(f"[bm32] attention magnets {dtype} d={d} {mode}", flush=True)
    Q, K, V, dO, qi, ki = _magnets(2, 256, d)
    Q, K, V = (t.to(dtype) for t in (Q, K, V))
    tol = TOL16[dtype]
    alpha, scale, k = 1.5, 0.125, 2
    q, kk, v, qd, kd = sa.ops.check_inputs(Q.to(dev), K.to(dev), V.to(dev), qi.to(dev),
                                           ki.to(dev))
    out, st = sa.ops.splash_forward(q, kk, v, qd, kd, alpha, k, scale, block_m=32)
    grads = sa.ops.splash_backward(q, kk, v, qd, kd, out, dO.to(dev), st, alpha, k, scale, mode)
    torch.cuda.synchronize()
    m = orc.GRAD_ENTMAX if mode == "entmax" else orc.GRAD_REFERENCE
    own, at, og = oracle_at_gpu_tau(np32(Q), np32(K), np32(V), np32(dO), qi.numpy(), ki.numpy(),
                                    alpha, scale, k, st.taus.cpu().numpy(), m, block_m=32)
    np.testing.assert_array_equal(st.mask.cpu().numpy(), own.mask)
    assert_close("out", np32(out), at.out, tol)
    for name, g, w in zip(("dQ", "dK", "dV"), grads, og):
        assert_close(name, np32(g), w, tol)
    out64, _ = sa.ops.splash_forward(q, kk, v, qd, kd, alpha, k, scale, with_support=False)
    assert float((out64.float() - out.float()).abs().max()) > 1e-2


def test_module_block_m32_bf16(dev):
    print("[bm32] module bf16 1x2x256x64 autograd", flush=True)
    Q, K, V, dO = make_inputs(1, 2, 256, 256, 64, seed=4, dtype=torch.bfloat16)
    attn = sa.AdaptiveSplashAttention(head_dim=64, alpha=1.5, k_keep=8, sm_scale=0.125,
                                      block_m=32)
    q, k, v = (t.to(dev).requires_grad_(True) for t in (Q, K, V))
    idx = causal_idx(2, 256)
    out = attn(q, k, v, idx.to(dev), idx.to(dev))
    out.backward(dO.to(dev))
    torch.cuda.synchronize()
    fw, (gq, gk, gv) = orc.attention(np32(Q), np32(K), np32(V), idx.numpy(), idx.numpy(),
                                     np32(dO), 1.5, 0.125, 8, block_m=32)
    assert_close("out", np32(out), fw.out, 2e-2)
    assert_close("dQ", np32(q.grad), gq, 2e-2)
    assert_close("dK", np32(k.grad), gk, 2e-2)
    assert_close("dV", np32(v.grad), gv, 2e-2)


def test_exact_tau_mode_rejects_block_m32(dev):
    Q, K, V, _ = make_inputs(1, 1, 64, 64, 64, seed=1)
    with pytest.raises(ValueError, match="block_m"):
        sa.splash_attention(Q.to(dev), K.to(dev), V.to(dev), tau_mode="exact", block_m=32)
