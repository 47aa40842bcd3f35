"""Forward and backward on the GPU vs the CPU oracle on identical seeded inputs.

Tolerances (max |gpu - oracle| / max |oracle| per tensor): 1e-5 for fp32,
2e-2 for bf16, 4e-3 for fp16 (11-bit MFMA operands P and ds, 16-bit
outputs).  Selection state (mask, CSR) must match exactly; tau must
match to 1e-5 relative (scores differ in the last bits between the MFMA
dot products and the oracle's double-precision ones).
Reference: adasplashattention.cu:150-700.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests._util import assert_close, assert_tau_close, causal_idx, make_inputs, np32, oracle_at_gpu_tau

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 4e-3}


def _gpu(dev, Q, K, V, dO, qidx, kidx, alpha, k, scale, mode):
    import splash_attention as sa

    q, kk, v = (t.to(dev) for t in (Q, K, V))
    qi, ki = qidx.to(dev), kidx.to(dev)
    q, kk, v, qi, ki = sa.ops.check_inputs(q, kk, v, qi, ki)
    out, st = sa.ops.splash_forward(q, kk, v, qi, ki, alpha, k, scale, with_topk=True)
    grads = sa.ops.splash_backward(q, kk, v, qi, ki, out, dO.to(dev), st, alpha, k, scale, mode)
    torch.cuda.synchronize()
    return out, st, grads


def _check(name, dtype, out, st, grads, fw, ograds, check_state=True):
    tol = TOL[dtype]
    if check_state:
        np.testing.assert_array_equal(st.mask.cpu().numpy(), fw.mask, err_msg=f"{name}: mask")
        np.testing.assert_array_equal(st.q_list.cpu().numpy(), fw.csr.q_list)
        np.testing.assert_array_equal(st.k_list.cpu().numpy(), fw.csr.k_list)
        assert_close(f"{name}: taus", st.taus.cpu().numpy(), fw.taus, 1e-5)
    e_out = assert_close(f"{name}: out", np32(out), fw.out, tol)
    errs = {"out": e_out}
    for gname, g, w in zip(("dQ", "dK", "dV"), grads, ograds):
        errs[gname] = assert_close(f"{name}: {gname}", np32(g), w, tol)
    print(f"  {name}: " + ", ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)


CASES = [
    # name, B, H, NQ, NK, d, alpha, k, scale, dtype
    ("c1_fp32", 1, 2, 256, 256, 64, 1.5, 8, 0.125, torch.float32),
    ("c1_fp32_k32", 1, 2, 256, 256, 64, 1.5, 32, 0.125, torch.float32),
    ("fp32_d128_sparsemax", 1, 2, 192, 192, 128, 2.0, 16, 128 ** -0.5, torch.float32),
    ("bf16_small", 1, 2, 256, 256, 64, 1.5, 32, 0.125, torch.bfloat16),
    ("bf16_d128_a125", 1, 2, 256, 256, 128, 1.25, 64, 128 ** -0.5, torch.bfloat16),
    ("fp16_small", 1, 2, 256, 256, 64, 1.5, 32, 0.125, torch.float16),
    ("fp16_d128_a125", 1, 2, 256, 256, 128, 1.25, 64, 128 ** -0.5, torch.float16),
    ("fp32_ragged", 2, 1, 100, 150, 64, 1.5, 8, 0.125, torch.float32),
    # 16-bit, d = 64: the forward runs query blocks in pairs; a ragged last
    # pair (197 rows: blocks 2 and 3, the second partial) and an odd block
    # count (130 rows: the last pair has one block), with sparse masks that
    # differ between the two blocks of a pair
    ("bf16_ragged_pairs", 2, 1, 197, 300, 64, 1.5, 16, 0.125, torch.bfloat16),
    ("fp16_odd_blocks", 1, 2, 130, 130, 64, 1.5, 8, 0.125, torch.float16),
    ("fp32_alpha_general", 1, 1, 128, 128, 64, 1.7, 8, 0.125, torch.float32),
    # the paired forward folds (alpha - 1) scale into its clip for the
    # integer power classes (p = v', v'^2, v'^4) when (alpha - 1) scale is in
    # [2^-8, 2^8]; a general alpha or a scale outside that range runs the
    # one-block forward at 16 bits and d = 64
    ("fp16_d64_sparsemax", 1, 2, 192, 192, 64, 2.0, 16, 0.125, torch.float16),
    ("bf16_d64_a125", 1, 2, 256, 256, 64, 1.25, 32, 0.125, torch.bfloat16),
    ("bf16_d64_alpha_general", 1, 2, 256, 256, 64, 1.7, 16, 0.125, torch.bfloat16),
    ("bf16_d64_small_scale", 1, 1, 128, 128, 64, 1.5, 8, 0.004, torch.bfloat16),
    # 16-bit d = 128 with k <= 32: the score pass's LDS ring holds three
    # tiles per wave there (four elsewhere)
    ("bf16_d128_k16", 1, 2, 320, 320, 128, 1.5, 16, 128 ** -0.5, torch.bfloat16),
]


# Each case with the paired forward wherever it applies ("always": on
# these small shapes the default runs one query block per workgroup, as it
# does on any problem whose pairs would not fill the GPU), and the 16-bit
# cases also with the default choice ("auto").
PCASES = [c + ("always",) for c in CASES] + [c + ("auto",) for c in CASES if c[-1] != torch.float32]


@pytest.mark.parametrize("mode", ["entmax", "reference"])
@pytest.mark.parametrize("name,B,H,NQ,NK,d,alpha,k,scale,dtype,pmode", PCASES,
                         ids=[f"{c[0]}-{c[-1]}" for c in PCASES])
def test_attention_parity(dev, pairing, name, B, H, NQ, NK, d, alpha, k, scale, dtype, pmode, mode):
    print(f"[attn] {name} mode={mode} pairing={pmode} B={B} H={H} NQ={NQ} NK={NK} d={d} "
          f"a={alpha} k={k} {dtype}", flush=True)
    pairing(pmode)
    Q, K, V, dO = make_inputs(B, H, NQ, NK, d, seed=0, dtype=dtype)
    BH = B * H
    qidx = causal_idx(BH, NQ) + (NK - NQ if NK > NQ else 0)
    kidx = causal_idx(BH, NK)
    out, st, grads = _gpu(dev, Q, K, V, dO, qidx, kidx, alpha, k, scale, mode)
    m = orc.GRAD_ENTMAX if mode == "entmax" else orc.GRAD_REFERENCE
    own, fw, og = oracle_at_gpu_tau(np32(Q), np32(K), np32(V), np32(dO), qidx.numpy(),
                                    kidx.numpy(), alpha, scale, k, st.taus.cpu().numpy(), m)
    assert_tau_close(st.taus.cpu().numpy(), own.taus, alpha)
    np.testing.assert_array_equal(st.mask.cpu().numpy(), own.mask, err_msg=f"{name}: mask")
    _check(f"{name}/{mode}", dtype, out, st, grads, fw, og, check_state=False)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 64), (torch.float16, 128)])
def test_pairing_modes_agree(dev, pairing, dtype, d):
    """The paired and the one-block forward kernels give the same output to
    the last ulps (the paired one folds the clip into its products); on a
    shape with few query-block pairs the default runs the one-block kernel,
    bit for bit."""
    print(f"[attn] pairing modes {dtype} d={d}", flush=True)
    B, H, N = 1, 2, 300
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=5, dtype=dtype)
    idx = causal_idx(B * H, N)
    res = {}
    for pm in ("always", "never", "auto"):
        pairing(pm)
        out, st, grads = _gpu(dev, Q, K, V, dO, idx, idx, 1.5, 16, d ** -0.5, "entmax")
        res[pm] = [np32(x) for x in (out, *grads)]
    for a, b in zip(res["auto"], res["never"]):
        np.testing.assert_array_equal(a, b)
    for n, a, b in zip(("out", "dQ", "dK", "dV"), res["always"], res["never"]):
        assert_close(f"{n}: paired against one-block", a, b, TOL[dtype])
