"""Head dimensions other than 64 and 128, and float16 inputs, end to end,
against the CPU oracle at the caller's (unpadded) shape.

The reference takes any head dimension up to D_MAX = 128
(adasplashattention.cu:542).  A head dimension that is a whole number of
16-byte chunks (a multiple of 8 in 16-bit types, of 4 in fp32) runs
natively: the kernels compute at 64 or 128 and read and write only the d
columns (no copy).  Others (d50_bf16, d6_fp32) are zero-padded to a whole
chunk first (ops.to_kernel_layout).  float16 inputs run on the float16
kernels; the default sm_scale is 1/sqrt(d) of the caller's d.
Checked through the autograd function, the custom operator and the
reference-style forward/backward.  Tolerances (max-norm relative): 1e-5
for float32; 2e-2 for bfloat16; 4e-3 for float16 (fp32 arithmetic on
float16 MFMA operands: the weights P and, in the dense passes, ds rounded
to 11 significant bits, 2^-11 relative each, plus outputs and gradients
rounded to float16).
"""
import numpy as np
import pytest
import torch

import splash_attention as sa
from oracle import oracle as orc
from tests._util import assert_close, causal_idx, make_inputs, np32, oracle_at_gpu_tau

pytestmark = pytest.mark.gpu

CASES = [
    # name, d, dtype, tol
    ("d8_fp32", 8, torch.float32, 1e-5),
    ("d32_fp32", 32, torch.float32, 1e-5),
    ("d100_fp32", 100, torch.float32, 1e-5),
    ("d96_bf16", 96, torch.bfloat16, 2e-2),
    ("d64_fp16", 64, torch.float16, 4e-3),
    ("d48_fp16", 48, torch.float16, 4e-3),
    ("d128_fp16", 128, torch.float16, 4e-3),
    ("d50_bf16", 50, torch.bfloat16, 2e-2),
    ("d6_fp32", 6, torch.float32, 1e-5),
]


def _leaf(t, dev):
    return t.to(dev).requires_grad_()


@pytest.mark.parametrize("mode", ["entmax", "reference"])
@pytest.mark.parametrize("name,d,dtype,tol", CASES, ids=[c[0] for c in CASES])
def test_general_inputs_match_oracle(dev, name, d, dtype, tol, mode):
    print(f"[general] {name} mode={mode}", flush=True)
    B, H, NQ, NK, alpha, k = 1, 2, 200, 200, 1.5, 8
    scale = d ** -0.5
    Q, K, V, dO = make_inputs(B, H, NQ, NK, d, seed=17, dtype=dtype)
    qi, ki = causal_idx(B * H, NQ), causal_idx(B * H, NK)
    Qg, Kg, Vg = _leaf(Q, dev), _leaf(K, dev), _leaf(V, dev)
    out = sa.splash_attention(Qg, Kg, Vg, qi.to(dev), ki.to(dev), alpha, k, None, mode)
    out.backward(dO.to(dev))
    # the selection state of the same inputs, for the oracle at the GPU's tau
    q, kk, v, qi_, ki_ = sa.ops.check_inputs(Q.to(dev), K.to(dev), V.to(dev), qi.to(dev),
                                             ki.to(dev))
    _, st = sa.ops.splash_forward(q, kk, v, qi_, ki_, alpha, k, scale, with_support=False)
    torch.cuda.synchronize()
    assert out.shape == Q.shape and out.dtype == dtype
    for g, t in zip((Qg.grad, Kg.grad, Vg.grad), (Q, K, V)):
        assert g.shape == t.shape and g.dtype == dtype
    m = orc.GRAD_ENTMAX if mode == "entmax" else orc.GRAD_REFERENCE
    own, fw, og = oracle_at_gpu_tau(np32(Q), np32(K), np32(V), np32(dO), qi.numpy(), ki.numpy(),
                                    alpha, scale, k, st.taus.cpu().numpy(), m)
    np.testing.assert_array_equal(st.mask.cpu().numpy(), own.mask)
    errs = [assert_close(f"{name}: out", np32(out.detach()), fw.out, tol)]
    for gname, g, w in zip(("dQ", "dK", "dV"), (Qg.grad, Kg.grad, Vg.grad), og):
        errs.append(assert_close(f"{name}: {gname}", np32(g), w, tol))
    print("  errs " + " ".join(f"{e:.2e}" for e in errs), flush=True)

    # the custom operator gives the same bits as the autograd function
    Q2, K2, V2 = _leaf(Q, dev), _leaf(K, dev), _leaf(V, dev)
    out2 = sa.library.attention(Q2, K2, V2, qi.to(dev), ki.to(dev), alpha, k, None, mode)
    out2.backward(dO.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(out2, out.detach())
    for a, b in zip((Q2.grad, K2.grad, V2.grad), (Qg.grad, Kg.grad, Vg.grad)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("d,dtype", [(40, torch.float16), (72, torch.float32)])
def test_reference_style_entry_points_general_inputs(dev, d, dtype):
    """forward/backward (adasplashattention.cu:702-705) at d not in {64, 128}
    return the caller's shape and dtype, and the same values as the autograd
    function (reference gradient)."""
    print(f"[general] pybind-style d={d} {dtype}", flush=True)
    B, H, N, alpha, k = 1, 2, 130, 1.5, 8
    scale = d ** -0.5
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=5, dtype=dtype)
    qi, ki = causal_idx(B * H, N).to(dev), causal_idx(B * H, N).to(dev)
    out = sa.forward(Q.to(dev), K.to(dev), V.to(dev), qi, ki, scale, alpha, k_keep=k)
    grads = sa.backward(Q.to(dev), K.to(dev), V.to(dev), qi, ki, scale, alpha, dO.to(dev),
                        k_keep=k)
    Qg, Kg, Vg = _leaf(Q, dev), _leaf(K, dev), _leaf(V, dev)
    # the reference-order calls default to the compiled reference's 32-row blocks
    ref = sa.splash_attention(Qg, Kg, Vg, qi, ki, alpha, k, scale, "reference", block_m=32)
    ref.backward(dO.to(dev))
    torch.cuda.synchronize()
    assert out.shape == Q.shape and out.dtype == dtype
    assert torch.equal(out, ref.detach())
    for g, w, t in zip(grads, (Qg.grad, Kg.grad, Vg.grad), (Q, K, V)):
        assert g.shape == t.shape and g.dtype == dtype
        assert torch.equal(g, w)
    with pytest.raises(ValueError):
        sa.backward(Q.to(dev), K.to(dev), V.to(dev), qi, ki, scale, alpha,
                    dO[..., :-1].to(dev), k_keep=k)
