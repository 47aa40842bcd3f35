"""Operands read where they lie: strided views and head dimensions other
than 64 and 128, with no copy on the way in.

The reference reads contiguous [B, H, N, d] tensors through data_ptr
(adasplashattention.cu:568-571) for any d <= 128 (:542).  Here Q, K, V and
dOut may be views with any batch, head and row strides that are whole
16-byte chunks (the C ABI's q_strides ... dout_strides), and d any whole
number of chunks; ops.check_inputs then hands the caller's tensors to the
kernels unchanged (asserted with `is`).  The same kernels read the same
values in the same order whatever the strides, so every result must equal,
bit for bit, the call on contiguous copies; head dimensions that are not
64 or 128 are checked against the CPU oracle in test_gpu_general_inputs.py
(which runs them natively) and here against the zero-padded inputs (the
kernels never read columns past d, so padding changes nothing).
"""
import pytest
import torch

import splash_attention as sa
from tests._util import causal_idx, make_inputs

pytestmark = pytest.mark.gpu

CASES = [
    # name, d, dtype
    ("d64_bf16", 64, torch.bfloat16),
    ("d96_bf16", 96, torch.bfloat16),
    ("d32_fp16", 32, torch.float16),
    ("d128_bf16", 128, torch.bfloat16),
    ("d64_fp32", 64, torch.float32),
    ("d40_fp32", 40, torch.float32),
]


def _bnhd(t):
    """[B, H, N, d] values as a [B, N, H, d] tensor viewed back as [B, H, N, d]
    (strides N H d, d, H d, 1): the layout of a fused projection's output."""
    return t.transpose(1, 2).contiguous().transpose(1, 2)


def _run(dev, Q, K, V, dO, qi, ki, mode, block_m=64, scale=0.125):
    Qg, Kg, Vg = (t.detach().requires_grad_() for t in (Q, K, V))
    out = sa.splash_attention(Qg, Kg, Vg, qi, ki, 1.5, 16, scale, mode, block_m=block_m)
    out.backward(dO)
    torch.cuda.synchronize()
    return out.detach(), Qg.grad, Kg.grad, Vg.grad


@pytest.mark.parametrize("mode", ["entmax", "reference"])
@pytest.mark.parametrize("name,d,dtype", CASES, ids=[c[0] for c in CASES])
def test_transposed_views_are_read_in_place(dev, name, d, dtype, mode):
    print(f"[layouts] transposed {name} {mode}", flush=True)
    B, H, N = 2, 3, 200
    Q, K, V, dO = (t.to(dev) for t in make_inputs(B, H, N, N, d, seed=41, dtype=dtype))
    qi = causal_idx(B * H, N).to(dev)
    Qt, Kt, Vt, dOt = (_bnhd(t) for t in (Q, K, V, dO))
    assert not Qt.is_contiguous() and torch.equal(Qt, Q)
    q, k, v, _, _ = sa.ops.check_inputs(Qt, Kt, Vt, qi, qi)
    assert q is Qt and k is Kt and v is Vt  # no copy
    want = _run(dev, Q, K, V, dO, qi, qi, mode)
    got = _run(dev, Qt, Kt, Vt, dOt, qi, qi, mode)
    for n, a, b in zip(("out", "dQ", "dK", "dV"), got, want):
        assert a.shape == b.shape and a.dtype == b.dtype
        assert torch.equal(a, b), f"{n}: strided result differs from the contiguous one"


@pytest.mark.parametrize("name,d,dtype", CASES[:3], ids=[c[0] for c in CASES[:3]])
def test_keys_shared_across_heads(dev, name, d, dtype):
    """K and V expanded over the heads (head stride 0, as grouped-query
    attention shares them): read in place, results equal to the expanded
    copies', and autograd sums the heads' dK, dV into the shared rows."""
    print(f"[layouts] shared keys {name}", flush=True)
    B, H, N = 1, 4, 160
    Q, K, V, dO = (t.to(dev) for t in make_inputs(B, H, N, N, d, seed=43, dtype=dtype))
    K1, V1 = K[:, :1], V[:, :1]
    Ke, Ve = K1.expand(B, H, N, d), V1.expand(B, H, N, d)
    qi = causal_idx(B * H, N).to(dev)
    _, k, v, _, _ = sa.ops.check_inputs(Q, Ke, Ve, qi, qi)
    assert k is Ke and v is Ve
    want = _run(dev, Q, Ke.contiguous(), Ve.contiguous(), dO, qi, qi, "entmax")
    Qg, Kg, Vg = Q.clone().requires_grad_(), K1.clone().requires_grad_(), V1.clone().requires_grad_()
    out = sa.splash_attention(Qg, Kg.expand(B, H, N, d), Vg.expand(B, H, N, d), qi, qi, 1.5, 16,
                              0.125)
    out.backward(dO)
    torch.cuda.synchronize()
    assert torch.equal(out, want[0]) and torch.equal(Qg.grad, want[1])
    for g, w in ((Kg.grad, want[2]), (Vg.grad, want[3])):
        assert torch.equal(g, w.sum(1, keepdim=True))


def test_broadcast_keys_single_row_and_all_dims(dev):
    """One key row shared by every head (NK = 1, head stride 0) and one key
    row repeated over the heads and rows of a single batch (head and row
    strides 0) are read in place; one key row broadcast along batch, heads
    and rows (all strides 0, the C ABI's mark for a contiguous operand) is
    copied first.  Each equals the call on contiguous copies bit for bit."""
    print("[layouts] broadcast key rows", flush=True)
    d, H = 64, 4
    g = torch.Generator().manual_seed(49)
    Q = torch.randn(1, H, 96, d, generator=g).to(torch.bfloat16).to(dev)
    k1 = torch.randn(1, 1, 1, d, generator=g).to(torch.bfloat16).to(dev)
    v1 = torch.randn(1, 1, 1, d, generator=g).to(torch.bfloat16).to(dev)
    dO = torch.randn(1, H, 96, d, generator=g).to(torch.bfloat16).to(dev)
    qi = causal_idx(H, 96).to(dev)
    ki = torch.zeros(H, 1, dtype=torch.int32, device=dev)
    Kh, Vh = k1.expand(1, H, 1, d), v1.expand(1, H, 1, d)
    _, k, v, _, _ = sa.ops.check_inputs(Q, Kh, Vh, qi, ki)
    assert k is Kh and v is Vh
    got = _run(dev, Q, Kh, Vh, dO, qi, ki, "entmax")
    want = _run(dev, Q, Kh.contiguous(), Vh.contiguous(), dO, qi, ki, "entmax")
    for n, a, b in zip(("out", "dQ", "dK", "dV"), got, want):
        assert torch.equal(a, b), f"{n}: head-shared key row differs"
    N = 80
    for B in (1, 2):
        Qb = Q[:, :, :N].expand(B, H, N, d).contiguous()
        dOb = dO[:, :, :N].expand(B, H, N, d).contiguous()
        qb = causal_idx(B * H, N).to(dev)
        Kb, Vb = k1.expand(B, H, N, d), v1.expand(B, H, N, d)
        _, k, v, _, _ = sa.ops.check_inputs(Qb, Kb, Vb, qb, qb)
        if B == 1:
            assert sa.ops.strides_of(Kb) == (H * N * d, 0, 0) and k is Kb
        else:
            assert sa.ops.strides_of(Kb) == (0, 0, 0)
            assert k is not Kb and k.is_contiguous() and torch.equal(k, Kb)
        got = _run(dev, Qb, Kb, Vb, dOb, qb, qb, "entmax")
        want = _run(dev, Qb, Kb.contiguous(), Vb.contiguous(), dOb, qb, qb, "entmax")
        for n, a, b in zip(("out", "dQ", "dK", "dV"), got, want):
            assert torch.equal(a, b), f"{n}: broadcast key rows differ (batch {B})"


def test_strided_dout_and_reference_order_calls(dev):
    """The reference-order backward with a transposed dOut and 32-row mask
    blocks (its defaults) equals the contiguous call; so does forward."""
    print("[layouts] reference-order calls", flush=True)
    B, H, N, d = 1, 2, 256, 64
    Q, K, V, dO = (t.to(dev) for t in make_inputs(B, H, N, N, d, seed=45, dtype=torch.bfloat16))
    qi = causal_idx(B * H, N).to(dev)
    args = (Q, K, V, qi, qi, 0.125, 1.5)
    targs = (_bnhd(Q), _bnhd(K), _bnhd(V), qi, qi, 0.125, 1.5)
    assert torch.equal(sa.forward(*targs), sa.forward(*args))
    for a, b in zip(sa.backward(*targs, _bnhd(dO)), sa.backward(*args, dO)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("d,dtype", [(96, torch.bfloat16), (48, torch.float16), (20, torch.float32)])
def test_native_head_dim_equals_zero_padded(dev, d, dtype):
    """d run natively (kernels at 64 / 128 reading only d columns) against
    the same inputs zero-padded to the kernel width: the padded columns add
    exact zeros to every product, so out and the gradients' first d columns
    agree bit for bit, and the kernels wrote no column past d."""
    print(f"[layouts] native d={d} {dtype}", flush=True)
    B, H, N = 1, 2, 192
    D = 64 if d <= 64 else 128
    Q, K, V, dO = (t.to(dev) for t in make_inputs(B, H, N, N, d, seed=47, dtype=dtype))
    qi = causal_idx(B * H, N).to(dev)
    pad = lambda t: torch.nn.functional.pad(t, (0, D - d))  # noqa: E731
    got = _run(dev, Q, K, V, dO, qi, qi, "entmax", scale=d ** -0.5)
    want = _run(dev, pad(Q), pad(K), pad(V), pad(dO), qi, qi, "entmax", scale=d ** -0.5)
    for n, a, b in zip(("out", "dQ", "dK", "dV"), got, want):
        assert a.shape[-1] == d
        assert torch.equal(a, b[..., :d]), f"{n} differs from the padded run"
        assert torch.count_nonzero(b[..., d:]) == 0
