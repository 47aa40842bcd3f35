"""Host-side behaviour of the Python API (no GPU needed)."""
import pytest
import torch

import splash_attention as sa
from splash_attention import ops


def _t(*shape, dtype=torch.float32):
    return torch.zeros(*shape, dtype=dtype)


def test_module_mirrors_readme_signature():
    m = sa.AdaptiveSplashAttention(head_dim=64, alpha=1.5, k_keep=8, adaptive_threshold=True,
                                   sm_scale=0.125)
    assert (m.head_dim, m.alpha, m.k_keep, m.sm_scale) == (64, 1.5, 8, 0.125)
    assert len(m.state_dict()) == 0 and len(list(m.parameters())) == 0
    assert "k_keep=8" in repr(m)
    assert sa.AdaptiveSplashAttention(head_dim=128).sm_scale == pytest.approx(128 ** -0.5)


@pytest.mark.parametrize("kw", [dict(head_dim=0), dict(head_dim=129), dict(k_keep=0),
                                dict(k_keep=200),
                                dict(grad_mode="exact")])
def test_module_rejects_bad_config(kw):
    with pytest.raises(ValueError):
        sa.AdaptiveSplashAttention(**kw)


def test_head_dim_limit_message_matches_reference():
    # adasplashattention.cu:542 (TORCH_CHECK: a RuntimeError)
    with pytest.raises(RuntimeError, match="Head dimension too large; increase D_MAX"):
        ops.check_inputs(_t(1, 1, 8, 256), _t(1, 1, 8, 256), _t(1, 1, 8, 256))
    with pytest.raises(ValueError, match="Head dimension too large; increase D_MAX"):
        ops.check_inputs(_t(1, 1, 8, 256), _t(1, 1, 8, 256), _t(1, 1, 8, 256))


def test_cpu_tensors_are_rejected_like_the_reference():
    # adasplashattention.cu:543
    with pytest.raises(RuntimeError, match="Tensors must be on CUDA device"):
        ops.check_inputs(_t(1, 2, 8, 64), _t(1, 2, 8, 64), _t(1, 2, 8, 64))


@pytest.mark.parametrize("Q,K,V,err", [
    (_t(1, 2, 8), _t(1, 2, 8, 64), _t(1, 2, 8, 64), ValueError),
    (_t(1, 2, 8, 64), _t(1, 3, 8, 64), _t(1, 3, 8, 64), ValueError),
    (_t(1, 2, 8, 64), _t(1, 2, 8, 64), _t(1, 2, 9, 64), ValueError),
    (_t(1, 2, 8, 0), _t(1, 2, 8, 0), _t(1, 2, 8, 0), ValueError),
    (_t(1, 2, 8, 64, dtype=torch.float64), _t(1, 2, 8, 64, dtype=torch.float64),
     _t(1, 2, 8, 64, dtype=torch.float64), TypeError),
    (_t(1, 2, 8, 64, dtype=torch.float16), _t(1, 2, 8, 64), _t(1, 2, 8, 64), TypeError),
    (_t(1, 2, 8, 64), _t(1, 2, 8, 64, dtype=torch.bfloat16), _t(1, 2, 8, 64), TypeError),
])
def test_shape_and_dtype_validation(Q, K, V, err):
    with pytest.raises(err):
        ops.check_inputs(Q, K, V)


def test_index_normalisation():
    dev = torch.device("cpu")
    a = ops._index(None, 6, 5, 2, 3, dev, "Q_idx")
    assert a.dtype == torch.int32 and a.shape == (6, 5) and a[3].tolist() == [0, 1, 2, 3, 4]
    b = ops._index(torch.arange(5, dtype=torch.int64), 6, 5, 2, 3, dev, "Q_idx")
    assert torch.equal(a, b)
    c = ops._index(torch.arange(5).expand(2, 3, 5), 6, 5, 2, 3, dev, "K_idx")
    assert torch.equal(a, c) and c.is_contiguous()
    with pytest.raises(ValueError, match="int32"):
        ops._index(torch.full((6, 5), 2 ** 40), 6, 5, 2, 3, dev, "Q_idx")
    with pytest.raises(TypeError):
        ops._index(torch.zeros(6, 5), 6, 5, 2, 3, dev, "Q_idx")
    with pytest.raises(ValueError, match=r"\[B\*H, N\]"):
        ops._index(torch.zeros(6, 4, dtype=torch.int32), 6, 5, 2, 3, dev, "Q_idx")


def test_alpha_clamp_matches_reference():
    # adasplashattention.cu:547
    assert ops.clamp_alpha(0.5) == 1.05 and ops.clamp_alpha(7.0) == 3.0
    assert ops.clamp_alpha(1.5) == 1.5


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from splash_attention import _build, _lib

    monkeypatch.setattr(_build, "LIB", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_handle", None)
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load()


def test_grad_mode_validation():
    with pytest.raises(ValueError):
        sa.splash_attention(_t(1, 1, 8, 64), _t(1, 1, 8, 64), _t(1, 1, 8, 64),
                            grad_mode="bogus")


@pytest.mark.parametrize("d", [1, 6, 40, 64, 65, 100, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_kernel_layout_pads(d, dtype):
    """A head dimension that is not a whole number of 16-byte chunks (8
    elements in 16-bit types, 4 in fp32) is padded to one with zero columns
    (scores unchanged), in the caller's dtype; gradients flow back through
    it.  Whole-chunk head dimensions are left alone."""
    e = 4 if dtype == torch.float32 else 8
    dk = -(-d // e) * e
    assert ops.kernel_head_dim(d, dtype) == dk
    g = torch.Generator().manual_seed(3)
    Q = torch.randn(1, 2, 5, d, generator=g).to(dtype).requires_grad_()
    K = torch.randn(1, 2, 7, d, generator=g).to(dtype)
    q, k = ops.to_kernel_layout(Q, K)
    assert q.shape == (1, 2, 5, dk) and k.shape == (1, 2, 7, dk)
    if dk == d:
        assert q is Q and k is K
    assert q.dtype == dtype
    assert torch.count_nonzero(q[..., d:]) == 0
    assert torch.equal(q[..., :d].to(dtype), Q.detach())
    s_pad = q.double() @ k.double().transpose(-1, -2)
    s = Q.detach().double() @ K.double().transpose(-1, -2)
    assert torch.equal(s_pad, s)
    back = ops.from_kernel_layout(q * 2, d, dtype)
    assert back.shape == Q.shape and back.dtype == dtype
    back.sum().backward()
    assert torch.equal(Q.grad, torch.full_like(Q, 2))


def test_operand_strides_for_the_c_abi():
    """Strides handed to the C ABI ({batch, head, row}, elements): a size-1
    dimension gets its contiguous stride, so {0, 0, 0} (the ABI's mark for
    a contiguous operand) never stands for a broadcast one; an operand
    broadcast along batch, heads and rows alike is copied instead of read
    in place (read in place, its all-zero strides would send the kernels
    over B*H*N rows of a one-row buffer)."""
    d = 64
    x = torch.zeros(2, 3, 5, d, dtype=torch.bfloat16)
    assert ops.strides_of(x) == (3 * 5 * d, 5 * d, d) and ops.readable_in_place(x)
    # one head's K shared by 4 heads, a single key row (batch 1)
    k1 = torch.zeros(1, 1, 1, d, dtype=torch.bfloat16)
    kh = k1.expand(1, 4, 1, d)
    assert ops.strides_of(kh) == (4 * d, 0, d)
    assert ops.readable_in_place(kh) and ops.kernel_operand(kh) is kh
    # shared across heads with several rows: head stride 0, rows in place
    k2 = torch.zeros(2, 1, 7, d, dtype=torch.bfloat16).expand(2, 3, 7, d)
    assert ops.strides_of(k2) == (7 * d, 0, d) and ops.readable_in_place(k2)
    # one row broadcast along all three: copied
    kb = k1.expand(2, 3, 5, d)
    assert ops.strides_of(kb) == (0, 0, 0) and not ops.readable_in_place(kb)
    c = ops.kernel_operand(kb)
    assert c is not kb and c.is_contiguous() and torch.equal(c, kb)
    assert ops.strides_of(c) == (3 * 5 * d, 5 * d, d)
    # a single row in every dimension: contiguous either way
    assert ops.strides_of(k1) == (d, d, d) and ops.readable_in_place(k1)
    # the ops-level entry points refuse what they cannot read in place
    from splash_attention import _lib
    prob = _lib.Problem()
    ops._set_strides(prob, q=x, k=kh)
    assert tuple(prob.k_strides) == (4 * d, 0, d)
    for bad in (kb, torch.zeros(2, 3, 5, 2 * d, dtype=torch.bfloat16)[..., ::2]):
        with pytest.raises(ValueError, match="cannot be read in place"):
            ops._set_strides(prob, k=bad)


def test_bwd_passes_option_is_checked():
    with pytest.raises(ValueError, match="bwd_passes"):
        sa.AdaptiveSplashAttention(bwd_passes="dense")
    with pytest.raises(ValueError, match="bwd_passes"):
        ops.check_bwd_passes("pairs")
    m = sa.AdaptiveSplashAttention(bwd_passes="tiles")
    assert m.bwd_passes == "tiles" and "bwd_passes='tiles'" in m.extra_repr()
    assert ops.check_bwd_passes("support") == "support"


def test_reference_order_defaults_are_the_compiled_references():
    """forward/backward default to the compiled reference's K_KEEP = 8 and
    BLOCK_M = 32 (adasplashattention.cu:8-9, :17-19) and apply its host
    fix-up (:599-606, :684-697) unless told not to."""
    import inspect

    for fn in (sa.forward, sa.backward):
        sig = inspect.signature(fn).parameters
        assert sig["k_keep"].default == 8
        assert sig["block_m"].default == 32
        assert sig["fix_nonfinite"].default is True
    assert inspect.signature(sa.backward).parameters["grad_mode"].default == "reference"


def test_host_fixup_follows_the_reference():
    """ops.fix_nonfinite on host tensors against the oracle's restatement of
    cu:599-606 / :684-697 and hand-written cases: NaN -> 0 with a warning;
    any inf clamps the whole tensor to [-100, 100] with a warning; finite
    tensors pass unchanged and silently."""
    import warnings

    import numpy as np

    from oracle import oracle as orc

    fin = torch.tensor([1.0, -250.0, 3.0])
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert torch.equal(ops.fix_nonfinite(fin, "dK"), fin)   # no inf: no clamp
    nan = torch.tensor([float("nan"), -250.0, 3.0])
    with pytest.warns(RuntimeWarning, match="NaN values detected in dQ, setting to zero"):
        got = ops.fix_nonfinite(nan, "dQ")
    assert got.tolist() == [0.0, -250.0, 3.0]
    inf = torch.tensor([float("inf"), -250.0, 3.0, float("nan"), -float("inf")])
    with pytest.warns(RuntimeWarning) as rec:
        got = ops.fix_nonfinite(inf, "dV")
    msgs = [str(r.message) for r in rec]
    assert msgs == ["NaN values detected in dV, setting to zero",
                    "Inf values detected in dV, clamping"]
    assert got.tolist() == [100.0, -100.0, 3.0, 0.0, -100.0]
    for x in (fin, nan, inf):
        want, _, _ = orc.host_fixup(x.numpy())
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            np.testing.assert_array_equal(ops.fix_nonfinite(x, "out").numpy(), want)
