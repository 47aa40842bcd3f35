"""Selection stage on the GPU vs the CPU oracle, given identical scores.

Top-k indices and values, block masks and CSR lists must be bit-exact; tau
must be bit-exact too (same fp32 recurrence, same rounding conventions).
Reference: adasplashattention.cu:35-242.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests._util import causal_idx

pytestmark = pytest.mark.gpu


def _run(dev, S, vis_qidx, vis_kidx, k, alpha, B, H, with_topk=True):
    import splash_attention as sa

    BH, NQ, NK = S.shape
    st = sa.ops.select_from_scores(torch.from_numpy(S).to(dev), vis_qidx.to(dev),
                                   vis_kidx.to(dev), alpha, k, batch=B, heads=H,
                                   with_topk=with_topk)
    torch.cuda.synchronize()
    return st


def _oracle(S, qidx, kidx, k, alpha):
    qi = qidx.numpy()
    ki = kidx.numpy()
    vis = (ki[:, None, :] <= qi[:, :, None]).astype(np.uint8)
    Sc = np.clip(S, -10, 10).astype(np.float32)
    sel = orc.select(Sc, vis, k, alpha)
    c = orc.csr(sel.mask)
    return sel, c


def _compare(st, sel, c):
    if st.topk_idx is not None:
        np.testing.assert_array_equal(st.topk_idx.cpu().numpy(), sel.topk_idx)
        np.testing.assert_array_equal(st.topk_val.cpu().numpy(), sel.topk_val)
    np.testing.assert_array_equal(st.mask.cpu().numpy(), sel.mask)
    np.testing.assert_array_equal(st.q_ptr.cpu().numpy(), c.q_ptr)
    np.testing.assert_array_equal(st.q_list.cpu().numpy(), c.q_list)
    np.testing.assert_array_equal(st.k_ptr.cpu().numpy(), c.k_ptr)
    np.testing.assert_array_equal(st.k_list.cpu().numpy(), c.k_list)
    taus = st.taus.cpu().numpy()
    np.testing.assert_array_equal(taus.view(np.uint32), sel.taus.astype(np.float32).view(np.uint32))


CASES = [
    # (name, B, H, NQ, NK, k, alpha, kind)
    ("causal_c1", 1, 2, 256, 256, 8, 1.5, "normal"),
    ("causal_k32", 1, 2, 320, 320, 32, 1.5, "normal"),
    ("sparsemax_k64", 1, 1, 256, 256, 64, 2.0, "normal"),
    ("alpha125_k128", 1, 1, 192, 192, 128, 1.25, "normal"),
    ("ties_quantised", 2, 1, 200, 200, 16, 1.5, "ties"),
    ("clamp_saturated", 1, 1, 128, 256, 8, 2.0, "saturated"),
    ("ragged_nq_ne_nk", 1, 3, 100, 333, 8, 1.5, "normal"),
    ("alpha_general", 1, 1, 130, 130, 8, 1.7, "normal"),
]


# with_topk=False is the path asa_forward takes: values sorted alone, the
# mask from the candidates scoring above the k-th value plus the
# lowest-index ties (the "ties" and "saturated" cases split tie runs at the
# k-th value)
@pytest.mark.parametrize("with_topk", [True, False], ids=["topk", "values"])
@pytest.mark.parametrize("name,B,H,NQ,NK,k,alpha,kind", CASES, ids=[c[0] for c in CASES])
def test_select_bit_exact(dev, name, B, H, NQ, NK, k, alpha, kind, with_topk):
    print(f"[select] {name} B={B} H={H} NQ={NQ} NK={NK} k={k} alpha={alpha} "
          f"topk={with_topk}", flush=True)
    rng = np.random.default_rng(hash(name) % 2**32)
    BH = B * H
    if kind == "normal":
        S = rng.normal(size=(BH, NQ, NK)).astype(np.float32)
    elif kind == "ties":
        S = (np.round(rng.normal(size=(BH, NQ, NK)) * 2) / 2).astype(np.float32)
    else:
        S = (rng.normal(size=(BH, NQ, NK)) * 30).astype(np.float32)
    qidx = causal_idx(BH, NQ) + (NK - NQ if NK > NQ else 0)
    kidx = causal_idx(BH, NK)
    st = _run(dev, S, qidx, kidx, k, alpha, B, H, with_topk)
    sel, c = _oracle(S, qidx, kidx, k, alpha)
    _compare(st, sel, c)


def test_select_noncausal_and_scattered_positions(dev):
    """Arbitrary (non-monotone) positions: visibility is K_idx <= Q_idx."""
    rng = np.random.default_rng(7)
    BH, NQ, NK, k = 2, 150, 260, 12
    S = rng.normal(size=(BH, NQ, NK)).astype(np.float32)
    qidx = torch.from_numpy(rng.integers(0, 300, size=(BH, NQ)).astype(np.int32))
    kidx = torch.from_numpy(rng.integers(0, 300, size=(BH, NK)).astype(np.int32))
    print("[select] scattered positions", flush=True)
    st = _run(dev, S, qidx, kidx, k, 1.5, 1, 2)
    sel, c = _oracle(S, qidx, kidx, k, 1.5)
    _compare(st, sel, c)



def _rising_scores(N, k):
    """Scores that make the score pass run many overflow rounds: in every
    64-key tile the keys at offsets below (k - 1) // R (R = 2 class maxima
    per tile offset for k <= 32, else 4: the tile ordinal mod R) score
    2 + 1e-4 j, rising with the key index j, and all other keys
    -1 - 1e-4 j.  Those offsets make fewer than k of the 64 R classes, so
    the floor falls among the low keys and every high key is a candidate;
    they arrive in ascending tile order, worst first, so each round's
    stored candidates give a threshold that only cap - k of them fail."""
    R = 2 if k <= 32 else 4
    nh = (k - 1) // R
    j = np.arange(N)
    row = np.where(j % 64 < nh, 2 + 1e-4 * j, -1 - 1e-4 * j).astype(np.float32)
    return np.broadcast_to(row, (1, N, N)).copy()


@pytest.mark.parametrize("with_topk", [True, False], ids=["topk", "values"])
@pytest.mark.parametrize("k,min_rounds", [(8, 2), (32, 4), (64, 4)])
def test_select_overflow_rounds_bit_exact(dev, k, min_rounds, with_topk):
    """Rows with many more candidates than the per-row capacity (k + 32)
    run several overflow rounds; the result must still be the oracle's,
    bit for bit, and the status word must report the rounds (without the
    round-bound flag)."""
    import splash_attention as sa

    N = 2048
    S = _rising_scores(N, k)
    idx = causal_idx(1, N)
    print(f"[select] overflow rounds N={N} k={k} topk={with_topk}", flush=True)
    st = _run(dev, S, idx, idx, k, 1.5, 1, 1, with_topk)
    rounds = st.overflow_rounds()
    print(f"[select] overflow rounds N={N} k={k}: {rounds} rounds", flush=True)
    assert not st.status_word() & sa._lib.STATUS_SELECT_ROUNDS
    assert rounds >= min_rounds, rounds
    sel, c = _oracle(S, idx, idx, k, 1.5)
    _compare(st, sel, c)
