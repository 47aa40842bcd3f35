"""CSR lists of large block masks.

Masks of more than 32 KB per head whose rows are whole 16-byte chunks are
compacted by many blocks per head (32 mask lines each, every block counting
the whole head mask for its lines' offsets and its share of the zero tail);
smaller masks by two blocks per head from an LDS copy, and large masks of
other widths by two blocks from global memory.  Whatever the path, the
lists must equal, entry for entry and zero tails included, the CPU oracle's
CSR of the same mask (asao_csr: the reference's build_lookup_kernel,
adasplashattention.cu:219-242, plus its key-major transpose).
"""
import numpy as np
import pytest
import torch

import splash_attention as sa
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

CASES = [
    # name, B, H, NQ, NK, block_m; mask bytes per head (lines x line length)
    ("square_192", 1, 2, 12288, 12288, 64),     # 192 x 192: chunked
    ("wide_192x256", 2, 1, 12288, 16384, 64),   # 192 x 256: chunked, NQ != NK
    ("halves_384x192", 1, 1, 12288, 12288, 32),  # 32-row lists, 384 x 192: chunked
    ("odd_192x191", 1, 2, 12288, 12224, 64),    # 191 columns: two blocks per head from global
    ("staged_64", 1, 2, 4096, 4096, 64),        # 64 x 64: two blocks per head from LDS
]


@pytest.mark.parametrize("name,B,H,NQ,NK,block_m", CASES, ids=[c[0] for c in CASES])
def test_csr_of_large_masks(dev, name, B, H, NQ, NK, block_m):
    print(f"[compact] {name}", flush=True)
    g = torch.Generator().manual_seed(51)
    d = 64
    Q = torch.randn(B, H, NQ, d, generator=g).to(torch.bfloat16).to(dev)
    K = torch.randn(B, H, NK, d, generator=g).to(torch.bfloat16).to(dev)
    V = torch.randn(B, H, NK, d, generator=g).to(torch.bfloat16).to(dev)
    # queries at the end of the key range (the last query sees every key)
    qi = (torch.arange(NQ, dtype=torch.int32) + (NK - NQ)).unsqueeze(0).expand(B * H, NQ)
    ki = torch.arange(NK, dtype=torch.int32).unsqueeze(0).expand(B * H, NK)
    q, k, v, qi, ki = sa.ops.check_inputs(Q, K, V, qi.contiguous().to(dev), ki.contiguous().to(dev))
    _, st = sa.ops.splash_forward(q, k, v, qi, ki, 1.5, 8, d ** -0.5, with_support=False,
                                  block_m=block_m)
    torch.cuda.synchronize()
    mask = st.mask.cpu().numpy()
    nq_lines = (NQ + block_m - 1) // block_m
    assert mask.shape == (B * H, nq_lines, (NK + 63) // 64)
    assert 0 < mask.sum() < mask.size  # a mask with both set and clear entries
    c = orc.csr(mask)
    for got, want in ((st.q_ptr, c.q_ptr), (st.q_list, c.q_list), (st.k_ptr, c.k_ptr),
                      (st.k_list, c.k_list)):
        np.testing.assert_array_equal(got.cpu().numpy().reshape(want.shape), want)
