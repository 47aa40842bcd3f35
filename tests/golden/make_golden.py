"""Writes the golden fixtures of tests/golden/ (regression anchors of the CPU oracle).

The reference ships no golden vectors for this path (its notebook prints
values for unseeded inputs only), so the fixtures are produced by the
oracle after it passed the checks of tests/test_oracle_pins.py, plus
hand-derived known answers.  Inputs follow the BASELINE.json configs[0]
convention: Q, K, V then dO drawn from N(0, 1) with torch.Generator seeds 0
and 1, float32, causal positions.  They are stored in the fixture, so the
check does not depend on torch's random stream.

Run from the repo root:  python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as orc  # noqa: E402


def c1_inputs(B=1, H=1, N=256, d=64):
    import torch

    g = torch.Generator().manual_seed(0)
    Q, K, V = (torch.randn(B * H, N, d, generator=g).numpy() for _ in range(3))
    dO = torch.randn(B * H, N, d, generator=torch.Generator().manual_seed(1)).numpy()
    idx = np.broadcast_to(np.arange(N, dtype=np.int32), (B * H, N)).copy()
    return Q, K, V, dO, idx


def main():
    Q, K, V, dO, idx = c1_inputs()
    alpha, scale, k = 1.5, 0.125, 8
    fw = orc.forward(Q, K, V, idx, idx, alpha, scale, k)
    g0 = orc.backward(Q, K, V, idx, idx, dO, alpha, scale, fw.taus, fw.csr.q_ptr, fw.csr.q_list,
                      orc.GRAD_ENTMAX)
    g1 = orc.backward(Q, K, V, idx, idx, dO, alpha, scale, fw.taus, fw.csr.q_ptr, fw.csr.q_list,
                      orc.GRAD_REFERENCE)
    np.savez_compressed(
        os.path.join(HERE, "c1_head0.npz"),
        Q=Q, K=K, V=V, dO=dO, idx=idx, alpha=alpha, scale=scale, k=k,
        out=fw.out, taus=fw.taus, norms=fw.norms, topk_idx=fw.topk_idx, topk_val=fw.topk_val,
        mask=fw.mask, q_ptr=fw.csr.q_ptr, q_list=fw.csr.q_list, k_ptr=fw.csr.k_ptr,
        k_list=fw.csr.k_list, dQ_entmax=g0[0], dK_entmax=g0[1], dV_entmax=g0[2],
        dQ_reference=g1[0], dK_reference=g1[1], dV_reference=g1[2])

    # Hand-derived known answers (derivations in tests/test_oracle_pins.py).
    known = {
        "tau": [
            {"s": [1.0, 0.0], "alpha": 2.0, "tau": 0.0},
            {"s": [1.0, 0.9], "alpha": 2.0, "tau": 0.45},
            {"s": [3.0], "alpha": 1.5, "tau": 1.5},
            {"s": [2.0, 2.0, 2.0, 2.0], "alpha": 1.25, "tau": 0.5},
            {"s": [0.3, -1e6, -1e6, -1e6], "alpha": 2.0, "tau": -0.7},
            # two rounds take the bisection fallback (cu:102-104)
            {"s": [9.0, -2.0, -14.0], "alpha": 1.5, "tau": 3.5000000555768707},
        ],
        "forward_outside_topk": {
            "scores": [1.0, 0.9, 0.8], "alpha": 2.0, "k": 2,
            "weights": [0.55, 0.45, 0.35], "eps": 1e-8,
        },
    }
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(known, f, indent=1)
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
