"""The CPU oracle against the committed golden fixtures (tests/golden/).

c1_head0.npz holds one head of BASELINE.json configs[0] (N=256, d=64, fp32,
alpha=1.5, k_keep=8, sm_scale=0.125, causal) with the oracle's outputs;
known_answers.json holds hand-derived values (derivations in
test_oracle_pins.py).  make_golden.py regenerates both.
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as orc

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def c1():
    return dict(np.load(os.path.join(HERE, "c1_head0.npz")))


def test_c1_forward_reproduces_fixture(c1):
    fw = orc.forward(c1["Q"], c1["K"], c1["V"], c1["idx"], c1["idx"], float(c1["alpha"]),
                     float(c1["scale"]), int(c1["k"]))
    for name in ("topk_idx", "mask", "q_ptr", "q_list", "k_ptr", "k_list"):
        got = getattr(fw, name) if hasattr(fw, name) else getattr(fw.csr, name)
        np.testing.assert_array_equal(got, c1[name], err_msg=name)
    np.testing.assert_array_equal(fw.topk_val, c1["topk_val"])
    np.testing.assert_array_equal(fw.taus, c1["taus"])
    np.testing.assert_allclose(fw.norms, c1["norms"], rtol=1e-6)
    np.testing.assert_allclose(fw.out, c1["out"], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("mode", ["entmax", "reference"])
def test_c1_backward_reproduces_fixture(c1, mode):
    m = orc.GRAD_ENTMAX if mode == "entmax" else orc.GRAD_REFERENCE
    g = orc.backward(c1["Q"], c1["K"], c1["V"], c1["idx"], c1["idx"], c1["dO"],
                     float(c1["alpha"]), float(c1["scale"]), c1["taus"], c1["q_ptr"], c1["q_list"],
                     m)
    for name, x in zip(("dQ", "dK", "dV"), g):
        ref = c1[f"{name}_{mode}"]
        np.testing.assert_allclose(x, ref, rtol=1e-6, atol=1e-6 * np.abs(ref).max())


def test_known_answers():
    ka = json.load(open(os.path.join(HERE, "known_answers.json")))
    for case in ka["tau"]:
        for prec, tol in (("f64", 1e-9), ("f32", 1e-6)):
            assert orc.entmax_threshold(case["s"], case["alpha"], prec) == pytest.approx(
                case["tau"], abs=tol * max(1.0, abs(case["tau"]))), (case, prec)
    f = ka["forward_outside_topk"]
    d = 64
    Q = np.zeros((1, 1, d))
    Q[0, 0, 0] = 1.0
    K = np.zeros((1, 3, d))
    K[0, :, 0] = f["scores"]
    V = np.eye(3, d)[None]
    fw = orc.forward(Q, K, V, np.array([[2]], np.int32), np.array([[0, 1, 2]], np.int32),
                     f["alpha"], 1.0, f["k"], precision="f64")
    w = np.array(f["weights"])
    np.testing.assert_allclose(fw.out[0, 0, :3], w / (w.sum() + f["eps"]), rtol=1e-10)
