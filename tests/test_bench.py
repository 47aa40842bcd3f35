"""bench.py's contract and arithmetic (no GPU): the one-GPU refusal, the
effective-FLOP convention, the algorithmic FLOP counts its roofline entries
divide by, and the roofline fraction itself."""
import importlib.util
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr


def test_effective_flops_convention(bench):
    # FlashAttention's dense causal fwd+bwd count: 3.5 * 4 * BH * d * N^2 / 2
    assert bench.effective_flops(4, 16, 4096, 64) == pytest.approx(481.036e9, rel=1e-6)
    assert bench.effective_flops(1, 1, 2, 1) == 3.5 * 4 * 4 / 2


def test_algorithmic_counts_at_the_headline(bench):
    B, H, N, d = 4, 16, 4096, 64
    nQB = nKB = N // 64
    nnzb = B * H * nQB * (nQB + 1) // 2  # every causal tile active (the headline's mask)
    m = bench.kernel_models(B, H, N, d, nnzb, nQB, nKB, 32, nsup=1000)
    # scores of every visible (query, key) pair once: 2 d FLOPs each
    assert m["select"]["flops"] == 2.0 * d * (B * H * N * (N + 1) // 2) == 68736253952.0
    # S = K Q^T and O += V^T P over each active 64 x 64 tile
    assert m["forward"]["flops"] == 4.0 * 64 * 64 * d * nnzb == 139586437120.0
    # support pairs: two dot products and two updates of d elements
    assert m["bwd_dq_sparse"]["flops"] == m["bwd_dkdv_sparse"]["flops"] == 8.0 * d * 1000


def test_roofline_fraction(bench):
    model = dict(bound="mfma", flops=2.5e12, bytes=1e9)
    r = bench.roofline_of(model, 2.0)  # 2.5 TFLOP in 2 ms = 1250 TFLOP/s
    assert r["achieved"] == pytest.approx(1250.0)
    assert r["peak"] == 2500.0 and r["unit"] == "TFLOP/s"
    assert r["frac"] == pytest.approx(0.5)
    h = bench.roofline_of(dict(bound="hbm", flops=0.0, bytes=4e9), 1.0)  # 4 TB/s
    assert h["unit"] == "GB/s" and h["achieved"] == pytest.approx(4000.0)
    assert h["frac"] == pytest.approx(0.5)
