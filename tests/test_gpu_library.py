"""The custom operators on the GPU: opcheck, and torch.compile (graph
capture through the fake implementations, aot_eager backend) giving the
eager result bit for bit."""
import pytest
import torch

import splash_attention as sa
from splash_attention import library
from tests._util import causal_idx, make_inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d,dtype", [(64, torch.float32), (40, torch.float16)])
def test_opcheck_forward(dev, d, dtype):
    print(f"[lib] opcheck forward {dtype} 1x2x128x{d}", flush=True)
    Q, K, V, _ = make_inputs(1, 2, 128, 128, d, seed=11, dtype=dtype)
    args = (Q.to(dev), K.to(dev), V.to(dev), None, None, 1.5, 8, 0.125, "entmax")
    torch.library.opcheck(library.forward_op, args,
                          test_utils=("test_schema", "test_faketensor"))
    torch.library.opcheck(library.forward_op, args + ("exact",),
                          test_utils=("test_schema", "test_faketensor"))
    torch.library.opcheck(library.forward_op, args + ("reference", 64, "tiles"),
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.parametrize("dtype,d,tau_mode,bwd_passes", [(torch.float32, 64, "reference", "support"),
                                                         (torch.bfloat16, 64, "reference", "support"),
                                                         (torch.float16, 40, "reference", "support"),
                                                         (torch.float32, 64, "exact", "support"),
                                                         (torch.bfloat16, 64, "reference", "tiles")])
def test_compile_matches_eager(dev, dtype, d, tau_mode, bwd_passes):
    print(f"[lib] torch.compile aot_eager {dtype} d={d} tau_mode={tau_mode} {bwd_passes}",
          flush=True)
    B, H, N = 1, 2, 192
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=12, dtype=dtype)
    idx = causal_idx(B * H, N).to(dev)
    attn = sa.AdaptiveSplashAttention(head_dim=d, alpha=1.5, k_keep=16, sm_scale=0.125,
                                      tau_mode=tau_mode, bwd_passes=bwd_passes)

    def run(fn):
        q, k, v = (t.to(dev).requires_grad_(True) for t in (Q, K, V))
        out = fn(q, k, v, idx, idx)
        out.backward(dO.to(dev))
        torch.cuda.synchronize()
        return [x.detach().cpu() for x in (out, q.grad, k.grad, v.grad)]

    eager = run(attn)
    compiled = run(torch.compile(attn, backend="aot_eager", fullgraph=True))
    for a, b in zip(eager, compiled):
        assert torch.equal(a, b)


@pytest.mark.parametrize("baseline,backward", [("entmax", False), ("vanilla", True)])
def test_benchmark_cli_fields(dev, baseline, backward):
    """The notebook's metric set (nb:1688-1712) for one small config.  No
    closeness is asserted: the reference's tau recurrence (kept here) does
    not converge on rows with fewer visible keys than k_keep (the -1e6
    sentinel enters the bracket), so it differs from exact entmax there."""
    from splash_attention import benchmark

    print(f"[lib] benchmark cli {baseline} backward={backward}", flush=True)
    r = benchmark.run_config(1, 2, 256, 64, 1.5, 8, torch.float32, baseline, backward,
                             input_scale=1.0, warmup=1, trials=2)
    for key in ("vanilla_time", "splash_time", "speedup", "mse_error", "max_error",
                "cosine_similarity", "vanilla_memory", "splash_memory"):
        assert key in r
    assert r["splash_time"] > 0 and r["vanilla_time"] > 0
    assert -1.0 <= r["cosine_similarity"] <= 1.0 + 1e-6
    assert r["mse_error"] >= 0 and r["max_error"] >= 0


def test_benchmark_cli_exact_mode_matches_dense_entmax(dev):
    """With tau_mode="exact" splash attention computes dense alpha-entmax,
    so against the CLI's dense "entmax" baseline (float32, 40 bisection
    steps) the notebook's error fields become a parity readout."""
    from splash_attention import benchmark

    print("[lib] benchmark cli exact mode", flush=True)
    r = benchmark.run_config(1, 2, 256, 64, 1.5, 8, torch.float32, "entmax", False,
                             input_scale=1.0, warmup=1, trials=2, tau_mode="exact")
    assert r["tau_mode"] == "exact"
    assert r["max_error"] <= 1e-5 and r["cosine_similarity"] > 1 - 1e-9, r


def test_benchmark_cli_kernel_times_and_cpu_baseline(dev):
    """--kernel-times lists the library's kernels with positive times;
    --cpu-baseline times the dense alpha-entmax on the host (all cores and
    one thread) and records the host."""
    from splash_attention import benchmark

    print("[lib] benchmark cli kernel times + cpu baseline", flush=True)
    r = benchmark.run_config(1, 2, 128, 64, 1.5, 8, torch.float32, "entmax", True,
                             input_scale=1.0, warmup=1, trials=2, kernel_times=True,
                             with_cpu=True)
    ks = r["kernel_us"]
    # reference tau mode: tau and the CSR lists run as one launch
    for name in ("select", "tau_compact", "forward", "bwd_dq_sparse", "bwd_dkdv_sparse"):
        assert ks[name] > 0, ks
    assert r["cpu_time"] > 0 and r["cpu_time_1thread"] > 0
    assert r["cpu_threads"] >= 1 and "model" in r["cpu_host"]


def test_benchmark_cli_rocprof_pmc(dev, tmp_path):
    """--rocprof-pmc runs the benchmark under rocprofv3 in a child process
    and summarises the library kernels' counters (one SQ counter: one
    hardware pass)."""
    import json
    import shutil
    import subprocess
    import sys

    if shutil.which("rocprofv3") is None:
        pytest.skip("rocprofv3 not installed")
    print("[lib] benchmark cli rocprof pmc SQ_WAVES", flush=True)
    out = subprocess.run(
        [sys.executable, "-m", "splash_attention.benchmark", "--config", "1x1x128x64",
         "--warmup", "1", "--trials", "1", "--rocprof-pmc", "SQ_WAVES",
         "--rocprof-dir", str(tmp_path)],
        capture_output=True, text=True, timeout=240, cwd=str(tmp_path),
        env={**__import__("os").environ,
             "PYTHONPATH": __import__("os").pathsep.join(sys.path)})
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-2000:]
    line = [ln for ln in out.stdout.splitlines() if ln.startswith('{"rocprof_pmc"')][-1]
    s = json.loads(line)["rocprof_pmc"]
    # one 128-row block per (batch, head): 4 waves per select launch
    assert s["select_kernel"]["SQ_WAVES"] >= 4, s
    assert "forward_kernel" in s


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_bwd_passes_agree(dev, dtype, tol):
    """bwd_passes "tiles" (whole active tiles on MFMA, no support masks
    recorded) and "support" (the support-pair passes) give the same
    gradients to the dtype's tolerance, through the module, the custom
    operator and the reference-order backward; the operator returns an
    empty support-mask tensor for "tiles"."""
    print(f"[lib] bwd_passes agree {dtype}", flush=True)
    B, H, N, d = 1, 2, 320, 64
    Q, K, V, dO = make_inputs(B, H, N, N, d, seed=13, dtype=dtype, scale=0.3)
    idx = causal_idx(B * H, N).to(dev)
    got = {}
    for passes in ("support", "tiles"):
        attn = sa.AdaptiveSplashAttention(head_dim=d, alpha=1.5, k_keep=16, bwd_passes=passes)
        q, k, v = (t.to(dev).requires_grad_(True) for t in (Q, K, V))
        out = attn(q, k, v, idx, idx)
        out.backward(dO.to(dev))
        ref_order = sa.backward(Q.to(dev), K.to(dev), V.to(dev), idx, idx, d ** -0.5, 1.5,
                                dO.to(dev), k_keep=16, grad_mode="entmax", block_m=64,
                                bwd_passes=passes)
        torch.cuda.synchronize()
        got[passes] = [x.detach().float().cpu() for x in (out, q.grad, k.grad, v.grad)]
        for a, b in zip(ref_order, got[passes][1:]):
            assert torch.equal(a.float().cpu(), b)
        sup = library.forward_op(Q.to(dev), K.to(dev), V.to(dev), idx, idx, 1.5, 16, d ** -0.5,
                                 "entmax", "reference", 64, passes)[-1]
        assert (sup.numel() > 0) == (passes == "support")
    for name, a, b in zip(("out", "dQ", "dK", "dV"), got["tiles"], got["support"]):
        err = (a - b).abs().max().item() / max(b.abs().max().item(), 1e-30)
        assert err <= tol, f"{name}: tiles against support {err:.2e} > {tol}"


def test_benchmark_cli_tile_backward(dev):
    """--bwd-passes tiles: the timed backward runs the dense tile passes
    (bwd_dq, bwd_dkdv), and the forward records no support masks."""
    from splash_attention import benchmark

    print("[lib] benchmark cli tile backward", flush=True)
    r = benchmark.run_config(1, 2, 128, 64, 1.5, 8, torch.float32, "entmax", True,
                             input_scale=0.1, warmup=1, trials=2, kernel_times=True,
                             bwd_passes="tiles")
    ks = r["kernel_us"]
    assert r["bwd_passes"] == "tiles"
    assert ks["bwd_dq"] > 0 and ks["bwd_dkdv"] > 0, ks
    assert "bwd_dq_sparse" not in ks and "bwd_dkdv_sparse" not in ks, ks
