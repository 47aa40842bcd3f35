"""Benchmark CLI with the metric set of the reference notebook.

The reference's harness (AdaSplashNotebook.ipynb, ``BenchmarkResult`` and
``benchmark_single_config``, nb:1688-1830) times its extension against a
dense attention and reports, per configuration: both times, the speed-up,
MSE / max absolute error / cosine similarity of the outputs, and the GPU
memory each one allocates.  This module reports the same fields for
``splash_attention`` against either

* ``entmax``  -- dense exact alpha-entmax attention in PyTorch (materialised
  scores, tau by bisection to float precision), the function the sparse
  attention approximates, or
* ``vanilla`` -- the notebook's ``vanilla_attention`` formula (softmax of
  scores / alpha, raised to alpha, renormalised), kept for comparison with
  the notebook's numbers.

Inputs follow the notebook's conventions: N(0, 1) * ``--input-scale``
(the notebook used 0.1), causal int32 ``arange`` positions, sm_scale =
1/sqrt(d).  ``--backward`` times forward + backward instead of the forward;
``--bwd-passes tiles`` runs that backward over whole active tiles instead
of the rows' support pairs (faster where the supports fill most of the
tiles, as they do on the 0.1-scaled inputs).

Beyond the notebook's fields:

* ``--kernel-times`` adds each library kernel's average time over the
  splash trials (HIP events the library records around its launches);
* ``--cpu-baseline`` times the dense alpha-entmax on the host CPU as well
  (all cores, and one thread), with the host's model and core count;
* ``--rocprof-pmc "COUNTER ..."`` runs the same benchmark under
  ``rocprofv3 --pmc`` (a child process; this process never touches the GPU
  then) and prints each library kernel's counter averages per dispatch.

    python -m splash_attention.benchmark --config 1x4x2048x64 --config 1x4x4096x64
"""
from __future__ import annotations

import argparse
import csv
import gc
import glob
import json
import math
import os
import re
import subprocess
import sys
import tempfile
import time

import torch

from . import _lib
from .function import splash_attention


def dense_entmax_attention(Q, K, V, alpha: float, sm_scale: float, iters: int = 40):
    """Exact alpha-entmax attention over causal scores (fp32 math); tau by
    bisection on [max - 1, max] of (alpha-1) * scores, iters steps."""
    q, k, v = (t.float() for t in (Q, K, V))
    S = torch.matmul(q, k.transpose(-1, -2).contiguous()) * sm_scale
    NQ, NK = S.shape[-2:]
    causal = torch.ones(NQ, NK, device=S.device, dtype=torch.bool).tril_(NK - NQ)
    z = (S * (alpha - 1.0)).masked_fill(~causal, -float("inf"))
    a = 1.0 / (alpha - 1.0)
    with torch.no_grad():
        hi = z.amax(-1, keepdim=True)
        lo = hi - 1.0
        for _ in range(iters):
            mid = 0.5 * (lo + hi)
            f = (z - mid).clamp(min=0).pow(a).sum(-1, keepdim=True) - 1.0
            lo = torch.where(f > 0, mid, lo)
            hi = torch.where(f > 0, hi, mid)
        tau = 0.5 * (lo + hi)
    P = (z - tau).clamp(min=0).pow(a)
    P = P / P.sum(-1, keepdim=True)
    return torch.matmul(P, v).to(Q.dtype)


def vanilla_attention(Q, K, V, alpha: float, sm_scale: float):
    """The notebook's comparison formula (nb:1715-1743): causal softmax of
    scores / alpha, raised to the power alpha and renormalised."""
    q, k, v = (t.float() for t in (Q, K, V))
    S = torch.matmul(q, k.transpose(-1, -2).contiguous()) * sm_scale
    NQ, NK = S.shape[-2:]
    S = S.masked_fill(~torch.ones(NQ, NK, device=S.device, dtype=torch.bool).tril_(NK - NQ),
                      -float("inf"))
    W = torch.softmax(S / alpha, dim=-1) if alpha != 1.0 else torch.softmax(S, dim=-1)
    if alpha != 1.0:
        W = torch.pow(W + 1e-8, alpha)
        W = W / W.sum(-1, keepdim=True)
    return torch.matmul(W, v).to(Q.dtype)


BASELINES = {"entmax": dense_entmax_attention, "vanilla": vanilla_attention}


def _time(fn, warmup: int, trials: int) -> tuple[float, float]:
    """(median ms, peak MB allocated above the starting point) of fn()."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    gc.collect()
    torch.cuda.empty_cache()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    times = []
    for _ in range(trials):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    peak = (torch.cuda.max_memory_allocated() - base) / 2 ** 20
    times.sort()
    return times[len(times) // 2], peak


def host_cpu() -> dict:
    """Model name, physical cores and logical CPUs of the host."""
    model, cores, phys, core = "unknown", set(), None, None
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                k, _, v = ln.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name":
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
    except OSError:
        pass
    return {"model": model, "physical_cores": len(cores) or None, "logical_cpus": os.cpu_count()}


def _time_cpu(fn, warmup: int, trials: int) -> float:
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(trials):
        t0 = time.perf_counter()
        fn()
        times.append((time.perf_counter() - t0) * 1e3)
    times.sort()
    return times[len(times) // 2]


def cpu_baseline(Q, K, V, dO, alpha: float, sm_scale: float, backward: bool, warmup: int,
                 trials: int) -> dict:
    """Dense alpha-entmax (dense_entmax_attention) on the host CPU: median ms
    with every core, and with one thread (one warm-up, three trials)."""
    q, k, v, g = (t.detach().float().cpu() for t in (Q, K, V, dO))

    def step():
        if backward:
            qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
            dense_entmax_attention(qq, kk, vv, alpha, sm_scale).backward(g)
        else:
            with torch.no_grad():
                dense_entmax_attention(q, k, v, alpha, sm_scale)

    prev = torch.get_num_threads()
    try:
        torch.set_num_threads(os.cpu_count() or 1)
        t_all = _time_cpu(step, warmup, trials)
        torch.set_num_threads(1)
        t_one = _time_cpu(step, 1, 3)
    finally:
        torch.set_num_threads(prev)
    return {"cpu_time": round(t_all, 3), "cpu_threads": os.cpu_count(),
            "cpu_time_1thread": round(t_one, 3), "cpu_host": host_cpu()}


def run_config(B: int, H: int, N: int, d: int, alpha: float = 1.5, k_keep: int = 8,
               dtype: torch.dtype = torch.float32, baseline: str = "entmax",
               backward: bool = False, input_scale: float = 0.1, warmup: int = 3,
               trials: int = 10, seed: int = 42, tau_mode: str = "reference",
               kernel_times: bool = False, with_cpu: bool = False,
               bwd_passes: str = "support") -> dict:
    """Benchmark one [B, H, N, d] configuration; returns the notebook's fields.
    tau_mode="exact" makes splash attention compute dense alpha-entmax, so
    against the "entmax" baseline the error fields measure parity.
    bwd_passes picks splash attention's backward ("support": over each row's
    support pairs; "tiles": over whole active tiles, faster when the supports
    fill most of them, as on the notebook's N(0,1) * 0.1 inputs)."""
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(seed)
    Q, K, V, dO = (torch.randn(B, H, N, d, generator=g).mul_(input_scale).to(dtype).to(dev)
                   for _ in range(4))
    idx = torch.arange(N, device=dev, dtype=torch.int32).unsqueeze(0).expand(B * H, N).contiguous()
    sm_scale = 1.0 / math.sqrt(d)
    dense = BASELINES[baseline]

    def make(fn):
        def step():
            if backward:
                q, k, v = (t.detach().requires_grad_(True) for t in (Q, K, V))
                fn(q, k, v).backward(dO)
            else:
                with torch.no_grad():
                    fn(Q, K, V)
        return step

    sp = lambda q, k, v: splash_attention(q, k, v, idx, idx, alpha, k_keep, sm_scale,
                                          tau_mode=tau_mode, bwd_passes=bwd_passes)
    dn = lambda q, k, v: dense(q, k, v, alpha, sm_scale)
    t_dense, m_dense = _time(make(dn), warmup, trials)
    t_splash, m_splash = _time(make(sp), warmup, trials)
    with torch.no_grad():
        a = sp(Q, K, V).float().flatten()
        b = dn(Q, K, V).float().flatten()
    mse = float(torch.mean((a - b) ** 2))
    max_err = float((a - b).abs().max())
    cos = float(torch.nn.functional.cosine_similarity(a, b, dim=0))
    extra = {}
    if kernel_times:
        # a second pass of the splash step with the library's launch events
        step = make(sp)
        torch.cuda.synchronize()
        _lib.profile_enable(True)
        try:
            for _ in range(trials):
                step()
            torch.cuda.synchronize()
            prof = _lib.profile_read()
        finally:
            _lib.profile_enable(False)
        extra["kernel_us"] = {name: round(ms / cnt * 1e3, 2) for name, (cnt, ms) in prof.items()}
    if with_cpu:
        extra.update(cpu_baseline(Q, K, V, dO, alpha, sm_scale, backward, warmup, trials))
    return {
        "config_name": f"{B}x{H}x{N}x{d}", "B": B, "H": H, "NQ": N, "NK": N, "d": d,
        "alpha": alpha, "k_keep": k_keep, "dtype": str(dtype).replace("torch.", ""),
        "baseline": baseline, "tau_mode": tau_mode, "pass": "fwd+bwd" if backward else "fwd",
        "bwd_passes": bwd_passes if backward else None,
        "vanilla_time": round(t_dense, 4), "splash_time": round(t_splash, 4),
        "speedup": round(t_dense / t_splash, 3),
        "mse_error": mse, "max_error": max_err, "cosine_similarity": cos,
        "vanilla_memory": round(m_dense, 2), "splash_memory": round(m_splash, 2),
        "memory_saving": round(m_dense / m_splash, 3) if m_splash > 0 else None,
        **extra,
    }


def parse_config(s: str) -> tuple[int, int, int, int]:
    parts = s.lower().split("x")
    if len(parts) != 4:
        raise argparse.ArgumentTypeError(f"config {s!r} must be BxHxNxd, e.g. 1x4x2048x64")
    try:
        return tuple(int(p) for p in parts)  # type: ignore[return-value]
    except ValueError as e:
        raise argparse.ArgumentTypeError(f"config {s!r}: {e}") from None


def build_parser() -> argparse.ArgumentParser:
    ap = argparse.ArgumentParser(prog="python -m splash_attention.benchmark",
                                 description="splash attention vs dense attention, "
                                             "the reference notebook's metric set")
    ap.add_argument("--config", type=parse_config, action="append",
                    help="BxHxNxd (repeatable); default 1x4x1024x64, 1x4x2048x64, 1x4x4096x64")
    ap.add_argument("--alpha", type=float, default=1.5)
    ap.add_argument("--k-keep", type=int, default=8)
    ap.add_argument("--dtype", choices=["fp32", "bf16", "fp16"], default="fp32")
    ap.add_argument("--baseline", choices=sorted(BASELINES), default="entmax")
    ap.add_argument("--backward", action="store_true", help="time forward + backward")
    ap.add_argument("--tau-mode", choices=["reference", "exact"], default="reference",
                    help="exact: the alpha-entmax threshold over the whole row")
    ap.add_argument("--bwd-passes", choices=["support", "tiles"], default="support",
                    help="backward of --backward: over support pairs, or over whole active "
                         "tiles (faster when the supports fill most of them, as on the "
                         "default --input-scale 0.1)")
    ap.add_argument("--input-scale", type=float, default=0.1)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--trials", type=int, default=10)
    ap.add_argument("--json", action="store_true", help="one JSON object per line")
    ap.add_argument("--kernel-times", action="store_true",
                    help="add each library kernel's average time (library launch events)")
    ap.add_argument("--cpu-baseline", action="store_true",
                    help="also time the dense alpha-entmax on the host CPU")
    ap.add_argument("--rocprof-pmc", metavar="COUNTERS",
                    help="run under rocprofv3 --pmc COUNTERS (space separated; one hardware "
                         "pass, e.g. 'SQ_INSTS_VALU SQ_INSTS_MFMA') and print per-kernel averages")
    ap.add_argument("--rocprof-dir", help="output directory of --rocprof-pmc (default: a "
                                          "temporary directory)")
    return ap


def rocprof_command(argv: list[str], counters: str, outdir: str) -> list[str]:
    """The child command of --rocprof-pmc: rocprofv3 with the counters around
    this benchmark, run by the Python interpreter itself (the program must
    follow "--" directly) with the rocprof options removed."""
    rest, skip = [], False
    for a in argv:
        if skip:
            skip = False
            continue
        if a in ("--rocprof-pmc", "--rocprof-dir"):
            skip = True
            continue
        if a.startswith("--rocprof-pmc=") or a.startswith("--rocprof-dir="):
            continue
        rest.append(a)
    return ["rocprofv3", "--pmc", *counters.split(), "--output-format", "csv", "-d", outdir,
            "-o", "run", "--", sys.executable, "-m", "splash_attention.benchmark", *rest]


def pmc_summary(outdir: str) -> dict[str, dict[str, float]]:
    """Per-dispatch counter averages of the library's kernels from a
    rocprofv3 counter-collection CSV: {kernel: {counter: mean}}."""
    acc: dict[str, dict[str, list[float]]] = {}
    for f in glob.glob(os.path.join(outdir, "**", "*counter_collection.csv"), recursive=True):
        with open(f) as fh:
            for row in csv.DictReader(fh):
                m = re.search(r"asa::[^:]*::(\w+_kernel)", row.get("Kernel_Name", ""))
                if not m:
                    continue
                acc.setdefault(m.group(1), {}).setdefault(row["Counter_Name"], []).append(
                    float(row["Counter_Value"]))
    return {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in acc.items()}


def run_under_rocprof(argv: list[str], counters: str, outdir: str | None) -> int:
    """Runs the benchmark under rocprofv3 as a child process (this process
    does not initialise the GPU) and prints the counter summary."""
    out = outdir or tempfile.mkdtemp(prefix="asa_pmc_")
    cmd = rocprof_command(argv, counters, out)
    print("running:", " ".join(cmd), flush=True)
    rc = subprocess.run(cmd).returncode
    summary = pmc_summary(out)
    if not summary:
        print(f"no counter records of the library's kernels under {out} (rocprofv3 exit {rc})",
              flush=True)
        return rc or 1
    for kern, cs in sorted(summary.items()):
        print(f"{kern:>22}: " + "  ".join(f"{c} {v:.4g}" for c, v in sorted(cs.items())),
              flush=True)
    print(json.dumps({"rocprof_pmc": summary, "dir": out}), flush=True)
    if rc:
        # rocprofv3 can exit non-zero while finalising after the program has
        # ended and its records are complete; the records are used
        print(f"note: rocprofv3 exited with {rc} after writing its records", flush=True)
    return 0


def main(argv=None) -> list[dict]:
    raw = list(sys.argv[1:] if argv is None else argv)
    args = build_parser().parse_args(raw)
    if args.rocprof_pmc:
        rc = run_under_rocprof(raw, args.rocprof_pmc, args.rocprof_dir)
        if rc:
            raise SystemExit(rc)
        return []
    configs = args.config or [(1, 4, 1024, 64), (1, 4, 2048, 64), (1, 4, 4096, 64)]
    dtype = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}[args.dtype]
    results = []
    for B, H, N, d in configs:
        r = run_config(B, H, N, d, args.alpha, args.k_keep, dtype, args.baseline, args.backward,
                       args.input_scale, args.warmup, args.trials, tau_mode=args.tau_mode,
                       kernel_times=args.kernel_times, with_cpu=args.cpu_baseline,
                       bwd_passes=args.bwd_passes)
        results.append(r)
        if args.json:
            print(json.dumps(r), flush=True)
        else:
            print(f"{r['config_name']:>14} {r['pass']:>7} {args.baseline:>7}: "
                  f"{r['vanilla_time']:9.3f} ms vs splash {r['splash_time']:8.3f} ms "
                  f"(x{r['speedup']:.1f})  mse {r['mse_error']:.2e}  max {r['max_error']:.2e}  "
                  f"cos {r['cosine_similarity']:.6f}  mem {r['vanilla_memory']:.0f} / "
                  f"{r['splash_memory']:.0f} MB", flush=True)
            if "kernel_us" in r:
                print("    kernels (us): " + ", ".join(f"{k} {v}" for k, v in r["kernel_us"].items()),
                      flush=True)
            if "cpu_time" in r:
                print(f"    dense CPU: {r['cpu_time']:.2f} ms on {r['cpu_threads']} threads, "
                      f"{r['cpu_time_1thread']:.2f} ms on 1 ({r['cpu_host']['model']})", flush=True)
    return results


if __name__ == "__main__":
    main()
