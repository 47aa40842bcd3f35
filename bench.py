#!/usr/bin/env python3
"""Headline benchmark: block-sparse alpha-entmax attention fwd+bwd on one MI355X.

Workload: B=4, H=16, N=4096, d=64, bf16,
alpha=1.5, k_keep=32, sm_scale=0.125, causal (Q_idx = K_idx = arange),
64x64 blocks, Q/K/V and the upstream gradient ~ N(0,1) (synthetic, seeded).

One step = forward (score pass, CSR compaction, block-sparse forward with
the rows' support masks) plus backward (dQ, dK/dV over the support pairs,
entmax-Jacobian gradient) through the autograd API, inputs resident in
HBM.  value = effective TFLOP/s with the FlashAttention
convention for dense causal fwd+bwd, 3.5 * 4 * BH * d * N^2 / 2 = 481.0 GFLOP
per step.

The K timed steps run uninstrumented, after W untimed ones.  The default
W = 100 (about 85 ms of GPU work) times the steady state: measured with
HIP events per step, the step time of a fresh process falls from ~0.91 to
~0.81 ms over its first ~40 steps of sustained load (the GPU's clocks
settling) and then holds.  Per-kernel durations come from a
second pass of K steps in which the library records HIP events around each
launch on the launch stream (asa_profile_*); the roofline of each kernel
uses its algorithmic FLOPs / bytes per launch.

The line also carries the same step with the other tau mode
(`exact_tau_mode`: the alpha-entmax threshold over the whole visible row,
i.e. dense alpha-entmax attention computed block-sparsely), timed the same
way; --tau-mode exact swaps the two.

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 100] [--tau-mode reference|exact]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "adaptive-splash-attention_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "fwd+bwd ms & eff. TFLOP/s at B4 H16 N4096 d64 bf16; % MFMA/HBM roofline"
WORK = dict(B=4, H=16, N=4096, d=64, alpha=1.5, k_keep=32, sm_scale=0.125)
PEAK_MFMA_BF16 = 2.5e15  # dense bf16 MFMA, FLOP/s
PEAK_HBM = 8.0e12        # HBM3E, bytes/s
ELEM = 2                 # bf16 bytes


COPY_BYTES = 256 << 20   # --copy-calibration copy size
# HBM bytes per launch of each kernel at this workload, measured with
# rocprofv3 FETCH_SIZE (x2.0) + WRITE_SIZE (x1.0), the factors a plain
# 256 MiB device copy gives (profiles/headline_hbm_traffic.md), on the
# library built from the sources whose hash is HBM_TRAFFIC_SOURCES
# (source_hash()).  A line from a library built from other sources reports
# traffic null and says why: counters of another build are not evidence.
HBM_TRAFFIC_SOURCES = "2d00522ce6db3e3c"
HBM_TRAFFIC = {'bounds': 1109233, 'select': 138861915, 'tau': 34745917, 'tau_compact': 37510848, 'refine': 109582540, 'compact': 2762350, 'forward': 329894294, 'bwd_dq_sparse': 240749933, 'bwd_dkdv_sparse': 287676950}


def source_hash() -> str:
    """sha256 (first 16 hex digits) of the library's sources: csrc/* and the
    C ABI header, in name order."""
    import hashlib
    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "adaptive-splash-attention_amd", "csrc")
    files = sorted(os.path.join(csrc, f) for f in os.listdir(csrc)
                   if f.endswith((".hip", ".hpp", ".cpp")))
    files.append(os.path.join(ROOT, "include", "adasplash.h"))
    for f in files:
        h.update(os.path.basename(f).encode())
        with open(f, "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def host_cpu() -> dict:
    """Model name and core counts of the host (from /proc/cpuinfo)."""
    model, cores = "unknown", set()
    phys = core = None
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
    return {"model": model, "physical_cores": len(cores) or None,
            "logical_cpus": os.cpu_count()}


def effective_flops(B, H, N, d):
    return 3.5 * 4 * B * H * d * N * N / 2


def support_pairs(st) -> int:
    """(row, key) pairs with u > 0 recorded in the state's support masks
    (active tile slots only: slot e < q_ptr[bh, nQB])."""
    import torch
    lut = torch.tensor([bin(i).count("1") for i in range(256)], dtype=torch.int32,
                       device=st.sup_mask.device)
    total = 0
    for bh in range(st.sup_mask.shape[0]):
        n = int(st.q_ptr[bh, -1])
        total += int(lut[st.sup_mask[bh, :n].contiguous().view(torch.uint8).long()].sum())
    return total


def kernel_models(B, H, N, d, nnzb, nQB, nKB, k_keep, nsup):
    """Algorithmic FLOPs and HBM bytes per launch of every kernel (nsup: the
    support pairs the sparse backward visits)."""
    BH = B * H
    rows = BH * N
    vis = BH * N * (N + 1) // 2          # visible (query, key) pairs, causal
    tile = 64 * d * ELEM                 # one 64-row tile of Q, K, V or dO
    csr = 4 * BH * (2 * nQB * nKB + nQB + nKB + 2)
    vis_blocks = BH * nQB * (nQB + 1) // 2
    return {
        "select": dict(bound="mfma", flops=2.0 * d * vis,
                       bytes=rows * d * ELEM + vis_blocks * tile + rows * k_keep * 4
                       + BH * nQB * nKB),
        "tau": dict(bound="hbm", flops=0.0, bytes=rows * k_keep * 4 + rows * 4),
        # exact tau mode: FLOPs of ONE full-row sweep (the kernel sweeps a
        # query block until its rows converge, a data-dependent count)
        "refine": dict(bound="mfma", flops=2.0 * d * vis,
                       bytes=rows * d * ELEM + vis_blocks * tile + rows * k_keep * 4),
        "bounds": dict(bound="hbm", flops=0.0, bytes=BH * N * 4 + BH * nKB * 8),
        "compact": dict(bound="hbm", flops=0.0, bytes=2 * BH * nQB * nKB + csr),
        # tau and compact in one launch (reference tau mode)
        "tau_compact": dict(bound="hbm", flops=0.0,
                            bytes=rows * k_keep * 4 + rows * 4 + 2 * BH * nQB * nKB + csr),
        # the forward's tile bytes are mostly L2-served (its algorithmic byte
        # rate exceeds the HBM peak); its MFMA work is the bound
        "forward": dict(bound="mfma", flops=4.0 * 64 * 64 * d * nnzb,
                        bytes=nnzb * 2 * tile + 2 * rows * d * ELEM + 2 * rows * 4
                        + 4 * BH * (nQB + 1 + nnzb // BH)),
        "bwd_dq": dict(bound="hbm", flops=8.0 * 64 * 64 * d * nnzb,
                       bytes=nnzb * 2 * tile + 3 * rows * d * ELEM + 4 * rows * 4),
        "bwd_dkdv": dict(bound="hbm", flops=8.0 * 64 * 64 * d * nnzb,
                         bytes=nnzb * 2 * tile + 4 * rows * d * ELEM + nnzb * 64 * 4 * 5),
        # support-mask backward: per listed pair, two gathered d-rows and
        # 8 d FLOPs (two dot products, two accumulations).  `bytes` is what
        # must cross HBM once (the rows read and written, 512 bytes of masks
        # per active tile, the row records); `l2_bytes` are the per-pair
        # gathers of rows that the passes re-read from L2 (a row is listed
        # by tens of pairs), priced as an L2 rate, not against HBM
        "bwd_dq_sparse": dict(bound="hbm", flops=8.0 * d * nsup,
                              bytes=5 * rows * d * ELEM + nnzb * 512 + rows * (8 + 16) + 4 * nnzb,
                              l2_bytes=nsup * 2 * d * ELEM),
        "bwd_dkdv_sparse": dict(bound="hbm", flops=8.0 * d * nsup,
                                bytes=6 * rows * d * ELEM + nnzb * 512 + rows * 16
                                + 4 * BH * nQB * nKB,
                                l2_bytes=nsup * (2 * d * ELEM + 16)),
    }


def roofline_of(model, ms):
    t = ms / 1e3
    mf = model["flops"] / t / PEAK_MFMA_BF16 if model["flops"] else 0.0
    hb = model["bytes"] / t / PEAK_HBM
    if model["bound"] == "mfma":
        ach, peak, unit = model["flops"] / t / 1e12, PEAK_MFMA_BF16 / 1e12, "TFLOP/s"
    else:
        ach, peak, unit = model["bytes"] / t / 1e9, PEAK_HBM / 1e9, "GB/s"
    r = {"bound": model["bound"], "achieved": round(ach, 3), "peak": peak, "unit": unit,
         "frac": round(ach / peak, 4), "traffic": None, "avg_ms": round(ms, 5),
         "mfma_frac": round(mf, 4), "hbm_frac_algorithmic": round(hb, 4),
         "alg_flops": model["flops"], "alg_bytes": model["bytes"]}
    if hb > 1.0:
        # more algorithmic bytes than HBM can deliver in this time: they come
        # from L2, so the byte model is not an HBM bound for this kernel
        r["model_note"] = "algorithmic bytes above the HBM peak rate: L2-served, not an HBM bound"
    if model.get("l2_bytes"):
        r["l2_bytes"] = model["l2_bytes"]
        r["l2_gather_GBps"] = round(model["l2_bytes"] / t / 1e9, 1)
        r["model_note"] = ("HBM fraction of the bytes that must cross HBM once; the per-pair row "
                           "gathers (l2_bytes) are L2-served, and the gather latency and the "
                           "VALU work per pair bound the pass")
    return r


def dense_entmax_fwd_bwd(Q, K, V, dO, alpha, scale, iters=40):
    """Dense exact alpha-entmax attention fwd+bwd in PyTorch on whatever
    device the tensors are on (fp32 math, materialised [BH, NQ, NK] scores
    clamped to [-10, 10] as the reference does, causal by position, tau by
    `iters` bisection steps on [max - 1, max] of (alpha-1) * scores, exact
    entmax Jacobian gradient).  Returns (O, dQ, dK, dV)."""
    import torch

    q, k, v, go = (t.float() for t in (Q, K, V, dO))
    kt = k.transpose(-1, -2).contiguous()
    S = torch.matmul(q, kt).mul_(scale).clamp_(-10.0, 10.0)
    NQ, NK = S.shape[-2:]
    causal = torch.ones(NQ, NK, device=S.device, dtype=torch.bool).tril_(NK - NQ)
    z = S.mul_(alpha - 1.0).masked_fill_(~causal, -float("inf"))
    a = 1.0 / (alpha - 1.0)
    hi = z.amax(-1, keepdim=True)
    lo = hi - 1.0
    for _ in range(iters):
        mid = 0.5 * (lo + hi)
        f = (z - mid).clamp_(min=0).pow_(a).sum(-1, keepdim=True) - 1.0
        pos = f > 0
        lo = torch.where(pos, mid, lo)
        hi = torch.where(pos, hi, mid)
    P = (z - 0.5 * (lo + hi)).clamp_(min=0).pow_(a)
    P = P / P.sum(-1, keepdim=True)
    O = torch.matmul(P, v)
    dP = torch.matmul(go, v.transpose(-1, -2).contiguous())
    g = torch.where(P > 0, P.pow(2.0 - alpha), torch.zeros_like(P))
    shift = (g * dP).sum(-1, keepdim=True) / g.sum(-1, keepdim=True)
    dS = g * (dP - shift)
    dQ = torch.matmul(dS, k) * scale
    dK = torch.matmul(dS.transpose(-1, -2).contiguous(), q) * scale
    dV = torch.matmul(P.transpose(-1, -2).contiguous(), go)
    return O, dQ, dK, dV


def dense_gpu_baseline(Q, K, V, dO, alpha, scale, iters=40, runs=5):
    """dense_entmax_fwd_bwd on the GPU; returns (median, min) ms per fwd+bwd
    over `runs` runs after one warm-up, and the run count."""
    import torch

    def run():
        return dense_entmax_fwd_bwd(Q, K, V, dO, alpha, scale, iters)

    run()
    torch.cuda.synchronize()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        run()
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(times), min(times), runs


def dense_cpu_baseline(warmup=3, trials=10):
    """The primary CPU baseline of the build's plan: dense exact alpha-entmax
    attention fwd+bwd in PyTorch (dense_entmax_fwd_bwd) on the host CPU at
    BASELINE configs[0] (c1) and configs[1] (c2), fp32, Q/K/V ~ N(0,1)
    (seed 0) and dO ~ N(0,1) (seed 1), with every core of the host and with
    one thread; median and min of `trials` runs after `warmup` warm-ups
    each.  The reference itself has no CPU path (adasplashattention.cu:543)."""
    import torch

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    prev = torch.get_num_threads()
    res = {"threads": threads, "host": host_cpu(), "kind": "dense PyTorch",
           "what": "dense exact alpha-entmax fwd+bwd in PyTorch on the host CPU, fp32, "
                   "[BH, N, N] scores, 40 bisection steps, exact entmax Jacobian; median "
                   f"of {trials} runs after {warmup} warm-ups"}
    try:
        for name, (B, H, N) in {"c1": (1, 2, 256), "c2": (2, 8, 1024)}.items():
            g = torch.Generator().manual_seed(0)
            Q, K, V = (torch.randn(B, H, N, 64, generator=g) for _ in range(3))
            dO = torch.randn(B, H, N, 64, generator=torch.Generator().manual_seed(1))
            fn = lambda: dense_entmax_fwd_bwd(Q, K, V, dO, 1.5, 0.125)
            entry = {"shape": f"B={B} H={H} N={N} d=64 fp32 alpha=1.5 causal, fwd+bwd"}
            for label, n in (("all_cores", threads), ("one_thread", 1)):
                torch.set_num_threads(n)
                med, mn = _time(fn, warmup, trials)
                entry[label] = {"ms": round(med * 1e3, 3), "min_ms": round(mn * 1e3, 3),
                                "threads": n,
                                "tflops": round(effective_flops(B, H, N, 64) / med / 1e12, 6)}
            res[name] = entry
    finally:
        torch.set_num_threads(prev)
    return res


def _oracle_run(heads, N, d, k, alpha, scale, seed=0):
    import numpy as np
    import torch

    from oracle import oracle as orc

    g = torch.Generator().manual_seed(seed)
    Q, K, V, dO = (torch.randn(heads, N, d, generator=g).to(torch.bfloat16).float().numpy()
                   for _ in range(4))
    idx = np.broadcast_to(np.arange(N, dtype=np.int32), (heads, N)).copy()
    return lambda: orc.attention(Q, K, V, idx, idx, dO, alpha, scale, k)


def _time(fn, warmup, trials):
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(trials):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), min(times)


def cpu_baseline(heads=16, warmup=3, trials=10):
    """The CPU oracle (C restatement of the reference algorithm, OpenMP over
    (batch, head) slices) on a bounded sample of the headline workload:
    `heads` of its 64 slices at full N = 4096 (one slice per core of a
    16-core share), bf16-rounded inputs in fp32; 3 warm-ups and 10 timed
    trials (the notebook's counts, nb:1757-1758), median and min.  Also a
    1-thread figure on one slice (1 warm-up, 3 trials: a 1-thread trial
    takes ~1.5 s), and the c1 / c2 configurations (BASELINE configs[0, 1])
    at the same thread count."""
    N, d = WORK["N"], WORK["d"]
    alpha, scale, k = WORK["alpha"], WORK["sm_scale"], WORK["k_keep"]
    from oracle import oracle as orc
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    orc.set_num_threads(threads)
    med, mn = _time(_oracle_run(heads, N, d, k, alpha, scale), warmup, trials)
    flops = effective_flops(1, heads, N, d)
    out = {"value": round(flops / med / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
           "kind": "port",
           "sample": f"oracle fwd+bwd (entmax grad) on {heads} of the 64 (batch, head) slices, "
                     f"N={N} d={d} k={k}, {threads} OpenMP threads, median of {trials} trials "
                     f"after {warmup} warm-ups: {med:.3f} s (min {mn:.3f} s)",
           "ms_per_step_scaled": round(med * 1e3 * 64 / heads, 1),
           "scaled": f"value and ms_per_step_scaled scale the {heads}-slice sample to the "
                     f"64 slices of the headline step (x{64 / heads:g})",
           "host": host_cpu()}
    # one thread, one slice (the OpenMP loops are over slices)
    from oracle import oracle as orc
    prev = orc.set_num_threads(1)
    try:
        m1, _ = _time(_oracle_run(1, N, d, k, alpha, scale), 1, 3)
    finally:
        orc.set_num_threads(prev)
    out["one_thread"] = {"value": round(effective_flops(1, 1, N, d) / m1 / 1e12, 6),
                         "unit": "TFLOP/s", "ms_per_slice": round(m1 * 1e3, 1),
                         "ms_per_step_scaled": round(m1 * 1e3 * 64, 1),
                         "sample": "1 of 64 slices, 1 thread, median of 3 after 1 warm-up"}
    cfgs = {}
    for name, (BH, Nc, kc) in {"c1": (2, 256, 8), "c2": (16, 1024, 8)}.items():
        mc, mnc = _time(_oracle_run(BH, Nc, 64, kc, 1.5, 0.125), warmup, trials)
        cfgs[name] = {"ms": round(mc * 1e3, 3), "min_ms": round(mnc * 1e3, 3),
                      "shape": f"BH={BH} N={Nc} d=64 fp32 k={kc} alpha=1.5 causal, fwd+bwd"}
    out["configs"] = cfgs
    out["dense_pytorch"] = dense_cpu_baseline(warmup, trials)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--grad-mode", default="entmax", choices=["entmax", "reference"])
    ap.add_argument("--tau-mode", default="reference", choices=["reference", "exact"],
                    help="reference: the reference's top-k threshold (the headline); exact: "
                         "the alpha-entmax threshold over the whole visible row")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-dense-baseline", action="store_true")
    ap.add_argument("--no-exact-line", action="store_true",
                    help="skip the exact_tau_mode entry (the other tau mode, same workload)")
    ap.add_argument("--layout", default="bhnd", choices=["bhnd", "bnhd"],
                    help="bhnd: contiguous [B, H, N, d] operands (the headline); bnhd: Q, K, V, "
                         "dO stored [B, N, H, d] and passed as transposed [B, H, N, d] views "
                         "(read in place by the strided kernel variants; the step then calls "
                         "the ops-level forward/backward, so autograd's gradient layout copies "
                         "stay out of the timed region)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run 3 plain device copies of 256 MiB (the reference kernel "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (no collectives or sharding); "
              "use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import splash_attention as sa
    from splash_attention import _lib

    dev = torch.device("cuda:0")
    B, H, N, d = WORK["B"], WORK["H"], WORK["N"], WORK["d"]
    alpha, k_keep, scale = WORK["alpha"], WORK["k_keep"], WORK["sm_scale"]
    g = torch.Generator().manual_seed(0)
    Q, K, V = (torch.randn(B, H, N, d, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    dO = torch.randn(B, H, N, d, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(dev)
    idx = torch.arange(N, dtype=torch.int32, device=dev).unsqueeze(0).expand(B * H, N).contiguous()
    q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
    if args.copy_calibration:
        src = torch.ones(COPY_BYTES, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    def step():
        q.grad = k.grad = v.grad = None
        out = sa.splash_attention(q, k, v, idx, idx, alpha, k_keep, scale, args.grad_mode,
                                  args.tau_mode)
        out.backward(dO)

    if args.layout == "bnhd":
        # the same values, stored [B, N, H, d]: views with row stride H d
        qt, kt, vt, dOt = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (Q, K, V, dO))
        qt, kt, vt, _, _ = sa.ops.check_inputs(qt, kt, vt, idx, idx)
        assert not qt.is_contiguous()  # read in place, not copied

        def step():
            out, st = sa.ops.splash_forward(qt, kt, vt, idx, idx, alpha, k_keep, scale,
                                            tau_mode=args.tau_mode)
            sa.ops.splash_backward(qt, kt, vt, idx, idx, out, dOt, st, alpha, k_keep, scale,
                                   args.grad_mode)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # The K timed steps run without instrumentation; a second pass of K
    # steps with HIP events around every kernel launch (asa_profile_enable)
    # gives the per-kernel times of the roofline entries.
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    _lib.profile_read()  # drop anything recorded so far
    _lib.profile_enable(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    kern = _lib.profile_read()

    # Block-mask density of this workload (same for every step: same inputs).
    _, st = sa.ops.splash_forward(*sa.ops.check_inputs(Q, K, V, idx, idx), alpha, k_keep, scale,
                                  tau_mode=args.tau_mode)
    nnzb = int(st.mask.sum().item())
    nsup = support_pairs(st)
    nQB = nKB = N // 64
    models = kernel_models(B, H, N, d, nnzb, nQB, nKB, k_keep, nsup)
    src = source_hash()
    traffic_ok = src == HBM_TRAFFIC_SOURCES
    kernels = {}
    for name, (cnt, tot) in kern.items():
        if name in models:
            kernels[name] = roofline_of(models[name], tot / cnt)
            kernels[name]["launches"] = cnt
            kernels[name]["traffic"] = HBM_TRAFFIC.get(name) if traffic_ok else None
            # measured HBM bytes over the same time: the algorithmic tile
            # bytes of the dense passes are mostly served by L2 (their
            # algorithmic HBM fraction can exceed 1)
            if traffic_ok and HBM_TRAFFIC.get(name):
                kr = kernels[name]
                kr["hbm_frac_measured"] = round(HBM_TRAFFIC[name] / (tot / cnt / 1e3) / PEAK_HBM, 4)
                if kr["bound"] == "hbm" and HBM_TRAFFIC[name] < 0.5 * kr["alg_bytes"] \
                        and "l2_bytes" not in kr:
                    # gathered rows that L2 serves: the byte model is an L2
                    # rate, not an HBM one
                    kr["model_note"] = (f"measured HBM traffic is "
                                        f"{HBM_TRAFFIC[name] / kr['alg_bytes']:.2f} of the "
                                        "algorithmic bytes: L2-served gathers")
    dominant = max(kernels, key=lambda n: kernels[n]["avg_ms"])
    roof = {kk: kernels[dominant][kk] for kk in ("bound", "achieved", "peak", "unit", "frac",
                                                 "traffic")}
    roof["kernel"] = dominant

    eff = effective_flops(B, H, N, d)
    line = {
        "metric": METRIC,
        "value": round(eff / (ms / 1e3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) inputs, seeded",
        "config": {"workload": "adaptive splash attention fwd+bwd (BASELINE configs[2])",
                   "B": B, "H": H, "N": N, "d": d, "alpha": alpha, "k_keep": k_keep,
                   "sm_scale": scale, "mask": "causal", "block": "64x64",
                   "grad_mode": args.grad_mode, "tau_mode": args.tau_mode,
                   "layout": args.layout,
                   "parallelism": "single GPU",
                   "active_block_pairs": nnzb,
                   "support_pairs": nsup,
                   "active_block_density_of_causal": round(nnzb / (B * H * nQB * (nQB + 1) / 2), 4)},
        "roofline": roof,
        "kernels": kernels,
        "library_sources": src,
    }
    if not traffic_ok:
        line["traffic_note"] = (f"HBM traffic table measured on sources {HBM_TRAFFIC_SOURCES}, "
                                f"this build is {src}: traffic not reported")
    if not args.no_exact_line:
        # the other tau mode on the same workload, timed the same way (the
        # headline fields above are the --tau-mode run's)
        other = "exact" if args.tau_mode == "reference" else "reference"

        def step_other():
            q.grad = k.grad = v.grad = None
            out = sa.splash_attention(q, k, v, idx, idx, alpha, k_keep, scale, args.grad_mode,
                                      other)
            out.backward(dO)

        for _ in range(args.warmup):
            step_other()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step_other()
        torch.cuda.synchronize()
        oms = (time.perf_counter() - t0) * 1e3 / args.steps
        line[f"{other}_tau_mode"] = {"ms_per_step": round(oms, 4),
                                     "value": round(eff / (oms / 1e3) / 1e12, 3),
                                     "unit": "TFLOP/s",
                                     "what": "same workload and step with tau_mode=" + repr(other)}
    if not args.no_dense_baseline:
        try:
            dms, dmin, dn = dense_gpu_baseline(Q, K, V, dO, alpha, scale)
            line["dense_gpu_baseline"] = {"ms_per_step": round(dms, 3), "min_ms": round(dmin, 3),
                                          "speedup": round(dms / ms, 2),
                                          "what": "PyTorch dense exact alpha-entmax fwd+bwd, fp32 "
                                                  "math, [64,4096,4096] scores, 40 bisection "
                                                  f"steps; median of {dn} runs after 1 warm-up"}
        except Exception as e:  # report, do not fail the bench line
            line["dense_gpu_baseline"] = {"error": repr(e)[:200]}
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
