"""Benchmark of the streaming semi-CRF scan on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg3] [--cpu-sample T] [--no-cpu] [--no-passes]

A step is one forward + backward (log semiring) over the whole synthetic
workload "cfg3" by default: B=1, T=1,000,000, C=24, K=300, emissions N(0,1)
cumsum'd along T, transition N(0,0.1), duration_bias[k,c] = -0.01k + N(0,0.05)
for k >= 1 (row 0 = 0), seed 20261203, generated on the host and resident in HBM
before timing.  Prints one JSON line.

Roofline: the path is bound by FP32 VALU and transcendental issue (log-sum-exp
over K*C^2 terms per position, ~10^4 ops per HBM byte), not by HBM or MFMA.
A cell is one (b, t, k, c_dst, c_src) term of the direct recursion; the
per-cell op counts below are fixed in advance and not re-tuned after measuring.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "torch-semimarkov_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

# FP32 VALU lane-op peak (packed-FP32 issue, 157.3/2 T/s) and transcendental
# (v_exp_f32 / v_log_f32, quarter rate) peak of one MI355X
V_PEAK = 78.6e12
T_PEAK = 9.83e12
# lane-op peak without packed FP32 (the kernels are built with packed FP32 off)
V_PEAK_NONPACKED = 39.3e12
# algorithmic ops per cell (b, t, k, c_dst, c_src) of the direct recursion:
# (VALU lane-ops, transcendentals).  The backward (14, 3) splits into the alpha
# recompute (5, 1), the beta recursion (4, 1) and the marginals (5, 1); this
# build stores alpha instead of recomputing it.
OPS = {"fwd_log": (5, 1), "bwd_log": (14, 3), "fwdbwd_log": (19, 4), "max": (3, 0)}
KERNEL_OPS = {"scan_fwd_kernel": (5, 1), "scan_bwd_kernel": (4, 1), "marginal_kernel": (5, 1)}
# What the kernels EXECUTE: the exact label factorisation.  Per position and
# sequence a pass evaluates max(K-1, 1)*C duration terms (t, k, c) and C^2
# label-mix terms (t, c', c) instead of K*C^2 cells.  Each term is priced with
# the ops of the pass it belongs to, (VALU lane-ops, transcendentals):
#   log forward     duration (5, 1) [edge add, + u, max, sub, exp+sum],  mix (5, 1)
#   beta scan       duration (4, 1),                                     mix (4, 1)
#   fused beta scan duration (9, 2) [beta (4, 1) + marginal (5, 1)],     mix (4, 1) [beta only;
#                   the transition gradient runs in its own kernel]
#   marginals       duration (5, 1),                                     mix (5, 1) [transition grad]
EXEC_OPS = {
    "scan_fwd_kernel": ((5, 1), (5, 1)),
    "scan_bwd_kernel": ((4, 1), (4, 1)),
    "scan_bwd_kernel_fused": ((9, 2), (4, 1)),
    "marginal_kernel": ((5, 1), (5, 1)),
}
PROFILES = os.path.join(ROOT, "profiles")


def roofline_cells_per_s(kind):
    nv, nt = OPS[kind]
    return 1.0 / (nv / V_PEAK + nt / T_PEAK)


def valu_equiv_ops_per_cell(kind):
    nv, nt = OPS[kind]
    return nv + nt * (V_PEAK / T_PEAK)


def executed_valu_ops(kernel, B, T, C, K):
    """VALU-equivalent lane-ops (transcendentals weighted by V_peak/T_peak) one
    launch of `kernel` executes on the factorised recursion: B*T positions times
    (duration terms * their ops + label-mix terms * theirs)."""
    (dv, dt), (mv, mt) = EXEC_OPS[kernel]
    w = V_PEAK / T_PEAK
    per_pos = max(K - 1, 1) * C * (dv + dt * w) + C * C * (mv + mt * w)
    return B * T * per_pos


def profiled_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` from the committed rocprofv3
    PMC summary (FETCH_SIZE and WRITE_SIZE scaled by a copy-kernel calibration),
    or None when no summary covers it.  Lines read: `traffic <kernel> <workload> <bytes>`."""
    path = os.path.join(PROFILES, "pmc_traffic.txt")
    try:
        with open(path) as f:
            for ln in f:
                parts = ln.split()
                if len(parts) == 4 and parts[0] == "traffic" and parts[1] == kernel and parts[2] == workload:
                    return float(parts[3])
    except OSError:
        pass
    return None


def profiled_executed(kernel, workload):
    """Executed VALU lane-op and transcendental rates of `kernel` from the committed
    SQ-counter summary (lines `executed <kernel> <workload> <lane-ops/s> <trans/s>`)."""
    path = os.path.join(PROFILES, f"pmc_instructions_{workload}.txt")
    out = None
    try:
        with open(path) as f:
            for ln in f:
                parts = ln.split()
                if len(parts) == 5 and parts[0] == "executed" and parts[1] == kernel and parts[2] == workload:
                    v, t = float(parts[3]), float(parts[4])
                    out = {"valu_lane_ops_per_s": v, "valu_frac_nonpacked_peak": v / V_PEAK_NONPACKED,
                           "transcendental_per_s": t, "transcendental_frac": t / T_PEAK,
                           "source": os.path.relpath(path, ROOT)}
                    break
    except OSError:
        pass
    # VALU-busy and LDS bank-conflict figures of the same kernel (lines
    # `busy <kernel> <workload> <VALUBusy%> <LDSBankConflict%> <conflicts/access>`)
    bpath = os.path.join(PROFILES, f"pmc_lds_valu_{workload}.txt")
    try:
        with open(bpath) as f:
            for ln in f:
                parts = ln.split()
                if len(parts) == 6 and parts[0] == "busy" and parts[1] == kernel and parts[2] == workload:
                    out = dict(out or {})
                    out.update({"valu_busy_pct": float(parts[3]), "lds_bank_conflict_pct": float(parts[4]),
                                "lds_conflicts_per_access": float(parts[5]),
                                "busy_source": os.path.relpath(bpath, ROOT)})
                    break
    except OSError:
        pass
    return out


def copy_calibration(mib=256, reps=3):
    """A plain device copy of known size, for scaling the FETCH_SIZE / WRITE_SIZE
    counters: run it under `rocprofv3 --pmc FETCH_SIZE` (then WRITE_SIZE)."""
    x = torch.empty(mib * 1024 * 1024 // 4, device="cuda")
    x.normal_()
    y = torch.empty_like(x)
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": x.numel() * 4, "bytes_written": y.numel() * 4, "reps": reps}))


CONFIGS = {
    "cfg1": dict(B=4, T=1000, C=24, K=100, H=512, seed=20261201),
    "cfg2": dict(B=32, T=10_000, C=8, K=1, seed=20261202),
    "cfg3": dict(B=1, T=1_000_000, C=24, K=300, seed=20261203),
    "cfg4": dict(B=64, T=8192, C=32, K=64, seed=20261204),
    "cfg5": dict(B=8, T=50_000, C=128, K=500, seed=20261205),
}


def make_inputs(name):
    """Host (CPU, fp32) inputs of a scan workload, drawn in the documented order
    with torch.Generator().manual_seed(seed): returns (cfg, cum (B,T+1,C),
    transition (C,C), duration_bias (K,C), lengths (B,) int64).  Also used by
    tests/golden/make_config_fixtures.py and the full-size parity tests, so the
    draws live in one place."""
    cfg = CONFIGS[name]
    B, T, C, K = cfg["B"], cfg["T"], cfg["C"], cfg["K"]
    g = torch.Generator().manual_seed(cfg["seed"])
    if name == "cfg4":
        L = torch.randint(4096, 8193, (B,), generator=g)
        em = torch.randn(B, T, C, generator=g)
        tr = 0.1 * torch.randn(C, C, generator=g)
        db = 0.1 * torch.randn(K, C, generator=g)
    else:
        em = torch.randn(B, T, C, generator=g)
        L = torch.full((B,), T, dtype=torch.long)
    if name == "cfg5":
        tr = 0.05 * torch.randn(C, C, generator=g)
        k = torch.arange(1, K, dtype=torch.float64)
        sigma, mu = 0.5, math.log(150.0) + 0.25
        shape = -torch.log(k * sigma * math.sqrt(2 * math.pi)) - (torch.log(k) - mu) ** 2 / (2 * sigma ** 2)
        db = torch.zeros(K, C)
        db[1:] = shape.float().unsqueeze(1) + 0.05 * torch.randn(K - 1, C, generator=g)
    elif name == "cfg2":
        tr = 0.1 * torch.randn(C, C, generator=g)
        db = 0.1 * torch.randn(1, C, generator=g)
    elif name == "cfg3":
        tr = 0.1 * torch.randn(C, C, generator=g)
        db = torch.zeros(K, C)
        db[1:] = -0.01 * torch.arange(1, K, dtype=torch.float32).unsqueeze(1) + 0.05 * torch.randn(K - 1, C, generator=g)
    cum = torch.zeros(B, T + 1, C)
    cum[:, 1:] = torch.cumsum(em, dim=1)
    return cfg, cum, tr, db, L


def make_head_inputs():
    """cfg1: SemiMarkovCRFHead(24, 100, 512) built right after torch.manual_seed(seed)
    (the reference's parameter order: transition, duration bias, projection), then
    h ~ N(0,1) (4, 1000, 512) and labels uniform in [0, 24) from
    torch.Generator().manual_seed(seed); lengths all 1000.  Host tensors."""
    import torch_semimarkov_amd as tsa

    cfg = CONFIGS["cfg1"]
    B, T, C, K, H, seed = cfg["B"], cfg["T"], cfg["C"], cfg["K"], cfg["H"], cfg["seed"]
    torch.manual_seed(seed)
    head = tsa.SemiMarkovCRFHead(C, K, hidden_dim=H)
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(B, T, H, generator=g)
    labels = torch.randint(0, C, (B, T), generator=g)
    L = torch.full((B,), T, dtype=torch.long)
    return cfg, head, h, L, labels


def bench_head(args):
    """cfg1: SemiMarkovCRFHead(24, 100, 512) on h ~ N(0,1) (4, 1000, 512), random labels:
    one step = compute_loss + backward, then decode_with_traceback; latency-bound."""
    cfg, head, h, L, labels = make_head_inputs()
    B, T, H, C, K, seed = cfg["B"], cfg["T"], cfg["H"], cfg["C"], cfg["K"], cfg["seed"]
    dev = torch.device("cuda", 0)
    head = head.to(dev)
    h, labels, L = h.to(dev), labels.to(dev), L.to(dev)

    def train_step():
        head.zero_grad(set_to_none=True)
        loss = head.compute_loss(h, L, labels)
        loss.backward()
        return loss

    for _ in range(args.warmup):
        train_step()
        head.decode_with_traceback(h, L)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        train_step()
    torch.cuda.synchronize()
    train_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    t0 = time.perf_counter()
    for _ in range(args.steps):
        res = head.decode_with_traceback(h, L)
    torch.cuda.synchronize()
    decode_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    cells = B * T * K * C * C
    print(json.dumps({
        "metric": "head compute_loss+backward cells/s (B*T*K*C^2), 1 GPU", "value": cells / (train_ms / 1e3),
        "unit": "cells/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": train_ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (random-init head, N(0,1) hidden states, uniform labels)",
        "config": {"workload": "cfg1: SemiMarkovCRFHead(24, 100, 512) loss + backward", "B": B, "T": T, "H": H,
                   "C": C, "K": K, "seed": seed},
        "decode_with_traceback_ms": decode_ms, "segments_seq0": len(res.segments[0]),
    }))


def bench_viterbi(args):
    """cfg4: Viterbi with backtrace (max semiring), 64 ragged sequences."""
    from torch_semimarkov_amd import _native as N
    from torch_semimarkov_amd.streaming import ops

    cfg, cum, tr, db, lengths = make_inputs("cfg4")
    B, T, C, K, seed = cfg["B"], cfg["T"], cfg["C"], cfg["K"], cfg["seed"]
    dev = torch.device("cuda", 0)
    cum, tr, db, L = cum.to(dev), tr.to(dev), db.to(dev), lengths.to(dev)

    def step():
        return ops.viterbi(cum, tr, db, L, K, None, None, True)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    # per-kernel HIP events on the launch stream, over the same steps again (outside the timed region)
    N.timing_enable(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ktimes = N.timing_read()
    N.timing_enable(False)
    cells_sum = int(lengths.sum()) * K * C * C
    print(json.dumps({
        "metric": "Viterbi + backtrace cells/s (sum_b L_b*K*C^2), 1 GPU", "value": cells_sum / (ms / 1e3),
        "unit": "cells/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "cfg4: Viterbi with traceback, ragged lengths in [4096, 8192]", "B": B,
                   "T_max": T, "C": C, "K": K, "seed": seed},
        "cells_B_Tmax": B * T * K * C * C, "value_B_Tmax": B * T * K * C * C / (ms / 1e3),
        "kernel_avg_ms": {k: v[0] / v[1] for k, v in sorted(ktimes.items())},
    }))


def host_facts():
    """Host CPU facts for the baseline: model name, physical cores, logical CPUs,
    and the CPUs this process may run on."""
    model, phys = "", set()
    try:
        cur = {}
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ":" not in ln:
                    if "physical id" in cur and "core id" in cur:
                        phys.add((cur["physical id"], cur["core id"]))
                    cur = {}
                    continue
                k, v = (x.strip() for x in ln.split(":", 1))
                cur[k] = v
                if k == "model name" and not model:
                    model = v
        if "physical id" in cur and "core id" in cur:
            phys.add((cur["physical id"], cur["core id"]))
    except OSError:
        model = platform.processor()
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = os.cpu_count() or 1
    return {"model": model or "unknown", "physical_cores": len(phys) or None, "logical_cpus": os.cpu_count(),
            "cpus_allowed": allowed}


def cpu_baseline(name, cum, tr, db, K, t_sample):
    """The oracle (fp32 PyTorch-CPU restatement of the reference's CPU streaming
    path, its arithmetic order kept) timed on this host: forward + backward on
    prefixes of the same workload of t_sample/2 and t_sample positions, median
    of 3 after one warm-up, extrapolated linearly in T to the full length (exact
    for T >> K: every position past K costs the same).  About 10-30 s of CPU."""
    from oracle import streaming_ref as R

    facts = host_facts()
    threads = max(1, min(facts["cpus_allowed"], 16))
    torch.set_num_threads(threads)
    B, Tp1, C = cum.shape
    T_full = Tp1 - 1
    t2 = min(t_sample, T_full)
    t1 = max(1, t2 // 2)

    def run(t):
        c = cum[:, : t + 1].contiguous()
        L = torch.full((B,), t, dtype=torch.long)
        t0 = time.perf_counter()
        part, ck, S = R.forward(c, tr, db, L, K, "log")
        R.backward(c, tr, db, L, K, part, ck, S, "log")
        return time.perf_counter() - t0

    run(max(1, min(t1, K + 16)))  # warm-up
    m1 = statistics.median(run(t1) for _ in range(3))
    m2 = statistics.median(run(t2) for _ in range(3))
    slope = (m2 - m1) / (t2 - t1) if t2 > t1 else m2 / t2
    full_s = m2 + slope * (T_full - t2)
    cells = B * T_full * K * C * C
    return {
        "value": cells / full_s,
        "unit": "cells/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{name}: oracle fp32 forward+backward on prefixes T={t1} and T={t2} (B={B}, C={C}, K={K}), "
                  f"median of 3 after a warm-up: {m1:.2f} s and {m2:.2f} s; extrapolated linearly to "
                  f"T={T_full}: {full_s:.0f} s (extrapolated)",
        "extrapolated_seconds_full": full_s,
        "median_seconds": {str(t1): m1, str(t2): m2},
        "host": facts,
        "torch_threads": torch.get_num_threads(),
    }


def measure_passes(args, cum, tr, db, L, K, cells, fwdbwd_ms, plan):
    """Per-pass rates on the same resident inputs: the no-grad forward (log
    partition only), forward + backward (the timed step) and Viterbi with
    backtrace (max semiring), each as nominal cells/s and as a fraction of that
    pass's roofline (ops per cell fixed in OPS).  Viterbi is timed only where
    the register-resident or the cooperative plan exists (the factorised
    max-plus scan); otherwise the exact kernel would run K*C^2 terms per step
    on one workgroup per sequence."""
    from torch_semimarkov_amd.streaming import ops

    def timed(fn):
        for _ in range(max(1, args.warmup)):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / args.steps

    with torch.no_grad():
        fwd = timed(lambda: ops.scan_forward(cum, tr, db, L, K, 0, None, None, False))
        vit = (timed(lambda: ops.viterbi(cum, tr, db, L, K, None, None, True))
               if (plan.get("fast") or plan.get("coop")) else None)

    def entry(ms, kind):
        rate = cells / (ms / 1e3)
        return {"ms": ms, "cells_per_s": rate, "nominal_roofline_frac": rate / roofline_cells_per_s(kind),
                "roofline_cells_per_s": roofline_cells_per_s(kind)}

    return {"forward_log": entry(fwd, "fwd_log"), "forward_backward_log": entry(fwdbwd_ms, "fwdbwd_log"),
            "viterbi_traceback": entry(vit, "max") if vit is not None else None}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="cfg3", choices=sorted(list(CONFIGS) + ["cfg1", "cfg4"]))
    ap.add_argument("--cpu-sample", type=int, default=1200)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-passes", action="store_true",
                    help="skip the per-pass timings (forward only, Viterbi), e.g. under a profiler")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy (PMC counter calibration)")
    ap.add_argument("--memory-budget", type=int, default=None,
                    help="time the bounded-memory backward (checkpointed windows) for this budget in "
                         "bytes (0: about eight windows) instead of the full-table backward")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        copy_calibration()
        return
    if args.config == "cfg1":
        bench_head(args)
        return
    if args.config == "cfg4":
        bench_viterbi(args)
        return

    import torch_semimarkov_amd as tsa
    from torch_semimarkov_amd import _native as N

    dev = torch.device("cuda", 0)
    cfg, cum_h, tr_h, db_h, L_h = make_inputs(args.config)
    B, T, C, K = cfg["B"], cfg["T"], cfg["C"], cfg["K"]
    cum = cum_h.to(dev).requires_grad_(True)
    tr = tr_h.to(dev).requires_grad_(True)
    db = db_h.to(dev).requires_grad_(True)
    L = L_h.to(dev)
    plan = N.plan_info(B, T, C, K)

    ev = []

    def step(record):
        cum.grad = tr.grad = db.grad = None
        if record:
            e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
            e0.record()
        part = tsa.semi_crf_streaming_forward(cum, tr, db, L, K, memory_budget=args.memory_budget)
        if record:
            e1.record()
        part.sum().backward()
        if record:
            e2.record()
            ev.append((e0, e1, e2))
        return part

    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    # the timed region (value): K steps, without the library's per-kernel events
    t0 = time.perf_counter()
    for _ in range(args.steps):
        part = step(True)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    # peak device memory of a step (inputs, outputs, saved tables, workspaces)
    peak_mem = torch.cuda.max_memory_allocated(dev)
    # the same K steps again with per-kernel HIP events, recorded by the library on
    # the stream each kernel runs on (kernel_avg_ms, roofline); the events add about
    # 1 % to the step, so they stay out of the timed region above
    N.timing_enable(True)
    for _ in range(args.steps):
        step(False)
    torch.cuda.synchronize()
    ktimes = N.timing_read()
    N.timing_enable(False)
    ms_step = dt * 1e3 / args.steps
    fwd_ms = statistics.mean(a.elapsed_time(b) for a, b, _ in ev)
    bwd_ms = statistics.mean(b.elapsed_time(c) for _, b, c in ev)

    cells = B * T * K * C * C
    value = cells / (ms_step / 1e3)
    passes = None if args.no_passes else measure_passes(args, cum.detach(), tr.detach(), db.detach(), L, K, cells,
                                                          ms_step, plan)
    # dominant kernel: the largest total time over the timed steps
    kops = dict(KERNEL_OPS)
    fused = bool(plan.get("mfused"))
    if fused:
        # the beta scan also accumulates the segment marginals: both passes' ops per cell
        kops["scan_bwd_kernel"] = tuple(a + b for a, b in zip(KERNEL_OPS["scan_bwd_kernel"], KERNEL_OPS["marginal_kernel"]))
    dom = max((k for k in ktimes if k in kops), key=lambda k: ktimes[k][0])
    dom_total, dom_launches = ktimes[dom]
    dom_avg_ms = dom_total / dom_launches
    nv, nt = kops[dom]
    # roofline on the executed (factorised) work, and the nominal per-cell pricing beside it
    exec_key = "scan_bwd_kernel_fused" if (dom == "scan_bwd_kernel" and fused) else dom
    exec_ops = executed_valu_ops(exec_key, B, T, C, K)
    achieved = exec_ops / (dom_avg_ms / 1e3) / 1e12
    nominal_achieved = cells * (nv + nt * V_PEAK / T_PEAK) / (dom_avg_ms / 1e3) / 1e12
    traffic = profiled_traffic(dom, args.config)
    peak = V_PEAK / 1e12
    out = {
        "metric": "fwd+bwd scan cells/s (B*T*K*C^2), 1 GPU",
        "value": value,
        "unit": "cells/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"{args.config}: streaming semi-CRF fwd+bwd, log semiring",
            "B": B, "T": T, "C": C, "K": K, "seed": cfg["seed"],
        },
        "roofline": {
            "bound": "valu",
            "kernel": dom,
            "achieved": achieved,
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": achieved / peak,
            "traffic": traffic,
            # what `achieved` counts: the factorised terms the kernel executes per launch
            "work": {
                "executed_terms_per_position": max(K - 1, 1) * C + C * C,
                "nominal_cells_per_position": K * C * C,
                "work_ratio": K * C * C / (max(K - 1, 1) * C + C * C),
                "ops_per_duration_term": dict(zip(("valu", "transcendental"), EXEC_OPS[exec_key][0])),
                "ops_per_mix_term": dict(zip(("valu", "transcendental"), EXEC_OPS[exec_key][1])),
                "valu_equiv_ops_per_launch": exec_ops,
                "formula": "B*T*(max(K-1,1)*C*(dv+dt*V/T) + C^2*(mv+mt*V/T)) / avg_launch_s / V_peak",
            },
            # nominal pricing: every B*T*K*C^2 cell of the direct recursion at the
            # pass's (VALU, transcendental) ops; above 1 because the factorisation skips most cells
            "nominal_frac": nominal_achieved / peak,
            "nominal_ops_per_cell": {"valu": nv, "transcendental": nt},
            # achieved HBM rate of the dominant kernel (profiled bytes / launch time) and of its
            # emission stream alone (the (B, T+1, C) fp32 cumulative scores, read once per pass)
            "hbm_gb_per_s": traffic / (dom_avg_ms / 1e3) / 1e9 if traffic else None,
            "emission_stream_gb_per_s": B * (T + 1) * C * 4 / (dom_avg_ms / 1e3) / 1e9,
            "hbm_peak_gb_per_s": 8000.0,
            "executed": profiled_executed(dom, args.config),
            "avg_launch_ms": dom_avg_ms,
        },
        "max_memory_allocated_bytes": peak_mem,
        "memory_budget": args.memory_budget,
        "nominal_roofline_frac_fwdbwd": value / roofline_cells_per_s("fwdbwd_log"),
        "passes": passes,
        "fwd_ms": fwd_ms,
        "bwd_ms": bwd_ms,
        "kernel_avg_ms": {k: v[0] / v[1] for k, v in sorted(ktimes.items())},
        "plan": plan,
        "logZ": float(part.detach()[0]),
    }
    if args.memory_budget is not None:
        from torch_semimarkov_amd.streaming import ops as tops
        w, nw, fw, bw = tops.checkpoint_plan(B, T, C, K, False, False, args.memory_budget)
        out["bounded"] = {"window": w, "n_windows": nw, "forward_workspace_bytes": fw,
                          "backward_workspace_bytes": bw}
    if not args.no_cpu and args.cpu_sample > 0:
        out["cpu_baseline"] = cpu_baseline(args.config, cum_h, tr_h, db_h, K, min(args.cpu_sample, T))
        out["speedup_vs_cpu"] = value / out["cpu_baseline"]["value"]
    print(json.dumps(out))


if __name__ == "__main__":
    main()
