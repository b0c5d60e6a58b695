"""Benchmark of the headline path: differential threshold attention (TDA), bf16,
B=4, H=16, N=4096, d=128 (BASELINE configs[2] forward, configs[3] forward+backward).

A step is one forward + backward pass over one batch of synthetic N(0,1) inputs through the
public API (tda_amd.differential_threshold_rela_triton + autograd), inputs resident in HBM.
`value` is forward+backward TFLOP/s counted as causal dense FLOPs (11 U, U = B*H*N^2*d);
the forward alone (3 U) is reported under "fwd".  Prints one JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fwd/fwd+bwd TFLOP/s + % bf16 MFMA peak, diff-TDA B4 H16 N4096 d128"
PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 FLOP/clk/CU)
PEAK_HBM_GBS = 8000.0
SHAPE = (4, 16, 4096, 128)
BETA, LAM, POWER = 1.0, 0.5, 2.0
FWD_UNITS, FWDBWD_UNITS = 3.0, 11.0          # counted causal-dense units (U = B*H*N^2*d)
REF_FWD_UNITS, REF_FWDBWD_UNITS = 4.0, 14.0  # the reference's two independent TRA calls
# HBM bytes moved by one forward call (key_norms + fwd_screen + fwd_pv_cand + fwd_pv) at SHAPE, from rocprofv3
# --pmc FETCH_SIZE and --pmc WRITE_SIZE runs of this script, each scaled by what the same counter
# reads for --copy-probe (a 2^30-byte device copy): FETCH_SIZE x 2.000, WRITE_SIZE x 1.000.
# Recorded with the command lines in profiles/tda_c2_bf16_counters.md; re-measure after kernel changes.
FWD_HBM_BYTES = 1.020e9


def units(shape, u):
    b, h, n, d = shape
    return u * b * h * float(n) * n * d


def cpu_baseline(budget_s: float = 12.0):
    """The oracle's PyTorch formula (fp32, full N x N per head) timed on the host cores on
    a bounded sample of the same workload: forward+backward of whole (b, h) heads of the
    configs[3] inputs, as many heads as fit in ~budget_s."""
    import torch

    from oracle.formula import tda

    cores = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(cores)
    _, _, n, d = SHAPE
    g = torch.Generator("cpu").manual_seed(2)
    head = (1, 1, n, d)
    xs = [torch.randn(head, generator=g).to(torch.bfloat16).float() for _ in range(5)]
    do = torch.randn(head, generator=torch.Generator("cpu").manual_seed(3)).to(torch.bfloat16).float()

    def one(backward: bool):
        leaves = [x.clone().requires_grad_(backward) for x in xs]
        bt = torch.tensor(BETA, requires_grad=backward)
        lt = torch.tensor(LAM, requires_grad=backward)
        if backward:
            out = tda(*leaves, bt, lt, POWER, True)
            out.backward(do)
        else:
            with torch.no_grad():
                tda(*leaves, bt, lt, POWER, True)

    one(True)  # warm-up
    t_fb, t_f = [], []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < budget_s or len(t_fb) < 2:
        t0 = time.perf_counter(); one(True); t_fb.append(time.perf_counter() - t0)
        t0 = time.perf_counter(); one(False); t_f.append(time.perf_counter() - t0)
        if len(t_fb) >= 64:
            break
    fb, f = statistics.median(t_fb), statistics.median(t_f)
    model = ""
    try:
        with open("/proc/cpuinfo") as fh:
            for ln in fh:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": units(head, FWDBWD_UNITS) / fb / 1e12,
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"oracle.formula.tda (fp32 torch, full NxN) fwd+bwd on one (b,h) head of configs[3] "
                   f"(N={n}, d={d}), median of {len(t_fb)} heads-runs, {fb:.3f} s/head; "
                   f"same 11U causal-dense count"),
        "fwd_value": units(head, FWD_UNITS) / f / 1e12,
        "fwd_s_per_head": f,
        "cpu_model": model,
    }


def side_configs(steps: int, warmup: int):
    """The BASELINE "report" configurations, timed like the headline forward (HIP events on
    the launch stream around `steps` calls after `warmup`): configs[1] (TRA, bf16,
    (4,16,2048,64), seed 1, beta 1, p 2, normalize) and configs[4] (TDA, bf16, (1,32,16384,128),
    seed 4, beta 2, lambda 0.3, normalize) at p = 1 and p = 1.5, with the kernels' tile counters;
    plus a KV-cache decode step (one query against 16384 keys)."""
    import torch

    from tda_amd import ops

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    res = {}

    def timed(fn):
        with torch.no_grad():
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(steps):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    def tiles(call):
        st = torch.zeros(3, dtype=torch.int64, device=dev)
        with torch.no_grad():
            call(st)
        visited, nonzero, kept = (int(x) for x in st.tolist())
        return {"tiles_visited": visited, "tiles_screen_kept": kept, "tiles_nonzero": nonzero,
                "skipped_tile_fraction": 1.0 - nonzero / max(visited, 1)}

    shape1 = (4, 16, 2048, 64)
    g = torch.Generator("cpu").manual_seed(1)
    q, k, v = (torch.randn(shape1, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    beta = torch.tensor(1.0, device=dev)
    ms = timed(lambda: ops.forward(q, k, None, None, v, beta, None, 2.0, True, 1))
    res["configs[1]"] = {"workload": "TRA fwd bf16 (4,16,2048,64) seed 1, beta=1, p=2, normalize, causal",
                         "ms": ms, "tflops": units(shape1, 2.0) / (ms * 1e-3) / 1e12,
                         "pct_peak": 100.0 * units(shape1, 2.0) / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                         "counted_units": 2.0,
                         **tiles(lambda st: ops.forward(q, k, None, None, v, beta, None, 2.0, True, 1, stats=st))}
    del q, k, v
    shape4 = (1, 32, 16384, 128)
    g = torch.Generator("cpu").manual_seed(4)
    xs = [torch.randn(shape4, generator=g).to(torch.bfloat16).to(dev) for _ in range(5)]
    q1, q2, k1, k2, v = xs
    beta, lam = torch.tensor(2.0, device=dev), torch.tensor(0.3, device=dev)
    for p in (1.0, 1.5):
        ms = timed(lambda: ops.forward(q1, k1, q2, k2, v, beta, lam, p, True, 2))
        res[f"configs[4] p={p}"] = {
            "workload": f"TDA fwd bf16 (1,32,16384,128) seed 4, beta=2, lambda=0.3, p={p}, normalize, causal",
            "ms": ms, "tflops": units(shape4, 3.0) / (ms * 1e-3) / 1e12,
            "pct_peak": 100.0 * units(shape4, 3.0) / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, "counted_units": 3.0,
            **tiles(lambda st: ops.forward(q1, k1, q2, k2, v, beta, lam, p, True, 2, stats=st))}
    # KV-cache decode (no BASELINE config; the position-offset extension): one query at the last
    # position of a 16384-key cache.  HBM-bound: the keys of both branches are read once, V
    # only for non-zero tiles; roofline = key bytes / time against 8 TB/s.
    B, H, NK, D = 4, 16, 16384, 128
    g = torch.Generator("cpu").manual_seed(5)
    qd1, qd2 = (torch.randn(B, H, 1, D, generator=g).to(torch.bfloat16).to(dev) for _ in range(2))
    del q1, q2, k1, k2, v, xs
    kd1, kd2, vd = (torch.randn(B, H, NK, D, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    beta, lam = torch.tensor(1.0, device=dev), torch.tensor(0.5, device=dev)
    ms = timed(lambda: ops.forward(qd1, kd1, qd2, kd2, vd, beta, lam, 2.0, True, 2, q_offset=NK - 1))
    kbytes = 2 * B * H * NK * D * 2
    res["decode"] = {"workload": f"TDA fwd bf16, one query at position {NK - 1} against ({B},{H},{NK},{D}) keys, "
                                 "beta=1, lambda=0.5, p=2, normalize (seed 5)",
                     "ms": ms, "bound": "hbm", "key_bytes": kbytes, "achieved_gbs": kbytes / (ms * 1e-3) / 1e9,
                     "frac_of_8tbs": kbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                     **tiles(lambda st: ops.forward(qd1, kd1, qd2, kd2, vd, beta, lam, 2.0, True, 2, stats=st,
                                                    q_offset=NK - 1))}
    return res


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-side", action="store_true", help="skip the configs[1] / configs[4] report figures")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 1 GiB device copy 3 times (calibrates HBM byte counters)")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (got --gpus {args.gpus}); the op shards "
              "over (batch, heads) with no exchange, so N GPUs run N independent copies.", file=sys.stderr)
        return 2

    import torch

    import tda_amd
    from tda_amd import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe:
        # a copy kernel of known size: reads and writes 2^30 bytes per dispatch
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": 1 << 30, "copy_probe_bytes_written": 1 << 30, "dispatches": 3}))
        return 0
    g = torch.Generator("cpu").manual_seed(2)
    xs = [torch.randn(SHAPE, generator=g).to(torch.bfloat16).to(dev) for _ in range(5)]
    do = torch.randn(SHAPE, generator=torch.Generator("cpu").manual_seed(3)).to(torch.bfloat16).to(dev)
    q1, q2, k1, k2, v = xs
    beta = torch.tensor(BETA, device=dev)
    lam = torch.tensor(LAM, device=dev)
    stream = torch.cuda.current_stream(dev)

    # ---- forward only (key_norms, fwd_screen, fwd_pv per call), timed with events on its stream
    with torch.no_grad():
        for _ in range(args.warmup):
            ops.forward(q1, k1, q2, k2, v, beta, lam, POWER, True, 2)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            ops.forward(q1, k1, q2, k2, v, beta, lam, POWER, True, 2)
        e1.record(stream)
        torch.cuda.synchronize()
        fwd_ms = e0.elapsed_time(e1) / args.steps

    # ---- forward + backward through the public API (the step)
    leaves = [x.clone().requires_grad_(True) for x in xs]
    bt = beta.clone().requires_grad_(True)
    lt = lam.clone().requires_grad_(True)

    def step():
        for t in (*leaves, bt, lt):
            t.grad = None
        out = tda_amd.differential_threshold_rela_triton(*leaves, bt, lt, relu_power=POWER, normalize=True)
        out.backward(do)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record(stream)
    for _ in range(args.steps):
        step()
    s1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    step_ms = s0.elapsed_time(s1) / args.steps

    # ---- skip statistics (untimed)
    stats = torch.zeros(3, dtype=torch.int64, device=dev)
    with torch.no_grad():
        ops.forward(q1, k1, q2, k2, v, beta, lam, POWER, True, 2, stats=stats)
    visited, computed, checked = (int(x) for x in stats.tolist())

    fwd_flop = units(SHAPE, FWD_UNITS)
    fb_flop = units(SHAPE, FWDBWD_UNITS)
    fwd_tf = fwd_flop / (fwd_ms * 1e-3) / 1e12
    fb_tf = fb_flop / (max(step_ms, wall_ms) * 1e-3) / 1e12
    res = {
        "metric": METRIC,
        "value": fb_tf,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": max(step_ms, wall_ms),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "configs[3]: differential TDA forward+backward, bf16 in / fp32 accumulate, "
                               "B=4 H=16 N=4096 d=128, beta=1 lambda=0.5 p=2 normalize causal; "
                               "forward alone = configs[2]",
                   "batch": SHAPE[0], "heads": SHAPE[1], "seq_len": SHAPE[2], "head_dim": SHAPE[3],
                   "parallelism": "single GPU"},
        "pct_peak": 100.0 * fb_tf / PEAK_BF16_TFLOPS,
        "fwd": {"ms": fwd_ms, "tflops": fwd_tf, "pct_peak": 100.0 * fwd_tf / PEAK_BF16_TFLOPS,
                "counted_units": FWD_UNITS, "tiles_visited": visited, "tiles_screen_kept": checked,
                "tiles_pv_computed": computed,
                "skipped_tile_fraction": 1.0 - computed / max(visited, 1)},
        "fwd_bwd": {"ms": max(step_ms, wall_ms), "event_ms": step_ms, "wall_ms": wall_ms, "tflops": fb_tf,
                    "pct_peak": 100.0 * fb_tf / PEAK_BF16_TFLOPS, "counted_units": FWDBWD_UNITS},
        "reference_equivalent": {
            "note": "FLOPs of two independent TRA calls (4U fwd, 14U fwd+bwd), as the reference executes",
            "fwd_tflops": units(SHAPE, REF_FWD_UNITS) / (fwd_ms * 1e-3) / 1e12,
            "fwd_bwd_tflops": units(SHAPE, REF_FWDBWD_UNITS) / (max(step_ms, wall_ms) * 1e-3) / 1e12},
        "roofline": {"kernel": "forward (key_norms + fwd_screen + fwd_pv_cand + fwd_pv), events around the launches",
                     "bound": "mfma",
                     "achieved": fwd_tf, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": fwd_tf / PEAK_BF16_TFLOPS, "traffic": FWD_HBM_BYTES,
                     "algorithmic": "3U = 4.1232e11 FLOP per launch (causal dense)",
                     "traffic_note": "HBM bytes per forward call (rocprofv3 FETCH_SIZE/WRITE_SIZE, copy-calibrated); "
                                     "compulsory 4.027e8",
                     "hbm_gbs_at_traffic": FWD_HBM_BYTES / (fwd_ms * 1e-3) / 1e9},
    }
    if not args.no_side:
        res["side_configs"] = side_configs(max(3, args.steps // 4), 2)
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(args.cpu_budget)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
