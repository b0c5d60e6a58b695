"""Benchmark of the headline path: differential threshold attention (TDA), bf16,
B=4, H=16, N=4096, d=128 (BASELINE configs[2] forward, configs[3] forward+backward).

A step is one forward + backward pass over one batch of synthetic N(0,1) inputs through the
public API (tda_amd.differential_threshold_rela_triton + autograd), inputs resident in HBM.
`value` is forward+backward TFLOP/s counted as causal dense FLOPs (11 U, U = B*H*N^2*d): a
dense-equivalent count that includes the work the kernels skip, so it can pass the MFMA peak.
The forward alone (3 U) is reported under "fwd".  `roofline` is the dominant kernel
(fwd_screen): its algorithmic FLOPs over its own average launch duration, measured with HIP
events the library records on the launch stream between its launches
(tda_amd.timing.LaunchTimer).  Prints one JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-side]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fwd/fwd+bwd TFLOP/s + % bf16 MFMA peak, diff-TDA B4 H16 N4096 d128"
PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 FLOP/clk/CU)
PEAK_F32_TFLOPS = 157.3     # MI355X dense fp32 MFMA
PEAK_I8_TOPS = 5033.2       # MI355X dense int8 MFMA (twice the bf16 rate; published as 5.0 POP/s)
PEAK_HBM_GBS = 8000.0
SHAPE = (4, 16, 4096, 128)
BETA, LAM, POWER = 1.0, 0.5, 2.0
FWD_UNITS, FWDBWD_UNITS = 3.0, 11.0          # counted causal-dense units (U = B*H*N^2*d)
REF_FWD_UNITS, REF_FWDBWD_UNITS = 4.0, 14.0  # the reference's two independent TRA calls
SCREEN_UNITS = 2.0                           # fwd_screen: Q1 K1^T and Q2 K2^T over the causal half
# (with normalize, fwd_screen runs v_mfma_i32_32x32x32_i8: 2U int8 operations, priced at the int8 peak)
# HBM bytes per forward-only launch of the dominant kernel (fwd_screen) at SHAPE, from rocprofv3
# --pmc FETCH_SIZE and --pmc WRITE_SIZE runs of this script, each scaled by what the same counter
# reads for --copy-probe (a 2^30-byte device copy): FETCH_SIZE x 2.000, WRITE_SIZE x 1.000 (300.2 MB
# read + 3.8 MB written, the mean of the forward-only dispatches).  The command lines and the
# per-kernel figures are in profiles/tda_c2_bf16_counters.md; re-measure after kernel changes.
SCREEN_HBM_BYTES = 3.040e8
SCREEN_KERNEL = "fwd_screen"
SETTLE_S = 0.3  # seconds of untimed steps before the first timed region (see settle)


def units(shape, u):
    b, h, n, d = shape
    return u * b * h * float(n) * n * d


def tile_flops(d):
    """FLOPs of one 32x32 tile of a contraction over d (a score tile, or an A.V tile)."""
    return 2.0 * 32 * 32 * d


def _cpu_model() -> str:
    """lscpu's model name with its family / model / stepping numbers (some hosts report only the
    product line, e.g. "AMD EPYC"), else /proc/cpuinfo's model name."""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        fields = {}
        for ln in out.splitlines():
            if ":" in ln:
                k, v = ln.split(":", 1)
                fields.setdefault(k.strip(), v.strip())
        if fields.get("Model name"):
            ids = [f"{k.lower()} {fields[k]}" for k in ("CPU family", "Model", "Stepping") if fields.get(k)]
            return fields["Model name"] + (f" ({', '.join(ids)})" if ids else "")
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as fh:
            for ln in fh:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _cpu_quota() -> float | None:
    """CPUs the cgroup grants this process (cpu.max), None when unlimited or unreadable."""
    try:
        with open("/sys/fs/cgroup/cpu.max") as fh:
            quota, period = fh.read().split()[:2]
        return None if quota == "max" else int(quota) / int(period)
    except (OSError, ValueError):
        return None


def cpu_baseline(budget_s: float = 12.0):
    """The oracle's PyTorch formula (fp32, full N x N per head) timed on all the host cores this
    process may run on (its affinity set) on a bounded sample of the same workload:
    forward+backward of whole (b, h) heads of the configs[3] inputs, as many heads as fit in
    ~budget_s."""
    import torch

    from oracle.formula import tda

    cores = len(os.sched_getaffinity(0))
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
    while time.perf_counter() - t_start < budget_s or len(t_fb) < 3:
        t0 = time.perf_counter(); one(True); t_fb.append(time.perf_counter() - t0)
        t0 = time.perf_counter(); one(False); t_f.append(time.perf_counter() - t0)
        if len(t_fb) >= 64:
            break
    fb, f = statistics.median(t_fb), statistics.median(t_f)
    return {
        "value": units(head, FWDBWD_UNITS) / fb / 1e12,
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"oracle.formula.tda (fp32 torch, full NxN) fwd+bwd on one (b,h) head of configs[3] "
                   f"(N={n}, d={d}), median of {len(t_fb)} runs, {fb:.3f} s/head, "
                   f"torch.set_num_threads({cores}) = the affinity set; same 11U causal-dense count"),
        "fwd_value": units(head, FWD_UNITS) / f / 1e12,
        "fwd_s_per_head": f,
        "cpu_model": _cpu_model(),
        "cgroup_cpu_quota": _cpu_quota(),
    }


def time_calls(stream, fn, steps, warmup):
    """Average milliseconds per fn() call: HIP events on `stream` around `steps` calls."""
    import torch

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


def settled_calls(stream, fn, steps, warmup, seconds=0.05):
    """time_calls after `seconds` of untimed calls (the side figures follow per-launch timings,
    which synchronise per call and leave the GPU idle between calls)."""
    settle(fn, seconds)
    return time_calls(stream, fn, steps, warmup)


def settle(fn, seconds):
    """Run fn() back to back for `seconds` of wall time, untimed, then synchronise.  The GPU's
    clocks ramp up over the first tens of milliseconds of work after an idle period: measured on
    the box, 20 steps right after 0.5 s idle took 381 us per step, the same 20 steps once the GPU
    had been busy 333-337 us, and 100 steps after 50 warm-ups 330 us.  Every timed region of this
    script starts on a busy GPU, so it measures the kernels at their steady clock."""
    import torch

    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        fn()
    torch.cuda.synchronize()


def time_launches(fn, calls, warmup):
    """Average microseconds of each kernel family of one C-ABI call made by fn(), from events
    the library records between its launches (tda_amd.timing.LaunchTimer)."""
    import torch

    from tda_amd.timing import LaunchTimer

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    timer = LaunchTimer(calls)
    for _ in range(calls):
        timer.arm()
        fn()
        timer.collect()
    return timer.mean_us(), timer.total_us()


def tile_stats(call, dev):
    """The kernels' own counters of one forward: (visited, non-zero, screen-kept) tiles."""
    import torch

    st = torch.zeros(3, dtype=torch.int64, device=dev)
    with torch.no_grad():
        call(st)
    visited, nonzero, kept = (int(x) for x in st.tolist())
    return {"tiles_visited": visited, "tiles_screen_kept": kept, "tiles_nonzero": nonzero,
            "skipped_tile_fraction": 1.0 - nonzero / max(visited, 1)}


def side_configs(steps: int, warmup: int):
    """The BASELINE "report" configurations, timed like the headline forward (HIP events on
    the launch stream around `steps` calls after `warmup`, and each launch on its own):
    configs[1] (TRA, bf16, (4,16,2048,64), seed 1, beta 1, p 2, normalize) and configs[4] (TDA,
    bf16, (1,32,16384,128), seed 4, beta 2, lambda 0.3, normalize) at p = 1 and p = 1.5, with
    the kernels' tile counters; a KV-cache decode step (one query against 16384 keys); and the
    fp32 path (the reference's own compute precision) at the README shape and at the headline
    shape."""
    import torch

    from tda_amd import ops

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    res = {}

    def timed(fn, n=steps, w=warmup):
        with torch.no_grad():
            return settled_calls(stream, fn, n, w)

    def per_launch(fn, n=steps):
        with torch.no_grad():
            us, _ = time_launches(fn, n, 1)
        return {k: round(v, 2) for k, v in us.items()}

    shape1 = (4, 16, 2048, 64)
    g = torch.Generator("cpu").manual_seed(1)
    q, k, v = (torch.randn(shape1, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    beta = torch.tensor(1.0, device=dev)
    f1 = lambda: ops.forward(q, k, None, None, v, beta, None, 2.0, True, 1)  # noqa: E731
    ms = timed(f1)
    st1 = tile_stats(lambda st: ops.forward(q, k, None, None, v, beta, None, 2.0, True, 1, stats=st), dev)
    lu = per_launch(f1)
    screen_ex = st1["tiles_visited"] * tile_flops(64)
    res["configs[1]"] = {"workload": "TRA fwd bf16 (4,16,2048,64) seed 1, beta=1, p=2, normalize, causal",
                         "ms": ms, "tflops": units(shape1, 2.0) / (ms * 1e-3) / 1e12,
                         "pct_peak": 100.0 * units(shape1, 2.0) / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                         "counted_units": 2.0, "launch_us": lu,
                         "screen_frac_of_i8_peak": (units(shape1, 1.0) / (lu.get(SCREEN_KERNEL, 1e9) * 1e-6) / 1e12
                                                    / PEAK_I8_TOPS),
                         "screen_executed_gflop": screen_ex / 1e9, **st1}
    del q, k, v
    shape4 = (1, 32, 16384, 128)
    g = torch.Generator("cpu").manual_seed(4)
    xs = [torch.randn(shape4, generator=g).to(torch.bfloat16).to(dev) for _ in range(5)]
    q1, q2, k1, k2, v = xs
    beta, lam = torch.tensor(2.0, device=dev), torch.tensor(0.3, device=dev)
    for p in (1.0, 1.5):
        f4 = lambda: ops.forward(q1, k1, q2, k2, v, beta, lam, p, True, 2)  # noqa: E731
        ms = timed(f4)
        res[f"configs[4] p={p}"] = {
            "workload": f"TDA fwd bf16 (1,32,16384,128) seed 4, beta=2, lambda=0.3, p={p}, normalize, causal",
            "ms": ms, "tflops": units(shape4, 3.0) / (ms * 1e-3) / 1e12,
            "pct_peak": 100.0 * units(shape4, 3.0) / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, "counted_units": 3.0,
            "launch_us": per_launch(f4, max(3, steps // 2)),
            **tile_stats(lambda st: ops.forward(q1, k1, q2, k2, v, beta, lam, p, True, 2, stats=st), dev)}
    del q1, q2, k1, k2, v, xs
    # KV-cache decode (no BASELINE config; the position-offset extension): one query at the last
    # position of a 16384-key cache.  HBM-bound: the keys of both branches are read once, V
    # only for non-zero tiles; roofline = key bytes / time against 8 TB/s.
    B, H, NK, D = 4, 16, 16384, 128
    g = torch.Generator("cpu").manual_seed(5)
    qd1, qd2 = (torch.randn(B, H, 1, D, generator=g).to(torch.bfloat16).to(dev) for _ in range(2))
    kd1, kd2, vd = (torch.randn(B, H, NK, D, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    beta, lam = torch.tensor(1.0, device=dev), torch.tensor(0.5, device=dev)
    fd = lambda: ops.forward(qd1, kd1, qd2, kd2, vd, beta, lam, 2.0, True, 2, q_offset=NK - 1)  # noqa: E731
    ms = timed(fd)
    kbytes = 2 * B * H * NK * D * 2
    res["decode"] = {"workload": f"TDA fwd bf16, one query at position {NK - 1} against ({B},{H},{NK},{D}) keys, "
                                 "beta=1, lambda=0.5, p=2, normalize (seed 5)",
                     "ms": ms, "bound": "hbm", "key_bytes": kbytes, "achieved_gbs": kbytes / (ms * 1e-3) / 1e9,
                     "frac_of_8tbs": kbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, "launch_us": per_launch(fd),
                     **tile_stats(lambda st: ops.forward(qd1, kd1, qd2, kd2, vd, beta, lam, 2.0, True, 2, stats=st,
                                                         q_offset=NK - 1), dev)}
    del qd1, qd2, kd1, kd2, vd
    res["fp32"] = fp32_figures(dev, stream)
    res["dense"] = dense_figures(dev, stream, steps)
    return res


def dense_figures(dev, stream, steps):
    """The reference's default call (threshold_rela_triton(q, k, v, beta): no normalisation,
    TTA:472-486, README.md:20-31) at the configs[1] shape (4, 16, 2048, 64), beta = 1, p = 2: raw
    dot products of N(0, 1) rows pass their threshold about half the time, so every tile holds
    weights (the dense regime).  bf16 forward and forward+backward (the step through autograd),
    and fp32 the same.  Counted FLOPs: forward 2U (Q K^T and A V over the causal half), forward +
    backward 7U (the backward's recomputed scores, dP = dO V^T, dQ, dK and dV).  The forward's
    dominant kernel, the tile pass fwd_pv, against the bf16 peak on the work it executes (a score
    tile and an A.V tile per non-zero tile, from the kernels' counters)."""
    import torch

    from tda_amd import ops, threshold_rela_triton

    shape = (4, 16, 2048, 64)
    out = {}
    for name, dt in (("bf16", torch.bfloat16), ("fp32", torch.float32)):
        g = torch.Generator("cpu").manual_seed(1)
        q, k, v = (torch.randn(shape, generator=g).to(dt).to(dev) for _ in range(3))
        do = torch.randn(shape, generator=torch.Generator("cpu").manual_seed(3)).to(dt).to(dev)
        beta = torch.tensor(1.0, device=dev)
        fwd = lambda: ops.forward(q, k, None, None, v, beta, None, 2.0, False, 1)  # noqa: E731
        with torch.no_grad():
            ms_f = settled_calls(stream, fwd, steps, 2)
            lu, _ = time_launches(fwd, max(3, steps // 2), 1)
        st = tile_stats(lambda s: ops.forward(q, k, None, None, v, beta, None, 2.0, False, 1, stats=s), dev)
        leaves = [x.clone().requires_grad_(True) for x in (q, k, v)]

        def step():
            for t in leaves:
                t.grad = None
            threshold_rela_triton(*leaves, beta, relu_power=2.0).backward(do)

        settle(step, 0.05)
        for _ in range(2):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        ms_s = e0.elapsed_time(e1) / steps
        peak = PEAK_BF16_TFLOPS if dt == torch.bfloat16 else PEAK_F32_TFLOPS
        rec = {"workload": f"TRA {name} {shape} seed 1, beta=1, p=2, normalize=False (the reference's default call)",
               "fwd_ms": ms_f, "fwd_tflops": units(shape, 2.0) / (ms_f * 1e-3) / 1e12,
               "fwd_pct_peak": 100.0 * units(shape, 2.0) / (ms_f * 1e-3) / 1e12 / peak,
               "fwd_launch_us": {kk: round(t, 2) for kk, t in lu.items()},
               "fwd_bwd_ms": ms_s, "fwd_bwd_tflops": units(shape, 7.0) / (ms_s * 1e-3) / 1e12,
               "fwd_bwd_pct_peak": 100.0 * units(shape, 7.0) / (ms_s * 1e-3) / 1e12 / peak,
               "peak_tflops": peak, **st}
        pv = lu.get("fwd_pv") or lu.get("fwd_wave")
        if pv:
            executed = st["tiles_nonzero"] * 2 * tile_flops(shape[3])
            rec["tile_pass"] = {"kernel": "fwd_pv" if "fwd_pv" in lu else "fwd_wave", "launch_us": pv,
                                "executed_gflop": executed / 1e9,
                                "achieved_tflops": executed / (pv * 1e-6) / 1e12,
                                "frac_of_peak": executed / (pv * 1e-6) / 1e12 / peak,
                                "note": "a score tile and an A.V tile per non-zero tile (the block pass "
                                        "scores every causal tile: executed counts the non-zero ones only)"}
        out[name] = rec
        del q, k, v, do, leaves
    return out


def fp32_figures(dev, stream):
    """The fp32 path (the reference computes every call in fp32): TRA at the README shape
    (1, 8, 128, 64), and differential TDA forward and forward+backward at the headline shape,
    against the 157.3 TFLOP/s fp32 MFMA peak (counted causal-dense FLOPs, as for bf16)."""
    import torch

    from tda_amd import ops

    out = {}
    g = torch.Generator("cpu").manual_seed(0)
    shp = (1, 8, 128, 64)
    q, k, v = (torch.randn(shp, generator=g).to(dev) for _ in range(3))
    beta = torch.tensor(1.0, device=dev)
    with torch.no_grad():
        ms = settled_calls(stream, lambda: ops.forward(q, k, None, None, v, beta, None, 2.0, False, 1), 50, 10)
    out["readme_tra"] = {"workload": "TRA fwd fp32 (1,8,128,64), beta=1, p=2 (README usage)", "ms": ms,
                         "tflops": units(shp, 2.0) / (ms * 1e-3) / 1e12,
                         "pct_f32_peak": 100.0 * units(shp, 2.0) / (ms * 1e-3) / 1e12 / PEAK_F32_TFLOPS}
    g = torch.Generator("cpu").manual_seed(2)
    xs = [torch.randn(SHAPE, generator=g).to(dev) for _ in range(5)]
    do = torch.randn(SHAPE, generator=torch.Generator("cpu").manual_seed(3)).to(dev)
    q1, q2, k1, k2, v = xs
    beta, lam = torch.tensor(BETA, device=dev), torch.tensor(LAM, device=dev)
    fwd = lambda: ops.forward(q1, k1, q2, k2, v, beta, lam, POWER, True, 2)  # noqa: E731
    with torch.no_grad():
        ms_f = settled_calls(stream, fwd, 10, 2)
    # the backward as a training step runs it: on the side outputs and pair lists of its forward
    norms, occ = ops.side_buffers(SHAPE, 2, True, dev)
    pairs = ops.pair_buffer(SHAPE, 2, dev)
    with torch.no_grad():
        ops.forward(q1, k1, q2, k2, v, beta, lam, POWER, True, 2, norms, occ, pairs=pairs)
        bwd = lambda: ops.backward(q1, k1, q2, k2, v, do, beta, lam, POWER, True, 2, norms, occ,  # noqa: E731
                                   pairs=pairs)
        ms_b = settled_calls(stream, bwd, 10, 2)
        bwd_launch_us, _ = time_launches(bwd, 5, 1)
    out["c2_tda"] = {"workload": "TDA fp32 (4,16,4096,128) seed 2, beta=1, lambda=0.5, p=2, normalize",
                     "fwd_ms": ms_f, "fwd_tflops": units(SHAPE, 3.0) / (ms_f * 1e-3) / 1e12,
                     "fwd_pct_f32_peak": 100.0 * units(SHAPE, 3.0) / (ms_f * 1e-3) / 1e12 / PEAK_F32_TFLOPS,
                     "bwd_ms": ms_b, "bwd_launch_us": {k: round(t, 2) for k, t in bwd_launch_us.items()},
                     "fwd_bwd_ms": ms_f + ms_b,
                     "fwd_bwd_tflops": units(SHAPE, 11.0) / ((ms_f + ms_b) * 1e-3) / 1e12,
                     "fwd_bwd_pct_f32_peak": (100.0 * units(SHAPE, 11.0) / ((ms_f + ms_b) * 1e-3) / 1e12
                                              / PEAK_F32_TFLOPS)}
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-side", action="store_true", help="skip the configs[1] / configs[4] / fp32 report figures")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--dense-only", action="store_true",
                    help="only the dense-regime figures (side_configs.dense), for a kernel trace of that regime")
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
        # and its rate: the HBM rate a kernel that reads and writes equal amounts can reach here
        ms = time_calls(torch.cuda.current_stream(dev), lambda: dst.copy_(src), 20, 3)
        print(json.dumps({"copy_probe_bytes_read": 1 << 30, "copy_probe_bytes_written": 1 << 30, "dispatches": 26,
                          "copy_gbs_read_plus_written": 2.0 * (1 << 30) / (ms * 1e-3) / 1e9}))
        return 0
    if args.dense_only:
        print(json.dumps({"dense": dense_figures(dev, torch.cuda.current_stream(dev), args.steps)}))
        return 0
    g = torch.Generator("cpu").manual_seed(2)
    xs = [torch.randn(SHAPE, generator=g).to(torch.bfloat16).to(dev) for _ in range(5)]
    do = torch.randn(SHAPE, generator=torch.Generator("cpu").manual_seed(3)).to(torch.bfloat16).to(dev)
    q1, q2, k1, k2, v = xs
    beta = torch.tensor(BETA, device=dev)
    lam = torch.tensor(LAM, device=dev)
    stream = torch.cuda.current_stream(dev)

    fwd = lambda: ops.forward(q1, k1, q2, k2, v, beta, lam, POWER, True, 2)  # noqa: E731
    leaves = [x.clone().requires_grad_(True) for x in xs]
    bt = beta.clone().requires_grad_(True)
    lt = lam.clone().requires_grad_(True)

    def step():
        for t in (*leaves, bt, lt):
            t.grad = None
        out = tda_amd.differential_threshold_rela_triton(*leaves, bt, lt, relu_power=POWER, normalize=True)
        out.backward(do)

    # the GPU busy before the first timed region (see settle); the timed regions then follow
    # one another with no idle time, and the per-launch timings (a synchronisation per call) come
    # after them
    settle(step, SETTLE_S)
    # ---- forward only (key_prep, fwd_screen, fwd_pv_cand, fwd_pv per call), events around the calls
    with torch.no_grad():
        fwd_ms = time_calls(stream, fwd, args.steps, args.warmup)

    # ---- forward + backward through the public API (the step)
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

    # ---- each launch of the forward on its own (events between the launches)
    with torch.no_grad():
        fwd_launch_us, fwd_launch_total = time_launches(fwd, args.steps, 2)

    # ---- each launch of the backward on its own: the call autograd makes in the step, on this
    # thread (gradient buffers cleared by the forward, only the non-zero rows stored: repeating
    # the call rewrites the same rows, so the buffers stay valid), and the call that stores every
    # row (no cleared buffers)
    norms, occ = ops.side_buffers(SHAPE, 2, True, dev)
    pairs = ops.pair_buffer(SHAPE, 2, dev)
    gbuf, grads = ops.grad_buffers(q1, k1, q2, k2, v, 2)
    with torch.no_grad():
        ops.forward(q1, k1, q2, k2, v, beta, lam, POWER, True, 2, norms, occ, pairs=pairs, zero=gbuf)
        bwd_launch_us, bwd_launch_total = time_launches(
            lambda: ops.backward(q1, k1, q2, k2, v, do, beta, lam, POWER, True, 2, norms, occ, pairs=pairs,
                                 grads=grads), args.steps, 2)
        full_launch_us, full_launch_total = time_launches(
            lambda: ops.backward(q1, k1, q2, k2, v, do, beta, lam, POWER, True, 2, norms, occ, pairs=pairs),
            args.steps, 2)
    del gbuf, grads

    # ---- skip statistics (untimed)
    st = tile_stats(lambda s: ops.forward(q1, k1, q2, k2, v, beta, lam, POWER, True, 2, stats=s), dev)

    fwd_flop = units(SHAPE, FWD_UNITS)
    fb_flop = units(SHAPE, FWDBWD_UNITS)
    fwd_tf = fwd_flop / (fwd_ms * 1e-3) / 1e12
    fb_ms = max(step_ms, wall_ms)
    fb_tf = fb_flop / (fb_ms * 1e-3) / 1e12
    d = SHAPE[3]
    screen_us = fwd_launch_us[SCREEN_KERNEL]
    screen_alg = units(SHAPE, SCREEN_UNITS)
    screen_tf = screen_alg / (screen_us * 1e-6) / 1e12
    # MFMA work the forward issues: every visited (query tile, key tile, branch) score tile in the
    # screen; the exact pass recomputes at most one score tile and one A.V tile per kept tile
    # (the candidate pass issues fewer: one of each per branch and query tile)
    screen_exec = st["tiles_visited"] * tile_flops(d)
    exact_exec_max = st["tiles_screen_kept"] * 2 * tile_flops(d)
    # fraction of the forward's time the matrix cores would need at their peaks for that work
    # (screen: int8 operations; exact pass: bf16 FLOPs)
    fwd_exec_frac = (screen_exec / (PEAK_I8_TOPS * 1e12) + exact_exec_max / (PEAK_BF16_TFLOPS * 1e12)) / (fwd_ms * 1e-3)
    res = {
        "metric": METRIC,
        "value": fb_tf,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": fb_ms,
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
        "value_kind": "dense-equivalent: 11U causal-dense FLOPs per step, skipped work included",
        "pct_peak": 100.0 * fb_tf / PEAK_BF16_TFLOPS,
        "fwd": {"ms": fwd_ms, "tflops": fwd_tf, "pct_peak": 100.0 * fwd_tf / PEAK_BF16_TFLOPS,
                "kind": "dense-equivalent (3U)", "counted_units": FWD_UNITS,
                "launch_us": {k: round(t, 2) for k, t in fwd_launch_us.items()},
                "launch_sum_us": round(fwd_launch_total, 2),
                "executed_screen_gop": screen_exec / 1e9, "executed_exact_gflop_max": exact_exec_max / 1e9,
                "executed_frac_of_peak_max": fwd_exec_frac,
                "executed_note": "int8 score tiles of every visited tile (screen, at the int8 peak) + at most "
                                 "one bf16 score and one A.V tile per screen-kept tile (exact pass, at the bf16 "
                                 "peak), over the forward's time; from the kernels' tile counters",
                **st},
        "fwd_bwd": {"ms": fb_ms, "event_ms": step_ms, "wall_ms": wall_ms, "tflops": fb_tf,
                    "pct_peak": 100.0 * fb_tf / PEAK_BF16_TFLOPS, "kind": "dense-equivalent (11U)",
                    "counted_units": FWDBWD_UNITS,
                    "bwd_launch_us": {k: round(t, 2) for k, t in bwd_launch_us.items()},
                    "bwd_launch_sum_us": round(bwd_launch_total, 2),
                    "bwd_note": "the step's backward: gradient buffers cleared by its forward (inside fwd_screen), "
                                "only rows a non-zero weight reaches stored",
                    "bwd_all_rows_launch_us": {k: round(t, 2) for k, t in full_launch_us.items()},
                    "bwd_all_rows_launch_sum_us": round(full_launch_total, 2)},
        "reference_equivalent": {
            "note": "FLOPs of two independent TRA calls (4U fwd, 14U fwd+bwd), as the reference executes",
            "fwd_tflops": units(SHAPE, REF_FWD_UNITS) / (fwd_ms * 1e-3) / 1e12,
            "fwd_bwd_tflops": units(SHAPE, REF_FWDBWD_UNITS) / (fb_ms * 1e-3) / 1e12},
        "roofline": {"kernel": SCREEN_KERNEL, "bound": "mfma", "mfma": "v_mfma_i32_32x32x32_i8",
                     "achieved": screen_tf, "peak": PEAK_I8_TOPS, "unit": "TOP/s",
                     "frac": screen_tf / PEAK_I8_TOPS, "traffic": SCREEN_HBM_BYTES,
                     "launch_us": screen_us,
                     "algorithmic": f"2U = {screen_alg:.4e} int8 operations per launch (Q1K1^T and Q2K2^T, "
                                    "causal half)",
                     "bf16_equivalent_frac": screen_tf / PEAK_BF16_TFLOPS,
                     "executed_tops": screen_exec / (screen_us * 1e-6) / 1e12,
                     "executed_gop": screen_exec / 1e9,
                     "timing": "HIP events recorded by the library on the launch stream before and after "
                               "this kernel, averaged over the timed forward calls",
                     "traffic_note": "HBM bytes per fwd_screen launch (rocprofv3 FETCH_SIZE/WRITE_SIZE, "
                                     "copy-calibrated); compulsory: Q1, Q2 (bf16) and the int8 K1, K2 with "
                                     "their scales once = 2.055e8"},
    }
    if SCREEN_HBM_BYTES:
        res["roofline"]["hbm_gbs_at_traffic"] = SCREEN_HBM_BYTES / (screen_us * 1e-6) / 1e9
    if not args.no_side:
        res["side_configs"] = side_configs(max(3, args.steps // 4), 2)
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(args.cpu_budget)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
