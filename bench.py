"""Benchmark of the MI355X batched prox / evaluation path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME]

Prints ONE JSON line (stdout).  The default workload is the headline of
batched top-k simplex prox, m=100 rows x n=4,000,000 columns,
k=5, rhs=1, fp32 data and arithmetic, entries N(0,1) with one uniformly drawn
label row per column shifted by +2.  A "step" is one pass of the prox over
the whole batch, out of place (read A, write the result), with the input
already resident in HBM.  Timing: W untimed steps, then K steps bracketed by
torch.cuda.synchronize(); each step is also bracketed by events on the stream
the kernels run on (torch's current stream), which gives the per-launch
duration used for the roofline.

Other workloads (--config): c1 (knapsack_eq f64 m=10 n=1e5), c2cone (top-k
cone on the headline input), c3 (entropy f64 m=1000 n=2e5), c3norm
(entropy_norm f64), lambert (W(exp(x)) f64 on 10M points), c5prox
(two_simplex f32 m=200 n=5e5, per-column p).

cpu_baseline: the reference's own prox loop (oracle/_ref, built from the
reference headers with -O3) - or the oracle restatement when that library is
absent - on a bounded sample of the same input, single-threaded as shipped,
on the host cores of the GPU box.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "prox columns/sec (top-k simplex m=100 k=5 fp32) + % HBM peak; eval ex/s"

CONFIGS = {
    "c2": dict(op="topk_simplex", m=100, n=4_000_000, dtype="f32", result="f32", k=5, rhs=1.0,
               gen="label_shifted", seed=102,
               desc="batched top-k simplex prox, m=100, n=4,000,000, k=5, rhs=1, fp32, "
                    "N(0,1) with the label row +2"),
    "c2cone": dict(op="topk_cone", m=100, n=4_000_000, dtype="f32", result="f32", k=5, rhs=1.0,
                   gen="label_shifted", seed=102,
                   desc="batched top-k cone prox, m=100, n=4,000,000, k=5, fp32, "
                        "N(0,1) with the label row +2"),
    "c1": dict(op="knapsack_eq", m=10, n=100_000, dtype="f64", result="f64", lo=0.0, hi=1.0,
               rhs=1.0, gen="normal", seed=101, rotate=40,
               desc="batched simplex projection (knapsack_eq lo=0 hi=1 rhs=1), m=10, "
                    "n=100,000, fp64, N(0,1)"),
    "c3": dict(op="entropy", m=1000, n=200_000, dtype="f64", result="f64", hi=1.0, rhs=1.0,
               gen="uniform10", seed=103,
               desc="batched entropic projection (exp map), m=1000, n=200,000, fp64, U(-10,10)"),
    "c3norm": dict(op="entropy_norm", m=1000, n=200_000, dtype="f64", result="f64", hi=1.0,
                   rhs=1.0, gen="uniform10", seed=103,
                   desc="batched entropic projection (Lambert W map), m=1000, n=200,000, fp64, "
                        "U(-10,10)"),
    "lambert": dict(op="lambert_w_exp", m=10_000_000, n=1, dtype="f64", result="f64",
                    gen="uniform50", seed=113, rotate=4,
                    desc="elementwise W(exp(x)), 10M points, fp64, U(-50,50)"),
    "c5prox": dict(op="two_simplex", m=200, n=500_000, dtype="f32", result="f32", rhs=1.0,
                   gen="normal", seed=4105, col_p=True,
                   desc="batched two-block simplex prox, m=200, n=500,000, fp32, N(0,1), "
                        "per-column p in [1,5]"),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    return ap.parse_args()


def make_input(cfg, torch, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(cfg["seed"])
    dt = torch.float32 if cfg["dtype"] == "f32" else torch.float64
    n, m = cfg["n"], cfg["m"]
    if cfg["gen"] == "label_shifted":
        x = torch.randn((n, m), generator=g, device=dev, dtype=torch.float32)
        lab = torch.randint(0, m, (n,), generator=g, device=dev)
        x[torch.arange(n, device=dev), lab] += 2.0
        x = x.to(dt)
    elif cfg["gen"] == "normal":
        x = torch.randn((n, m), generator=g, device=dev, dtype=dt)
    elif cfg["gen"] == "uniform10":
        x = torch.rand((n, m), generator=g, device=dev, dtype=dt) * 20 - 10
    elif cfg["gen"] == "uniform50":
        x = torch.rand((n, m), generator=g, device=dev, dtype=dt) * 100 - 50
    else:
        raise ValueError(cfg["gen"])
    col_p = None
    if cfg.get("col_p"):
        col_p = torch.randint(1, 6, (n,), generator=g, device=dev, dtype=torch.int64)
    return x.contiguous(), col_p


def kwargs_of(cfg):
    kw = {}
    for key in ("lo", "hi", "rhs", "k"):
        if key in cfg:
            kw[key] = cfg[key]
    return kw


def cpu_baseline(cfg, x_sample, col_p_sample, seconds):
    """Time the reference (or oracle) prox loop single-threaded on a sample."""
    import numpy as np
    from oracle import binding
    lib = binding.reference()
    kind = "reference"
    if lib is None:
        lib = binding.oracle()
        kind = "port"
    op = cfg["op"]
    res = 0 if cfg["result"] == "f32" else 1
    params = binding.make_params(**kwargs_of(cfg))
    total_cols = 0
    elapsed = 0.0
    if op == "lambert_w_exp":
        unit_count = x_sample.size
    n_avail = x_sample.shape[0]
    # Calibrate on a small slice, then run ~`seconds` of work.
    probe = max(1, min(n_avail, 2000 if op != "lambert_w_exp" else 1))
    work = x_sample[:probe].copy()
    t0 = time.perf_counter()
    lib.prox(op, work, result=res, params=params,
             col_p=None if col_p_sample is None else col_p_sample[:probe])
    dt_probe = time.perf_counter() - t0
    if op == "lambert_w_exp":
        units_per_s = x_sample.size / max(dt_probe, 1e-9)
        return {"value": units_per_s, "unit": "points/s", "cores": 1, "kind": kind,
                "sample": f"{x_sample.size} points of the same input, 1 thread"}
    per_col = dt_probe / probe
    ncols = int(min(n_avail, max(probe, seconds / max(per_col, 1e-12))))
    work = x_sample[:ncols].copy()
    t0 = time.perf_counter()
    lib.prox(op, work, result=res, params=params,
             col_p=None if col_p_sample is None else col_p_sample[:ncols])
    elapsed = time.perf_counter() - t0
    total_cols = ncols
    return {"value": total_cols / elapsed, "unit": "columns/s", "cores": 1, "kind": kind,
            "sample": f"first {total_cols} columns of the same input, 1 thread, {elapsed:.1f} s"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the prox columns and evaluation examples shard across GPUs without exchange; "
              "see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch

    import libsdca_amd as sd

    cfg = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    x, col_p = make_input(cfg, torch, dev)
    rotate = cfg.get("rotate", 1)
    xs = [x] + [x.clone() for _ in range(rotate - 1)]
    out = torch.empty_like(x)
    kw = kwargs_of(cfg)
    res = "float" if cfg["result"] == "f32" else "double"
    stream = torch.cuda.current_stream()

    def step(i):
        sd.prox(cfg["op"], xs[i % rotate], out=out, result=res, col_p=col_p, **kw)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        starts[i].record(stream)
        step(i)
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launch_ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    avg_ms = sum(launch_ms) / len(launch_ms)
    ms_per_step = wall * 1e3 / args.steps

    esz = 4 if cfg["dtype"] == "f32" else 8
    if cfg["op"] == "lambert_w_exp":
        units = cfg["m"] * cfg["n"]
        unit = "points/s"
        bytes_per_unit = 2 * esz
    else:
        units = cfg["n"]
        unit = "columns/s"
        bytes_per_unit = 2 * cfg["m"] * esz + (8 if cfg.get("col_p") else 0)
    value = units / (ms_per_step / 1e3)
    achieved = units * bytes_per_unit / (avg_ms / 1e3) / 1e9

    result = {
        "metric": METRIC,
        "value": value,
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded on the device)",
        "config": {"workload": cfg["desc"], "op": cfg["op"], "m": cfg["m"], "n": cfg["n"],
                   "result": cfg["result"], **kw},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "note": f"algorithmic {bytes_per_unit} B per unit x {units} units per launch "
                             f"/ mean event-timed launch {avg_ms:.4f} ms"},
    }
    if not args.no_cpu:
        import numpy as np
        if cfg["op"] == "lambert_w_exp":
            sample = x.reshape(-1)[:1_000_000].cpu().numpy().reshape(1, -1)
        else:
            sample = x[: min(cfg["n"], 2_000_000)].cpu().numpy()
        cps = None if col_p is None else col_p[: sample.shape[0]].cpu().numpy()
        result["cpu_baseline"] = cpu_baseline(cfg, np.ascontiguousarray(sample), cps,
                                              args.cpu_seconds)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
