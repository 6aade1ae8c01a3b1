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
(two_simplex f32 m=200 n=5e5, per-column p), c4 (evaluation pass d=4096
m=1000 n=1e5: examples/s, roofline on the fp32 MFMA score GEMM), c4f64 (the
same pass in double: roofline on the fp64 MFMA score GEMM), c5eval
(multilabel evaluation d=1024 m=200 n=5e5), c4epoch (one SDCA epoch on the C4
data: examples/s, the reference's own epoch loop as cpu_baseline), c4kepoch
(one SDCA epoch on kernel input, K of n = 20,000 examples, m = 1000).

The default run (c2) also times the whole C4 evaluation pass under the same
clock and nests it as "c4" (examples/s, an MFMA roofline for the score GEMM
and for the whole pass, its own cpu_baseline); --no-c4 skips it.  It nests
one SDCA epoch on the C4 shape as "c4epoch" and one on kernel input as
"c4kepoch" likewise (--no-epoch skips both).

cpu_baseline: the reference's own prox loop (oracle/_ref, built from the
reference headers with -O3) - or the oracle restatement when that library is
absent - on a bounded sample of the same input, single-threaded as shipped,
on the host cores of the GPU box, plus "all_cores": the same loop
harness-parallel over the box's CPU share (16 threads).  For the evaluation
pass: the reference's evaluate_dataset with MKL as its CBLAS.
"""
import argparse
import json
import os
import re
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
               rhs=1.0, gen="normal", seed=101, rotate=40, graph=True,
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
    # The operators next to the path, on the same inputs as above.
    "c2sbias": dict(op="topk_simplex_biased", m=100, n=4_000_000, dtype="f32", result="f32", k=5,
                    rhs=1.0, rho=1.0, gen="label_shifted", seed=102,
                    desc="batched biased top-k simplex prox (rho=1), m=100, n=4,000,000, k=5, "
                         "rhs=1, fp32, N(0,1) with the label row +2"),
    "c2cbias": dict(op="topk_cone_biased", m=100, n=4_000_000, dtype="f32", result="f32", k=5,
                    rho=1.0, gen="label_shifted", seed=102,
                    desc="batched biased top-k cone prox (rho=1), m=100, n=4,000,000, k=5, "
                         "fp32, N(0,1) with the label row +2"),
    "c1lebias": dict(op="knapsack_le_biased", m=10, n=100_000, dtype="f64", result="f64", lo=0.0,
                     hi=1.0, rhs=1.0, rho=1.0, gen="normal", seed=101, rotate=40, graph=True,
                     desc="batched biased knapsack_le prox (lo=0 hi=1 rhs=1 rho=1), m=10, "
                          "n=100,000, fp64, N(0,1)"),
    "c5sort": dict(op="two_simplex_sort", m=200, n=500_000, dtype="f32", result="f32", rhs=1.0,
                   gen="normal", seed=4105, col_p=True,
                   desc="batched two-block simplex prox by sort and scan, m=200, n=500,000, "
                        "fp32, N(0,1), per-column p in [1,5]"),
    "c5ent": dict(op="two_entropy", m=200, n=500_000, dtype="f32", result="f32", alpha=1.0,
                  gen="normal", seed=4105, col_p=True,
                  desc="batched two-block entropic prox (alpha=1), m=200, n=500,000, fp32, "
                       "N(0,1), per-column p in [1,5]"),
    "c3ebias": dict(op="topk_entropy_biased", m=1000, n=200_000, dtype="f64", result="f64", k=5,
                    alpha=1.0, gen="uniform10", seed=103,
                    desc="batched biased top-k entropy prox (k=5, alpha=1), m=1000, n=200,000, "
                         "fp64, U(-10,10)"),
    "c4": dict(op="eval", d=4096, m=1000, n=100_000, dtype="f32", result="f32", seed=104,
               objs=[("l2_hinge_topk_smooth", 1.0, 1.0, 5), ("l2_entropy", 1.0, 1.0, 1)],
               desc="evaluation pass, fp32: X d=4096 x n=100,000 (N(0,1), unit columns), "
                    "W d x m=1000 (N(0,0.01^2)), scores W'X, smooth top-5 hinge (gamma=1) and "
                    "softmax cross-entropy with c=1 (lambda=1/n), top-1/top-5 accuracy"),
    "c4f64": dict(op="eval", d=4096, m=1000, n=100_000, dtype="f64", result="f64", seed=104,
                  objs=[("l2_hinge_topk_smooth", 1.0, 1.0, 5), ("l2_entropy", 1.0, 1.0, 1)],
                  desc="evaluation pass, fp64: the C4 input in double (X d=4096 x n=100,000, "
                       "W d x m=1000), scores W'X on the fp64 matrix cores, smooth top-5 hinge "
                       "(gamma=1) and softmax cross-entropy with c=1, top-1/top-5 accuracy"),
    "c4epoch": dict(op="epoch", d=4096, m=1000, n=100_000, dtype="f32", result="f32", seed=104,
                    obj=("l2_hinge_topk_smooth", 1.0, 1.0, 5), steps=2, warmup=1,
                    desc="one SDCA epoch (update_variables over the reference solver's shuffled "
                         "order), fp32: X d=4096 x n=100,000 (N(0,1), unit columns), m=1000, "
                         "smooth top-5 hinge (gamma=1, c=1), W and A from zero"),
    "c4kepoch": dict(op="epoch", kernel=True, d=4096, m=1000, n=20_000, dtype="f32", result="f32",
                     seed=107, obj=("l2_hinge_topk_smooth", 1.0, 1.0, 5), steps=2, warmup=1,
                     desc="one SDCA epoch on kernel input (the kernel form of update_variables "
                          "over the reference solver's shuffled order), fp32: K = X'X (n = "
                          "20,000 unit-norm N(0,1) features of d = 4096), m=1000, smooth top-5 "
                          "hinge (gamma=1, c=1), A from zero"),
    "c4kernel": dict(op="eval", kernel=True, d=4096, m=1000, n=20_000, dtype="f32", result="f32",
                     seed=106, objs=[("l2_hinge_topk_smooth", 1.0, 1.0, 5), ("l2_entropy", 1.0, 1.0, 1)],
                     desc="kernel-input evaluation pass, fp32: K = X'X (n = n_train = 20,000 "
                          "unit-norm N(0,1) features of d = 4096), dual variables A m=1000 x n "
                          "(N(0,0.01^2)), scores A K_i, smooth top-5 hinge (gamma=1) and softmax "
                          "cross-entropy with c=1, top-1/top-5 accuracy, dual regularizer"),
    "c5eval": dict(op="eval", d=1024, m=200, n=500_000, dtype="f32", result="f32", seed=105,
                   multilabel=True,
                   objs=[("l2_multilabel_hinge_smooth", 1.0, 1.0, 1),
                         ("l2_multilabel_entropy", 1.0, 1.0, 1)],
                   desc="multilabel evaluation pass, fp32: d=1024, m=200, n=500,000, 1-5 "
                        "positive labels per example, smooth multilabel hinge and multilabel "
                        "cross-entropy with c=1, rank loss"),
}
# Nested in the default (c2) run: the other configurations of the path.
NESTED_PROX = ("c1", "c3", "c3norm", "lambert", "c5prox")
NESTED_EVAL = ("c5eval",)
EPOCH_KEYS = ("value", "unit", "ms_per_step", "steps", "warmup", "dtype", "config", "roofline",
              "note", "cpu_baseline")
PROX_KEYS = ("value", "unit", "ms_per_step", "steps", "warmup", "dtype", "config", "roofline",
             "launch_floor", "cpu_baseline")
EVAL_KEYS = ("value", "unit", "ms_per_step", "steps", "warmup", "dtype", "config", "roofline",
             "roofline_pass", "eval", "cpu_baseline")
# Operators whose step is two launches: the column kernel and the kernel
# that finishes the columns it deferred (an empty list for most inputs).
LISTED_OPS = ("topk_simplex", "topk_cone", "topk_simplex_biased", "topk_cone_biased",
              "knapsack_le_biased", "two_simplex_sort")
MFMA_F32_PEAK_TFLOPS = 157.3
MFMA_F64_PEAK_TFLOPS = 78.6
CPU_THREADS = min(16, os.cpu_count() or 1)  # the GPU box's CPU share


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # Defaults 20 and 50 (the epoch configuration: 2 and 1).  50 untimed
    # steps (about 30 ms of C2 work): the clocks settle; after 5 the first
    # timed steps still ran ~5 % slow.
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-c4", action="store_true",
                    help="default run: skip the nested C4 evaluation-pass measurement")
    ap.add_argument("--no-epoch", action="store_true",
                    help="default run: skip the nested SDCA epoch measurement")
    ap.add_argument("--trace-steps", action="store_true",
                    help="also record an event after every timed step and print the per-step "
                         "durations (per_step_ms)")
    ap.add_argument("--no-nested", action="store_true",
                    help="default run: skip the nested c1, c3, c3norm, lambert, c5prox and "
                         "c5eval measurements")
    ap.add_argument("--nested-steps", type=int, default=20)
    ap.add_argument("--nested-warmup", type=int, default=20)
    ap.add_argument("--nested-cpu-seconds", type=float, default=3.0)
    ap.add_argument("--epoch-steps", type=int, default=2)
    ap.add_argument("--epoch-warmup", type=int, default=1)
    ap.add_argument("--c4-steps", type=int, default=10)
    # GPU clocks keep rising over the first few dozen passes of 8 ms.
    ap.add_argument("--c4-warmup", type=int, default=15)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="time a plain device copy of the headline input's size instead "
                         "(the reference kernel for scaling FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


def traffic_of(config):
    """HBM bytes per launch of the config's dominant kernel, from the rocprofv3
    FETCH_SIZE / WRITE_SIZE passes summarised in profiles/hbm_traffic.md (each
    counter scaled by what it reads for a plain copy of known size); None when
    that workload has not been profiled."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        m = re.match(r"^- (\w+): traffic ([0-9.eE+]+) B per launch", line)
        if m and m.group(1) == config:
            return float(m.group(2))
    return None


def copy_calibration(args, torch):
    """A device-to-device copy of the headline input (n x m fp32), timed like a
    prox step: the known-size kernel that calibrates the HBM byte counters."""
    cfg = CONFIGS["c2"]
    dev = torch.device("cuda:0")
    x = torch.empty((cfg["n"], cfg["m"]), dtype=torch.float32, device=dev).normal_()
    out = torch.empty_like(x)
    for _ in range(args.warmup):
        out.copy_(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out.copy_(x)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    nbytes = x.numel() * x.element_size()
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes,
                      "ms_per_copy": dt * 1e3, "GB/s": 2 * nbytes / dt / 1e9}))


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


def units_of(cfg):
    """(units per step, unit name, algorithmic HBM bytes per unit): one read
    and one write of each column (+ its int64 split point), or of each
    point for the elementwise map."""
    esz = 4 if cfg["dtype"] == "f32" else 8
    if cfg["op"] == "lambert_w_exp":
        return cfg["m"] * cfg["n"], "points/s", 2 * esz
    return cfg["n"], "columns/s", 2 * cfg["m"] * esz + (8 if cfg.get("col_p") else 0)


def units_bytes(cfg):
    units, _, per = units_of(cfg)
    return units * per


def kwargs_of(cfg):
    kw = {}
    for key in ("lo", "hi", "rhs", "rho", "alpha", "k"):
        if key in cfg:
            kw[key] = cfg[key]
    return kw


def cpu_baseline(cfg, x_sample, col_p_sample, seconds):
    """Time the reference's (or the oracle's) prox loop single-threaded on a
    sample of the same input: a first slice sized to ~`seconds` of work, run
    again until that much time has been measured."""
    from oracle import binding
    lib = binding.reference()
    kind = "reference"
    if lib is None:
        lib = binding.oracle()
        kind = "port"
    op = cfg["op"]
    res = 0 if cfg["result"] == "f32" else 1
    params = binding.make_params(**kwargs_of(cfg))
    n_avail = x_sample.shape[0]

    def timed(ncols):
        work = x_sample[:ncols].copy()
        cp = None if col_p_sample is None else col_p_sample[:ncols]
        t0 = time.perf_counter()
        lib.prox(op, work, result=res, params=params, col_p=cp)
        return time.perf_counter() - t0

    def timed_par(ncols):
        work = x_sample[:ncols].copy()
        cp = None if col_p_sample is None else col_p_sample[:ncols]
        t0 = time.perf_counter()
        lib.prox(op, work, result=res, params=params, col_p=cp, nthreads=CPU_THREADS)
        return time.perf_counter() - t0

    probe = max(1, min(n_avail, 2000))
    per_col = timed(probe) / probe
    ncols = int(min(n_avail, max(probe, seconds / max(per_col, 1e-12))))
    elapsed, passes = 0.0, 0
    while elapsed < 0.8 * seconds and passes < 200:
        elapsed += timed(ncols)
        passes += 1
    # harness-parallel: columns split over the host cores (the reference's
    # functions are re-entrant; each thread has its own aux), the same
    # columns per thread as the single-thread sample where the input allows
    npar = int(min(n_avail, ncols * CPU_THREADS))
    elapsed_p, passes_p = 0.0, 0
    while elapsed_p < 0.5 * seconds and passes_p < 200:
        elapsed_p += timed_par(npar)
        passes_p += 1
    if op == "lambert_w_exp":  # rows of the sample are runs of points
        per, unit, what = x_sample.shape[1], "points/s", f"runs of {x_sample.shape[1]} points"
    else:
        per, unit, what = 1, "columns/s", "columns"
    return {"value": ncols * per * passes / elapsed, "unit": unit, "cores": 1, "kind": kind,
            "sample": f"first {ncols} {what} of the same input x {passes} passes, 1 thread, "
                      f"{elapsed:.1f} s",
            "all_cores": {"value": npar * per * passes_p / elapsed_p, "unit": unit,
                          "cores": CPU_THREADS,
                          "sample": f"first {npar} {what} x {passes_p} passes over "
                                    f"{CPU_THREADS} threads, {elapsed_p:.1f} s, harness-parallel"}}


def make_eval_input(cfg, torch, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(cfg["seed"])
    n, m, d = cfg["n"], cfg["m"], cfg["d"]
    X = torch.randn((n, d), generator=g, device=dev, dtype=torch.float32)
    X /= X.norm(dim=1, keepdim=True)
    if cfg.get("kernel"):
        # Kernel input: the Gram matrix of the features (n x n, symmetric) and
        # dual variables A (rows are the reference's columns).
        K = (X @ X.T).contiguous()
        del X
        A = torch.randn((n, m), generator=g, device=dev, dtype=torch.float32) * 0.01
        labels = torch.randint(0, m, (n,), generator=g, device=dev)
        return K, A, labels, None
    W = torch.randn((m, d), generator=g, device=dev, dtype=torch.float32) * 0.01
    if cfg.get("multilabel"):
        # 1-5 distinct sorted labels per example, drawn uniformly without replacement.
        p = torch.randint(1, 6, (n,), generator=g, device=dev)
        keys = torch.rand((n, m), generator=g, device=dev)
        order = keys.argsort(dim=1)[:, :5]
        ar = torch.arange(5, device=dev)[None, :]
        chosen = torch.where(ar < p[:, None], order, torch.full_like(order, m))
        chosen, _ = chosen.sort(dim=1)
        labels = chosen[chosen < m].contiguous()
        offsets = torch.zeros(n + 1, dtype=torch.int64, device=dev)
        offsets[1:] = torch.cumsum(p, 0)
        return X, W, labels, offsets
    labels = torch.randint(0, m, (n,), generator=g, device=dev)
    if cfg["dtype"] == "f64":  # the same values in double
        X, W = X.double(), W.double()
    return X, W, labels, None


def bench_eval(cfg, args, torch, sd, steps=None, warmup=None, config_name=None,
               cpu_seconds=None):
    """Times the evaluation pass of `cfg`; returns the result dict."""
    cpu_seconds = args.cpu_seconds if cpu_seconds is None else cpu_seconds
    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    config_name = args.config if config_name is None else config_name
    dev = torch.device("cuda:0")
    X, W, labels, offsets = make_eval_input(cfg, torch, dev)
    objs = cfg["objs"]
    stream = torch.cuda.current_stream()

    kernel = bool(cfg.get("kernel"))

    def step(fused=False):
        if kernel:  # X = K (n x n_train), W = A (n_train x m)
            return sd.eval_kernel(objs, X, W, labels, offsets=offsets)
        return sd.eval_features(objs, X, W, labels, offsets=offsets, fused=fused)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        recs, acc, _ = step()  # each call ends with a host synchronisation
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / steps
    # The fused form of the same pass (scores and epilogue in one kernel,
    # scores not stored; SDCA_EVAL_FUSED), timed the same way after the
    # measured steps where it applies: the default two-kernel form is the
    # faster on MI355X.  Its records must equal the two-kernel form's to the
    # rounding of the scores (bit for bit below 2^32 multiply-adds or 512
    # classes, where both take the scores from the same MFMA sequence;
    # above, the two-kernel form's come from hipBLASLt).
    fused_ms = None
    if not kernel and not cfg.get("multilabel") and cfg["dtype"] == "f32":
        step(fused=True)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(steps):
            recs_f, _, _ = step(fused=True)
        torch.cuda.synchronize()
        fused_ms = (time.perf_counter() - t1) * 1e3 / steps
        for a, b in zip(recs_f, recs):
            for key in a:
                x, y = float(a[key]), float(b[key])
                if abs(x - y) > 1e-5 * max(1.0, abs(y)):
                    raise RuntimeError(f"fused and two-kernel evaluation records differ: {key} "
                                       f"{x!r} against {y!r}")
    # The dominant kernel is the score GEMM: time it on its own, event-timed
    # on the stream it runs on.
    S = torch.empty((cfg["n"], cfg["m"]), dtype=X.dtype, device=dev)
    Wg = W.T.contiguous() if kernel else W   # the GEMM's W operand: A' for kernel input
    for _ in range(5):
        sd.scores(X, Wg, out=S)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        sd.scores(X, Wg, out=S)
    e1.record(stream)
    torch.cuda.synchronize()
    gemm_ms = e0.elapsed_time(e1) / steps
    inner = cfg["n"] if kernel else cfg["d"]  # contraction length: n_train or d
    flops = 2.0 * cfg["n"] * cfg["m"] * inner
    achieved = flops / (gemm_ms / 1e3) / 1e12
    achieved_pass = flops / (ms_per_step / 1e3) / 1e12
    peak = MFMA_F64_PEAK_TFLOPS if cfg["dtype"] == "f64" else MFMA_F32_PEAK_TFLOPS
    value = cfg["n"] / (ms_per_step / 1e3)
    extra = {"records": recs, "fused_form_ms_per_step": fused_ms}
    if not cfg.get("multilabel"):
        extra["top1"] = float(acc[0])
        extra["top5"] = float(acc[4])
    result = {
        "metric": METRIC,
        "value": value,
        "unit": "examples/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded on the device)",
        "config": {"workload": cfg["desc"], "d": cfg["d"], "m": cfg["m"], "n": cfg["n"],
                   "input": "kernel" if kernel else "features",
                   "objectives": [o[0] for o in objs]},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": peak,
                     "unit": "TFLOP/s", "frac": achieved / peak,
                     "traffic": traffic_of(config_name),
                     "note": f"score GEMM 2 n m {'n_train' if kernel else 'd'} = {flops:.3e} "
                             f"flop / mean event-timed launch "
                             f"{gemm_ms:.3f} ms; full pass {ms_per_step:.3f} ms"},
        "roofline_pass": {"bound": "mfma", "achieved": achieved_pass,
                          "peak": peak, "unit": "TFLOP/s",
                          "frac": achieved_pass / peak,
                          "note": "the same flops over the whole pass (GEMM, epilogue, "
                                  "reductions, records) on the host clock"},
        "eval": extra,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_eval(cfg, X, W, labels, offsets, cpu_seconds,
                                                   kernel)
    return result


def bench_epoch(cfg, args, torch, sd, steps=None, warmup=None):
    """Times SDCA epochs (sdca_epoch_features) over the reference solver's
    orders: `warmup` untimed epochs from W = 0, A = 0, then `steps` timed ones
    (each call ends with a host synchronisation); value = examples per second."""
    import numpy as np
    if steps is None:
        steps = cfg["steps"] if args.steps is None else args.steps
    if warmup is None:
        warmup = cfg["warmup"] if args.warmup is None else args.warmup
    dev = torch.device("cuda:0")
    kernel = bool(cfg.get("kernel"))
    X, _, labels, _ = make_eval_input(cfg, torch, dev)  # X = K (n x n) for kernel input
    n, m, d = cfg["n"], cfg["m"], cfg["d"]
    A = torch.zeros((n, m), dtype=torch.float32, device=dev)
    if kernel:
        W = norms = None
    else:
        W = torch.zeros((m, d), dtype=torch.float32, device=dev)
        norms = (X * X).sum(dim=1).contiguous()
    orders = [torch.from_numpy(sd.epoch_order(n, e)).to(dev) for e in range(warmup + steps)]
    res = "float" if cfg["result"] == "f32" else "double"

    def epoch(e):
        if kernel:
            sd.epoch_kernel(cfg["obj"], X, A, labels, order=orders[e], result=res)
        else:
            sd.epoch_features(cfg["obj"], X, W, A, labels, order=orders[e], norms=norms,
                              result=res)

    for e in range(warmup):
        epoch(e)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e in range(warmup, warmup + steps):
        epoch(e)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    if kernel:
        recs, _, _ = sd.eval_kernel([cfg["obj"]], X, A, labels, result="double")
    else:
        recs, _, _ = sd.eval_features([cfg["obj"]], X, W, labels, A=A, result="double")
    r = recs[0]
    gap = (r["primal"] - r["dual"]) / max(abs(r["primal"]), abs(r["dual"]))
    result = {
        "metric": "SDCA epoch examples/s", "value": n / (ms / 1e3), "unit": "examples/s",
        "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": cfg["dtype"], "data": "synthetic (seeded on the device)",
        "config": {"workload": cfg["desc"], "d": d, "m": m, "n": n,
                   "input": "kernel" if kernel else "features", "objective": list(cfg["obj"])},
        "roofline": None,
        "note": "latency-bound: the dual updates run in order in one workgroup per block of "
                "32 examples (profiles/ has the per-kernel split); relative duality gap after "
                f"{warmup + steps} epochs: {gap:.4g}",
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_epoch(cfg, X, labels, sd, args.cpu_seconds)
    return result


def cpu_baseline_epoch(cfg, X, labels, sd, seconds):
    """The reference's own epoch loop (sdca::update_variables, oracle/_ref with
    MKL) from W = 0, A = 0 over the first examples of epoch 0's order, one
    thread as shipped (the loop is sequential)."""
    import numpy as np
    from oracle import binding
    ref = binding.reference()
    if ref is None:
        return None
    oname = {"l2_hinge_topk_smooth": "hinge_topk_smooth"}
    obj = (oname[cfg["obj"][0]],) + tuple(cfg["obj"][1:])
    n, m, d = cfg["n"], cfg["m"], cfg["d"]
    kernel = bool(cfg.get("kernel"))
    Xh = X.cpu().numpy()  # K for kernel input
    lab = labels.cpu().numpy()
    order = sd.epoch_order(n, 0)
    res = 0 if cfg["result"] == "f32" else 1

    def run(count):
        A = np.zeros((n, m), np.float32)
        t0 = time.perf_counter()
        if kernel:
            ref.epoch_kernel(obj, Xh, A, lab, order[:count], result=res)
        else:
            W = np.zeros((m, d), np.float32)
            ref.epoch_features(obj, Xh, W, A, lab, order[:count], result=res)
        return time.perf_counter() - t0

    count = 64
    t = run(count)
    count = max(64, min(n, int(count * seconds / max(t, 1e-3))))
    t = run(count)
    return {"value": count / t, "unit": "examples/s", "cores": 1, "kind": "reference",
            "sample": f"the first {count} examples of epoch 0's order from "
                      f"{'A = 0' if kernel else 'W = 0, A = 0'}, 1 thread ({t:.1f} s): the "
                      f"reference's update_variables ({'kernel' if kernel else 'feature'} "
                      "input) with MKL"}


def cpu_baseline_eval(cfg, X, W, labels, offsets, seconds, kernel=False):
    """The reference's evaluate_dataset (solver/eval.h:15-51, oracle/_ref:
    the reference headers with Intel MKL as their CBLAS) on a bounded sample
    of the same examples: one thread as shipped, and harness-parallel over
    the host cores (examples split over threads, records merged).  Kernel
    input, or a box without the reference build, falls back to the oracle's
    restatement (gemv loop plus epilogue, kind "port")."""
    import numpy as np
    from oracle import binding
    oname = {"l2_hinge_topk_smooth": "hinge_topk_smooth", "l2_entropy": "entropy",
             "l2_multilabel_hinge_smooth": "multilabel_hinge_smooth",
             "l2_multilabel_entropy": "multilabel_entropy"}
    objs = [(oname[o[0]], o[1], o[2], o[3]) for o in cfg["objs"]]
    lab = labels.cpu().numpy()
    off = None if offsets is None else offsets.cpu().numpy()
    ref = None if kernel else binding.reference()
    if ref is not None:
        Wh = W.cpu().numpy()

        def run(ne, nthreads):
            Xs = X[:ne].cpu().numpy()
            A = np.zeros((ne, cfg["m"]), dtype=Xs.dtype)  # cold start: A = 0
            ls = lab[:ne] if off is None else lab[: off[ne]]
            os_ = None if off is None else off[: ne + 1]
            t0 = time.perf_counter()
            ref.evaluate_dataset(objs, Xs, Wh, A, ls, os_, nthreads=nthreads)
            return time.perf_counter() - t0
        kind = "reference"
        what = (f"the reference's evaluate_dataset (MKL {'d' if cfg['dtype'] == 'f64' else 's'}"
                "gemv scores), all objectives")
    else:
        lib = binding.oracle()
        Wh = np.ascontiguousarray(W.T.cpu().numpy()) if kernel else W.cpu().numpy()
        Ah = W.cpu().numpy() if kernel else None

        def run(ne, nthreads):
            Xs = X[:ne].cpu().numpy()
            t0 = time.perf_counter()
            S = lib.scores(Xs, Wh, nthreads=nthreads)
            if kernel:
                lib.dual_regularizer(Ah[:ne], S)
                lib.eval_scores(objs, S, Ah[:ne], lab[:ne], nthreads=nthreads)
            elif off is None:
                lib.eval_scores(objs, S, None, lab[:ne], nthreads=nthreads)
            else:
                lib.eval_scores(objs, S, None, lab[: off[ne]], off[: ne + 1], nthreads=nthreads)
            return time.perf_counter() - t0
        kind = "port"
        what = "the oracle's restated gemv loop and epilogue"

    probe = 200
    dt = run(probe, 1)
    ne = int(min(cfg["n"], max(probe, seconds / max(dt / probe, 1e-9))))
    dt = run(ne, 1)
    # harness-parallel: the same work per thread as the single-thread sample
    nep = int(min(cfg["n"], ne * CPU_THREADS))
    dtp = run(nep, CPU_THREADS)
    return {"value": ne / dt, "unit": "examples/s", "cores": 1, "kind": kind,
            "sample": f"first {ne} examples, 1 thread ({dt:.1f} s): {what}",
            "all_cores": {"value": nep / dtp, "unit": "examples/s", "cores": CPU_THREADS,
                          "sample": f"first {nep} examples over {CPU_THREADS} threads "
                                    f"({dtp:.1f} s), harness-parallel"}}


def bench_prox(cfg, args, torch, sd, steps, warmup, config_name, cpu_seconds):
    """Times the batched prox of `cfg` (W untimed steps, then K steps timed on
    the host clock and by one event pair on the kernels' stream); returns the
    result dict, with the cpu_baseline unless --no-cpu."""
    dev = torch.device("cuda:0")
    x, col_p = make_input(cfg, torch, dev)
    rotate = cfg.get("rotate", 1)
    xs = [x] + [x.clone() for _ in range(rotate - 1)]
    out = torch.empty_like(x)
    kw = kwargs_of(cfg)
    res = "float" if cfg["result"] == "f32" else "double"
    stream = torch.cuda.current_stream()

    if col_p is not None:  # validated once here, not inside the timed steps
        assert 1 <= int(col_p.min()) and int(col_p.max()) <= cfg["m"] - 1

    def step(i):
        sd.prox(cfg["op"], xs[i % rotate], out=out, result=res, col_p=col_p, check_col_p=False,
                **kw)

    graph = bool(cfg.get("graph"))
    if graph:
        # Launch-bound workload (a step is a few microseconds of GPU work):
        # the K timed steps are captured once into a HIP graph on a side
        # stream, warmed up first so that the library's per-stream workspace
        # exists before the capture, and replayed as one launch.
        gs = torch.cuda.Stream()
        with torch.cuda.stream(gs):
            for i in range(warmup):
                step(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=gs):
            for i in range(steps):
                step(i)
        torch.cuda.synchronize()
        g.replay()  # untimed
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record(stream)
        g.replay()
        end.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        avg_ms = start.elapsed_time(end) / steps
        # The launch floor of that graph: per step, as many launches of a
        # kernel with no work (a one-element fill) as the step makes (one
        # column kernel, plus the deferred-column kernel for the listed
        # operators), captured and replayed the same way.
        launches = 2 if cfg["op"] in LISTED_OPS else 1
        tiny = torch.zeros(1, device=dev)
        gf = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gf, stream=gs):
            for i in range(steps * launches):
                tiny.fill_(float(i & 1))
        torch.cuda.synchronize()
        gf.replay()  # untimed
        torch.cuda.synchronize()
        f0, f1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        f0.record(stream)
        gf.replay()
        f1.record(stream)
        torch.cuda.synchronize()
        floor_ms = f0.elapsed_time(f1) / steps
        floor = {"ms_per_step": floor_ms, "launches_per_step": launches,
                 "frac_at_floor": units_bytes(cfg) / (floor_ms / 1e3) / 1e9 / HBM_PEAK_GBS,
                 "note": "the same K-step graph with each launch replaced by a one-element "
                         "fill kernel: the step time no kernel of this launch count goes "
                         "below, and the HBM fraction the workload would reach at it"}
    else:
        for i in range(warmup):
            step(i)
        torch.cuda.synchronize()
        # One pair of events on the kernels' stream brackets the K timed
        # steps: the mean launch duration is their span / K.  (An event pair
        # per step adds its own stream packets between the steps: about 30 us
        # of the 0.55 ms C2 step.)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        # --trace-steps: an event after every step as well, for the per-step
        # durations (the transient after a cold start); the mean stays the
        # span of the K steps / K.
        marks = ([torch.cuda.Event(enable_timing=True) for _ in range(steps)]
                 if args.trace_steps else None)
        t0 = time.perf_counter()
        start.record(stream)
        for i in range(steps):
            step(i)
            if marks:
                marks[i].record(stream)
        end.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        avg_ms = start.elapsed_time(end) / steps
        if marks:
            per_step = [start.elapsed_time(marks[0])] + [
                marks[i - 1].elapsed_time(marks[i]) for i in range(1, steps)]
    ms_per_step = wall * 1e3 / steps

    units, unit, bytes_per_unit = units_of(cfg)
    value = units / (ms_per_step / 1e3)
    achieved = units * bytes_per_unit / (avg_ms / 1e3) / 1e9

    result = {
        "metric": METRIC,
        "value": value,
        "unit": unit,
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded on the device)",
        "config": {"workload": cfg["desc"], "op": cfg["op"], "m": cfg["m"], "n": cfg["n"],
                   "result": cfg["result"], **kw, **({"hip_graph": True} if graph else {})},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic_of(config_name),
                     "note": f"algorithmic {bytes_per_unit} B per unit x {units} units per launch "
                             f"/ mean launch {avg_ms:.4f} ms (HIP events on the kernels' stream "
                             f"around the {steps} timed steps; a step is the column kernel"
                             + (" and the deferred-column kernel)" if cfg["op"] in LISTED_OPS
                                else ")")
                             + (" (the K steps replayed from one captured HIP graph)" if graph else "")},
    }
    if graph:
        result["launch_floor"] = floor
    if not graph and args.trace_steps:
        result["per_step_ms"] = [round(v, 4) for v in per_step]
    if not args.no_cpu:
        import numpy as np
        if cfg["op"] == "lambert_w_exp":
            # 64 runs of 62,500 points: split over the threads for all_cores
            sample = x.reshape(-1)[:4_000_000].cpu().numpy().reshape(64, -1)
        else:
            sample = x[: min(cfg["n"], 4_000_000)].cpu().numpy()
        cps = None if col_p is None else col_p[: sample.shape[0]].cpu().numpy()
        result["cpu_baseline"] = cpu_baseline(cfg, np.ascontiguousarray(sample), cps,
                                              cpu_seconds)
        del sample
    return result


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(prox columns and evaluation examples shard across GPUs with no exchange "
              "other than a final sum of the evaluation records)", file=sys.stderr)
        sys.exit(2)
    import torch

    import libsdca_amd as sd

    cfg = CONFIGS[args.config]
    if cfg["op"] == "epoch" and not args.copy_calibration:
        print(json.dumps(bench_epoch(cfg, args, torch, sd)))
        return
    # The epoch has its own defaults; every other workload takes 20 / 50.
    args.steps = 20 if args.steps is None else args.steps
    args.warmup = 50 if args.warmup is None else args.warmup
    if args.copy_calibration:
        copy_calibration(args, torch)
        return
    if cfg["op"] == "eval":
        print(json.dumps(bench_eval(cfg, args, torch, sd)))
        return
    result = bench_prox(cfg, args, torch, sd, args.steps, args.warmup, args.config,
                        args.cpu_seconds)
    if args.config == "c2" and not args.no_c4:
        # The second north-star workload under the same clock: the whole C4
        # evaluation pass, nested (the headline value stays the prox's).
        torch.cuda.empty_cache()
        ev = bench_eval(CONFIGS["c4"], args, torch, sd, steps=args.c4_steps,
                        warmup=args.c4_warmup, config_name="c4")
        result["c4"] = {key: ev[key] for key in EVAL_KEYS if key in ev}
    if args.config == "c2" and not args.no_nested:
        # The other configurations of the path, each under the same clock with
        # its own roofline and a shorter cpu_baseline sample.
        for name in NESTED_PROX:
            torch.cuda.empty_cache()
            r = bench_prox(CONFIGS[name], args, torch, sd, args.nested_steps,
                           args.nested_warmup, name, args.nested_cpu_seconds)
            result[name] = {key: r[key] for key in PROX_KEYS if key in r}
        for name in NESTED_EVAL:
            torch.cuda.empty_cache()
            ev = bench_eval(CONFIGS[name], args, torch, sd, steps=args.c4_steps,
                            warmup=args.c4_warmup, config_name=name,
                            cpu_seconds=args.nested_cpu_seconds)
            result[name] = {key: ev[key] for key in EVAL_KEYS if key in ev}
    if args.config == "c2" and not args.no_epoch:
        # The epoch row (the solver's inner loop over the prox operators) on
        # the C4 shape, nested likewise, with its own step counts.
        torch.cuda.empty_cache()
        ep = bench_epoch(CONFIGS["c4epoch"], args, torch, sd, steps=args.epoch_steps,
                         warmup=args.epoch_warmup)
        result["c4epoch"] = {key: ep[key] for key in EPOCH_KEYS if key in ep}
        torch.cuda.empty_cache()
        ep = bench_epoch(CONFIGS["c4kepoch"], args, torch, sd, steps=args.epoch_steps,
                         warmup=args.epoch_warmup)
        result["c4kepoch"] = {key: ep[key] for key in EPOCH_KEYS if key in ep}
    print(json.dumps(result))


if __name__ == "__main__":
    main()
