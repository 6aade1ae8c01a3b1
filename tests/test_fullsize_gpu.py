"""Parity at the full sizes of the benchmark workloads.

Each test builds the bench's own seeded input (bench.make_input /
bench.make_eval_input, so the tested workload is the timed one), runs the HIP
path once through the C ABI, and checks

  * every column against the CPU oracle, in chunks, with the error-aware
    criterion of test_prox_gpu.parity (rtol 1e-5 for fp32, 1e-12 for fp64,
    plus the reference's own rounding error E), where the oracle finishes in
    seconds; a seeded sample of columns where it does not (the Lambert-map
    entropic projection);
  * size-independent properties on every column, computed independently on
    the GPU in float64: feasibility of the projection (bounds, sums), the
    optimality certificate of the top-k cone/simplex projections, the softmax
    closed form of the entropic projection (hi >= rhs), idempotence;
  * for the evaluation pass, the top-k accuracy counts recomputed exactly from
    the GPU's own scores, the rank loss recomputed from them, and the
    per-example losses of a sample against the oracle on the same scores.
"""
import os

import numpy as np
import pytest

from tests.test_eval_gpu import LONG_DOUBLE, compare_per_example, oracle_objs
from tests.test_prox_gpu import parity

pytestmark = pytest.mark.gpu

F32, F64 = 0, 1
CHUNK = 250_000
THREADS = min(16, os.cpu_count() or 1)  # the GPU box's CPU share


def bench_input(name, cuda):
    import torch
    import bench
    cfg = bench.CONFIGS[name]
    x, col_p = bench.make_input(cfg, torch, cuda)
    return cfg, x, col_p


def run(cfg, x, col_p=None):
    import torch
    import bench
    import libsdca_amd as sd
    out = torch.empty_like(x)
    res = "float" if cfg["result"] == "f32" else "double"
    sd.prox(cfg["op"], x, out=out, result=res, col_p=col_p, **bench.kwargs_of(cfg))
    torch.cuda.synchronize()
    return out


def chunked_parity(oracle, cfg, x, out, col_p=None, chunk=CHUNK, stride=1):
    """Every `stride`-th chunk of `chunk` columns against the oracle."""
    import bench
    res = F32 if cfg["result"] == "f32" else F64
    kw = bench.kwargs_of(cfg)
    n = x.shape[0]
    starts = list(range(0, n, chunk))[::stride]
    for b in starts:
        e = min(n, b + chunk)
        xs = x[b:e].cpu().numpy()
        got = out[b:e].cpu().numpy()
        ckw = dict(kw)
        if col_p is not None:
            ckw["col_p"] = col_p[b:e].cpu().numpy()
        parity(oracle, cfg["op"], xs, got, res, f"{cfg['op']} columns {b}:{e}", THREADS, **ckw)
    return len(starts)


def scale_of(x64):
    return x64.abs().amax(dim=1).clamp_min(1.0)


def test_c2_topk_simplex_full(cuda, oracle):
    """m=100, k=5, rhs=1, fp32, n=4,000,000: every column."""
    import torch
    cfg, x, _ = bench_input("c2", cuda)
    out = run(cfg, x)
    k, rhs, rtol = cfg["k"], cfg["rhs"], 1e-5
    for b in range(0, x.shape[0], 1_000_000):
        a = x[b:b + 1_000_000].double()
        p = out[b:b + 1_000_000].double()
        s = scale_of(a)
        tot = p.sum(dim=1)
        assert (p >= 0).all()
        assert (tot <= rhs + rtol * s).all()
        assert (p <= (tot / k)[:, None] + rtol * s[:, None]).all()
        # Optimality: <r, y - p> <= 0 over the vertices y of the top-k simplex,
        # 0 and (rhs/j) 1_S with |S| = j >= k, whose maximum is
        # max(0, (rhs/k) * sum of the k largest r).
        r = a - p
        lhs = torch.clamp((rhs / k) * r.topk(k, dim=1).values.sum(dim=1), min=0)
        rp = (r * p).sum(dim=1)
        cert_tol = 64 * 100 * 1.2e-7 * s * s
        assert (lhs <= rp + cert_tol).all(), f"certificate fails: {(lhs - rp - cert_tol).max()}"
    chunked_parity(oracle, cfg, x, out)


def test_c2_topk_simplex_idempotent(cuda):
    """The projection of a projected batch is itself, within the fp32
    tolerance 1e-5 (s = max(1, max|p|) = 1 for these columns)."""
    cfg, x, _ = bench_input("c2", cuda)
    p = run(cfg, x)
    q = run(cfg, p)
    err = (q.double() - p.double()).abs().amax()
    assert err <= 1e-5, f"max |P(P(a)) - P(a)| = {err}"


def test_c2_topk_cone_full(cuda, oracle):
    """Top-k cone on the headline input, every column."""
    import torch
    cfg, x, _ = bench_input("c2cone", cuda)
    out = run(cfg, x)
    k, rtol = cfg["k"], 1e-5
    for b in range(0, x.shape[0], 1_000_000):
        a = x[b:b + 1_000_000].double()
        p = out[b:b + 1_000_000].double()
        s = scale_of(a)
        tot = p.sum(dim=1)
        assert (p >= 0).all()
        assert (p <= (tot / k)[:, None] + rtol * s[:, None]).all()
        # The cone's extreme rays are 1_S / |S| with |S| >= k, and p is the
        # projection iff <r, p> = 0 and the k largest r sum to <= 0.
        r = a - p
        cert_tol = 64 * 100 * 1.2e-7 * s * s
        assert (r.topk(k, dim=1).values.sum(dim=1) <= cert_tol).all()
        assert ((r * p).sum(dim=1).abs() <= cert_tol).all()
    chunked_parity(oracle, cfg, x, out)


def test_c1_knapsack_eq_full(cuda, oracle):
    """Simplex projection m=10, n=100,000, fp64: every column, plus sum = 1."""
    cfg, x, _ = bench_input("c1", cuda)
    out = run(cfg, x)
    tot = out.sum(dim=1)
    assert ((tot - 1).abs() <= 1e-12 * 10).all()
    assert ((out >= 0) & (out <= 1)).all()
    chunked_parity(oracle, cfg, x, out)


@pytest.mark.timeout(300)
def test_c3_entropy_full(cuda, oracle):
    """Entropic projection m=1000, n=200,000, fp64, hi = rhs = 1: the exact
    solution is softmax(a) on every column; the oracle on one chunk."""
    import torch
    cfg, x, _ = bench_input("c3", cuda)
    out = run(cfg, x)
    want = torch.softmax(x, dim=1)
    err = (out - want).abs().amax()
    assert err <= 1e-12, f"max |x - softmax(a)| = {err}"
    chunked_parity(oracle, cfg, x, out, chunk=20_000, stride=10)


@pytest.mark.timeout(300)
def test_c3_entropy_norm_full(cuda, oracle):
    """Lambert-map entropic projection m=1000, n=200,000, fp64: feasibility on
    every column, the oracle on a seeded sample of 5,000 columns."""
    import torch
    cfg, x, _ = bench_input("c3norm", cuda)
    out = run(cfg, x)
    tot = out.sum(dim=1)
    assert ((tot - cfg["rhs"]).abs() <= 1e-12 * 1000).all()
    assert ((out >= 0) & (out <= cfg["hi"])).all()
    idx = torch.from_numpy(np.sort(np.random.default_rng(7).choice(x.shape[0], 5000, replace=False))).to(cuda)
    xs = x.index_select(0, idx).cpu().numpy()
    got = out.index_select(0, idx).cpu().numpy()
    parity(oracle, "entropy_norm", xs, got, F64, "entropy_norm sample", THREADS, hi=cfg["hi"],
           rhs=cfg["rhs"])


def test_lambert_full(cuda, oracle):
    """W(exp(x)) on 10,000,000 points x ~ U(-50, 50), fp64: every point."""
    cfg, x, _ = bench_input("lambert", cuda)
    out = run(cfg, x)
    xs = x.cpu().numpy().reshape(-1, 1000)  # elementwise: any (n, m) view of the points
    got = out.cpu().numpy().reshape(-1, 1000)
    want = xs.copy()
    oracle.prox("lambert_w_exp", want, result=F64, nthreads=THREADS)
    rel = np.abs(got - want) / np.maximum(1.0, np.abs(want))
    assert rel.max() <= 1e-12, f"max rel err {rel.max():.3e} at x = {xs.reshape(-1)[rel.argmax()]}"


def test_c5_two_simplex_full(cuda, oracle):
    """Multilabel dual prox: two-block simplex m=200, n=500,000, fp32,
    per-column split p in [1, 5]: every column, plus sum(x_P) = sum(x_N) <= 1."""
    import torch
    cfg, x, col_p = bench_input("c5prox", cuda)
    out = run(cfg, x, col_p)
    o = out.double()
    ar = torch.arange(x.shape[1], device=cuda)[None, :]
    pos = ar < col_p[:, None]
    sp = torch.where(pos, o, 0).sum(dim=1)
    sn = torch.where(pos, 0, o).sum(dim=1)
    s = scale_of(x.double())
    assert (out >= 0).all()
    assert ((sp - sn).abs() <= 1e-5 * s).all()
    assert (sp <= cfg["rhs"] + 1e-5 * s).all()
    chunked_parity(oracle, cfg, x, out, col_p)


@pytest.mark.timeout(300)
def test_c4_eval_full(cuda, oracle):
    """Evaluation pass d=4096, m=1000, n=100,000 (smooth top-5 hinge, softmax
    cross-entropy): accuracy counts exact on every example from the GPU's own
    scores, per-example losses of 5,000 examples against the oracle."""
    import torch
    import bench
    import libsdca_amd as sd
    cfg = bench.CONFIGS["c4"]
    X, W, labels, _ = bench.make_eval_input(cfg, torch, cuda)
    objs = cfg["objs"]
    recs, acc, pe = sd.eval_features(objs, X, W, labels, per_example=True)
    S = sd.scores(X, W)
    torch.cuda.synchronize()
    n, m = S.shape
    sy = S.gather(1, labels[:, None])
    cnt = (S >= sy).sum(dim=1) - 1  # other classes scoring >= the label (ties count against)
    hist = torch.bincount(cnt, minlength=m).cpu().numpy()
    # eval_end in the Result type (float here): partial sums times 1 / n
    want_acc = (np.cumsum(hist).astype(np.float32) * (np.float32(1) / np.float32(n))).astype(np.float64)
    assert np.array_equal(acc, want_acc)
    idx = np.sort(np.random.default_rng(11).choice(n, 5000, replace=False))
    it = torch.from_numpy(idx).to(cuda)
    Ss = S.index_select(0, it).cpu().numpy()
    ys = labels.index_select(0, it).cpu().numpy()
    _, _, o_pe = oracle.eval_scores(oracle_objs(objs), Ss, None, ys, result=F32, per_example=True,
                                    nthreads=THREADS)
    _, _, x_pe = oracle.eval_scores(oracle_objs(objs), Ss, None, ys, result=LONG_DOUBLE,
                                    per_example=True, nthreads=THREADS)
    got = pe.index_select(0, it).cpu().numpy()
    compare_per_example(got[:, :, 0], o_pe[:, :, 0], 1e-5, "c4 primal", exact=x_pe[:, :, 0])
    compare_per_example(got[:, :, 1], o_pe[:, :, 1], 1e-5, "c4 dual", exact=x_pe[:, :, 1])
    # eval_end: primal_loss = coeff * sum (objective_base.h:116-128)
    tot = pe.sum(dim=0).cpu().numpy()
    coeff = [c / g for (_, c, g, _) in objs[:1]] + [objs[1][1]]
    for o in range(len(objs)):
        assert abs(recs[o]["primal_loss"] - coeff[o] * tot[o, 0]) <= 1e-9 * max(1, abs(recs[o]["primal_loss"]))


@pytest.mark.timeout(300)
def test_c4_scores_and_counts_vs_fp64(cuda):
    """C4 end to end against float64 host scores (the count parity of the
    evaluation pass): on a 4,000-example sample, every GPU score lies within
    the fp32 d-term dot-product bound of the float64 product, and each
    example's count #{j != y : s_j >= s_y} (and so its top-1 / top-5 hit)
    from the GPU's scores equals the one from the float64 scores, except on
    examples with a near tie - some |s_j - s_y| (float64) within the two
    scores' rounding bounds - which are listed with both results."""
    import torch
    import bench
    import libsdca_amd as sd
    cfg = bench.CONFIGS["c4"]
    X, W, labels, _ = bench.make_eval_input(cfg, torch, cuda)
    S = sd.scores(X, W)
    torch.cuda.synchronize()
    n, m = S.shape
    d = X.shape[1]
    idx = np.sort(np.random.default_rng(13).choice(n, 4000, replace=False))
    it = torch.from_numpy(idx).to(cuda)
    Xs = X.index_select(0, it).double().cpu().numpy()
    Wh = W.double().cpu().numpy()
    S64 = Xs @ Wh.T
    bound = 4 * np.sqrt(d) * np.finfo(np.float32).eps * (np.abs(Xs) @ np.abs(Wh).T) + 1e-30
    got = S.index_select(0, it).double().cpu().numpy()
    assert (np.abs(got - S64) <= bound).all(), f"max err/bound {(np.abs(got - S64) / bound).max():.2f}"
    y = labels.index_select(0, it).cpu().numpy()
    r = np.arange(len(idx))
    gap = S64 - S64[r, y][:, None]
    near = (np.abs(gap) <= bound + bound[r, y][:, None])
    near[r, y] = False
    near_tie = near.any(axis=1)
    cnt_gpu = (got >= got[r, y][:, None]).sum(axis=1) - 1
    cnt_64 = (S64 >= S64[r, y][:, None]).sum(axis=1) - 1
    differ = cnt_gpu != cnt_64
    assert not (differ & ~near_tie).any(), f"counts differ away from ties: {np.flatnonzero(differ & ~near_tie)[:8]}"
    for k in (1, 5):
        hit_gpu, hit_64 = cnt_gpu < k, cnt_64 < k
        assert not ((hit_gpu != hit_64) & ~near_tie).any(), f"top-{k} differs away from ties"
    print(f"c4 counts vs fp64: {int(near_tie.sum())} near-tie examples of {len(idx)}, "
          f"{int(differ.sum())} with a different count; top-1 {float((cnt_64 < 1).mean()):.4f}, "
          f"top-5 {float((cnt_64 < 5).mean()):.4f} (fp64)")
    for i in np.flatnonzero(near_tie)[:20]:
        print(f"  near tie: example {idx[i]} count gpu {cnt_gpu[i]} fp64 {cnt_64[i]}")


@pytest.mark.timeout(300)
def test_c4_eval_with_duals_full(cuda, oracle):
    """The C4 pass with dual variables A ~ N(0, 0.01^2) (m x n, the A != 0
    variant that exercises the dual losses; seed 3104): per-example primal and
    dual losses of 4,000 examples against the oracle on the GPU's own scores,
    and the dual-loss totals against the per-example sums."""
    import torch
    import bench
    import libsdca_amd as sd
    cfg = bench.CONFIGS["c4"]
    X, W, labels, _ = bench.make_eval_input(cfg, torch, cuda)
    n, m = cfg["n"], cfg["m"]
    g = torch.Generator(device=cuda)
    g.manual_seed(3104)
    A = torch.randn((n, m), generator=g, device=cuda, dtype=torch.float32) * 0.01
    objs = cfg["objs"]
    recs, acc, pe = sd.eval_features(objs, X, W, labels, A=A, per_example=True)
    S = sd.scores(X, W)
    torch.cuda.synchronize()
    idx = np.sort(np.random.default_rng(14).choice(n, 4000, replace=False))
    it = torch.from_numpy(idx).to(cuda)
    Ss = S.index_select(0, it).cpu().numpy()
    As = A.index_select(0, it).cpu().numpy()
    ys = labels.index_select(0, it).cpu().numpy()
    _, _, o_pe = oracle.eval_scores(oracle_objs(objs), Ss, As, ys, result=F32, per_example=True,
                                    nthreads=THREADS)
    _, _, x_pe = oracle.eval_scores(oracle_objs(objs), Ss, As, ys, result=LONG_DOUBLE,
                                    per_example=True, nthreads=THREADS)
    got = pe.index_select(0, it).cpu().numpy()
    compare_per_example(got[:, :, 0], o_pe[:, :, 0], 1e-5, "c4+A primal", exact=x_pe[:, :, 0])
    compare_per_example(got[:, :, 1], o_pe[:, :, 1], 1e-5, "c4+A dual", exact=x_pe[:, :, 1])
    tot = pe.sum(dim=0).cpu().numpy()
    for o in range(len(objs)):
        want = tot[o, 1]
        assert abs(recs[o]["dual_loss"] - want) <= 1e-9 * max(1.0, abs(want)), (o, recs[o]["dual_loss"], want)


@pytest.mark.timeout(300)
def test_c5_eval_full(cuda, oracle):
    """Multilabel evaluation d=1024, m=200, n=500,000: rank loss recomputed on
    every example from the GPU's own scores, per-example losses of 5,000
    examples against the oracle."""
    import torch
    import bench
    import libsdca_amd as sd
    cfg = bench.CONFIGS["c5eval"]
    X, W, labels, offsets = bench.make_eval_input(cfg, torch, cuda)
    objs = cfg["objs"]
    recs, _, pe = sd.eval_features(objs, X, W, labels, offsets=offsets, per_example=True)
    S = sd.scores(X, W)
    torch.cuda.synchronize()
    n, m = S.shape
    npos = offsets[1:] - offsets[:-1]
    row = torch.repeat_interleave(torch.arange(n, device=cuda), npos)
    posmask = torch.zeros((n, m), dtype=torch.bool, device=cuda)
    posmask[row, labels] = True
    slot = torch.arange(labels.numel(), device=cuda) - offsets[:-1][row]
    lab5 = torch.zeros((n, 5), dtype=torch.int64, device=cuda)
    lab5[row, slot] = labels
    rank = torch.zeros(n, dtype=torch.float64, device=cuda)
    for j in range(5):
        valid = j < npos
        sp = S.gather(1, lab5[:, j:j + 1])
        c = ((S >= sp) & ~posmask).sum(dim=1).double()
        rank += torch.where(valid, c, 0.0)
    rank /= (npos * (m - npos)).double()
    want = float(rank.sum()) / n
    # Result is float: the reference forms each example's rank term in float
    # (eval/primal.h:70-79), so the total carries fp32 rounding: rtol 1e-5.
    for r in recs:
        assert abs(r["rank_loss"] - want) <= 1e-5 * max(1.0, want), (r["rank_loss"], want)
    idx = np.sort(np.random.default_rng(12).choice(n, 5000, replace=False))
    off = offsets.cpu().numpy()
    lab = labels.cpu().numpy()
    Ss = S.index_select(0, torch.from_numpy(idx).to(cuda)).cpu().numpy()
    sl = [lab[off[i]:off[i + 1]] for i in idx]
    so = np.concatenate([[0], np.cumsum([len(v) for v in sl])]).astype(np.int64)
    sl = np.concatenate(sl).astype(np.int64)
    _, _, o_pe = oracle.eval_scores(oracle_objs(objs), Ss, None, sl, so, result=F32,
                                    per_example=True, nthreads=THREADS)
    _, _, x_pe = oracle.eval_scores(oracle_objs(objs), Ss, None, sl, so, result=LONG_DOUBLE,
                                    per_example=True, nthreads=THREADS)
    got = pe.index_select(0, torch.from_numpy(idx).to(cuda)).cpu().numpy()
    compare_per_example(got[:, :, 0], o_pe[:, :, 0], 1e-5, "c5 primal", exact=x_pe[:, :, 0])


def test_c2_biased_simplex_full(cuda, oracle):
    """Biased top-k simplex (rho=1) on the C2 input, m=100, n=4,000,000, fp32:
    every column, plus 0 <= x <= sum(x)/k and sum(x) <= rhs."""
    cfg, x, _ = bench_input("c2sbias", cuda)
    out = run(cfg, x)
    o = out.double()
    s = o.sum(dim=1)
    sc = scale_of(x.double())
    assert (out >= 0).all()
    assert (o.amax(dim=1) <= s / cfg["k"] + 1e-5 * sc).all()
    assert (s <= cfg["rhs"] + 1e-5 * sc).all()
    chunked_parity(oracle, cfg, x, out)


def test_c2_biased_cone_full(cuda, oracle):
    """Biased top-k cone (rho=1) on the C2 input: every column, plus
    0 <= x <= sum(x)/k."""
    cfg, x, _ = bench_input("c2cbias", cuda)
    out = run(cfg, x)
    o = out.double()
    sc = scale_of(x.double())
    assert (out >= 0).all()
    assert (o.amax(dim=1) <= o.sum(dim=1) / cfg["k"] + 1e-5 * sc).all()
    chunked_parity(oracle, cfg, x, out)


def test_c1_biased_knapsack_full(cuda, oracle):
    """Biased knapsack_le (rho=1) on the C1 input, m=10, n=100,000, fp64: every
    column, plus lo <= x <= hi and sum(x) <= rhs."""
    cfg, x, _ = bench_input("c1lebias", cuda)
    out = run(cfg, x)
    assert ((out >= cfg["lo"]) & (out <= cfg["hi"])).all()
    assert (out.sum(dim=1) <= cfg["rhs"] + 1e-12 * 10).all()
    chunked_parity(oracle, cfg, x, out)


def test_c5_two_simplex_sort_full(cuda, oracle):
    """Sort-based two-block simplex on the C5 input, m=200, n=500,000, fp32,
    per-column p: every column, plus sum(x_P) = sum(x_N) <= rhs."""
    import torch
    cfg, x, col_p = bench_input("c5sort", cuda)
    out = run(cfg, x, col_p)
    o = out.double()
    ar = torch.arange(x.shape[1], device=cuda)[None, :]
    pos = ar < col_p[:, None]
    sp = torch.where(pos, o, 0).sum(dim=1)
    sn = torch.where(pos, 0, o).sum(dim=1)
    s = scale_of(x.double())
    assert (out >= 0).all()
    assert ((sp - sn).abs() <= 1e-5 * s).all()
    assert (sp <= cfg["rhs"] + 1e-5 * s).all()
    chunked_parity(oracle, cfg, x, out, col_p)


@pytest.mark.timeout(300)
def test_c5_two_entropy_full(cuda, oracle):
    """Two-block entropy (alpha=1) on the C5 input, m=200, n=500,000, fp32,
    per-column p: every column, plus x >= 0 and sum(x) = 1."""
    cfg, x, col_p = bench_input("c5ent", cuda)
    out = run(cfg, x, col_p)
    assert (out >= 0).all()
    assert ((out.double().sum(dim=1) - 1).abs() <= 1e-5 * 200).all()
    chunked_parity(oracle, cfg, x, out, col_p)


@pytest.mark.timeout(300)
def test_c3_biased_entropy_full(cuda, oracle):
    """Biased top-k entropy (k=5, alpha=1) on the C3 input, m=1000, n=200,000,
    fp64: 0 <= x <= sum(x)/k and sum(x) <= 1 on every column; the oracle on a
    seeded sample of 4,000 columns (all settled on this input)."""
    import torch
    from tests.test_prox_gpu import entbias_settled
    cfg, x, _ = bench_input("c3ebias", cuda)
    out = run(cfg, x)
    o = out.double()
    s = o.sum(dim=1)
    assert (out >= 0).all()
    assert (o.amax(dim=1) <= s / cfg["k"] + 1e-12 * 1000).all()
    assert (s <= 1 + 1e-12 * 1000).all()
    idx = torch.from_numpy(np.sort(np.random.default_rng(8).choice(x.shape[0], 4000, replace=False))).to(cuda)
    xs = x.index_select(0, idx).cpu().numpy()
    got = out.index_select(0, idx).cpu().numpy()
    assert entbias_settled(oracle, xs, cfg["alpha"], F64).all()
    parity(oracle, "topk_entropy_biased", xs, got, F64, "topk_entropy_biased sample", THREADS,
           k=cfg["k"], alpha=cfg["alpha"])


@pytest.mark.timeout(300)
def test_c4_kernel_eval_full(cuda, oracle):
    """Kernel-input evaluation n = n_train = 20,000, m=1000, fp32: the top-k
    accuracy recomputed exactly from the GPU's own scores A K_i, the dual
    regularizer against the oracle on those scores, and the per-example
    losses of a 2,000-example sample against the oracle."""
    import torch
    import bench
    import libsdca_amd as sd
    cfg = bench.CONFIGS["c4kernel"]
    K, A, labels, _ = bench.make_eval_input(cfg, torch, cuda)
    objs = cfg["objs"]
    recs, acc, pe = sd.eval_kernel(objs, K, A, labels, per_example=True)
    S = sd.scores(K, A.T.contiguous())
    torch.cuda.synchronize()
    sy = S.gather(1, labels[:, None])
    cnt = (S >= sy).sum(dim=1) - 1  # classes other than the label scoring >= it
    hist = torch.bincount(cnt, minlength=cfg["m"]).cpu().numpy()
    want_acc = (np.cumsum(hist).astype(np.float32) * (np.float32(1) / np.float32(cfg["n"])))
    assert np.array_equal(acc, want_acc.astype(np.float64))
    Sh, Ah = S.cpu().numpy(), A.cpu().numpy()
    preg, dreg = oracle.dual_regularizer(Ah, Sh)
    for r in recs:
        assert abs(r["dual_regularizer"] - dreg) <= 1e-5 * max(1, abs(dreg))
    idx = np.sort(np.random.default_rng(9).choice(cfg["n"], 2000, replace=False))
    lab = labels.cpu().numpy()[idx]
    _, _, o_pe = oracle.eval_scores(oracle_objs(objs), Sh[idx], Ah[idx], lab, per_example=True,
                                    nthreads=THREADS)
    _, _, x_pe = oracle.eval_scores(oracle_objs(objs), Sh[idx], Ah[idx], lab, result=LONG_DOUBLE,
                                    per_example=True, nthreads=THREADS)
    pe = pe.cpu().numpy()[idx]
    compare_per_example(pe[:, :, 0], o_pe[:, :, 0], 1e-5, "kernel eval primal", x_pe[:, :, 0])
    compare_per_example(pe[:, :, 1], o_pe[:, :, 1], 1e-5, "kernel eval dual", x_pe[:, :, 1])


def test_c4_epoch_full(cuda):
    """One SDCA epoch at the bench's c4epoch size (d=4096, m=1000, n=100,000,
    smooth top-5 hinge from W = 0, A = 0) and two size-independent
    properties that any correct epoch keeps:
      * W = A' X exactly in exact arithmetic (every update adds
        x_i (a_new - a_old)'; eval_recompute_primal, eval/core.h:148-182,
        relies on it): 64 classes of W against a float64 product, within
        32 sqrt(n) eps of the classes' largest magnitude, well below one
        example's contribution (about |W| / sqrt(n)), so a missed or doubled
        update shows;
      * the dual constraints of the top-k hinge (l2_hinge_topk.h:44-68): the
        label's variable a_y = -sum of the others' (or at most c), a_y >= 0,
        the others <= 0 and >= -a_y / k (within rounding), on every example."""
    import torch
    import bench
    import libsdca_amd as sd
    cfg = bench.CONFIGS["c4epoch"]
    X, _, labels, _ = bench.make_eval_input(cfg, torch, cuda)
    n, m, d = cfg["n"], cfg["m"], cfg["d"]
    W = torch.zeros((m, d), dtype=torch.float32, device=cuda)
    A = torch.zeros((n, m), dtype=torch.float32, device=cuda)
    sd.epoch_features(cfg["obj"], X, W, A, labels, order=sd.epoch_order(n, 0))
    torch.cuda.synchronize()
    cls = torch.arange(0, m, m // 64, device=cuda)[:64]
    Wref = (A[:, cls].double().T @ X.double())
    eps = float(np.finfo(np.float32).eps)
    err = float((W[cls].double() - Wref).abs().max())
    tol = 8 * np.sqrt(n) * eps * float(Wref.abs().max())
    print(f"epoch W vs A'X: max |W - A'X| {err:.3e}, tol {tol:.3e}, max|W| {float(Wref.abs().max()):.3e}")
    assert err <= tol
    c, k = cfg["obj"][1], cfg["obj"][3]
    A64 = A.double()
    y = labels.long()
    ay = A64.gather(1, y[:, None])[:, 0]
    others = A64.sum(dim=1) - ay
    mask = torch.ones_like(A64, dtype=torch.bool)
    mask[torch.arange(n, device=cuda), y] = False
    tiny = 8 * eps * max(1.0, float(ay.abs().max()))
    assert float(ay.min()) >= -tiny and float(ay.max()) <= c + tiny
    off = A64[mask]
    assert float(off.max()) <= tiny
    # a_y = min(c, sum p) with p = -a_j the projected entries, each p_j at
    # most sum(p) / k; a_y is an fp32 sum of the m - 1 entries, within
    # 4 sqrt(m) ulps of the exact one with a wide margin
    sp = -others
    sum_tol = 4 * np.sqrt(m) * eps * (sp.abs() + eps)
    assert bool(((ay - torch.clamp(sp, max=c)).abs() <= sum_tol + tiny).all())
    assert bool((A64 >= -(sp[:, None] / k) - tiny - sum_tol[:, None]).all())
    assert float(ay.max()) > 0.01
