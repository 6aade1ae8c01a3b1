"""GPU record sets and branches (sdca_prox_with_sets) against the oracle.

Each case runs libsdca_amd.prox(..., thresholds=True, sets=True) and the
oracle's oracle_prox_sets (whose sets equal the reference's first / last
exactly and whose branch tags are pinned in tests/test_prox_sets_oracle.py)
on the same input, and requires, record by record:
  * the same branch;
  * the same (n_hi, n_mid) where the branch fixes them by construction (the
    k largest at hi, the zero record, the top-k entropy's U, the records of
    the biased top-k entropy and the two-block entropy);
  * otherwise the same sets up to the entries tied with the record's cuts:
    |dn_hi| at most the number of entries within the band of the hi cut
    (t + hi; t + log hi for the exp map, t + hi + log hi for the Lambert
    map), |d(n_hi + n_mid)| at most the number within the band of the lo cut
    (t + lo), where the band is the two records' difference plus 64 ulps of
    the column's scale (the reference's own epsilon tests are 16 ulps).
    Most such records are the degenerate ones where every entry is at a
    bound: any t of an interval gives the projection, the reference's
    iteration ends at an end of it (an entry exactly on its cut, counted
    free) and the GPU takes another point (the entry at hi), so the count
    moves by the entries on the cut.
The kernels' paths are covered: the register kernels (m = 37, 100, 200),
the deferred sorted-column list (the top-k cone's U, the biased searches),
the workgroup-per-column kernels (m = 3000, k > 8), the streamed columns
(m = 40,000) and the Lambert-map wave kernels.
"""
import numpy as np
import pytest

from tests.test_prox_sets_oracle import B, TWO_BLOCK, columns, params

pytestmark = pytest.mark.gpu

STRUCTURAL = {B["zero"], B["default"], B["constant"], B["u_empty"], B["u_grown"]}


def run_gpu(cuda, op, x, result, kw, host=False):
    import torch
    import libsdca_amd as sd
    if host:
        y = x.copy()
        _, thr, sets = sd.prox(op, y, result=result, thresholds=True, sets=True, **kw)
        return y, thr, sets
    t = torch.from_numpy(x).to(cuda)
    _, thr, sets = sd.prox(op, t, result=result, thresholds=True, sets=True, **kw)
    torch.cuda.synchronize()
    return t.cpu().numpy(), thr.cpu().numpy(), sets.cpu().numpy()


def run_oracle(oracle, op, x, result, kw):
    from oracle import binding
    y = x.copy()
    kw = dict(kw)
    col_p = kw.pop("col_p", None)
    thr, sets = oracle.prox_sets(op, y, result=result, params=binding.make_params(**kw),
                                 col_p=col_p)
    return y, thr, sets


def blocks(op, n, m, kw):
    """(column, first row, last row) of each record: blocks [0, p), [p, m)
    of each column for the two-block operators (col_p or p)."""
    if op not in TWO_BLOCK:
        return [(j, 0, m) for j in range(n)]
    col_p = kw.get("col_p")
    out = []
    for j in range(n):
        pj = int(col_p[j]) if col_p is not None else int(kw.get("p", 1))
        out += [(j, 0, pj), (j, pj, m)]
    return out


def hi_cut(op, t, hi):
    if op in ("entropy", "topk_entropy"):
        return t + np.log(hi) if hi > 0 else -np.inf
    if op == "entropy_norm":
        return t + hi + np.log(hi)
    return t + hi


def check(cuda, oracle, op, x, result, kw, host=False, label=""):
    _, thr_g, set_g = run_gpu(cuda, op, x, result, kw, host=host)
    _, thr_o, set_o = run_oracle(oracle, op, x, result, kw)
    n, m = x.shape
    u = float(np.finfo(np.float32 if result == 0 else np.float64).eps)
    bad_branch, tied = [], 0
    counts = {}
    for r, (j, a0, a1) in enumerate(blocks(op, n, m, kw)):
        bo, bg = int(set_o[r, 2]), int(set_g[r, 2])
        counts[bo] = counts.get(bo, 0) + 1
        if bo != bg:
            bad_branch.append((r, bo, bg))
            continue
        ho, mo = int(set_o[r, 0]), int(set_o[r, 1])
        hg, mg = int(set_g[r, 0]), int(set_g[r, 1])
        if (ho, mo) == (hg, mg):
            continue
        what = (f"{op} {label} record {r} (column {j}) branch {bo}: gpu sets ({hg}, {mg}), "
                f"oracle ({ho}, {mo}); records gpu {thr_g[r]}, oracle {thr_o[r]}")
        assert bo not in STRUCTURAL and op not in ("topk_entropy_biased", "two_entropy"), what
        xs = x[j, a0:a1].astype(np.float64)
        to, lo_o, hi_o = (float(v) for v in thr_o[r])
        tg, lo_g, hi_g = (float(v) for v in thr_g[r])
        band = (abs(tg - to) + abs(hi_g - hi_o) + abs(lo_g - lo_o)
                + 64 * u * max(1.0, float(np.abs(xs).max()), abs(to), abs(hi_o)))
        near_hi = int((np.abs(xs - hi_cut(op, to, hi_o)) <= band).sum())
        assert abs(hg - ho) <= near_hi, what + f" ({near_hi} entries near the hi cut)"
        if op not in ("entropy", "entropy_norm"):
            near_lo = int((np.abs(xs - (to + lo_o)) <= band).sum())
            assert abs((hg + mg) - (ho + mo)) <= near_lo, what + f" ({near_lo} near the lo cut)"
        tied += 1
    print(f"{op} {label}: branches {sorted(counts.items())}, records with tied entries "
          f"{tied}, branch mismatches {len(bad_branch)}", flush=True)
    assert not bad_branch, f"{op} {label}: branch (record, oracle, gpu) {bad_branch[:8]}"


REG_OPS = ["knapsack_eq", "knapsack_le", "topk_simplex", "topk_cone", "entropy", "entropy_norm",
           "topk_entropy", "two_simplex", "knapsack_le_biased", "topk_simplex_biased",
           "topk_cone_biased", "topk_entropy_biased", "two_simplex_sort", "two_entropy"]


@pytest.mark.parametrize("dtype,result", [(np.float32, 0), (np.float32, 1), (np.float64, 1)])
@pytest.mark.parametrize("m", [37, 100, 200])
@pytest.mark.parametrize("op", REG_OPS)
def test_sets_register_kernels(cuda, oracle, op, m, dtype, result):
    for k, seed in ((1, 11), (3, 12), (8, 13)):
        kw = params(op, k=k, p=min(5, m - 1))
        x = columns(dtype, n=400, m=m, seed=seed + m)
        check(cuda, oracle, op, x, result, kw, label=f"m={m} k={k} {np.dtype(dtype).name}/{result}")


@pytest.mark.parametrize("op", ["knapsack_eq", "knapsack_le", "topk_simplex", "topk_cone",
                                "entropy", "entropy_norm", "topk_entropy", "two_simplex",
                                "knapsack_le_biased", "topk_simplex_biased", "topk_cone_biased",
                                "two_simplex_sort"])
def test_sets_wide_columns(cuda, oracle, op):
    """m = 3000: the sorted-column and workgroup-wide kernels."""
    kw = params(op, k=5, p=700)
    x = columns(np.float64, n=24, m=3000, seed=21)
    check(cuda, oracle, op, x, 1, kw, label="m=3000")


@pytest.mark.parametrize("op", ["topk_simplex", "topk_cone", "topk_simplex_biased",
                                "topk_cone_biased"])
def test_sets_large_k(cuda, oracle, op):
    """k = 20 > 8: the top-k operators' workgroup-per-column kernel."""
    kw = params(op, k=20)
    x = columns(np.float32, n=200, m=100, seed=23)
    check(cuda, oracle, op, x, 1, kw, label="k=20")


@pytest.mark.parametrize("op", ["knapsack_eq", "knapsack_le", "entropy", "entropy_norm"])
def test_sets_streamed_columns(cuda, oracle, op):
    """m = 40,000 fp32: columns streamed from global memory."""
    kw = params(op)
    if op == "knapsack_le":
        kw["rhs"] = 500.0  # some columns active, some not
    x = columns(np.float32, n=9, m=40_000, seed=25)
    check(cuda, oracle, op, x, 1, kw, label="m=40000")


def test_sets_host_staging_and_per_column_split(cuda, oracle):
    """numpy arrays (SDCA_HOST_PTR) and a per-column split col_p."""
    x = columns(np.float64, n=120, m=50, seed=27)
    col_p = np.random.default_rng(28).integers(1, 50, 120)
    for op in ("knapsack_le", "two_simplex"):
        kw = params(op, k=3)
        if op == "two_simplex":
            kw["col_p"] = col_p
        check(cuda, oracle, op, x, 1, kw, host=True, label="host")


def test_sets_refused_for_lambert(cuda):
    import torch
    import libsdca_amd as sd
    with pytest.raises(sd.SdcaError) as e:
        sd.prox("lambert_w_exp", torch.zeros((2, 4), device=cuda, dtype=torch.float64), sets=True)
    assert e.value.status == 2
