"""The oracle's record sets and branch tags (oracle_prox_sets), pinned.

The reference's threshold record carries iterators first and last over its
permuted scratch copy (proxdef.h:29-67): [begin, first) at hi, [first, last)
free.  The oracle restates each threshold function with the same
partitions, so its (first - begin, last - first) must equal the reference's
exactly, for every operator and input (checked against oracle/_ref, the
reference headers compiled here).

The branch (which return of the threshold function produced the record) is
not part of the reference's record, so each tag is pinned by what the
mathematics fixes for that branch, on the oracle's own output:
  * top-k ZERO / DEFAULT: the projection is 0 and the record (0, 0, 0);
  * top-k CONSTANT: exactly the k largest at hi = (sum of the k largest) /
    divisor, nothing free;
  * KNAPSACK (top-k simplex, knapsack_le, biased knapsack): the output sums
    to rhs, within the upper bound rhs / k for the top-k simplex;
  * top-k simplex SCAN (the cone's solution): its sum is below rhs, and
    hi k = sum (the cone's constraint x_i <= <1, x> / k is tight);
  * knapsack_le INACTIVE: t = 0 and the clamped input sums to at most rhs;
  * biased knapsack SCAN: t = rho <1, x> (its optimality condition);
  * top-k entropy U_EMPTY: no entry at hi, the record (t, 0, 1) / s;
    U_GROWN: the n_hi largest entries are at hi;
  * two-block simplex SEARCH: each block sums to rhs; BELOW_RHS: both blocks
    sum to the same r < rhs.
A tag swapped between two branches fails one of these.
"""
import numpy as np
import pytest

from oracle import binding

OPS = ["knapsack_eq", "knapsack_le", "topk_simplex", "topk_cone", "entropy", "entropy_norm",
       "topk_entropy", "two_simplex", "knapsack_le_biased", "topk_simplex_biased",
       "topk_cone_biased", "topk_entropy_biased", "two_simplex_sort", "two_entropy"]
TWO_BLOCK = {"two_simplex", "two_simplex_sort", "two_entropy"}
B = {"search": 0, "inactive": 1, "zero": 2, "constant": 3, "knapsack": 4, "scan": 5,
     "default": 6, "u_empty": 7, "u_grown": 8, "below_rhs": 9}


def columns(dtype, n=240, m=37, seed=0):
    """Normal columns at several scales plus the special cases: zero, all
    negative, k large values, ties, a constant column."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, m)) * rng.choice([0.05, 0.5, 2.0, 8.0], size=(n, 1))
    x[0] = 0.0
    x[1] = -1.0
    x[2, :5] = 3.0
    x[3] = 0.25
    x[4, :3] = [9.0, 9.0, 9.0]
    x[5] += 4.0
    # the k largest equal and the rest negative: the top-k CONSTANT case
    # for k = 8, 3, 1
    for row, cnt in ((6, 8), (7, 3), (8, 1)):
        x[row] = -1.0
        x[row, :cnt] = 0.1
    return np.ascontiguousarray(x.astype(dtype))


def params(op, k=3, p=5):
    lo = -0.5 if op.startswith("knapsack") else 0.0
    hi = 0.3 if op.startswith("entropy") else 1.0
    rhs = 2.0 if op.startswith("entropy") else 1.0
    return dict(lo=lo, hi=hi, rhs=rhs, rho=0.5, alpha=1.0, k=k, p=p)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("op", OPS)
def test_oracle_sets_equal_reference(oracle, reference, op, dtype):
    for k, seed in ((1, 1), (3, 2), (8, 3)):
        kw = params(op, k=k)
        x = columns(dtype, seed=seed)
        a, b = x.copy(), x.copy()
        tr, sr = reference.prox_sets(op, a, params=binding.make_params(**kw))
        to, so = oracle.prox_sets(op, b, params=binding.make_params(**kw))
        np.testing.assert_array_equal(to, tr)
        np.testing.assert_array_equal(so[:, :2], sr[:, :2], err_msg=f"{op} k={k}")
        assert (sr[:, 2] == -1).all()
        assert np.isin(so[:, 2], list(B.values())).all()


def blocks(op, n, m, p):
    if op not in TWO_BLOCK:
        return [(j, 0, m) for j in range(n)]
    return [bl for j in range(n) for bl in ((j, 0, p), (j, p, m))]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("op", OPS)
def test_oracle_branch_tags(oracle, op, dtype):
    """Each tag against the mathematics of its branch (module docstring)."""
    seen = set()
    u = float(np.finfo(dtype).eps)
    for k, seed in ((1, 4), (3, 5), (8, 6)):
        kw = params(op, k=k)
        x = columns(dtype, seed=seed)
        n, m = x.shape
        y = x.copy()
        thr, sets = oracle.prox_sets(op, y, params=binding.make_params(**kw))
        for r, (j, a0, a1) in enumerate(blocks(op, n, m, kw["p"])):
            t, lo, hi = thr[r]
            n_hi, n_mid, br = (int(v) for v in sets[r])
            xs = x[j, a0:a1].astype(np.float64)
            ys = y[j, a0:a1].astype(np.float64)
            tol = 64 * u * max(1.0, float(np.abs(xs).max()), abs(kw["rhs"]))
            seen.add(br)
            what = f"{op} k={k} column {j} branch {br}"
            if br in (B["zero"], B["default"]):
                assert (t, lo, hi) == (0, 0, 0) and n_hi == 0 and n_mid == 0, what
                assert not ys.any(), what
            elif br == B["constant"]:
                assert n_hi == k and n_mid == 0, what
                top = np.sort(xs)[::-1][:k]
                div = k + (kw["rho"] * k * k if op.endswith("biased") else 0)
                assert abs(hi - top.sum() / div) <= tol, what
                assert np.sort(ys)[::-1][:k].min() >= hi - tol, what
                assert np.sort(ys)[::-1][k:].max(initial=0) <= tol, what
            elif br == B["knapsack"]:
                assert abs(ys.sum() - kw["rhs"]) <= tol * m, what
                if op.startswith("topk"):
                    assert abs(hi - kw["rhs"] / k) <= tol, what
                if op == "knapsack_le_biased":
                    assert t >= kw["rho"] * kw["rhs"] - tol, what
            elif br == B["scan"]:
                if op.startswith("topk_simplex"):
                    assert ys.sum() < kw["rhs"] + tol * m, what
                if op in ("topk_simplex", "topk_cone"):
                    assert abs(hi * k - ys.sum()) <= tol * m, what
                if op == "knapsack_le_biased":
                    assert abs(t - kw["rho"] * ys.sum()) <= tol * m, what
            elif br == B["inactive"]:
                assert t == 0, what
                assert np.clip(xs, kw["lo"], kw["hi"]).sum() <= kw["rhs"] + tol * m, what
            elif br == B["u_empty"]:
                assert n_hi == 0 and n_mid == m, what
                if op == "topk_entropy":
                    assert hi == 1, what
                else:
                    assert ys.max() < hi * (1 + 1e-3) or k == 1, what
            elif br == B["u_grown"]:
                if op == "topk_entropy":
                    assert n_hi >= 1 and n_hi + n_mid == m, what
                    idx = np.argsort(-xs, kind="stable")[:n_hi]
                    assert (np.abs(ys[idx] - hi) <= tol).all(), what
                else:
                    assert (n_hi, n_mid) == (0, m) and (np.abs(ys - hi) <= tol).any(), what
            elif br == B["below_rhs"]:
                assert op in ("two_simplex", "two_simplex_sort"), what
                other = r + 1 if r % 2 == 0 else r - 1
                ja, a0b, a1b = blocks(op, n, m, kw["p"])[other]
                s_other = y[ja, a0b:a1b].astype(np.float64).sum()
                assert abs(ys.sum() - s_other) <= tol * m and ys.sum() < kw["rhs"] + tol * m, what
            else:
                assert br == B["search"], what
                if op in ("two_simplex", "two_simplex_sort"):
                    assert abs(ys.sum() - kw["rhs"]) <= tol * m, what
                if op in ("knapsack_eq", "entropy", "entropy_norm"):
                    assert abs(ys.sum() - kw["rhs"]) <= tol * m * 8, what
                    if op == "knapsack_eq":
                        # the sets agree with the record's cuts outside ties
                        z = xs - t
                        assert int((z > hi + tol).sum()) <= n_hi <= int((z > hi - tol).sum()), what
                        assert (int((z > lo + tol).sum()) <= n_hi + n_mid
                                <= int((z > lo - tol).sum())), what
    expected = {
        "knapsack_eq": {B["search"]}, "knapsack_le": {B["inactive"], B["knapsack"]},
        "topk_simplex": {B["zero"], B["constant"], B["knapsack"], B["scan"]},
        "topk_cone": {B["zero"], B["constant"], B["scan"]},
        "entropy": {B["search"]}, "entropy_norm": {B["search"]},
        "topk_entropy": {B["u_empty"], B["u_grown"]},
        "two_simplex": {B["search"], B["below_rhs"]}, "two_simplex_sort": {B["search"], B["below_rhs"]},
        "knapsack_le_biased": {B["knapsack"], B["scan"]},
        "topk_simplex_biased": {B["zero"], B["constant"], B["knapsack"], B["scan"]},
        "topk_cone_biased": {B["zero"], B["constant"], B["scan"]},
        "topk_entropy_biased": {B["u_empty"], B["u_grown"]}, "two_entropy": {B["search"]},
    }[op]
    assert seen <= expected, (op, seen)
    print(op, np.dtype(dtype).name, "branches seen", sorted(seen))
