"""The oracle restatement against the reference headers themselves.

oracle/_ref/libsdca_ref.so is our shim compiled against /root/reference's
headers (built by __graft_entry__.build() where that tree exists).  Both are
compiled with the same g++ and flags, so every prox output, threshold record,
per-example loss and top-k count must agree bit for bit.  Inputs follow the
reference tests' generators (positive, negative, mixed decades, growing
cumulative vectors; test/prox/*.cpp) plus the benchmark distributions and
hand-made edge columns (ties, constants, zeros, k = m).
"""
import numpy as np
import pytest

from oracle import binding
from tests import inputs

OPS = [
    ("knapsack_eq", dict()),
    ("knapsack_eq", dict(lo=-0.5, hi=0.25, rhs=0.7)),
    ("knapsack_le", dict(hi=0.3, rhs=1.0)),
    ("knapsack_le", dict(lo=-1.0, hi=2.0, rhs=0.5)),
    ("topk_simplex", dict(k=1)),
    ("topk_simplex", dict(k=5, rhs=1.0)),
    ("topk_simplex", dict(k=3, rhs=2.5)),
    ("topk_cone", dict(k=1)),
    ("topk_cone", dict(k=5)),
    ("entropy", dict()),
    ("entropy", dict(hi=0.1, rhs=0.5)),
    ("entropy_norm", dict()),
    ("entropy_norm", dict(hi=0.2, rhs=0.9)),
    ("topk_entropy", dict(k=1)),
    ("topk_entropy", dict(k=4)),
    ("two_simplex", dict(p=1)),
    ("two_simplex", dict(p=3, rhs=2.0)),
    ("lambert_w_exp", dict()),
    ("knapsack_le_biased", dict(rho=1.0)),
    ("knapsack_le_biased", dict(lo=-0.5, hi=0.3, rhs=2.0, rho=0.5)),
    ("knapsack_le_biased", dict(lo=0.0, hi=1.0, rhs=1.0, rho=0.0)),
    ("topk_simplex_biased", dict(k=1, rho=1.0)),
    ("topk_simplex_biased", dict(k=5, rhs=1.0, rho=0.5)),
    ("topk_simplex_biased", dict(k=3, rhs=2.5, rho=2.0)),
    ("topk_cone_biased", dict(k=1, rho=1.0)),
    ("topk_cone_biased", dict(k=3, rho=0.25)),
    ("topk_entropy_biased", dict(k=1, alpha=1.0)),
    ("topk_entropy_biased", dict(k=3, alpha=0.5)),
    ("topk_entropy_biased", dict(k=5, alpha=2.0)),
    ("two_simplex_sort", dict(p=1)),
    ("two_simplex_sort", dict(p=3, rhs=2.0)),
    ("two_entropy", dict(p=1, alpha=1.0)),
    ("two_entropy", dict(p=3, alpha=0.3)),
    ("two_entropy", dict(p=2, alpha=4.0)),
]
DTYPES = [(np.float32, 0), (np.float32, 1), (np.float64, 1), (np.float64, 0)]


def columns(m, dtype, seed):
    n = 60
    parts = [
        inputs.normal(n, m, dtype, seed),
        inputs.label_shifted(n, m, dtype, seed + 1),
        inputs.decades(n, m, dtype, seed + 2, -3, 3),
        inputs.decades(n, m, dtype, seed + 3, -3, 3, sign=-1.0),
        inputs.mixed_signs(n, m, dtype, seed + 4, -3, 3),
        np.cumsum(inputs.uniform(n, m, dtype, seed + 5, 0, 1), axis=1).astype(dtype),
        inputs.uniform(n, m, dtype, seed + 6, -10, 10),
        inputs.decade_blocks(n, m, dtype, seed + 8, -3, 3, block=max(1, min(25, m // 4))),
    ]
    if m >= 1:
        parts.append(inputs.edge_columns(m, dtype, seed + 7))
    return np.ascontiguousarray(np.concatenate(parts, axis=0))


@pytest.mark.parametrize("dtype,result", DTYPES)
@pytest.mark.parametrize("m", [1, 2, 5, 10, 31, 100])
@pytest.mark.parametrize("op,kw", OPS)
def test_prox_bit_exact(oracle, reference, op, kw, m, dtype, result):
    if op in ("two_simplex", "two_simplex_sort", "two_entropy") and (m < 2 or kw["p"] >= m):
        pytest.skip("p must be in [1, m-1]")
    if op in ("topk_simplex", "topk_cone", "topk_entropy", "topk_simplex_biased",
              "topk_cone_biased", "topk_entropy_biased") and kw["k"] > m:
        pytest.skip("k > m")
    if op in ("knapsack_eq",) and (kw.get("hi", 1.0) * m < kw.get("rhs", 1.0) or kw.get("lo", 0.0) * m > kw.get("rhs", 1.0)):
        pytest.skip("infeasible")
    if op in ("entropy", "entropy_norm") and kw.get("hi", 1.0) * m < kw.get("rhs", 1.0):
        pytest.skip("infeasible")
    x = columns(m, dtype, 1000 + m)
    params = binding.make_params(**kw)
    a, b = x.copy(), x.copy()
    want_thr = op != "lambert_w_exp"
    ta = oracle.prox(op, a, result=result, params=params, thresholds=want_thr)
    tb = reference.prox(op, b, result=result, params=params, thresholds=want_thr)
    assert np.array_equal(a, b, equal_nan=True), f"{op}: outputs differ (max {np.nanmax(np.abs(a - b))})"
    if want_thr:
        assert np.array_equal(ta, tb, equal_nan=True), f"{op}: thresholds differ"


@pytest.mark.parametrize("op", ["two_simplex", "two_simplex_sort", "two_entropy"])
def test_prox_per_column_split_bit_exact(oracle, reference, op):
    rng = np.random.default_rng(3)
    x = inputs.normal(500, 40, np.float32, 4)
    col_p = rng.integers(1, 6, 500)
    a, b = x.copy(), x.copy()
    params = binding.make_params(rhs=1.0)
    oracle.prox(op, a, params=params, col_p=col_p)
    reference.prox(op, b, params=params, col_p=col_p)
    assert np.array_equal(a, b)


MC = [("hinge_topk", 1.0, 1.0, 5), ("hinge_topk_smooth", 1.0, 1.0, 5), ("topk_hinge", 1.0, 1.0, 3),
      ("topk_hinge_smooth", 0.5, 0.7, 3), ("entropy", 1.0, 1.0, 1), ("entropy_topk", 2.0, 1.0, 3)]
ML = [("multilabel_hinge", 1.0, 1.0, 1), ("multilabel_hinge_smooth", 1.0, 0.5, 1),
      ("multilabel_entropy", 1.5, 1.0, 1)]


@pytest.mark.parametrize("dtype,result", [(np.float32, 0), (np.float32, 1), (np.float64, 1)])
@pytest.mark.parametrize("m", [6, 50, 300])
def test_eval_multiclass_bit_exact(oracle, reference, m, dtype, result):
    rng = np.random.default_rng(m)
    n = 400
    S = (rng.standard_normal((n, m)) * 2).astype(dtype)
    y = rng.integers(0, m, n)
    S[: n // 8, 1] = S[np.arange(n // 8), y[: n // 8]]  # ties with the label score
    A = (rng.standard_normal((n, m)) * 0.01).astype(dtype)
    A[np.arange(n), y] = np.abs(A[np.arange(n), y])
    ro, ao, po = oracle.eval_scores(MC, S, A, y, result=result, per_example=True)
    rr, ar, pr = reference.eval_scores(MC, S, A, y, result=result, per_example=True)
    assert np.array_equal(ao, ar)
    assert np.array_equal(po[:, :, 0], pr[:, :, 0])
    # dual losses that need no BLAS in the reference shim
    for o, (name, *_rest) in enumerate(MC):
        if not name.endswith("smooth"):
            assert np.array_equal(po[:, o, 1], pr[:, o, 1]), name
    for a, b in zip(ro, rr):
        assert a["primal_loss"] == b["primal_loss"]


@pytest.mark.parametrize("dtype,result", [(np.float32, 0), (np.float64, 1)])
@pytest.mark.parametrize("m", [3, 40, 200])
def test_eval_multilabel_bit_exact(oracle, reference, m, dtype, result):
    rng = np.random.default_rng(m + 1)
    n = 300
    S = (rng.standard_normal((n, m)) * 2).astype(dtype)
    A = (rng.standard_normal((n, m)) * 0.01).astype(dtype)
    off = [0]
    lab = []
    for _ in range(n):
        p = int(rng.integers(1, min(5, m - 1) + 1))
        lab += sorted(rng.choice(m, p, replace=False).tolist())
        off.append(len(lab))
    ro, _, po = oracle.eval_scores(ML, S, A, lab, off, result=result, per_example=True)
    rr, _, pr = reference.eval_scores(ML, S, A, lab, off, result=result, per_example=True)
    assert np.array_equal(po[:, :, 0], pr[:, :, 0])
    for o, (name, *_rest) in enumerate(ML):
        if not name.endswith("smooth"):
            assert np.array_equal(po[:, o, 1], pr[:, o, 1]), name
    for a, b in zip(ro, rr):
        assert a["rank_loss"] == b["rank_loss"]
        assert a["primal_loss"] == b["primal_loss"]
