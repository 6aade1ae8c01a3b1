"""The oracle restatement against the reference headers themselves.

oracle/_ref/libsdca_ref.so is our shim compiled against /root/reference's
headers (built by __graft_entry__.build() where that tree exists), linked to
Intel MKL for the reference's CBLAS calls.  Both are compiled with the same
g++ and flags, so every prox output, threshold record, per-example primal
loss and top-k count must agree bit for bit.  Where the reference calls
CBLAS (the dot of the smooth objectives' dual losses, the regularizer dots,
the scores gemv) the oracle models the call as the exact result rounded to
the data type, and MKL's own summation order is allowed the standard
forward-error bound of an n-term dot product, n u sum |x_i y_i|.  Inputs follow the
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


def dot_bound(dtype, n, absdot):
    """Forward-error bound of an n-term dot product in dtype (both the
    oracle's exactly rounded model and MKL's sum lie within it of the exact
    value), plus the rounding of the loss itself."""
    u = np.finfo(dtype).eps / 2
    return 2 * (n + 2) * u * absdot + 4 * u * (1 + absdot)


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
    for o, (name, c, gamma, _k) in enumerate(MC):
        if not name.endswith("smooth"):
            assert np.array_equal(po[:, o, 1], pr[:, o, 1]), name
        else:
            # A_0 - gamma/(2c) dot(A_1:, A_1:) with the label moved to the front
            rest = A.astype(np.float64).copy()
            rest[np.arange(n), y] = 0.0
            bound = dot_bound(dtype, m, gamma / (2 * c) * (rest ** 2).sum(axis=1))
            assert (np.abs(po[:, o, 1] - pr[:, o, 1]) <= bound).all(), name
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
    for o, (name, c, gamma, _k) in enumerate(ML):
        if not name.endswith("smooth"):
            assert np.array_equal(po[:, o, 1], pr[:, o, 1]), name
        else:
            # (sum_P A - sum_N A - gamma/c dot(A, A)) / 2
            bound = dot_bound(dtype, m, 0.5 * gamma / c * (A.astype(np.float64) ** 2).sum(axis=1))
            assert (np.abs(po[:, o, 1] - pr[:, o, 1]) <= bound).all(), name
    for a, b in zip(ro, rr):
        assert a["rank_loss"] == b["rank_loss"]
        assert a["primal_loss"] == b["primal_loss"]


def labels_csr(rng, n, m):
    off, lab = [0], []
    for _ in range(n):
        p = int(rng.integers(1, min(5, m - 1) + 1))
        lab += sorted(rng.choice(m, p, replace=False).tolist())
        off.append(len(lab))
    return np.array(lab), np.array(off)


@pytest.mark.parametrize("dtype,result", [(np.float32, 0), (np.float32, 1), (np.float64, 1)])
@pytest.mark.parametrize("multilabel", [False, True])
@pytest.mark.parametrize("prox_mode", [False, True])
def test_evaluate_dataset_end_to_end(oracle, reference, dtype, result, multilabel, prox_mode):
    """The reference's whole evaluate_dataset (solver/eval.h:15-51: MKL gemv
    scores, regularizers, dual and primal losses, eval_end) against the
    oracle's pipeline.  Given the reference's own scores, the oracle's
    epilogue, regularizers and eval_end reproduce every record field and
    accuracy bit for bit, except the BLAS dots (dual losses of the smooth
    objectives, the regularizers), which keep the dot-product bound; the
    oracle's own gemv stays within that bound of MKL's scores."""
    rng = np.random.default_rng(77 + multilabel + 2 * prox_mode)
    n, d, m = 240, 96, 40
    X = rng.standard_normal((n, d)).astype(dtype)
    X /= np.linalg.norm(X, axis=1, keepdims=True).astype(dtype)
    W = (rng.standard_normal((m, d)) * 0.5).astype(dtype)
    W0 = (rng.standard_normal((m, d)) * 0.1).astype(dtype) if prox_mode else None
    A = (rng.standard_normal((n, m)) * 0.05).astype(dtype)
    if multilabel:
        lab, off = labels_csr(rng, n, m)
        objs = ML
    else:
        lab, off = rng.integers(0, m, n), None
        objs = MC
    A0 = A.copy()
    recs, acc = reference.evaluate_dataset(objs, X, W, A, lab, off, W0=W0, result=result)
    assert np.array_equal(A, A0), "evaluate_dataset must restore the dual variables"
    # the reference's scores, one cblas gemv per example (eval/scores.h:9-27)
    if dtype == np.float32:
        S = reference.blas_scores(X, W)
        So = oracle.scores(X, W)
        exact = X.astype(np.float64) @ W.astype(np.float64).T
        absd = np.abs(X.astype(np.float64)) @ np.abs(W.astype(np.float64)).T
        assert (np.abs(S - exact) <= dot_bound(dtype, d, absd)).all()
        assert (np.abs(So - exact) <= dot_bound(dtype, d, absd)).all()
    else:
        S = oracle.scores(X, W)
    preg, dreg = oracle.regularizers(W, W0, result=result)
    ro, ao, _ = oracle.eval_scores(objs, S, A, lab, off, preg=preg, dreg=dreg, result=result)
    wsq = float((W.astype(np.float64) ** 2).sum())
    reg_bound = dot_bound(dtype if result == 0 else np.float64, W.size, wsq) + \
        dot_bound(dtype, W.size, wsq)
    for (name, c, gamma, _k), a, b in zip(objs, recs, ro):
        assert abs(a["primal_regularizer"] - b["primal_regularizer"]) <= reg_bound, name
        assert abs(a["dual_regularizer"] - b["dual_regularizer"]) <= reg_bound, name
        if dtype == np.float32:
            assert a["primal_loss"] == b["primal_loss"], name
        else:
            # the oracle's plain gemv loop, not MKL's: rounding-level differences
            assert abs(a["primal_loss"] - b["primal_loss"]) <= 1e-10 * max(1.0, abs(a["primal_loss"]))
        dual_bound = dot_bound(dtype, m, float((A.astype(np.float64) ** 2).sum()) * gamma / c)
        assert abs(a["dual_loss"] - b["dual_loss"]) <= dual_bound + 1e-12 * abs(a["dual_loss"]), name
        assert a["rank_loss"] == b["rank_loss"] or dtype == np.float64, name
    if not multilabel and dtype == np.float32:
        assert np.array_equal(acc, ao)


def test_evaluate_dataset_harness_parallel(reference):
    """The harness-parallel timing mode (examples split over threads, records
    merged) gives the single-threaded records up to summation order."""
    rng = np.random.default_rng(5)
    n, d, m = 400, 64, 50
    X = rng.standard_normal((n, d)).astype(np.float32)
    W = (rng.standard_normal((m, d)) * 0.5).astype(np.float32)
    A = (rng.standard_normal((n, m)) * 0.01).astype(np.float32)
    y = rng.integers(0, m, n)
    r1, a1 = reference.evaluate_dataset(MC, X, W, A, y, nthreads=1)
    r4, a4 = reference.evaluate_dataset(MC, X, W, A, y, nthreads=4)
    for a, b in zip(r1, r4):
        for f in ("primal", "dual", "primal_loss", "dual_loss"):
            assert abs(a[f] - b[f]) <= 1e-5 * max(1.0, abs(a[f])), f
    assert np.allclose(a1, a4, rtol=0, atol=1e-6)
