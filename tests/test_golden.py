"""The oracle against the golden vectors made from the reference headers.

tests/golden/reference_vectors.npz was written by tests/golden/make_golden.py
from oracle/_ref (our shim compiled against the reference's own headers):
prox outputs and thresholds for every operator and (Data, Result) pair, and
per-example losses / top-k histograms of the evaluation objectives, and
whole evaluate_dataset passes with the scores the reference's CBLAS (MKL)
produced.  The oracle must reproduce them bit for bit, except where the
reference calls CBLAS for a dot product (the smooth objectives' dual losses,
the regularizers): there the oracle's exactly rounded model and MKL's sum
must both lie within the n-term dot-product bound.  This keeps the oracle
pinned where the reference tree is absent.
"""
import os

import numpy as np
import pytest

from oracle import binding

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "reference_vectors.npz")
RESULT = {"f32f32": 0, "f32f64": 1, "f64f64": 1}
PARAMS = {
    "knapsack_eq": dict(lo=0.0, hi=1.0, rhs=1.0), "knapsack_le": dict(lo=0.0, hi=0.3, rhs=1.0),
    "topk_simplex": dict(k=5, rhs=1.0), "topk_cone": dict(k=5), "entropy": dict(hi=1.0, rhs=1.0),
    "entropy_norm": dict(hi=1.0, rhs=1.0), "topk_entropy": dict(k=3),
    "two_simplex": dict(p=2, rhs=1.0), "lambert_w_exp": dict(),
    "knapsack_le_biased": dict(lo=0.0, hi=1.0, rhs=1.0, rho=0.5),
    "topk_simplex_biased": dict(k=5, rhs=1.0, rho=0.5), "topk_cone_biased": dict(k=5, rho=0.5),
    "topk_entropy_biased": dict(k=3, alpha=0.7),
    "two_simplex_sort": dict(p=2, rhs=1.0), "two_entropy": dict(p=2, alpha=0.7),
}
def dot_bound(dtype, n, absdot):
    """Forward-error bound of an n-term dot product in dtype, plus the
    rounding of the loss itself."""
    u = np.finfo(dtype).eps / 2
    return 2 * (n + 2) * u * absdot + 4 * u * (1 + absdot)


MC = [("hinge_topk", 1.0, 1.0, 5), ("hinge_topk_smooth", 1.0, 1.0, 5), ("topk_hinge", 1.0, 1.0, 3),
      ("topk_hinge_smooth", 0.5, 0.7, 3), ("entropy", 1.0, 1.0, 1), ("entropy_topk", 2.0, 1.0, 3)]
ML = [("multilabel_hinge", 1.0, 1.0, 1), ("multilabel_hinge_smooth", 1.0, 0.5, 1),
      ("multilabel_entropy", 1.5, 1.0, 1)]


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def prox_keys():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return sorted({k.rsplit("/", 1)[0] for k in z.files if k.startswith("prox/")})


@pytest.mark.parametrize("key", prox_keys())
def test_prox_golden(oracle, golden, key):
    _, op, _m, tag = key.split("/")
    x = golden[key + "/in"].copy()
    thr = oracle.prox(op, x, result=RESULT[tag], params=binding.make_params(**PARAMS[op]),
                      thresholds=op != "lambert_w_exp")
    assert np.array_equal(x, golden[key + "/out"], equal_nan=True)
    if thr is not None:
        assert np.array_equal(thr, golden[key + "/thr"], equal_nan=True)


@pytest.mark.parametrize("tag", ["f32f32", "f32f64", "f64f64"])
def test_eval_golden(oracle, golden, tag):
    key = f"eval/multiclass/{tag}"
    S, A, y = golden[key + "/S"], golden[key + "/A"], golden[key + "/y"]
    _, acc, pe = oracle.eval_scores(MC, S, A, y, result=RESULT[tag], per_example=True)
    assert np.array_equal(pe[:, :, 0], golden[key + "/primal"])
    want_dual = golden[key + "/dual"]
    dtype = S.dtype
    for o, (name, c, gamma, _k) in enumerate(MC):
        if not name.endswith("smooth"):
            assert np.array_equal(pe[:, o, 1], want_dual[:, o])
        else:  # A_0 - gamma/(2c) dot(A_1:, A_1:): a CBLAS dot in the reference
            rest = A.astype(np.float64).copy()
            rest[np.arange(len(y)), y] = 0.0
            bound = dot_bound(dtype, S.shape[1], gamma / (2 * c) * (rest ** 2).sum(axis=1))
            assert (np.abs(pe[:, o, 1] - want_dual[:, o]) <= bound).all(), name
    assert np.array_equal(acc, golden[key + "/acc"])
    key = f"eval/multilabel/{tag}"
    recs, _, pe = oracle.eval_scores(ML, golden[key + "/S"], golden[key + "/A"],
                                     golden[key + "/labels"], golden[key + "/offsets"],
                                     result=RESULT[tag], per_example=True)
    assert np.array_equal(pe[:, :, 0], golden[key + "/primal"])
    assert np.array_equal(np.array([r["rank_loss"] for r in recs]), golden[key + "/rank"])
    A = golden[key + "/A"]
    for o, (name, c, gamma, _k) in enumerate(ML):
        want = golden[key + "/dual"][:, o]
        if not name.endswith("smooth"):
            assert np.array_equal(pe[:, o, 1], want)
        else:  # (sum_P A - sum_N A - gamma/c dot(A, A)) / 2
            bound = dot_bound(A.dtype, A.shape[1], 0.5 * gamma / c * (A.astype(np.float64) ** 2).sum(axis=1))
            assert (np.abs(pe[:, o, 1] - want) <= bound).all(), name


FIELDS = ["primal", "dual", "primal_loss", "dual_loss", "primal_regularizer",
          "dual_regularizer", "rank_loss"]


@pytest.mark.parametrize("kind", ["multiclass", "multilabel"])
@pytest.mark.parametrize("tag", ["f32f32", "f32f64", "f64f64"])
def test_evaluate_dataset_golden(oracle, golden, tag, kind):
    """The oracle's evaluation pipeline (scores, regularizers, epilogue,
    eval_end) against whole reference evaluate_dataset passes in prox mode
    (W0 given).  On the reference's own fp32 scores every loss total and the
    accuracies are bit-exact; the regularizers and the smooth dual losses keep
    the dot-product bound; fp64 scores come from the oracle's own gemv and
    keep rounding level."""
    key = f"eval/dataset/{kind}/{tag}"
    X, W, W0, A = (golden[key + "/" + f] for f in ("X", "W", "W0", "A"))
    want = golden[key + "/records"]
    dtype = X.dtype
    if kind == "multiclass":
        lab, off, objs = golden[key + "/y"], None, MC
    else:
        lab, off, objs = golden[key + "/labels"], golden[key + "/offsets"], ML
    if dtype == np.float32:
        S = golden[key + "/S"]
        exact = X.astype(np.float64) @ W.astype(np.float64).T
        absd = np.abs(X.astype(np.float64)) @ np.abs(W.astype(np.float64)).T
        assert (np.abs(oracle.scores(X, W) - exact) <= dot_bound(dtype, X.shape[1], absd)).all()
    else:
        S = oracle.scores(X, W)
    preg, dreg = oracle.regularizers(W, W0, result=RESULT[tag])
    recs, acc, _ = oracle.eval_scores(objs, S, A, lab, off, preg=preg, dreg=dreg, result=RESULT[tag])
    wsq = float((W.astype(np.float64) ** 2).sum() + np.abs(W0.astype(np.float64) * W).sum())
    reg_bound = 2 * dot_bound(dtype, W.size, wsq)
    asq = float((A.astype(np.float64) ** 2).sum())
    for o, (name, c, gamma, _k) in enumerate(objs):
        got = recs[o]
        ref = dict(zip(FIELDS, want[o]))
        for f in ("primal_regularizer", "dual_regularizer"):
            assert abs(got[f] - ref[f]) <= reg_bound, (name, f)
        if dtype == np.float32:
            assert got["primal_loss"] == ref["primal_loss"], name
            assert got["rank_loss"] == ref["rank_loss"], name
        else:
            assert abs(got["primal_loss"] - ref["primal_loss"]) <= 1e-10 * max(1, abs(ref["primal_loss"]))
            assert abs(got["rank_loss"] - ref["rank_loss"]) <= 1e-12
        bound = dot_bound(dtype, A.shape[1], asq * gamma / c) + 1e-12 * abs(ref["dual_loss"])
        assert abs(got["dual_loss"] - ref["dual_loss"]) <= bound, name
        assert abs(got["primal"] - ref["primal"]) <= reg_bound + 1e-10 * max(1, abs(ref["primal"]))
        assert abs(got["dual"] - ref["dual"]) <= reg_bound + bound
    if kind == "multiclass" and dtype == np.float32:
        assert np.array_equal(acc, golden[key + "/acc"])
