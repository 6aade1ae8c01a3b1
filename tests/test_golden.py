"""The oracle against the golden vectors made from the reference headers.

tests/golden/reference_vectors.npz was written by tests/golden/make_golden.py
from oracle/_ref (our shim compiled against the reference's own headers):
prox outputs and thresholds for every operator and (Data, Result) pair, and
per-example losses / top-k histograms of the evaluation objectives.  The
oracle must reproduce them bit for bit; this keeps it pinned where the
reference tree is absent.
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
    for o, (name, *_r) in enumerate(MC):
        if not name.endswith("smooth"):  # the reference's BLAS dot is not built
            assert np.array_equal(pe[:, o, 1], want_dual[:, o])
    assert np.array_equal(acc, golden[key + "/acc"])
    key = f"eval/multilabel/{tag}"
    recs, _, pe = oracle.eval_scores(ML, golden[key + "/S"], golden[key + "/A"],
                                     golden[key + "/labels"], golden[key + "/offsets"],
                                     result=RESULT[tag], per_example=True)
    assert np.array_equal(pe[:, :, 0], golden[key + "/primal"])
    assert np.array_equal(np.array([r["rank_loss"] for r in recs]), golden[key + "/rank"])
