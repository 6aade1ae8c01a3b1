"""Writes the golden vectors in this directory from the reference headers.

Runs only where the reference shim oracle/_ref/libsdca_ref.so was built (it is
compiled from /root/reference's own headers by oracle/Makefile).  Every
fixture holds seeded inputs and the reference's outputs: projected columns
and threshold records for each prox operator and (Data, Result) pair, and the
per-example primal losses, dual losses and top-k histogram of the evaluation
objectives, and whole evaluate_dataset passes (solver/eval.h:15-51) over a
small feature input with the scores the reference's CBLAS (MKL) produced.  tests/test_golden.py checks the oracle against them, so the
oracle stays pinned where the reference tree is absent.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import binding  # noqa: E402
from tests import inputs  # noqa: E402

PROX_CASES = [
    ("knapsack_eq", dict(lo=0.0, hi=1.0, rhs=1.0), [10, 33]),
    ("knapsack_le", dict(lo=0.0, hi=0.3, rhs=1.0), [10, 33]),
    ("topk_simplex", dict(k=5, rhs=1.0), [10, 100]),
    ("topk_cone", dict(k=5), [10, 100]),
    ("entropy", dict(hi=1.0, rhs=1.0), [10, 64]),
    ("entropy_norm", dict(hi=1.0, rhs=1.0), [10, 64]),
    ("topk_entropy", dict(k=3), [10, 64]),
    ("two_simplex", dict(p=2, rhs=1.0), [10, 33]),
    ("lambert_w_exp", dict(), [64]),
    ("knapsack_le_biased", dict(lo=0.0, hi=1.0, rhs=1.0, rho=0.5), [10, 33]),
    ("topk_simplex_biased", dict(k=5, rhs=1.0, rho=0.5), [10, 100]),
    ("topk_cone_biased", dict(k=5, rho=0.5), [10, 100]),
    ("topk_entropy_biased", dict(k=3, alpha=0.7), [10, 64]),
    ("two_simplex_sort", dict(p=2, rhs=1.0), [10, 33]),
    ("two_entropy", dict(p=2, alpha=0.7), [10, 33]),
]
DTYPES = [("f32f32", np.float32, 0), ("f32f64", np.float32, 1), ("f64f64", np.float64, 1)]
MC = [("hinge_topk", 1.0, 1.0, 5), ("hinge_topk_smooth", 1.0, 1.0, 5), ("topk_hinge", 1.0, 1.0, 3),
      ("topk_hinge_smooth", 0.5, 0.7, 3), ("entropy", 1.0, 1.0, 1), ("entropy_topk", 2.0, 1.0, 3)]
ML = [("multilabel_hinge", 1.0, 1.0, 1), ("multilabel_hinge_smooth", 1.0, 0.5, 1),
      ("multilabel_entropy", 1.5, 1.0, 1)]


def prox_inputs(m, dtype, seed):
    n = 24
    return np.ascontiguousarray(np.concatenate([
        inputs.normal(n, m, dtype, seed),
        inputs.label_shifted(n, m, dtype, seed + 1),
        inputs.mixed_signs(n, m, dtype, seed + 2, -3, 3),
        inputs.uniform(n, m, dtype, seed + 3, -10, 10),
        inputs.edge_columns(m, dtype, seed + 4),
    ]))


def main():
    ref = binding.reference()
    if ref is None:
        raise SystemExit("oracle/_ref was not built: run __graft_entry__.build() where "
                         "/root/reference exists")
    out = {}
    for op, kw, ms in PROX_CASES:
        for m in ms:
            for tag, dtype, result in DTYPES:
                x = prox_inputs(m, dtype, 500 + m)
                if op == "lambert_w_exp":
                    x = (x * 5).astype(dtype)
                y = x.copy()
                thr = ref.prox(op, y, result=result, params=binding.make_params(**kw),
                               thresholds=op != "lambert_w_exp")
                key = f"prox/{op}/m{m}/{tag}"
                out[key + "/in"] = x
                out[key + "/out"] = y
                if thr is not None:
                    out[key + "/thr"] = thr
    for tag, dtype, result in DTYPES:
        rng = np.random.default_rng(600)
        n, m = 120, 30
        S = (rng.standard_normal((n, m)) * 2).astype(dtype)
        y = rng.integers(0, m, n)
        S[:10, 1] = S[np.arange(10), y[:10]]
        A = (rng.standard_normal((n, m)) * 0.01).astype(dtype)
        A[np.arange(n), y] = np.abs(A[np.arange(n), y])
        recs, acc, pe = ref.eval_scores(MC, S, A, y, result=result, per_example=True)
        key = f"eval/multiclass/{tag}"
        out[key + "/S"], out[key + "/A"], out[key + "/y"] = S, A, y
        out[key + "/primal"], out[key + "/dual"], out[key + "/acc"] = pe[:, :, 0], pe[:, :, 1], acc
        off = [0]
        lab = []
        for _ in range(n):
            p = int(rng.integers(1, 6))
            lab += sorted(rng.choice(m, p, replace=False).tolist())
            off.append(len(lab))
        recs, _, pe = ref.eval_scores(ML, S, A, lab, off, result=result, per_example=True)
        key = f"eval/multilabel/{tag}"
        out[key + "/S"], out[key + "/A"] = S, A
        out[key + "/labels"], out[key + "/offsets"] = np.array(lab), np.array(off)
        out[key + "/primal"], out[key + "/dual"] = pe[:, :, 0], pe[:, :, 1]
        out[key + "/rank"] = np.array([r["rank_loss"] for r in recs])
    fields = ["primal", "dual", "primal_loss", "dual_loss", "primal_regularizer",
              "dual_regularizer", "rank_loss"]
    for tag, dtype, result in DTYPES:
        for ml in (False, True):
            rng = np.random.default_rng(700 + ml)
            n, d, m = 96, 48, 24
            X = rng.standard_normal((n, d)).astype(dtype)
            W = (rng.standard_normal((m, d)) * 0.5).astype(dtype)
            W0 = (rng.standard_normal((m, d)) * 0.1).astype(dtype)
            A = (rng.standard_normal((n, m)) * 0.05).astype(dtype)
            key = f"eval/dataset/{'multilabel' if ml else 'multiclass'}/{tag}"
            if ml:
                off, lab = [0], []
                for _ in range(n):
                    p = int(rng.integers(1, 6))
                    lab += sorted(rng.choice(m, p, replace=False).tolist())
                    off.append(len(lab))
                lab, off = np.array(lab), np.array(off)
                out[key + "/labels"], out[key + "/offsets"] = lab, off
                objs = ML
            else:
                lab, off = rng.integers(0, m, n), None
                out[key + "/y"] = lab
                objs = MC
            recs, acc = ref.evaluate_dataset(objs, X, W, A, lab, off, W0=W0, result=result)
            out[key + "/X"], out[key + "/W"], out[key + "/W0"], out[key + "/A"] = X, W, W0, A
            out[key + "/records"] = np.array([[r[f] for f in fields] for r in recs])
            if not ml:
                out[key + "/acc"] = acc
            if dtype == np.float32:
                out[key + "/S"] = ref.blas_scores(X, W)
    path = os.path.join(HERE, "reference_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path) / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
