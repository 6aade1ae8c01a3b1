"""Seeded random cases of the evaluation epilogue on given scores: number of
classes m (drawn mostly next to the epilogue's lane-group edges), batch size,
types, objectives with their parameters, multiclass or multilabel labels,
with and without dual variables, checked per example against the oracle as
in tests/test_eval_gpu.py.  The case list is fixed by the seed.
"""
import numpy as np
import pytest

from tests.test_eval_gpu import (LONG_DOUBLE, RTOL, compare_per_example, multilabel_labels,
                                 oracle_objs)

pytestmark = pytest.mark.gpu

F32, F64 = 0, 1
TYPES = [(np.float32, F32), (np.float32, F64), (np.float64, F64)]
EDGES = [4, 64, 256, 1024, 2048]
MC = ["l2_hinge_topk", "l2_hinge_topk_smooth", "l2_topk_hinge", "l2_topk_hinge_smooth",
      "l2_entropy", "l2_entropy_topk"]
ML = ["l2_multilabel_hinge", "l2_multilabel_hinge_smooth", "l2_multilabel_entropy"]
N_CASES = 180


def draw_case(i):
    rng = np.random.default_rng(3000 + i)
    multilabel = i % 3 == 2
    if rng.random() < 0.7:
        m = int(np.clip(int(rng.choice(EDGES)) + rng.integers(-2, 2), 2, 2048))
    else:
        m = int(rng.integers(2, 2049))
    if multilabel:
        m = max(m, 3)
    n = int(rng.integers(1, 300))
    dtype, result = TYPES[int(rng.integers(0, len(TYPES)))]
    names = ML if multilabel else MC
    chosen = rng.choice(len(names), size=int(rng.integers(1, 4)), replace=False)
    objs = []
    for j in chosen:
        c = float(rng.choice([1.0, 0.5, 1.0 / n]))
        gamma = float(rng.choice([1.0, 0.3, 2.0]))
        k = int(min(rng.choice([1, 2, 5, 8]), m - 1))
        objs.append((names[j], c, gamma, k))
    S = (rng.standard_normal((n, m)) * float(rng.choice([0.02, 1.0, 3.0]))).astype(dtype)
    if multilabel:
        lab, off = multilabel_labels(rng, n, m)
    else:
        lab, off = rng.integers(0, m, n), None
        ties = rng.random(n) < 0.1
        S[ties, 0] = S[np.nonzero(ties)[0], lab[ties]]
    A = None
    if rng.random() < 0.6:
        A = (rng.standard_normal((n, m)) * 0.01).astype(dtype)
        if not multilabel:
            A[np.arange(n), lab] = np.abs(A[np.arange(n), lab])
            mask = np.ones_like(A, dtype=bool)
            mask[np.arange(n), lab] = False
            A[mask] = -np.abs(A[mask])
    return m, n, result, objs, S, lab, off, A


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_eval_case(cuda, oracle, i):
    import torch
    import libsdca_amd as sd
    m, n, result, objs, S, lab, off, A = draw_case(i)
    what = f"case {i}: m={m} n={n} {S.dtype.name}->{'f32' if result == F32 else 'f64'} {objs}"
    print(what, "multilabel" if off is not None else "multiclass",
          "with A" if A is not None else "", flush=True)
    recs, acc, pe = sd.eval_scores(objs, torch.from_numpy(S).to(cuda), lab,
                                   A=None if A is None else torch.from_numpy(A).to(cuda),
                                   offsets=off, result=result, per_example=True)
    torch.cuda.synchronize()
    pe = pe.cpu().numpy()
    o_recs, o_acc, o_pe = oracle.eval_scores(oracle_objs(objs), S, A, lab, off, result=result,
                                             per_example=True)
    _, _, x_pe = oracle.eval_scores(oracle_objs(objs), S, A, lab, off, result=LONG_DOUBLE,
                                    per_example=True)
    rtol = RTOL[result]
    if S.dtype == np.float32:
        rtol = max(rtol, RTOL[F32])
    compare_per_example(pe[:, :, 0], o_pe[:, :, 0], rtol, f"{what} primal", x_pe[:, :, 0])
    if A is not None:
        compare_per_example(pe[:, :, 1], o_pe[:, :, 1], rtol, f"{what} dual", x_pe[:, :, 1])
    if off is None:
        # top-k counts are integers: the accuracies are the same fractions
        assert np.allclose(acc, o_acc, rtol=0, atol=0.5 / n), f"{what}: accuracy differs"
    else:
        for r, o in zip(recs, o_recs):
            assert abs(r["rank_loss"] - o["rank_loss"]) <= 1e-6 * max(1, abs(o["rank_loss"])), what


@pytest.mark.parametrize("i", range(40))
def test_random_scores_gemm(cuda, i):
    """S = X W^T for random n, m (both class-tile widths: 128, and 224 where it
    pads m less, e.g. m in (128, 224] or (384, 448]), d (odd included, which
    takes the unvectorised loads) and fp32/fp64, against an fp64 product
    with the sqrt(d) eps bound of test_eval_gpu.test_scores_gemm."""
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(4000 + i)
    n = int(rng.integers(1, 2000))
    m = int(rng.choice([int(rng.integers(1, 2049)), int(rng.integers(129, 225)),
                        int(rng.integers(385, 449))]))
    d = int(rng.choice([int(rng.integers(1, 3000)), 4 * int(rng.integers(1, 600))]))
    dtype = np.float64 if i % 5 == 4 else np.float32
    X = rng.standard_normal((n, d)).astype(dtype)
    W = (rng.standard_normal((m, d)) * 0.01).astype(dtype)
    print(f"case {i}: n={n} m={m} d={d} {np.dtype(dtype).name}", flush=True)
    S = sd.scores(torch.from_numpy(X).to(cuda), torch.from_numpy(W).to(cuda))
    torch.cuda.synchronize()
    got = S.cpu().numpy().astype(np.float64)
    want = X.astype(np.float64) @ W.astype(np.float64).T
    eps = np.finfo(dtype).eps
    bound = np.sqrt(d) * eps * (np.abs(X).astype(np.float64) @ np.abs(W).astype(np.float64).T)
    err = np.abs(got - want)
    assert (err <= 4 * bound + 1e-30).all(), f"case {i}: max err/bound {(err / (bound + 1e-30)).max():.2f}"


@pytest.mark.parametrize("i", range(24))
def test_random_recompute_primal(cuda, i):
    """W = W0 + X A' (eval/core.h:148-182) for random n, m (both GEMM tile
    widths), d, fp32/fp64, with and without W0, against float64 within the
    n-term dot bound of test_eval_gpu.test_recompute_primal."""
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(7000 + i)
    n = int(rng.integers(1, 1500))
    m = int(rng.choice([int(rng.integers(1, 1100)), int(rng.integers(129, 225))]))
    d = int(rng.integers(1, 700))
    dtype = np.float64 if i % 4 == 3 else np.float32
    X = rng.standard_normal((n, d)).astype(dtype)
    A = (rng.standard_normal((n, m)) * 0.1).astype(dtype)
    W0 = (rng.standard_normal((m, d)) * 0.01).astype(dtype) if i % 2 else None
    print(f"case {i}: n={n} m={m} d={d} {np.dtype(dtype).name} W0={W0 is not None}", flush=True)
    W = sd.recompute_primal(torch.from_numpy(X).to(cuda), torch.from_numpy(A).to(cuda),
                            None if W0 is None else torch.from_numpy(W0).to(cuda))
    torch.cuda.synchronize()
    W = W.cpu().numpy()
    want = A.astype(np.float64).T @ X.astype(np.float64)
    mag = np.abs(A.astype(np.float64)).T @ np.abs(X.astype(np.float64))
    if W0 is not None:
        want += W0
        mag += np.abs(W0)
    eps = np.finfo(dtype).eps
    assert (np.abs(W - want) <= 4 * np.sqrt(n) * eps * mag + 1e-30).all(), f"case {i}"


@pytest.mark.parametrize("i", range(24))
def test_random_eval_kernel(cuda, oracle, i):
    """Kernel-input evaluation (scores_i = A K_i) for random n_train, n
    (training set or test set), m and objectives: the per-example losses
    against the oracle's evaluation of the float64 scores' rounding, as the
    fixed cases in test_eval_gpu do."""
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(8000 + i)
    n_train = int(rng.integers(2, 600))
    test = i % 3 == 2
    n = int(rng.integers(1, 400)) if test else n_train
    m = int(rng.choice([3, 10, 64, 200, int(rng.integers(2, 1025))]))
    objs = [("l2_entropy", 1.0, 1.0, 1), ("l2_hinge_topk_smooth", 1.0, 1.0, int(min(3, m - 1)))]
    K = rng.standard_normal((n, n_train)).astype(np.float32) * 0.1
    A = (rng.standard_normal((n_train, m)) * 0.05).astype(np.float32)
    y = rng.integers(0, m, n)
    print(f"case {i}: n_train={n_train} n={n} m={m} test={test}", flush=True)
    recs, acc, pe = sd.eval_kernel(objs, torch.from_numpy(K).to(cuda), torch.from_numpy(A).to(cuda),
                                   y, per_example=True, test=test)
    torch.cuda.synchronize()
    pe = pe.cpu().numpy()
    # The GPU's scores: the same contraction, recomputed here to feed the oracle.
    S = sd.scores(torch.from_numpy(K).to(cuda),
                  torch.from_numpy(np.ascontiguousarray(A.T)).to(cuda)).cpu().numpy()
    o_recs, o_acc, o_pe = oracle.eval_scores(oracle_objs(objs), S, None, y, result=F32,
                                             per_example=True)
    _, _, x_pe = oracle.eval_scores(oracle_objs(objs), S, None, y, result=LONG_DOUBLE,
                                    per_example=True)
    compare_per_example(pe[:, :, 0], o_pe[:, :, 0], RTOL[F32], f"case {i} primal", x_pe[:, :, 0])
    assert np.allclose(acc, o_acc, rtol=0, atol=0.5 / n), f"case {i}: accuracy"
    if test:
        for r in recs:
            assert r["dual_loss"] == 0 and r["dual_regularizer"] == 0, f"case {i}"
        return
    # A training set: the dual losses from A's rows, the dual regularizer
    # sum_i 0.5 <a_i, s_i> in both terms, and the totals, against the oracle
    # on the GPU's scores and the regularizer against float64 A K.
    preg, dreg = oracle.dual_regularizer(A, S, result=F32)
    o_recs, _, o_pe = oracle.eval_scores(oracle_objs(objs), S, A, y, preg=preg, dreg=dreg,
                                         result=F32, per_example=True)
    _, _, x_pe = oracle.eval_scores(oracle_objs(objs), S, A, y, result=LONG_DOUBLE,
                                    per_example=True)
    compare_per_example(pe[:, :, 1], o_pe[:, :, 1], RTOL[F32], f"case {i} dual", x_pe[:, :, 1])
    A64 = A.astype(np.float64)
    closed = 0.5 * float(((K.astype(np.float64) @ A64) * A64).sum())
    mag = 0.5 * float(((np.abs(K).astype(np.float64) @ np.abs(A64)) * np.abs(A64)).sum())
    # The records' totals by the per-entry rule: within 1e-5 of the float
    # reference plus that reference's own error (against the same sums in
    # long double, the regularizer's dots included).
    xp, xd = oracle.dual_regularizer(A, S, result=LONG_DOUBLE)
    x_recs, _, _ = oracle.eval_scores(oracle_objs(objs), S, A, y, preg=xp, dreg=xd,
                                      result=LONG_DOUBLE, per_example=True)
    for r, o, x in zip(recs, o_recs, x_recs):
        assert r["primal_regularizer"] == r["dual_regularizer"], f"case {i}"
        assert abs(r["dual_regularizer"] - closed) <= 1e-5 * max(1.0, mag), f"case {i}"
        for f in ("dual_loss", "primal", "dual"):
            compare_per_example(np.array([[r[f]]]), np.array([[o[f]]]), RTOL[F32],
                                f"case {i} record {f}", np.array([[x[f]]]))
