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
