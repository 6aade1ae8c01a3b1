"""The SDCA epoch's oracle and example order against the reference itself.

* The order: sdca_epoch_order (the C ABI, host only) gives the reference
  solver's shuffled order of each epoch (solver.h:75-112).  Pinned by running
  the reference's own solve() for several epochs (oracle/_ref) and, from the
  same start, the reference's update_variables over our orders one epoch at
  a time: the same code on the same order must give identical W and A.
* The restatement (oracle/oracle_epoch.hpp) against the reference's
  update_variables (update.h:52-85) with MKL for its BLAS calls, for the six
  multiclass objectives and the three precision pairs, two epochs: every
  entry of W and A within 4 times the spread of the restatement's two
  roundings of the scores (exact dot products, and Data accumulation from
  the last term) plus 8 ulps of the largest magnitude - the reference's own
  BLAS rounds the scores in a third, unpinned order.
"""
import numpy as np
import pytest

OBJS = [("hinge_topk", 1.0, 1.0, 3), ("hinge_topk_smooth", 1.0, 0.5, 3),
        ("topk_hinge", 1.0, 1.0, 2), ("topk_hinge_smooth", 0.7, 0.5, 2),
        ("entropy", 1.0, 1.0, 1), ("entropy_topk", 1.5, 1.0, 3)]
PAIRS = [(np.float32, 0), (np.float32, 1), (np.float64, 1)]


def problem(dtype, n=80, d=24, m=12, seed=0):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, d))
    X /= np.linalg.norm(X, axis=1, keepdims=True)
    X[3] = 0.0  # norm2 = 0: the reference skips the example
    y = rng.integers(0, m, n)
    return X.astype(dtype), y, m


def run(lib, obj, X, y, m, result, orders, reverse=False):
    n, d = X.shape
    W = np.zeros((m, d), X.dtype)
    A = np.zeros((n, m), X.dtype)
    for order in orders:
        lib.epoch_features(obj, X, W, A, y, order, result=result, reverse=reverse)
    return W, A


def test_epoch_order_is_the_reference_solvers(reference):
    import libsdca_amd as sd
    X, y, m = problem(np.float64)
    n, d = X.shape
    obj = ("hinge_topk_smooth", 1.0, 0.5, 3)
    W1, A1 = np.zeros((m, d)), np.zeros((n, m))
    reference.epoch_features(obj, X, W1, A1, y, epochs=3)
    orders = [sd.epoch_order(n, e) for e in range(3)]
    W2, A2 = run(reference, obj, X, y, m, 1, orders)
    assert np.array_equal(W1, W2) and np.array_equal(A1, A2)
    assert sorted(orders[1]) == list(range(n)) and not np.array_equal(orders[0], orders[1])


@pytest.mark.parametrize("dtype,result", PAIRS)
@pytest.mark.parametrize("obj", OBJS)
def test_epoch_restatement_vs_reference(oracle, reference, obj, dtype, result):
    import libsdca_amd as sd
    X, y, m = problem(dtype, seed=len(obj[0]))
    n = X.shape[0]
    orders = [sd.epoch_order(n, e) for e in range(2)]
    Wr, Ar = run(reference, obj, X, y, m, result, orders)
    Wo, Ao = run(oracle, obj, X, y, m, result, orders)
    Wv, Av = run(oracle, obj, X, y, m, result, orders, reverse=True)
    eps = np.finfo(dtype).eps
    for name, r, o, v in (("W", Wr, Wo, Wv), ("A", Ar, Ao, Av)):
        spread = float(np.abs(o - v).max())
        tol = 4 * spread + 8 * eps * max(1.0, float(np.abs(r).max()))
        err = float(np.abs(o - r).max())
        assert err <= tol, f"{obj[0]} {name}: |oracle - ref| {err:.3e} > {tol:.3e}"
    # the epoch moved the variables (a vacuous comparison pins nothing)
    assert np.abs(Ar).max() > 0.01 and np.abs(Wr).max() > 0.01
    # the skipped example's duals stay at zero (update.h:62)
    assert not Ar[3].any()


ML_OBJS = [("multilabel_hinge", 1.0, 1.0, 1), ("multilabel_hinge_smooth", 0.7, 0.5, 1),
           ("multilabel_entropy", 1.0, 1.0, 1)]


def ml_labels(rng, n, m, max_labels=4):
    """Sorted, distinct labels per example (validate_labels, output.h:169-208),
    1..max_labels of them, as CSR."""
    counts = rng.integers(1, max_labels + 1, n)
    labels = np.concatenate([np.sort(rng.choice(m, c, replace=False)) for c in counts])
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    return labels.astype(np.int64), offsets


def run_ml(lib, obj, X, lab, off, m, result, orders, reverse=False):
    n, d = X.shape
    W = np.zeros((m, d), X.dtype)
    A = np.zeros((n, m), X.dtype)
    for order in orders:
        lib.epoch_features(obj, X, W, A, lab, order, result=result, reverse=reverse, offsets=off)
    return W, A


@pytest.mark.parametrize("dtype,result", PAIRS)
@pytest.mark.parametrize("obj", ML_OBJS)
def test_epoch_multilabel_restatement_vs_reference(oracle, reference, obj, dtype, result):
    """The multilabel objectives' epoch (labels first by the reference's
    swaps, the two-block prox, move_back) against the reference's own
    update_variables, two epochs, the same spread criterion."""
    import libsdca_amd as sd
    X, _, m = problem(dtype, seed=11 + len(obj[0]))
    n = X.shape[0]
    lab, off = ml_labels(np.random.default_rng(5), n, m)
    orders = [sd.epoch_order(n, e) for e in range(2)]
    Wr, Ar = run_ml(reference, obj, X, lab, off, m, result, orders)
    Wo, Ao = run_ml(oracle, obj, X, lab, off, m, result, orders)
    Wv, Av = run_ml(oracle, obj, X, lab, off, m, result, orders, reverse=True)
    eps = np.finfo(dtype).eps
    for name, r, o, v in (("W", Wr, Wo, Wv), ("A", Ar, Ao, Av)):
        spread = float(np.abs(o - v).max())
        tol = 4 * spread + 8 * eps * max(1.0, float(np.abs(r).max()))
        err = float(np.abs(o - r).max())
        assert err <= tol, f"{obj[0]} {name}: |oracle - ref| {err:.3e} > {tol:.3e}"
    assert np.abs(Ar).max() > 0.01 and np.abs(Wr).max() > 0.01
    assert not Ar[3].any()


def test_epoch_multilabel_dual_feasible(oracle):
    """Mathematics: after an epoch every example's multilabel hinge duals
    satisfy the constraints of the two-simplex dual (a_label >= 0, the rest
    <= 0, sum(a_label) = -sum(rest) <= c), whatever the order."""
    import libsdca_amd as sd
    X, _, m = problem(np.float64, seed=3)
    n = X.shape[0]
    lab, off = ml_labels(np.random.default_rng(9), n, m)
    c = 0.8
    _, A = run_ml(oracle, ("multilabel_hinge", c, 1.0, 1), X, lab, off, m, 1,
                  [sd.epoch_order(n, 0)])
    for i in range(n):
        pos = lab[off[i]:off[i + 1]]
        neg = np.setdiff1d(np.arange(m), pos)
        assert (A[i, pos] >= -1e-12).all() and (A[i, neg] <= 1e-12).all()
        assert abs(A[i, pos].sum() + A[i, neg].sum()) <= 1e-9
        assert A[i, pos].sum() <= c + 1e-9


def run_kernel(lib, obj, K, y, m, result, orders, reverse=False, offsets=None):
    n = K.shape[0]
    A = np.zeros((n, m), K.dtype)
    for order in orders:
        lib.epoch_kernel(obj, K, A, y, order, result=result, reverse=reverse, offsets=offsets)
    return A


@pytest.mark.parametrize("dtype,result", PAIRS)
@pytest.mark.parametrize("obj", OBJS + ML_OBJS)
def test_epoch_kernel_restatement_vs_reference(oracle, reference, obj, dtype, result):
    """The kernel-input epoch (update.h:88-107: norm2 = K_ii, scores = A' K_i,
    no primal update) of the restatement against the reference's own
    update_variables on a kernel_input context, two epochs, the spread
    criterion of the feature epoch; K = X X' of unit rows, with one zero row
    (K_ii = 0: the reference skips the example)."""
    import libsdca_amd as sd
    X, y, m = problem(dtype, seed=21 + len(obj[0]))
    K = (X.astype(np.float64) @ X.astype(np.float64).T).astype(dtype)
    n = K.shape[0]
    off = None
    if obj in ML_OBJS:
        y, off = ml_labels(np.random.default_rng(7), n, m)
    orders = [sd.epoch_order(n, e) for e in range(2)]
    Ar = run_kernel(reference, obj, K, y, m, result, orders, offsets=off)
    Ao = run_kernel(oracle, obj, K, y, m, result, orders, offsets=off)
    Av = run_kernel(oracle, obj, K, y, m, result, orders, reverse=True, offsets=off)
    eps = np.finfo(dtype).eps
    spread = float(np.abs(Ao - Av).max())
    tol = 4 * spread + 8 * eps * max(1.0, float(np.abs(Ar).max()))
    err = float(np.abs(Ao - Ar).max())
    assert err <= tol, f"{obj[0]}: |oracle - ref| {err:.3e} > {tol:.3e}"
    assert np.abs(Ar).max() > 0.01
    assert not Ar[3].any()


@pytest.mark.parametrize("obj", OBJS[:1] + OBJS[4:5] + ML_OBJS[:1])
def test_epoch_kernel_equals_feature_epoch(oracle, obj):
    """Mathematics: with K = X X' the kernel-input epoch is the feature
    epoch (scores W' x_i = A' X x_i = A' K_i with W = X' A, and norm2 =
    ||x_i||^2 = K_ii): the dual variables agree to the rounding of the
    scores, in double with the restatement's exact dot products."""
    import libsdca_amd as sd
    X, y, m = problem(np.float64, seed=31)
    K = X @ X.T
    n, d = X.shape
    off = None
    if obj in ML_OBJS:
        y, off = ml_labels(np.random.default_rng(9), n, m)
    orders = [sd.epoch_order(n, e) for e in range(2)]
    W = np.zeros((m, d))
    A = np.zeros((n, m))
    for order in orders:
        oracle.epoch_features(obj, X, W, A, y, order, result=1, offsets=off)
    Ak = run_kernel(oracle, obj, K, y, m, 1, orders, offsets=off)
    assert np.abs(A).max() > 0.01
    assert np.abs(Ak - A).max() <= 1e-12 * max(1.0, float(np.abs(A).max()))
