"""The C++ drop-in (include/sdca_hip.hpp) on the GPU, next to the reference.

oracle/_ref/libsdca_dropin.so (oracle/dropin_shim.cpp, built where the
reference tree exists and shipped with the tree) builds the reference's own
solver_context / dataset / objective objects and calls, on copies of the same
data, the reference function (sdca::evaluate_dataset, sdca::prox_*: CPU,
MKL for its CBLAS calls) and the drop-in of the same name and arguments
(sdca::hip::...: the GPU through the C ABI).  The evaluation records the
drop-in appends are checked field by field against the reference's (and
against the C ABI called directly, bit for bit), for a training set and a
test set; the batched prox calls column by column with the tolerance rule of
tests/test_prox_gpu.py.
"""
import ctypes
import os

import numpy as np
import pytest

from tests import inputs

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DROPIN = os.path.join(ROOT, "oracle", "_ref", "libsdca_dropin.so")
FIELDS = ["primal", "dual", "primal_loss", "dual_loss", "primal_regularizer",
          "dual_regularizer", "rank_loss"]
KIND = {"l2_hinge_topk": 0, "l2_hinge_topk_smooth": 1, "l2_topk_hinge": 2,
        "l2_topk_hinge_smooth": 3, "l2_entropy": 4, "l2_entropy_topk": 5,
        "l2_multilabel_hinge": 6, "l2_multilabel_hinge_smooth": 7, "l2_multilabel_entropy": 8}


@pytest.fixture(scope="module")
def dropin(cuda):
    if not os.path.exists(DROPIN):
        pytest.skip("oracle/_ref/libsdca_dropin.so was not built (needs /root/reference at "
                    "build time)")
    import libsdca_amd as sd
    sd.library()  # the product library first, so that the shim binds to the same instance
    lib = ctypes.CDLL(DROPIN)
    lib.dropin_evaluate_features.restype = ctypes.c_int
    lib.dropin_prox.restype = ctypes.c_int
    return lib


def ptr(a):
    return ctypes.c_void_p(a.ctypes.data if a is not None else None)


def labels_csr(rng, n, m):
    off, lab = [0], []
    for _ in range(n):
        p = int(rng.integers(1, min(5, m - 1) + 1))
        lab += sorted(rng.choice(m, p, replace=False).tolist())
        off.append(len(lab))
    return np.array(lab, dtype=np.int64), np.array(off, dtype=np.int64)


CASES = [("l2_hinge_topk", 1.0, 1.0, 3), ("l2_hinge_topk_smooth", 1.0, 1.0, 5),
         ("l2_topk_hinge", 0.5, 1.0, 2), ("l2_topk_hinge_smooth", 1.0, 0.7, 3),
         ("l2_entropy", 1.0, 1.0, 1), ("l2_entropy_topk", 2.0, 1.0, 3),
         ("l2_multilabel_hinge", 1.0, 1.0, 1), ("l2_multilabel_hinge_smooth", 1.0, 0.5, 1),
         ("l2_multilabel_entropy", 1.5, 1.0, 1)]


@pytest.mark.parametrize("prox_mode", [False, True])
@pytest.mark.parametrize("name,c,gamma,k", CASES)
def test_evaluate_dataset_dropin(cuda, dropin, name, c, gamma, k, prox_mode):
    """sdca::hip::evaluate_dataset(ctx, dataset, scratch, id) against
    sdca::evaluate_dataset on the reference's own context: the appended
    eval_train (training set) and eval_test (test set) records.  Scores are
    well separated (a margin far above the fp32 GEMM rounding), so the top-k
    accuracies must agree exactly; losses and objectives within 1e-5 of
    their magnitude (fp32 data, double Result; the reference's scores come
    from MKL's sgemv, the GPU's from its MFMA GEMM)."""
    import libsdca_amd as sd
    rng = np.random.default_rng(KIND[name] + 10 * prox_mode)
    n, d, m = 300, 64, 20
    multilabel = "multilabel" in name
    X = rng.standard_normal((n, d)).astype(np.float32)
    X /= np.linalg.norm(X, axis=1, keepdims=True)
    W = (rng.standard_normal((m, d)) * 2.0).astype(np.float32)
    W0 = (rng.standard_normal((m, d)) * 0.1).astype(np.float32) if prox_mode else None
    A = (rng.standard_normal((n, m)) * 0.05).astype(np.float32)
    if multilabel:
        lab, off = labels_csr(rng, n, m)
    else:
        lab, off = rng.integers(0, m, n).astype(np.int64), None
    rec_gpu, rec_ref = np.zeros(14), np.zeros(14)
    acc_gpu, acc_ref = np.zeros(2 * m), np.zeros(2 * m)
    rc = dropin.dropin_evaluate_features(
        ctypes.c_int(KIND[name]), ctypes.c_double(c), ctypes.c_double(gamma), ctypes.c_int64(k),
        ctypes.c_int64(d), ctypes.c_int64(m), ctypes.c_int64(n), ptr(X), ptr(W), ptr(W0),
        ptr(A), ptr(lab), ptr(off), ptr(rec_gpu), ptr(acc_gpu), ptr(rec_ref), ptr(acc_ref))
    assert rc == 0, f"drop-in failed with status {rc}: {sd.library().sdca_last_error().decode()}"
    for part, base in (("train", 0), ("test", 7)):
        for i, f in enumerate(FIELDS):
            g, r = rec_gpu[base + i], rec_ref[base + i]
            assert abs(g - r) <= 1e-5 * max(1.0, abs(r)), f"{name} {part} {f}: {g} vs {r}"
    if not multilabel:
        assert np.array_equal(acc_gpu, acc_ref), f"{name}: accuracies {acc_gpu[:5]} vs {acc_ref[:5]}"
    # The drop-in forwards exactly what the C ABI computes.
    recs, acc, _ = sd.eval_features([(name, c, gamma, k)], X, W, lab, A=A, W0=W0, offsets=off,
                                    result="double")
    for i, f in enumerate(FIELDS):
        assert recs[0][f] == rec_gpu[i], f
    if not multilabel:
        assert np.array_equal(acc, acc_gpu[:m])


@pytest.mark.parametrize("op,dtype,m,k", [(0, np.float64, 10, 1), (1, np.float32, 100, 5),
                                          (2, np.float64, 200, 1), (3, np.float32, 40, 3),
                                          (4, np.float32, 100, 5)])
def test_prox_dropin(cuda, oracle, dropin, op, dtype, m, k):
    """sdca::hip::prox_* (dim, first, last, aux, params...) against the
    reference's sdca::prox_* with the same arguments, every column."""
    from tests.test_prox_gpu import parity
    name, kw = {0: ("knapsack_eq", dict(lo=0.0, hi=1.0, rhs=1.0)),
                1: ("topk_simplex", dict(k=k, rhs=1.0)),
                2: ("entropy_norm", dict(hi=1.0, rhs=1.0)),
                3: ("two_simplex", dict(p=k, rhs=1.0)),
                4: ("topk_cone", dict(k=k))}[op]
    x = inputs.label_shifted(400, m, dtype, 700 + op)
    g, r = x.copy(), x.copy()
    rc = dropin.dropin_prox(ctypes.c_int(op), ctypes.c_int64(m), ctypes.c_int64(x.shape[0]),
                            ctypes.c_int64(k), ptr(g), ptr(r))
    assert rc == 0
    # the Result type the reference deduces: that of the floating argument,
    # double for the cone (topk_cone.h:187-199)
    result = 1 if (dtype == np.float64 or op == 4) else 0
    parity(oracle, name, x, g, result, f"drop-in {name}", **kw)
    # and the reference's own output is the oracle's (the oracle is pinned to it)
    want = x.copy()
    from oracle import binding
    oracle.prox(name, want, result=result, params=binding.make_params(**kw))
    assert np.array_equal(r, want)


EPOCH_OBJS = [("l2_hinge_topk", 1.0, 1.0, 3), ("l2_hinge_topk_smooth", 1.0, 0.5, 3),
              ("l2_topk_hinge", 1.0, 1.0, 2), ("l2_topk_hinge_smooth", 0.7, 0.5, 2),
              ("l2_entropy", 1.0, 1.0, 1), ("l2_entropy_topk", 1.5, 1.0, 3),
              ("l2_multilabel_hinge", 1.0, 1.0, 1), ("l2_multilabel_hinge_smooth", 0.7, 0.5, 1),
              ("l2_multilabel_entropy", 1.0, 1.0, 1)]


@pytest.mark.parametrize("obj", EPOCH_OBJS)
def test_dropin_update_epoch(dropin, oracle, obj):
    """sdca::hip::update_epoch (host staging through the C ABI) against the
    reference's own loop of update_variables over the solver's order, on
    copies of one reference context (float data, double results; multiclass
    or multilabel output), two epochs from zero.  The scores round differently on each side (MKL's
    sgemv, the block GEMM), so the bound is the sum of the two pinned ones
    (reference vs restatement, restatement vs GPU: 4 spreads of the
    restatement's two roundings plus 8 ulps each)."""
    import libsdca_amd as sd
    rng = np.random.default_rng(17)
    n, d, m = 150, 24, 11
    X = rng.standard_normal((n, d))
    X /= np.linalg.norm(X, axis=1, keepdims=True)
    X = X.astype(np.float32)
    multilabel = "multilabel" in obj[0]
    if multilabel:
        counts = rng.integers(1, 4, n)
        y = np.concatenate([np.sort(rng.choice(m, c, replace=False)) for c in counts]).astype(np.int64)
        off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    else:
        y = rng.integers(0, m, n).astype(np.int64)
        off = None
    W0 = np.zeros((m, d), np.float32)
    A0 = np.zeros((n, m), np.float32)
    Wg, Ag, Wr, Ar = W0.copy(), A0.copy(), W0.copy(), A0.copy()
    orders = [sd.epoch_order(n, e) for e in range(2)]
    for order in orders:
        rc = dropin.dropin_update_epoch(
            ctypes.c_int(KIND[obj[0]]), ctypes.c_double(obj[1]), ctypes.c_double(obj[2]),
            ctypes.c_int64(obj[3]), ctypes.c_int64(d), ctypes.c_int64(m), ctypes.c_int64(n),
            ptr(X), ptr(y), ptr(off), ptr(order), ctypes.c_int64(len(order)), ptr(Wg), ptr(Ag),
            ptr(Wr), ptr(Ar))
        assert rc == 0, rc
    name = (obj[0][3:],) + tuple(obj[1:])
    Wo, Ao, Wv, Av = W0.copy(), A0.copy(), W0.copy(), A0.copy()
    for order in orders:
        oracle.epoch_features(name, X, Wo, Ao, y, order, result=1, offsets=off)
        oracle.epoch_features(name, X, Wv, Av, y, order, result=1, reverse=True, offsets=off)
    eps = np.finfo(np.float32).eps
    for what, g, r, o, v in (("W", Wg, Wr, Wo, Wv), ("A", Ag, Ar, Ao, Av)):
        tol = 8 * float(np.abs(o - v).max()) + 16 * eps * max(1.0, float(np.abs(o).max()))
        err = float(np.abs(g - r).max())
        assert err <= tol, f"{obj[0]} {what}: |drop-in - reference| {err:.3e} > {tol:.3e}"
    assert np.abs(Ar).max() > 0.01


@pytest.mark.parametrize("obj", EPOCH_OBJS)
def test_dropin_update_epoch_kernel(dropin, oracle, obj):
    """The kernel_input overload of sdca::hip::update_epoch against the
    reference's own loop of update_variables on a kernel input
    (solver/update.h:88-107), a Gaussian kernel, two epochs from zero, with
    the bound of the feature form's drop-in test."""
    import libsdca_amd as sd
    rng = np.random.default_rng(19)
    n, d, m = 150, 8, 11
    X = rng.standard_normal((n, d))
    X /= np.linalg.norm(X, axis=1, keepdims=True)
    sq = (X * X).sum(1)
    K = np.exp(-0.5 * np.maximum(sq[:, None] + sq[None, :] - 2 * X @ X.T, 0.0)).astype(np.float32)
    multilabel = "multilabel" in obj[0]
    if multilabel:
        counts = rng.integers(1, 4, n)
        y = np.concatenate([np.sort(rng.choice(m, c, replace=False)) for c in counts]).astype(np.int64)
        off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    else:
        y = rng.integers(0, m, n).astype(np.int64)
        off = None
    Ag, Ar = np.zeros((n, m), np.float32), np.zeros((n, m), np.float32)
    orders = [sd.epoch_order(n, e) for e in range(2)]
    for order in orders:
        rc = dropin.dropin_update_epoch_kernel(
            ctypes.c_int(KIND[obj[0]]), ctypes.c_double(obj[1]), ctypes.c_double(obj[2]),
            ctypes.c_int64(obj[3]), ctypes.c_int64(m), ctypes.c_int64(n), ptr(K), ptr(y), ptr(off),
            ptr(order), ctypes.c_int64(len(order)), ptr(Ag), ptr(Ar))
        assert rc == 0, rc
    name = (obj[0][3:],) + tuple(obj[1:])
    Ao, Av = np.zeros((n, m), np.float32), np.zeros((n, m), np.float32)
    for order in orders:
        oracle.epoch_kernel(name, K, Ao, y, order, result=1, offsets=off)
        oracle.epoch_kernel(name, K, Av, y, order, result=1, reverse=True, offsets=off)
    eps = np.finfo(np.float32).eps
    tol = 8 * float(np.abs(Ao - Av).max()) + 16 * eps * max(1.0, float(np.abs(Ao).max()))
    err = float(np.abs(Ag - Ar).max())
    assert err <= tol, f"{obj[0]} A: |drop-in - reference| {err:.3e} > {tol:.3e}"
    assert np.abs(Ar).max() > 0.01
