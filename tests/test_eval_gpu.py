"""GPU parity of the evaluation pass against the CPU oracle.

* scores: the MFMA GEMM against a float64 product; the bound is the fp32
  dot-product forward error, sqrt(d) eps sum|x_l w_l| (a d-term sum).
* epilogue on identical scores: per-example primal and dual losses of every
  objective against the oracle (bit-exact with the reference on these
  inputs), top-k counts exactly, totals after eval_end.
* end to end: eval_features against the oracle run on the GPU's own scores
  (so that the integer counts can be compared exactly) and against the
  oracle's own float scores within the fp32 score tolerance.

Tolerance for per-example losses, relative to max(1, |loss|): rtol = 1e-5
when the arithmetic (Result) type or the data type is float and 1e-12 when
both are double, plus the reference's own rounding error E_i of that example
and objective, |ref - exact| / s with "exact" the oracle in long double:
|gpu - ref| / s <= rtol + 3 E_i and |gpu - exact| / s <= rtol + 2 E_i.  As for the prox
operators, E is needed because the smooth losses go through a Kiwiel
projection of m - 1 values: in float the reference's own loss at m = 1000 is
~1e-2 away from the long-double value, and any other summation order rounds
differently.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32, F64 = 0, 1
RTOL = {F32: 1e-5, F64: 1e-12}

MC_OBJS = [("l2_hinge_topk", 1.0, 1.0, 5), ("l2_hinge_topk_smooth", 1.0, 1.0, 5),
           ("l2_topk_hinge", 1.0, 1.0, 3), ("l2_topk_hinge_smooth", 0.5, 0.7, 3),
           ("l2_entropy", 1.0, 1.0, 1), ("l2_entropy_topk", 1.0, 1.0, 3)]
ML_OBJS = [("l2_multilabel_hinge", 1.0, 1.0, 1), ("l2_multilabel_hinge_smooth", 1.0, 1.0, 1),
           ("l2_multilabel_entropy", 1.0, 1.0, 1)]
ORACLE_NAME = {"l2_hinge_topk": "hinge_topk", "l2_hinge_topk_smooth": "hinge_topk_smooth",
               "l2_topk_hinge": "topk_hinge", "l2_topk_hinge_smooth": "topk_hinge_smooth",
               "l2_entropy": "entropy", "l2_entropy_topk": "entropy_topk",
               "l2_multilabel_hinge": "multilabel_hinge",
               "l2_multilabel_hinge_smooth": "multilabel_hinge_smooth",
               "l2_multilabel_entropy": "multilabel_entropy"}


def oracle_objs(objs):
    return [(ORACLE_NAME[n], c, g, k) for (n, c, g, k) in objs]


def multilabel_labels(rng, n, m, pmax=5):
    off = [0]
    lab = []
    for _ in range(n):
        p = int(rng.integers(1, min(pmax, m - 1) + 1))
        lab += sorted(rng.choice(m, p, replace=False).tolist())
        off.append(len(lab))
    return np.array(lab, dtype=np.int64), np.array(off, dtype=np.int64)


@pytest.mark.parametrize("n,m,d", [(3000, 300, 1000), (517, 1000, 4096), (1000, 200, 1024),
                                   (64, 5, 37), (130, 129, 16),
                                   # from 2^32 multiply-adds and 512 classes on: the
                                   # hipBLASLt path
                                   (2000, 1000, 2200), (4099, 600, 1800)])
def test_scores_gemm(cuda, n, m, d):
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(n + m + d)
    X = rng.standard_normal((n, d)).astype(np.float32)
    W = (rng.standard_normal((m, d)) * 0.01).astype(np.float32)
    S = sd.scores(torch.from_numpy(X).to(cuda), torch.from_numpy(W).to(cuda))
    torch.cuda.synchronize()
    got = S.cpu().numpy().astype(np.float64)
    want = X.astype(np.float64) @ W.astype(np.float64).T
    bound = np.sqrt(d) * np.finfo(np.float32).eps * (np.abs(X).astype(np.float64) @ np.abs(W).astype(np.float64).T)
    err = np.abs(got - want)
    assert (err <= 4 * bound + 1e-30).all(), f"max err/bound {(err / (bound + 1e-30)).max():.2f}"


LONG_DOUBLE = 2


def compare_per_example(got, want, rtol, what, exact=None):
    """Entry by entry (example i, objective o), with s = max(1, |want|) and
    E_io = |want - exact| / s the reference's own error on that entry:
    |got - want| / s <= rtol + 3 E_io and |got - exact| / s <= rtol + 2 E_io.
    The count of entries above a flat rtol is printed."""
    scale = np.maximum(1.0, np.abs(want))
    err = np.abs(got - want) / scale
    E = np.zeros_like(want)
    if exact is not None:
        E = np.abs(want - exact) / scale
        E = np.where(np.isnan(E), 0.0, E)
    ok = np.isnan(want) | (err <= rtol + 3 * E)
    bad = np.argwhere(~ok)
    assert bad.size == 0, (f"{what}: {len(bad)} entries differ beyond rtol + 3 E_io, max scaled "
                           f"err {np.nanmax(err):.3e}; first {bad[0]}: got "
                           f"{got[tuple(bad[0])]} want {want[tuple(bad[0])]} "
                           f"(E_io {E[tuple(bad[0])]:.3e})")
    if exact is not None:
        e_gpu = np.abs(got - exact) / scale
        bad = np.argwhere(~(np.isnan(want) | (e_gpu <= rtol + 2 * E)))
        assert bad.size == 0, (f"{what}: GPU error vs exact {e_gpu[tuple(bad[0])]:.3e} > rtol + 2 E_io "
                               f"({E[tuple(bad[0])]:.3e}) in {len(bad)} entries")
    over = int(np.count_nonzero(err[~np.isnan(want)] > rtol))
    if over:
        print(f"{what}: {over} of {err.size} entries above a flat {rtol:g}, each within "
              f"rtol + 3 E_io")


@pytest.mark.parametrize("dtype,result", [(np.float32, F32), (np.float32, F64), (np.float64, F64)])
@pytest.mark.parametrize("m", [2, 10, 100, 257, 1000])
@pytest.mark.parametrize("with_a", [False, True])
def test_epilogue_multiclass(cuda, oracle, dtype, result, m, with_a):
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(m + 7)
    n = 700
    S = (rng.standard_normal((n, m)) * 2).astype(dtype)
    y = rng.integers(0, m, n)
    # some exact ties with the label score
    S[: n // 10, 0] = S[np.arange(n // 10), y[: n // 10]]
    A = (rng.standard_normal((n, m)) * 0.01).astype(dtype) if with_a else None
    if A is not None:
        A[np.arange(n), y] = np.abs(A[np.arange(n), y])
        mask = np.ones_like(A, dtype=bool)
        mask[np.arange(n), y] = False
        A[mask] = -np.abs(A[mask])
    objs = [o for o in MC_OBJS if o[3] <= m - 1]
    recs, acc, pe = sd.eval_scores(objs, torch.from_numpy(S).to(cuda), y,
                                   A=None if A is None else torch.from_numpy(A).to(cuda),
                                   result=result, per_example=True)
    torch.cuda.synchronize()
    pe = pe.cpu().numpy()
    o_recs, o_acc, o_pe = oracle.eval_scores(oracle_objs(objs), S, A, y, result=result,
                                             per_example=True)
    _, _, x_pe = oracle.eval_scores(oracle_objs(objs), S, A, y, result=LONG_DOUBLE,
                                    per_example=True)
    rtol = RTOL[result]
    if dtype == np.float32:
        rtol = max(rtol, RTOL[F32])
    compare_per_example(pe[:, :, 0], o_pe[:, :, 0], rtol, f"primal m={m}", x_pe[:, :, 0])
    compare_per_example(pe[:, :, 1], o_pe[:, :, 1], rtol, f"dual m={m}", x_pe[:, :, 1])
    # top-k counts are integers: accuracy must match exactly
    assert np.array_equal(acc * n, o_acc * n) or np.allclose(acc, o_acc, rtol=0, atol=0.5 / n), \
        f"accuracy differs: {acc[:5]} vs {o_acc[:5]}"
    # Totals after eval_end: the per-example bound summed over the batch (the
    # coefficient scales the primal loss), plus the reference's own
    # accumulation error in the Result type.
    eps_r = np.finfo(np.float32 if result == F32 else np.float64).eps
    for oi, (r, o, ob) in enumerate(zip(recs, o_recs, objs)):
        for key, col in (("primal_loss", 0), ("dual_loss", 1)):
            coeff = r["primal_loss"] / pe[:, oi, 0].sum() if col == 0 and pe[:, oi, 0].sum() else 1.0
            scale = np.maximum(1.0, np.abs(o_pe[:, oi, col]))
            E = np.nanmax(np.abs(o_pe[:, oi, col] - x_pe[:, oi, col]) / scale)
            tol = abs(coeff) * (np.sum(scale) * (rtol + 3 * E) + n * eps_r * np.abs(o_pe[:, oi, col]).sum())
            assert abs(r[key] - o[key]) <= tol + 1e-300, f"{ob[0]} {key}: {r[key]} vs {o[key]} (tol {tol})"


@pytest.mark.parametrize("dtype,result", [(np.float32, F32), (np.float64, F64)])
@pytest.mark.parametrize("m", [3, 20, 150, 200, 1000])
def test_epilogue_multilabel(cuda, oracle, dtype, result, m):
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(m + 11)
    n = 500
    S = (rng.standard_normal((n, m)) * 2).astype(dtype)
    lab, off = multilabel_labels(rng, n, m)
    A = (rng.standard_normal((n, m)) * 0.01).astype(dtype)
    recs, _, pe = sd.eval_scores(ML_OBJS, torch.from_numpy(S).to(cuda), lab,
                                 A=torch.from_numpy(A).to(cuda), offsets=off, result=result,
                                 per_example=True)
    torch.cuda.synchronize()
    pe = pe.cpu().numpy()
    o_recs, _, o_pe = oracle.eval_scores(oracle_objs(ML_OBJS), S, A, lab, off, result=result,
                                         per_example=True)
    _, _, x_pe = oracle.eval_scores(oracle_objs(ML_OBJS), S, A, lab, off, result=LONG_DOUBLE,
                                    per_example=True)
    rtol = RTOL[result]
    compare_per_example(pe[:, :, 0], o_pe[:, :, 0], rtol, f"multilabel primal m={m}", x_pe[:, :, 0])
    compare_per_example(pe[:, :, 1], o_pe[:, :, 1], rtol, f"multilabel dual m={m}", x_pe[:, :, 1])
    for r, o in zip(recs, o_recs):
        assert abs(r["rank_loss"] - o["rank_loss"]) <= 1e-6 * max(1, abs(o["rank_loss"]))


@pytest.mark.parametrize("m,d", [(1000, 4096), (200, 1024), (37, 100)])
def test_eval_features_end_to_end(cuda, oracle, m, d):
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(m + d)
    n = 1500
    X = rng.standard_normal((n, d)).astype(np.float32)
    X /= np.linalg.norm(X, axis=1, keepdims=True)
    W = (rng.standard_normal((m, d)) * 0.01).astype(np.float32)
    W0 = (rng.standard_normal((m, d)) * 0.01).astype(np.float32)
    y = rng.integers(0, m, n)
    objs = [("l2_hinge_topk_smooth", 1.0, 1.0, 5), ("l2_entropy", 1.0, 1.0, 1)]
    tX, tW = torch.from_numpy(X).to(cuda), torch.from_numpy(W).to(cuda)
    recs, acc, pe = sd.eval_features(objs, tX, tW, y, W0=torch.from_numpy(W0).to(cuda),
                                     per_example=True)
    S = sd.scores(tX, tW)
    torch.cuda.synchronize()
    S = S.cpu().numpy()
    pe = pe.cpu().numpy()
    preg, dreg = oracle.regularizers(W, W0)
    o_recs, o_acc, o_pe = oracle.eval_scores(oracle_objs(objs), S, None, y, preg=preg, dreg=dreg,
                                             per_example=True)
    _, _, x_pe = oracle.eval_scores(oracle_objs(objs), S, None, y, result=LONG_DOUBLE,
                                    per_example=True)
    # Same scores: counts exact, losses within the fp32 tolerance.
    assert np.allclose(acc, o_acc, rtol=0, atol=0.5 / n)
    compare_per_example(pe[:, :, 0], o_pe[:, :, 0], 1e-5, "features primal", x_pe[:, :, 0])
    # Regularizers 0.5 <W, W> - <W0, W> and 0.5 <W, W>, against float64.
    W64, W064 = W.astype(np.float64), W0.astype(np.float64)
    preg64 = 0.5 * np.sum(W64 * W64) - np.sum(W064 * W64)
    dreg64 = 0.5 * np.sum(W64 * W64)
    for r, o in zip(recs, o_recs):
        assert abs(r["primal_regularizer"] - preg64) <= 1e-6 * max(1, abs(preg64))
        assert abs(r["dual_regularizer"] - dreg64) <= 1e-6 * max(1, abs(dreg64))
        assert abs(r["primal"] - o["primal"]) <= 1e-4 * max(1, abs(o["primal"]))


def test_eval_host_pointers(oracle):
    """numpy in, records out through the library's staging."""
    import libsdca_amd as sd
    rng = np.random.default_rng(5)
    n, m, d = 300, 50, 64
    X = rng.standard_normal((n, d)).astype(np.float32)
    W = (rng.standard_normal((m, d)) * 0.1).astype(np.float32)
    y = rng.integers(0, m, n)
    objs = [("l2_hinge_topk", 1.0, 1.0, 2), ("l2_entropy", 2.0, 1.0, 1)]
    recs, acc, _ = sd.eval_features(objs, X, W, y)
    S = sd.scores(X, W)
    preg, dreg = oracle.regularizers(W)
    o_recs, o_acc, _ = oracle.eval_scores(oracle_objs(objs), S, None, y, preg=preg, dreg=dreg)
    assert np.allclose(acc, o_acc, rtol=0, atol=0.5 / n)
    for r, o in zip(recs, o_recs):
        assert abs(r["primal"] - o["primal"]) <= 1e-4 * max(1, abs(o["primal"]))


def gram(rng, n_rows, n_cols_from, d, dtype):
    """Kernel columns K_i = X_train x_i of unit-norm features: (n, n_train)."""
    Xt = rng.standard_normal((n_cols_from, d))
    Xt /= np.linalg.norm(Xt, axis=1, keepdims=True)
    Xq = rng.standard_normal((n_rows, d))
    Xq /= np.linalg.norm(Xq, axis=1, keepdims=True)
    return (Xq @ Xt.T).astype(dtype), Xt


@pytest.mark.parametrize("dtype,result", [(np.float32, F32), (np.float32, F64), (np.float64, F64)])
@pytest.mark.parametrize("m,multilabel", [(10, False), (300, False), (40, True)])
def test_eval_kernel_training_set(cuda, oracle, dtype, result, m, multilabel):
    """Kernel input (eval/scores.h:30-47): scores_i = A K_i on the matrix cores
    (A transposed once), the dual losses from A's columns, and the dual
    regularizer sum_i 0.5 <a_i, s_i> in both terms (eval/regularizer.h:81-98).
    The epilogue and the regularizer are checked against the oracle on the
    GPU's own scores, the scores against float64."""
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(700 + m)
    n = 700
    K, _ = gram(rng, n, n, 48, dtype)
    A = (rng.standard_normal((n, m)) * 0.05).astype(dtype)
    if multilabel:
        y, off = multilabel_labels(rng, n, m)
        objs = ML_OBJS
    else:
        y, off = rng.integers(0, m, n), None
        objs = [o for o in MC_OBJS if o[3] < m]
    tK, tA = torch.from_numpy(K).to(cuda), torch.from_numpy(A).to(cuda)
    res = "float" if result == F32 else "double"
    recs, acc, pe = sd.eval_kernel(objs, tK, tA, y, offsets=off, result=res, per_example=True)
    S = sd.scores(tK, tA.T.contiguous())
    torch.cuda.synchronize()
    S, pe = S.cpu().numpy(), pe.cpu().numpy()
    # Scores against float64: the d-term forward error bound with d = n_train.
    S64 = K.astype(np.float64) @ A.astype(np.float64)
    eps = np.finfo(dtype).eps
    bound = np.sqrt(n) * eps * (np.abs(K).astype(np.float64) @ np.abs(A).astype(np.float64)) + 1e-30
    assert (np.abs(S - S64) <= 4 * bound).all()
    preg, dreg = oracle.dual_regularizer(A, S, result=result)
    o_recs, o_acc, o_pe = oracle.eval_scores(oracle_objs(objs), S, A, y, off, preg=preg, dreg=dreg,
                                             result=result, per_example=True)
    _, _, x_pe = oracle.eval_scores(oracle_objs(objs), S, A, y, off, result=LONG_DOUBLE,
                                    per_example=True)
    rtol = RTOL[F32 if (dtype == np.float32 or result == F32) else F64]
    compare_per_example(pe[:, :, 0], o_pe[:, :, 0], rtol, "kernel primal", x_pe[:, :, 0])
    compare_per_example(pe[:, :, 1], o_pe[:, :, 1], rtol, "kernel dual", x_pe[:, :, 1])
    if not multilabel:
        assert np.allclose(acc, o_acc, rtol=0, atol=0.5 / n)
    closed = 0.5 * np.trace(A.astype(np.float64).T @ K.astype(np.float64) @ A.astype(np.float64))
    for r, o in zip(recs, o_recs):
        assert r["primal_regularizer"] == r["dual_regularizer"]
        assert abs(r["dual_regularizer"] - preg) <= max(rtol, 1e-9) * 10 * max(1, abs(preg))
        assert abs(r["dual_regularizer"] - closed) <= 1e-4 * max(1, abs(closed))
        for f in ("primal", "dual", "primal_loss", "dual_loss", "rank_loss"):
            assert abs(r[f] - o[f]) <= 1e-4 * max(1, abs(o[f])), (f, r[f], o[f])


@pytest.mark.parametrize("multilabel", [False, True])
def test_eval_test_sets(cuda, oracle, multilabel):
    """eval_test records (eval/types.h:128-172, eval/core.h:98-132) for
    feature and kernel input: the primal loss times the loss coefficient and
    the accuracy or rank loss, the other fields zero."""
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(41 + multilabel)
    n_train, n_test, m, d = 500, 350, 30, 64
    K, Xt = gram(rng, n_test, n_train, d, np.float32)
    A = (rng.standard_normal((n_train, m)) * 0.05).astype(np.float32)
    Xq = rng.standard_normal((n_test, d)).astype(np.float32)
    W = (rng.standard_normal((m, d)) * 0.1).astype(np.float32)
    if multilabel:
        y, off = multilabel_labels(rng, n_test, m)
        objs = ML_OBJS
    else:
        y, off = rng.integers(0, m, n_test), None
        objs = MC_OBJS
    tK, tA = torch.from_numpy(K).to(cuda), torch.from_numpy(A).to(cuda)
    tX, tW = torch.from_numpy(Xq).to(cuda), torch.from_numpy(W).to(cuda)
    for name, run, S in [
        ("kernel", lambda: sd.eval_kernel(objs, tK, tA, y, offsets=off, test=True),
         lambda: sd.scores(tK, tA.T.contiguous())),
        ("features", lambda: sd.eval_features(objs, tX, tW, y, offsets=off, test=True),
         lambda: sd.scores(tX, tW))]:
        recs, acc, _ = run()
        Sg = S()
        torch.cuda.synchronize()
        Sg = Sg.cpu().numpy()
        o_recs, o_acc, _ = oracle.eval_scores(oracle_objs(objs), Sg, None, y, off)
        if not multilabel:
            assert np.allclose(acc, o_acc, rtol=0, atol=0.5 / n_test), name
        for r, o in zip(recs, o_recs):
            assert abs(r["primal_loss"] - o["primal_loss"]) <= 1e-4 * max(1, abs(o["primal_loss"]))
            assert r["primal"] == r["primal_loss"]
            assert r["rank_loss"] == pytest.approx(o["rank_loss"], rel=1e-6, abs=1e-9)
            for f in ("dual", "dual_loss", "primal_regularizer", "dual_regularizer"):
                assert r[f] == 0.0, (name, f)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("n,m,d", [(3000, 300, 1000), (517, 37, 100), (64, 2, 1)])
@pytest.mark.parametrize("with_w0", [False, True])
def test_recompute_primal(cuda, dtype, n, m, d, with_w0):
    """W = W0 + X A' (eval/core.h:148-182) against float64, within the
    n-term dot forward error sqrt(n) eps (sum |x_q a_q| + |w0|)."""
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(n + m + d)
    X = rng.standard_normal((n, d)).astype(dtype)
    A = (rng.standard_normal((n, m)) * 0.1).astype(dtype)
    W0 = (rng.standard_normal((m, d)) * 0.01).astype(dtype) if with_w0 else None
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
    assert (np.abs(W - want) <= 4 * np.sqrt(n) * eps * mag + 1e-30).all()
    if dtype == np.float32 and n == 517:
        Wh = sd.recompute_primal(X, A, W0)  # host pointers through the staging
        assert np.array_equal(Wh, W)


@pytest.mark.parametrize("m", [10, 300])
def test_device_labels_are_checked(cuda, m):
    """Device-resident labels are not visible to the host checks: the
    epilogue kernels check them (data/output.h:169-208) and the call fails
    with the label status instead of reading outside the score rows."""
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(m)
    n = 700
    S = torch.from_numpy((rng.standard_normal((n, m)) * 2).astype(np.float32)).to(cuda)
    y = rng.integers(0, m, n)
    good, _, _ = sd.eval_scores(MC_OBJS, S, torch.from_numpy(y).to(cuda))
    for at, v in [(0, m), (n // 2, -1), (n - 1, m + 1000), (n - 1, 2**40)]:
        yb = y.copy()
        yb[at] = v
        with pytest.raises(sd.SdcaError) as e:
            sd.eval_scores(MC_OBJS, S, torch.from_numpy(yb).to(cuda))
        assert e.value.status == 8, (at, v)
        again, _, _ = sd.eval_scores(MC_OBJS, S, torch.from_numpy(y).to(cuda))
        assert again == good


def test_device_multilabel_offsets_are_checked(cuda):
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(5)
    n, m = 400, 20
    S = torch.from_numpy((rng.standard_normal((n, m)) * 2).astype(np.float32)).to(cuda)
    lab, off = multilabel_labels(rng, n, m)
    good, _, _ = sd.eval_scores(ML_OBJS, S, torch.from_numpy(lab).to(cuda),
                                offsets=torch.from_numpy(off).to(cuda))
    p0 = int(off[1] - off[0])
    cases = []
    bl = lab.copy(); bl[0] = m; cases.append(("label >= m", bl, off))  # noqa: E702
    bl = lab.copy(); bl[-1] = -3; cases.append(("negative label", bl, off))  # noqa: E702
    i = int(np.argmax(np.diff(off) >= 2))
    bl = lab.copy(); bl[off[i]], bl[off[i] + 1] = bl[off[i] + 1], bl[off[i]]  # noqa: E702
    cases.append(("unsorted", bl, off))
    bl = lab.copy(); bl[off[i] + 1] = bl[off[i]]; cases.append(("repeated", bl, off))  # noqa: E702
    bo = off.copy(); bo[1] = bo[0]; cases.append(("example without labels", lab, bo))  # noqa: E702
    bo = off.copy(); bo[1] = bo[2] + 7; cases.append(("offsets decrease", lab, bo))  # noqa: E702
    bo = off.copy(); bo[0] = 1 if p0 >= 2 else -1; cases.append(("first offset", lab, bo))  # noqa: E702
    many = np.arange(m, dtype=np.int64)
    cases.append(("m labels", np.concatenate([many, lab[off[1]:]]),
                  np.concatenate([[0], off[1:] - off[1] + m])))
    for what, bl, bo in cases:
        with pytest.raises(sd.SdcaError) as e:
            sd.eval_scores(ML_OBJS, S, torch.from_numpy(bl).to(cuda),
                           offsets=torch.from_numpy(bo).to(cuda))
        assert e.value.status == 8, what
    again, _, _ = sd.eval_scores(ML_OBJS, S, torch.from_numpy(lab).to(cuda),
                                 offsets=torch.from_numpy(off).to(cuda))
    assert again == good


def dominant_class_inputs(rng, n, m, frac=0.25):
    """X, W with d = m and W = 10 I, so s_ij = 10 x_ij; a fraction of the
    examples get one class far above the label and the rest far below it
    (h = 6 for that class, -9 for the others): the smooth top-k hinge's
    top-k simplex then needs the reference's topk_cone_search with U
    non-empty, which the per-example kernels defer to eval_slow_kernel."""
    X = (rng.standard_normal((n, m)) * 0.05).astype(np.float32)
    y = rng.integers(0, m, n)
    idx = np.flatnonzero(rng.random(n) < frac)
    for i in idx:
        j1 = (y[i] + 1 + rng.integers(0, m - 1)) % m
        X[i, :] = -0.5
        X[i, y[i]] = 0.5
        X[i, j1] = 1.0
    W = (np.eye(m) * 10.0).astype(np.float32)
    return X, W, y


@pytest.mark.parametrize("m", [2, 10, 100, 128, 129, 200, 257, 513, 1000, 1024])
@pytest.mark.parametrize("objs", [[("l2_hinge_topk_smooth", 1.0, 1.0, 5), ("l2_entropy", 1.0, 1.0, 1)],
                                  [("l2_entropy", 2.0, 1.0, 1)],
                                  [("l2_hinge_topk_smooth", 0.5, 0.7, 8)],
                                  [("l2_hinge_topk_smooth", 1.0, 1.0, 1)]])
@pytest.mark.parametrize("result", ["float", "double"])
def test_fused_matches_unfused(cuda, m, objs, result):
    """The fused pass (scores and epilogue in one kernel, scores not stored)
    against the two-kernel form: the scores are formed by the same MFMA
    sequence, so every per-example loss, count-derived accuracy and record
    must be bit-identical.  n is not a multiple of the 32-example workgroup,
    d not of the 8-wide slab or of 4 (the scalar load path) in half the
    cases, and some examples take the deferred top-k cone search (their
    score rows are the only ones the fused kernel writes)."""
    import torch
    import libsdca_amd as sd
    objs = [o for o in objs if o[3] <= m - 1]
    if not objs:
        pytest.skip("k > m - 1")
    rng = np.random.default_rng(m + len(objs))
    n = 1000 + m % 7
    if m <= 1024 and m % 2 == 0:
        X, W, y = dominant_class_inputs(rng, n, m)
    else:
        d = 37 if m % 3 else 64
        X = rng.standard_normal((n, d)).astype(np.float32)
        X /= np.linalg.norm(X, axis=1, keepdims=True)
        W = (rng.standard_normal((m, d)) * 0.5).astype(np.float32)
        y = rng.integers(0, m, n)
    tX, tW = torch.from_numpy(X).to(cuda), torch.from_numpy(W).to(cuda)
    for test in (False, True):
        r_f, a_f, p_f = sd.eval_features(objs, tX, tW, y, result=result, per_example=True, test=test,
                                         fused=True)
        r_u, a_u, p_u = sd.eval_features(objs, tX, tW, y, result=result, per_example=True, test=test)
        torch.cuda.synchronize()
        assert torch.equal(p_f, p_u), f"m={m} test={test}: per-example losses differ"
        assert np.array_equal(a_f, a_u), f"m={m} test={test}: accuracy differs"
        for a, b in zip(r_f, r_u):
            assert a == b, f"m={m} test={test}: records differ"


@pytest.mark.parametrize("result", ["float", "double"])
def test_fused_against_library_scores(cuda, result):
    """From 2^32 multiply-adds and 512 classes on the two-kernel pass takes
    its scores from hipBLASLt, whose k order is not the fused kernel's: the
    per-example losses then agree to the rounding of the scores (float
    scores of d = 1100 unit-norm features: relative 1e-5 of max(1, |loss|)),
    and the top-k accuracies to the rare example whose k-th and (k+1)-th
    scores tie at that rounding."""
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(7)
    n, m, d = 4000, 1000, 1100
    X = rng.standard_normal((n, d)).astype(np.float32)
    X /= np.linalg.norm(X, axis=1, keepdims=True)
    W = (rng.standard_normal((m, d)) * 0.5).astype(np.float32)
    y = rng.integers(0, m, n)
    objs = [("l2_hinge_topk_smooth", 1.0, 1.0, 5), ("l2_entropy", 1.0, 1.0, 1)]
    tX, tW = torch.from_numpy(X).to(cuda), torch.from_numpy(W).to(cuda)
    r_f, a_f, p_f = sd.eval_features(objs, tX, tW, y, result=result, per_example=True, fused=True)
    r_u, a_u, p_u = sd.eval_features(objs, tX, tW, y, result=result, per_example=True)
    torch.cuda.synchronize()
    pf, pu = p_f.cpu().numpy(), p_u.cpu().numpy()
    err = np.abs(pf - pu) / np.maximum(1.0, np.abs(pu))
    assert err.max() <= 1e-5, f"per-example losses differ by {err.max():.3e}"
    assert np.abs(np.asarray(a_f) - np.asarray(a_u)).max() <= 2.0 / n, "accuracies differ"


@pytest.mark.parametrize("dtype,result", [(np.float32, F32), (np.float32, F64), (np.float64, F64)])
@pytest.mark.parametrize("m", [12, 100, 300, 1000])
@pytest.mark.parametrize("k", [9, 11, 40])
def test_epilogue_large_k(cuda, oracle, dtype, result, m, k):
    """Top-k objectives with k above the register list (8): the k + 1
    largest by passes of a group argmax, the smooth top-k hinge's knapsack
    over every slot (l2_hinge_topk.h:71-86, 162-179; l2_topk_hinge.h:72-87,
    166-183; l2_entropy_topk.h:74-94), against the oracle per example, with
    and without dual variables; untrained and spread scores."""
    import torch
    import libsdca_amd as sd
    if k > m - 1:
        pytest.skip("k > m - 1")
    rng = np.random.default_rng(m * 7 + k)
    n = 400
    for spread in (0.01, 3.0):
        S = (rng.standard_normal((n, m)) * spread).astype(dtype)
        y = rng.integers(0, m, n)
        S[: n // 10, 0] = S[np.arange(n // 10), y[: n // 10]]  # ties with the label
        A = (rng.standard_normal((n, m)) * 0.01).astype(dtype)
        objs = [("l2_hinge_topk", 1.0, 1.0, k), ("l2_hinge_topk_smooth", 1.0, 1.0, k),
                ("l2_topk_hinge", 0.7, 1.0, k), ("l2_topk_hinge_smooth", 1.0, 0.5, k),
                ("l2_entropy_topk", 1.0, 1.0, k)]
        recs, acc, pe = sd.eval_scores(objs, torch.from_numpy(S).to(cuda), y,
                                       A=torch.from_numpy(A).to(cuda), result=result,
                                       per_example=True)
        torch.cuda.synchronize()
        pe = pe.cpu().numpy()
        _, o_acc, o_pe = oracle.eval_scores(oracle_objs(objs), S, A, y, result=result,
                                            per_example=True)
        _, _, x_pe = oracle.eval_scores(oracle_objs(objs), S, A, y, result=LONG_DOUBLE,
                                        per_example=True)
        rtol = max(RTOL[result], RTOL[F32] if dtype == np.float32 else RTOL[F64])
        compare_per_example(pe[:, :, 0], o_pe[:, :, 0], rtol, f"large k={k} m={m} primal",
                            x_pe[:, :, 0])
        compare_per_example(pe[:, :, 1], o_pe[:, :, 1], rtol, f"large k={k} m={m} dual",
                            x_pe[:, :, 1])
        assert np.allclose(acc, o_acc, rtol=0, atol=0.5 / n)


# Largest m per element type: 128 KiB of scores per example.
MAX_ROWS = {np.float32: 32768, np.float64: 16384}


def wide_scores(rng, n, m, dtype):
    """Scores with ties against the label, and a quarter of the examples with
    one class far above the label and the rest far below it (the smooth top-k
    hinge's cone search with U non-empty: the deferred-example kernel)."""
    S = (rng.standard_normal((n, m)) * 2).astype(dtype)
    y = rng.integers(0, m, n)
    S[: n // 10, 0] = S[np.arange(n // 10), y[: n // 10]]
    for i in range(n // 10, n // 10 + n // 4):
        S[i, :] = -5.0
        S[i, y[i]] = 5.0
        S[i, (y[i] + 1 + int(rng.integers(0, m - 1))) % m] = 10.0
    return S, y


def check_wide_multiclass(cuda, oracle, dtype, result, m, n, with_a, seed):
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(seed)
    S, y = wide_scores(rng, n, m, dtype)
    A = None
    if with_a:
        A = -np.abs(rng.standard_normal((n, m)) * 0.01).astype(dtype)
        A[np.arange(n), y] = np.abs(A[np.arange(n), y])
    objs = MC_OBJS + [("l2_hinge_topk_smooth", 1.0, 1.0, 12), ("l2_topk_hinge", 1.0, 1.0, 20)]
    recs, acc, pe = sd.eval_scores(objs, torch.from_numpy(S).to(cuda), y,
                                   A=None if A is None else torch.from_numpy(A).to(cuda),
                                   result=result, per_example=True)
    torch.cuda.synchronize()
    pe = pe.cpu().numpy()
    _, o_acc, o_pe = oracle.eval_scores(oracle_objs(objs), S, A, y, result=result,
                                        per_example=True)
    _, _, x_pe = oracle.eval_scores(oracle_objs(objs), S, A, y, result=LONG_DOUBLE,
                                    per_example=True)
    rtol = max(RTOL[result], RTOL[F32] if dtype == np.float32 else RTOL[F64])
    compare_per_example(pe[:, :, 0], o_pe[:, :, 0], rtol, f"wide primal m={m}", x_pe[:, :, 0])
    compare_per_example(pe[:, :, 1], o_pe[:, :, 1], rtol, f"wide dual m={m}", x_pe[:, :, 1])
    assert np.array_equal(np.rint(acc * n), np.rint(o_acc * n)), \
        f"m={m}: top-k counts differ: {acc[:5]} vs {o_acc[:5]}"


@pytest.mark.parametrize("dtype,result", [(np.float32, F32), (np.float32, F64), (np.float64, F64)])
@pytest.mark.parametrize("m", [3000, 5000])
@pytest.mark.parametrize("with_a", [False, True])
def test_epilogue_wide_multiclass(cuda, oracle, dtype, result, m, with_a):
    """m above one wave's registers: one example per workgroup (group sums
    through LDS), every multiclass objective incl. k above the register list,
    deferred examples at these sizes (eval.h:36-47, l2_hinge_topk.h:71-86,
    162-179, l2_topk_hinge.h:72-87, 166-183, l2_entropy.h:77-91,
    l2_entropy_topk.h:74-94)."""
    check_wide_multiclass(cuda, oracle, dtype, result, m, 120, with_a, m + 17)


@pytest.mark.parametrize("dtype,result", [(np.float32, F32), (np.float64, F64)])
def test_epilogue_widest_multiclass(cuda, oracle, dtype, result):
    """The largest rows (32768 fp32, 16384 fp64) and a configuration step."""
    for m in (MAX_ROWS[dtype], 8192, 8193):
        check_wide_multiclass(cuda, oracle, dtype, result, m, 16, True, m + 19)


@pytest.mark.parametrize("dtype,result", [(np.float32, F32), (np.float64, F64)])
@pytest.mark.parametrize("m", [3000, 5000, "max"])
def test_epilogue_wide_multilabel(cuda, oracle, dtype, result, m):
    import torch
    import libsdca_amd as sd
    m = MAX_ROWS[dtype] if m == "max" else m
    rng = np.random.default_rng(m + 23)
    n = 60
    S = (rng.standard_normal((n, m)) * 2).astype(dtype)
    lab, off = multilabel_labels(rng, n, m, pmax=40)
    A = (rng.standard_normal((n, m)) * 0.01).astype(dtype)
    recs, _, pe = sd.eval_scores(ML_OBJS, torch.from_numpy(S).to(cuda), lab,
                                 A=torch.from_numpy(A).to(cuda), offsets=off, result=result,
                                 per_example=True)
    torch.cuda.synchronize()
    pe = pe.cpu().numpy()
    o_recs, _, o_pe = oracle.eval_scores(oracle_objs(ML_OBJS), S, A, lab, off, result=result,
                                         per_example=True)
    _, _, x_pe = oracle.eval_scores(oracle_objs(ML_OBJS), S, A, lab, off, result=LONG_DOUBLE,
                                    per_example=True)
    rtol = RTOL[result]
    compare_per_example(pe[:, :, 0], o_pe[:, :, 0], rtol, f"wide multilabel primal m={m}",
                        x_pe[:, :, 0])
    compare_per_example(pe[:, :, 1], o_pe[:, :, 1], rtol, f"wide multilabel dual m={m}",
                        x_pe[:, :, 1])
    for r, o in zip(recs, o_recs):
        assert abs(r["rank_loss"] - o["rank_loss"]) <= 1e-6 * max(1, abs(o["rank_loss"]))


def test_eval_rows_limit(cuda):
    """Rows above 128 KiB per example are refused with SDCA_ERR_NOT_IMPLEMENTED."""
    import torch
    import libsdca_amd as sd
    for dt, npdt in ((torch.float32, np.float32), (torch.float64, np.float64)):
        m = MAX_ROWS[npdt] + 1
        S = torch.zeros((2, m), dtype=dt, device=cuda)
        with pytest.raises(sd.SdcaError) as e:
            sd.eval_scores([("l2_entropy", 1.0, 1.0, 1)], S, np.zeros(2, np.int64))
        assert e.value.status == 4
