"""GPU parity of the SDCA epoch (sdca_epoch_features) against the oracle.

The epoch's arithmetic is the sequential loop's (update.h:52-85 per example,
in the reference solver's order from sdca_epoch_order) except for the order
of the sums in the scores: the GPU forms them from a block GEMM and the
block's earlier rank-1 updates.  Each case runs two epochs from zero on the
GPU and in the oracle (restatement pinned to the reference's own epoch in
tests/test_epoch_oracle.py) and requires every entry of W and A within
4 times the spread of the oracle's two roundings of the scores (exact dot
products against Data accumulation) plus 8 ulps of the largest magnitude:
a different rounding of the scores must not move the epoch further than
another valid rounding does.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

OBJS = [("hinge_topk", 1.0, 1.0, 3), ("hinge_topk_smooth", 1.0, 0.5, 3),
        ("topk_hinge", 1.0, 1.0, 2), ("topk_hinge_smooth", 0.7, 0.5, 2),
        ("entropy", 1.0, 1.0, 1), ("entropy_topk", 1.5, 1.0, 3)]
PAIRS = [(np.float32, 0), (np.float32, 1), (np.float64, 1)]
ORACLE_NAME = {"hinge_topk": "l2_hinge_topk", "hinge_topk_smooth": "l2_hinge_topk_smooth",
               "topk_hinge": "l2_topk_hinge", "topk_hinge_smooth": "l2_topk_hinge_smooth",
               "entropy": "l2_entropy", "entropy_topk": "l2_entropy_topk"}


def problem(dtype, n, d, m, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, d))
    X /= np.linalg.norm(X, axis=1, keepdims=True)
    X[3] = 0.0  # norm2 = 0: the example changes nothing
    y = rng.integers(0, m, n)
    y[:2] = [0, m - 1]
    return X.astype(dtype), y


def oracle_epochs(oracle, obj, X, y, m, result, orders, reverse=False):
    n, d = X.shape
    W = np.zeros((m, d), X.dtype)
    A = np.zeros((n, m), X.dtype)
    for order in orders:
        oracle.epoch_features(obj, X, W, A, y, order, result=result, reverse=reverse)
    return W, A


def gpu_epochs(cuda, obj, X, y, m, result, orders):
    import torch
    import libsdca_amd as sd
    n, d = X.shape
    Xt = torch.from_numpy(X).to(cuda)
    W = torch.zeros((m, d), dtype=Xt.dtype, device=cuda)
    A = torch.zeros((n, m), dtype=Xt.dtype, device=cuda)
    name = (ORACLE_NAME[obj[0]],) + tuple(obj[1:])
    for order in orders:
        sd.epoch_features(name, Xt, W, A, y, order=order, result=result)
    torch.cuda.synchronize()
    return W.cpu().numpy(), A.cpu().numpy()


def check(oracle, cuda, obj, dtype, result, n, d, m, seed, epochs=2):
    import libsdca_amd as sd
    X, y = problem(dtype, n, d, m, seed)
    orders = [sd.epoch_order(n, e) for e in range(epochs)]
    Wg, Ag = gpu_epochs(cuda, obj, X, y, m, result, orders)
    Wo, Ao = oracle_epochs(oracle, obj, X, y, m, result, orders)
    Wv, Av = oracle_epochs(oracle, obj, X, y, m, result, orders, reverse=True)
    eps = np.finfo(dtype).eps
    for name, g, o, v in (("W", Wg, Wo, Wv), ("A", Ag, Ao, Av)):
        spread = float(np.abs(o - v).max())
        tol = 4 * spread + 8 * eps * max(1.0, float(np.abs(o).max()))
        err = float(np.abs(g - o).max())
        print(f"{obj[0]} {np.dtype(dtype).name}/{result} n={n} d={d} m={m} {name}: "
              f"|gpu - oracle| {err:.2e}, spread {spread:.2e}")
        assert err <= tol, f"{obj[0]} m={m} {name}: |gpu - oracle| {err:.3e} > {tol:.3e}"
    assert np.abs(Ao).max() > 0.01
    assert not Ag[3].any()
    return Wg, Ag


@pytest.mark.parametrize("dtype,result", PAIRS)
@pytest.mark.parametrize("obj", OBJS)
@pytest.mark.parametrize("m", [2, 20, 257])
def test_epoch(cuda, oracle, obj, dtype, result, m):
    if obj[3] > m - 1:
        pytest.skip("k > m - 1")
    check(oracle, cuda, obj, dtype, result, 300, 64, m, 7 + m)


@pytest.mark.parametrize("obj", [OBJS[1], OBJS[3], OBJS[4], OBJS[5]])
def test_epoch_c4_like(cuda, oracle, obj):
    """A block-heavy shape (4,000 examples in 125 blocks, m = 1000)."""
    check(oracle, cuda, obj, np.float32, 0, 4000, 256, 1000, 99, epochs=1)


def test_epoch_partial_order_and_bad_index(cuda, oracle):
    """count < n with an explicit order (a prefix of the epoch's order), and
    an index out of range: reported as SDCA_ERR_LABELS after the call, which
    read it as example 0 (no access leaves the arrays)."""
    import torch
    import libsdca_amd as sd
    obj = OBJS[1]
    X, y = problem(np.float32, 200, 32, 10, 5)
    order = sd.epoch_order(200, 0)[:77]
    Wg, Ag = gpu_epochs(cuda, obj, X, y, 10, 0, [order])
    Wo, Ao = oracle_epochs(oracle, obj, X, y, 10, 0, [order])
    assert np.abs(Wg - Wo).max() <= 1e-5 and np.abs(Ag - Ao).max() <= 1e-5
    untouched = np.setdiff1d(np.arange(200), order)
    assert not Ag[untouched].any()
    Xt = torch.from_numpy(X).to(cuda)
    W = torch.zeros((10, 32), device=cuda)
    A = torch.zeros((200, 10), device=cuda)
    with pytest.raises(sd.SdcaError) as e:
        sd.epoch_features(("l2_hinge_topk", 1.0, 1.0, 1), Xt, W, A, y, order=[0, 5, 200, 7])
    assert e.value.status == 8
    bad = y.copy()
    bad[4] = 10
    with pytest.raises(sd.SdcaError) as e:
        sd.epoch_features(("l2_hinge_topk", 1.0, 1.0, 1), Xt, W, A, bad, order=[4])
    assert e.value.status == 8


def test_epoch_duality_gap_closes(cuda):
    """Size-independent property: the relative duality gap of the evaluation
    pass falls over epochs (SDCA's dual ascent) on a separable-ish problem."""
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(3)
    n, d, m = 3000, 128, 50
    centers = rng.standard_normal((m, d)) * 2
    y = rng.integers(0, m, n)
    X = centers[y] + rng.standard_normal((n, d))
    X /= np.linalg.norm(X, axis=1, keepdims=True)
    Xt = torch.from_numpy(X.astype(np.float32)).to(cuda)
    W = torch.zeros((m, d), device=cuda)
    A = torch.zeros((n, m), device=cuda)
    c = 1.0 / (1e-3 * n)  # c = 1 / (lambda n)
    obj = ("l2_hinge_topk_smooth", c, 1.0, 1)
    gaps = []
    for e in range(4):
        sd.epoch_features(obj, Xt, W, A, y, order=sd.epoch_order(n, e))
        recs, _, _ = sd.eval_features([obj], Xt, W, y, A=A, result="double")
        r = recs[0]
        gaps.append((r["primal"] - r["dual"]) / max(abs(r["primal"]), abs(r["dual"])))
    print("relative gaps", gaps)
    assert all(g > -1e-5 for g in gaps)
    assert gaps[-1] < gaps[0] and gaps[-1] < 0.5 * gaps[0]


@pytest.mark.parametrize("obj", [OBJS[1], OBJS[2], OBJS[4], OBJS[5]])
@pytest.mark.parametrize("m", [1500, 3000])
def test_epoch_wide_rows(cuda, oracle, obj, m):
    """Rows above 1024 classes (eight register slots per thread, delta rows in
    global memory) and above 2048 (the vector in LDS, no register slots)."""
    check(oracle, cuda, obj, np.float32, 0, 160, 48, m, 31 + m)


@pytest.mark.parametrize("dtype,result", [(np.float32, 1), (np.float64, 1)])
def test_epoch_wide_rows_double(cuda, oracle, dtype, result):
    check(oracle, cuda, OBJS[1], dtype, result, 160, 48, 1500, 77)


def test_epoch_large_k(cuda, oracle):
    """k > 8 for the top-k hinge: the sorted-column thresholds for every
    example."""
    check(oracle, cuda, ("hinge_topk", 1.0, 1.0, 11), np.float32, 0, 200, 32, 40, 13)


def test_epoch_repeated_examples(cuda, oracle):
    """An order that repeats examples, next to each other inside a block and
    across a block boundary (positions 31 and 32): each occurrence must see the
    previous one's update of a_i and W, as in the sequential loop."""
    import libsdca_amd as sd
    n, m = 120, 15
    X, y = problem(np.float32, n, 24, m, 21)
    base = [int(i) for i in sd.epoch_order(n, 0)]
    order = base[:31] + [base[30], base[30]] + base[31:50] + [base[49]] * 3 + base[50:90]
    for obj in (OBJS[1], OBJS[4]):
        Wg, Ag = gpu_epochs(cuda, obj, X, y, m, 0, [np.array(order, np.int64)])
        Wo, Ao = oracle_epochs(oracle, obj, X, y, m, 0, [np.array(order, np.int64)])
        Wv, Av = oracle_epochs(oracle, obj, X, y, m, 0, [np.array(order, np.int64)],
                               reverse=True)
        eps = np.finfo(np.float32).eps
        for g, o, v in ((Wg, Wo, Wv), (Ag, Ao, Av)):
            tol = 4 * float(np.abs(o - v).max()) + 8 * eps * max(1.0, float(np.abs(o).max()))
            assert float(np.abs(g - o).max()) <= tol


ML_OBJS = [("l2_multilabel_hinge", 1.0, 1.0, 1), ("l2_multilabel_hinge_smooth", 0.7, 0.5, 1),
           ("l2_multilabel_entropy", 1.0, 1.0, 1)]


def ml_labels(rng, n, m, max_labels=4):
    """Sorted, distinct labels per example, 1..min(max_labels, m - 1) each,
    as CSR (labels, offsets)."""
    counts = rng.integers(1, min(max_labels, m - 1) + 1, n)
    labels = np.concatenate([np.sort(rng.choice(m, c, replace=False)) for c in counts])
    return labels.astype(np.int64), np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)


def check_ml(oracle, cuda, obj, dtype, result, n, d, m, seed, epochs=2, max_labels=4):
    import torch
    import libsdca_amd as sd
    X, _ = problem(dtype, n, d, m, seed)
    lab, off = ml_labels(np.random.default_rng(seed + 1), n, m, max_labels)
    orders = [sd.epoch_order(n, e) for e in range(epochs)]
    Xt = torch.from_numpy(X).to(cuda)
    Wt = torch.zeros((m, d), dtype=Xt.dtype, device=cuda)
    At = torch.zeros((n, m), dtype=Xt.dtype, device=cuda)
    for order in orders:
        sd.epoch_features(obj, Xt, Wt, At, lab, order=order, result=result, offsets=off)
    torch.cuda.synchronize()
    Wg, Ag = Wt.cpu().numpy(), At.cpu().numpy()
    name = (obj[0][3:],) + tuple(obj[1:])
    res = []
    for reverse in (False, True):
        W = np.zeros((m, d), X.dtype)
        A = np.zeros((n, m), X.dtype)
        for order in orders:
            oracle.epoch_features(name, X, W, A, lab, order, result=result, reverse=reverse,
                                  offsets=off)
        res.append((W, A))
    (Wo, Ao), (Wv, Av) = res
    eps = np.finfo(dtype).eps
    for what, g, o, v in (("W", Wg, Wo, Wv), ("A", Ag, Ao, Av)):
        spread = float(np.abs(o - v).max())
        tol = 4 * spread + 8 * eps * max(1.0, float(np.abs(o).max()))
        err = float(np.abs(g - o).max())
        print(f"{obj[0]} {np.dtype(dtype).name}/{result} m={m} {what}: |gpu - oracle| "
              f"{err:.2e}, spread {spread:.2e}")
        assert err <= tol, f"{obj[0]} m={m} {what}: |gpu - oracle| {err:.3e} > {tol:.3e}"
    assert np.abs(Ao).max() > 0.01
    assert not Ag[3].any()


@pytest.mark.parametrize("dtype,result", PAIRS)
@pytest.mark.parametrize("obj", ML_OBJS)
@pytest.mark.parametrize("m", [3, 20, 257])
def test_epoch_multilabel(cuda, oracle, obj, dtype, result, m):
    check_ml(oracle, cuda, obj, dtype, result, 300, 64, m, 5 + m)


@pytest.mark.parametrize("obj", ML_OBJS)
def test_epoch_multilabel_wide(cuda, oracle, obj):
    """m = 1500 (eight register slots per thread) with up to 40 labels per
    example, and m = 3000 (the vector in LDS; for the hinges the two-block
    simplex over the LDS column).  fp32 data
    with fp64 arithmetic: in fp32 arithmetic the two-block projection's own
    sums over ~1500 rows round differently on the GPU (tree order) than in
    the reference (sequential), by more than the scores' rounding spread
    that the criterion measures; the fp32 pair is covered up to m = 257."""
    check_ml(oracle, cuda, obj, np.float32, 1, 160, 48, 1500, 41, max_labels=40)
    check_ml(oracle, cuda, obj, np.float32, 1, 120, 32, 3000, 43, max_labels=40)


def test_epoch_multilabel_errors(cuda):
    """Label rules (1..m-1 distinct sorted labels per example): a broken
    example is skipped and reported as SDCA_ERR_LABELS after the epoch; m
    above 524280 is refused."""
    import torch
    import libsdca_amd as sd
    n, d, m = 40, 16, 9
    X, _ = problem(np.float32, n, d, m, 3)
    rows = [[1, 4] if i % 2 else [0, 3, 7] for i in range(n)]
    rows[5] = [6, 2]  # not sorted
    lab = np.array([l for r in rows for l in r], np.int64)
    off = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int64)
    Xt = torch.from_numpy(X).to(cuda)
    W = torch.zeros((m, d), device=cuda)
    A = torch.zeros((n, m), device=cuda)
    with pytest.raises(sd.SdcaError) as e:
        sd.epoch_features(ML_OBJS[0], Xt, W, A, lab, offsets=off)
    assert e.value.status == 8
    assert not A[5].any()  # skipped
    assert A.abs().max() > 0
    with pytest.raises(sd.SdcaError) as e:
        Xw = torch.zeros((4, 8), device=cuda)
        sd.epoch_features(ML_OBJS[1], Xw, torch.zeros((524281, 8), device=cuda),
                          torch.zeros((4, 524281), device=cuda), [0, 1, 2, 3],
                          offsets=[0, 1, 2, 3, 4])
    assert e.value.status == 4


@pytest.mark.parametrize("dtype,result,m", [(np.float32, 1, 16384), (np.float32, 1, 16385),
                                            (np.float32, 1, 40000), (np.float64, 1, 8192),
                                            (np.float64, 1, 8193), (np.float64, 1, 20000)])
def test_epoch_wide_rows_lds_and_global(cuda, oracle, dtype, result, m):
    """Rows at the block kernel's LDS limit (16384 fp32, 8192 fp64) and
    beyond it, where its vectors live in global memory; the C ABI refuses
    m above 524280 (the rank update's grid) before any launch.  The epoch
    starts from a small random W (A = 0): from
    W = 0 the first example's m - 1 off-label values are all equal, a tie
    whose branch in the top-k special cases turns on the last bit of sums
    over thousands of equal terms (summed in another order by the
    reference), which this criterion, the scores' rounding spread, does not
    measure.  Double arithmetic for the same reason."""
    import torch
    import libsdca_amd as sd
    n, d = 40, 16
    X, y = problem(dtype, n, d, m, 17)
    W0 = (np.random.default_rng(18).standard_normal((m, d)) * 0.01).astype(dtype)
    order = sd.epoch_order(n, 0)
    # Above 2048 classes the thresholds come from the sorted row with
    # compensated sums, where the reference's sequential sums over thousands
    # of terms carry an error of their own (E, against the same epoch in
    # long double): the bar adds it, as the prox parity tests do.
    Xt = torch.from_numpy(X).to(cuda)
    Wt = torch.from_numpy(W0.copy()).to(cuda)
    At = torch.zeros((n, m), dtype=Xt.dtype, device=cuda)
    obj = OBJS[1]
    sd.epoch_features((ORACLE_NAME[obj[0]],) + tuple(obj[1:]), Xt, Wt, At, y, order=order,
                      result=result)
    torch.cuda.synchronize()
    Wg, Ag = Wt.cpu().numpy(), At.cpu().numpy()
    res = []
    for reverse, res_t in ((False, result), (True, result), (False, 2)):
        W = W0.copy()
        A = np.zeros((n, m), dtype)
        oracle.epoch_features(obj, X, W, A, y, order, result=res_t, reverse=reverse)
        res.append((W, A))
    (Wo, Ao), (Wv, Av), (Wx, Ax) = res
    eps = np.finfo(dtype).eps
    for name, g, o, v, xx in (("W", Wg, Wo, Wv, Wx), ("A", Ag, Ao, Av, Ax)):
        spread = float(np.abs(o - v).max())
        E = float(np.abs(o - xx).max())
        base = 4 * spread + 8 * eps * max(1.0, float(np.abs(o).max()))
        err = float(np.abs(g - o).max())
        err_x = float(np.abs(g - xx).max())
        print(f"max m={m} {np.dtype(dtype).name}/{result} {name}: |gpu - oracle| {err:.2e}, "
              f"|gpu - exact| {err_x:.2e}, spread {spread:.2e}, reference error {E:.2e}")
        assert err <= base + 3 * E, f"m={m} {name}: |gpu - oracle| {err:.3e}"
        assert err_x <= base + 2 * E, f"m={m} {name}: |gpu - exact| {err_x:.3e}"
    assert np.abs(Ao).max() > 0.01
    if m == 40000:
        Xz = torch.zeros((4, 8), dtype=Xt.dtype, device=cuda)
        with pytest.raises(sd.SdcaError) as e:
            sd.epoch_features(("l2_hinge_topk_smooth", 1.0, 0.5, 3), Xz,
                              torch.zeros((524281, 8), dtype=Xt.dtype, device=cuda),
                              torch.zeros((4, 524281), dtype=Xt.dtype, device=cuda),
                              [0, 1, 2, 3])
        assert e.value.status == 4


@pytest.mark.parametrize("obj", ML_OBJS)
def test_epoch_multilabel_wide_rows(cuda, oracle, obj):
    """The multilabel objectives keep the example's labels in LDS too: at
    m = 12200 fp32 the block kernel's LDS is full (the hinges' two-block
    simplex over the LDS column), at 12201 and 30000 its vectors and labels
    are in global memory."""
    for m, seed in ((12200, 45), (12201, 46), (30000, 47)):
        check_ml(oracle, cuda, obj, np.float32, 1, 24, 16, m, seed, epochs=1, max_labels=6)
