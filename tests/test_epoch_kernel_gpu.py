"""GPU parity of the SDCA epoch on kernel input (sdca_epoch_kernel) against
the oracle.

The reference's kernel form of update_variables (solver/update.h:88-107)
takes norm2 = K_ii (no update when it is <= 0) and scores A k_i over the
current dual variables of every example (solver/eval/scores.h:28-45).  The
GPU forms a block's scores from one matrix-core product with the dual
variables before the block and the block's earlier updates through the
block's Gram matrix, read from K: the sums of the scores are ordered
differently from the reference's gemv.  Each case runs epochs from zero on
the GPU and in the oracle (restatement pinned to the reference's own kernel
epoch, and to the feature epoch on K = X X', in tests/test_epoch_oracle.py)
and requires every entry of A within 4 times the spread of the oracle's two
roundings of the scores plus 8 ulps of the largest magnitude, the bar of the
feature-input epoch's tests.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

OBJS = [("hinge_topk", 1.0, 1.0, 3), ("hinge_topk_smooth", 1.0, 0.5, 3),
        ("topk_hinge", 1.0, 1.0, 2), ("topk_hinge_smooth", 0.7, 0.5, 2),
        ("entropy", 1.0, 1.0, 1), ("entropy_topk", 1.5, 1.0, 3)]
ML_OBJS = [("multilabel_hinge", 1.0, 1.0, 1), ("multilabel_hinge_smooth", 0.7, 0.5, 1),
           ("multilabel_entropy", 1.0, 1.0, 1)]
PAIRS = [(np.float32, 0), (np.float32, 1), (np.float64, 1)]


def kernel_problem(dtype, n, d, m, seed, kind="linear"):
    """A training kernel matrix and labels.  Linear: K = X X' of unit rows,
    row 3 zero (K_33 = 0: the example is never updated).  Gaussian: exp(-|x_i
    - x_j|^2 / 2) (K_ii = 1)."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, d))
    X /= np.linalg.norm(X, axis=1, keepdims=True)
    if kind == "linear":
        X[3] = 0.0
        K = X @ X.T
    else:
        sq = (X * X).sum(1)
        K = np.exp(-0.5 * np.maximum(sq[:, None] + sq[None, :] - 2 * X @ X.T, 0.0))
    y = rng.integers(0, m, n)
    y[:2] = [0, m - 1]
    return np.ascontiguousarray(K.astype(dtype)), y


def ml_labels(rng, n, m, max_labels=4):
    counts = rng.integers(1, min(max_labels, m - 1) + 1, n)
    labels = np.concatenate([np.sort(rng.choice(m, c, replace=False)) for c in counts])
    return labels.astype(np.int64), np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)


def gpu_epochs(cuda, obj, K, y, m, result, orders, offsets=None, host=False):
    import torch
    import libsdca_amd as sd
    n = K.shape[0]
    name = ("l2_" + obj[0],) + tuple(obj[1:])
    if host:
        A = np.zeros((n, m), K.dtype)
        for order in orders:
            sd.epoch_kernel(name, K, A, y, order=order, result=result, offsets=offsets)
        return A
    Kt = torch.from_numpy(K).to(cuda)
    A = torch.zeros((n, m), dtype=Kt.dtype, device=cuda)
    for order in orders:
        sd.epoch_kernel(name, Kt, A, y, order=order, result=result, offsets=offsets)
    torch.cuda.synchronize()
    return A.cpu().numpy()


def oracle_epochs(oracle, obj, K, y, m, result, orders, reverse=False, offsets=None):
    n = K.shape[0]
    A = np.zeros((n, m), K.dtype)
    for order in orders:
        oracle.epoch_kernel(obj, K, A, y, order, result=result, reverse=reverse, offsets=offsets)
    return A


def compare(oracle, cuda, obj, K, y, m, result, orders, offsets=None, host=False, label=""):
    Ag = gpu_epochs(cuda, obj, K, y, m, result, orders, offsets=offsets, host=host)
    Ao = oracle_epochs(oracle, obj, K, y, m, result, orders, offsets=offsets)
    Av = oracle_epochs(oracle, obj, K, y, m, result, orders, reverse=True, offsets=offsets)
    eps = np.finfo(K.dtype).eps
    spread = float(np.abs(Ao - Av).max())
    tol = 4 * spread + 8 * eps * max(1.0, float(np.abs(Ao).max()))
    err = float(np.abs(Ag - Ao).max())
    print(f"kernel epoch {obj[0]} {label} {K.dtype.name}/{result} n={K.shape[0]} m={m}: "
          f"|gpu - oracle| {err:.2e}, spread {spread:.2e}", flush=True)
    assert err <= tol, f"{obj[0]} {label} m={m}: |gpu - oracle| {err:.3e} > {tol:.3e}"
    assert np.abs(Ao).max() > 0.01
    return Ag, Ao


@pytest.mark.parametrize("dtype,result", PAIRS)
@pytest.mark.parametrize("obj", OBJS)
@pytest.mark.parametrize("m", [2, 20, 257])
def test_epoch_kernel(cuda, oracle, obj, dtype, result, m):
    import libsdca_amd as sd
    if obj[3] > m - 1:
        pytest.skip("k > m - 1")
    n = 300
    orders = [sd.epoch_order(n, e) for e in range(2)]
    K, y = kernel_problem(dtype, n, 64, m, 7 + m)
    Ag, _ = compare(oracle, cuda, obj, K, y, m, result, orders, label="linear")
    assert not Ag[3].any()  # K_33 = 0
    K, y = kernel_problem(dtype, n, 8, m, 9 + m, kind="gauss")
    compare(oracle, cuda, obj, K, y, m, result, orders, label="gauss")


@pytest.mark.parametrize("obj", [OBJS[1], OBJS[4], OBJS[5]])
def test_epoch_kernel_many_blocks(cuda, oracle, obj):
    """2,000 examples (63 blocks), m = 200, fp32; the skinny products split
    over n = 2,000 (the products' inner dimension)."""
    import libsdca_amd as sd
    n, m = 2000, 200
    K, y = kernel_problem(np.float32, n, 16, m, 55, kind="gauss")
    compare(oracle, cuda, obj, K, y, m, 0, [sd.epoch_order(n, 0)], label="gauss")


def test_epoch_kernel_host_staging(cuda, oracle):
    """numpy arrays through SDCA_HOST_PTR: K and A staged through device
    memory, A copied back."""
    import libsdca_amd as sd
    n, m = 150, 12
    K, y = kernel_problem(np.float64, n, 16, m, 3)
    compare(oracle, cuda, OBJS[4], K, y, m, 1, [sd.epoch_order(n, 0)], host=True, label="host")


def test_epoch_kernel_order_repeats_and_errors(cuda, oracle):
    """A partial order that repeats examples inside a block and across a
    block boundary; examples outside the order keep a_i = 0; an index out of
    range and a label out of range are reported as SDCA_ERR_LABELS; m above
    524280 is refused."""
    import torch
    import libsdca_amd as sd
    n, m = 120, 15
    K, y = kernel_problem(np.float32, n, 24, m, 21, kind="gauss")
    base = [int(i) for i in sd.epoch_order(n, 0)]
    order = np.array(base[:31] + [base[30], base[30]] + base[31:50] + [base[49]] * 3 + base[50:90],
                     np.int64)
    for obj in (OBJS[1], OBJS[4]):
        Ag, _ = compare(oracle, cuda, obj, K, y, m, 0, [order], label="repeats")
        untouched = np.setdiff1d(np.arange(n), order)
        assert not Ag[untouched].any()
    Kt = torch.from_numpy(K).to(cuda)
    A = torch.zeros((n, m), device=cuda)
    with pytest.raises(sd.SdcaError) as e:
        sd.epoch_kernel(("l2_hinge_topk", 1.0, 1.0, 1), Kt, A, y, order=[0, 5, n, 7])
    assert e.value.status == 8
    bad = y.copy()
    bad[4] = m
    with pytest.raises(sd.SdcaError) as e:
        sd.epoch_kernel(("l2_hinge_topk", 1.0, 1.0, 1), Kt, A, bad, order=[4])
    assert e.value.status == 8
    with pytest.raises(sd.SdcaError) as e:
        sd.epoch_kernel(("l2_hinge_topk", 1.0, 1.0, 1), Kt, torch.zeros((n, 524281), device=cuda), y)
    assert e.value.status == 4


@pytest.mark.parametrize("obj", ML_OBJS)
@pytest.mark.parametrize("dtype,result", [(np.float32, 0), (np.float64, 1)])
def test_epoch_kernel_multilabel(cuda, oracle, obj, dtype, result):
    import libsdca_amd as sd
    n, m = 200, 20
    K, _ = kernel_problem(dtype, n, 32, m, 61)
    lab, off = ml_labels(np.random.default_rng(62), n, m)
    orders = [sd.epoch_order(n, e) for e in range(2)]
    Ag, _ = compare(oracle, cuda, obj, K, lab, m, result, orders, offsets=off, label="multilabel")
    assert not Ag[3].any()


@pytest.mark.parametrize("obj", [OBJS[1], OBJS[4], OBJS[5]])
def test_epoch_kernel_rows_beyond_lds(cuda, oracle, obj):
    """m = 20,000 fp32: the block kernel's vectors in global memory."""
    import libsdca_amd as sd
    n, m = 48, 20000
    K, y = kernel_problem(np.float32, n, 16, m, 71, kind="gauss")
    compare(oracle, cuda, obj, K, y, m, 1, [sd.epoch_order(n, 0)], label="global rows")


@pytest.mark.parametrize("obj", [OBJS[1], OBJS[4]])
def test_epoch_kernel_wide_rows(cuda, oracle, obj):
    """m = 1500: eight register slots per thread, the delta rows in global
    memory."""
    import libsdca_amd as sd
    n, m = 160, 1500
    K, y = kernel_problem(np.float32, n, 48, m, 31, kind="gauss")
    compare(oracle, cuda, obj, K, y, m, 1, [sd.epoch_order(n, e) for e in range(2)], label="wide")


def test_epoch_kernel_duality_gap_closes(cuda):
    """Size-independent property at n = 4,000: the relative duality gap of
    the kernel evaluation pass falls over epochs."""
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(3)
    n, d, m = 4000, 32, 50
    centers = rng.standard_normal((m, d)) * 2
    y = rng.integers(0, m, n)
    X = centers[y] + rng.standard_normal((n, d))
    X /= np.linalg.norm(X, axis=1, keepdims=True)
    K = torch.from_numpy((X @ X.T).astype(np.float32)).to(cuda)
    A = torch.zeros((n, m), device=cuda)
    c = 1.0 / (1e-3 * n)
    obj = ("l2_hinge_topk_smooth", c, 1.0, 1)
    gaps = []
    for e in range(4):
        sd.epoch_kernel(obj, K, A, y, order=sd.epoch_order(n, e))
        recs, _, _ = sd.eval_kernel([obj], K, A, y, result="double")
        r = recs[0]
        gaps.append((r["primal"] - r["dual"]) / max(abs(r["primal"]), abs(r["dual"])))
    print("relative gaps", gaps, flush=True)
    assert all(g > -1e-5 for g in gaps)
    assert gaps[-1] < 0.5 * gaps[0]


def test_epoch_kernel_equals_feature_epoch(cuda):
    """On K = X X' the kernel epoch and the feature epoch are the same
    iteration (the feature form's W = X' A): the dual variables agree to the
    rounding of the scores (the feature form also skips W updates below
    epsilon, which these well-scaled updates never are)."""
    import torch
    import libsdca_amd as sd
    rng = np.random.default_rng(8)
    n, d, m = 400, 48, 30
    X = rng.standard_normal((n, d))
    X /= np.linalg.norm(X, axis=1, keepdims=True)
    y = rng.integers(0, m, n)
    Xt = torch.from_numpy(X).to(cuda)
    Kt = Xt @ Xt.T
    W = torch.zeros((m, d), dtype=torch.float64, device=cuda)
    Af = torch.zeros((n, m), dtype=torch.float64, device=cuda)
    Ak = torch.zeros((n, m), dtype=torch.float64, device=cuda)
    obj = ("l2_entropy_topk", 1.0, 1.0, 3)
    for e in range(2):
        order = sd.epoch_order(n, e)
        sd.epoch_features(obj, Xt, W, Af, y, order=order)
        sd.epoch_kernel(obj, Kt, Ak, y, order=order)
    torch.cuda.synchronize()
    err = float((Af - Ak).abs().max())
    print(f"|A_features - A_kernel| {err:.2e}", flush=True)
    assert err <= 1e-10
    assert float((W - Af.T @ Xt).abs().max()) <= 1e-10
