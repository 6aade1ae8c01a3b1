"""GPU parity of the batched prox operators against the CPU oracle.

Every case runs the HIP path through the C ABI (libsdca_amd.prox on torch
CUDA tensors, or numpy through the host-staging path) and the oracle
restatement (bit-exact with the reference headers) on the same seeded input,
and compares the projected columns elementwise, scaled by the column
magnitude s = max(1, max|a|):

  * |gpu - ref| / s <= rtol + 3 E, and
  * |gpu - exact| / s <= rtol + 2 E (the GPU is at least as accurate as the
    reference),

with rtol = 1e-5 when the arithmetic (Result) type or the element (Data) type
is float and 1e-12 when both are double (the north star's tolerances), "exact" the same algorithm run by the
oracle in long double, and E = max over the batch of |ref - exact| / s: the
reference's own rounding error.  E is not a fudge factor: the thresholds come
from sums of m terms whose rounding depends on summation order (the
reference's std::partition order is not reproducible in parallel), and for
float at m = 1000 the reference itself is ~2e-4 away from the exact
projection, so a flat 1e-5 would fail any implementation that sums in another
order.  E is printed for every case that needs it.
"""
import numpy as np
import pytest

from tests import inputs

pytestmark = pytest.mark.gpu

F32, F64 = 0, 1
RTOL = {F32: 1e-5, F64: 1e-12}


def run_gpu(op, x, result, cuda, **kw):
    import torch
    import libsdca_amd as sd
    t = torch.from_numpy(x).to(cuda)
    out, thr = sd.prox(op, t, result=result, thresholds=True, **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy(), thr.cpu().numpy()


def run_oracle(oracle, op, x, result, nthreads=1, **kw):
    from oracle import binding
    y = x.copy()
    col_p = kw.pop("col_p", None)
    thr = oracle.prox(op, y, result=result, params=binding.make_params(**kw), col_p=col_p,
                      thresholds=op != "lambert_w_exp", nthreads=nthreads)
    return y, thr


LONG_DOUBLE = 2


def parity(oracle, op, x, got, result, what, nthreads=1, keep=None, **kw):
    """Check got (GPU) against the oracle at the Result type and in long double
    (over the columns `keep` selects, all by default)."""
    ref, _ = run_oracle(oracle, op, x, result, nthreads, **dict(kw))
    exact, _ = run_oracle(oracle, op, x, LONG_DOUBLE, nthreads, **dict(kw))
    if keep is not None:
        x, got, ref, exact = x[keep], got[keep], ref[keep], exact[keep]
    scale = np.maximum(1.0, np.abs(x.astype(np.float64)).max(axis=1, keepdims=True))
    g = got.astype(np.float64)
    r = ref.astype(np.float64)
    e = exact.astype(np.float64)
    d_ref = np.abs(g - r) / scale
    err_gpu = np.abs(g - e) / scale
    err_ref = float((np.abs(r - e) / scale).max())
    # Outputs are stored in the Data type: float data caps the precision.
    rtol = max(RTOL[result], RTOL[F32] if x.dtype == np.float32 else RTOL[F64])
    bad = np.argwhere(d_ref > rtol + 3 * err_ref)
    assert bad.size == 0, (
        f"{what}: {len(np.unique(bad[:, 0]))} columns differ from the reference, max scaled "
        f"err {d_ref.max():.3e} (reference error E={err_ref:.3e}); column {bad[0, 0]}: "
        f"got {got[bad[0, 0]][:6]} want {ref[bad[0, 0]][:6]}")
    assert err_gpu.max() <= rtol + 2 * err_ref, (
        f"{what}: GPU error vs exact {err_gpu.max():.3e} exceeds rtol + 2E "
        f"(E={err_ref:.3e})")
    if d_ref.max() > rtol:
        print(f"{what}: max |gpu-ref|/s {d_ref.max():.2e} within rtol + 3E, E={err_ref:.2e}")


DTYPES = [(np.float32, F32), (np.float32, F64), (np.float64, F64)]
# One m per register configuration (G lanes x C slots), plus the sizes of the
# benchmark configurations.
MS = [1, 3, 10, 16, 17, 64, 100, 101, 128, 150, 200, 512, 999, 1000, 2048]


def cases(m, dtype, seed):
    n = 300
    yield "normal", inputs.normal(n, m, dtype, seed)
    yield "label+2", inputs.label_shifted(n, m, dtype, seed + 1)
    yield "pos", inputs.decades(n, m, dtype, seed + 2, -3, 3)
    yield "neg", inputs.decades(n, m, dtype, seed + 3, -3, 3, sign=-1.0)
    yield "mixed", inputs.mixed_signs(n, m, dtype, seed + 4, -3, 3)
    yield "decade blocks", inputs.decade_blocks(n, m, dtype, seed + 6, -3, 3,
                                                block=max(1, min(25, m // 4)))
    yield "edge", inputs.edge_columns(m, dtype, seed + 5)


@pytest.mark.parametrize("dtype,result", DTYPES)
@pytest.mark.parametrize("m", MS)
@pytest.mark.parametrize("op,kw", [
    ("knapsack_eq", dict(lo=0.0, hi=1.0, rhs=1.0)),
    ("knapsack_eq", dict(lo=-0.5, hi=0.25, rhs=0.7)),
    ("knapsack_le", dict(lo=0.0, hi=0.3, rhs=1.0)),
])
def test_knapsack(cuda, oracle, op, kw, m, dtype, result):
    if kw["hi"] * m < kw["rhs"] or kw["lo"] * m > kw["rhs"]:
        pytest.skip("infeasible bounds for this m")
    for name, x in cases(m, dtype, 10 + m):
        got, _ = run_gpu(op, x, result, cuda, **kw)
        parity(oracle, op, x, got, result, f"{op} {name} m={m}", **kw)


@pytest.mark.parametrize("dtype,result", DTYPES)
@pytest.mark.parametrize("m", MS)
@pytest.mark.parametrize("op", ["topk_simplex", "topk_cone"])
@pytest.mark.parametrize("k", [1, 2, 5, 8, 11])
def test_topk(cuda, oracle, op, k, m, dtype, result):
    if k > m:
        pytest.skip("k > m")
    kw = dict(k=k, rhs=1.0)
    for name, x in cases(m, dtype, 20 + m + k):
        got, _ = run_gpu(op, x, result, cuda, **kw)
        parity(oracle, op, x, got, result, f"{op} k={k} {name} m={m}", **kw)


@pytest.mark.parametrize("dtype,result", DTYPES)
@pytest.mark.parametrize("m", MS)
@pytest.mark.parametrize("k,rhs", [(5, 30.0), (2, 7.0), (11, 400.0)])
def test_topk_simplex_many_candidates(cuda, oracle, k, rhs, m, dtype, result):
    """A large rhs (hi = rhs / k) makes most of the column candidates for the
    knapsack: the variable fixing then runs over every slot, with its working
    copy in the column's LDS slots instead of the candidate registers."""
    if k > m:
        pytest.skip("k > m")
    kw = dict(k=k, rhs=rhs)
    for name, x in cases(m, dtype, 40 + m + k):
        got, _ = run_gpu("topk_simplex", x, result, cuda, **kw)
        parity(oracle, "topk_simplex", x, got, result, f"topk_simplex k={k} rhs={rhs} {name} m={m}",
               **kw)


@pytest.mark.parametrize("dtype,result", DTYPES)
@pytest.mark.parametrize("m", [1, 10, 100, 200, 1000, 2048])
@pytest.mark.parametrize("op,kw", [
    ("entropy", dict(hi=1.0, rhs=1.0)),
    ("entropy", dict(hi=0.1, rhs=0.5)),
    ("entropy_norm", dict(hi=1.0, rhs=1.0)),
    ("entropy_norm", dict(hi=0.2, rhs=0.9)),
])
def test_entropic(cuda, oracle, op, kw, m, dtype, result):
    if kw["hi"] * m < kw["rhs"]:
        pytest.skip("infeasible bounds for this m")
    n = 200
    for name, x in [("uniform", inputs.uniform(n, m, dtype, 30 + m, -10, 10)),
                    ("normal", inputs.normal(n, m, dtype, 31 + m, 3.0)),
                    ("edge", inputs.edge_columns(m, dtype, 32 + m))]:
        got, _ = run_gpu(op, x, result, cuda, **kw)
        parity(oracle, op, x, got, result, f"{op} {name} m={m}", **kw)


@pytest.mark.parametrize("dtype,result", DTYPES)
@pytest.mark.parametrize("m", [2, 10, 100, 999])
@pytest.mark.parametrize("k", [1, 3, 5, 12])
def test_topk_entropy(cuda, oracle, k, m, dtype, result):
    if k > m:
        pytest.skip("k > m")
    n = 200
    for name, x in [("normal", inputs.normal(n, m, dtype, 40 + m, 2.0)),
                    ("label+2", inputs.label_shifted(n, m, dtype, 41 + m)),
                    ("edge", inputs.edge_columns(m, dtype, 42 + m))]:
        got, _ = run_gpu("topk_entropy", x, result, cuda, k=k)
        parity(oracle, "topk_entropy", x, got, result, f"topk_entropy k={k} {name} m={m}", k=k)


@pytest.mark.parametrize("dtype,result", DTYPES)
@pytest.mark.parametrize("m", [2, 10, 159, 200, 1000])
def test_two_simplex(cuda, oracle, m, dtype, result):
    n = 300
    rng = np.random.default_rng(50 + m)
    col_p = rng.integers(1, min(m - 1, 5) + 1, n)
    for rhs in [1.0, 2.0]:
        for name, x in [("normal", inputs.normal(n, m, dtype, 51 + m)),
                        ("mixed", inputs.mixed_signs(n, m, dtype, 52 + m, -2, 2))]:
            got, _ = run_gpu("two_simplex", x, result, cuda, rhs=rhs, col_p=col_p)
            parity(oracle, "two_simplex", x, got, result, f"two_simplex rhs={rhs} {name} m={m}", rhs=rhs, col_p=col_p)
            # scalar p for every column
            got, _ = run_gpu("two_simplex", x, result, cuda, rhs=rhs, p=1)
            parity(oracle, "two_simplex", x, got, result, f"two_simplex p=1 rhs={rhs} {name} m={m}", rhs=rhs, p=1)


def test_two_simplex_regression_vector(cuda, oracle):
    """The hard-coded vector of test/prox/two_simplex.cpp:55-64 (p=1, rhs=2)."""
    x = np.array([[-0.49371069182389915] + [0.49371069182390021] * 158], dtype=np.float64)
    got, _ = run_gpu("two_simplex", x, F64, cuda, rhs=2.0, p=1)
    parity(oracle, "two_simplex", x, got, F64, "two_simplex regression vector", rhs=2.0, p=1)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_lambert_w_exp(cuda, oracle, dtype):
    rng = np.random.default_rng(60)
    x = rng.uniform(-50, 50, (1, 100000)).astype(dtype)
    edges = np.array([-1e4, -746, -745.9, -104, -36, -20, -18, -1, 0, 4, 8, 2.0**29, 2.0**59,
                      1e20, 36.5, -0.5], dtype=dtype)
    x = np.concatenate([x, edges[None, :]], axis=1)
    got, _ = run_gpu_plain("lambert_w_exp", x, cuda)
    want = oracle.lambert_w_exp(x).reshape(x.shape)
    r = F32 if dtype == np.float32 else F64
    tol = {F32: 4e-7, F64: 4e-16}[r]
    err = np.abs(got.astype(np.float64) - want) / np.maximum(1.0, np.abs(want))
    assert err.max() <= tol, f"max rel err {err.max():.3e}"


@pytest.mark.parametrize("lo,hi", [(-708.0, -36.0), (-745.5, -708.0)])
def test_exp_through_lambert_tail(cuda, lo, hi):
    """On (-746, -36] the double Lambert map returns e^x itself
    (math/lambert.h:153): the kernels' double exponential, held here to
    2 ulp of numpy's (1 ulp of the smallest subnormal below 2^-1022)."""
    rng = np.random.default_rng(61)
    x = rng.uniform(lo, hi, (1, 200000))
    x[0, :3] = [lo, hi, np.nextafter(hi, 0.0)]
    got, _ = run_gpu_plain("lambert_w_exp", x, cuda)
    want = np.exp(x)
    ulp = np.spacing(want)
    err = np.abs(got - want) / ulp
    normal = want >= np.finfo(np.float64).tiny
    assert err[normal].max(initial=0.0) <= 2.0, f"max {err[normal].max():.2f} ulp"
    assert err[~normal].max(initial=0.0) <= 1.0, f"subnormal max {err[~normal].max():.2f} ulp"


def run_gpu_plain(op, x, cuda):
    import torch
    import libsdca_amd as sd
    t = torch.from_numpy(x).to(cuda)
    sd.prox(op, t)
    torch.cuda.synchronize()
    return t.cpu().numpy(), None


def test_host_pointer_path(oracle):
    """numpy in, numpy out through the library's own staging."""
    import libsdca_amd as sd
    x = inputs.label_shifted(1000, 100, np.float32, 70)
    got = x.copy()
    sd.prox_topk_simplex(100, got, k=5, rhs=1.0)
    parity(oracle, "topk_simplex", x, got, F32, "host path topk_simplex", k=5, rhs=1.0)


def test_out_of_place(cuda, oracle):
    import torch
    import libsdca_amd as sd
    x = inputs.normal(5000, 10, np.float64, 71)
    t = torch.from_numpy(x).to(cuda)
    o = torch.empty_like(t)
    sd.prox("knapsack_eq", t, out=o)
    torch.cuda.synchronize()
    assert np.array_equal(t.cpu().numpy(), x), "input modified by an out-of-place call"
    parity(oracle, "knapsack_eq", x, o.cpu().numpy(), F64, "out of place knapsack_eq")


def test_deferred_list_reuse(cuda, oracle):
    """Consecutive calls on one stream share the deferred-column list, whose
    counters the deferred-column kernel resets: a call with many deferred
    columns (top-k cone with one dominant entry per column: the cone search
    with U non-empty), a smaller one, then one with none, each against the
    oracle."""
    rng = np.random.default_rng(77)
    for n in (5000, 300, 4000):
        x = rng.standard_normal((n, 50)).astype(np.float32)
        if n != 4000:
            x[np.arange(n), rng.integers(0, 50, n)] += 40.0
        for op in ("topk_cone", "topk_simplex"):
            got, _ = run_gpu(op, x, F32, cuda, k=5)
            parity(oracle, op, x, got, F32, f"{op} n={n}", k=5)


@pytest.mark.parametrize("dtype,result", DTYPES)
@pytest.mark.parametrize("m", [2049, 3000, 4096])
@pytest.mark.parametrize("op,kw", [
    ("knapsack_eq", dict(lo=0.0, hi=1.0, rhs=1.0)),
    ("knapsack_le", dict(lo=-0.5, hi=0.3, rhs=2.0)),
    ("topk_simplex", dict(k=5, rhs=1.0)),
    ("topk_cone", dict(k=3)),
])
def test_large_m_workgroup_per_column(cuda, oracle, op, kw, m, dtype, result):
    """m beyond the register kernel (2048): one workgroup per column, the
    column sorted in LDS."""
    n = 40
    for name, x in [("normal", inputs.normal(n, m, dtype, 90 + m)),
                    ("label+2", inputs.label_shifted(n, m, dtype, 91 + m)),
                    ("edge", inputs.edge_columns(m, dtype, 92 + m))]:
        got, _ = run_gpu(op, x, result, cuda, **kw)
        parity(oracle, op, x, got, result, f"{op} {name} m={m}", **kw)


def test_large_m_limits(cuda):
    """Sizes past the workgroup-per-column kernel's LDS, and the operators
    without it, are refused with SDCA_ERR_NOT_IMPLEMENTED (4)."""
    import torch
    import libsdca_amd as sd
    for op, m, dt in [("topk_simplex", 8193, torch.float32), ("knapsack_eq", 4097, torch.float64),
                      ("entropy", 2049, torch.float64), ("two_simplex", 2049, torch.float32)]:
        x = torch.zeros((3, m), dtype=dt, device=cuda)
        with pytest.raises(sd.SdcaError) as e:
            sd.prox(op, x, k=5, p=1)
        assert e.value.status == 4, op


@pytest.mark.parametrize("dtype,result", DTYPES)
@pytest.mark.parametrize("m", [1, 5, 17, 100, 1000])
@pytest.mark.parametrize("op,kw", [
    ("knapsack_le_biased", dict(lo=0.0, hi=1.0, rhs=1.0, rho=1.0)),
    ("knapsack_le_biased", dict(lo=-0.5, hi=0.3, rhs=2.0, rho=0.5)),
    ("knapsack_le_biased", dict(lo=0.0, hi=1.0, rhs=1.0, rho=0.0)),
    ("topk_simplex_biased", dict(k=1, rhs=1.0, rho=1.0)),
    ("topk_simplex_biased", dict(k=5, rhs=1.0, rho=0.5)),
    ("topk_cone_biased", dict(k=1, rho=1.0)),
    ("topk_cone_biased", dict(k=3, rho=0.25)),
])
def test_biased(cuda, oracle, op, kw, m, dtype, result):
    """The biased operators (rho <1,x>^2 / 2 added to the objective), one
    workgroup per sorted column."""
    if kw.get("k", 1) > m:
        pytest.skip("k > m")
    for name, x in cases(m, dtype, 110 + m):
        got, thr = run_gpu(op, x, result, cuda, **kw)
        parity(oracle, op, x, got, result, f"{op} {name} m={m}", **kw)


@pytest.mark.parametrize("dtype,result", DTYPES)
@pytest.mark.parametrize("m", [2, 10, 159, 200, 1000, 3000])
def test_two_simplex_sort(cuda, oracle, m, dtype, result):
    """The sort-and-scan two-block simplex (the register kernel, with the
    columns whose optimum is zero deferred to the sort-and-scan kernel, and
    that kernel alone for m > 2048), with a per-column and a common split p."""
    n = 120
    rng = np.random.default_rng(150 + m)
    col_p = rng.integers(1, min(m - 1, 5) + 1, n)
    for rhs in [1.0, 2.0]:
        neg = -np.abs(inputs.normal(n, m, dtype, 153 + m)) - dtype(0.1)  # optimum x = y = 0
        neg[::2] = inputs.normal(n // 2, m, dtype, 154 + m)  # interleaved with ordinary columns
        for name, x in [("normal", inputs.normal(n, m, dtype, 151 + m)),
                        ("mixed", inputs.mixed_signs(n, m, dtype, 152 + m, -2, 2)),
                        ("zero-optimum", np.ascontiguousarray(neg))]:
            got, _ = run_gpu("two_simplex_sort", x, result, cuda, rhs=rhs, col_p=col_p)
            parity(oracle, "two_simplex_sort", x, got, result,
                   f"two_simplex_sort rhs={rhs} {name} m={m}", rhs=rhs, col_p=col_p)
            p = max(1, m // 3)
            got, _ = run_gpu("two_simplex_sort", x, result, cuda, rhs=rhs, p=p)
            parity(oracle, "two_simplex_sort", x, got, result,
                   f"two_simplex_sort p={p} rhs={rhs} {name} m={m}", rhs=rhs, p=p)


def entbias_settled(oracle, x, alpha, result):
    """Columns on which the reference's uncapped solve ends on a root.

    That solve (topk_entropy_biased.h:48-61) does not depend on k, so its
    iterate t is the threshold of the k = 1 result.  It should be a root of
    g(t) = W(e^(alpha - t)) + sum_i W(e^(a_i - t)) - alpha.  From a start far
    below the root (every entry far below zero) the order-4 correction can
    point away from it, and the reference returns its 32nd iterate.  Where that
    path hinges on the rounding of the sums, no other summation order can
    reproduce the iterate, so those columns have no parity target and are left
    out.  A settled iterate has |g| at rounding level (that of t itself
    included: |g'(t)| * 8 eps |t|); the cut at 1e-3 of the sum's size above it
    is far from both that and an unsettled iterate's |g| ~ alpha.
    """
    _, thr = run_oracle(oracle, "topk_entropy_biased", x, result, 8, k=1, alpha=alpha)
    return entbias_is_root(oracle, x, alpha, result, thr[:, 0])


def entbias_is_root(oracle, x, alpha, result, t):
    """|g(t)| at rounding level, column by column (g as in entbias_settled)."""
    z = np.concatenate([x.astype(np.float64) - t[:, None],
                        (alpha - t)[:, None]], axis=1)
    oracle.prox("lambert_w_exp", z)
    total = z.sum(axis=1)
    slope = (z / (1 + z)).sum(axis=1)
    eps = np.finfo(np.float32 if result == F32 else np.float64).eps
    return np.abs(total - alpha) <= 1e-3 * (alpha + total) + 8 * eps * np.abs(t) * slope


@pytest.mark.parametrize("dtype,result", DTYPES)
@pytest.mark.parametrize("m", [1, 5, 17, 64, 100, 1000])
@pytest.mark.parametrize("k,alpha", [(1, 1.0), (3, 0.5), (5, 2.0)])
def test_topk_entropy_biased(cuda, oracle, k, alpha, m, dtype, result):
    """Biased top-k entropy, one wave per column (both the uncapped
    Householder solve and the growing capped set)."""
    if k > m:
        pytest.skip("k > m")
    for name, x in cases(m, dtype, 170 + m):
        if name == "label+2":
            x = x.copy()
            x[: len(x) // 2, :2] += 6.0  # dominant entries: the capped branch
        keep = entbias_settled(oracle, x, alpha, result)
        assert keep.mean() >= 0.95, f"{name}: {np.count_nonzero(~keep)} unsettled columns"
        if not keep.all():
            print(f"topk_entropy_biased {name} m={m}: {np.count_nonzero(~keep)} of {len(keep)} "
                  f"columns where the reference's uncapped solve ends unsettled")
        got, thr = run_gpu("topk_entropy_biased", x, result, cuda, k=k, alpha=alpha)
        parity(oracle, "topk_entropy_biased", x, got, result,
               f"topk_entropy_biased k={k} alpha={alpha} {name} m={m}", nthreads=8, keep=keep,
               k=k, alpha=alpha)
        if k == 1 and not keep.all():
            # Where the reference stops short, the GPU's threshold is a root.
            assert entbias_is_root(oracle, x[~keep], alpha, result, thr[~keep, 0]).all()


@pytest.mark.parametrize("dtype,result,m", [(np.float32, F32, 8192), (np.float64, F64, 4096)])
def test_topk_entropy_biased_largest_m(cuda, oracle, dtype, result, m):
    x = inputs.normal(16, m, dtype, 180, 2.0)
    x[:8, :3] += 8.0
    assert entbias_settled(oracle, x, 1.5, result).all()
    got, _ = run_gpu("topk_entropy_biased", x, result, cuda, k=4, alpha=1.5)
    parity(oracle, "topk_entropy_biased", x, got, result, f"topk_entropy_biased m={m}",
           nthreads=8, k=4, alpha=1.5)


@pytest.mark.parametrize("dtype,result", DTYPES)
@pytest.mark.parametrize("m", [2, 5, 17, 100, 200, 1000])
@pytest.mark.parametrize("alpha", [1.0, 0.3, 4.0])
def test_two_entropy(cuda, oracle, alpha, m, dtype, result):
    """The two-block entropic projection of the multilabel entropy dual, one
    wave per column, with a per-column and a common split p."""
    n = 150
    rng = np.random.default_rng(190 + m)
    col_p = rng.integers(1, min(m - 1, 5) + 1, n)
    for name, x in [("normal", inputs.normal(n, m, dtype, 191 + m)),
                    ("mixed", inputs.mixed_signs(n, m, dtype, 192 + m, -2, 2)),
                    ("uniform", inputs.uniform(n, m, dtype, 193 + m, -10, 10))]:
        got, thr = run_gpu("two_entropy", x, result, cuda, alpha=alpha, col_p=col_p)
        parity(oracle, "two_entropy", x, got, result, f"two_entropy alpha={alpha} {name} m={m}",
               nthreads=8, alpha=alpha, col_p=col_p)
        p = max(1, m // 3)
        got, _ = run_gpu("two_entropy", x, result, cuda, alpha=alpha, p=p)
        parity(oracle, "two_entropy", x, got, result,
               f"two_entropy p={p} alpha={alpha} {name} m={m}", nthreads=8, alpha=alpha, p=p)
