"""Seeded random cases of the batched prox operators: operator, column length
m (drawn mostly next to the kernel's register-configuration edges G*C, where
the slot padding and the LDS slack change), batch size n (not a multiple of
the columns per workgroup), element and arithmetic types, parameters and
input family, each checked against the oracle with the tolerances of
tests/test_prox_gpu.py.  The case list is fixed by the seed, so a failing
case is reproduced by its index.
"""
import numpy as np
import pytest

from tests import inputs
from tests.test_prox_gpu import DTYPES, parity, run_gpu

pytestmark = pytest.mark.gpu

# Register configurations of the column kernel: m <= G * C for each (G, C).
EDGES = [16, 64, 100, 128, 200, 256, 512, 1024, 2048]
OPS = ["knapsack_eq", "knapsack_le", "topk_simplex", "topk_cone", "entropy", "entropy_norm",
       "topk_entropy", "two_simplex", "knapsack_le_biased", "topk_simplex_biased",
       "topk_cone_biased", "two_simplex_sort"]
N_CASES = 240


def draw_case(i):
    rng = np.random.default_rng(1000 + i)
    op = OPS[i % len(OPS)]
    if rng.random() < 0.7:
        e = int(rng.choice(EDGES))
        m = int(np.clip(e + rng.integers(-3, 2), 1, 2048))
    else:
        m = int(rng.integers(1, 2049))
    if op in ("two_simplex", "two_simplex_sort"):
        m = max(m, 2)
    n = int(rng.integers(1, 400))
    dtype, result = DTYPES[int(rng.integers(0, len(DTYPES)))]
    kw = {}
    if op in ("knapsack_eq", "knapsack_le", "knapsack_le_biased"):
        lo = float(rng.choice([0.0, -0.5]))
        hi = float(rng.choice([1.0, 0.3, 2.0]))
        rhs = float(rng.choice([1.0, 0.7, 3.0]))
        if op == "knapsack_eq" and not (lo * m <= rhs <= hi * m):
            rhs = 0.5 * (lo + hi) * m
        kw = dict(lo=lo, hi=hi, rhs=rhs)
        if op == "knapsack_le_biased":
            kw["rho"] = float(rng.choice([0.0, 0.5, 1.0, 4.0]))
    elif op in ("topk_simplex", "topk_cone", "topk_simplex_biased", "topk_cone_biased",
                "topk_entropy"):
        k = int(rng.choice([1, 2, 3, 5, 8, 11]))
        kw = dict(k=min(k, m))
        if op in ("topk_simplex", "topk_simplex_biased"):
            kw["rhs"] = float(rng.choice([1.0, 0.5, 4.0]))
        if op in ("topk_simplex_biased", "topk_cone_biased"):
            kw["rho"] = float(rng.choice([0.5, 1.0, 2.0]))
    elif op in ("entropy", "entropy_norm"):
        hi = float(rng.choice([1.0, 0.2, 0.05]))
        rhs = float(rng.choice([1.0, 0.5]))
        if hi * m < rhs:
            hi = 1.0
        kw = dict(hi=hi, rhs=min(rhs, hi * m))
    elif op in ("two_simplex", "two_simplex_sort"):
        kw = dict(rhs=float(rng.choice([1.0, 2.0])))
        if rng.random() < 0.5:
            kw["col_p"] = rng.integers(1, min(m - 1, 7) + 1, n)
        else:
            kw["p"] = int(rng.integers(1, m))
    family = int(rng.integers(0, 5))
    seed = 2000 + i
    if family == 0:
        x = inputs.normal(n, m, dtype, seed, float(rng.choice([1.0, 3.0])))
    elif family == 1:
        x = inputs.label_shifted(n, m, dtype, seed)
    elif family == 2:
        x = inputs.mixed_signs(n, m, dtype, seed, -3, 3)
    elif family == 3:
        x = inputs.uniform(n, m, dtype, seed, -10.0, 10.0)
    else:
        x = inputs.decade_blocks(n, m, dtype, seed, -3, 3, block=max(1, min(25, m // 4)))
    return op, m, n, result, x, kw


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_case(cuda, oracle, i):
    op, m, n, result, x, kw = draw_case(i)
    host = i % 5 == 0  # every fifth case through the host-pointer staging path
    what = (f"case {i}: {op} m={m} n={n} {x.dtype.name}->{'f32' if result == 0 else 'f64'} {kw}"
            f"{' (host pointers)' if host else ''}")
    print(what, flush=True)
    if host:
        import libsdca_amd as sd
        got = x.copy()
        _, thr = sd.prox(op, got, result=result, thresholds=True, **kw)
    else:
        got, thr = run_gpu(op, x, result, cuda, **kw)
    parity(oracle, op, x, got, result, what, thr=thr, **kw)


N_LAMBERT = 40


@pytest.mark.parametrize("i", range(N_LAMBERT))
def test_random_lambert_map_case(cuda, oracle, i):
    """Seeded random cases of the two Lambert-map operators (biased top-k
    entropy, two-block entropy), with the biased one held to parity on the
    columns where the reference's uncapped solve settles (and to a root
    elsewhere) as in tests/test_prox_gpu.py."""
    from tests.test_prox_gpu import entbias_is_root, entbias_settled
    rng = np.random.default_rng(5000 + i)
    op = "topk_entropy_biased" if i % 2 == 0 else "two_entropy"
    m = int(np.clip(int(rng.choice([64, 100, 200, 256, 1000, 1024])) + rng.integers(-2, 2), 2, 2048))
    n = int(rng.integers(1, 120))
    dtype, result = DTYPES[int(rng.integers(0, len(DTYPES)))]
    alpha = float(rng.choice([0.5, 1.0, 2.0]))
    family = int(rng.integers(0, 3))
    if family == 0:
        x = inputs.normal(n, m, dtype, 6000 + i, 2.0)
    elif family == 1:
        x = inputs.mixed_signs(n, m, dtype, 6000 + i, -2, 2)
    else:
        x = inputs.uniform(n, m, dtype, 6000 + i, -10.0, 10.0)
    what = f"case {i}: {op} m={m} n={n} {x.dtype.name}->{'f32' if result == 0 else 'f64'} alpha={alpha}"
    print(what, flush=True)
    if op == "topk_entropy_biased":
        k = int(min(rng.choice([1, 2, 5]), m))
        keep = entbias_settled(oracle, x, alpha, result)
        assert keep.mean() >= 0.95, f"{what}: {np.count_nonzero(~keep)} unsettled columns"
        got, thr = run_gpu(op, x, result, cuda, k=k, alpha=alpha)
        parity(oracle, op, x, got, result, what + f" k={k}", nthreads=8, keep=keep, k=k,
               alpha=alpha, thr=thr)
        if not keep.all():
            # No parity target where the reference stops short: the GPU's
            # result there is feasible (0 <= x <= sum(x)/k, sum(x) <= 1) and,
            # at k = 1, its threshold is a root.
            g = got[~keep].astype(np.float64)
            tot = g.sum(axis=1)
            eps = 8 * np.finfo(x.dtype).eps
            assert (g >= 0).all() and (tot <= 1 + eps).all(), what
            assert (g <= tot[:, None] / k + eps).all(), what
            if k == 1:
                assert entbias_is_root(oracle, x[~keep], alpha, result, thr[~keep, 0]).all(), what
    else:
        kw = dict(alpha=alpha)
        if rng.random() < 0.5:
            kw["col_p"] = rng.integers(1, min(m - 1, 7) + 1, n)
        else:
            kw["p"] = int(rng.integers(1, m))
        got, thr = run_gpu(op, x, result, cuda, **kw)
        parity(oracle, op, x, got, result, what, nthreads=8, thr=thr, **kw)
