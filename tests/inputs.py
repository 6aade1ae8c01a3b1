"""Seeded input generators shared by the parity tests and the bench.

Columns are rows of a C-contiguous (n, m) array (the reference's column-major
m x n matrix).  The decade sweeps follow the reference tests'
test_populate_real (test/test_util.h:31-51): uniforms in [10^p, 10^(p+1))
times a sign.
"""
import numpy as np


def normal(n, m, dtype, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal((n, m)) * scale).astype(dtype)


def uniform(n, m, dtype, seed, lo, hi):
    return np.random.default_rng(seed).uniform(lo, hi, (n, m)).astype(dtype)


def label_shifted(n, m, dtype, seed, shift=2.0):
    """N(0,1) with one uniformly drawn label row per column shifted by +shift
    (the top-k simplex benchmark input)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, m))
    lab = rng.integers(0, m, n)
    x[np.arange(n), lab] += shift
    return x.astype(dtype)


def decades(n, m, dtype, seed, pow_from, pow_to, sign=1.0):
    """Each column draws its magnitude decade uniformly in [pow_from, pow_to)."""
    rng = np.random.default_rng(seed)
    p = rng.integers(pow_from, pow_to, (n, 1)).astype(np.float64)
    u = rng.uniform(0, 1, (n, m))
    x = sign * (10.0 ** p) * (1.0 + 9.0 * u)
    return x.astype(dtype)


def decade_blocks(n, m, dtype, seed, pow_from, pow_to, block=25):
    """Columns made of consecutive blocks of `block` entries, block b drawn
    from decade pow_from + (b // 2) % (pow_to - pow_from) with sign + for
    even b and - for odd b: the concatenated vectors of the reference tests
    (test_populate_real called per decade with coeff = +1 then -1, e.g.
    test/prox/topk_simplex.cpp and test/prox/knapsack_eq.cpp)."""
    rng = np.random.default_rng(seed)
    b = np.arange(m) // block
    p = pow_from + (b // 2) % (pow_to - pow_from)
    sign = np.where(b % 2 == 0, 1.0, -1.0)
    u = rng.uniform(0, 1, (n, m))
    x = sign * (10.0 ** p) * (1.0 + 9.0 * u)
    return x.astype(dtype)


def mixed_signs(n, m, dtype, seed, pow_from, pow_to):
    rng = np.random.default_rng(seed)
    s = rng.choice([-1.0, 1.0], (n, m))
    return (decades(n, m, np.float64, seed + 1, pow_from, pow_to) * s).astype(dtype)


def edge_columns(m, dtype, seed=0):
    """Hand-made columns: ties, constants, zeros, tiny and huge values."""
    rng = np.random.default_rng(seed)
    cols = [
        np.zeros(m),
        np.ones(m),
        -np.ones(m),
        np.full(m, 0.5),
        np.linspace(-1, 1, m),
        np.linspace(1, -1, m),
        np.resize(np.repeat(rng.standard_normal(max(1, m // 4)), 4), m),
        np.where(np.arange(m) % 2 == 0, 1.0, -1.0),
        rng.standard_normal(m) * 1e-6,
        rng.standard_normal(m) * 1e6,
        np.concatenate([[10.0], np.zeros(m - 1)]) if m > 1 else np.array([10.0]),
        np.concatenate([np.full(min(m, 3), 2.0), -np.ones(m - min(m, 3))]),
        rng.integers(-3, 4, m).astype(np.float64),
    ]
    return np.stack(cols).astype(dtype)
