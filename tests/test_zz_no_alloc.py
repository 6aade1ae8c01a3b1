"""sdca_prox_noalloc through the C ABI against sdca_prox.

The entry point without allocation shares every kernel with sdca_prox and
differs only in where the deferred-column list lives (a fixed device array
of the library instead of the per-stream workspace), so its outputs and
threshold records must equal sdca_prox's bit for bit.  Two calls in a row,
the second smaller, check that the shared array's state from one call does
not leak into the next; the top-k cone input has columns that take the
deferred path.
"""
import ctypes

import numpy as np
import pytest

from tests import inputs

pytestmark = pytest.mark.gpu


def _abi():
    import libsdca_amd as sd
    lib = sd.library()
    lib.sdca_prox_noalloc.restype = ctypes.c_int
    lib.sdca_prox_noalloc.argtypes = [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(sd.ProxParams), ctypes.c_void_p,
        ctypes.c_void_p, ctypes.c_void_p]
    lib.sdca_prox_noalloc_max_columns.restype = ctypes.c_int64
    return sd, lib


def _run(lib, fn, op, x, params, stream, col_p=None):
    import torch
    n, m = x.shape
    out = torch.empty_like(x)
    thr = torch.zeros((2 * n, 3), dtype=torch.float64, device=x.device)
    data = 0 if x.dtype == torch.float32 else 1
    rc = fn(op, data, data, m, n, ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
            ctypes.byref(params), ctypes.c_void_p(col_p.data_ptr() if col_p is not None else None),
            ctypes.c_void_p(thr.data_ptr()), *([ctypes.c_uint(0)] if fn is lib.sdca_prox else []),
            stream)
    assert rc == 0, lib.sdca_last_error().decode()
    return out, thr


CASES = [
    # op, m, n of the first call, n of the second call, k, input
    ("topk_simplex", 100, 300_000, 70_000, 5, "label"),
    ("topk_cone", 100, 200_000, 30_000, 5, "cone"),
    ("two_simplex_sort", 40, 120_000, 9_000, 1, "normal"),
    ("knapsack_eq", 10, 100_000, 1_000, 1, "normal"),
]


@pytest.mark.parametrize("op,m,n1,n2,k,gen", CASES)
def test_noalloc_matches_prox(cuda, op, m, n1, n2, k, gen):
    import torch
    sd, lib = _abi()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    params = sd.ProxParams(0.0, 1.0, 1.0, 1.0, 1.0, k, 1)
    code = sd.OPS[op]
    for n in (n1, n2):
        print(f"{op} m={m} n={n}", flush=True)
        if gen == "label":
            x = inputs.label_shifted(n, m, np.float32, 900 + n % 97)
        elif gen == "cone":
            # columns with a few large entries: some need the sorted cone search
            x = inputs.normal(n, m, np.float32, 901 + n % 97)
            x[::7, :3] += 4.0
        else:
            x = inputs.normal(n, m, np.float32, 902 + n % 97)
        t = torch.from_numpy(x).to(cuda)
        col_p = None
        if op == "two_simplex_sort":
            col_p = torch.from_numpy(np.random.default_rng(n).integers(1, 6, n)).to(cuda)
        want, want_thr = _run(lib, lib.sdca_prox, code, t, params, stream, col_p)
        got, got_thr = _run(lib, lib.sdca_prox_noalloc, code, t, params, stream, col_p)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{op} n={n}: outputs differ"
        assert torch.equal(got_thr, want_thr), f"{op} n={n}: threshold records differ"


def test_noalloc_rejects_oversized(cuda):
    """More columns than the fixed list holds: a clear error, nothing launched."""
    import torch
    sd, lib = _abi()
    cap = int(lib.sdca_prox_noalloc_max_columns())
    assert cap == 4_194_304
    params = sd.ProxParams(0.0, 1.0, 1.0, 1.0, 1.0, 5, 1)
    # A real (cap + 1) x 100 batch (1.7 GB): rejected before any launch.
    x = torch.zeros((cap + 1, 100), dtype=torch.float32, device=cuda)
    rc = lib.sdca_prox_noalloc(sd.OPS["topk_simplex"], 0, 0, 100, cap + 1,
                               ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                               ctypes.byref(params), None, None,
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 2
    assert "fixed scratch" in lib.sdca_last_error().decode()


def test_noalloc_allocates_nothing_on_a_fresh_stream(cuda):
    """The property the entry point exists for: its first call on a stream
    the library has never used allocates no device memory (the free memory
    the driver reports is unchanged), where sdca_prox's first call on such a
    stream allocates that stream's deferred-column list (the control, which
    shows the measurement can see an allocation of that size).  Each stream
    runs one torch kernel first: the runtime sets up a new stream's hardware
    queue (2 MiB of device memory) at its first launch, whoever launches."""
    import torch
    sd, lib = _abi()
    n, m = 2_000_000, 100
    x = torch.from_numpy(inputs.label_shifted(n, m, np.float32, 905)).to(cuda)
    params = sd.ProxParams(0.0, 1.0, 1.0, 1.0, 1.0, 5, 1)
    code = sd.OPS["topk_simplex"]
    # Load the kernels' code first (the runtime's own one-time cost of any
    # first launch), on a stream of its own.
    warm = torch.cuda.Stream()
    _run(lib, lib.sdca_prox_noalloc, code, x[:1000].contiguous(), params,
         ctypes.c_void_p(warm.cuda_stream))
    out = torch.empty_like(x)
    thr = torch.zeros((n, 3), dtype=torch.float64, device=cuda)
    torch.cuda.synchronize()

    def free_after(fn, stream):
        torch.cuda.synchronize()
        before = torch.cuda.mem_get_info()[0]
        rc = fn(code, 0, 0, m, n, ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                ctypes.byref(params), None, ctypes.c_void_p(thr.data_ptr()),
                *([ctypes.c_uint(0)] if fn is lib.sdca_prox else []),
                ctypes.c_void_p(stream.cuda_stream))
        assert rc == 0, lib.sdca_last_error().decode()
        torch.cuda.synchronize()
        return before - torch.cuda.mem_get_info()[0]

    def new_stream():
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            torch.zeros(1, device=cuda).add_(1.0)
        torch.cuda.synchronize()
        return st

    fresh = new_stream()
    assert free_after(lib.sdca_prox_noalloc, fresh) == 0
    control = new_stream()
    grown = free_after(lib.sdca_prox, control)
    print(f"sdca_prox on a fresh stream took {grown} bytes")
    assert grown >= 4 * n  # its list of n column indices
