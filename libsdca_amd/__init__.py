"""libsdca_amd - MI355X (gfx950) batched prox operators and evaluation pass.

Python host side of the C ABI in include/sdca_hip.h.  The functions keep the
names and argument meaning of libsdca's batched C++ API
(include/sdca/prox/*.h, the `dim` overloads) and of the Matlab front end's
operator table (src/matlab/mex_prox.cpp:145-172):

    prox_knapsack_eq(dim, A, lo=0, hi=1, rhs=1)
    prox_knapsack_le(dim, A, lo=0, hi=1, rhs=1)
    prox_topk_simplex(dim, A, k=1, rhs=1)
    prox_topk_cone(dim, A, k=1)
    prox_entropy(dim, A, hi=1, rhs=1)
    prox_entropy_norm(dim, A, hi=1, rhs=1)
    prox_topk_entropy(dim, A, k=1)
    prox_two_simplex(dim, p, A, rhs=1)
    prox_knapsack_le_biased(dim, A, lo=0, hi=1, rhs=1, rho=1)
    prox_topk_simplex_biased(dim, A, k=1, rhs=1, rho=1)
    prox_topk_cone_biased(dim, A, k=1, rho=1)
    prox_topk_entropy_biased(dim, A, k=1, alpha=1)
    prox_two_simplex_sort(dim, p, A, rhs=1)
    prox_two_entropy(dim, p, A, alpha=1)
    lambert_w_exp(A)

`A` holds n columns of length dim, contiguous (a C-contiguous (n, dim) array
or tensor, i.e. the column-major dim x n matrix of the reference).  A torch
CUDA tensor is processed in place on the device (stream-ordered on torch's
current stream); a numpy array is staged through device memory and updated in
place.  There is no CPU fallback: without the built HIP library every call
raises.
"""
import ctypes
import os

import numpy as np

__all__ = [
    "SdcaError", "library", "prox", "prox_knapsack_eq", "prox_knapsack_le",
    "prox_topk_simplex", "prox_topk_cone", "prox_entropy", "prox_entropy_norm",
    "prox_topk_entropy", "prox_two_simplex", "prox_knapsack_le_biased",
    "prox_topk_simplex_biased", "prox_topk_cone_biased", "prox_topk_entropy_biased",
    "prox_two_simplex_sort", "prox_two_entropy", "lambert_w_exp", "OPS", "F32", "F64",
    "OBJECTIVES", "objective", "scores", "eval_features", "eval_kernel", "eval_scores",
    "recompute_primal", "epoch_order", "epoch_features", "epoch_kernel", "BRANCHES",
]

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsdca_hip.so")

F32, F64, LONG_DOUBLE = 0, 1, 2
HOST_PTR = 1
OPS = {
    "knapsack_eq": 0, "knapsack": 0, "knapsack_le": 1, "topk_simplex": 2,
    "topk_cone": 3, "entropy": 4, "entropy_norm": 5, "topk_entropy": 6,
    "two_simplex": 7, "lambert_w_exp": 8, "knapsack_le_biased": 9,
    "topk_simplex_biased": 10, "topk_cone_biased": 11,
    "topk_entropy_biased": 12, "two_simplex_sort": 13, "two_entropy": 14,
}
# sdca_prox_branch (include/sdca_hip.h): the return of the threshold
# function that produced a record.
BRANCHES = {
    0: "search", 1: "inactive", 2: "zero", 3: "constant", 4: "knapsack", 5: "scan",
    6: "default", 7: "u_empty", 8: "u_grown", 9: "below_rhs",
}
STATUS = {
    0: "OK", 1: "ARG_NULL", 2: "ARG_RANGE", 3: "PRECISION", 4: "NOT_IMPLEMENTED",
    5: "OUT_OF_MEMORY", 6: "HIP", 7: "PROX", 8: "LABELS",
}


class SdcaError(RuntimeError):
    """A failed C ABI call; .status is the sdca_status code."""

    def __init__(self, status, message):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status


class ProxParams(ctypes.Structure):
    _fields_ = [("lo", ctypes.c_double), ("hi", ctypes.c_double),
                ("rhs", ctypes.c_double), ("rho", ctypes.c_double),
                ("alpha", ctypes.c_double), ("k", ctypes.c_int64),
                ("p", ctypes.c_int64)]


class Thresholds(ctypes.Structure):
    _fields_ = [("t", ctypes.c_double), ("lo", ctypes.c_double), ("hi", ctypes.c_double)]


class Objective(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("c", ctypes.c_double), ("gamma", ctypes.c_double), ("k", ctypes.c_int64)]


class EvalRecord(ctypes.Structure):
    _fields_ = [("primal", ctypes.c_double), ("dual", ctypes.c_double),
                ("primal_loss", ctypes.c_double), ("dual_loss", ctypes.c_double),
                ("primal_regularizer", ctypes.c_double),
                ("dual_regularizer", ctypes.c_double), ("rank_loss", ctypes.c_double)]


# Objectives of the evaluation pass, named after the reference's makers
# (objective.h:55-160: make_objective_l2_hinge_topk, ...).
OBJECTIVES = {
    "l2_hinge_topk": 0, "l2_hinge_topk_smooth": 1, "l2_topk_hinge": 2,
    "l2_topk_hinge_smooth": 3, "l2_entropy": 4, "l2_entropy_topk": 5,
    "l2_multilabel_hinge": 6, "l2_multilabel_hinge_smooth": 7,
    "l2_multilabel_entropy": 8,
}


def objective(name, c=1.0, gamma=1.0, k=1):
    """An objective for eval_features / eval_scores (c = 1 / (lambda n))."""
    return (name, float(c), float(gamma), int(k))


_lib = None


def library():
    """The loaded libsdca_hip.so (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise SdcaError(6, f"{LIB_PATH} is missing: build it with "
                               "`python -c 'import __graft_entry__ as g; g.build()'`")
        # torch ships its own HIP runtime under the same soname; loading torch
        # first makes the library bind to it, so that a process that uses both
        # holds one runtime (two runtimes in one process leave the second
        # without a device).
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        lib = ctypes.CDLL(LIB_PATH)
        lib.sdca_prox.restype = ctypes.c_int
        lib.sdca_prox_with_sets.restype = ctypes.c_int
        lib.sdca_prox.argtypes = [
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ProxParams), ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_uint, ctypes.c_void_p]
        lib.sdca_last_error.restype = ctypes.c_char_p
        lib.sdca_abi_version.restype = ctypes.c_int
        _lib = lib
    return _lib


def check(rc):
    if rc != 0:
        msg = library().sdca_last_error().decode(errors="replace")
        raise SdcaError(rc, msg)


def _is_torch(x):
    return type(x).__module__.startswith("torch")


def _dtype_code(x):
    if _is_torch(x):
        import torch
        return {torch.float32: F32, torch.float64: F64}.get(x.dtype, -1)
    return {np.dtype(np.float32): F32, np.dtype(np.float64): F64}.get(x.dtype, -1)


def _need(x, name, shape, like):
    """Checks that x can be handed to the C ABI beside `like`: the same kind
    (numpy array, or tensor on like's device), like's element type, the given
    shape, contiguous.  The library reads and writes through raw pointers, so
    a mismatch here would otherwise become an out-of-bounds access."""
    if x is None:
        return
    if _is_torch(x) != _is_torch(like):
        raise SdcaError(2, f"{name}: numpy arrays and torch tensors cannot be mixed in one call")
    if _is_torch(x):
        if x.device != like.device:
            raise SdcaError(2, f"{name} is on {x.device}, expected {like.device}")
        contiguous = x.is_contiguous()
    else:
        contiguous = x.flags.c_contiguous
    if x.dtype != like.dtype:
        raise SdcaError(3, f"{name} has element type {x.dtype}, expected {like.dtype}")
    if tuple(int(v) for v in x.shape) != tuple(shape):
        raise SdcaError(2, f"{name} has shape {tuple(x.shape)}, expected {tuple(shape)}")
    if not contiguous:
        raise SdcaError(2, f"{name} must be contiguous")


def _label_arrays(labels, offsets, n, like):
    """int64 label (and CSR offset) arrays of the kind of `like`, with the
    lengths the C ABI reads: n labels, or n + 1 offsets and offsets[n] labels."""
    if _is_torch(like):
        import torch
        lab = torch.as_tensor(labels, dtype=torch.int64, device=like.device).contiguous().reshape(-1)
        off = None if offsets is None else torch.as_tensor(
            offsets, dtype=torch.int64, device=like.device).contiguous().reshape(-1)
    else:
        lab = np.ascontiguousarray(labels, dtype=np.int64).reshape(-1)
        off = None if offsets is None else np.ascontiguousarray(offsets, dtype=np.int64).reshape(-1)
    if off is None:
        if lab.shape[0] != n:
            raise SdcaError(8, f"{lab.shape[0]} labels for {n} examples")
    else:
        if off.shape[0] != n + 1:
            raise SdcaError(8, f"{off.shape[0]} offsets for {n} examples (need n + 1)")
        if int(off[-1]) != lab.shape[0]:
            raise SdcaError(8, f"offsets end at {int(off[-1])} but {lab.shape[0]} labels are given")
        if int(off[0]) != 0:
            raise SdcaError(8, f"offsets start at {int(off[0])}, not 0")
        if n > 0 and bool((off[1:] < off[:-1]).any()):
            raise SdcaError(8, "offsets decrease")
    return lab, off


def _stream_ptr():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def prox(op, A, out=None, result=None, lo=0.0, hi=1.0, rhs=1.0, rho=1.0,
         alpha=1.0, k=1, p=1, col_p=None, thresholds=False, check_col_p=True, sets=False):
    """Batched prox over the rows of A (each row is one column of the
    reference's dim x n matrix).  Returns out (A itself when out is None) and,
    with thresholds=True, an (n, 3) (or (2n, 3) for the two-block operators) array of
    (t, lo, hi) per column/block; with sets=True also an int64 array of the
    same shape of (n_hi, n_mid, branch) per record (sdca_prox_with_sets: the
    sizes of the record's set at hi and free set, and its sdca_prox_branch).
    A device col_p is checked against [1, dim - 1] here (one
    synchronisation) unless check_col_p=False, for callers that validated it
    already (the kernels clamp it into range either way)."""
    lib = library()
    code = OPS[op] if isinstance(op, str) else int(op)
    data = _dtype_code(A)
    if data < 0:
        raise SdcaError(3, f"unsupported element type {A.dtype}")
    res = data if result is None else ({"float": F32, "single": F32, "double": F64,
                                        "long double": LONG_DOUBLE}.get(result, result))
    if A.ndim == 1:
        A = A.reshape(1, -1)
        if out is not None:
            out = out.reshape(1, -1)
    if A.ndim != 2:
        raise SdcaError(2, f"A must be 1-D or 2-D (got {A.ndim} dimensions)")
    n, m = int(A.shape[0]), int(A.shape[1])
    if out is None:
        out = A
    _need(A, "A", (n, m), A)
    _need(out, "out", (n, m), A)
    params = ProxParams(lo, hi, rhs, rho, alpha, int(k), int(p))
    nthr = 2 * n if code in (OPS["two_simplex"], OPS["two_simplex_sort"],
                             OPS["two_entropy"]) else n
    if _is_torch(A):
        import torch
        if not A.is_cuda:
            raise SdcaError(2, "torch inputs must be CUDA tensors")
        thr = torch.zeros((nthr, 3), dtype=torch.float64, device=A.device) if thresholds else None
        # sdca_prox_sets is {int64, int64, int32, int32}: the third int64 word
        # reads as the branch (the reserved half is 0).
        st = torch.zeros((nthr, 3), dtype=torch.int64, device=A.device) if sets else None
        cp = None
        if col_p is not None:
            cp = torch.as_tensor(col_p, dtype=torch.int64, device=A.device).contiguous().reshape(-1)
            if cp.shape[0] != n:
                raise SdcaError(2, f"col_p has {cp.shape[0]} entries for {n} columns")
            if check_col_p and n > 0:
                lo_p, hi_p = torch.aminmax(cp)
                if int(lo_p) < 1 or int(hi_p) > m - 1:
                    raise SdcaError(2, f"col_p must lie in [1, {m - 1}] (got {int(lo_p)}..{int(hi_p)})")
        if st is not None:
            check(lib.sdca_prox_with_sets(
                code, data, res, ctypes.c_int64(m), ctypes.c_int64(n), ctypes.c_void_p(A.data_ptr()),
                ctypes.c_void_p(out.data_ptr()), ctypes.byref(params),
                ctypes.c_void_p(cp.data_ptr() if cp is not None else None),
                ctypes.c_void_p(thr.data_ptr() if thr is not None else None),
                ctypes.c_void_p(st.data_ptr()), ctypes.c_uint(0), _stream_ptr()))
        else:
            check(lib.sdca_prox(code, data, res, m, n, A.data_ptr(), out.data_ptr(),
                                ctypes.byref(params), cp.data_ptr() if cp is not None else None,
                                thr.data_ptr() if thr is not None else None, 0, _stream_ptr()))
        return _prox_result(out, thr, st, thresholds, sets)
    thr = np.zeros((nthr, 3), dtype=np.float64) if thresholds else None
    st = np.zeros((nthr, 3), dtype=np.int64) if sets else None
    cp = None if col_p is None else np.ascontiguousarray(col_p, dtype=np.int64).reshape(-1)
    if cp is not None and cp.shape[0] != n:
        raise SdcaError(2, f"col_p has {cp.shape[0]} entries for {n} columns")
    if st is not None:
        check(lib.sdca_prox_with_sets(
            code, data, res, ctypes.c_int64(m), ctypes.c_int64(n), ctypes.c_void_p(A.ctypes.data),
            ctypes.c_void_p(out.ctypes.data), ctypes.byref(params),
            ctypes.c_void_p(cp.ctypes.data if cp is not None else None),
            ctypes.c_void_p(thr.ctypes.data if thr is not None else None),
            ctypes.c_void_p(st.ctypes.data), ctypes.c_uint(HOST_PTR), None))
    else:
        check(lib.sdca_prox(code, data, res, m, n, A.ctypes.data, out.ctypes.data,
                            ctypes.byref(params), cp.ctypes.data if cp is not None else None,
                            thr.ctypes.data if thr is not None else None, HOST_PTR, None))
    return _prox_result(out, thr, st, thresholds, sets)


def _prox_result(out, thr, st, thresholds, sets):
    res = (out,) + ((thr,) if thresholds else ()) + ((st,) if sets else ())
    return res if len(res) > 1 else out


def _rows(dim, A):
    if A.ndim == 2 and A.shape[1] == dim:
        return A
    return A.reshape(-1, dim)


# The reference's batched overloads (`dim` first).  Result follows the
# reference: deduced from the floating parameter's type in C++; here the
# element type unless `result` is given.  prox_topk_cone, prox_topk_entropy
# and prox_topk_entropy_biased default to double, as their C++ templates do
# (topk_cone.h:187-199, topk_entropy.h:106-118, topk_entropy_biased.h:302-315).
def prox_knapsack_eq(dim, A, lo=0.0, hi=1.0, rhs=1.0, result=None):
    return prox("knapsack_eq", _rows(dim, A), lo=lo, hi=hi, rhs=rhs, result=result)


def prox_knapsack_le(dim, A, lo=0.0, hi=1.0, rhs=1.0, result=None):
    return prox("knapsack_le", _rows(dim, A), lo=lo, hi=hi, rhs=rhs, result=result)


def prox_topk_simplex(dim, A, k=1, rhs=1.0, result=None):
    return prox("topk_simplex", _rows(dim, A), k=k, rhs=rhs, result=result)


def prox_topk_cone(dim, A, k=1, result="double"):
    return prox("topk_cone", _rows(dim, A), k=k, result=result)


def prox_entropy(dim, A, hi=1.0, rhs=1.0, result=None):
    return prox("entropy", _rows(dim, A), hi=hi, rhs=rhs, result=result)


def prox_entropy_norm(dim, A, hi=1.0, rhs=1.0, result=None):
    return prox("entropy_norm", _rows(dim, A), hi=hi, rhs=rhs, result=result)


def prox_topk_entropy(dim, A, k=1, result="double"):
    return prox("topk_entropy", _rows(dim, A), k=k, result=result)


def prox_two_simplex(dim, p, A, rhs=1.0, result=None):
    return prox("two_simplex", _rows(dim, A), p=p, rhs=rhs, result=result)


def prox_knapsack_le_biased(dim, A, lo=0.0, hi=1.0, rhs=1.0, rho=1.0, result=None):
    return prox("knapsack_le_biased", _rows(dim, A), lo=lo, hi=hi, rhs=rhs, rho=rho, result=result)


def prox_topk_simplex_biased(dim, A, k=1, rhs=1.0, rho=1.0, result=None):
    return prox("topk_simplex_biased", _rows(dim, A), k=k, rhs=rhs, rho=rho, result=result)


def prox_topk_cone_biased(dim, A, k=1, rho=1.0, result=None):
    return prox("topk_cone_biased", _rows(dim, A), k=k, rho=rho, result=result)


def prox_topk_entropy_biased(dim, A, k=1, alpha=1.0, result="double"):
    return prox("topk_entropy_biased", _rows(dim, A), k=k, alpha=alpha, result=result)


def prox_two_entropy(dim, p, A, alpha=1.0, result=None):
    """Batched form of prox_two_entropy(p, first, last, aux, alpha)
    (two_entropy.h:280-292), which the reference has per column only."""
    return prox("two_entropy", _rows(dim, A), p=p, alpha=alpha, result=result)


def prox_two_simplex_sort(dim, p, A, rhs=1.0, result=None):
    return prox("two_simplex_sort", _rows(dim, A), p=p, rhs=rhs, result=result)


def lambert_w_exp(A):
    """Elementwise W(exp(x)) in place (apply(dim, ..., lambert_w_exp_map))."""
    return prox("lambert_w_exp", A if A.ndim == 2 else A.reshape(1, -1))


# ---------------------------------------------------------------------------
# Evaluation pass (evaluate_dataset, eval.h:15-51, for feature input).
# X: (n, d) examples, W: (m, d) classes, S/A: (n, m); all C-contiguous, i.e.
# the reference's column-major d x n, d x m and m x n matrices.
# ---------------------------------------------------------------------------
def _objs(objs):
    arr = (Objective * len(objs))()
    for i, (name, c, gamma, k) in enumerate(objs):
        arr[i] = Objective(OBJECTIVES[name], 0, c, gamma, k)
    return arr


def _ptr(x):
    if x is None:
        return None
    return x.data_ptr() if _is_torch(x) else x.ctypes.data


def scores(X, W, out=None):
    """S = X W^T (scores of every example for every class)."""
    lib = library()
    n, d = int(X.shape[0]), int(X.shape[1])
    m = int(W.shape[0])
    data = _dtype_code(X)
    _need(X, "X", (n, d), X)
    _need(W, "W", (m, d), X)
    _need(out, "out", (n, m), X)
    if _is_torch(X):
        import torch
        S = out if out is not None else torch.empty((n, m), dtype=X.dtype, device=X.device)
        check(lib.sdca_scores(data, ctypes.c_int64(d), ctypes.c_int64(m), ctypes.c_int64(n),
                              ctypes.c_void_p(X.data_ptr()), ctypes.c_void_p(W.data_ptr()),
                              ctypes.c_void_p(S.data_ptr()), ctypes.c_uint(0), _stream_ptr()))
        return S
    S = out if out is not None else np.zeros((n, m), dtype=X.dtype)
    check(lib.sdca_scores(data, ctypes.c_int64(d), ctypes.c_int64(m), ctypes.c_int64(n),
                          ctypes.c_void_p(X.ctypes.data), ctypes.c_void_p(W.ctypes.data),
                          ctypes.c_void_p(S.ctypes.data), ctypes.c_uint(HOST_PTR), None))
    return S


def epoch_order(n, epoch):
    """The reference solver's example order for epoch `epoch` (0-based) of a
    solve over n examples (solver.h:75-112): int64 numpy array."""
    lib = library()
    out = np.zeros(int(n), dtype=np.int64)
    lib.sdca_epoch_order.restype = ctypes.c_int
    rc = lib.sdca_epoch_order(ctypes.c_int64(int(n)), ctypes.c_int64(int(epoch)),
                              ctypes.c_void_p(out.ctypes.data))
    if rc != 0:
        raise SdcaError(rc, lib.sdca_last_error().decode())
    return out


def epoch_features(obj, X, W, A, labels, order=None, norms=None, result=None, offsets=None):
    """One SDCA epoch on feature input (update_variables for each example of
    `order`, update.h:52-85) for an objective (name, c, gamma, k):
    X (n, d), W (m, d), A (n, m), W and A updated in place and returned.
    CUDA tensors run on torch's current stream; numpy arrays (C-contiguous,
    X's dtype) go through the host-staging path.  order: example indices
    (None: 0..n-1), e.g. epoch_order(n, e); norms: (n,) squared row norms of
    X, or None; offsets: (n + 1,) CSR row starts into labels for the
    multilabel objectives."""
    lib = library()
    n, d = int(X.shape[0]), int(X.shape[1])
    m = int(W.shape[0])
    objarr = _objs([obj])
    lib.sdca_epoch_features.restype = ctypes.c_int
    if _is_torch(X):
        if not X.is_cuda:
            raise SdcaError(2, "epoch_features takes CUDA tensors or numpy arrays")
        import torch
        _need(X, "X", (n, d), X)
        _need(W, "W", (m, d), X)
        _need(A, "A", (n, m), X)
        _need(norms, "norms", (n,), X)
        od = None
        if order is not None:
            od = torch.as_tensor(order, dtype=torch.int64, device=X.device).contiguous().reshape(-1)
        flags, stream = 0, _stream_ptr()
        ptr = _ptr
    else:
        for name, a, shape in (("X", X, (n, d)), ("W", W, (m, d)), ("A", A, (n, m)),
                               ("norms", norms, (n,))):
            if a is None:
                continue
            if (not isinstance(a, np.ndarray) or a.dtype != X.dtype or tuple(a.shape) != shape
                    or not a.flags.c_contiguous):
                raise SdcaError(2, f"{name}: expected a C-contiguous {X.dtype} array {shape}")
        od = None if order is None else np.ascontiguousarray(order, dtype=np.int64).reshape(-1)
        flags, stream = HOST_PTR, None

        def ptr(a):
            return None if a is None else a.ctypes.data
    data = _dtype_code(X)
    res = data if result is None else ({"float": F32, "single": F32, "double": F64}.get(result, result))
    # n labels, or n + 1 offsets from 0, non-decreasing, ending at len(labels)
    lab, off = _label_arrays(labels, offsets, n, X)
    count = n if od is None else int(od.shape[0])
    rc = lib.sdca_epoch_features(objarr, ctypes.c_int(data), ctypes.c_int(res), ctypes.c_int64(d),
                                 ctypes.c_int64(m), ctypes.c_int64(n), ctypes.c_void_p(ptr(X)),
                                 ctypes.c_void_p(ptr(W)), ctypes.c_void_p(ptr(A)),
                                 ctypes.c_void_p(ptr(lab)), ctypes.c_void_p(ptr(off)),
                                 ctypes.c_void_p(ptr(od)),
                                 ctypes.c_int64(count), ctypes.c_void_p(ptr(norms)),
                                 ctypes.c_uint(flags), stream)
    if rc != 0:
        raise SdcaError(rc, lib.sdca_last_error().decode())
    return W, A


def epoch_kernel(obj, K, A, labels, order=None, result=None, offsets=None):
    """One SDCA epoch on kernel input (the kernel form of update_variables,
    update.h:88-107, for each example of `order`) for an objective (name, c,
    gamma, k): K (n, n) the symmetric training kernel matrix, A (n, m)
    updated in place and returned.  CUDA tensors run on torch's current
    stream; numpy arrays (C-contiguous, K's dtype) go through the
    host-staging path.  order, result and offsets: as epoch_features."""
    lib = library()
    n = int(K.shape[0])
    m = int(A.shape[1])
    objarr = _objs([obj])
    lib.sdca_epoch_kernel.restype = ctypes.c_int
    if _is_torch(K):
        if not K.is_cuda:
            raise SdcaError(2, "epoch_kernel takes CUDA tensors or numpy arrays")
        import torch
        _need(K, "K", (n, n), K)
        _need(A, "A", (n, m), K)
        od = None
        if order is not None:
            od = torch.as_tensor(order, dtype=torch.int64, device=K.device).contiguous().reshape(-1)
        flags, stream = 0, _stream_ptr()
        ptr = _ptr
    else:
        for name, a, shape in (("K", K, (n, n)), ("A", A, (n, m))):
            if (not isinstance(a, np.ndarray) or a.dtype != K.dtype or tuple(a.shape) != shape
                    or not a.flags.c_contiguous):
                raise SdcaError(2, f"{name}: expected a C-contiguous {K.dtype} array {shape}")
        od = None if order is None else np.ascontiguousarray(order, dtype=np.int64).reshape(-1)
        flags, stream = HOST_PTR, None

        def ptr(a):
            return None if a is None else a.ctypes.data
    data = _dtype_code(K)
    res = data if result is None else ({"float": F32, "single": F32, "double": F64}.get(result, result))
    lab, off = _label_arrays(labels, offsets, n, K)
    count = n if od is None else int(od.shape[0])
    rc = lib.sdca_epoch_kernel(objarr, ctypes.c_int(data), ctypes.c_int(res), ctypes.c_int64(m),
                               ctypes.c_int64(n), ctypes.c_void_p(ptr(K)), ctypes.c_void_p(ptr(A)),
                               ctypes.c_void_p(ptr(lab)), ctypes.c_void_p(ptr(off)),
                               ctypes.c_void_p(ptr(od)), ctypes.c_int64(count),
                               ctypes.c_uint(flags), stream)
    if rc != 0:
        raise SdcaError(rc, lib.sdca_last_error().decode())
    return A


def recompute_primal(X, A, W0=None, out=None):
    """W = W0 + A^T X (the reference's W = W0 + X A' of eval_recompute_primal,
    eval/core.h:148-182): X (n, d) features, A (n, m) dual variables, W0 and
    the result (m, d)."""
    lib = library()
    n, d = int(X.shape[0]), int(X.shape[1])
    m = int(A.shape[1])
    data = _dtype_code(X)
    _need(X, "X", (n, d), X)
    _need(A, "A", (n, m), X)
    _need(W0, "W0", (m, d), X)
    _need(out, "out", (m, d), X)
    lib.sdca_recompute_primal.restype = ctypes.c_int
    if _is_torch(X):
        import torch
        W = out if out is not None else torch.empty((m, d), dtype=X.dtype, device=X.device)
        check(lib.sdca_recompute_primal(data, ctypes.c_int64(d), ctypes.c_int64(m), ctypes.c_int64(n),
                                        ctypes.c_void_p(X.data_ptr()), ctypes.c_void_p(A.data_ptr()),
                                        ctypes.c_void_p(_ptr(W0)), ctypes.c_void_p(W.data_ptr()),
                                        ctypes.c_uint(0), _stream_ptr()))
        return W
    W = out if out is not None else np.zeros((m, d), dtype=X.dtype)
    check(lib.sdca_recompute_primal(data, ctypes.c_int64(d), ctypes.c_int64(m), ctypes.c_int64(n),
                                    ctypes.c_void_p(X.ctypes.data), ctypes.c_void_p(A.ctypes.data),
                                    ctypes.c_void_p(_ptr(W0)), ctypes.c_void_p(W.ctypes.data),
                                    ctypes.c_uint(HOST_PTR), None))
    return W


EVAL_TEST = 2  # SDCA_EVAL_TEST


EVAL_FUSED = 4  # SDCA_EVAL_FUSED


def _eval(fn_name, objs, lead_args, m, n, labels, offsets, A, result, per_example, torch_mode,
          data, tail_args=(), test=False, fused=False):
    lib = library()
    res = data if result is None else ({"float": F32, "single": F32, "double": F64}.get(result, result))
    objarr = _objs(objs)
    recs = (EvalRecord * len(objs))()
    acc = np.zeros(m, dtype=np.float64)
    pe = None
    lab, off = _label_arrays(labels, offsets, n, lead_args[0])
    if torch_mode:
        import torch
        dev = lead_args[0].device
        if per_example:
            pe = torch.zeros((n, len(objs), 2), dtype=torch.float64, device=dev)
        flags, stream = 0, _stream_ptr()
    else:
        if per_example:
            pe = np.zeros((n, len(objs), 2), dtype=np.float64)
        flags, stream = HOST_PTR, None
    if test:
        flags |= EVAL_TEST
    if fused:
        flags |= EVAL_FUSED
    fn = getattr(lib, fn_name)
    fn.restype = ctypes.c_int
    args = [objarr, ctypes.c_int(len(objs)), ctypes.c_int(data), ctypes.c_int(res)]
    args += list(lead_args[1])
    args += [ctypes.c_void_p(_ptr(A)), *tail_args, ctypes.c_void_p(_ptr(lab)),
             ctypes.c_void_p(_ptr(off)), recs, ctypes.c_void_p(acc.ctypes.data),
             ctypes.c_void_p(_ptr(pe)), ctypes.c_uint(flags), stream]
    check(fn(*args))
    records = [{f: getattr(r, f) for f, _ in EvalRecord._fields_} for r in recs]
    return records, acc, pe


def eval_features(objs, X, W, labels, A=None, W0=None, offsets=None, result=None,
                  per_example=False, test=False, fused=False):
    """evaluate_dataset for feature input.  objs: list of objective(...).
    Returns (records, accuracy, per_example): one eval record per objective
    (primal, dual, primal_loss, dual_loss, primal/dual regularizer, rank_loss),
    the top-(i+1) accuracies (multiclass) and optionally the (n, n_obj, 2)
    per-example (primal, dual) losses before the loss coefficient.
    test=True gives a test set's records (eval_test: primal loss and
    accuracy / rank loss only).  fused=True runs the one-kernel form where it
    applies (SDCA_EVAL_FUSED; slower on MI355X; bit-identical results below
    2^32 multiply-adds n m d or 512 classes, equal to score rounding above,
    where the two-kernel form's scores come from hipBLASLt)."""
    n, d = int(X.shape[0]), int(X.shape[1])
    m = int(W.shape[0])
    _need(X, "X", (n, d), X)
    _need(W, "W", (m, d), X)
    _need(A, "A", (n, m), X)
    _need(W0, "W0", (m, d), X)
    lead = (X, [ctypes.c_int64(d), ctypes.c_int64(m), ctypes.c_int64(n),
                ctypes.c_void_p(_ptr(X)), ctypes.c_void_p(_ptr(W))])
    return _eval("sdca_eval_features", objs, lead, m, n, labels, offsets, A, result, per_example,
                 _is_torch(X), _dtype_code(X), tail_args=(ctypes.c_void_p(_ptr(W0)),), test=test,
                 fused=fused)


def eval_kernel(objs, K, A, labels, offsets=None, result=None, per_example=False, test=False):
    """evaluate_dataset for kernel input (data/input.h:44-76): K is (n, n_train),
    row i the kernel column K_i of example i; A is (n_train, m), the dual
    variables (rows are the reference's columns); scores_i = A K_i.  For a
    training set (n == n_train) the dual losses come from A's rows and the
    dual regularizer is sum_i 0.5 <a_i, s_i>; test=True gives a test set's
    records."""
    n, n_train = int(K.shape[0]), int(K.shape[1])
    m = int(A.shape[1])
    _need(K, "K", (n, n_train), K)
    _need(A, "A", (n_train, m), K)
    lead = (K, [ctypes.c_int64(n_train), ctypes.c_int64(m), ctypes.c_int64(n),
                ctypes.c_void_p(_ptr(K))])
    return _eval("sdca_eval_kernel", objs, lead, m, n, labels, offsets, A, result, per_example,
                 _is_torch(K), _dtype_code(K), test=test)


def eval_scores(objs, S, labels, A=None, offsets=None, primal_regularizer=0.0,
                dual_regularizer=0.0, result=None, per_example=False):
    """The per-example part of evaluate_dataset on precomputed scores S."""
    n, m = int(S.shape[0]), int(S.shape[1])
    _need(S, "S", (n, m), S)
    _need(A, "A", (n, m), S)
    lib = library()
    res = _dtype_code(S) if result is None else ({"float": F32, "single": F32, "double": F64}.get(result, result))
    torch_mode = _is_torch(S)
    objarr = _objs(objs)
    recs = (EvalRecord * len(objs))()
    acc = np.zeros(m, dtype=np.float64)
    lab, off = _label_arrays(labels, offsets, n, S)
    if torch_mode:
        import torch
        pe = torch.zeros((n, len(objs), 2), dtype=torch.float64, device=S.device) if per_example else None
        flags, stream = 0, _stream_ptr()
    else:
        pe = np.zeros((n, len(objs), 2), dtype=np.float64) if per_example else None
        flags, stream = HOST_PTR, None
    lib.sdca_eval_scores.restype = ctypes.c_int
    check(lib.sdca_eval_scores(objarr, ctypes.c_int(len(objs)), ctypes.c_int(_dtype_code(S)),
                               ctypes.c_int(res), ctypes.c_int64(m), ctypes.c_int64(n),
                               ctypes.c_void_p(_ptr(S)), ctypes.c_void_p(_ptr(A)),
                               ctypes.c_void_p(_ptr(lab)), ctypes.c_void_p(_ptr(off)),
                               ctypes.c_double(primal_regularizer), ctypes.c_double(dual_regularizer),
                               recs, ctypes.c_void_p(acc.ctypes.data), ctypes.c_void_p(_ptr(pe)),
                               ctypes.c_uint(flags), stream))
    records = [{f: getattr(r, f) for f, _ in EvalRecord._fields_} for r in recs]
    return records, acc, pe
