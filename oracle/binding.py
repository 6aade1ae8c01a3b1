"""ctypes binding of the CPU checker (TEST INFRASTRUCTURE ONLY).

Loads oracle/liboracle.so (the restatement) and, when it was built,
oracle/_ref/libsdca_ref.so (our shim over the reference headers).  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module; the product package never does.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libsdca_ref.so")
REFERENCE_TREE = "/root/reference"

F32, F64 = 0, 1
OPS = {
    "knapsack_eq": 0, "knapsack_le": 1, "topk_simplex": 2, "topk_cone": 3,
    "entropy": 4, "entropy_norm": 5, "topk_entropy": 6, "two_simplex": 7,
    "lambert_w_exp": 8, "knapsack_le_biased": 9, "topk_simplex_biased": 10,
    "topk_cone_biased": 11, "topk_entropy_biased": 12, "two_simplex_sort": 13,
    "two_entropy": 14,
}
OBJECTIVES = {
    "hinge_topk": 0, "hinge_topk_smooth": 1, "topk_hinge": 2,
    "topk_hinge_smooth": 3, "entropy": 4, "entropy_topk": 5,
    "multilabel_hinge": 6, "multilabel_hinge_smooth": 7,
    "multilabel_entropy": 8,
}


# sdca_prox_sets (include/sdca_hip.h)
SETS_DTYPE = np.dtype([("n_hi", "<i8"), ("n_mid", "<i8"), ("branch", "<i4"), ("reserved", "<i4")])


class ProxParams(ctypes.Structure):
    _fields_ = [("lo", ctypes.c_double), ("hi", ctypes.c_double),
                ("rhs", ctypes.c_double), ("rho", ctypes.c_double),
                ("alpha", ctypes.c_double), ("k", ctypes.c_int64),
                ("p", ctypes.c_int64)]


class Objective(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("c", ctypes.c_double), ("gamma", ctypes.c_double),
                ("k", ctypes.c_int64)]


class EvalRecord(ctypes.Structure):
    _fields_ = [("primal", ctypes.c_double), ("dual", ctypes.c_double),
                ("primal_loss", ctypes.c_double), ("dual_loss", ctypes.c_double),
                ("primal_regularizer", ctypes.c_double),
                ("dual_regularizer", ctypes.c_double),
                ("rank_loss", ctypes.c_double)]


def build(with_reference=True):
    """Compile liboracle.so, and the reference shim when the tree exists."""
    subprocess.check_call(["make", "-s", "-B", "-C", HERE, "all"])
    if with_reference and os.path.isdir(os.path.join(REFERENCE_TREE, "include")):
        subprocess.check_call(["make", "-s", "-B", "-C", HERE, "ref"])
        # needs the product library, built first by __graft_entry__.build()
        if os.path.exists(os.path.join(HERE, "..", "libsdca_amd", "libsdca_hip.so")):
            subprocess.check_call(["make", "-s", "-B", "-C", HERE, "dropin"])


_libs = {}


def _load(path):
    if path not in _libs:
        lib = ctypes.CDLL(path)
        _libs[path] = lib
    return _libs[path]


def oracle():
    if not os.path.exists(ORACLE_SO):
        build(with_reference=False)
    return Library(_load(ORACLE_SO), "oracle")


def reference():
    """The reference shim, or None when it was not built."""
    if not os.path.exists(REF_SO):
        return None
    return Library(_load(REF_SO), "ref")


def make_params(lo=0.0, hi=1.0, rhs=1.0, rho=1.0, alpha=1.0, k=1, p=1):
    return ProxParams(lo, hi, rhs, rho, alpha, k, p)


def make_objectives(objs):
    """objs: list of (name, c, gamma, k)."""
    arr = (Objective * len(objs))()
    for i, (name, c, gamma, k) in enumerate(objs):
        arr[i] = Objective(OBJECTIVES[name], 0, c, gamma, k)
    return arr


def _dt(a):
    return F32 if a.dtype == np.float32 else F64


class Library:
    def __init__(self, lib, prefix):
        self.lib = lib
        self.prefix = prefix
        self._prox = getattr(lib, prefix + "_prox")
        self._prox.restype = ctypes.c_int
        self._prox.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                               ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                               ctypes.POINTER(ProxParams), ctypes.c_void_p,
                               ctypes.c_void_p, ctypes.c_int]
        self._eval = getattr(lib, prefix + "_eval_scores")
        self._eval.restype = ctypes.c_int
        self._lw64 = getattr(lib, prefix + "_lambert_w_exp_f64")
        self._lw64.restype = ctypes.c_double
        self._lw64.argtypes = [ctypes.c_double]
        self._lw32 = getattr(lib, prefix + "_lambert_w_exp_f32")
        self._lw32.restype = ctypes.c_float
        self._lw32.argtypes = [ctypes.c_float]

    def prox(self, op, x, result=None, params=None, col_p=None,
             thresholds=False, nthreads=1):
        """In-place batched prox over the columns of x (m x n, Fortran order,
        given as an (n, m) C-contiguous array: row j = column j)."""
        assert x.flags.c_contiguous
        n, m = x.shape
        data = _dt(x)
        result = data if result is None else result
        params = params or make_params()
        thr = None
        if thresholds:
            cnt = 2 * n if op in ("two_simplex", "two_simplex_sort", "two_entropy") else n
            thr = np.zeros((cnt, 3), dtype=np.float64)
        cp = None
        if col_p is not None:
            cp = np.ascontiguousarray(col_p, dtype=np.int64)
        rc = self._prox(OPS[op], data, result, m, n, x.ctypes.data,
                        ctypes.byref(params),
                        cp.ctypes.data if cp is not None else None,
                        thr.ctypes.data if thr is not None else None, nthreads)
        if rc != 0:
            raise RuntimeError(f"{self.prefix}_prox failed: {rc}")
        return thr

    def prox_sets(self, op, x, result=None, params=None, col_p=None, nthreads=1):
        """prox with each record's thresholds and sets: returns (thr, sets),
        thr (records, 3) = (t, lo, hi), sets (records, 3) int64 = (n_hi,
        n_mid, branch): first - begin and last - first of the threshold
        function's record (proxdef.h:29-67), and the return that produced it
        (-1 from the reference, which does not record it)."""
        assert x.flags.c_contiguous
        n, m = x.shape
        data = _dt(x)
        result = data if result is None else result
        params = params or make_params()
        cnt = 2 * n if op in ("two_simplex", "two_simplex_sort", "two_entropy") else n
        thr = np.zeros((cnt, 3), dtype=np.float64)
        raw = np.zeros(cnt, dtype=SETS_DTYPE)
        cp = None if col_p is None else np.ascontiguousarray(col_p, dtype=np.int64)
        f = getattr(self.lib, f"{self.prefix}_prox_sets")
        f.restype = ctypes.c_int
        rc = f(ctypes.c_int(OPS[op]), ctypes.c_int(data), ctypes.c_int(result), ctypes.c_int64(m),
               ctypes.c_int64(n), ctypes.c_void_p(x.ctypes.data), ctypes.byref(params),
               ctypes.c_void_p(cp.ctypes.data if cp is not None else None),
               ctypes.c_void_p(thr.ctypes.data), ctypes.c_void_p(raw.ctypes.data),
               ctypes.c_int(nthreads))
        if rc != 0:
            raise RuntimeError(f"{self.prefix}_prox_sets failed: {rc}")
        sets = np.stack([raw["n_hi"], raw["n_mid"], raw["branch"].astype(np.int64)], axis=1)
        return thr, sets

    def eval_scores(self, objs, S, A, labels, offsets=None, preg=0.0, dreg=0.0,
                    result=None, per_example=False, nthreads=1):
        """S, A: (n, m) C-contiguous (row i = example i's m scores)."""
        n, m = S.shape
        data = _dt(S)
        result = data if result is None else result
        objarr = make_objectives(objs)
        recs = (EvalRecord * len(objs))()
        acc = np.zeros(m, dtype=np.float64)
        pe = np.zeros((n, len(objs), 2), dtype=np.float64) if per_example else None
        labels = np.ascontiguousarray(labels, dtype=np.int64)
        off = None if offsets is None else np.ascontiguousarray(offsets, dtype=np.int64)
        args = [objarr, ctypes.c_int(len(objs)), ctypes.c_int(data), ctypes.c_int(result),
                ctypes.c_int64(m), ctypes.c_int64(n), ctypes.c_void_p(S.ctypes.data),
                ctypes.c_void_p(A.ctypes.data if A is not None else None),
                ctypes.c_void_p(labels.ctypes.data),
                ctypes.c_void_p(off.ctypes.data if off is not None else None),
                ctypes.c_double(preg), ctypes.c_double(dreg), recs,
                ctypes.c_void_p(acc.ctypes.data),
                ctypes.c_void_p(pe.ctypes.data if pe is not None else None)]
        if self.prefix == "oracle":
            args.append(ctypes.c_int(nthreads))
        rc = self._eval(*args)
        if rc != 0:
            raise RuntimeError(f"{self.prefix}_eval_scores failed: {rc}")
        out = [{f: getattr(r, f) for f, _ in EvalRecord._fields_} for r in recs]
        return out, acc, pe

    def lambert_w_exp(self, x):
        if np.asarray(x).dtype == np.float32:
            return np.array([self._lw32(float(v)) for v in np.ravel(x)], dtype=np.float32)
        return np.array([self._lw64(float(v)) for v in np.ravel(x)], dtype=np.float64)

    # Only the reference shim has these three.
    def evaluate_dataset(self, objs, X, W, A, labels, offsets=None, W0=None, result=None,
                         nthreads=1):
        """The reference's evaluate_dataset (solver/eval.h:15-51) over a
        feature input: X (n, d), W and W0 (m, d), A (n, m), all C-contiguous
        (the reference's column-major d x n, d x m, m x n).  A is swapped in
        place and restored, as the reference does.  Returns (records, accuracy)."""
        n, d = X.shape
        m = W.shape[0]
        data = _dt(X)
        result = data if result is None else result
        objarr = make_objectives(objs)
        recs = (EvalRecord * len(objs))()
        acc = np.zeros(m, dtype=np.float64)
        labels = np.ascontiguousarray(labels, dtype=np.int64)
        off = None if offsets is None else np.ascontiguousarray(offsets, dtype=np.int64)
        f = self.lib.ref_evaluate_dataset
        f.restype = ctypes.c_int
        rc = f(objarr, ctypes.c_int(len(objs)), ctypes.c_int(data), ctypes.c_int(result),
               ctypes.c_int64(d), ctypes.c_int64(m), ctypes.c_int64(n),
               ctypes.c_void_p(X.ctypes.data), ctypes.c_void_p(W.ctypes.data),
               ctypes.c_void_p(W0.ctypes.data if W0 is not None else None),
               ctypes.c_void_p(A.ctypes.data), ctypes.c_void_p(labels.ctypes.data),
               ctypes.c_void_p(off.ctypes.data if off is not None else None), recs,
               ctypes.c_void_p(acc.ctypes.data), ctypes.c_int(nthreads))
        if rc != 0:
            raise RuntimeError(f"ref_evaluate_dataset failed: {rc}")
        return [{f_: getattr(r, f_) for f_, _ in EvalRecord._fields_} for r in recs], acc

    def epoch_features(self, obj, X, W, A, labels, order=None, result=None, epochs=0,
                       reverse=False, offsets=None):
        """One SDCA epoch on feature input (solver.h:39-51, update.h:52-85)
        over `order` (None: 0..n-1): X (n, d), W (m, d), A (n, m)
        C-contiguous; W and A are updated in place (and returned).  The
        reference shim runs sdca::update_variables; with epochs > 0 instead
        the reference's own solve() for that many epochs (its shuffled
        order).  The restatement takes reverse=True for its second rounding
        of the scores.  offsets: CSR row starts into labels (n + 1) for the
        multilabel objectives."""
        n, d = X.shape
        m = W.shape[0]
        data = _dt(X)
        result = data if result is None else result
        objarr = make_objectives([obj])
        labels = np.ascontiguousarray(labels, dtype=np.int64)
        od = None if order is None else np.ascontiguousarray(order, dtype=np.int64)
        off = None if offsets is None else np.ascontiguousarray(offsets, dtype=np.int64)
        count = n if od is None else od.size
        common = (objarr, ctypes.c_int(data), ctypes.c_int(result), ctypes.c_int64(d),
                  ctypes.c_int64(m), ctypes.c_int64(n), ctypes.c_void_p(X.ctypes.data),
                  ctypes.c_void_p(W.ctypes.data), ctypes.c_void_p(A.ctypes.data),
                  ctypes.c_void_p(labels.ctypes.data),
                  ctypes.c_void_p(off.ctypes.data if off is not None else None),
                  ctypes.c_void_p(od.ctypes.data if od is not None else None),
                  ctypes.c_int64(count))
        if hasattr(self.lib, "ref_epoch_features"):
            f = self.lib.ref_epoch_features
            f.restype = ctypes.c_int
            rc = f(*common, ctypes.c_int64(epochs))
        else:
            assert epochs == 0
            f = self.lib.oracle_epoch_features
            f.restype = ctypes.c_int
            rc = f(*common, ctypes.c_int(1 if reverse else 0))
        if rc != 0:
            raise RuntimeError(f"epoch_features failed: {rc}")
        return W, A

    def epoch_kernel(self, obj, K, A, labels, order=None, result=None, epochs=0, reverse=False,
                     offsets=None):
        """One SDCA epoch on kernel input (update.h:88-107) over `order`
        (None: 0..n-1): K (n, n) the training set's kernel matrix (row i =
        K_i), A (n, m) C-contiguous, updated in place (and returned).  The
        reference shim runs sdca::update_variables on a kernel_input
        context; with epochs > 0 instead the reference's own solve().  The
        restatement takes reverse=True for its second rounding of the
        scores."""
        n = K.shape[0]
        m = A.shape[1]
        data = _dt(K)
        result = data if result is None else result
        objarr = make_objectives([obj])
        labels = np.ascontiguousarray(labels, dtype=np.int64)
        od = None if order is None else np.ascontiguousarray(order, dtype=np.int64)
        off = None if offsets is None else np.ascontiguousarray(offsets, dtype=np.int64)
        count = n if od is None else od.size
        common = (objarr, ctypes.c_int(data), ctypes.c_int(result), ctypes.c_int64(m),
                  ctypes.c_int64(n), ctypes.c_void_p(K.ctypes.data),
                  ctypes.c_void_p(A.ctypes.data), ctypes.c_void_p(labels.ctypes.data),
                  ctypes.c_void_p(off.ctypes.data if off is not None else None),
                  ctypes.c_void_p(od.ctypes.data if od is not None else None),
                  ctypes.c_int64(count))
        if hasattr(self.lib, "ref_epoch_kernel"):
            f = self.lib.ref_epoch_kernel
            f.restype = ctypes.c_int
            rc = f(*common, ctypes.c_int64(epochs))
        else:
            assert epochs == 0
            f = self.lib.oracle_epoch_kernel
            f.restype = ctypes.c_int
            rc = f(*common, ctypes.c_int(1 if reverse else 0))
        if rc != 0:
            raise RuntimeError(f"epoch_kernel failed: {rc}")
        return A

    def blas_scores(self, X, W):
        """The reference's scores W' x_i (eval/scores.h:9-27, cblas_sgemv) of
        every example: X (n, d), W (m, d) float32 -> S (n, m)."""
        n, d = X.shape
        m = W.shape[0]
        S = np.zeros((n, m), dtype=np.float32)
        f = self.lib.ref_blas_sgemv_t
        f.restype = None
        for i in range(n):
            f(ctypes.c_int(d), ctypes.c_int(m), ctypes.c_void_p(W.ctypes.data),
              ctypes.c_void_p(X[i].ctypes.data), ctypes.c_void_p(S[i].ctypes.data))
        return S

    def blas_dot(self, x, y):
        """The reference's sdca_blas_dot (math/blas.h:191-219)."""
        x = np.ascontiguousarray(x)
        y = np.ascontiguousarray(y, dtype=x.dtype)
        if x.dtype == np.float32:
            f = self.lib.ref_blas_sdot
            f.restype = ctypes.c_float
        else:
            f = self.lib.ref_blas_ddot
            f.restype = ctypes.c_double
        return f(ctypes.c_int(x.size), ctypes.c_void_p(x.ctypes.data), ctypes.c_void_p(y.ctypes.data))

    # Only the restatement has these two.
    def scores(self, X, W, nthreads=1):
        """X: (n, d), W: (m, d) C-contiguous -> S (n, m)."""
        n, d = X.shape
        m = W.shape[0]
        S = np.zeros((n, m), dtype=X.dtype)
        f = self.lib.oracle_scores
        f.restype = ctypes.c_int
        rc = f(ctypes.c_int(_dt(X)), ctypes.c_int64(d), ctypes.c_int64(m), ctypes.c_int64(n),
               ctypes.c_void_p(X.ctypes.data), ctypes.c_void_p(W.ctypes.data),
               ctypes.c_void_p(S.ctypes.data), ctypes.c_int(nthreads))
        assert rc == 0
        return S

    def dual_regularizer(self, A, S, result=None):
        """Kernel-input dual regularizer: A, S (n, m) -> (preg, dreg)."""
        data = _dt(A)
        result = data if result is None else result
        preg = ctypes.c_double()
        dreg = ctypes.c_double()
        f = self.lib.oracle_dual_regularizer
        f.restype = ctypes.c_int
        rc = f(ctypes.c_int(data), ctypes.c_int(result), ctypes.c_int64(A.shape[1]),
               ctypes.c_int64(A.shape[0]), ctypes.c_void_p(A.ctypes.data),
               ctypes.c_void_p(S.ctypes.data), ctypes.byref(preg), ctypes.byref(dreg))
        assert rc == 0
        return preg.value, dreg.value

    def regularizers(self, W, W0=None, result=None):
        data = _dt(W)
        result = data if result is None else result
        preg = ctypes.c_double()
        dreg = ctypes.c_double()
        f = self.lib.oracle_regularizers
        f.restype = ctypes.c_int
        rc = f(ctypes.c_int(data), ctypes.c_int(result), ctypes.c_int64(W.size),
               ctypes.c_void_p(W.ctypes.data),
               ctypes.c_void_p(W0.ctypes.data if W0 is not None else None),
               ctypes.byref(preg), ctypes.byref(dreg))
        assert rc == 0
        return preg.value, dreg.value
