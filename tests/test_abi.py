"""The C ABI library without a GPU: it loads, exports every entry point that
include/sdca_hip.h declares, and rejects invalid arguments with the status
codes of the Matlab front end's checks (src/matlab/mex_prox.cpp:132-136)
before touching the device."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sdca_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sdca_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for want in ("sdca_prox", "sdca_eval_features", "sdca_eval_kernel", "sdca_eval_scores",
                 "sdca_scores",
                 "sdca_last_error", "sdca_prox_params_default", "sdca_abi_version"):
        assert want in names


def test_library_exports_every_declared_symbol():
    import libsdca_amd as sd
    lib = sd.library()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in sdca_hip.h but not exported"
    assert lib.sdca_abi_version() == 1


def test_params_default():
    import libsdca_amd as sd
    p = sd.ProxParams()
    sd.library().sdca_prox_params_default(ctypes.byref(p))
    assert (p.lo, p.hi, p.rhs, p.rho, p.alpha, p.k, p.p) == (0, 1, 1, 1, 1, 1, 1)


@pytest.mark.parametrize("kw,status", [
    (dict(k=0), 2), (dict(k=6), 2), (dict(rhs=-1.0), 2), (dict(rho=-1.0), 2),
    (dict(alpha=0.0), 2),
])
def test_prox_argument_checks(kw, status):
    import libsdca_amd as sd
    x = np.zeros((3, 5), np.float32)
    with pytest.raises(sd.SdcaError) as e:
        sd.prox("topk_simplex", x, **kw)
    assert e.value.status == status
    assert sd.library().sdca_last_error()


def test_prox_operator_and_precision_checks():
    import libsdca_amd as sd
    x = np.zeros((3, 5), np.float32)
    with pytest.raises(sd.SdcaError) as e:
        sd.prox(42, x)
    assert e.value.status == 7  # LIBSDCA:prox
    with pytest.raises(sd.SdcaError) as e:
        sd.prox("topk_entropy_biased", x, k=6)
    assert e.value.status == 2
    with pytest.raises(sd.SdcaError) as e:
        sd.prox("topk_entropy_biased", x, alpha=0.0)
    assert e.value.status == 2
    with pytest.raises(sd.SdcaError) as e:
        sd.prox("topk_simplex", x, result="long double")
    assert e.value.status == 4
    with pytest.raises(sd.SdcaError) as e:
        sd.prox("two_simplex", x, p=5)
    assert e.value.status == 2
    with pytest.raises(sd.SdcaError) as e:  # the evaluation takes no (double, float) pair
        sd.eval_scores([sd.objective("l2_entropy")], np.zeros((3, 5)), [0, 1, 2], result="float")
    assert e.value.status == 4
    with pytest.raises(sd.SdcaError) as e:
        sd.prox("two_simplex", x, col_p=[1, 9, 1])
    assert e.value.status == 2


def test_eval_argument_checks():
    import libsdca_amd as sd
    X = np.zeros((4, 3), np.float32)
    W = np.zeros((5, 3), np.float32)
    with pytest.raises(sd.SdcaError) as e:  # label out of range (data/output.h:169-182)
        sd.eval_features([sd.objective("l2_entropy")], X, W, [0, 1, 2, 9])
    assert e.value.status == 8
    with pytest.raises(sd.SdcaError) as e:  # k > m - 1
        sd.eval_features([sd.objective("l2_hinge_topk", k=5)], X, W, [0, 1, 2, 3])
    assert e.value.status == 2
    with pytest.raises(sd.SdcaError) as e:  # multilabel objective with multiclass labels
        sd.eval_features([sd.objective("l2_multilabel_hinge")], X, W, [0, 1, 2, 3])
    assert e.value.status == 2
    with pytest.raises(sd.SdcaError) as e:  # unsorted multilabel labels (output.h:201-205)
        sd.eval_features([sd.objective("l2_multilabel_entropy")], X, W, [2, 1, 0, 1, 2, 3],
                         offsets=[0, 2, 3, 4, 6])
    assert e.value.status == 8


HPP_PROGRAM = r"""
#include "sdca_hip.hpp"
#include <vector>
int main() {
  std::vector<float> a(100 * 8, 0.f), aux(100);
  std::vector<double> b(10 * 4, 0.0), bux(10);
  float* f = a.data();
  double* d = b.data();
  // the reference's batched call shapes (topk_simplex.h, topk_cone.h, ...)
  sdca::hip::prox_topk_simplex(100, f, f + a.size(), aux.data(), 5, 1.0f);
  sdca::hip::prox_topk_cone(100, f, f + a.size(), aux.data(), 5);
  sdca::hip::prox_knapsack_eq(10, d, d + b.size(), bux.data(), 0.0, 1.0, 1.0);
  sdca::hip::prox_knapsack_le(10, d, d + b.size(), bux.data(), 0.0, 1.0, 1.0);
  sdca::hip::prox_entropy(10, d, d + b.size(), bux.data(), 1.0, 1.0);
  sdca::hip::prox_entropy_norm(10, d, d + b.size(), bux.data(), 1.0, 1.0);
  sdca::hip::prox_topk_entropy(10, d, d + b.size(), bux.data(), 2);
  sdca::hip::prox_two_simplex(10, 3, d, d + b.size(), bux.data(), 1.0);
  sdca::hip::apply_lambert_w_exp(10, d, d + b.size());
  sdca::hip::prox_knapsack_le_biased(10, d, d + b.size(), bux.data(), 0.0, 1.0, 1.0, 0.5);
  sdca::hip::prox_topk_simplex_biased(100, f, f + a.size(), aux.data(), 5, 1.0f, 0.5f);
  sdca::hip::prox_topk_cone_biased(100, f, f + a.size(), aux.data(), 5, 0.5f);
  sdca::hip::prox_topk_entropy_biased(100, f, f + a.size(), aux.data(), 5, 0.5f);
  sdca::hip::prox_two_entropy(100, 3, f, f + a.size(), aux.data(), 0.5f);
  std::vector<sdca_objective> objs(1);
  objs[0].kind = SDCA_OBJ_ENTROPY; objs[0].c = 1; objs[0].gamma = 1; objs[0].k = 1;
  std::vector<int64_t> y(4, 0);
  std::vector<float> X(3 * 4), W(3 * 5);
  std::vector<sdca::hip::eval_record> r =
      sdca::hip::evaluate_features<float>(objs, 3, 5, 4, X.data(), W.data(), y);
  std::vector<float> K(4 * 4), A(5 * 4);
  std::vector<sdca::hip::eval_record> rk =
      sdca::hip::evaluate_kernel<float>(objs, 4, 5, 4, K.data(), A.data(), y,
                                        std::vector<int64_t>(), true);
  std::vector<float> Wn(3 * 5);
  sdca::hip::recompute_primal<float>(3, 5, 4, X.data(), A.data(), W.data(), Wn.data());
  return r.empty() || rk.empty();
}
"""


def test_cpp_header_compiles_and_links(tmp_path):
    """include/sdca_hip.hpp is plain C++11 and links against the C ABI library."""
    import shutil
    import subprocess
    import libsdca_amd as sd
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    src = tmp_path / "use_hpp.cpp"
    src.write_text(HPP_PROGRAM)
    libdir = os.path.dirname(sd.LIB_PATH)
    cmd = [gxx, "-std=c++11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src),
           "-o", str(tmp_path / "use_hpp"), "-L", libdir, "-l:" + os.path.basename(sd.LIB_PATH),
           "-Wl,--allow-shlib-undefined"]
    out = subprocess.run(cmd, capture_output=True, text=True)
    assert out.returncode == 0, out.stderr


def test_wrapper_shape_and_type_checks():
    """The Python layer hands raw pointers to the C ABI: arrays whose shape,
    element type or layout does not match are refused before any call."""
    import libsdca_amd as sd
    x = np.zeros((3, 5), np.float32)
    bad_out = [np.zeros((3, 4), np.float32), np.zeros((3, 5), np.float64),
               np.zeros((5, 3), np.float32).T]
    for out in bad_out:
        with pytest.raises(sd.SdcaError):
            sd.prox("topk_simplex", x, out=out, k=2)
    with pytest.raises(sd.SdcaError):
        sd.prox("two_simplex", x, col_p=[1, 2], p=1)  # one entry per column
    X = np.zeros((4, 3), np.float32)
    W = np.zeros((5, 3), np.float32)
    obj = [sd.objective("l2_entropy")]
    for kw in (dict(W=np.zeros((5, 2), np.float32)), dict(W=np.zeros((5, 3), np.float64)),
               dict(A=np.zeros((4, 4), np.float32)), dict(W0=np.zeros((4, 3), np.float32))):
        args = dict(W=W, A=None, W0=None)
        args.update(kw)
        with pytest.raises(sd.SdcaError):
            sd.eval_features(obj, X, args["W"], [0, 1, 2, 3], A=args["A"], W0=args["W0"])
    with pytest.raises(sd.SdcaError) as e:
        sd.eval_features(obj, X, W, [0, 1, 2])  # one label short
    assert e.value.status == 8
    ml = [sd.objective("l2_multilabel_entropy")]
    with pytest.raises(sd.SdcaError) as e:
        sd.eval_features(ml, X, W, [0, 1, 2, 3, 4], offsets=[0, 2, 3, 4])  # n + 1 offsets needed
    assert e.value.status == 8
    with pytest.raises(sd.SdcaError) as e:
        sd.eval_features(ml, X, W, [0, 1, 2, 3, 4], offsets=[0, 2, 3, 4, 6])  # ends past the labels
    assert e.value.status == 8
    with pytest.raises(sd.SdcaError):
        sd.eval_kernel(obj, np.zeros((4, 4), np.float32), np.zeros((3, 5), np.float32), [0, 1, 2, 3])
    with pytest.raises(sd.SdcaError):
        sd.scores(X, np.zeros((5, 4), np.float32))
    with pytest.raises(sd.SdcaError):
        sd.recompute_primal(X, np.zeros((3, 5), np.float32))
    torch = pytest.importorskip("torch")
    with pytest.raises(sd.SdcaError):
        sd.scores(X, torch.zeros((5, 3)))  # numpy and torch mixed


def test_epoch_label_structure_checks():
    """The epoch refuses label arrays whose CSR structure would make it read
    outside them, before touching the device: labels shorter than the
    offsets say, offsets that do not start at 0 or that decrease (the Python
    layer), and the same offsets handed to the C ABI directly."""
    import libsdca_amd as sd
    n, d, m = 4, 3, 6
    X = np.zeros((n, d), np.float32)
    W = np.zeros((m, d), np.float32)
    A = np.zeros((n, m), np.float32)
    ml = ("l2_multilabel_entropy", 1.0, 1.0, 1)
    for labels, offsets in (([0, 1, 2], [0, 1, 2, 3, 4]),       # one label short
                            ([0, 1, 2, 3], [-1, 1, 2, 3, 4]),   # negative start
                            ([0, 1, 2, 3], [1, 1, 2, 3, 4]),    # does not start at 0
                            ([0, 1, 2, 3], [0, 2, 1, 3, 4])):   # decreasing
        with pytest.raises(sd.SdcaError) as e:
            sd.epoch_features(ml, X, W, A, labels, offsets=offsets)
        assert e.value.status == 8, (labels, offsets)
    with pytest.raises(sd.SdcaError) as e:
        sd.epoch_features(("l2_hinge_topk", 1.0, 1.0, 1), X, W, A, [0, 1, 2])  # one label short
    assert e.value.status == 8
    lib = sd.library()
    obj = sd._objs([ml])
    lab = np.array([0, 1, 2, 3], np.int64)
    for off in ([-1, 1, 2, 3, 4], [0, 2, 1, 3, 4]):
        o = np.array(off, np.int64)
        rc = lib.sdca_epoch_features(obj, ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int64(d),
                                     ctypes.c_int64(m), ctypes.c_int64(n),
                                     ctypes.c_void_p(X.ctypes.data), ctypes.c_void_p(W.ctypes.data),
                                     ctypes.c_void_p(A.ctypes.data),
                                     ctypes.c_void_p(lab.ctypes.data),
                                     ctypes.c_void_p(o.ctypes.data), None, ctypes.c_int64(n),
                                     None, ctypes.c_uint(1), None)
        assert rc == 8, lib.sdca_last_error()
