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
    for want in ("sdca_prox", "sdca_eval_features", "sdca_eval_scores", "sdca_scores",
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
        sd.prox("two_simplex_sort", x)
    assert e.value.status == 4  # not on this path
    with pytest.raises(sd.SdcaError) as e:
        sd.prox("topk_simplex", x, result="long double")
    assert e.value.status == 4
    with pytest.raises(sd.SdcaError) as e:
        sd.prox("two_simplex", x, p=5)
    assert e.value.status == 2
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
