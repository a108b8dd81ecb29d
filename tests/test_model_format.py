"""Model-JSON contract and the C-ABI surface, without a GPU.

* The reference's own fixture (cmake/fixtures/xgboost-parser.json, copied to
  tests/golden/) is accepted by the restated reader, and the 23 malformed
  variants listed at the reference's class_io_checks.cpp:46-78 are rejected.
* libdpgbdt_hip.so loads and exports every function include/dpgbdt.h
  declares; the calls that touch no device return what the reference's
  adapter checks (class_model_native_adapter.cuh:24).
"""
import copy
import ctypes
import json
import os
import re

import pytest

import model_reader

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "xgboost-parser.json")


def _fixture():
    with open(FIXTURE) as f:
        return json.load(f)


def _tree(j):
    return j["learner"]["gradient_booster"]["model"]["trees"][0]


def _ens(j):
    return j["learner"]["gradient_booster"]["model"]


def _backward(j):
    t = _tree(j)
    t["tree_param"]["num_nodes"] = "5"
    t["left_children"] = [3, -1, -1, 1, -1]
    t["right_children"] = [4, -1, -1, 2, -1]
    t["split_indices"] = [0, 0, 0, 0, 0]
    t["split_conditions"] = [0.5, -1.0, 1.0, 0.25, 2.0]
    t["split_type"] = [0, 0, 0, 0, 0]
    t["default_left"] = [True, False, False, True, False]


def _permuted(j):
    t = _tree(j)
    t["left_children"][0], t["right_children"][0] = t["right_children"][0], t["left_children"][0]


MALFORMED = {
    "non-unit-weight": lambda j: _ens(j).__setitem__("weight_drop", [0.5]),
    "weight-count": lambda j: _ens(j).__setitem__("weight_drop", [1.0, 1.0]),
    "weight-object": lambda j: _ens(j).__setitem__("weight_drop", {}),
    "weight-string": lambda j: _ens(j).__setitem__("weight_drop", ["1"]),
    "weight-null": lambda j: _ens(j).__setitem__("weight_drop", [None]),
    "permuted-successors": _permuted,
    "backward-successors": _backward,
    "wrong-version": lambda j: j.__setitem__("version", [3, 4, 0]),
    "fractional-version": lambda j: j["version"].__setitem__(0, 3.0),
    "decimal-suffix": lambda j: j["learner"]["learner_model_param"].__setitem__("num_feature", "54junk"),
    "fractional-channel": lambda j: _ens(j)["tree_info"].__setitem__(0, 0.5),
    "wrong-tree-id": lambda j: _tree(j).__setitem__("id", 2),
    "wrong-node-count": lambda j: _tree(j)["tree_param"].__setitem__("num_nodes", "1"),
    "wrong-tree-count": lambda j: _ens(j)["gbtree_model_param"].__setitem__("num_trees", "2"),
    "wrong-iteration-start": lambda j: _ens(j).__setitem__("iteration_indptr", [1, 1]),
    "wrong-iteration-end": lambda j: _ens(j).__setitem__("iteration_indptr", [0, 0]),
    "unordered-iterations": lambda j: _ens(j).__setitem__("iteration_indptr", [0, 2, 1]),
    "invalid-default": lambda j: _tree(j)["default_left"].__setitem__(0, 2),
    "fractional-default": lambda j: _tree(j)["default_left"].__setitem__(0, 1.0),
    "fractional-feature": lambda j: _tree(j)["split_indices"].__setitem__(0, 0.5),
    "wrong-split-array": lambda j: _tree(j).__setitem__("split_type", []),
    "shared-successor": lambda j: _tree(j)["right_children"].__setitem__(0, _tree(j)["left_children"][0]),
    "cycle": lambda j: _tree(j)["left_children"].__setitem__(0, 0),
}


def test_reference_fixture_accepted():
    f, k, trees = model_reader.read_model(_fixture(), converter_rules=True)
    assert (f, k, len(trees)) == (2, 2, 1)
    for weights in ([], [1.0]):
        j = _fixture()
        _ens(j)["weight_drop"] = weights
        model_reader.read_model(j, converter_rules=True)


@pytest.mark.parametrize("name", sorted(MALFORMED))
def test_reference_malformed_cases_rejected(name):
    j = copy.deepcopy(_fixture())
    MALFORMED[name](j)
    with pytest.raises((model_reader.ModelError, KeyError, TypeError, ValueError)):
        model_reader.read_model(j, converter_rules=True)


def test_malformed_case_count_matches_reference():
    assert len(MALFORMED) == 23  # the list at class_io_checks.cpp:46-78


def test_fixture_routing():
    """split_conditions [0.5, leaf -1, leaf 1]: x0 < 0.5 -> node 1, NaN -> default left."""
    import numpy as np

    x = np.array([[0.2, 0.0], [0.5, 0.0], [np.nan, 0.0]], dtype=np.float32)
    m = model_reader.predict_margin(_fixture(), x)
    np.testing.assert_array_equal(m[:, 0], [-1.0, 1.0, -1.0])


def _declared_functions():
    with open(os.path.join(os.path.dirname(HERE), "include", "dpgbdt.h")) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(\w+)\s*\(", text, flags=re.M)
    return sorted({n for n in names if n not in ("if", "while", "return", "sizeof")})


def test_library_exports_every_declared_symbol(dp):
    lib = dp.load()
    declared = _declared_functions()
    assert "XGBoosterUpdateOneIter" in declared and "dp_hist_build" in declared
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing
    assert len(declared) >= 35


def test_version_and_build_info(dp):
    assert dp.version() == (3, 4, 1)
    info = dp.build_info()
    assert info["USE_CUDA"] is True and info["GPU_ARCH"] == "gfx950"


def test_errors_are_reported_not_raised(dp):
    lib = dp.load()
    out = ctypes.c_void_p()
    rc = lib.XGDMatrixCreateFromCudaArrayInterface(b"{not json", b"{}", ctypes.byref(out))
    assert rc == -1
    assert lib.XGBGetLastError()
    rc = lib.XGBoosterSetParam(None, b"eta", b"0.3")
    assert rc == -1 and b"null" in lib.XGBGetLastError()


def test_num_feature_of_an_empty_booster(dp):
    """XGBoosterGetNumFeature, which the converter's native oracle calls right after
    loading a model (native/class_model_convert.cpp:112): 0 for a booster with neither a
    model nor a training matrix, and a null output pointer is an error.  A loaded model's
    count is checked on the GPU (test_gpu_booster.py::test_resident_model_sequence)."""
    lib = dp.load()
    h = ctypes.c_void_p()
    assert lib.XGBoosterCreate(None, 0, ctypes.byref(h)) == 0
    try:
        n = ctypes.c_uint64(99)
        assert lib.XGBoosterGetNumFeature(h, ctypes.byref(n)) == 0 and n.value == 0
        assert lib.XGBoosterGetNumFeature(h, None) == -1
        assert b"null" in lib.XGBGetLastError()
    finally:
        lib.XGBoosterFree(h)
