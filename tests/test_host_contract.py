"""Host-side contract of the trainer, without a GPU: hyperparameter validation
as the reference performs it before training (native/class_native_training.cuh:16-33,
reached through ResidentTrainer::validate_hyperparameters), including the three
refusals of native/class_study_train_checks.cpp:14 and the accepted case of :13."""
import ctypes
import json

import pytest


def validate(dp, hp, classes=3):
    lib = dp.load()
    n, out = ctypes.c_uint64(), ctypes.c_char_p()
    lib.DPValidateHyperparameters.argtypes = [ctypes.c_char_p, ctypes.c_uint32,
                                              ctypes.POINTER(ctypes.c_uint64),
                                              ctypes.POINTER(ctypes.c_char_p)]
    rc = lib.DPValidateHyperparameters(json.dumps(hp).encode(), classes, ctypes.byref(n),
                                       ctypes.byref(out))
    if rc != 0:
        raise dp.DPError(lib.XGBGetLastError().decode())
    return json.loads(ctypes.string_at(out, n.value).decode())


def test_reference_accepted_case(dp):
    hp = validate(dp, {"rounds": 2, "max_depth": 3}, 3)
    assert hp["rounds"] == 2 and hp["max_depth"] == 3
    assert (hp["max_bin"], hp["seed"], hp["eta"], hp["lambda"], hp["alpha"], hp["gamma"],
            hp["min_child_weight"]) == (256, 0, 0.3, 1.0, 0.0, 0.0, 1.0)
    assert "subsample" not in hp


@pytest.mark.parametrize("hp", [
    {"rounds": 0, "max_depth": 2},
    {"rounds": 2, "max_depth": 2, "unknown": 1},
    {"rounds": 2, "max_depth": 2, "eta": 0.0},
])
def test_reference_refusals(dp, hp):
    with pytest.raises(dp.DPError):
        validate(dp, hp, 3)


@pytest.mark.parametrize("hp,msg", [
    ({"rounds": -1, "max_depth": 2}, "nonnegative"),
    ({"rounds": 2.0, "max_depth": 2}, "integer"),
    ({"rounds": 2, "max_depth": 0}, "positive"),
    ({"max_depth": 2}, "rounds"),
    ({"rounds": 2, "max_depth": 2, "eta": 1.5}, "range"),
    ({"rounds": 2, "max_depth": 2, "lambda": -1}, "range"),
    ({"rounds": 2, "max_depth": 2, "subsample": 0}, "range"),
    ({"rounds": 2, "max_depth": 2, "max_bin": 1}, "max_bin"),
    ({"rounds": 2**31 // 3 + 1, "max_depth": 2}, "capacity"),
    ({"rounds": 2, "max_depth": 2, "gamma": "1"}, "numeric"),
])
def test_more_refusals(dp, hp, msg):
    with pytest.raises(dp.DPError, match=msg):
        validate(dp, hp, 3)


def test_sampling_keys_kept_when_given(dp):
    hp = validate(dp, {"rounds": 5, "max_depth": 4, "subsample": 1, "colsample_bynode": 0.5,
                       "eta": 1, "max_bin": 64, "seed": 7}, 10)
    assert hp["subsample"] == 1.0 and hp["colsample_bynode"] == 0.5
    assert (hp["eta"], hp["max_bin"], hp["seed"]) == (1.0, 64, 7)


def _raw_validate(dp, text, classes=3):
    lib = dp.load()
    n, out = ctypes.c_uint64(), ctypes.c_char_p()
    lib.DPValidateHyperparameters.argtypes = [ctypes.c_char_p, ctypes.c_uint32,
                                              ctypes.POINTER(ctypes.c_uint64),
                                              ctypes.POINTER(ctypes.c_char_p)]
    rc = lib.DPValidateHyperparameters(text.encode(), classes, ctypes.byref(n), ctypes.byref(out))
    return rc, lib.XGBGetLastError().decode()


@pytest.mark.parametrize("depth,msg", [(100, "eta must be numeric"), (600, "nesting deeper")])
def test_json_nesting_is_capped(dp, depth, msg):
    """The JSON reader descends recursively: nesting beyond 512 levels is refused
    with an error instead of exhausting the host stack."""
    text = '{"rounds":2,"max_depth":2,"eta":' + "[" * depth + "]" * depth + "}"
    rc, err = _raw_validate(dp, text)
    assert rc == -1 and msg in err


def test_deeply_nested_model_buffer_is_refused(dp):
    """XGBoosterLoadModelFromBuffer takes caller bytes: a 100,000-deep array
    fails with status -1 (the process survives)."""
    lib = dp.load()
    h = ctypes.c_void_p()
    assert lib.XGBoosterCreate(None, 0, ctypes.byref(h)) == 0
    try:
        buf = b"[" * 100000 + b"]" * 100000
        lib.XGBoosterLoadModelFromBuffer.argtypes = [ctypes.c_void_p, ctypes.c_char_p,
                                                     ctypes.c_uint64]
        assert lib.XGBoosterLoadModelFromBuffer(h, buf, len(buf)) == -1
        assert "nesting deeper" in lib.XGBGetLastError().decode()
    finally:
        lib.XGBoosterFree(h)


def test_train_one_iter_refuses_host_gradients(dp):
    """XGBoosterTrainOneIter's quantiser reads the caller's gradient arrays in place on the
    device, so a host pointer is refused with an error before any launch (without a GPU the
    pointer cannot be device memory either)."""
    import numpy as np

    lib = dp.load()
    h = ctypes.c_void_p()
    assert lib.XGBoosterCreate(None, 0, ctypes.byref(h)) == 0
    try:
        g = np.zeros(16, dtype=np.float32)

        def iface(a):
            return json.dumps({"data": [a.ctypes.data, True], "shape": [16], "strides": None,
                               "typestr": "<f4", "version": 3}).encode()

        rc = lib.XGBoosterTrainOneIter(h, None, 0, iface(g), iface(g))
        assert rc == -1
        assert "grad must be device memory" in lib.XGBGetLastError().decode()
    finally:
        lib.XGBoosterFree(h)


def test_quantum_ratio_closed_forms():
    """bench.py's report of this build's fixed-point step against upstream's: for n rows of
    g = +-1/2 (half each) and h = 1/4, the step here is 2^-30 (g) and 2^-31 (h); upstream
    rounds sum(g > 0) = n/4 and sum(h) = n/4 up to powers of two and divides by 2^62, so with
    n = 2^14 both sums are 2^12 (exactly, so the (1 - 2 n eps) guard lifts them to 2^13)
    and the ratios are 62 - 30 - 13 = 19 and 62 - 31 - 13 = 18.  A sign mix that makes the
    negative sum the larger one must give the same g ratio, and a [min, max] pair is
    reported when outputs differ."""
    import os
    import sys

    import numpy as np

    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench

    n = 1 << 14
    g = np.where(np.arange(n) % 2 == 0, 0.5, -0.5).astype(np.float32).reshape(-1, 1)
    h = np.full((n, 1), 0.25, dtype=np.float32)
    assert bench.quantum_ratio(g, h, [[30, 31]]) == {"g": 19, "h": 18}
    flipped = np.where(np.arange(n) % 4 == 0, 0.5, -0.5).astype(np.float32).reshape(-1, 1)
    # negative sum 3n/8 = 6144: frexp exponent 13 -> the same ratio
    assert bench.quantum_ratio(flipped, h, [[30, 31]])["g"] == 19
    # second output: one row at 2 (max|g| = 2, step 2^-28), the sums still below 2^13
    outlier = g.copy()
    outlier[0, 0] = 2.0
    r = bench.quantum_ratio(np.concatenate([g, outlier], axis=1),
                            np.concatenate([h, h], axis=1), [[30, 31], [28, 31]])
    assert r == {"g": [19, 21], "h": 18}


def test_layout_pair_tiles(dp):
    """dp_layout_pair_tiles: adjacent 16-feature tiles are paired left to right when every
    feature of both has at most 16 bins (pad features count as such); a 17-bin feature breaks
    a pair, a matrix with missing values gets none, and bit 62 is the last pair's."""
    import numpy as np
    from dpgbdt import ops

    def pairs(n_bins, missing_bin=-1):
        lay = ops.layout(100, len(n_bins), 0, missing_bin)
        ptr = np.concatenate([[0], np.cumsum(n_bins)]).astype(np.int32)
        return ops.layout_pair_tiles(lay, ptr).paired_tiles

    nb = np.full(90, 16)  # six tiles, the last with 10 features and 6 pad features
    nb[50] = 17           # tile 3 is wide
    assert pairs(nb) == (1 << 0) | (1 << 4)  # (0, 1), then 2 alone, 3 wide, (4, 5)
    nb[50] = 16
    assert pairs(nb) == (1 << 0) | (1 << 2) | (1 << 4)
    nb[5] = 256           # tile 0 wide: (1, 2), (3, 4), 5 alone
    assert pairs(nb) == (1 << 1) | (1 << 3)
    assert pairs(np.full(90, 2), missing_bin=255) == 0
    assert pairs(np.full(16, 3)) == 0  # one tile: nothing to pair with
    assert pairs(np.full(70 * 16, 8)) == int("01" * 32, 2)  # tiles 0..63 in 32 pairs
    assert ctypes.sizeof(dp.BinLayout) == 32
    lay = ops.layout(100, 90, 0, -1)
    assert ops.layout_bytes(lay) == 6 * 100 * 16
    ops.layout_pair_tiles(lay, np.concatenate([[0], np.cumsum(np.full(90, 16))]))
    assert ops.layout_bytes(lay) == (6 + 3) * 100 * 16  # three joint tiles follow
    lay = ops.layout(100, 40, 0, -1)
    with pytest.raises(dp.DPError, match="cut_ptr must not decrease"):
        ops.layout_pair_tiles(lay, np.array([0, 5, 3] + [3] * 38, dtype=np.int32))
