"""Python binding of libdpgbdt_hip.so (the MI355X training hot path).

Two layers mirror the two layers of ``include/dpgbdt.h``:

* ``DMatrix`` / ``Booster``: the XGBoost C-API subset the reference trainer
  drives (native/class_native_training.cuh:47-70): create a matrix from a
  device array interface, set labels, create a booster, set parameters,
  ``update(iter)``, save the model JSON.
* ``ops``: the kernel-level operators (histogram, subtraction, split
  evaluation, partition, gradients, quantisation, cuts, binning), taking torch
  device tensors.

torch is used only to own device memory and name streams.  There is no CPU
fallback: loading fails loudly when the HIP library has not been built.
"""
from __future__ import annotations

import ctypes
import json
import os
from ctypes import POINTER, Structure, c_char_p, c_double, c_float, c_int, c_int32, c_int64
from ctypes import c_size_t, c_uint8, c_uint64, c_void_p

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libdpgbdt_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(_HERE)), "include", "dpgbdt.h")

DP_OBJ_LOGISTIC, DP_OBJ_SOFTPROB, DP_OBJ_SQUARED = 0, 1, 2
QUANT_BITS = 30


class DPError(RuntimeError):
    """A call into libdpgbdt_hip.so returned a failure status."""


class BinLayout(Structure):
    _fields_ = [("n_rows", c_int64), ("n_features", c_int32), ("tile_width", c_int32),
                ("n_tiles", c_int32), ("missing_bin", c_int32), ("paired_tiles", c_uint64)]


class TrainParam(Structure):
    _fields_ = [("eta", c_float), ("lambda_", c_float), ("alpha", c_float), ("gamma", c_float),
                ("min_child_weight", c_float), ("max_depth", c_int32)]


class SplitRecord(Structure):
    _fields_ = [("loss_chg", c_double), ("gl", c_int64), ("hl", c_int64), ("feature", c_int32),
                ("bin", c_int32), ("default_left", c_int32), ("valid", c_int32),
                ("expand", c_int32), ("pad", c_int32)]


class TreeView(Structure):
    _fields_ = [("n_nodes", c_int32), ("left_children", POINTER(c_int32)),
                ("right_children", POINTER(c_int32)), ("parents", POINTER(c_int32)),
                ("split_indices", POINTER(c_int32)), ("split_bins", POINTER(c_int32)),
                ("split_conditions", POINTER(c_float)), ("default_left", POINTER(c_uint8)),
                ("base_weights", POINTER(c_float)), ("loss_changes", POINTER(c_float)),
                ("sum_hessian", POINTER(c_float)), ("sum_qg", POINTER(c_int64)),
                ("sum_qh", POINTER(c_int64)), ("row_counts", POINTER(c_int64))]


_lib = None


def load():
    """Loads libdpgbdt_hip.so once; raises when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise DPError(f"{LIB_PATH} is missing: run __graft_entry__.build() first "
                      "(there is no CPU fallback)")
    # A process must hold one HIP runtime.  torch ships its own
    # libamdhip64.so.7 / libhsa-runtime64.so.1; loading torch first lets the
    # dynamic linker satisfy this library's dependencies (same sonames) with
    # torch's copies instead of starting a second runtime that cannot open the
    # device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(LIB_PATH)
    H = c_void_p
    sig = {
        "XGBoostVersion": (None, [POINTER(c_int), POINTER(c_int), POINTER(c_int)]),
        "XGBuildInfo": (c_int, [POINTER(c_char_p)]),
        "XGBGetLastError": (c_char_p, []),
        "XGDMatrixCreateFromCudaArrayInterface": (c_int, [c_char_p, c_char_p, POINTER(H)]),
        "XGDMatrixSetInfoFromInterface": (c_int, [H, c_char_p, c_char_p]),
        "XGDMatrixNumRow": (c_int, [H, POINTER(c_uint64)]),
        "XGDMatrixNumCol": (c_int, [H, POINTER(c_uint64)]),
        "XGDMatrixFree": (c_int, [H]),
        "XGBoosterCreate": (c_int, [POINTER(H), c_uint64, POINTER(H)]),
        "XGBoosterFree": (c_int, [H]),
        "XGBoosterSetParam": (c_int, [H, c_char_p, c_char_p]),
        "XGBoosterUpdateOneIter": (c_int, [H, c_int, H]),
        "XGBoosterTrainOneIter": (c_int, [H, H, c_int, c_char_p, c_char_p]),
        "XGBoosterBoostedRounds": (c_int, [H, POINTER(c_int)]),
        "XGBoosterSaveJsonConfig": (c_int, [H, POINTER(c_uint64), POINTER(c_char_p)]),
        "XGBoosterSaveModel": (c_int, [H, c_char_p]),
        "XGBoosterSaveModelToBuffer": (c_int, [H, c_char_p, POINTER(c_uint64), POINTER(c_char_p)]),
        "XGBoosterPredictFromCudaArray": (c_int, [H, c_char_p, c_char_p, H,
                                                  POINTER(POINTER(c_uint64)), POINTER(c_uint64),
                                                  POINTER(POINTER(ctypes.c_float))]),
        "XGBoosterLoadModelFromBuffer": (c_int, [H, c_void_p, c_uint64]),
        "XGBoosterLoadModel": (c_int, [H, c_char_p]),
        "XGBoosterSlice": (c_int, [H, c_int, c_int, c_int, POINTER(H)]),
        "XGBoosterGetNumFeature": (c_int, [H, POINTER(c_uint64)]),
        "DPValidateHyperparameters": (c_int, [c_char_p, ctypes.c_uint32, POINTER(c_uint64),
                                              POINTER(c_char_p)]),
        "DPBoosterNumTrees": (c_int, [H, POINTER(c_int)]),
        "DPBoosterGetTree": (c_int, [H, c_int, POINTER(TreeView)]),
        "DPBoosterGetMargins": (c_int, [H, c_void_p, c_uint64]),
        "DPBoosterGetLastGradients": (c_int, [H, c_void_p, c_void_p, c_uint64, c_void_p]),
        "DPBoosterGetLastPositions": (c_int, [H, c_void_p, c_uint64]),
        "DPBoosterGetTuning": (c_int, [H, POINTER(c_uint64), POINTER(c_char_p)]),
        "DPDMatrixGetCuts": (c_int, [H, c_int32, c_void_p, c_void_p, c_uint64, POINTER(c_int32)]),
        "dp_workspace_create": (c_int, [POINTER(H)]),
        "dp_workspace_free": (c_int, [H]),
        "dp_layout_init": (c_int, [c_int64, c_int32, c_int32, c_int32, POINTER(BinLayout)]),
        "dp_layout_bytes": (c_size_t, [POINTER(BinLayout)]),
        "dp_layout_pair_tiles": (c_int, [POINTER(BinLayout), c_void_p]),
        "dp_join_tiles": (c_int, [c_void_p, POINTER(BinLayout), c_void_p]),
        "dp_sketch_cuts": (c_int, [H, c_void_p, c_int64, c_int32, c_int32, c_void_p, c_void_p,
                                   c_void_p, POINTER(c_int32), c_void_p]),
        "dp_bin_values": (c_int, [c_void_p, POINTER(BinLayout), c_void_p, c_void_p, c_void_p,
                                  c_void_p]),
        "dp_objective_gradients": (c_int, [c_int32, c_void_p, c_void_p, c_int64, c_int32,
                                           c_void_p, c_void_p, c_void_p]),
        "dp_quantise_gradients": (c_int, [H, c_void_p, c_void_p, c_int64, c_int32, c_void_p,
                                          c_void_p, c_void_p, c_void_p]),
        "dp_hist_build": (c_int, [H, c_void_p, POINTER(BinLayout), c_void_p, c_void_p, c_void_p,
                                  c_void_p, c_int32, c_int32, c_void_p, c_void_p]),
        "dp_hist_accumulate": (c_int, [H, c_void_p, POINTER(BinLayout), c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p]),
        "dp_hist_subtract": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
        "dp_hist_tuning": (c_int, [POINTER(BinLayout), c_int32, POINTER(c_uint64),
                                   POINTER(c_char_p)]),
        "dp_evaluate_splits": (c_int, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                       c_int32, c_int32, POINTER(TrainParam), c_void_p,
                                       c_void_p]),
        "dp_evaluate_splits_noalloc": (c_int, [c_void_p, c_int32, c_int32, c_int32, c_void_p,
                                               c_void_p, c_int32, c_int32, POINTER(TrainParam),
                                               c_void_p, c_void_p]),
        "dp_partition": (c_int, [H, c_void_p, POINTER(BinLayout), c_void_p, c_void_p, c_void_p,
                                 c_void_p, c_void_p, c_int32, c_void_p, c_void_p]),
        "dp_update_margin": (c_int, [H, c_void_p, c_void_p, c_void_p, c_void_p, c_int32,
                                     c_void_p, c_int64, c_void_p]),
        "dp_synth": (c_int, [c_int32, c_uint64, c_int64, c_int32, c_void_p, c_void_p, c_void_p,
                             c_void_p, c_void_p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status):
    if status != 0:
        raise DPError(load().XGBGetLastError().decode())


def version():
    a, b, c = c_int(), c_int(), c_int()
    load().XGBoostVersion(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
    return a.value, b.value, c.value


def build_info():
    out = c_char_p()
    check(load().XGBuildInfo(ctypes.byref(out)))
    return json.loads(out.value.decode())


def array_interface(t):
    """__cuda_array_interface__-style JSON for a contiguous device tensor."""
    import torch

    assert t.is_cuda and t.is_contiguous()
    typestr = {torch.float32: "<f4", torch.int32: "<i4", torch.uint32: "<u4"}[t.dtype]
    return json.dumps({"data": [t.data_ptr(), True], "shape": list(t.shape), "strides": None,
                       "typestr": typestr, "version": 3, "stream": 1})


class DMatrix:
    """Training matrix (copied into library-owned device memory)."""

    def __init__(self, values, labels=None, missing=float("nan")):
        lib = load()
        self.handle = c_void_p()
        cfg = json.dumps({"missing": missing, "nthread": 2}).replace("NaN", "NaN")
        check(lib.XGDMatrixCreateFromCudaArrayInterface(array_interface(values).encode(),
                                                        cfg.encode(), ctypes.byref(self.handle)))
        if labels is not None:
            check(lib.XGDMatrixSetInfoFromInterface(self.handle, b"label",
                                                    array_interface(labels).encode()))

    def num_row(self):
        out = c_uint64()
        check(load().XGDMatrixNumRow(self.handle, ctypes.byref(out)))
        return out.value

    def num_col(self):
        out = c_uint64()
        check(load().XGDMatrixNumCol(self.handle, ctypes.byref(out)))
        return out.value

    def cuts(self, max_bin):
        import numpy as np

        f = self.num_col()
        cut_ptr = np.zeros(f + 1, dtype=np.int32)
        values = np.zeros(f * 256, dtype=np.float32)
        missing = c_int32()
        check(load().DPDMatrixGetCuts(self.handle, max_bin, cut_ptr.ctypes.data,
                                      values.ctypes.data, values.size, ctypes.byref(missing)))
        return cut_ptr, values[: cut_ptr[-1]].copy(), missing.value

    def __del__(self):
        if getattr(self, "handle", None) and _lib is not None:
            _lib.XGDMatrixFree(self.handle)
            self.handle = None


class Booster:
    """XGBoost-style booster over libdpgbdt_hip.so."""

    def __init__(self, params=None, cache=()):
        lib = load()
        self._cache = list(cache)
        arr = (c_void_p * max(1, len(self._cache)))(*[d.handle for d in self._cache])
        self.handle = c_void_p()
        check(lib.XGBoosterCreate(arr, len(self._cache), ctypes.byref(self.handle)))
        for k, v in (params or {}).items():
            self.set_param(k, v)

    def set_param(self, key, value):
        if isinstance(value, bool):
            value = int(value)
        check(load().XGBoosterSetParam(self.handle, key.encode(), str(value).encode()))

    def update(self, dtrain, iteration):
        check(load().XGBoosterUpdateOneIter(self.handle, iteration, dtrain.handle))

    def boost(self, dtrain, iteration, grad, hess):
        check(load().XGBoosterTrainOneIter(self.handle, dtrain.handle, iteration,
                                           array_interface(grad).encode(),
                                           array_interface(hess).encode()))

    def num_features(self):
        out = c_uint64()
        check(load().XGBoosterGetNumFeature(self.handle, ctypes.byref(out)))
        return out.value

    def num_boosted_rounds(self):
        out = c_int()
        check(load().XGBoosterBoostedRounds(self.handle, ctypes.byref(out)))
        return out.value

    def save_config(self):
        n, p = c_uint64(), c_char_p()
        check(load().XGBoosterSaveJsonConfig(self.handle, ctypes.byref(n), ctypes.byref(p)))
        return ctypes.string_at(p, n.value).decode()

    def save_raw(self):
        n, p = c_uint64(), c_char_p()
        check(load().XGBoosterSaveModelToBuffer(self.handle, b'{"format":"json"}',
                                                ctypes.byref(n), ctypes.byref(p)))
        return ctypes.string_at(p, n.value).decode()

    def save_model(self, path):
        check(load().XGBoosterSaveModel(self.handle, str(path).encode()))

    def predict(self, values, margin=False, iteration_begin=0, iteration_end=0, strict=True,
                missing=float("nan")):
        """Device prediction -> torch tensor (a copy of the library-owned output)."""
        import torch

        shape_p = POINTER(c_uint64)()
        dim = c_uint64()
        out = POINTER(ctypes.c_float)()
        cfg = json.dumps({"type": 1 if margin else 0, "training": False,
                          "iteration_begin": iteration_begin, "iteration_end": iteration_end,
                          "strict_shape": bool(strict), "cache_id": 0, "missing": missing})
        check(load().XGBoosterPredictFromCudaArray(self.handle, array_interface(values).encode(),
                                                   cfg.encode(), None, ctypes.byref(shape_p),
                                                   ctypes.byref(dim), ctypes.byref(out)))
        shape = [shape_p[i] for i in range(dim.value)]
        n = 1
        for d in shape:
            n *= d
        # wrap the device pointer with torch through a raw copy
        res = torch.empty(shape, dtype=torch.float32, device=values.device)
        if n:
            import ctypes as _c
            hip = _hip_memcpy()
            hip(_c.c_void_p(res.data_ptr()), _c.c_void_p(_c.addressof(out.contents)), n * 4)
        return res

    @classmethod
    def from_buffer(cls, text):
        b = cls()
        raw = text.encode() if isinstance(text, str) else bytes(text)
        buf = ctypes.create_string_buffer(raw, len(raw))
        check(load().XGBoosterLoadModelFromBuffer(b.handle, buf, len(raw)))
        return b

    def slice(self, begin, end, step=1):
        out = c_void_p()
        check(load().XGBoosterSlice(self.handle, begin, end, step, ctypes.byref(out)))
        b = Booster.__new__(Booster)
        b._cache = []
        b.handle = out
        return b

    def num_trees(self):
        out = c_int()
        check(load().DPBoosterNumTrees(self.handle, ctypes.byref(out)))
        return out.value

    def tree(self, index):
        """Node arrays of one tree as numpy copies."""
        import numpy as np

        v = TreeView()
        check(load().DPBoosterGetTree(self.handle, index, ctypes.byref(v)))
        n = v.n_nodes

        def arr(ptr, dtype):
            return np.ctypeslib.as_array(ptr, shape=(n,)).astype(dtype, copy=True)

        return {
            "left": arr(v.left_children, np.int32), "right": arr(v.right_children, np.int32),
            "parent": arr(v.parents, np.int32), "feature": arr(v.split_indices, np.int32),
            "split_bin": arr(v.split_bins, np.int32),
            "split_condition": arr(v.split_conditions, np.float32),
            "default_left": arr(v.default_left, np.int32),
            "base_weight": arr(v.base_weights, np.float32),
            "loss_chg": arr(v.loss_changes, np.float32), "sum_hess": arr(v.sum_hessian, np.float32),
            "sum_qg": arr(v.sum_qg, np.int64), "sum_qh": arr(v.sum_qh, np.int64),
            "rows": arr(v.row_counts, np.int64),
        }

    def margins(self, n_rows, n_groups):
        import numpy as np

        out = np.zeros((n_rows, n_groups), dtype=np.float32)
        check(load().DPBoosterGetMargins(self.handle, out.ctypes.data, out.size))
        return out

    def last_gradients(self, n_rows, n_groups):
        import numpy as np

        g = np.zeros((n_rows, n_groups), dtype=np.float32)
        h = np.zeros((n_rows, n_groups), dtype=np.float32)
        exps = np.zeros((n_groups, 2), dtype=np.int32)
        check(load().DPBoosterGetLastGradients(self.handle, g.ctypes.data, h.ctypes.data, g.size,
                                               exps.ctypes.data))
        return g, h, exps

    def last_positions(self, n_rows):
        import numpy as np

        out = np.zeros(n_rows, dtype=np.int32)
        check(load().DPBoosterGetLastPositions(self.handle, out.ctypes.data, n_rows))
        return out

    def tuning(self):
        """The histogram launch shapes of the last round (autotuner report)."""
        n, out = c_uint64(), c_char_p()
        check(load().DPBoosterGetTuning(self.handle, ctypes.byref(n), ctypes.byref(out)))
        return json.loads(ctypes.string_at(out, n.value).decode())

    def __del__(self):
        if getattr(self, "handle", None) and _lib is not None:
            _lib.XGBoosterFree(self.handle)
            self.handle = None


_memcpy = None


def _hip_memcpy():
    """hipMemcpy (default kind) from the HIP runtime this process already uses."""
    global _memcpy
    if _memcpy is None:
        import torch  # noqa: F401  (its HIP runtime is the one loaded)

        rt = ctypes.CDLL("libamdhip64.so.7")
        fn = rt.hipMemcpy
        fn.argtypes = [c_void_p, c_void_p, c_size_t, c_int]
        fn.restype = c_int

        def copy(dst, src, nbytes):
            status = fn(dst, src, nbytes, 4)  # hipMemcpyDefault
            if status != 0:
                raise DPError(f"hipMemcpy failed with status {status}")

        _memcpy = copy
    return _memcpy


from . import ops  # noqa: E402  (kernel-level operators)
