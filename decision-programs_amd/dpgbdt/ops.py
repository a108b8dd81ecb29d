"""Kernel-level operators of libdpgbdt_hip.so on torch device tensors.

Every function launches on torch's current stream of the tensors' device, so
torch.cuda.Event timing and ordering with torch work as usual.  Host arrays
(node segments) are numpy/int sequences.
"""
from __future__ import annotations

import ctypes
from ctypes import c_int32, c_void_p

import numpy as np

from . import BinLayout, SplitRecord, TrainParam, check, load

SPLIT_DTYPE = np.dtype([("loss_chg", "<f8"), ("gl", "<i8"), ("hl", "<i8"), ("feature", "<i4"),
                        ("bin", "<i4"), ("default_left", "<i4"), ("valid", "<i4"),
                        ("expand", "<i4"), ("pad", "<i4")])
assert SPLIT_DTYPE.itemsize == ctypes.sizeof(SplitRecord)


def _stream():
    import torch

    return c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return c_void_p(t.data_ptr()) if t is not None else c_void_p(0)


class Workspace:
    """Device scratch reused by the operator entry points."""

    def __init__(self):
        self.handle = c_void_p()
        check(load().dp_workspace_create(ctypes.byref(self.handle)))

    def __del__(self):
        lib = load()
        if getattr(self, "handle", None):
            lib.dp_workspace_free(self.handle)
            self.handle = None


def layout(n_rows, n_features, tile_width=0, missing_bin=-1):
    out = BinLayout()
    check(load().dp_layout_init(n_rows, n_features, tile_width, missing_bin, ctypes.byref(out)))
    return out


def layout_pair_tiles(lay, cut_ptr):
    """Pairs the layout's tiles whose features all have at most 16 bins (host cut_ptr, as
    sketch_cuts returns it); returns the layout (changed in place)."""
    ptr = np.ascontiguousarray(cut_ptr, dtype=np.int32)
    check(load().dp_layout_pair_tiles(ctypes.byref(lay), ptr.ctypes.data))
    return lay


def join_tiles(bins, lay):
    """Writes the joint tiles of a paired layout into device bins (after its n_tiles tiles)."""
    check(load().dp_join_tiles(_ptr(bins), ctypes.byref(lay), _stream()))
    return bins


def layout_bytes(lay):
    return load().dp_layout_bytes(ctypes.byref(lay))


def to_tiles(bins_rowmajor, lay):
    """Host row-major [n, F] uint8 -> tile-major bytes of `lay` (numpy)."""
    n, f = bins_rowmajor.shape
    tw, nt = lay.tile_width, lay.n_tiles
    pad = np.zeros((n, nt * tw), dtype=np.uint8)
    pad[:, :f] = bins_rowmajor
    return np.ascontiguousarray(pad.reshape(n, nt, tw).transpose(1, 0, 2)).reshape(-1)


def from_tiles(tiles, lay):
    """Tile-major bytes -> row-major [n, F] uint8 (numpy)."""
    n, f, tw, nt = lay.n_rows, lay.n_features, lay.tile_width, lay.n_tiles
    return np.ascontiguousarray(tiles.reshape(nt, n, tw).transpose(1, 0, 2).reshape(n, nt * tw)[:, :f])


def sketch_cuts(ws, values, max_bin):
    """Quantile cuts of a device [n, F] float32 tensor -> (cut_ptr, cut_values, mins, missing)."""
    n, f = values.shape
    cut_ptr = np.zeros(f + 1, dtype=np.int32)
    cuts = np.zeros(f * max_bin, dtype=np.float32)
    mins = np.zeros(f, dtype=np.float32)
    has_missing = c_int32()
    check(load().dp_sketch_cuts(ws.handle, _ptr(values), n, f, max_bin, cut_ptr.ctypes.data,
                                cuts.ctypes.data, mins.ctypes.data, ctypes.byref(has_missing),
                                _stream()))
    return cut_ptr, cuts[: cut_ptr[-1]].copy(), mins, bool(has_missing.value)


def bin_values(values, lay, cut_ptr, cut_values):
    """Device bins (tile-major uint8 tensor) of a device float32 matrix."""
    import torch

    dev = values.device
    cp = torch.as_tensor(np.asarray(cut_ptr, dtype=np.int32), device=dev)
    cv = torch.as_tensor(np.asarray(cut_values, dtype=np.float32), device=dev)
    bins = torch.empty(layout_bytes(lay), dtype=torch.uint8, device=dev)
    check(load().dp_bin_values(_ptr(values), ctypes.byref(lay), _ptr(cp), _ptr(cv), _ptr(bins),
                               _stream()))
    return bins


def objective_gradients(objective, margin, label, n_classes):
    import torch

    n = label.shape[0]
    grad = torch.empty((n, n_classes), dtype=torch.float32, device=margin.device)
    hess = torch.empty_like(grad)
    check(load().dp_objective_gradients(objective, _ptr(margin), _ptr(label), n, n_classes,
                                        _ptr(grad), _ptr(hess), _stream()))
    return grad, hess


def quantise(ws, grad, hess):
    """-> (exps [K,2] int32, gpair [K,n,2] int32, sums [K,2] int64) device tensors."""
    import torch

    if grad.dim() == 1:
        grad, hess = grad.reshape(-1, 1), hess.reshape(-1, 1)
    n, k = grad.shape
    dev = grad.device
    exps = torch.empty((k, 2), dtype=torch.int32, device=dev)
    gpair = torch.empty((k, n, 2), dtype=torch.int32, device=dev)
    sums = torch.empty((k, 2), dtype=torch.int64, device=dev)
    check(load().dp_quantise_gradients(ws.handle, _ptr(grad.contiguous()), _ptr(hess.contiguous()),
                                       n, k, _ptr(exps), _ptr(gpair), _ptr(sums), _stream()))
    return exps, gpair, sums


def hist_build(ws, bins, lay, gpair, segments, bin_stride, ridx=None, out=None):
    """Histograms [len(segments), F, bin_stride, 2] int64 of row segments."""
    import torch

    seg = np.asarray(segments, dtype=np.int64).reshape(-1, 2)
    begin = np.ascontiguousarray(seg[:, 0])
    end = np.ascontiguousarray(seg[:, 1])
    n_nodes = seg.shape[0]
    if out is None:
        out = torch.empty((n_nodes, lay.n_features, bin_stride, 2), dtype=torch.int64,
                          device=bins.device)
    check(load().dp_hist_build(ws.handle, _ptr(bins), ctypes.byref(lay), _ptr(gpair), _ptr(ridx),
                               begin.ctypes.data, end.ctypes.data, n_nodes, bin_stride, _ptr(out),
                               _stream()))
    return out


def hist_accumulate(ws, bins, lay, gpair, segments, hist, ridx=None):
    """Adds the histograms of row segments into `hist` [n_nodes, F, stride, 2]."""
    seg = np.asarray(segments, dtype=np.int64).reshape(-1, 2)
    begin = np.ascontiguousarray(seg[:, 0])
    end = np.ascontiguousarray(seg[:, 1])
    check(load().dp_hist_accumulate(ws.handle, _ptr(bins), ctypes.byref(lay), _ptr(gpair),
                                    _ptr(ridx), begin.ctypes.data, end.ctypes.data, seg.shape[0],
                                    hist.shape[2], _ptr(hist), _stream()))
    return hist


def hist_tuning(lay, bin_stride):
    """The autotuner's report for contiguous histograms of this layout ({} before tuning)."""
    import json

    n, out = ctypes.c_uint64(), ctypes.c_char_p()
    check(load().dp_hist_tuning(ctypes.byref(lay), bin_stride, ctypes.byref(n),
                                ctypes.byref(out)))
    return json.loads(ctypes.string_at(out, n.value).decode())


def hist_subtract(parent, built):
    import torch

    out = torch.empty_like(parent)
    check(load().dp_hist_subtract(_ptr(parent), _ptr(built), _ptr(out), parent.numel(), _stream()))
    return out


def train_param(eta=0.3, lam=1.0, alpha=0.0, gamma=0.0, min_child_weight=1.0, max_depth=6):
    return TrainParam(eta, lam, alpha, gamma, min_child_weight, max_depth)


def evaluate_splits(ws, hist, n_bins, node_sums, exp_g, exp_h, param):
    """Best split per node -> device tensor of split records (see splits_to_numpy)."""
    import torch

    n_nodes, f, stride, _ = hist.shape
    out = torch.empty((n_nodes, ctypes.sizeof(SplitRecord)), dtype=torch.uint8, device=hist.device)
    check(load().dp_evaluate_splits(ws.handle, _ptr(hist), n_nodes, f, stride, _ptr(n_bins),
                                    _ptr(node_sums),
                                    int(exp_g), int(exp_h), ctypes.byref(param), _ptr(out),
                                    _stream()))
    return out


def splits_to_numpy(records):
    return np.frombuffer(records.cpu().numpy().tobytes(), dtype=SPLIT_DTYPE)


def partition(ws, bins, lay, ridx_in, segments, splits):
    """Stable partition -> (ridx_out tensor, left_count tensor)."""
    import torch

    seg = np.asarray(segments, dtype=np.int64).reshape(-1, 2)
    begin = np.ascontiguousarray(seg[:, 0])
    end = np.ascontiguousarray(seg[:, 1])
    ridx_out = ridx_in.clone()
    left = torch.zeros(seg.shape[0], dtype=torch.int64, device=bins.device)
    check(load().dp_partition(ws.handle, _ptr(bins), ctypes.byref(lay), _ptr(ridx_in),
                              _ptr(ridx_out), begin.ctypes.data, end.ctypes.data, _ptr(splits),
                              seg.shape[0], _ptr(left), _stream()))
    return ridx_out, left


def update_margin(ws, ridx, segments, values, margin, stride=1):
    seg = np.asarray(segments, dtype=np.int64).reshape(-1, 2)
    begin = np.ascontiguousarray(seg[:, 0])
    end = np.ascontiguousarray(seg[:, 1])
    vals = np.ascontiguousarray(np.asarray(values, dtype=np.float32))
    check(load().dp_update_margin(ws.handle, _ptr(ridx), begin.ctypes.data, end.ctypes.data,
                                  vals.ctypes.data, seg.shape[0], _ptr(margin), stride, _stream()))
    return margin


SYNTH_FEATURES = {1: 8, 2: 28, 3: 128, 4: 784, 5: 1000}


def synth(config, n_rows, seed, device="cuda", n_features=None, want_grad=False):
    """Synthetic benchmark inputs -> (values, labels, grad, hess) device tensors."""
    import torch

    f = n_features or SYNTH_FEATURES[config]
    values = torch.empty((n_rows, f), dtype=torch.float32, device=device)
    labels = torch.empty(n_rows, dtype=torch.float32, device=device)
    grad = hess = None
    if want_grad:
        grad = torch.empty(n_rows, dtype=torch.float32, device=device)
        hess = torch.empty(n_rows, dtype=torch.float32, device=device)
    check(load().dp_synth(config, seed, n_rows, f, _ptr(values), _ptr(labels), _ptr(grad),
                          _ptr(hess), _stream()))
    return values, labels, grad, hess
