"""ctypes wrapper of oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
as the checker; the product library never uses it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, Structure, c_double, c_float, c_int32, c_int64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

OBJ_LOGISTIC, OBJ_SOFTPROB, OBJ_SQUARED = 0, 1, 2
QBITS = 30


class Params(Structure):
    _fields_ = [("eta", c_float), ("lambda_", c_float), ("alpha", c_float), ("gamma", c_float),
                ("min_child_weight", c_float), ("max_depth", c_int32)]


class Split(Structure):
    _fields_ = [("loss_chg", c_double), ("feature", c_int32), ("bin", c_int32),
                ("default_left", c_int32), ("valid", c_int32), ("gl", c_int64), ("hl", c_int64)]


class Sampling(Structure):
    _fields_ = [("seed", ctypes.c_uint64), ("round", c_int32), ("output", c_int32),
                ("subsample", c_float), ("colsample_bytree", c_float),
                ("colsample_bylevel", c_float), ("colsample_bynode", c_float)]


class Tree(Structure):
    _fields_ = [("n_nodes", c_int32)] + [
        (n, POINTER(c_int32)) for n in ("left", "right", "parent", "feature", "split_bin",
                                        "default_left")
    ] + [(n, POINTER(c_float)) for n in ("split_condition", "base_weight", "leaf_value",
                                          "loss_chg", "sum_hess")] + [
        ("sum_qg", POINTER(c_int64)), ("sum_qh", POINTER(c_int64)),
        ("seg_begin", POINTER(c_int32)), ("seg_end", POINTER(c_int32))]


_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        lib = ctypes.CDLL(LIB_PATH)
        P = c_void_p
        lib.dpo_compute_cuts.argtypes = [P, c_int64, c_int64, c_int32, P, P, P]
        lib.dpo_compute_cuts.restype = c_int32
        lib.dpo_bin_matrix.argtypes = [P, c_int64, c_int64, P, P, c_int32, P]
        lib.dpo_expf.argtypes = [c_float]
        lib.dpo_expf.restype = c_float
        lib.dpo_gradients.argtypes = [c_int32, P, P, c_int64, c_int32, P, P]
        lib.dpo_quantiser.argtypes = [P, P, c_int64, c_int64, P, P]
        lib.dpo_quantise.argtypes = [P, P, c_int64, c_int64, c_int32, c_int32, P, P]
        lib.dpo_unscale.argtypes = [c_int32]
        lib.dpo_unscale.restype = c_double
        lib.dpo_hist.argtypes = [P, c_int64, P, P, P, c_int64, c_int32, c_int32, P]
        lib.dpo_hist_parallel.argtypes = [P, c_int64, P, P, c_int64, c_int32, c_int32, c_int32, P]
        lib.dpo_hist_subtract.argtypes = [P, P, c_int64, P]
        lib.dpo_calc_gain.argtypes = [POINTER(Params), c_double, c_double]
        lib.dpo_calc_gain.restype = c_double
        lib.dpo_calc_weight.argtypes = [POINTER(Params), c_double, c_double]
        lib.dpo_calc_weight.restype = c_double
        lib.dpo_evaluate_split.argtypes = [P, c_int64, c_int32, P, c_int64, c_int64, c_double,
                                           c_double, POINTER(Params), POINTER(Split)]
        lib.dpo_partition.argtypes = [P, c_int64, c_int64, P, c_int64, c_int32, c_int32, c_int32,
                                      c_int32, P]
        lib.dpo_partition.restype = c_int64
        lib.dpo_grow_tree.argtypes = [P, c_int64, c_int64, P, P, c_int32, P, P, c_int32, c_int32,
                                      POINTER(Params), c_int32, P, POINTER(Tree)]
        lib.dpo_grow_tree.restype = c_int32
        lib.dpo_grow_tree_sampled.argtypes = [P, c_int64, c_int64, P, P, c_int32, P, P, c_int32,
                                              c_int32, POINTER(Params), c_int32,
                                              POINTER(Sampling), P, POINTER(Tree)]
        lib.dpo_grow_tree_sampled.restype = c_int32
        lib.dpo_evaluate_split_masked.argtypes = [P, c_int64, c_int32, P, c_int64, c_int64,
                                                  c_double, c_double, POINTER(Params), P,
                                                  POINTER(Split)]
        lib.dpo_mix64.argtypes = [ctypes.c_uint64]
        lib.dpo_mix64.restype = ctypes.c_uint64
        lib.dpo_sample_prefix.argtypes = [ctypes.c_uint64] * 4
        lib.dpo_sample_prefix.restype = ctypes.c_uint64
        lib.dpo_sample_draw.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        lib.dpo_sample_draw.restype = ctypes.c_uint32
        lib.dpo_stage_keep.argtypes = [c_float, c_int32]
        lib.dpo_stage_keep.restype = c_int32
        lib.dpo_sample_rows.argtypes = [POINTER(Sampling), c_int64, P]
        lib.dpo_colsample.argtypes = [POINTER(Sampling), c_int32, c_int32, c_int64, P]
        lib.dpo_set_threads.argtypes = [c_int32]
        lib.dpo_get_threads.restype = c_int32
        lib.dpo_tree_free.argtypes = [POINTER(Tree)]
        lib.dpo_tree_update_margin.argtypes = [POINTER(Tree), P, P, c_int64]
        lib.dpo_predict_tree.argtypes = [POINTER(Tree), P]
        lib.dpo_predict_tree.restype = c_float
        _lib = lib
    return _lib


def _p(a):
    # data_as keeps a reference to the array, so a temporary made in the call's
    # argument list (np.ascontiguousarray of a strided view) lives until the
    # call returns instead of being freed before the C code reads it.
    return a.ctypes.data_as(c_void_p) if a is not None else c_void_p(0)


def params(eta=0.3, lam=1.0, alpha=0.0, gamma=0.0, min_child_weight=1.0, max_depth=6):
    return Params(eta, lam, alpha, gamma, min_child_weight, max_depth)


def effective_max_bin(max_bin, has_missing):
    """The bins the cuts are computed with: max_bin (at most 256) whether or not values are
    missing (the missing marker gets a symbol of its own; see missing_symbol)."""
    del has_missing
    return min(max_bin, 256)


def missing_symbol(cut_ptr, has_missing):
    """The bin symbol that marks a missing value: -1 without missing values, 255 when every
    feature has at most 255 bins (uint8 symbols), else 256 (uint16 symbols: some feature uses
    all 256 bins and values are missing)."""
    if not has_missing:
        return -1
    return 256 if int(np.diff(np.asarray(cut_ptr)).max()) > 255 else 255


def _bins(bins, missing_bin):
    """Contiguous symbols of the width missing_bin implies (uint16 for 256)."""
    wide = missing_bin > 255
    if not wide:
        assert bins.dtype == np.uint8, "uint8 symbols expected"
    return np.ascontiguousarray(bins, dtype=np.uint16 if wide else np.uint8)


def compute_cuts(x, max_bin):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, f = x.shape
    cut_ptr = np.zeros(f + 1, dtype=np.int32)
    cuts = np.zeros(f * max_bin, dtype=np.float32)
    mins = np.zeros(f, dtype=np.float32)
    rc = load().dpo_compute_cuts(_p(x), n, f, max_bin, _p(cut_ptr), _p(cuts), _p(mins))
    assert rc == 0
    return cut_ptr, cuts[: cut_ptr[-1]].copy(), mins


def bin_matrix(x, cut_ptr, cuts, missing_bin):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, f = x.shape
    bins = np.zeros((n, f), dtype=np.uint16 if missing_bin > 255 else np.uint8)
    load().dpo_bin_matrix(_p(x), n, f, _p(np.ascontiguousarray(cut_ptr, dtype=np.int32)),
                          _p(np.ascontiguousarray(cuts, dtype=np.float32)), missing_bin, _p(bins))
    return bins


def expf(x):
    return load().dpo_expf(float(x))


def gradients(objective, margin, label, n_classes):
    margin = np.ascontiguousarray(margin, dtype=np.float32)
    label = np.ascontiguousarray(label, dtype=np.float32)
    n = label.shape[0]
    g = np.zeros((n, n_classes), dtype=np.float32)
    h = np.zeros((n, n_classes), dtype=np.float32)
    load().dpo_gradients(objective, _p(margin), _p(label), n, n_classes, _p(g), _p(h))
    return g, h


def quantise(g, h):
    """Per column: (exp_g, exp_h, qg, qh); g/h are [n] or [n, K]."""
    g = np.ascontiguousarray(g, dtype=np.float32)
    h = np.ascontiguousarray(h, dtype=np.float32)
    if g.ndim == 1:
        g, h = g[:, None], h[:, None]
    n, k = g.shape
    out = []
    for c in range(k):
        gc = np.ascontiguousarray(g[:, c])
        hc = np.ascontiguousarray(h[:, c])
        eg, eh = c_int32(), c_int32()
        load().dpo_quantiser(_p(gc), _p(hc), n, 1, ctypes.byref(eg), ctypes.byref(eh))
        qg = np.zeros(n, dtype=np.int32)
        qh = np.zeros(n, dtype=np.int32)
        load().dpo_quantise(_p(gc), _p(hc), n, 1, eg.value, eh.value, _p(qg), _p(qh))
        out.append((eg.value, eh.value, qg, qh))
    return out


def unscale(e):
    return load().dpo_unscale(e)


def hist(bins, qg, qh, rows=None, bin_stride=256, missing_bin=-1):
    bins = _bins(bins, missing_bin)
    n, f = bins.shape
    out = np.zeros((f, bin_stride, 2), dtype=np.int64)
    r = None if rows is None else np.ascontiguousarray(rows, dtype=np.uint32)
    nr = n if rows is None else r.shape[0]
    load().dpo_hist(_p(bins), f, _p(np.ascontiguousarray(qg, dtype=np.int32)),
                    _p(np.ascontiguousarray(qh, dtype=np.int32)), _p(r), nr, bin_stride,
                    missing_bin, _p(out))
    return out


def hist_parallel(bins, qg, qh, bin_stride=256, missing_bin=-1, threads=0):
    bins = np.ascontiguousarray(bins, dtype=np.uint8)
    n, f = bins.shape
    out = np.zeros((f, bin_stride, 2), dtype=np.int64)
    load().dpo_hist_parallel(_p(bins), f, _p(np.ascontiguousarray(qg, dtype=np.int32)),
                             _p(np.ascontiguousarray(qh, dtype=np.int32)), n, bin_stride,
                             missing_bin, threads, _p(out))
    return out


def calc_gain(p, g, h):
    return load().dpo_calc_gain(ctypes.byref(p), g, h)


def calc_weight(p, g, h):
    return load().dpo_calc_weight(ctypes.byref(p), g, h)


def evaluate_split(hist_, n_bins, gp, hp, exp_g, exp_h, p):
    hist_ = np.ascontiguousarray(hist_, dtype=np.int64)
    f, stride, _ = hist_.shape
    s = Split()
    load().dpo_evaluate_split(_p(hist_), f, stride, _p(np.ascontiguousarray(n_bins, dtype=np.int32)),
                              int(gp), int(hp), unscale(exp_g), unscale(exp_h), ctypes.byref(p),
                              ctypes.byref(s))
    return {"loss_chg": s.loss_chg, "feature": s.feature, "bin": s.bin,
            "default_left": s.default_left, "valid": s.valid, "gl": s.gl, "hl": s.hl}


def partition(ridx, begin, end, bins, feature, split_bin, default_left, missing_bin):
    ridx = np.array(ridx, dtype=np.uint32, copy=True)
    bins = _bins(bins, missing_bin)
    scratch = np.zeros(max(1, end - begin), dtype=np.uint32)
    nl = load().dpo_partition(_p(ridx), begin, end, _p(bins), bins.shape[1], feature, split_bin,
                              default_left, missing_bin, _p(scratch))
    return ridx, nl


def set_threads(n):
    """OpenMP threads of the oracle's cuts, binning, histograms, split search and partition
    (1: serial); results are identical for any count."""
    load().dpo_set_threads(int(n))


def get_threads():
    return load().dpo_get_threads()


def sampling(seed=0, round_=0, output=0, subsample=1.0, bytree=1.0, bylevel=1.0, bynode=1.0):
    return Sampling(seed, round_, output, subsample, bytree, bylevel, bynode)


def mix64(z):
    return load().dpo_mix64(z)


def sample_rows(smp, n):
    keep = np.zeros(n, dtype=np.uint8)
    load().dpo_sample_rows(ctypes.byref(smp), n, _p(keep))
    return keep.astype(bool)


def colsample(smp, depth, nid, n_features):
    allowed = np.zeros(n_features, dtype=np.uint8)
    load().dpo_colsample(ctypes.byref(smp), depth, nid, n_features, _p(allowed))
    return allowed.astype(bool)


def stage_keep(fraction, m):
    return load().dpo_stage_keep(fraction, m)


def evaluate_split_masked(hist_, n_bins, gp, hp, exp_g, exp_h, p, allowed):
    hist_ = np.ascontiguousarray(hist_, dtype=np.int64)
    f, stride, _ = hist_.shape
    s = Split()
    a = np.ascontiguousarray(allowed, dtype=np.uint8)
    load().dpo_evaluate_split_masked(_p(hist_), f, stride,
                                     _p(np.ascontiguousarray(n_bins, dtype=np.int32)), int(gp),
                                     int(hp), unscale(exp_g), unscale(exp_h), ctypes.byref(p),
                                     _p(a), ctypes.byref(s))
    return {"loss_chg": s.loss_chg, "feature": s.feature, "bin": s.bin,
            "default_left": s.default_left, "valid": s.valid, "gl": s.gl, "hl": s.hl}


def grow_tree(bins, cut_ptr, cuts, missing_bin, qg, qh, exp_g, exp_h, p, bin_stride=256,
              smp=None):
    """One tree -> (dict of node arrays, final ridx); smp: column sampling (Sampling)."""
    bins = _bins(bins, missing_bin)
    n, f = bins.shape
    ridx = np.arange(n, dtype=np.uint32)
    t = Tree()
    rc = load().dpo_grow_tree_sampled(_p(bins), n, f,
                                      _p(np.ascontiguousarray(cut_ptr, dtype=np.int32)),
                                      _p(np.ascontiguousarray(cuts, dtype=np.float32)),
                                      missing_bin, _p(np.ascontiguousarray(qg, dtype=np.int32)),
                                      _p(np.ascontiguousarray(qh, dtype=np.int32)), exp_g, exp_h,
                                      ctypes.byref(p), bin_stride,
                                      ctypes.byref(smp) if smp is not None else None, _p(ridx),
                                      ctypes.byref(t))
    assert rc == 0
    k = t.n_nodes

    def a(ptr, dt):
        return np.ctypeslib.as_array(ptr, shape=(k,)).astype(dt, copy=True)

    out = {
        "left": a(t.left, np.int32), "right": a(t.right, np.int32), "parent": a(t.parent, np.int32),
        "feature": a(t.feature, np.int32), "split_bin": a(t.split_bin, np.int32),
        "default_left": a(t.default_left, np.int32),
        "split_condition": a(t.split_condition, np.float32),
        "base_weight": a(t.base_weight, np.float32), "leaf_value": a(t.leaf_value, np.float32),
        "loss_chg": a(t.loss_chg, np.float32), "sum_hess": a(t.sum_hess, np.float32),
        "sum_qg": a(t.sum_qg, np.int64), "sum_qh": a(t.sum_qh, np.int64),
        "seg_begin": a(t.seg_begin, np.int32), "seg_end": a(t.seg_end, np.int32),
    }
    load().dpo_tree_free(ctypes.byref(t))
    return out, ridx


def positions(tree, ridx, n):
    """Leaf id of every row from the tree's leaf segments."""
    pos = np.full(n, -1, dtype=np.int32)
    for nid in range(len(tree["left"])):
        if tree["left"][nid] == -1:
            pos[ridx[tree["seg_begin"][nid]:tree["seg_end"][nid]]] = nid
    return pos


def predict_tree(tree, x):
    """Leaf value of every row of float matrix x by walking the tree (x < cond -> left)."""
    x = np.asarray(x, dtype=np.float32)
    out = np.zeros(x.shape[0], dtype=np.float32)
    left, right, feat, cond, dl = (tree["left"], tree["right"], tree["feature"],
                                   tree["split_condition"], tree["default_left"])
    for i in range(x.shape[0]):
        nid = 0
        while left[nid] != -1:
            v = x[i, feat[nid]]
            if np.isnan(v):
                nid = left[nid] if dl[nid] else right[nid]
            else:
                nid = left[nid] if v < cond[nid] else right[nid]
        out[i] = tree["leaf_value"][nid] if "leaf_value" in tree else cond[nid]
    return out


def train(bins, cut_ptr, cuts, missing_bin, objective, labels, n_classes, p, rounds,
          base_margin=0.0, bin_stride=256, injected=None, sample=None):
    """Whole booster on the CPU: per round gradients -> quantise -> K trees -> margins.

    injected: optional callable(round) -> (g [n,K], h [n,K]) replacing the objective.
    sample: optional dict(seed, subsample, bytree, bylevel, bynode) of row and column
    sampling: tree (round r, output k) zeroes the (g, h) of its dropped rows before the
    quantiser and restricts each node's split candidates to its column sample.
    Returns (trees, margins, per-round gradients)."""
    n = bins.shape[0]
    margin = np.full((n, n_classes), base_margin, dtype=np.float32)
    trees, grads = [], []
    for r in range(rounds):
        if injected is not None:
            g, h = injected(r)
        else:
            g, h = gradients(objective, margin if n_classes > 1 else margin[:, 0], labels,
                             n_classes)
        grads.append((g.copy(), h.copy()))
        g = np.array(g, dtype=np.float32).reshape(n, -1)
        h = np.array(h, dtype=np.float32).reshape(n, -1)
        smps = [None] * n_classes
        if sample is not None:
            for k in range(n_classes):
                smps[k] = sampling(sample.get("seed", 0), r, k, sample.get("subsample", 1.0),
                                   sample.get("bytree", 1.0), sample.get("bylevel", 1.0),
                                   sample.get("bynode", 1.0))
                keep = sample_rows(smps[k], n)
                g[~keep, k] = 0.0
                h[~keep, k] = 0.0
        q = quantise(g, h)
        for k in range(n_classes):
            eg, eh, qg, qh = q[k]
            tree, ridx = grow_tree(bins, cut_ptr, cuts, missing_bin, qg, qh, eg, eh, p, bin_stride,
                                   smp=smps[k])
            col = np.ascontiguousarray(margin[:, k])
            for nid in range(len(tree["left"])):
                if tree["left"][nid] == -1:
                    rows = ridx[tree["seg_begin"][nid]:tree["seg_end"][nid]]
                    col[rows] += tree["leaf_value"][nid]
            margin[:, k] = col
            tree["positions"] = positions(tree, ridx, n)
            trees.append(tree)
    return trees, margin, grads
