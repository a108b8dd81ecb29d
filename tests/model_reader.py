"""Structural reader of XGBoost-3.4.1 model JSON, restating the checks that the
reference's model consumers apply (native/class_io.hpp:99-240,
native/class_native_source_contract.hpp:9-31).  It decides whether a model
file written by this library would be accepted downstream.  Objective and
class-count restrictions that are specific to the reference's converter
(multi:softprob, 2..7 classes; class_io.hpp:135-140) are optional here.
"""
import json
import math


class ModelError(ValueError):
    pass


def _need(ok, msg):
    if not ok:
        raise ModelError(msg)


def _decimal(v, field):
    _need(isinstance(v, str) and v.isdigit() and v != "", f"{field} must be a decimal string")
    return int(v)


def _int(v, field):
    _need(isinstance(v, int) and not isinstance(v, bool), f"invalid integer field: {field}")
    _need(-2**31 <= v < 2**31, f"integer field exceeds int32: {field}")
    return v


def _ints(v, field):
    _need(isinstance(v, list), f"{field} must be an integer array")
    return [_int(x, field) for x in v]


def read_model(doc, converter_rules=False):
    """Validates a parsed model document; returns (features, outputs, trees)."""
    learner = doc["learner"]
    booster = learner["gradient_booster"]
    params = learner["learner_model_param"]
    _need(booster["name"] == "gbtree", "gbtree required")
    if converter_rules:
        _need(learner["objective"]["name"] == "multi:softprob", "multi:softprob required")
    features = _decimal(params["num_feature"], "num_feature")
    outputs = _decimal(params["num_class"], "num_class")
    _need(features >= 1, "features must be positive")
    if converter_rules:
        _need(2 <= outputs <= 7, "2..7 classes")
    if "num_target" in params:
        _need(_decimal(params["num_target"], "num_target") == 1, "multi-target unsupported")
    _need(_ints(doc["version"], "version") == [3, 4, 1], "version must be 3.4.1")
    bias = params["base_score"]
    if isinstance(bias, str):
        bias = json.loads(bias)
    if not isinstance(bias, list):
        bias = [bias]
    _need(all(isinstance(b, (int, float)) and math.isfinite(b) for b in bias), "nonfinite bias")
    model = booster["model"]
    trees = model["trees"]
    channels = _ints(model["tree_info"], "tree_info")
    _need(isinstance(trees, list) and len(trees) == len(channels) and trees, "tree count")
    if "weight_drop" in model:
        w = model["weight_drop"]
        _need(isinstance(w, list), "weight_drop must be an array")
        if w:
            _need(len(w) == len(trees), "weight count")
            _need(all(isinstance(x, (int, float)) and not isinstance(x, bool) and x == 1.0
                      for x in w), "non-unit weights")
    _need(_decimal(model["gbtree_model_param"]["num_trees"], "num_trees") == len(trees),
          "num_trees differs")
    it = _ints(model["iteration_indptr"], "iteration_indptr")
    _need(len(it) >= 2 and it[0] == 0 and it[-1] == len(trees) and it == sorted(it),
          "iteration offsets")
    max_channel = max(outputs, 1)
    for t, tree in enumerate(trees):
        _need(_int(tree["id"], "tree id") == t, "tree id differs from order")
        _need(_decimal(tree["tree_param"]["size_leaf_vector"], "size_leaf_vector") in (0, 1),
              "vector leaves")
        _need(tree["categories"] == [], "categorical unsupported")
        stype = _ints(tree["split_type"], "split_type")
        _need(all(s == 0 for s in stype), "categorical split")
        left = _ints(tree["left_children"], "left_children")
        right = _ints(tree["right_children"], "right_children")
        feat = _ints(tree["split_indices"], "split_indices")
        cond = tree["split_conditions"]
        dl = tree["default_left"]
        n = len(left)
        _need(n and len(right) == n and len(feat) == n and len(cond) == n and len(dl) == n
              and len(stype) == n, "node arrays differ in size")
        _need(_decimal(tree["tree_param"]["num_nodes"], "num_nodes") == n, "num_nodes differs")
        _need(0 <= channels[t] < max_channel, "invalid class channel")
        for i in range(n):
            terminal = left[i] == -1 and right[i] == -1
            if not terminal:
                _need(0 <= left[i] < n and 0 <= right[i] < n, "fork needs two valid children")
                _need(left[i] > i and right[i] == left[i] + 1,
                      "successors must advance and be consecutive")
                _need(0 <= feat[i] < features and not (isinstance(cond[i], float) and math.isnan(cond[i])),
                      "invalid predicate")
            else:
                _need(isinstance(cond[i], (int, float)) and math.isfinite(cond[i]), "nonfinite leaf")
            d = dl[i]
            _need(isinstance(d, bool) or (isinstance(d, int) and d in (0, 1)),
                  "default_left must be Boolean or 0/1")
        seen = [0] * n
        stack = [0]
        reached = 0
        while stack:
            node = stack.pop()
            _need(0 <= node < n and not seen[node], "cyclic or shared children")
            seen[node] = 1
            reached += 1
            if left[node] >= 0:
                stack += [right[node], left[node]]
        _need(reached == n, "unreachable nodes")
    return features, outputs, trees


def predict_margin(doc, x):
    """Sum of leaves per output (x < split_condition -> left, NaN -> default)."""
    import numpy as np

    model = doc["learner"]["gradient_booster"]["model"]
    params = doc["learner"]["learner_model_param"]
    k = max(int(params["num_class"]), 1)
    out = np.zeros((x.shape[0], k), dtype=np.float32)
    for tree, ch in zip(model["trees"], model["tree_info"]):
        left = np.asarray(tree["left_children"])
        right = np.asarray(tree["right_children"])
        feat = np.asarray(tree["split_indices"])
        cond = np.asarray(tree["split_conditions"], dtype=np.float32)
        dl = np.asarray(tree["default_left"]).astype(bool)
        nid = np.zeros(x.shape[0], dtype=np.int64)
        active = left[nid] != -1
        while active.any():
            v = x[np.arange(x.shape[0]), feat[nid]]
            nxt = np.where(np.where(np.isnan(v), dl[nid], v < cond[nid]), left[nid], right[nid])
            nid = np.where(active, nxt, nid)
            active = left[nid] != -1
        out[:, ch] += cond[nid]
    return out
