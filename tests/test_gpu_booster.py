"""Whole-booster parity: libdpgbdt_hip.so trained through the XGBoost C-API
subset versus the CPU oracle's booster on identical seeded inputs.

Trees must be identical node for node (feature, bin, default direction,
threshold, leaf value, quantised sums), the row partition (final leaf of every
row) and the training margins bit-exact, and the saved model must predict the
training margins when walked with the routing rule x < threshold -> left,
NaN -> default (native/class_native_source_contract.hpp:24-31).
"""
import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TREE_KEYS_EXACT = ["left", "right", "parent", "feature", "split_bin", "default_left",
                   "sum_qg", "sum_qh"]
TREE_KEYS_BITS = ["split_condition", "base_weight", "sum_hess"]


def _train_both(dp, oracle, device, config, n, f, objective, k, p, rounds, seed, injected=False,
                max_bin=256, base_score=None, extra=None, mutate=None, sample=None,
                values_labels=None, record=1):
    """Trains the booster and the oracle's booster on the same inputs.  record: the
    booster's dp_record_positions.  With 1 the row positions are read back after every
    round; with 0 (the default training path, the one the bench and the trainer process
    run) the last split level's count launch stores the leaf values and no scatter or
    level-D planner runs, and no positions are returned (gpu_positions is None)."""
    import torch
    from dpgbdt import ops

    if values_labels is not None:
        values, labels = values_labels
        g = h = None
    else:
        values, labels, g, h = ops.synth(config, n, seed, n_features=f, want_grad=injected)
    if mutate is not None:
        values = mutate(values)
    obj_name = {0: "binary:logistic", 1: "multi:softmax", 2: "reg:squarederror"}[objective]
    dtrain = dp.DMatrix(values, labels)
    params = {"objective": obj_name, "tree_method": "hist", "device": "cuda:0", "max_bin": max_bin,
              "max_depth": p["max_depth"], "eta": p["eta"], "lambda": p.get("lam", 1.0),
              "alpha": p.get("alpha", 0.0), "gamma": p.get("gamma", 0.0),
              "min_child_weight": p.get("min_child_weight", 1.0),
              "dp_record_positions": int(record)}
    if objective == 1:
        params["num_class"] = k
    if base_score is not None:
        params["base_score"] = base_score
    if sample is not None:  # row / column sampling: booster keys and the oracle's draws
        params["seed"] = sample.get("seed", 0)
        for key, name in (("subsample", "subsample"), ("bytree", "colsample_bytree"),
                          ("bylevel", "colsample_bylevel"), ("bynode", "colsample_bynode")):
            if key in sample:
                params[name] = sample[key]
    params.update(extra or {})
    bst = dp.Booster(params, [dtrain])
    gpu_positions = [] if record else None
    for r in range(rounds):
        if injected:
            gr = torch.roll(g, shifts=r).contiguous()
            hr = torch.roll(h, shifts=r).contiguous()
            bst.boost(dtrain, r, gr, hr)
        else:
            bst.update(dtrain, r)
        if record:
            gpu_positions.append(bst.last_positions(n))
    x = values.cpu().numpy()
    has_missing = bool(np.isnan(x).any())
    eff = oracle.effective_max_bin(max_bin, has_missing)
    cut_ptr, cuts, _ = oracle.compute_cuts(x, eff)
    mb = oracle.missing_symbol(cut_ptr, has_missing)
    bins = oracle.bin_matrix(x, cut_ptr, cuts, mb)
    op = oracle.params(eta=p["eta"], lam=p.get("lam", 1.0), alpha=p.get("alpha", 0.0),
                       gamma=p.get("gamma", 0.0), min_child_weight=p.get("min_child_weight", 1.0),
                       max_depth=p["max_depth"])
    inj = None
    if injected:
        gn, hn = g.cpu().numpy(), h.cpu().numpy()
        inj = lambda r: (np.roll(gn, r)[:, None], np.roll(hn, r)[:, None])  # noqa: E731
    base_margin = 0.0
    if base_score is not None and objective != 0:
        base_margin = float(base_score)
    o_trees, o_margin, _ = oracle.train(bins, cut_ptr, cuts, mb, objective, labels.cpu().numpy(),
                                        k, op, rounds, base_margin=base_margin,
                                        bin_stride=int(np.diff(cut_ptr).max()), injected=inj,
                                        sample=sample)
    return bst, x, o_trees, o_margin, gpu_positions, n


def _compare(bst, o_trees, o_margin, gpu_positions, n, k):
    """Trees node for node, row counts, margins bit for bit, and the row positions of every
    round unless gpu_positions is None (a booster that did not record them)."""
    assert bst.num_trees() == len(o_trees)
    for t, ot in enumerate(o_trees):
        gt = bst.tree(t)
        for key in TREE_KEYS_EXACT:
            np.testing.assert_array_equal(gt[key], ot[key], err_msg=f"tree {t} {key}")
        for key in TREE_KEYS_BITS:
            np.testing.assert_array_equal(gt[key].view(np.uint32), ot[key].view(np.uint32),
                                          err_msg=f"tree {t} {key}")
        leaves = ot["left"] == -1
        np.testing.assert_array_equal(gt["loss_chg"][~leaves].view(np.uint32),
                                      ot["loss_chg"][~leaves].view(np.uint32))
        # row counts: leaves from the oracle's partition, internal nodes as their children's sum
        counts = np.bincount(ot["positions"], minlength=len(ot["left"]))
        np.testing.assert_array_equal(gt["rows"][leaves], counts[leaves], err_msg=f"tree {t} rows")
        inner = np.nonzero(~leaves)[0]
        np.testing.assert_array_equal(gt["rows"][inner],
                                      gt["rows"][ot["left"][inner]] + gt["rows"][ot["right"][inner]])
        assert gt["rows"][0] == n
    for r, pos in enumerate(gpu_positions or []):
        np.testing.assert_array_equal(pos, o_trees[(r + 1) * k - 1]["positions"],
                                      err_msg=f"round {r} positions")
    np.testing.assert_array_equal(bst.margins(n, k).view(np.uint32), o_margin.view(np.uint32))


def _predict_model(model, x, k, base):
    """Walk the saved model JSON: sum of leaves per output plus the base margin."""
    trees = model["learner"]["gradient_booster"]["model"]["trees"]
    info = model["learner"]["gradient_booster"]["model"]["tree_info"]
    out = np.tile(np.asarray(base, dtype=np.float32), (x.shape[0], 1))
    for t, tree in enumerate(trees):
        left = np.array(tree["left_children"])
        right = np.array(tree["right_children"])
        feat = np.array(tree["split_indices"])
        cond = np.array(tree["split_conditions"], dtype=np.float32)
        dl = np.array(tree["default_left"]).astype(bool)
        nid = np.zeros(x.shape[0], dtype=np.int64)
        active = left[nid] != -1
        while active.any():
            v = x[np.arange(x.shape[0]), feat[nid]]
            go_left = np.where(np.isnan(v), dl[nid], v < cond[nid])
            nxt = np.where(go_left, left[nid], right[nid])
            nid = np.where(active, nxt, nid)
            active = left[nid] != -1
        out[:, info[t]] += cond[nid]
    return out


def test_c1_binary_logistic(dp, oracle, device):
    """C1: 10,000 x 8 U(0,1), 256 bins, depth 6, 10 trees, eta 0.3, lambda 1."""
    p = {"max_depth": 6, "eta": 0.3}
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 1, 10000, 8, 0, 1, p, 10,
                                                    20261201)
    _compare(bst, o_trees, o_margin, pos, n, 1)
    model = json.loads(bst.save_raw())
    assert model["version"] == [3, 4, 1]
    m = _predict_model(model, x, 1, [0.0])
    np.testing.assert_array_equal(m.view(np.uint32), o_margin.view(np.uint32))
    cfg = json.loads(bst.save_config())
    assert cfg["learner"]["generic_param"]["device"] == "cuda:0"
    assert [u["name"] for u in cfg["learner"]["gradient_booster"]["updater"]] == ["grow_gpu_hist"]


def test_c2_reduced_logistic_depth8(dp, oracle, device):
    p = {"max_depth": 8, "eta": 0.1}
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 2, 40000, 28, 0, 1, p, 3,
                                                    20261202)
    _compare(bst, o_trees, o_margin, pos, n, 1)


def test_c4_reduced_softmax(dp, oracle, device):
    p = {"max_depth": 4, "eta": 0.3}
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 4, 2000, 784, 1, 10, p, 2,
                                                    20261204)
    _compare(bst, o_trees, o_margin, pos, n, 10)
    model = json.loads(bst.save_raw())
    assert model["learner"]["gradient_booster"]["model"]["tree_info"] == list(range(10)) * 2
    assert model["learner"]["gradient_booster"]["model"]["iteration_indptr"] == [0, 10, 20]


# dp_sparse_hist 1: histograms from the present-value layout (5 % present); 0: dense tiles
@pytest.mark.parametrize("sparse", [1, 0])
def test_c5_reduced_missing_squared(dp, oracle, device, sparse):
    p = {"max_depth": 7, "eta": 0.3}
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 5, 6000, 120, 2, 1, p, 3,
                                                    20261205, max_bin=65,
                                                    extra={"dp_sparse_hist": sparse})
    _compare(bst, o_trees, o_margin, pos, n, 1)
    assert any(t["default_left"].any() for t in o_trees), "learned default direction unused"
    m = _predict_model(json.loads(bst.save_raw()), x, 1, [0.0])
    np.testing.assert_array_equal(m.view(np.uint32), o_margin.view(np.uint32))


@pytest.mark.parametrize("max_bin,f", [(256, 50), (64, 300)])
def test_present_value_histograms_forced(dp, oracle, device, max_bin, f):
    """The present-value layout forced on a matrix with 40 % missing values: 32- and 128-feature
    sparse tiles with a partial last tile, multi-chunk nodes (partial slots) and single-chunk
    nodes (direct stores), against the oracle."""
    import torch

    def holes(v):
        g = torch.Generator(device="cpu").manual_seed(11)
        m = torch.rand(v.shape, generator=g) < 0.4
        v = v.clone()
        v[m.to(v.device)] = float("nan")
        return v

    p = {"max_depth": 6, "eta": 0.3}
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 1, 40000, f, 0, 1, p, 2,
                                                    20261207, max_bin=max_bin,
                                                    extra={"dp_sparse_hist": 2}, mutate=holes)
    _compare(bst, o_trees, o_margin, pos, n, 1)


@pytest.mark.parametrize("max_bin", [256, 64])
def test_wide_dense_levels_with_missing_values(dp, oracle, device, max_bin):
    """The dense layout of a wide matrix (300 features: feature-major partial slots and the
    reduce and evaluation in one launch on every level below the root) with 40 % missing
    values, single- and multi-chunk nodes, 255 and 64 bins, against the oracle."""
    import torch

    def holes(v):
        g = torch.Generator(device="cpu").manual_seed(13)
        m = torch.rand(v.shape, generator=g) < 0.4
        v = v.clone()
        v[m.to(v.device)] = float("nan")
        return v

    p = {"max_depth": 6, "eta": 0.3}
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 1, 40000, 300, 0, 1, p, 2,
                                                    20261208, max_bin=max_bin,
                                                    extra={"dp_sparse_hist": 0}, mutate=holes)
    _compare(bst, o_trees, o_margin, pos, n, 1)


def test_c3_reduced_injected_gradients(dp, oracle, device):
    p = {"max_depth": 8, "eta": 0.3}
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 3, 30000, 128, 2, 1, p, 2,
                                                    20261203, injected=True)
    _compare(bst, o_trees, o_margin, pos, n, 1)


def test_wide_tree_level_synced(dp, oracle, device):
    """Depth 17 over 150,000 rows: a level may hold more than 65,536 nodes, so the
    grower reads each level's size back and sizes its buffers per level instead
    of enqueueing the whole tree (the path large trees take)."""
    p = {"max_depth": 17, "eta": 0.3}
    print("[booster] C1 150000 x 8, depth 17 (level-synced growth)", flush=True)
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 1, 150000, 8, 0, 1, p, 2,
                                                    20261211)
    _compare(bst, o_trees, o_margin, pos, n, 1)
    assert max(len(t["left"]) for t in o_trees) > 2 ** 12, "tree too small to exercise the path"


def test_deep_eager_tree(dp, oracle, device):
    """Depth 12 over 60,000 rows, enqueued whole: levels whose node bound is at most 1024 run
    the planner beside the scatter in one launch (level 10 at the 1024 bound), the deeper ones
    run them as two launches."""
    p = {"max_depth": 12, "eta": 0.3}
    print("[booster] C1 60000 x 8, depth 12 (merged and separate planner launches)", flush=True)
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 1, 60000, 8, 0, 1, p, 2,
                                                    20261213)
    _compare(bst, o_trees, o_margin, pos, n, 1)
    assert max(len(t["left"]) for t in o_trees) > 2 ** 11, "tree too small to exercise the path"


def test_large_matrix_grouped_partition(dp, oracle, device):
    """4,300,000 rows: matrices of 4M rows or more take the partition kernels that
    load four 256-row steps per group (from the column copy of the bins)."""
    p = {"max_depth": 6, "eta": 0.3}
    print("[booster] C1 4300000 x 8, depth 6 (grouped partition loads)", flush=True)
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 1, 4_300_000, 8, 0, 1, p, 2,
                                                    20261212)
    _compare(bst, o_trees, o_margin, pos, n, 1)


@pytest.mark.parametrize("record", [0, 1])
def test_c2_full_size(dp, oracle, device, record):
    """C2 at its benchmark size and parameters (1,000,000 x 28, depth 8, eta 0.1,
    logistic): two rounds, every tree, the margins (and, recording them, the row
    partition) bit-exact against the oracle.  record 0 is the path the bench times."""
    p = {"max_depth": 8, "eta": 0.1}
    print(f"[booster] C2 1000000 x 28, depth 8 (benchmark size), record {record}", flush=True)
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 2, 1_000_000, 28, 0, 1, p, 2,
                                                    20261201 + 2, record=record)
    _compare(bst, o_trees, o_margin, pos, n, 1)


@pytest.mark.parametrize("record", [0, 1])
def test_c4_full_size(dp, oracle, device, record):
    """C4 at its benchmark size (60,000 x 784, 10 classes, depth 6, eta 0.3): two
    rounds of ten trees, grown concurrently on four streams, against the oracle (the
    second round's gradients add the first round's leaf values when record is 0)."""
    p = {"max_depth": 6, "eta": 0.3}
    print(f"[booster] C4 60000 x 784, 10 classes, depth 6 (benchmark size), record {record}",
          flush=True)
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 4, 60_000, 784, 1, 10, p, 2,
                                                    20261201 + 4, record=record)
    _compare(bst, o_trees, o_margin, pos, n, 10)


def test_depth_one_and_single_chunk(dp, oracle, device):
    """Smallest shapes: stumps (max_depth 1) and a matrix of one histogram chunk."""
    for n, depth in [(50, 1), (4000, 3), (5000, 1)]:
        p = {"max_depth": depth, "eta": 0.5}
        print(f"[booster] C1 {n} x 8, depth {depth}", flush=True)
        bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 1, n, 8, 0, 1, p, 3,
                                                        20261212 + n)
        _compare(bst, o_trees, o_margin, pos, n, 1)


@pytest.mark.parametrize("sparse", [0, 2])
def test_degenerate_features_and_tiny_matrices(dp, oracle, device, sparse):
    """A feature that is all missing, a constant feature and a feature missing in every other
    row, on 1, 2, 63 and 5000 rows, dense and present-value histograms, against the oracle."""
    def degenerate(v):
        v = v.clone()
        v[:, 0] = float("nan")
        v[:, 1] = 0.25
        v[::2, 2] = float("nan")
        return v

    for n in [1, 2, 63, 5000]:
        p = {"max_depth": 4, "eta": 0.5}
        print(f"[booster] degenerate {n} x 12, sparse {sparse}", flush=True)
        bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 1, n, 12, 0, 1, p, 2,
                                                        20261220 + n,
                                                        extra={"dp_sparse_hist": sparse},
                                                        mutate=degenerate)
        _compare(bst, o_trees, o_margin, pos, n, 1)


def test_regularisation_paths(dp, oracle, device):
    """alpha, gamma and min_child_weight change the chosen splits identically."""
    p = {"max_depth": 5, "eta": 0.5, "alpha": 0.7, "gamma": 2.0, "min_child_weight": 8.0,
         "lam": 0.0}
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 1, 8000, 8, 0, 1, p, 3,
                                                    31)
    _compare(bst, o_trees, o_margin, pos, n, 1)


def _small_booster(dp, config, n, f, objective, k, rounds, depth=5, seed=7, max_bin=256):
    from dpgbdt import ops

    values, labels, _, _ = ops.synth(config, n, seed, n_features=f)
    obj = {0: "binary:logistic", 1: "multi:softmax", 2: "reg:squarederror"}[objective]
    params = {"objective": obj, "max_depth": depth, "eta": 0.3, "max_bin": max_bin}
    if objective == 1:
        params["num_class"] = k
    dtrain = dp.DMatrix(values, labels)
    bst = dp.Booster(params, [dtrain])
    for r in range(rounds):
        bst.update(dtrain, r)
    return bst, values, labels


@pytest.mark.parametrize("config,n,f,objective,k,depth,mcw", [(2, 30000, 28, 0, 1, 6, 1.0),
                                                               (4, 1500, 784, 1, 10, 4, 1.0),
                                                               (5, 4000, 60, 2, 1, 7, 1.0),
                                                               (1, 3000, 8, 0, 1, 1, 1.0),
                                                               (1, 3000, 8, 0, 1, 8, 4.0),
                                                               (1, 3000, 8, 0, 1, 8, 40.0)])
def test_margins_without_leaf_ids(dp, device, config, n, f, objective, k, depth, mcw):
    """Without leaf ids recorded, the last split level's count launch adds the leaf values of
    its children and of that level's own leaves to the margins (no scatter and no separate
    margin pass there); margins and models must equal a booster's that records leaf ids, whose
    margins the oracle tests pin."""
    from dpgbdt import ops

    values, labels, _, _ = ops.synth(config, n, 11, n_features=f)
    obj = {0: "binary:logistic", 1: "multi:softmax", 2: "reg:squarederror"}[objective]
    out = []
    for record in (0, 1):
        params = {"objective": obj, "max_depth": depth, "eta": 0.3, "max_bin": 256,
                  "min_child_weight": mcw, "dp_record_positions": record}
        if objective == 1:
            params["num_class"] = k
        dtrain = dp.DMatrix(values, labels)
        bst = dp.Booster(params, [dtrain])
        for r in range(3):
            bst.update(dtrain, r)
        model = json.loads(bst.save_raw())["learner"]["gradient_booster"]["model"]
        out.append((bst.margins(n, k), model))
    np.testing.assert_array_equal(out[0][0].view(np.uint32), out[1][0].view(np.uint32))
    assert out[0][1] == out[1][1]
    # leaves by depth: with a larger min_child_weight, nodes stop at the last split level
    # (their own leaf values come from the count launch) or trees end before it
    depths = []
    for t in out[0][1]["trees"]:
        left = np.array(t["left_children"])
        d = np.zeros(len(left), dtype=np.int64)
        for i in range(len(left)):
            if left[i] != -1:
                d[left[i]] = d[i] + 1
                d[left[i] + 1] = d[i] + 1
        depths.extend(d[left == -1].tolist())
    print(f"[margins] depth {depth} mcw {mcw}: leaves by depth "
          f"{np.bincount(depths).tolist()}", flush=True)


@pytest.mark.parametrize("config,n,f,objective,k", [(1, 5000, 8, 0, 1), (4, 1500, 784, 1, 10),
                                                     (5, 4000, 60, 2, 1)])
def test_prediction_equals_training_margins(dp, device, config, n, f, objective, k):
    import model_reader

    bst, values, labels = _small_booster(dp, config, n, f, objective, k, 4)
    margins = bst.margins(n, k)
    pm = bst.predict(values, margin=True).cpu().numpy()
    np.testing.assert_array_equal(pm.view(np.uint32), margins.view(np.uint32))
    doc = json.loads(bst.save_raw())
    model_reader.read_model(doc)
    walked = model_reader.predict_margin(doc, values.cpu().numpy())
    base = 0.0
    np.testing.assert_array_equal((walked + base).view(np.uint32), margins.view(np.uint32))
    # iteration ranges and slices agree
    p2 = bst.predict(values, margin=True, iteration_end=2).cpu().numpy()
    s2 = bst.slice(0, 2).predict(values, margin=True).cpu().numpy()
    np.testing.assert_array_equal(p2, s2)
    assert not np.array_equal(p2, pm)
    # a reloaded model predicts the same bits
    again = dp.Booster.from_buffer(bst.save_raw())
    np.testing.assert_array_equal(again.predict(values, margin=True).cpu().numpy(), pm)
    assert again.num_boosted_rounds() == 4


def test_prediction_transforms(dp, device):
    bst, values, labels = _small_booster(dp, 1, 5000, 8, 0, 1, 3)
    m = bst.predict(values, margin=True).cpu().numpy()[:, 0].astype(np.float64)
    p = bst.predict(values).cpu().numpy()[:, 0]
    np.testing.assert_allclose(p, 1 / (1 + np.exp(-m)), rtol=3e-6, atol=1e-7)
    bst, values, labels = _small_booster(dp, 4, 1500, 784, 1, 10, 3)
    m = bst.predict(values, margin=True).cpu().numpy()
    cls = bst.predict(values).cpu().numpy()
    assert cls.shape == (1500, 1)
    np.testing.assert_array_equal(cls[:, 0], np.argmax(m, axis=1).astype(np.float32))
    # the reference's probability view: slice a full clone, switch to softprob
    view = bst.slice(0, 0)
    view.set_param("objective", "multi:softprob")
    prob = view.predict(values).cpu().numpy()
    assert prob.shape == (1500, 10)
    np.testing.assert_allclose(prob.sum(axis=1), 1.0, atol=2e-6)
    e = np.exp(m - m.max(axis=1, keepdims=True))
    np.testing.assert_allclose(prob, e / e.sum(axis=1, keepdims=True), atol=2e-6)
    model = json.loads(view.save_raw())
    assert model["learner"]["objective"]["name"] == "multi:softprob"


def test_invalid_labels_are_refused(dp, device):
    import torch
    from dpgbdt import ops

    values, _, _, _ = ops.synth(1, 1000, 3)
    bad = torch.full((1000,), 3.0, device=device)
    dtrain = dp.DMatrix(values, bad)
    bst = dp.Booster({"objective": "multi:softmax", "num_class": 3}, [dtrain])
    with pytest.raises(dp.DPError, match="class ids"):
        bst.update(dtrain, 0)
    half = torch.full((1000,), 0.5, device=device)
    dtrain = dp.DMatrix(values, half)
    bst = dp.Booster({"objective": "multi:softmax", "num_class": 3}, [dtrain])
    with pytest.raises(dp.DPError, match="class ids"):
        bst.update(dtrain, 0)
    two = torch.full((1000,), 2.0, device=device)
    dtrain = dp.DMatrix(values, two)
    bst = dp.Booster({"objective": "binary:logistic"}, [dtrain])
    with pytest.raises(dp.DPError, match=r"\[0, 1\]"):
        bst.update(dtrain, 0)
    inf = values.clone()
    inf[3, 2] = float("inf")
    with pytest.raises(dp.DPError, match="inf"):
        dp.DMatrix(inf, half)


@pytest.mark.parametrize("objective,k", [(0, 1), (1, 3)])
def test_graph_replays_equal_direct_launches(dp, device, objective, k):
    """Rounds replayed from cached HIP graphs give the same model, margins and row positions
    as rounds launched directly; a parameter change between rounds captures a new graph, and
    caller gradients (a graph without the objective kernel) replay the same way.  Rounds left
    in flight back to back (trees collected one call later, each round's leaf values added by
    the next round's gradient kernel instead of a margin read) give the same model and the
    same final margins too."""
    import torch
    from dpgbdt import ops

    n, f = 20_000, 12
    values, labels, g, h = ops.synth(1, n, 7, n_features=f, want_grad=True)
    if objective == 1:
        labels = (torch.arange(n, device=values.device) % k).to(torch.float32)
    values[::97, 3] = float("nan")
    obj_name = {0: "binary:logistic", 1: "multi:softmax"}[objective]

    def train(graphs, inspect=True):
        dtrain = dp.DMatrix(values, labels)
        params = {"objective": obj_name, "max_depth": 5, "eta": 0.3, "dp_record_positions": 1,
                  "dp_graphs": graphs}
        if objective == 1:
            params["num_class"] = k
        bst = dp.Booster(params, [dtrain])
        positions, margins = [], []
        for r in range(6):
            if r == 3:
                bst.set_param("eta", 0.1)
            bst.update(dtrain, r)
            if inspect:  # collects the round; otherwise rounds stay in flight back to back
                positions.append(bst.last_positions(n))
                margins.append(bst.margins(n, k))
        gk = g.repeat_interleave(k).reshape(n, k).contiguous() if k > 1 else g
        hk = h.repeat_interleave(k).reshape(n, k).contiguous() if k > 1 else h
        for r in range(6, 9):
            bst.boost(dtrain, r, gk, hk)
            if inspect:
                positions.append(bst.last_positions(n))
                margins.append(bst.margins(n, k))
        assert bst.num_boosted_rounds() == 9
        # the last rounds' leaf values are in the margins however the rounds were read
        return bst.save_raw(), positions, margins, bst.margins(n, k)

    raw_direct, pos_direct, m_direct, end_direct = train(0)
    raw_graph, pos_graph, m_graph, end_graph = train(1)
    assert raw_graph == raw_direct
    for graphs in (1, 0):
        raw, _, _, end = train(graphs, inspect=False)
        assert raw == raw_direct
        np.testing.assert_array_equal(np.asarray(end).view(np.uint32),
                                      np.asarray(end_direct).view(np.uint32))
    np.testing.assert_array_equal(np.asarray(end_graph).view(np.uint32),
                                  np.asarray(end_direct).view(np.uint32))
    for r, (a, b) in enumerate(zip(pos_graph, pos_direct)):
        np.testing.assert_array_equal(a, b, err_msg=f"round {r} positions")
    for r, (a, b) in enumerate(zip(m_graph, m_direct)):
        np.testing.assert_array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32),
                                      err_msg=f"round {r} margins")


def test_matrix_freed_with_round_in_flight(dp, device):
    """Freeing the training matrix right after a round (whose trees are still being collected
    asynchronously) collects that round first: the model equals one whose rounds were collected
    call by call."""
    import gc

    from dpgbdt import ops

    values, labels, _, _ = ops.synth(2, 50_000, 3, n_features=28)
    params = {"objective": "binary:logistic", "max_depth": 6, "eta": 0.3}

    def train(inspect):
        dtrain = dp.DMatrix(values, labels)
        bst = dp.Booster(params, [dtrain])
        for r in range(4):
            bst.update(dtrain, r)
            if inspect:
                assert bst.num_boosted_rounds() == r + 1
        # the booster's Python cache keeps the wrapper alive: free the matrix through the C API
        assert dp.load().XGDMatrixFree(dtrain.handle) == 0
        dtrain.handle = None
        gc.collect()
        return bst.save_raw()

    assert train(False) == train(True)


def test_concurrent_class_trees_equal_sequential(dp, device):
    """The class trees of a round grown on 1, 2, 3 or 4 streams give the same model."""
    import torch
    from dpgbdt import ops

    n, k = 30_000, 5
    values, _, _, _ = ops.synth(1, n, 9, n_features=64)
    labels = (torch.arange(n, device=values.device) % k).to(torch.float32)
    dtrain = dp.DMatrix(values, labels)
    models = []
    for lanes in (1, 2, 3, 4):
        bst = dp.Booster({"objective": "multi:softprob", "num_class": k, "max_depth": 5,
                          "eta": 0.3, "dp_concurrent_trees": lanes}, [dtrain])
        for r in range(3):
            bst.update(dtrain, r)
        models.append(bst.save_raw())
    assert all(m == models[0] for m in models[1:])


def test_reused_buffers_give_the_same_model(dp, device):
    """Training buffers come back from the allocation cache with the contents a
    previous booster left in them: a booster trained after boosters of other
    shapes (whose blocks it may reuse) and after one of its own shape must save
    the same model as the first one trained in a fresh state."""
    from dpgbdt import ops

    def train(config, n, f, params, rounds):
        values, labels, _, _ = ops.synth(config, n, 31, n_features=f)
        dtrain = dp.DMatrix(values, labels)
        bst = dp.Booster(dict(params, dp_record_positions=1), [dtrain])
        for r in range(rounds):
            bst.update(dtrain, r)
        return bst.save_raw(), bst.last_positions(n)

    logistic = {"objective": "binary:logistic", "max_depth": 6, "eta": 0.3}
    first, first_pos = train(1, 20_000, 8, logistic, 3)
    train(5, 30_000, 120, {"objective": "reg:squarederror", "max_depth": 7, "eta": 0.3,
                           "max_bin": 64}, 2)
    train(1, 20_000, 8, dict(logistic, max_depth=8), 2)
    again, again_pos = train(1, 20_000, 8, logistic, 3)
    assert again == first
    assert (again_pos == first_pos).all()


def test_c5_full_size_layouts_agree(dp, device):
    """C5 at its benchmark size and parameters (2,000,000 x 1,000, 95 % missing,
    64 bins, depth 10, squared error), where the CPU oracle would take minutes:
    two independent histogram paths -- the present-value layout and the dense
    16-feature tiles -- must give the same model, the same final row partition
    and the same margins, round after round."""
    import torch
    from dpgbdt import ops

    n, f = 2_000_000, 1000
    print(f"[booster] C5 {n} x {f}, depth 10: present-value vs dense histograms", flush=True)
    values, labels, _, _ = ops.synth(5, n, 20261201 + 5, n_features=f)
    dtrain = dp.DMatrix(values, labels)
    del values
    out = []
    for sparse in (1, 0):
        bst = dp.Booster({"objective": "reg:squarederror", "max_depth": 10, "eta": 0.3,
                          "max_bin": 64, "dp_sparse_hist": sparse, "dp_record_positions": 1},
                         [dtrain])
        positions = []
        for r in range(2):
            bst.update(dtrain, r)
            positions.append(bst.last_positions(n))
        out.append((bst.save_raw(), positions, bst.margins(n, 1)))
        del bst
        torch.cuda.empty_cache()
    (m1, p1, g1), (m0, p0, g0) = out
    assert m1 == m0
    for a, b in zip(p1, p0):
        np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(np.asarray(g1).view(np.uint32), np.asarray(g0).view(np.uint32))
    assert len(json.loads(m1)["learner"]["gradient_booster"]["model"]["trees"]) == 2


@pytest.mark.parametrize("case", ["level_synced", "large"])
def test_last_level_margins_synced_and_large(dp, oracle, device, case):
    """The last split level's margin scatter (taken when leaf ids are not recorded) on the
    paths the other margin test leaves out: a level-synced tree (depth 17, so the host reads
    each level's size back) whose levels hold at most 1024 nodes and that reaches its last
    split level, and a 4,300,000-row matrix (the partition's grouped-load instantiation).
    Margins and models equal a booster's that records leaf ids; for the level-synced case
    both also equal the oracle's margins."""
    import torch
    from dpgbdt import ops

    if case == "level_synced":
        n, depth, mcw = 1000, 17, 0.0
        rng = np.random.default_rng(5)
        x = rng.random((n, 8), dtype=np.float32)
        y = (rng.random(n) < 0.5).astype(np.float32)
        values = torch.as_tensor(x, device=device)
        labels = torch.as_tensor(y, device=device)
    else:
        n, depth, mcw = 4_300_000, 6, 1.0
        values, labels, _, _ = ops.synth(1, n, 13, n_features=8)
    print(f"[booster] last-level margins, {case}: {n} rows, depth {depth}", flush=True)
    out = []
    for record in (0, 1):
        dtrain = dp.DMatrix(values, labels)
        bst = dp.Booster({"objective": "binary:logistic", "max_depth": depth, "eta": 0.3,
                          "min_child_weight": mcw, "dp_record_positions": record}, [dtrain])
        for r in range(2):
            bst.update(dtrain, r)
        model = json.loads(bst.save_raw())["learner"]["gradient_booster"]["model"]
        out.append((bst.margins(n, 1), model, bst))
    np.testing.assert_array_equal(out[0][0].view(np.uint32), out[1][0].view(np.uint32))
    assert out[0][1] == out[1][1]
    if case == "level_synced":
        trees = out[0][1]["trees"]
        for t in trees:  # the tree reaches its last split level, every level narrow
            left = np.array(t["left_children"])
            d = np.zeros(len(left), dtype=np.int64)
            for i in range(len(left)):
                if left[i] != -1:
                    d[left[i]] = d[i] + 1
                    d[left[i] + 1] = d[i] + 1
            assert d.max() == depth and np.bincount(d).max() <= 1024
        cut_ptr, cuts, _ = oracle.compute_cuts(x, 256)
        bins = oracle.bin_matrix(x, cut_ptr, cuts, -1)
        p = oracle.params(eta=0.3, min_child_weight=mcw, max_depth=depth)
        _, o_margin, _ = oracle.train(bins, cut_ptr, cuts, -1, 0, y, 1, p, 2,
                                      bin_stride=int(np.diff(cut_ptr).max()))
        np.testing.assert_array_equal(out[0][0].view(np.uint32), o_margin.view(np.uint32))


@pytest.mark.parametrize("record", [0, 1])
def test_c5_own_parameters(dp, oracle, device, record):
    """C5's own parameters against the oracle (200,000 x 1,000, 95 % missing, max_bin 64,
    depth 10, squared error, two rounds): the evaluation kernel for at most 64 bins, the
    present-value histograms and the depth-10 planner together, node for node; record 0 is
    the path the bench times."""
    p = {"max_depth": 10, "eta": 0.3}
    print(f"[booster] C5 200000 x 1000, 64 bins, depth 10 vs the oracle, record {record}",
          flush=True)
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 5, 200_000, 1000, 2, 1, p,
                                                    2, 20261201 + 5, max_bin=64, record=record)
    _compare(bst, o_trees, o_margin, pos, n, 1)
    assert max(len(t["left"]) for t in o_trees) > 500, "trees too small for depth 10"
    assert any(t["default_left"].any() for t in o_trees), "learned default direction unused"


def test_c3_tree_one_million_rows(dp, oracle, device):
    """C3's tree on 1,000,000 of its rows (128 features, 256 bins, depth 8, injected
    gradients), one round against the oracle: the gathered row-major histograms at
    multi-chunk node sizes, subtraction, evaluation and partition at depth 8."""
    p = {"max_depth": 8, "eta": 0.3}
    print("[booster] C3 1000000 x 128, depth 8 vs the oracle", flush=True)
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 3, 1_000_000, 128, 2, 1, p,
                                                    1, 20261203, injected=True)
    _compare(bst, o_trees, o_margin, pos, n, 1)


def test_c3_full_size_tree(dp, oracle, device):
    """C3 at its full size -- 10,000,000 rows x 128 features, 256 bins, depth 8, injected
    gradients -- one round against the oracle's booster on all host cores: every split record,
    row count, leaf value and the margins of a booster without row positions recorded (the
    bench's path) and of one with them, whose 10M row positions are compared too.  The oracle takes the GPU's
    cuts and uint8 bins (bit-identical to its own on every configuration's shape,
    test_gpu_kernels.py::test_cuts_and_bins_bit_exact), as the bench's CPU leg does, so the
    check covers the boosting round: the root pass over all rows, the gathered passes with
    their fitted chunks, the fused reduce-evaluate over many-chunk nodes and the partition of
    10M rows at every level."""
    import os

    import torch
    from dpgbdt import ops

    n, f = 10_000_000, 128
    print("[booster] C3 10000000 x 128, depth 8 vs the oracle (host threads)", flush=True)
    values, labels, g, h = ops.synth(3, n, 20261204, want_grad=True)
    dtrain = dp.DMatrix(values, labels)
    boosters = []
    for record in (0, 1):  # 0: the path the bench times; 1: also the row positions
        bst = dp.Booster({"objective": "reg:squarederror", "max_depth": 8, "eta": 0.3,
                          "max_bin": 256, "dp_record_positions": record}, [dtrain])
        bst.boost(dtrain, 0, g.reshape(-1, 1).contiguous(), h.reshape(-1, 1).contiguous())
        boosters.append((bst, [bst.last_positions(n)] if record else None))
    assert not bool(torch.isnan(values).any().item())  # C3 has no missing values
    ws = ops.Workspace()
    cut_ptr, cuts, _, _ = ops.sketch_cuts(ws, values, 256)
    lay = ops.layout(n, f, 0, -1)
    bins = ops.from_tiles(ops.bin_values(values, lay, cut_ptr, cuts).cpu().numpy(), lay)
    gn, hn = g.cpu().numpy()[:, None], h.cpu().numpy()[:, None]
    y = labels.cpu().numpy()
    del values, labels, g, h
    torch.cuda.empty_cache()
    oracle.set_threads(len(os.sched_getaffinity(0)))
    try:
        o_trees, o_margin, _ = oracle.train(bins, cut_ptr, cuts, -1, 2, y, 1,
                                            oracle.params(eta=0.3, max_depth=8), 1,
                                            bin_stride=int(np.diff(cut_ptr).max()),
                                            injected=lambda r: (gn, hn))
    finally:
        oracle.set_threads(1)
    for bst, gpu_positions in boosters:
        _compare(bst, o_trees, o_margin, gpu_positions, n, 1)


def _random_case(rng, large=False):
    """One random training problem: matrix shape, value kinds per column (continuous, few
    distinct integers, constant, mostly zero), missing share, bins, objective, tree and
    regularisation parameters, rounds, sampling, histogram layout and launch shape.  large:
    200,000 to 1,000,000 rows of at most 40 features, depth up to 17 (level-synced growth
    past the device planner's levels), up to 10 classes."""
    if large:
        n = int(rng.choice([200000, 500000, 1000000]))
        f = int(rng.choice([1, 5, 17, 28, 40]))
    else:
        n = int(rng.choice([1, 2, 3, 17, 100, 640, 2000, 5000, 9000, 40000, 120000]))
        f = int(rng.choice([1, 2, 5, 15, 16, 17, 33, 70, 130, 300]))
    if n * f > 1_500_000:
        f = max(1, 1_500_000 // n)
    x = np.empty((n, f), dtype=np.float32)
    for j in range(f):
        kind = rng.choice(["normal", "ints", "const", "zeros"], p=[0.5, 0.3, 0.05, 0.15])
        if kind == "normal":
            x[:, j] = rng.normal(size=n) * rng.choice([1e-3, 1.0, 1e3])
        elif kind == "ints":
            x[:, j] = rng.integers(0, int(rng.integers(2, 40)), size=n)
        elif kind == "const":
            x[:, j] = 0.5
        else:
            x[:, j] = np.where(rng.random(n) < 0.8, 0.0, rng.random(n))
    missing = float(rng.choice([0.0, 0.0, 0.1, 0.5, 0.95]))
    if missing > 0:
        x[rng.random((n, f)) < missing] = np.nan
    objective = int(rng.integers(0, 3))
    k = int(rng.integers(2, 11 if large else 5)) if objective == 1 else 1
    z = np.nan_to_num(x, nan=0.0) @ rng.normal(size=(f, k)).astype(np.float32)
    z = z / (np.abs(z).max() + 1e-6) * 3 + rng.normal(size=(n, k)).astype(np.float32)
    if objective == 0:
        y = (z[:, 0] > 0).astype(np.float32)
    elif objective == 1:
        y = z.argmax(axis=1).astype(np.float32)
    else:
        y = z[:, 0].astype(np.float32)
    p = {"max_depth": int(rng.integers(1, 18 if large else 11)),
         "eta": float(rng.choice([0.1, 0.3, 1.0])),
         "lam": float(rng.choice([0.0, 1.0, 5.0])), "alpha": float(rng.choice([0.0, 0.5])),
         "gamma": float(rng.choice([0.0, 0.2])),
         "min_child_weight": float(rng.choice([0.0, 1.0, 4.0]))}
    extra = {"dp_graphs": int(rng.integers(0, 2)),
             "dp_sparse_hist": int(rng.choice([0, 1, 2])) if missing > 0 else 0,
             "dp_hist_tiles": int(rng.choice([0, 1, 2])),
             "dp_hist_unroll": int(rng.choice([0, 1, 2])),
             "dp_hist_split": int(rng.choice([0, 4, 5]))}
    if missing == 0:
        extra["dp_skip_bin"] = int(rng.choice([0, 1, 2]))
    if objective == 1:
        extra["dp_concurrent_trees"] = int(rng.choice([1, 3]))
    sample = None
    if rng.random() < 0.3:
        sample = {"seed": int(rng.integers(0, 1000))}
        for key in ("subsample", "bytree", "bylevel", "bynode"):
            if rng.random() < 0.5:
                sample[key] = float(rng.choice([0.5, 0.8]))
    case = {"n": n, "f": f, "missing": missing, "objective": objective, "k": k,
            "max_bin": int(rng.choice([2, 3, 7, 16, 63, 64, 65, 128, 255, 256])),
            "rounds": int(rng.integers(1, 4)), "p": p, "extra": extra, "sample": sample}
    return x, y, case


def _random_problems(dp, oracle, device, seed, count, large=False):
    """Trains `count` random problems against the oracle; returns how many grew a split."""
    import torch

    rng = np.random.default_rng(seed)
    # dp_record_positions per problem from a generator of its own, so the problems
    # themselves stay the ones the seed has always drawn
    record_rng = np.random.default_rng(seed + 1)
    grown = 0
    for t in range(count):
        x, y, case = _random_case(rng, large)
        record = int(record_rng.integers(0, 2))
        print(f"[booster] random problem {t} (record {record}): {case}", flush=True)
        values = torch.from_numpy(x).to(device)
        labels = torch.from_numpy(y).to(device)
        bst, _, o_trees, o_margin, pos, n = _train_both(
            dp, oracle, device, 1, case["n"], case["f"], case["objective"], case["k"], case["p"],
            case["rounds"], 0, max_bin=case["max_bin"], extra=case["extra"],
            sample=case["sample"], values_labels=(values, labels), record=record)
        _compare(bst, o_trees, o_margin, pos, n, case["k"])
        # the predictor, walking the saved trees on the raw values, gives the same margins
        pm = bst.predict(values, margin=True).cpu().numpy()
        np.testing.assert_array_equal(pm.reshape(o_margin.shape).view(np.uint32),
                                      o_margin.view(np.uint32))
        grown += any(bool((ot["left"] != -1).any()) for ot in o_trees)
    return grown


def test_random_problems_match_the_oracle(dp, oracle, device):
    """A hundred seeded random problems -- 1 to 120,000 rows, 1 to 300 features of mixed kinds
    (tied integers, constants, mostly-zero columns), 0-95 % missing, 2-256 bins, every
    objective, depth 1-10, random regularisation, sampling, histogram layout, skip bins,
    launch shape and graph use -- each trained for 1-3 rounds against the oracle's booster:
    split records, row counts, leaf values, margins and (for the problems drawn to record
    them) row positions, bit for bit, and the predictor's margins over the raw values equal
    to them.  About half the problems run without row positions recorded, the default
    training path."""
    grown = _random_problems(dp, oracle, device, 20261202, 100)
    assert grown >= 60, f"only {grown} of 100 problems grew a split"


def test_random_large_problems_match_the_oracle(dp, oracle, device):
    """Twenty seeded random problems of 200,000 to 1,000,000 rows, depth up to 17 and up to
    10 classes (the rest as in the small ones), against the oracle's booster on all host
    threads."""
    import os

    oracle.set_threads(len(os.sched_getaffinity(0)))
    try:
        grown = _random_problems(dp, oracle, device, 4242, 20, large=True)
    finally:
        oracle.set_threads(1)
    assert grown >= 15, f"only {grown} of 20 problems grew a split"


def test_strided_label_interface_is_refused(dp, device):
    """A label array interface with strides is copied as one contiguous block, so strides must
    be the C-contiguous ones: a column slice of an [n, 2] array ([n, 1] with a row stride of 8
    bytes) is refused, a contiguous [n, 1] with explicit strides is accepted."""
    import ctypes

    import torch
    from dpgbdt import ops

    n = 1000
    values, _, _, _ = ops.synth(1, n, 3)
    both = torch.zeros((n, 2), dtype=torch.float32, device=device)
    dtrain = dp.DMatrix(values)
    lib = dp.load()

    def set_labels(ptr, strides):
        doc = json.dumps({"data": [ptr, True], "shape": [n, 1], "strides": strides,
                          "typestr": "<f4", "version": 3})
        return lib.XGDMatrixSetInfoFromInterface(dtrain.handle, b"label", doc.encode())

    assert set_labels(both.data_ptr(), [8, 4]) == -1
    assert "C-contiguous" in lib.XGBGetLastError().decode()
    col = torch.zeros((n, 1), dtype=torch.float32, device=device)
    assert set_labels(col.data_ptr(), [4, 4]) == 0
    assert ctypes.sizeof(ctypes.c_float) == 4



SAMPLING_CASES = {
    "subsample": {"seed": 7, "subsample": 0.8},
    "bytree": {"seed": 7, "bytree": 0.5},
    "bynode": {"seed": 7, "bynode": 0.5},
    "bylevel": {"seed": 3, "bylevel": 0.6},
    "all": {"seed": 11, "subsample": 0.7, "bytree": 0.8, "bylevel": 0.7, "bynode": 0.6},
}


@pytest.mark.parametrize("case", list(SAMPLING_CASES))
def test_sampling_parity(dp, oracle, device, case):
    """Row and column sampling (subsample, colsample_by{tree,level,node}, seed) train the
    same trees, row partitions and margins as the oracle's booster, round after round
    (the draws depend on the round, read by replayed round graphs from device memory)."""
    p = {"max_depth": 6, "eta": 0.3}
    sample = SAMPLING_CASES[case]
    print(f"[booster] sampling {case}: C2 40000 x 28, depth 6, 4 rounds", flush=True)
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 2, 40000, 28, 0, 1, p, 4,
                                                    20261202, sample=sample)
    _compare(bst, o_trees, o_margin, pos, n, 1)
    cfg = json.loads(bst.save_config())
    tp = cfg["learner"]["gradient_booster"]["updater"][0]["train_param"]
    assert tp["subsample"] == str(sample.get("subsample", 1))


@pytest.mark.parametrize("shape", ["few_features", "softmax", "present_value", "level_synced",
                                   "injected"])
def test_sampling_parity_paths(dp, oracle, device, shape):
    """Sampling on the other evaluation and growth paths: at most 16 features (one workgroup
    per node), ten concurrent class trees (each its own draws), present-value histograms of
    a mostly-missing matrix, level-synced growth (depth 17), and caller gradients."""
    import torch

    if shape == "few_features":
        p, sample = {"max_depth": 6, "eta": 0.3}, {"seed": 5, "subsample": 0.75, "bytree": 0.5,
                                                    "bynode": 0.75}
        args = (1, 10000, 8, 0, 1, p, 3, 20261201)
        kw = {}
    elif shape == "softmax":
        p, sample = {"max_depth": 4, "eta": 0.3}, {"seed": 9, "subsample": 0.8, "bynode": 0.5}
        args = (4, 2000, 784, 1, 10, p, 2, 20261204)
        kw = {}
    elif shape == "present_value":
        p, sample = {"max_depth": 7, "eta": 0.3}, {"seed": 2, "subsample": 0.9, "bylevel": 0.5,
                                                    "bynode": 0.8}
        args = (5, 6000, 120, 2, 1, p, 3, 20261205)
        kw = {"max_bin": 64, "extra": {"dp_sparse_hist": 1}}
    elif shape == "level_synced":
        p, sample = {"max_depth": 17, "eta": 0.3, "min_child_weight": 0.0}, \
            {"seed": 4, "subsample": 0.9, "bytree": 0.9, "bynode": 0.7}
        rng = np.random.default_rng(5)
        xv = rng.random((1000, 8), dtype=np.float32)
        yv = (rng.random(1000) < 0.5).astype(np.float32)
        args = (1, 1000, 8, 0, 1, p, 2, 0)
        kw = {"values_labels": (torch.as_tensor(xv, device=device),
                                torch.as_tensor(yv, device=device))}
    else:
        p, sample = {"max_depth": 8, "eta": 0.3}, {"seed": 6, "subsample": 0.5, "bytree": 0.5}
        args = (3, 30000, 128, 2, 1, p, 2, 20261203)
        kw = {"injected": True}
    print(f"[booster] sampling path {shape}", flush=True)
    bst, x, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, *args, sample=sample, **kw)
    _compare(bst, o_trees, o_margin, pos, n, args[4])


def test_sampled_graph_replays_equal_direct_launches(dp, device):
    """With sampling on, rounds replayed from cached graphs equal direct launches (each round
    stores its index for the sampling kernels before the replay)."""
    from dpgbdt import ops

    values, labels, _, _ = ops.synth(2, 20000, 5, n_features=28)
    models = []
    for graphs in (0, 1):
        dtrain = dp.DMatrix(values, labels)
        bst = dp.Booster({"objective": "binary:logistic", "max_depth": 5, "subsample": 0.7,
                          "colsample_bynode": 0.5, "seed": 3, "dp_graphs": graphs}, [dtrain])
        for r in range(6):
            bst.update(dtrain, r)
        models.append(bst.save_raw())
    assert models[0] == models[1]


def test_max_bin_is_not_changed_silently(dp, device):
    """max_bin above 256 is refused; the saved configuration reports the bins used: 256 with
    and without missing values (with them, a matrix some of whose features use all 256 bins
    keeps 16-bit symbols, missing = 256), and a matrix whose features have fewer bins keeps
    uint8 symbols with byte 255 for missing values."""
    import torch
    from dpgbdt import ops

    values, labels, _, _ = ops.synth(1, 5000, 7)
    dtrain = dp.DMatrix(values, labels)
    bst = dp.Booster({"objective": "binary:logistic", "max_bin": 1024}, [dtrain])
    with pytest.raises(dp.DPError, match="max_bin above 256"):
        bst.update(dtrain, 0)
    for holes, max_bin, symbol in ((False, 256, -1), (True, 256, 256), (True, 200, 255)):
        v = values.clone()
        if holes:
            v[::3, 2] = float("nan")
        d = dp.DMatrix(v, labels)
        b = dp.Booster({"objective": "binary:logistic", "max_bin": max_bin, "max_depth": 3}, [d])
        b.update(d, 0)
        cfg = json.loads(b.save_config())
        used = cfg["learner"]["gradient_booster"]["updater"][0]["hist_train_param"]["max_bin"]
        assert used == str(max_bin)
        cut_ptr, _, missing = d.cuts(max_bin)
        assert missing == symbol and np.diff(cut_ptr).max() == max_bin



@pytest.mark.parametrize("objective", ["multi:softprob", "multi:softmax"])
def test_resident_model_sequence(dp, oracle, device, objective):
    """The converter's native oracle (ResidentModel, native/class_model_convert.cpp:96-156)
    replayed call for call on a model this library trained: XGBoostVersion and XGBuildInfo
    checks, XGBoosterCreate(NULL, 0), XGBoosterLoadModelFromBuffer, SetParam device and
    nthread, XGBoosterGetNumFeature against the source's feature count, the
    XGBoosterSaveJsonConfig field checks, then XGBoosterPredictFromCudaArray with
    strict_shape and "missing":NaN for margins and values.  The margins must equal the
    oracle's training margins bit for bit."""
    import ctypes

    import torch

    rng = np.random.default_rng(31)
    n, f, k = 3000, 6, 3
    x = rng.normal(size=(n, f)).astype(np.float32)
    x[rng.random((n, f)) < 0.1] = np.nan
    y = (np.nan_to_num(x[:, 0]) + np.nan_to_num(x[:, 1]) > 0).astype(np.float32) + \
        (np.nan_to_num(x[:, 2]) > 0.5).astype(np.float32)
    values = torch.from_numpy(x).to(device)
    labels = torch.from_numpy(y).to(device)
    p = {"max_depth": 4, "eta": 0.3}
    bst, _, o_trees, o_margin, _, _ = _train_both(dp, oracle, device, 1, n, f, 1, k, p, 3, 0,
                                                 values_labels=(values, labels), record=0)
    # trained as multi:softmax (the reference trainer's objective); the softprob case
    # names the other objective the converter accepts in the saved model
    doc = json.loads(bst.save_raw())
    assert doc["learner"]["objective"]["name"] == "multi:softmax"
    doc["learner"]["objective"]["name"] = objective
    model = json.dumps(doc).encode()

    lib = dp.load()
    H = ctypes.c_void_p
    major, minor, patch = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    lib.XGBoostVersion(ctypes.byref(major), ctypes.byref(minor), ctypes.byref(patch))
    assert (major.value, minor.value, patch.value) == (3, 4, 1)
    info = ctypes.c_char_p()
    assert lib.XGBuildInfo(ctypes.byref(info)) == 0
    assert json.loads(info.value.decode())["USE_CUDA"] is True
    h = H()
    assert lib.XGBoosterCreate(None, 0, ctypes.byref(h)) == 0, lib.XGBGetLastError()
    try:
        buf = ctypes.create_string_buffer(model, len(model))
        assert lib.XGBoosterLoadModelFromBuffer(h, buf, len(model)) == 0, lib.XGBGetLastError()
        assert lib.XGBoosterSetParam(h, b"device", b"cuda:0") == 0
        assert lib.XGBoosterSetParam(h, b"nthread", b"4") == 0
        features = ctypes.c_uint64()
        assert lib.XGBoosterGetNumFeature(h, ctypes.byref(features)) == 0
        assert features.value == f
        size, text = ctypes.c_uint64(), ctypes.c_char_p()
        assert lib.XGBoosterSaveJsonConfig(h, ctypes.byref(size), ctypes.byref(text)) == 0
        cfg = json.loads(ctypes.string_at(text, size.value).decode())["learner"]
        assert cfg["generic_param"]["device"] == "cuda:0"
        assert cfg["gradient_booster"]["name"] == "gbtree"
        assert cfg["objective"]["name"] == objective
        assert int(cfg["learner_model_param"]["num_class"]) == k
        torch.cuda.synchronize()
        array = json.dumps({"data": [values.data_ptr(), True], "shape": [n, f], "strides": None,
                            "typestr": "<f4", "version": 3, "stream": 1})
        for margin in (True, False):
            options = json.dumps({"type": 1 if margin else 0, "training": False,
                                  "iteration_begin": 0, "iteration_end": 0,
                                  "strict_shape": True, "cache_id": 0})[:-1] + ',"missing":NaN}'
            shape = ctypes.POINTER(ctypes.c_uint64)()
            dims = ctypes.c_uint64()
            out = ctypes.POINTER(ctypes.c_float)()
            assert lib.XGBoosterPredictFromCudaArray(
                h, array.encode(), options.encode(), None, ctypes.byref(shape),
                ctypes.byref(dims), ctypes.byref(out)) == 0, lib.XGBGetLastError()
            columns = k if margin or objective == "multi:softprob" else 1
            assert dims.value == 2 and (shape[0], shape[1]) == (n, columns)
            got = torch.empty((n, columns), dtype=torch.float32, device=device)
            from dpgbdt import _hip_memcpy
            _hip_memcpy()(ctypes.c_void_p(got.data_ptr()),
                          ctypes.c_void_p(ctypes.addressof(out.contents)), n * columns * 4)
            torch.cuda.synchronize()
            got = got.cpu().numpy()
            if margin:
                np.testing.assert_array_equal(got.view(np.uint32), o_margin.view(np.uint32))
            elif objective == "multi:softmax":
                np.testing.assert_array_equal(got[:, 0],
                                              np.argmax(o_margin, axis=1).astype(np.float32))
            else:
                m = o_margin.astype(np.float64)
                prob = np.exp(m - m.max(axis=1, keepdims=True))
                prob /= prob.sum(axis=1, keepdims=True)
                np.testing.assert_allclose(got, prob, rtol=1e-5, atol=1e-7)
    finally:
        lib.XGBoosterFree(h)


def test_caller_gradients_may_be_overwritten_after_return(dp, device):
    """XGBoosterTrainOneIter returns only once its quantiser has read the caller's arrays:
    overwriting them from a non-blocking stream right after each call (with nothing ordering
    that stream after the library's) leaves the model and margins equal to a run whose
    buffers stay untouched."""
    import torch
    from dpgbdt import ops

    n = 200_000
    values, labels, g, h = ops.synth(1, n, 7, n_features=16, want_grad=True)
    g, h = g.reshape(-1, 1).contiguous(), h.reshape(-1, 1).contiguous()
    dtrain = dp.DMatrix(values, labels)
    params = {"objective": "reg:squarederror", "max_depth": 6, "eta": 0.3}
    side = torch.cuda.Stream(device=device)  # non-blocking with respect to the null stream
    out = []
    for overwrite in (False, True):
        bst = dp.Booster(params, [dtrain])
        gb, hb = g.clone(), h.clone()
        for r in range(3):
            torch.cuda.synchronize()
            gb.copy_(torch.roll(g, r))
            hb.copy_(torch.roll(h, r))
            torch.cuda.synchronize()
            bst.boost(dtrain, r, gb, hb)
            if overwrite:
                with torch.cuda.stream(side):
                    gb.fill_(1e6)
                    hb.fill_(-3.0)
        torch.cuda.synchronize()
        out.append((bst.save_raw(), bst.margins(n, 1)))
    assert out[0][0] == out[1][0]
    np.testing.assert_array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))


def test_train_one_iter_refuses_foreign_arrays(dp, device):
    """Gradient arrays the quantiser could not read in bounds are refused with an error: host
    memory, and a device allocation shorter than the declared shape."""
    import ctypes

    import torch
    from dpgbdt import ops

    n = 4096
    values, labels, _, _ = ops.synth(1, n, 3)
    dtrain = dp.DMatrix(values, labels)
    bst = dp.Booster({"objective": "reg:squarederror", "max_depth": 3}, [dtrain])
    lib = dp.load()

    def iface(ptr, rows):
        return json.dumps({"data": [ptr, True], "shape": [rows, 1], "strides": None,
                           "typestr": "<f4", "version": 3}).encode()

    ok = torch.zeros((n, 1), dtype=torch.float32, device=device)
    host = np.zeros(n, dtype=np.float32)
    assert lib.XGBoosterTrainOneIter(bst.handle, dtrain.handle, 0, iface(host.ctypes.data, n),
                                     iface(ok.data_ptr(), n)) == -1
    assert "grad must be device memory" in lib.XGBGetLastError().decode()
    # a hipMalloc allocation declared one float longer than the runtime says it is
    rt = ctypes.CDLL("libamdhip64.so.7")
    rt.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    rt.hipFree.argtypes = [ctypes.c_void_p]
    rt.hipMemGetAddressRange.argtypes = [ctypes.POINTER(ctypes.c_void_p),
                                         ctypes.POINTER(ctypes.c_size_t), ctypes.c_void_p]
    p = ctypes.c_void_p()
    assert rt.hipMalloc(ctypes.byref(p), 1 << 20) == 0
    try:
        base, size = ctypes.c_void_p(), ctypes.c_size_t()
        assert rt.hipMemGetAddressRange(ctypes.byref(base), ctypes.byref(size), p) == 0
        assert base.value == p.value and size.value >= 1 << 20
        rows = size.value // 4 + 1
        assert lib.XGBoosterTrainOneIter(bst.handle, dtrain.handle, 0, iface(p.value, rows),
                                         iface(p.value, rows)) == -1
        assert "exceed its device allocation" in lib.XGBGetLastError().decode()
    finally:
        rt.hipFree(p)
    # the booster is unharmed: a valid round still trains
    bst.boost(dtrain, 0, ok.clone(), torch.ones((n, 1), dtype=torch.float32, device=device))
    assert bst.num_boosted_rounds() == 1


@pytest.mark.parametrize("record", [0, 1])
def test_256_bins_with_missing_values(dp, oracle, device, record):
    """The reference's default max_bin (256) on data with missing values
    (native/class_native_training.cuh:24, :51): a C5-shaped matrix (200,000 x 1,000, N(0,1)
    values, 10 % missing, squared error on the sum of 20 features) trains 256 bins per
    feature, with the missing marker a symbol of its own, bit-exact against the oracle; the
    saved configuration reports 256."""
    import torch

    n, f = 200_000, 1000
    print(f"[booster] 256 bins with 10 % missing values, {n} x {f}, record {record}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(97)
    x = torch.randn((n, f), generator=g)
    x[torch.rand((n, f), generator=g) < 0.1] = float("nan")
    cols = torch.randperm(f, generator=g)[:20]
    y = torch.nan_to_num(x[:, cols], nan=0.0).sum(dim=1) + 0.1 * torch.randn(n, generator=g)
    values, labels = x.to(device), y.to(device)
    del x
    p = {"max_depth": 6, "eta": 0.3}
    bst, xs, o_trees, o_margin, pos, n = _train_both(dp, oracle, device, 5, n, f, 2, 1, p, 2, 0,
                                                     values_labels=(values, labels),
                                                     record=record)
    _compare(bst, o_trees, o_margin, pos, n, 1)
    cfg = json.loads(bst.save_config())
    assert cfg["learner"]["gradient_booster"]["updater"][0]["hist_train_param"]["max_bin"] == "256"
    assert bst.tuning()["layout"] == "present-value"
    assert any(t["default_left"].any() for t in o_trees), "learned default direction unused"
    # every feature has 256 bins, so missing values take symbol 256 (16-bit symbols)
    cut_ptr, _, _ = oracle.compute_cuts(xs, 256)
    assert np.diff(cut_ptr).min() == 256
    assert oracle.missing_symbol(cut_ptr, True) == 256
