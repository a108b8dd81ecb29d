"""The histogram autotuner (tune.cpp) and the launch shapes it chooses among.

Every launch shape computes the same exact integer sums, so a booster trained
with any forced shape (tiles per work item, rows per lane per step, work items
per pass) must save the model, row partition and margins of the default shape,
which the oracle-parity tests pin.  The autotuner's report names timed
candidates and picks one of them; dp_autotune=0 keeps the defaults.
"""
import itertools
import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SHAPES = [dict(zip(("dp_hist_tiles", "dp_hist_unroll", "dp_hist_items", "dp_hist_split",
                    "dp_hist_deep"), c))
          for c in itertools.product((1, 2), (1, 2), (512, 1024, 2048), (0, 4, 5), (0, 1))
          if (c[0] == 2 or c[3] == 0) and (c[3] == 0 or c[4] == 0)]


def _train(dp, values, labels, params, rounds, n, k):
    dtrain = dp.DMatrix(values, labels)
    bst = dp.Booster(dict(params, dp_record_positions=1), [dtrain])
    for r in range(rounds):
        bst.update(dtrain, r)
    return bst.save_raw(), bst.last_positions(n), bst.margins(n, k), bst


@pytest.mark.parametrize("case", ["c2_two_tiles", "c3_paired_tiles", "odd_pair", "c4_odd_tiles",
                                  "missing", "present_value"])
def test_every_launch_shape_trains_the_same_model(dp, device, case):
    """Trees, partitions and margins are identical under all 36 forced launch shapes
    (two tiles per item over an odd tile count leaves a one-tile last group, with and without
    the lanes' swapped tile order; one or three blocks of rows in flight; C3's tiles 6 and 7
    paired, a pair item for one-tile and for two-tile shapes; tiles 1 and 2 paired, which
    only one-tile shapes use; the MISSING kernels; present-value histograms take the
    work-item count only)."""
    import torch
    from dpgbdt import ops

    if case == "c2_two_tiles":
        values, labels, _, _ = ops.synth(2, 60000, 3, n_features=28)
        params, k = {"objective": "binary:logistic", "max_depth": 7, "eta": 0.3}, 1
    elif case == "c3_paired_tiles":
        values, labels, _, _ = ops.synth(3, 40000, 6, n_features=128)
        params, k = {"objective": "binary:logistic", "max_depth": 6, "eta": 0.3}, 1
    elif case == "odd_pair":  # tile 0: 256 bins; tiles 1 and 2: 16 values each
        g = torch.Generator(device="cpu").manual_seed(7)
        n = 30000
        wide = torch.randn((n, 16), generator=g)
        narrow = torch.randint(0, 16, (n, 32), generator=g).to(torch.float32)
        values = torch.cat([wide, narrow], dim=1).contiguous().to(device)
        score = values[:, 0] + 0.25 * values[:, 20] - 0.2 * values[:, 33]
        labels = (torch.sigmoid(score) > torch.rand(n, generator=g).to(device)).to(torch.float32)
        params, k = {"objective": "binary:logistic", "max_depth": 6, "eta": 0.3}, 1
    elif case == "c4_odd_tiles":
        values, labels, _, _ = ops.synth(4, 3000, 4, n_features=784)
        params, k = {"objective": "multi:softprob", "num_class": 10, "max_depth": 4,
                     "eta": 0.3}, 10
    elif case == "missing":
        values, labels, _, _ = ops.synth(1, 50000, 5, n_features=40)
        g = torch.Generator(device="cpu").manual_seed(3)
        values[(torch.rand(values.shape, generator=g) < 0.3).to(values.device)] = float("nan")
        params, k = {"objective": "binary:logistic", "max_depth": 6, "eta": 0.3,
                     "dp_sparse_hist": 0}, 1
    else:
        values, labels, _, _ = ops.synth(5, 40000, 200, n_features=200)
        params, k = {"objective": "reg:squarederror", "max_depth": 6, "eta": 0.3,
                     "max_bin": 64}, 1
    n = values.shape[0]
    base = _train(dp, values, labels, dict(params, dp_autotune=0), 3, n, k)
    assert base[3].tuning()["defaults"] is True
    want = {"c3_paired_tiles": 1 << 6, "odd_pair": 1 << 1}.get(case, 0)
    assert base[3].tuning()["paired_tiles"] == want
    unpaired = _train(dp, values, labels, dict(params, dp_autotune=0, dp_hist_pair=0), 3, n, k)
    assert unpaired[0] == base[0]
    for shape in SHAPES:
        if case == "present_value" and (shape["dp_hist_tiles"] == 2 or shape["dp_hist_deep"]):
            continue  # one present-value tile per item: only the item count applies
        print(f"[tuning] {case} {shape}", flush=True)
        got = _train(dp, values, labels, dict(params, **shape), 3, n, k)
        assert got[3].tuning()["forced"] is True
        assert got[0] == base[0], shape
        np.testing.assert_array_equal(got[1], base[1])
        np.testing.assert_array_equal(np.asarray(got[2]).view(np.uint32),
                                      np.asarray(base[2]).view(np.uint32))


def test_autotuner_report_and_choice(dp, device):
    """The autotuned booster reports every timed candidate of the root and gathered passes
    and chooses, of the candidates within 3 % of the fastest (5 % for the gathered passes),
    the one with the fewest work items (then one row per step, then the fastest); its model
    equals the default shape's."""
    from dpgbdt import ops

    values, labels, _, _ = ops.synth(2, 200000, 8, n_features=28)
    params = {"objective": "binary:logistic", "max_depth": 6, "eta": 0.3}
    tuned = _train(dp, values, labels, params, 2, 200000, 1)
    report = tuned[3].tuning()
    for name in ("root", "gathered"):
        cands = report[name]
        # (1 tile + 2 tiles x 3 orders) x 2 unrolls x 3 items, and on the root pass also the
        # three-block prefetch of each unswapped shape (1 tile + 2 tiles) x 2 unrolls x 3 items
        assert len(cands) == (36 if name == "root" else 24)
        assert all(c["ms"] > 0 for c in cands)
        fastest = min(c["ms"] for c in cands)
        band = 1.03 if name == "root" else 1.05  # the gathered passes' wider near-tie band
        near = [c for c in cands if c["ms"] <= fastest * band]
        best = min(near, key=lambda c: (c["items"], c["unroll"], c["ms"]))
        assert report["chosen"][name] == {key: best[key]
                                          for key in ("tiles", "unroll", "items", "split", "deep")}
    base = _train(dp, values, labels, dict(params, dp_autotune=0), 2, 200000, 1)
    assert tuned[0] == base[0]
    # the choice is cached per process: a second booster of the shape reports the same
    again = _train(dp, values, labels, params, 1, 200000, 1)
    assert again[3].tuning() == report
    print(json.dumps(report["chosen"]), flush=True)


@pytest.mark.parametrize("case", ["c4_zero_pixels", "c1_few_features", "c2_wide_bins",
                                  "le64_bins"])
def test_skip_bins_train_the_oracle_model(dp, oracle, device, case):
    """Skip bins (each feature's most frequent bin left out of the histograms and restored
    from the node totals by the evaluation) train the oracle's trees, partitions and
    margins bit for bit, forced on (dp_skip_bin 2) for every evaluation kernel: at most 16
    features (one workgroup per node), 256 bins (one feature per wavefront), at most 64
    bins (four features per wavefront), and C4's zero-dominated pixels, where the automatic
    rule takes them; dp_skip_bin 0 gives the same model."""
    import test_gpu_booster as tb

    if case == "c4_zero_pixels":
        args, p, kw = (4, 3000, 784, 1, 10), {"max_depth": 5, "eta": 0.3}, {}
    elif case == "c1_few_features":
        args, p, kw = (1, 20000, 8, 0, 1), {"max_depth": 6, "eta": 0.3}, {}
    elif case == "c2_wide_bins":
        args, p, kw = (2, 30000, 28, 0, 1), {"max_depth": 6, "eta": 0.3}, {}
    else:
        args, p, kw = (1, 20000, 40, 0, 1), {"max_depth": 6, "eta": 0.3}, {"max_bin": 64}
    config, n, f, objective, k = args
    models = []
    for mode in (2, 0):
        print(f"[skip] {case} dp_skip_bin={mode}", flush=True)
        bst, x, o_trees, o_margin, pos, n = tb._train_both(
            dp, oracle, device, config, n, f, objective, k, p, 2, 20261230, **kw,
            extra={"dp_skip_bin": mode})
        tb._compare(bst, o_trees, o_margin, pos, n, k)
        models.append(bst.save_raw())
    assert models[0] == models[1]


def test_automatic_skip_rule_counts_padding(dp, device):
    """dp_skip_bin=1 takes skip bins when they remove at least 20 % of the element atomics,
    counting the last tile's padding features: 8 features in a 16-wide tile qualify (share
    >= 0.5), 28 quantile-binned features in two tiles (4 padding slots of 32) do not."""
    from dpgbdt import ops

    for config, f, expect in ((1, 8, True), (2, 28, False)):
        values, labels, _, _ = ops.synth(config, 20000, 3, n_features=f)
        dtrain = dp.DMatrix(values, labels)
        bst = dp.Booster({"objective": "binary:logistic", "max_depth": 4}, [dtrain])
        bst.update(dtrain, 0)
        report = bst.tuning()
        print(f"[skip rule] {f} features: skip_bins {report['skip_bins']}, "
              f"share {report.get('skip_share')}", flush=True)
        assert report["skip_bins"] is expect
        slots = 16 * ((f + 15) // 16)
        assert report["skip_share"] >= (slots - f) / slots
