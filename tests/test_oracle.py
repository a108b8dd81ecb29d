"""Pins the CPU oracle (oracle/dp_oracle.c) to what the mathematics fixes.

XGBoost 3.4.1 -- where the reference's implementation of this path lives --
is absent, and the reference holds no numeric fixtures for it, so each oracle
function is checked against something independent of its own formula:

  expf            float64 numpy exp (ulp bound)
  cuts / bins     the stated quantile definition via numpy sort/unique, the
                  quantile property, np.searchsorted and the routing identity
                  x < cut[b]  <=>  bin(x) <= b
  gradients       float64 closed forms (sigmoid, softmax) and sum_k g_k = 0
  quantiser       round-to-nearest of x * 2^e, |q| <= 2^30, frexp exponent
  histogram       int64 np.add.at per feature; counts = np.bincount; the
                  OpenMP version equals the serial one
  subtraction     hist(P) = hist(L) + hist(R) for a random partition
  gain / weight   numerical minimisation (scipy) of the regularised
                  second-order objective G w + (H + lambda) w^2 / 2 + alpha |w|
  split search    brute force over every (feature, threshold, missing side)
                  computed from raw rows, not from histograms
  partition       stable order of numpy masks
  tree            an independent pure-Python depth-wise builder on raw rows
"""
import numpy as np
import pytest
from scipy.optimize import minimize_scalar


def ulp_distance(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, np.int64(-2**31) - a, a)
    b = np.where(b < 0, np.int64(-2**31) - b, b)
    return np.abs(a - b)


def test_expf_ulp(oracle):
    xs = np.linspace(-86.9, 88.7, 200001, dtype=np.float32)
    got = np.array([oracle.expf(x) for x in xs[::7]], dtype=np.float32)
    ref = np.exp(xs[::7].astype(np.float64)).astype(np.float32)
    assert ulp_distance(got, ref).max() <= 2
    assert oracle.expf(0.0) == 1.0
    assert oracle.expf(-100.0) == 0.0
    assert np.isinf(oracle.expf(89.0))
    assert np.isnan(oracle.expf(float("nan")))


def _expected_cuts(col, max_bin):
    """The stated exact quantile definition, via numpy."""
    v = col[~np.isnan(col)].astype(np.float32)
    v = np.where(v == 0, np.float32(0), v)
    if v.size == 0:
        return np.array([np.float32(1e-5)], np.float32)
    v = np.sort(v)
    u = np.unique(v)
    last = np.float32(v[-1] + (np.float32(abs(v[-1])) + np.float32(1e-5)))
    if u.size <= max_bin:
        return np.concatenate([u[1:], [last]]).astype(np.float32)
    out, prev = [], v[0]
    for i in range(1, max_bin):
        c = v[(i * v.size) // max_bin]
        if c > prev:
            out.append(c)
            prev = c
    return np.array(out + [last], np.float32)


@pytest.mark.parametrize("max_bin", [2, 16, 64, 255, 256])
def test_cuts_definition_and_quantiles(oracle, max_bin):
    rng = np.random.default_rng(max_bin)
    n = 5000
    x = np.stack([rng.normal(size=n), rng.lognormal(size=n), rng.integers(0, 16, n),
                  rng.integers(0, 400, n), np.full(n, 3.5), np.full(n, np.nan)],
                 axis=1).astype(np.float32)
    x[rng.random(n) < 0.3, 1] = np.nan
    x[:5, 2] = -0.0
    cut_ptr, cuts, mins = oracle.compute_cuts(x, max_bin)
    for f in range(x.shape[1]):
        c = cuts[cut_ptr[f]:cut_ptr[f + 1]]
        np.testing.assert_array_equal(c.view(np.uint32), _expected_cuts(x[:, f], max_bin).view(np.uint32))
        assert np.all(np.diff(c) > 0) and 1 <= c.size <= max_bin
    # quantile property: continuous feature, bins hold ~n/max_bin rows each
    bins = oracle.bin_matrix(x, cut_ptr, cuts, 255 if max_bin <= 255 else -1)
    counts = np.bincount(bins[:, 0], minlength=max_bin)[: cut_ptr[1] - cut_ptr[0]]
    assert counts.max() <= 2 * n / max_bin + 2


def test_binning_routing_identity(oracle):
    rng = np.random.default_rng(5)
    x = rng.normal(size=(3000, 4)).astype(np.float32)
    x[::11, 2] = np.nan
    cut_ptr, cuts, _ = oracle.compute_cuts(x, 32)
    bins = oracle.bin_matrix(x, cut_ptr, cuts, 255)
    for f in range(4):
        c = cuts[cut_ptr[f]:cut_ptr[f + 1]]
        col = x[:, f]
        ok = ~np.isnan(col)
        expect = np.minimum(np.searchsorted(c, col[ok], side="right"), c.size - 1)
        np.testing.assert_array_equal(bins[ok, f], expect)
        assert np.all(bins[~ok, f] == 255)
        for b in range(c.size):  # x < cut[b]  <=>  bin <= b
            np.testing.assert_array_equal(col[ok] < c[b], bins[ok, f] <= b)


def test_gradients_closed_forms(oracle):
    rng = np.random.default_rng(9)
    n, k = 4000, 5
    m = (rng.normal(size=n) * 3).astype(np.float32)
    y = rng.integers(0, 2, n).astype(np.float32)
    g, h = oracle.gradients(oracle.OBJ_LOGISTIC, m, y, 1)
    p = 1 / (1 + np.exp(-m.astype(np.float64)))
    np.testing.assert_allclose(g[:, 0], p - y, rtol=0, atol=3e-7)
    # float32 1 - p cancels near p = 1: bound the error by a few ulp of 1
    np.testing.assert_allclose(h[:, 0], np.maximum(p * (1 - p), 1e-16), rtol=3e-6, atol=2e-7)
    mm = (rng.normal(size=(n, k)) * 3).astype(np.float32)
    yy = rng.integers(0, k, n).astype(np.float32)
    g, h = oracle.gradients(oracle.OBJ_SOFTPROB, mm, yy, k)
    e = np.exp(mm - mm.max(axis=1, keepdims=True))
    sp = e / e.sum(axis=1, keepdims=True)
    onehot = np.eye(k)[yy.astype(int)]
    np.testing.assert_allclose(g, sp - onehot, atol=3e-7)
    np.testing.assert_allclose(h, np.maximum(2 * sp * (1 - sp), 1e-16), rtol=3e-6, atol=4e-7)
    assert np.abs(g.astype(np.float64).sum(axis=1)).max() < 1e-6
    g, h = oracle.gradients(oracle.OBJ_SQUARED, m, y, 1)
    np.testing.assert_array_equal(g[:, 0], m - y)
    assert np.all(h == 1)


def test_quantiser_round_to_nearest(oracle):
    rng = np.random.default_rng(1)
    g = (rng.normal(size=10000) * 7).astype(np.float32)
    h = rng.uniform(0.01, 0.25, 10000).astype(np.float32)
    eg, eh, qg, qh = oracle.quantise(g, h)[0]
    assert eg == 30 - np.frexp(np.abs(g).max())[1]
    assert eh == 30 - np.frexp(np.abs(h).max())[1]
    np.testing.assert_array_equal(qg, np.rint(np.ldexp(g.astype(np.float64), eg)).astype(np.int32))
    np.testing.assert_array_equal(qh, np.rint(np.ldexp(h.astype(np.float64), eh)).astype(np.int32))
    assert np.abs(qg).max() <= 2**30 and np.abs(qg).max() > 2**29
    assert oracle.unscale(eg) == 2.0 ** -eg


def _quantised_case(oracle, n=2000, f=6, nb=24, seed=3, missing=True):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(n, f)).astype(np.float32)
    x[:, 1] = rng.integers(0, 5, n)
    if missing:
        x[rng.random((n, f)) < 0.15] = np.nan
    cut_ptr, cuts, _ = oracle.compute_cuts(x, nb)
    mb = 255 if missing else -1
    bins = oracle.bin_matrix(x, cut_ptr, cuts, mb)
    g = rng.normal(size=n).astype(np.float32)
    h = rng.uniform(0.05, 1.0, n).astype(np.float32)
    eg, eh, qg, qh = oracle.quantise(g, h)[0]
    return x, bins, cut_ptr, cuts, mb, qg, qh, eg, eh


def test_histogram_counts_and_parallel(oracle):
    x, bins, cut_ptr, cuts, mb, qg, qh, eg, eh = _quantised_case(oracle)
    hist = oracle.hist(bins, qg, qh, bin_stride=32, missing_bin=mb)
    for f in range(bins.shape[1]):
        keep = bins[:, f] != mb
        ref = np.zeros((32, 2), np.int64)
        np.add.at(ref[:, 0], bins[keep, f], qg[keep].astype(np.int64))
        np.add.at(ref[:, 1], bins[keep, f], qh[keep].astype(np.int64))
        np.testing.assert_array_equal(hist[f], ref)
    counts = oracle.hist(bins, np.ones_like(qg), np.zeros_like(qh), bin_stride=32, missing_bin=mb)
    for f in range(bins.shape[1]):
        keep = bins[:, f] != mb
        np.testing.assert_array_equal(counts[f, :, 0], np.bincount(bins[keep, f], minlength=32))
    par = oracle.hist_parallel(bins, qg, qh, bin_stride=32, missing_bin=mb, threads=4)
    np.testing.assert_array_equal(par, hist)


def test_subtraction_identity(oracle):
    x, bins, cut_ptr, cuts, mb, qg, qh, eg, eh = _quantised_case(oracle, seed=8)
    rng = np.random.default_rng(0)
    perm = rng.permutation(bins.shape[0]).astype(np.uint32)
    left, right = perm[:700], perm[700:]
    hp = oracle.hist(bins, qg, qh, bin_stride=32, missing_bin=mb)
    hl = oracle.hist(bins, qg, qh, rows=left, bin_stride=32, missing_bin=mb)
    hr = oracle.hist(bins, qg, qh, rows=right, bin_stride=32, missing_bin=mb)
    np.testing.assert_array_equal(hp, hl + hr)


@pytest.mark.parametrize("lam,alpha,mcw", [(1.0, 0.0, 1.0), (0.5, 0.8, 0.0), (0.0, 2.0, 3.0)])
def test_gain_and_weight_minimise_objective(oracle, lam, alpha, mcw):
    """gain(G,H) = -2 min_w [G w + (H+lambda) w^2/2 + alpha|w|], weight = argmin."""
    p = oracle.params(lam=lam, alpha=alpha, min_child_weight=mcw)
    rng = np.random.default_rng(2)
    for _ in range(40):
        G = float(rng.normal() * 5)
        H = float(rng.uniform(0.1, 10.0))
        res = minimize_scalar(lambda w: G * w + 0.5 * (H + lam) * w * w + alpha * abs(w),
                              bounds=(-1e3, 1e3), method="bounded", options={"xatol": 1e-12})
        if H < mcw:
            assert oracle.calc_gain(p, G, H) == 0.0 and oracle.calc_weight(p, G, H) == 0.0
            continue
        assert abs(oracle.calc_gain(p, G, H) + 2 * res.fun) < 1e-6 * max(1.0, abs(res.fun))
        assert abs(oracle.calc_weight(p, G, H) - res.x) < 1e-5


def _brute_force_split(bins, qg, qh, rows, nb_per_feature, mb, ug, uh, p, allowed=None):
    """Every (feature, bin, missing side) from raw row selections; tie rule:
    larger loss, then lower feature, then lower bin, then missing-right.
    allowed: optional boolean mask of the candidate features."""
    lam, alpha, mcw = float(p.lambda_), float(p.alpha), float(p.min_child_weight)

    def gain(G, H):
        if H < mcw or H <= 0:
            return 0.0
        t = G - alpha if G > alpha else (G + alpha if G < -alpha else 0.0)
        return (t * t) / (H + lam)

    qg_r = qg[rows].astype(np.int64)
    qh_r = qh[rows].astype(np.int64)
    GP, HP = int(qg_r.sum()), int(qh_r.sum())
    parent = gain(GP * ug, HP * uh)
    best = (-np.inf, None)
    for f in range(bins.shape[1]):
        if allowed is not None and not allowed[f]:
            continue
        col = bins[rows, f].astype(np.int64)
        miss = col == mb
        for b in range(nb_per_feature[f]):
            for dl in (0, 1):
                left = (~miss & (col <= b)) | (miss & bool(dl))
                gl, hl = int(qg_r[left].sum()), int(qh_r[left].sum())
                gr, hr = GP - gl, HP - hl
                if hl <= 0 or hr <= 0 or hl * uh < mcw or hr * uh < mcw:
                    continue
                loss = (gain(gl * ug, hl * uh) + gain(gr * ug, hr * uh)) - parent
                key = (loss, -f, -b, -dl)
                if best[1] is None or key > best[0]:
                    best = (key, (f, b, dl, gl, hl))
    return best


@pytest.mark.parametrize("seed", [3, 4, 5])
def test_split_search_matches_brute_force(oracle, seed):
    x, bins, cut_ptr, cuts, mb, qg, qh, eg, eh = _quantised_case(oracle, n=300, f=4, nb=8,
                                                                  seed=seed)
    nbf = np.diff(cut_ptr).astype(np.int32)
    rows = np.arange(0, 300, 2, dtype=np.uint32)
    for p in (oracle.params(), oracle.params(lam=0.0, alpha=0.3, min_child_weight=2.0)):
        hist = oracle.hist(bins, qg, qh, rows=rows, bin_stride=8, missing_bin=mb)
        got = oracle.evaluate_split(hist, nbf, qg[rows].astype(np.int64).sum(),
                                    qh[rows].astype(np.int64).sum(), eg, eh, p)
        key, val = _brute_force_split(bins, qg, qh, rows, nbf, mb, oracle.unscale(eg),
                                      oracle.unscale(eh), p)
        assert got["valid"] == 1
        assert (got["feature"], got["bin"], got["default_left"], got["gl"], got["hl"]) == val
        assert got["loss_chg"] == key[0]


def test_split_never_picks_an_empty_bin(oracle):
    """The evaluation's pick is never an empty bin past the first.  An empty bin b > 0 has the
    left sums of bin b - 1, so its candidate has bin b - 1's loss and the tie goes to the lower
    bin; the GPU evaluation of small nodes relies on this and evaluates only the non-empty bins
    (and bin 0).  Random sparse 64-bin features with missing mass, under three parameter sets;
    the cases where an empty bin directly follows the pick (a tie the rule resolves) are
    counted, so the check is exercised."""
    rng = np.random.default_rng(17)
    ties = 0
    for p in (oracle.params(), oracle.params(lam=0.0, alpha=0.3, min_child_weight=2.0),
              oracle.params(lam=5.0, min_child_weight=0.0)):
        for _ in range(400):
            nb = int(rng.integers(2, 65))
            hist = np.zeros((1, 64, 2), dtype=np.int64)
            live = rng.choice(nb, size=int(rng.integers(1, min(nb, 20) + 1)), replace=False)
            hist[0, live, 0] = rng.integers(-(1 << 20), 1 << 20, size=live.size)
            hist[0, live, 1] = rng.integers(1, 1 << 20, size=live.size)
            mg = int(rng.integers(-(1 << 22), 1 << 22)) if rng.random() < 0.7 else 0
            mh = int(rng.integers(1, 1 << 22)) if mg else 0
            gp, hp = int(hist[0, :, 0].sum()) + mg, int(hist[0, :, 1].sum()) + mh
            got = oracle.evaluate_split(hist, np.array([nb], dtype=np.int32), gp, hp, 16, 16, p)
            if not got["valid"]:
                continue
            b = got["bin"]
            assert b == 0 or hist[0, b].any(), (nb, b)
            if b + 1 < nb and not hist[0, b + 1].any():
                ties += 1
    assert ties > 300  # 730 of 1,172 valid cases with this seed


def test_partition_is_stable(oracle):
    x, bins, cut_ptr, cuts, mb, qg, qh, eg, eh = _quantised_case(oracle, seed=11)
    rng = np.random.default_rng(3)
    ridx = rng.permutation(bins.shape[0]).astype(np.uint32)
    for feat, b, dl in [(0, 5, 0), (1, 2, 1), (3, 0, 1)]:
        out, nl = oracle.partition(ridx, 100, 1500, bins, feat, b, dl, mb)
        seg = ridx[100:1500]
        col = bins[seg, feat].astype(np.int64)
        left = np.where(col == mb, bool(dl), col <= b)
        np.testing.assert_array_equal(out[100:1500], np.concatenate([seg[left], seg[~left]]))
        assert nl == left.sum()
        np.testing.assert_array_equal(out[:100], ridx[:100])
        np.testing.assert_array_equal(out[1500:], ridx[1500:])


def _reference_tree(bins, qg, qh, cut_ptr, mb, ug, uh, p, allowed_fn=None):
    """Independent depth-wise builder on raw rows (no histograms, no subtraction).
    allowed_fn(depth, nid): optional candidate-feature mask of each node."""
    nbf = np.diff(cut_ptr).astype(np.int32)
    nodes = [{"rows": np.arange(bins.shape[0], dtype=np.uint32), "depth": 0}]
    out = []
    level = [0]
    while level:
        nxt = []
        for nid in level:
            nd = nodes[nid]
            rec = {"nid": nid, "left": -1}
            if nd["depth"] < p.max_depth:
                allowed = allowed_fn(nd["depth"], nid) if allowed_fn else None
                key, val = _brute_force_split(bins, qg, qh, nd["rows"], nbf, mb, ug, uh, p,
                                              allowed)
                if val is not None and key[0] > 1e-6 and key[0] >= p.gamma:
                    f, b, dl, gl, hl = val
                    col = bins[nd["rows"], f].astype(np.int64)
                    left = np.where(col == mb, bool(dl), col <= b)
                    lid, rid = len(nodes), len(nodes) + 1
                    nodes.append({"rows": nd["rows"][left], "depth": nd["depth"] + 1})
                    nodes.append({"rows": nd["rows"][~left], "depth": nd["depth"] + 1})
                    rec.update(left=lid, right=rid, feature=f, bin=b, dl=dl)
                    nxt += [lid, rid]
            out.append(rec)
        level = nxt
    out.sort(key=lambda r: r["nid"])
    return out, nodes


def test_tree_matches_independent_builder(oracle):
    x, bins, cut_ptr, cuts, mb, qg, qh, eg, eh = _quantised_case(oracle, n=400, f=3, nb=6, seed=21)
    p = oracle.params(max_depth=4, eta=0.5)
    tree, ridx = oracle.grow_tree(bins, cut_ptr, cuts, mb, qg, qh, eg, eh, p, bin_stride=8)
    ref, nodes = _reference_tree(bins, qg, qh, cut_ptr, mb, oracle.unscale(eg), oracle.unscale(eh), p)
    assert len(ref) == len(tree["left"])
    for r in ref:
        nid = r["nid"]
        assert tree["left"][nid] == r["left"]
        if r["left"] != -1:
            assert (tree["right"][nid], tree["feature"][nid], tree["split_bin"][nid],
                    tree["default_left"][nid]) == (r["right"], r["feature"], r["bin"], r["dl"])
        else:
            rows = nodes[nid]["rows"]
            G = qg[rows].astype(np.int64).sum() * oracle.unscale(eg)
            H = qh[rows].astype(np.int64).sum() * oracle.unscale(eh)
            assert tree["leaf_value"][nid] == np.float32(oracle.calc_weight(p, G, H) * 0.5)
            np.testing.assert_array_equal(np.sort(ridx[tree["seg_begin"][nid]:tree["seg_end"][nid]]),
                                          np.sort(rows))
    # routing of the float matrix through split_conditions agrees with the partition
    pos = oracle.positions(tree, ridx, bins.shape[0])
    leaf_of = {nid: tree["leaf_value"][nid] for nid in range(len(tree["left"]))}
    pred = oracle.predict_tree(tree, x)
    np.testing.assert_array_equal(pred, np.array([leaf_of[i] for i in pos], np.float32))


def _wide_case(oracle, n=600, seed=4):
    """Missing values beside features that use all 256 bins: missing is symbol 256."""
    rng = np.random.default_rng(seed)
    x = np.stack([rng.normal(size=n), rng.permutation(n).astype(np.float64),
                  rng.integers(0, 7, n)], axis=1).astype(np.float32)
    x[rng.random(n) < 0.2, 0] = np.nan
    x[rng.random(n) < 0.1, 1] = np.nan
    cut_ptr, cuts, _ = oracle.compute_cuts(x, 256)
    mb = oracle.missing_symbol(cut_ptr, True)
    bins = oracle.bin_matrix(x, cut_ptr, cuts, mb)
    g = rng.normal(size=n).astype(np.float32)
    h = rng.uniform(0.05, 1.0, n).astype(np.float32)
    eg, eh, qg, qh = oracle.quantise(g, h)[0]
    return x, bins, cut_ptr, cuts, mb, qg, qh, eg, eh


def test_wide_symbols_for_256_bins_with_missing(oracle):
    """max_bin 256 on a matrix with missing values: features with more than 256 distinct
    values get 256 bins, so the missing marker is symbol 256 in uint16 bins; the bins equal
    searchsorted on the cuts, the histogram leaves missing rows out and puts bin 255's rows
    in slot 255, and the partition at bin 255 sends every present row left and the missing
    rows to the default side."""
    x, bins, cut_ptr, cuts, mb, qg, qh, eg, eh = _wide_case(oracle)
    nbf = np.diff(cut_ptr)
    assert mb == 256 and bins.dtype == np.uint16 and nbf.max() == 256
    assert oracle.missing_symbol(cut_ptr, False) == -1
    assert oracle.missing_symbol(np.array([0, 255, 300]), True) == 255
    for f in range(x.shape[1]):
        c = cuts[cut_ptr[f]:cut_ptr[f + 1]]
        ok = ~np.isnan(x[:, f])
        np.testing.assert_array_equal(bins[ok, f],
                                      np.minimum(np.searchsorted(c, x[ok, f], side="right"),
                                                 c.size - 1))
        assert np.all(bins[~ok, f] == 256)
    assert (bins[:, 1] == 255).any()  # the top bin is used beside the missing marker
    hist = oracle.hist(bins, qg, qh, bin_stride=256, missing_bin=mb)
    for f in range(x.shape[1]):
        keep = bins[:, f] != mb
        ref = np.zeros((256, 2), np.int64)
        np.add.at(ref[:, 0], bins[keep, f], qg[keep].astype(np.int64))
        np.add.at(ref[:, 1], bins[keep, f], qh[keep].astype(np.int64))
        np.testing.assert_array_equal(hist[f], ref)
    ridx = np.arange(x.shape[0], dtype=np.uint32)
    for dl in (0, 1):
        out, nl = oracle.partition(ridx, 0, x.shape[0], bins, 1, 255, dl, mb)
        present = ~np.isnan(x[:, 1])
        left = present | (bool(dl) & ~present)
        np.testing.assert_array_equal(out, np.concatenate([ridx[left], ridx[~left]]))
        assert nl == left.sum()


def test_wide_tree_matches_independent_builder(oracle):
    """A tree over 256-bin features with missing values (uint16 symbols) equals the
    independent brute-force builder's, node for node."""
    x, bins, cut_ptr, cuts, mb, qg, qh, eg, eh = _wide_case(oracle, n=300, seed=7)
    p = oracle.params(max_depth=3, eta=0.5)
    tree, ridx = oracle.grow_tree(bins, cut_ptr, cuts, mb, qg, qh, eg, eh, p, bin_stride=256)
    ref, nodes = _reference_tree(bins, qg, qh, cut_ptr, mb, oracle.unscale(eg), oracle.unscale(eh), p)
    assert len(ref) == len(tree["left"]) > 1
    for r in ref:
        nid = r["nid"]
        assert tree["left"][nid] == r["left"]
        if r["left"] != -1:
            assert (tree["right"][nid], tree["feature"][nid], tree["split_bin"][nid],
                    tree["default_left"][nid]) == (r["right"], r["feature"], r["bin"], r["dl"])
    pos = oracle.positions(tree, ridx, bins.shape[0])
    leaf_of = {nid: tree["leaf_value"][nid] for nid in range(len(tree["left"]))}
    np.testing.assert_array_equal(oracle.predict_tree(tree, x),
                                  np.array([leaf_of[i] for i in pos], np.float32))


def test_booster_reduces_logloss(oracle):
    rng = np.random.default_rng(0)
    n = 3000
    x = rng.uniform(size=(n, 4)).astype(np.float32)
    y = (rng.uniform(size=n) < 1 / (1 + np.exp(-(4 * x[:, 0] - 2 + 3 * x[:, 1] * x[:, 2])))).astype(np.float32)
    cut_ptr, cuts, _ = oracle.compute_cuts(x, 64)
    bins = oracle.bin_matrix(x, cut_ptr, cuts, -1)
    trees, margin, _ = oracle.train(bins, cut_ptr, cuts, -1, oracle.OBJ_LOGISTIC, y, 1,
                                    oracle.params(eta=0.3, max_depth=3), 10, bin_stride=64)
    p = 1 / (1 + np.exp(-margin[:, 0].astype(np.float64)))
    ll = -np.mean(y * np.log(p) + (1 - y) * np.log(1 - p))
    assert ll < 0.69 * 0.85
    walked = sum(oracle.predict_tree(t, x) for t in trees)
    np.testing.assert_allclose(walked, margin[:, 0], atol=1e-5)


def test_strided_arguments_stay_alive(oracle):
    """Arguments the binding copies to contiguous arrays (strided views) must live
    through the C call: 2M rows make the copies large enough to be returned to
    the system as soon as they are freed."""
    rng = np.random.default_rng(3)
    n, f = 2_000_000, 4
    bins = rng.integers(0, 256, (n, f), dtype=np.uint8)
    q = rng.integers(-2 ** 20, 2 ** 20, (n, 2), dtype=np.int32)
    strided = oracle.hist_parallel(bins, q[:, 0], q[:, 1], threads=2)
    ref = oracle.hist(bins, np.ascontiguousarray(q[:, 0]), np.ascontiguousarray(q[:, 1]))
    np.testing.assert_array_equal(strided, ref)
    np.testing.assert_array_equal(strided[:, :, 0].sum(axis=1),
                                  np.full(f, q[:, 0].astype(np.int64).sum()))


# ---- row and column sampling ------------------------------------------------
def test_mix64_is_splitmix64(oracle):
    """The draws' mixing function is SplitMix64's output function: seeded with 0,
    SplitMix64 (state += 0x9E3779B97F4A7C15, then the output function) yields
    0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F."""
    golden = 0x9E3779B97F4A7C15
    got = [oracle.mix64((i * golden) % 2**64) for i in range(3)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


@pytest.mark.parametrize("subsample", [0.3, 0.8])
def test_row_sampling_fraction_and_streams(oracle, subsample):
    """Kept rows are a Bernoulli(subsample) sample: the kept share is within 5 sigma of
    subsample, rounds and outputs draw independent samples (overlap ~ subsample^2), and
    subsample 1 keeps every row."""
    n = 200_000
    a = oracle.sample_rows(oracle.sampling(7, 0, 0, subsample), n)
    sigma = np.sqrt(subsample * (1 - subsample) / n)
    assert abs(a.mean() - subsample) < 5 * sigma
    for other in (oracle.sampling(7, 1, 0, subsample), oracle.sampling(7, 0, 1, subsample),
                  oracle.sampling(8, 0, 0, subsample)):
        b = oracle.sample_rows(other, n)
        assert abs((a & b).mean() - subsample ** 2) < 6 * np.sqrt(subsample ** 2 / n)
    assert oracle.sample_rows(oracle.sampling(7, 0, 0, 1.0), 1000).all()
    # the same key draws the same sample
    np.testing.assert_array_equal(a, oracle.sample_rows(oracle.sampling(7, 0, 0, subsample), n))


def test_stage_count_rule(oracle):
    """n = max(1, (int)(fraction * m)) with the product formed in float, as upstream's
    ColumnSampler computes it: 0.7 of 10 keeps 7 (0.7f * 10 rounds to 7.0f), 0.7 of 3
    keeps 2, 0.01 of 10 keeps 1, 1.0 keeps all."""
    assert oracle.stage_keep(0.7, 10) == 7
    assert oracle.stage_keep(0.7, 3) == 2
    assert oracle.stage_keep(0.01, 10) == 1
    assert oracle.stage_keep(0.5, 1000) == 500
    assert oracle.stage_keep(1.0, 37) == 37
    for m in range(1, 300):
        for frac in (0.1, 0.25, 0.3, 0.5, 0.7, 0.9):
            x = np.float32(frac) * np.float32(m)
            assert oracle.stage_keep(frac, m) == max(1, int(x))


@pytest.mark.parametrize("f", [1, 7, 28, 128, 1000])
def test_colsample_counts_and_nesting(oracle, f):
    """Each stage keeps exactly its count, chosen among the previous stage's features:
    tree set (bytree of all), level set (bylevel of the tree set, per depth) and node set
    (bynode of the level set, per node id)."""
    bt, bl, bn = 0.7, 0.6, 0.5
    tree = oracle.colsample(oracle.sampling(3, 4, 1, 1.0, bt), 0, 0, f)
    n1 = oracle.stage_keep(bt, f)
    assert tree.sum() == n1
    for depth in (0, 1, 5):
        level = oracle.colsample(oracle.sampling(3, 4, 1, 1.0, bt, bl), depth, 99, f)
        n2 = oracle.stage_keep(bl, n1)
        assert level.sum() == n2 and not (level & ~tree).any()
        for nid in (0, 3, 1000):
            node = oracle.colsample(oracle.sampling(3, 4, 1, 1.0, bt, bl, bn), depth, nid, f)
            assert node.sum() == oracle.stage_keep(bn, n2)
            assert not (node & ~level).any()


def test_colsample_is_uniform(oracle):
    """Over 4,000 node draws each of 40 features is kept with frequency n/F (chi-square,
    39 degrees of freedom, far tail), and different nodes draw different sets."""
    f, draws = 40, 4000
    counts = np.zeros(f)
    sets = set()
    for nid in range(draws):
        m = oracle.colsample(oracle.sampling(11, 2, 0, 1.0, 1.0, 1.0, 0.25), 3, nid, f)
        counts += m
        sets.add(m.tobytes())
    expected = draws * 10 / f
    chi2 = ((counts - expected) ** 2 / expected).sum()
    assert chi2 < 100  # 39 dof: P(chi2 > 100) < 1e-6
    assert len(sets) > draws * 0.99


def test_sampled_tree_matches_independent_builder(oracle):
    """A tree grown with row and column sampling equals the independent raw-row builder
    given the same dropped rows (zero gradient pairs) and, at every node, the same
    candidate features (the oracle's column sample of that node's depth and id)."""
    x, bins, cut_ptr, cuts, mb, qg, qh, eg, eh = _quantised_case(oracle, n=500, f=6, nb=8,
                                                                  seed=31)
    smp = oracle.sampling(5, 2, 1, 0.7, 0.85, 0.8, 0.5)
    keep = oracle.sample_rows(smp, bins.shape[0])
    assert 0 < keep.sum() < keep.size
    qg = np.where(keep, qg, 0).astype(np.int32)
    qh = np.where(keep, qh, 0).astype(np.int32)
    p = oracle.params(max_depth=4, eta=0.5, min_child_weight=0.0)
    tree, ridx = oracle.grow_tree(bins, cut_ptr, cuts, mb, qg, qh, eg, eh, p, bin_stride=8,
                                  smp=smp)
    ref, nodes = _reference_tree(bins, qg, qh, cut_ptr, mb, oracle.unscale(eg),
                                 oracle.unscale(eh), p,
                                 lambda depth, nid: oracle.colsample(smp, depth, nid, 6))
    assert len(ref) == len(tree["left"]) and len(ref) > 7
    used = set()
    for r in ref:
        nid = r["nid"]
        assert tree["left"][nid] == r["left"]
        if r["left"] != -1:
            assert (tree["feature"][nid], tree["split_bin"][nid], tree["default_left"][nid]) == \
                (r["feature"], r["bin"], r["dl"])
            used.add(r["feature"])
    unsampled, _ = oracle.grow_tree(bins, cut_ptr, cuts, mb, qg, qh, eg, eh, p, bin_stride=8)
    assert not (np.array_equal(unsampled["feature"], tree["feature"]) and
                np.array_equal(unsampled["left"], tree["left"])), "sampling changed nothing"


def test_booster_row_sampling_zeroes_dropped_pairs(oracle):
    """train(sample=subsample) equals train on caller gradients whose dropped rows are zero
    before the quantiser (round by round, the tree's own sample)."""
    x, bins, cut_ptr, cuts, mb, qg, qh, eg, eh = _quantised_case(oracle, n=3000, f=5, nb=16,
                                                                  seed=41)
    rng = np.random.default_rng(2)
    g = rng.normal(size=3000).astype(np.float32)
    h = rng.uniform(0.1, 0.3, size=3000).astype(np.float32)
    p = oracle.params(max_depth=4, eta=0.3)
    inj = lambda r: (np.roll(g, r)[:, None], np.roll(h, r)[:, None])  # noqa: E731
    sample = {"seed": 4, "subsample": 0.6}
    t1, m1, _ = oracle.train(bins, cut_ptr, cuts, mb, 3, None, 1, p, 3, bin_stride=16,
                             injected=inj, sample=sample)

    def masked(r):
        keep = oracle.sample_rows(oracle.sampling(4, r, 0, 0.6), 3000)
        gr, hr = inj(r)
        return np.where(keep[:, None], gr, 0).astype(np.float32), \
            np.where(keep[:, None], hr, 0).astype(np.float32)

    t2, m2, _ = oracle.train(bins, cut_ptr, cuts, mb, 3, None, 1, p, 3, bin_stride=16,
                             injected=masked)
    for a, b in zip(t1, t2):
        for key in ("left", "feature", "split_bin", "sum_qg", "sum_qh"):
            np.testing.assert_array_equal(a[key], b[key])
    np.testing.assert_array_equal(m1.view(np.uint32), m2.view(np.uint32))


def test_threads_give_identical_results(oracle):
    """The oracle's OpenMP loops (cuts, binning, histograms, split search, stable
    partition) give the serial results bit for bit: the same cuts, bins, trees and
    margins with 1 and 4 threads, on a matrix large enough to take every parallel path."""
    rng = np.random.default_rng(8)
    n, f = 120_000, 12
    x = rng.normal(size=(n, f)).astype(np.float32)
    x[rng.random((n, f)) < 0.1] = np.nan
    y = (rng.random(n) < 1 / (1 + np.exp(-x[:, 0]))).astype(np.float32)
    out = []
    try:
        for threads in (1, 4):
            oracle.set_threads(threads)
            cut_ptr, cuts, _ = oracle.compute_cuts(x, 255)
            bins = oracle.bin_matrix(x, cut_ptr, cuts, 255)
            trees, margin, _ = oracle.train(bins, cut_ptr, cuts, 255, oracle.OBJ_LOGISTIC, y, 1,
                                            oracle.params(max_depth=7, eta=0.3), 2,
                                            bin_stride=int(np.diff(cut_ptr).max()),
                                            sample={"seed": 1, "bynode": 0.7})
            out.append((cut_ptr, cuts, bins, trees, margin))
    finally:
        oracle.set_threads(1)
    (c1, v1, b1, t1, m1), (c4, v4, b4, t4, m4) = out
    np.testing.assert_array_equal(c1, c4)
    np.testing.assert_array_equal(v1.view(np.uint32), v4.view(np.uint32))
    np.testing.assert_array_equal(b1, b4)
    for a, b in zip(t1, t4):
        for key in ("left", "feature", "split_bin", "default_left", "sum_qg", "sum_qh",
                    "positions"):
            np.testing.assert_array_equal(a[key], b[key])
    np.testing.assert_array_equal(m1.view(np.uint32), m4.view(np.uint32))
