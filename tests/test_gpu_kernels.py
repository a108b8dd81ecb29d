"""GPU parity of every kernel on the path against the CPU oracle.

Each test drives one operator through the C ABI (libdpgbdt_hip.so) and the
oracle on the same seeded inputs.  The bar: bit-exact for cuts, bins, counts,
fixed-point histograms, subtraction, split records (feature, bin, default
direction, loss change, left sums) and partitions; the float histogram
equivalent is checked against float64 sums within 1e-5 relative.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _synth(ops, config, n, seed, f=None, grad=False):
    values, labels, g, h = ops.synth(config, n, seed, n_features=f, want_grad=grad)
    return values, labels, g, h


def _prepare(dp, oracle, ws, values, max_bin=256):
    """GPU cuts + bins, checked bit-exactly against the oracle's; returns both."""
    from dpgbdt import ops

    x = values.cpu().numpy()
    has_missing = bool(np.isnan(x).any())
    # the operator API's uint8 bins keep byte 255 for missing values: at most 255 bins then
    eff = min(max_bin, 255) if has_missing else min(max_bin, 256)
    cut_ptr, cuts, mins, gpu_missing = ops.sketch_cuts(ws, values, eff)
    o_ptr, o_cuts, o_mins = oracle.compute_cuts(x, eff)
    assert gpu_missing == has_missing
    np.testing.assert_array_equal(cut_ptr, o_ptr)
    np.testing.assert_array_equal(cuts.view(np.uint32), o_cuts.view(np.uint32))
    np.testing.assert_array_equal(mins.view(np.uint32), o_mins.view(np.uint32))
    missing_bin = 255 if has_missing else -1
    lay = ops.layout(x.shape[0], x.shape[1], 0, missing_bin)
    bins = ops.bin_values(values, lay, cut_ptr, cuts)
    o_bins = oracle.bin_matrix(x, o_ptr, o_cuts, missing_bin)
    np.testing.assert_array_equal(ops.from_tiles(bins.cpu().numpy(), lay), o_bins)
    n_bins = np.diff(cut_ptr).astype(np.int32)
    return lay, bins, o_bins, cut_ptr, cuts, n_bins, missing_bin


@pytest.mark.parametrize("config,n,f", [(1, 10000, 8), (3, 20000, 128), (4, 3000, 784),
                                        (5, 3000, 200), (2, 20000, 28)])
def test_cuts_and_bins_bit_exact(dp, oracle, ws, device, config, n, f):
    from dpgbdt import ops

    values, *_ = _synth(ops, config, n, 20261201 + config, f)
    _prepare(dp, oracle, ws, values)


def test_cuts_small_max_bin_and_ties(dp, oracle, ws, device):
    """Rank path with heavy ties and a tiny max_bin; distinct path for few values."""
    import torch
    from dpgbdt import ops

    rng = np.random.default_rng(7)
    x = np.stack([rng.integers(0, 40, 5000).astype(np.float32),
                  rng.normal(size=5000).astype(np.float32),
                  np.where(rng.random(5000) < 0.5, np.float32(0.0), np.float32(-0.0)),
                  np.full(5000, np.nan, dtype=np.float32)], axis=1)
    x[::7, 1] = np.nan
    values = torch.as_tensor(x, device=device)
    _prepare(dp, oracle, ws, values, max_bin=16)


@pytest.mark.parametrize("objective,k", [(0, 1), (1, 10), (2, 1)])
def test_gradients_bit_exact(dp, oracle, device, objective, k):
    import torch
    from dpgbdt import ops

    rng = np.random.default_rng(11 + objective)
    n = 50000
    margin = (rng.normal(size=(n, k)) * 4).astype(np.float32)
    margin[:7, 0] = [0.0, 90.0, -90.0, 88.0, -87.5, 1e-30, -1e-30]
    if objective == 1:
        label = rng.integers(0, k, n).astype(np.float32)
    elif objective == 0:
        label = rng.integers(0, 2, n).astype(np.float32)
    else:
        label = rng.normal(size=n).astype(np.float32)
    g, h = ops.objective_gradients(objective, torch.as_tensor(margin, device=device),
                                   torch.as_tensor(label, device=device), k)
    og, oh = oracle.gradients(objective, margin if k > 1 else margin[:, 0], label, k)
    np.testing.assert_array_equal(g.cpu().numpy().view(np.uint32), og.view(np.uint32))
    np.testing.assert_array_equal(h.cpu().numpy().view(np.uint32), oh.view(np.uint32))


def test_quantise_bit_exact(dp, oracle, ws, device):
    import torch
    from dpgbdt import ops

    rng = np.random.default_rng(3)
    n, k = 40000, 3
    g = rng.normal(size=(n, k)).astype(np.float32)
    h = rng.uniform(0.01, 0.25, size=(n, k)).astype(np.float32)
    g[:, 2] *= 1e-20  # tiny scale still quantises to full precision
    exps, gpair, sums = ops.quantise(ws, torch.as_tensor(g, device=device),
                                     torch.as_tensor(h, device=device))
    exps, gpair, sums = exps.cpu().numpy(), gpair.cpu().numpy(), sums.cpu().numpy()
    for c, (eg, eh, qg, qh) in enumerate(oracle.quantise(g, h)):
        assert (exps[c, 0], exps[c, 1]) == (eg, eh)
        np.testing.assert_array_equal(gpair[c, :, 0], qg)
        np.testing.assert_array_equal(gpair[c, :, 1], qh)
        assert sums[c, 0] == qg.astype(np.int64).sum() and sums[c, 1] == qh.astype(np.int64).sum()
        assert np.abs(qg).max() <= 2 ** 30 and np.abs(qh).max() <= 2 ** 30


def _check_float_sums(oracle, hist, o_bins, gn, hn, eg, eh, missing_bin, features):
    """The histogram's sums as floats (the fixed-point sums times 2^-exp) against the float64
    sums of the raw float32 gradients, for g and for h, per (feature, bin): within 1e-5
    relative wherever the bin's |sum| is at least 1e-3 of its sum of magnitudes, and within
    1e-5 of that sum of magnitudes in the cancelling bins (where a relative bound on a sum
    near zero means nothing).  The quantiser's step is 2^-30 of max|x| per item, so the
    bound holds with a margin of about 20x on these inputs."""
    stride = hist.shape[1]
    checked = 0
    for c, (x, e) in enumerate(((gn, eg), (hn, eh))):
        got = hist[..., c] * oracle.unscale(e)
        for feat in features:
            col = o_bins[:, feat]
            keep = col != missing_bin if missing_bin >= 0 else slice(None)
            cb, xv = col[keep], x[keep].astype(np.float64)
            exact = np.bincount(cb, weights=xv, minlength=stride)[:stride]
            mass = np.bincount(cb, weights=np.abs(xv), minlength=stride)[:stride]
            err = np.abs(got[feat] - exact)
            live = np.abs(exact) >= 1e-3 * mass
            bad = live & (err > 1e-5 * np.abs(exact))
            assert not bad.any(), (c, feat, np.nonzero(bad)[0][:5], err[bad][:5], exact[bad][:5])
            assert np.all(err[~live] <= 1e-5 * mass[~live]), (c, feat)
            checked += int(live.sum())
    return checked


def _gpair(ws, device, g, h):
    import torch
    from dpgbdt import ops

    exps, gpair, sums = ops.quantise(ws, torch.as_tensor(g, device=device),
                                     torch.as_tensor(h, device=device))
    return exps.cpu().numpy()[0], gpair[0].contiguous(), sums.cpu().numpy()[0]


@pytest.mark.parametrize("config,n,f", [(1, 10000, 8), (3, 60000, 128), (5, 20000, 300),
                                        (4, 4000, 784)])
def test_root_histogram_bit_exact(dp, oracle, ws, device, config, n, f):
    import torch
    from dpgbdt import ops

    values, _, g, h = _synth(ops, config, n, 99 + config, f, grad=True)
    lay, bins, o_bins, cut_ptr, cuts, n_bins, mb = _prepare(dp, oracle, ws, values)
    stride = int(n_bins.max())
    gn, hn = g.cpu().numpy(), h.cpu().numpy()
    (eg, eh), gpair, _ = _gpair(ws, device, gn, hn)
    hist = ops.hist_build(ws, bins, lay, gpair, [(0, n)], stride).cpu().numpy()[0]
    q = oracle.quantise(gn, hn)[0]
    ref = oracle.hist(o_bins, q[2], q[3], bin_stride=stride, missing_bin=mb)
    np.testing.assert_array_equal(hist, ref)
    # counts: the same kernel with unit gradients equals np.bincount
    ones = torch.ones((n, 2), dtype=torch.int32, device=device)
    counts = ops.hist_build(ws, bins, lay, ones, [(0, n)], stride).cpu().numpy()[0]
    for feat in range(0, f, max(1, f // 16)):
        col = o_bins[:, feat]
        col = col[col != 255] if mb == 255 else col
        np.testing.assert_array_equal(counts[feat, :, 0], np.bincount(col, minlength=stride)[:stride])
    # g and h sums as floats within 1e-5 relative of the float64 sums of the raw gradients
    assert _check_float_sums(oracle, hist, o_bins, gn, hn, eg, eh, mb, range(f)) > 0


def test_c3_root_histogram_full_size(dp, oracle, ws, device):
    """The benchmark's C3 root pass at its size (10,000,000 x 128, 256 bins): the
    device bins (whose cuts and binning the tests above pin against the oracle
    at smaller sizes) are read back and histogrammed by the oracle's parallel
    histogram; the GPU histogram, with and without paired tiles, must equal it
    bit for bit, and every feature's sums must equal the sums of the quantised
    gradients (no row lost or counted twice)."""
    from dpgbdt import ops

    n, f = 10_000_000, 128
    print(f"[kernels] C3 root histogram {n} x {f}", flush=True)
    values, _, g, h = _synth(ops, 3, n, 20261201 + 3, f, grad=True)
    cut_ptr, cuts, _, missing = ops.sketch_cuts(ws, values, 256)
    assert not missing
    lay = ops.layout(n, f, 0, -1)
    # features 96-127 take 16 values: tiles 6 and 7 pair, as in the benchmark's pass
    # (the bins buffer: the 8 tiles, then the pair's joint tile)
    paired = ops.layout_pair_tiles(ops.layout(n, f, 0, -1), cut_ptr)
    assert paired.paired_tiles == 1 << 6
    bins = ops.bin_values(values, paired, cut_ptr, cuts)
    del values
    stride = int(np.diff(cut_ptr).max())
    (eg, eh), gpair, sums = _gpair(ws, device, g.cpu().numpy(), h.cpu().numpy())
    hist = ops.hist_build(ws, bins, lay, gpair, [(0, n)], stride).cpu().numpy()[0]
    qgqh = gpair.cpu().numpy()
    np.testing.assert_array_equal(hist[:, :, 0].sum(axis=1), np.full(f, sums[0]))
    np.testing.assert_array_equal(hist[:, :, 1].sum(axis=1), np.full(f, sums[1]))
    hist_paired = ops.hist_build(ws, bins, paired, gpair, [(0, n)], stride).cpu().numpy()[0]
    host_bins = ops.from_tiles(bins[: ops.layout_bytes(lay)].cpu().numpy(), lay)
    del bins
    ref = oracle.hist_parallel(host_bins, qgqh[:, 0], qgqh[:, 1], bin_stride=stride)
    np.testing.assert_array_equal(hist, ref)
    np.testing.assert_array_equal(hist_paired, ref)
    # every feature's g and h sums as floats, within 1e-5 relative of float64 sums
    live = _check_float_sums(oracle, hist, host_bins, g.cpu().numpy(), h.cpu().numpy(), eg, eh,
                             -1, range(f))
    print(f"[kernels] C3 float sums: {live} (feature, bin, g|h) sums within 1e-5 relative",
          flush=True)


def test_c5_float_sums(dp, oracle, ws, device):
    """C5's shape at 200,000 x 1,000 (95 % missing, 64 bins plus the missing byte): the root
    histogram's g and h sums as floats, for every feature, within 1e-5 relative of the float64
    sums of the raw gradients over the present values (bit-exact fixed point against the
    oracle first)."""
    from dpgbdt import ops

    n, f = 200_000, 1000
    print(f"[kernels] C5 float sums {n} x {f}", flush=True)
    values, _, g, h = _synth(ops, 5, n, 20261201 + 5, f, grad=True)
    lay, bins, o_bins, cut_ptr, cuts, n_bins, mb = _prepare(dp, oracle, ws, values, 64)
    assert mb == 255
    stride = int(n_bins.max())
    gn, hn = g.cpu().numpy(), h.cpu().numpy()
    (eg, eh), gpair, _ = _gpair(ws, device, gn, hn)
    hist = ops.hist_build(ws, bins, lay, gpair, [(0, n)], stride).cpu().numpy()[0]
    q = oracle.quantise(gn, hn)[0]
    np.testing.assert_array_equal(hist, oracle.hist(o_bins, q[2], q[3], bin_stride=stride,
                                                    missing_bin=mb))
    live = _check_float_sums(oracle, hist, o_bins, gn, hn, eg, eh, mb, range(f))
    print(f"[kernels] C5 float sums: {live} (feature, bin, g|h) sums within 1e-5 relative",
          flush=True)


@pytest.mark.parametrize("max_bin", [64, 128])
def test_sparse_histograms_bit_exact(dp, oracle, ws, device, max_bin):
    """Missing values with at most 128 bins take the compacting kernel (present
    entries queued per wavefront, then full-wave atomics): contiguous and
    gathered rows, against the oracle and against np.bincount counts."""
    import torch
    from dpgbdt import ops

    n, f = 30000, 200
    values, _, g, h = _synth(ops, 5, n, 41 + max_bin, f, grad=True)
    lay, bins, o_bins, cut_ptr, cuts, n_bins, mb = _prepare(dp, oracle, ws, values, max_bin)
    assert mb == 255
    stride = int(n_bins.max())
    assert stride <= 128
    gn, hn = g.cpu().numpy(), h.cpu().numpy()
    _, gpair, _ = _gpair(ws, device, gn, hn)
    q = oracle.quantise(gn, hn)[0]
    root = ops.hist_build(ws, bins, lay, gpair, [(0, n)], stride).cpu().numpy()[0]
    np.testing.assert_array_equal(root, oracle.hist(o_bins, q[2], q[3], bin_stride=stride,
                                                    missing_bin=mb))
    rng = np.random.default_rng(3)
    ridx = rng.permutation(n).astype(np.uint32)
    segs = [(0, 1), (1, 333), (333, 9000), (9000, n)]
    hist = ops.hist_build(ws, bins, lay, gpair, segs, stride,
                          ridx=torch.as_tensor(ridx.view(np.int32), device=device)).cpu().numpy()
    for i, (b, e) in enumerate(segs):
        ref = oracle.hist(o_bins, q[2], q[3], rows=ridx[b:e], bin_stride=stride, missing_bin=mb)
        np.testing.assert_array_equal(hist[i], ref, err_msg=f"segment {i}")
    ones = torch.ones((n, 2), dtype=torch.int32, device=device)
    counts = ops.hist_build(ws, bins, lay, ones, [(0, n)], stride).cpu().numpy()[0]
    for feat in range(0, f, 13):
        col = o_bins[:, feat]
        np.testing.assert_array_equal(counts[feat, :, 0],
                                      np.bincount(col[col != 255], minlength=stride)[:stride])


def test_gathered_histograms_and_subtraction(dp, oracle, ws, device):
    import torch
    from dpgbdt import ops

    n, f = 50000, 128
    values, _, g, h = _synth(ops, 3, n, 5, f, grad=True)
    lay, bins, o_bins, cut_ptr, cuts, n_bins, mb = _prepare(dp, oracle, ws, values)
    stride = int(n_bins.max())
    gn, hn = g.cpu().numpy(), h.cpu().numpy()
    _, gpair, _ = _gpair(ws, device, gn, hn)
    q = oracle.quantise(gn, hn)[0]
    rng = np.random.default_rng(1)
    ridx = rng.permutation(n).astype(np.uint32)
    segs = [(0, 1), (1, 700), (700, 20000), (20000, 20000), (20000, n)]
    d_ridx = torch.as_tensor(ridx.view(np.int32), device=device)
    hist = ops.hist_build(ws, bins, lay, gpair, segs, stride, ridx=d_ridx)
    hn_ = hist.cpu().numpy()
    for i, (b, e) in enumerate(segs):
        ref = oracle.hist(o_bins, q[2], q[3], rows=ridx[b:e], bin_stride=stride, missing_bin=mb)
        np.testing.assert_array_equal(hn_[i], ref)
    parent = ops.hist_build(ws, bins, lay, gpair, [(0, n)], stride)
    sib = ops.hist_subtract(parent[0], hist[2] + hist[0] + hist[1] + hist[3])
    np.testing.assert_array_equal(sib.cpu().numpy(), hn_[4])


def test_workspace_staging_reuse(dp, oracle, ws, device):
    """A workspace skips re-uploading work lists identical to its last upload: calls with
    lists A, A (no upload), B, A (uploads again), and accumulating calls on A, each give the
    oracle's histograms."""
    import torch
    from dpgbdt import ops

    n, f = 30000, 40
    values, _, g, h = _synth(ops, 1, n, 9, f, grad=True)
    lay, bins, o_bins, cut_ptr, cuts, n_bins, mb = _prepare(dp, oracle, ws, values)
    stride = int(n_bins.max())
    gn, hn = g.cpu().numpy(), h.cpu().numpy()
    _, gpair, _ = _gpair(ws, device, gn, hn)
    q = oracle.quantise(gn, hn)[0]
    ridx = np.random.default_rng(4).permutation(n).astype(np.uint32)
    d_ridx = torch.as_tensor(ridx.view(np.int32), device=device)
    lists = {"A": [(0, 9000), (9000, 30000)], "B": [(0, 17), (17, 25000), (25000, 30000)]}
    refs = {k: [oracle.hist(o_bins, q[2], q[3], rows=ridx[b:e], bin_stride=stride, missing_bin=mb)
                for b, e in segs] for k, segs in lists.items()}
    for name in ("A", "A", "B", "A"):
        got = ops.hist_build(ws, bins, lay, gpair, lists[name], stride, ridx=d_ridx).cpu().numpy()
        for i, ref in enumerate(refs[name]):
            np.testing.assert_array_equal(got[i], ref, err_msg=f"list {name}, segment {i}")
    acc = torch.zeros((2, f, stride, 2), dtype=torch.int64, device=device)
    for _ in range(3):
        ops.hist_accumulate(ws, bins, lay, gpair, lists["A"], acc, ridx=d_ridx)
    got = acc.cpu().numpy()
    for i, ref in enumerate(refs["A"]):
        np.testing.assert_array_equal(got[i], 3 * ref)


# 128 features: feature-parallel items (256 bins: one feature per wavefront),
# then a select kernel; up to 64 bins: four features per wavefront (40 features:
# the last group holds unused rows); 8 features: one workgroup per node.
@pytest.mark.parametrize("config,f,max_bin", [(3, 128, 256), (1, 8, 256), (5, 300, 64),
                                              (5, 40, 64)])
def test_split_evaluation_bit_exact(dp, oracle, ws, device, config, f, max_bin):
    import torch
    from dpgbdt import ops

    n = 30000
    values, _, g, h = _synth(ops, config, n, 17, f, grad=True)
    lay, bins, o_bins, cut_ptr, cuts, n_bins, mb = _prepare(dp, oracle, ws, values, max_bin)
    stride = int(n_bins.max())
    gn, hn = g.cpu().numpy(), h.cpu().numpy()
    (eg, eh), gpair, sums = _gpair(ws, device, gn, hn)
    q = oracle.quantise(gn, hn)[0]
    rng = np.random.default_rng(2)
    ridx = rng.permutation(n).astype(np.uint32)
    segs = [(0, n // 2), (n // 2, n // 2 + 40), (n // 2 + 40, n)]
    hist = ops.hist_build(ws, bins, lay, gpair, segs, stride,
                          ridx=torch.as_tensor(ridx.view(np.int32), device=device))
    node_sums = []
    for b, e in segs:
        rows = ridx[b:e]
        node_sums.append((q[2][rows].astype(np.int64).sum(), q[3][rows].astype(np.int64).sum()))
    d_sums = torch.as_tensor(np.array(node_sums, dtype=np.int64), device=device)
    d_nbins = torch.as_tensor(n_bins, device=device)
    for prm in [dict(), dict(lam=0.0, alpha=0.5, gamma=1.0, min_child_weight=3.0)]:
        rec = ops.splits_to_numpy(ops.evaluate_splits(ws, hist, d_nbins, d_sums, eg, eh,
                                                          ops.train_param(**prm)))
        p = oracle.params(**prm)
        for i in range(len(segs)):
            o = oracle.evaluate_split(hist[i].cpu().numpy(), n_bins, node_sums[i][0],
                                      node_sums[i][1], eg, eh, p)
            assert rec[i]["valid"] == o["valid"]
            assert (rec[i]["feature"], rec[i]["bin"], rec[i]["default_left"]) == \
                (o["feature"], o["bin"], o["default_left"])
            assert np.float64(rec[i]["loss_chg"]).tobytes() == np.float64(o["loss_chg"]).tobytes()
            assert (rec[i]["gl"], rec[i]["hl"]) == (o["gl"], o["hl"])


def test_random_operator_calls_match_the_oracle(dp, oracle, ws, device):
    """Forty seeded random inputs through the C ABI, one operator after another, each against
    the oracle: cuts and bins (mixed value kinds, missing values, 2-256 bins), the quantiser,
    histograms of random row sets (contiguous or gathered, empty sets included),
    accumulation, subtraction, split evaluation under random regularisation, and the
    partition of every row set by its own chosen split."""
    import torch
    from dpgbdt import ops

    rng = np.random.default_rng(20261203)
    for t in range(40):
        n = int(rng.choice([1, 5, 100, 3000, 20000, 70000]))
        f = int(rng.choice([1, 3, 16, 17, 40, 130]))
        max_bin = int(rng.choice([2, 16, 64, 200, 256]))
        missing = float(rng.choice([0.0, 0.0, 0.3]))
        gather = bool(rng.integers(0, 2))
        print(f"[kernels] random call {t}: {n} x {f}, max_bin {max_bin}, missing {missing}, "
              f"gather {gather}", flush=True)
        x = np.empty((n, f), dtype=np.float32)
        for j in range(f):
            if rng.random() < 0.5:
                x[:, j] = rng.normal(size=n)
            else:
                x[:, j] = rng.integers(0, int(rng.integers(1, 30)), size=n)
        if missing > 0:
            x[rng.random((n, f)) < missing] = np.nan
        values = torch.as_tensor(x, device=device)
        lay, bins, o_bins, cut_ptr, cuts, n_bins, mb = _prepare(dp, oracle, ws, values, max_bin)
        stride = max(1, int(n_bins.max()))
        g = (rng.normal(size=n) * rng.choice([1e-4, 1.0, 1e4])).astype(np.float32)
        h = (rng.random(size=n) * rng.choice([1e-3, 1.0, 50.0])).astype(np.float32)
        (eg, eh), gpair, _ = _gpair(ws, device, g, h)
        q = oracle.quantise(g, h)[0]
        assert (eg, eh) == (q[0], q[1])
        gp = gpair.cpu().numpy().reshape(n, 2)
        np.testing.assert_array_equal(gp[:, 0], q[2])
        np.testing.assert_array_equal(gp[:, 1], q[3])
        ridx = rng.permutation(n).astype(np.uint32) if gather else np.arange(n, dtype=np.uint32)
        d_ridx = torch.as_tensor(ridx.view(np.int32), device=device)
        bounds = [0, *sorted(int(v) for v in rng.integers(0, n + 1, size=int(rng.integers(1, 6)))), n]
        segs = [(bounds[i], bounds[i + 1]) for i in range(len(bounds) - 1)]
        hist = ops.hist_build(ws, bins, lay, gpair, segs, stride, ridx=d_ridx if gather else None)
        hn_ = hist.cpu().numpy()
        refs = [oracle.hist(o_bins, q[2], q[3], rows=ridx[b:e], bin_stride=stride, missing_bin=mb)
                for b, e in segs]
        for i in range(len(segs)):
            np.testing.assert_array_equal(hn_[i], refs[i], err_msg=f"histogram {i} of {segs}")
        twice = ops.hist_accumulate(ws, bins, lay, gpair, segs, hist.clone(),
                                    ridx=d_ridx if gather else None)
        np.testing.assert_array_equal(twice.cpu().numpy(), 2 * hn_)
        parent = ops.hist_build(ws, bins, lay, gpair, [(0, n)], stride)
        rest = oracle.hist(o_bins, q[2], q[3], rows=ridx[segs[0][1]:], bin_stride=stride,
                           missing_bin=mb)
        np.testing.assert_array_equal(ops.hist_subtract(parent[0], hist[0]).cpu().numpy(), rest)
        sums = [(int(q[2][ridx[b:e]].astype(np.int64).sum()),
                 int(q[3][ridx[b:e]].astype(np.int64).sum())) for b, e in segs]
        prm = {"lam": float(rng.choice([0.0, 1.0, 3.0])), "alpha": float(rng.choice([0.0, 0.3])),
               "gamma": float(rng.choice([0.0, 0.5])),
               "min_child_weight": float(rng.choice([0.0, 1.0, 5.0]))}
        d_rec = ops.evaluate_splits(ws, hist, torch.as_tensor(n_bins, device=device),
                                    torch.as_tensor(np.array(sums, dtype=np.int64), device=device),
                                    eg, eh, ops.train_param(**prm))
        rec = ops.splits_to_numpy(d_rec)
        p = oracle.params(**prm)
        for i in range(len(segs)):
            o = oracle.evaluate_split(refs[i], n_bins, sums[i][0], sums[i][1], eg, eh, p)
            assert rec[i]["valid"] == o["valid"], f"split {i}"
            if not o["valid"]:
                continue
            assert (rec[i]["feature"], rec[i]["bin"], rec[i]["default_left"]) == \
                (o["feature"], o["bin"], o["default_left"]), f"split {i}"
            assert np.float64(rec[i]["loss_chg"]).tobytes() == np.float64(o["loss_chg"]).tobytes()
            assert (rec[i]["gl"], rec[i]["hl"]) == (o["gl"], o["hl"])
        out, left = ops.partition(ws, bins, lay, d_ridx, segs, d_rec)
        out, left = out.cpu().numpy().view(np.uint32), left.cpu().numpy()
        for i, (b, e) in enumerate(segs):
            if not rec[i]["expand"]:
                assert left[i] == 0
                continue
            part, nl = oracle.partition(ridx, b, e, o_bins, int(rec[i]["feature"]),
                                        int(rec[i]["bin"]), int(rec[i]["default_left"]), mb)
            assert left[i] == nl, f"partition {i}"
            np.testing.assert_array_equal(out[b:e], part[b:e], err_msg=f"partition {i}")


# 4,300,000 rows: matrices of 4M rows or more take the partition kernels that
# load four 256-row steps per group (one step per group below).
@pytest.mark.parametrize("n,f", [(30000, 200), (4_300_000, 24)])
def test_partition_bit_exact(dp, oracle, ws, device, n, f):
    import torch
    from dpgbdt import ops

    print(f"[kernels] partition {n} x {f}", flush=True)
    values, *_ = _synth(ops, 5, n, 23, f)
    lay, bins, o_bins, *_ , mb = _prepare(dp, oracle, ws, values)
    rng = np.random.default_rng(4)
    ridx = rng.permutation(n).astype(np.uint32)
    cut = n // 3
    segs = [(0, cut), (cut, cut + 1), (cut + 1, n - 5000), (n - 5000, n)]
    rec = np.zeros(len(segs), dtype=ops.SPLIT_DTYPE)
    choices = [(3, 10, 1, 1), (5, 0, 0, 1), (17, 30, 0, 0), (f - 1, 5, 1, 1)]
    for i, (feat, b, dl, ex) in enumerate(choices):
        rec[i]["feature"], rec[i]["bin"], rec[i]["default_left"], rec[i]["expand"] = feat, b, dl, ex
        rec[i]["valid"] = 1
    d_rec = torch.as_tensor(np.frombuffer(rec.tobytes(), dtype=np.uint8).copy(), device=device)
    d_ridx = torch.as_tensor(ridx.view(np.int32), device=device)
    out, left = ops.partition(ws, bins, lay, d_ridx, segs, d_rec)
    out = out.cpu().numpy().view(np.uint32)
    left = left.cpu().numpy()
    expect = ridx.copy()
    for i, ((b, e), (feat, sb, dl, ex)) in enumerate(zip(segs, choices)):
        if not ex:
            assert left[i] == 0
            continue
        part, nl = oracle.partition(ridx, b, e, o_bins, feat, sb, dl, mb)
        expect[b:e] = part[b:e]
        assert left[i] == nl
    for (b, e), (*_, ex) in zip(segs, choices):
        if ex:
            np.testing.assert_array_equal(out[b:e], expect[b:e])


def test_update_margin(dp, ws, device):
    import torch
    from dpgbdt import ops

    n = 70000
    rng = np.random.default_rng(6)
    ridx = rng.permutation(n).astype(np.uint32)
    segs = [(0, 30000), (30000, 30001), (30001, n)]
    vals = [0.25, -1.5, 3.0]
    margin = torch.zeros(n * 2, dtype=torch.float32, device=device)
    ops.update_margin(ws, torch.as_tensor(ridx.view(np.int32), device=device), segs, vals,
                      margin[1:], stride=2)
    m = margin.cpu().numpy().reshape(n, 2)
    expect = np.zeros(n, np.float32)
    for (b, e), v in zip(segs, vals):
        expect[ridx[b:e]] += np.float32(v)
    np.testing.assert_array_equal(m[:, 1], expect)
    assert not m[:, 0].any()
