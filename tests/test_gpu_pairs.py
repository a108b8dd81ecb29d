"""Paired tiles on the GPU: two 16-feature tiles whose features all have at most 16
bins are histogrammed as one tile of joint bytes (tile t's bin * 16 + tile t + 1's,
the pair's joint tile after the matrix's tiles) and split back into both tiles'
histograms when the item is stored.  The joint tiles must hold exactly those bytes
(dp_join_tiles, and dp_bin_values for a paired layout), and every result
must equal the unpaired build and the oracle's histogram bit for bit: direct
single-chunk stores, partial slots (LDS image and the booster's feature-major
slots), accumulation, gathered rows, bin strides above, at and below 16, and a
paired last tile with pad features; and trees trained with and without pairing
are identical."""
import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _matrix(rng, n, n_bins):
    """Row-major uint8 bins with n_bins[f] bins per feature (every bin used when n
    allows), and the cut_ptr those bin counts give."""
    cols = [rng.integers(0, b, size=n, dtype=np.int64) for b in n_bins]
    bins = np.stack(cols, axis=1).astype(np.uint8)
    ptr = np.concatenate([[0], np.cumsum(n_bins)]).astype(np.int32)
    return np.ascontiguousarray(bins), ptr


def _gpair(rng, n):
    g = rng.integers(-(1 << 30), 1 << 30, size=n, dtype=np.int64).astype(np.int32)
    h = rng.integers(0, 1 << 30, size=n, dtype=np.int64).astype(np.int32)
    return g, h


@pytest.mark.parametrize("case", ["wide", "sixteen", "twelve"])
def test_paired_histograms_bit_exact(dp, oracle, ws, device, case):
    import torch
    from dpgbdt import ops

    rng = np.random.default_rng({"wide": 1, "sixteen": 2, "twelve": 3}[case])
    n = 100_000
    if case == "wide":  # tiles: (0, 1) paired, 2 alone, 3 wide, (4, 5) paired with 6 pads
        f = 90
        n_bins = rng.integers(2, 17, size=f)
        n_bins[[0, 16, 40, 72]] = 16
        n_bins[48:64] = 256
        n_bins[55] = 200
        expect = (1 << 0) | (1 << 4)
    elif case == "sixteen":  # every feature 16 bins: (0, 1), 2 alone; stride 16
        f = 40
        n_bins = np.full(f, 16)
        expect = 1 << 0
    else:  # at most 12 bins: stride 12, below the joint byte's 16
        f = 64
        n_bins = rng.integers(1, 13, size=f)
        n_bins[3] = 12
        expect = (1 << 0) | (1 << 2)
    bins, ptr = _matrix(rng, n, n_bins)
    stride = int(n_bins.max())
    print(f"[pairs] {case}: {n} x {f}, stride {stride}", flush=True)
    plain = ops.layout(n, f, 0, -1)
    paired = ops.layout_pair_tiles(ops.layout(n, f, 0, -1), ptr)
    assert paired.paired_tiles == expect
    d_bins = torch.zeros(ops.layout_bytes(paired), dtype=torch.uint8, device=device)
    d_bins[: ops.layout_bytes(plain)] = torch.as_tensor(ops.to_tiles(bins, plain), device=device)
    ops.join_tiles(d_bins, paired)
    # joint tile k of pair (t, t + 1): (tile t's byte << 4) | tile t + 1's byte
    tiles = ops.to_tiles(bins, plain).reshape(plain.n_tiles, n, 16)
    joint = d_bins[ops.layout_bytes(plain):].cpu().numpy().reshape(-1, n, 16)
    firsts = [t for t in range(64) if (expect >> t) & 1]
    assert joint.shape[0] == len(firsts)
    for k, t in enumerate(firsts):
        np.testing.assert_array_equal(joint[k], (tiles[t] << 4) | tiles[t + 1])
    g, h = _gpair(rng, n)
    gp = torch.as_tensor(np.stack([g, h], axis=1), device=device).contiguous()
    ridx = rng.permutation(n).astype(np.uint32)
    d_ridx = torch.as_tensor(ridx.view(np.int32), device=device)
    segs = [(0, n)]
    multi = [(0, 1), (1, 700), (700, 40_000), (40_000, 40_000), (40_000, n)]
    for name, s, r in (("root", segs, None), ("nodes", multi, None),
                       ("gathered", multi, d_ridx)):
        got = ops.hist_build(ws, d_bins, paired, gp, s, stride, ridx=r).cpu().numpy()
        ref = ops.hist_build(ws, d_bins, plain, gp, s, stride, ridx=r).cpu().numpy()
        np.testing.assert_array_equal(got, ref, err_msg=name)
        for i, (b, e) in enumerate(s):
            rows = None if r is None else ridx[b:e]
            if r is None:
                rows = np.arange(b, e, dtype=np.uint32)
            want = oracle.hist(bins, g, h, rows=rows, bin_stride=stride)
            np.testing.assert_array_equal(got[i], want, err_msg=f"{name} segment {i}")
    # accumulation (every chunk through an LDS-image partial slot), twice
    acc = torch.zeros((len(multi), f, stride, 2), dtype=torch.int64, device=device)
    ops.hist_accumulate(ws, d_bins, paired, gp, multi, acc)
    ops.hist_accumulate(ws, d_bins, paired, gp, multi, acc)
    once = ops.hist_build(ws, d_bins, plain, gp, multi, stride)
    np.testing.assert_array_equal(acc.cpu().numpy(), 2 * once.cpu().numpy())


def test_paired_tiles_refused_with_missing_values(dp, ws, device):
    """The kernel's pairs need bins below 16 in both tiles: a layout that claims pairs on a
    matrix with missing values (byte 255) is refused before any launch."""
    import torch
    from dpgbdt import ops

    n, f = 5000, 32
    lay = ops.layout(n, f, 0, 255)
    lay.paired_tiles = 1
    bins = torch.zeros(ops.layout_bytes(lay), dtype=torch.uint8, device=device)
    gp = torch.zeros((n, 2), dtype=torch.int32, device=device)
    with pytest.raises(dp.DPError, match="paired tiles need a matrix without missing values"):
        ops.hist_build(ws, bins, lay, gp, [(0, n)], 16)
    lay = ops.layout(n, f, 0, -1)
    lay.paired_tiles = 2  # tile 1 with a tile 2 the matrix does not have
    with pytest.raises(dp.DPError, match="paired tile beyond the matrix"):
        ops.hist_build(ws, bins, lay, gp, [(0, n)], 16)


def test_paired_layout_refuses_a_buffer_sized_before_pairing(dp, ws, device):
    """dp_layout_bytes counts a paired layout's joint tiles; a bins buffer sized for the
    unpaired layout (a dedicated 32 MiB allocation, 16 MiB short of the paired size) is
    refused before any launch by the histogram, binning and joining calls."""
    import ctypes

    import torch
    from dpgbdt import ops

    n, f = 1 << 20, 32
    plain = ops.layout(n, f, 0, -1)
    paired = ops.layout_pair_tiles(ops.layout(n, f, 0, -1), np.arange(0, 16 * f + 1, 16))
    assert paired.paired_tiles == 1
    assert ops.layout_bytes(paired) == ops.layout_bytes(plain) + n * 16
    rt = ctypes.CDLL("libamdhip64.so.7")
    rt.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    rt.hipFree.argtypes = [ctypes.c_void_p]
    buf = ctypes.c_void_p()
    assert rt.hipMalloc(ctypes.byref(buf), ops.layout_bytes(plain)) == 0
    try:
        lib = dp.load()
        gp = torch.zeros((n, 2), dtype=torch.int32, device=device)
        hist = torch.zeros((1, f, 16, 2), dtype=torch.int64, device=device)
        begin, end = np.array([0], dtype=np.int64), np.array([n], dtype=np.int64)
        rc = lib.dp_hist_build(ws.handle, buf, ctypes.byref(paired), gp.data_ptr(), None,
                               begin.ctypes.data, end.ctypes.data, 1, 16, hist.data_ptr(), None)
        assert rc == -1 and "pair the layout before sizing" in lib.XGBGetLastError().decode()
        rc = lib.dp_join_tiles(buf, ctypes.byref(paired), None)
        assert rc == -1 and "pair the layout before sizing" in lib.XGBGetLastError().decode()
        torch.cuda.synchronize()
    finally:
        rt.hipFree(buf)


def _train(dp, values, labels, pair, rounds, extra=None):
    dtrain = dp.DMatrix(values, labels)
    params = {"objective": "binary:logistic", "max_depth": 8, "eta": 0.1, "max_bin": 256,
              "dp_hist_pair": pair}
    params.update(extra or {})
    bst = dp.Booster(params, [dtrain])
    for r in range(rounds):
        bst.update(dtrain, r)
    return bst


@pytest.mark.parametrize("extra", [None, {"dp_hist_items": 512, "dp_hist_tiles": 1,
                                          "dp_hist_unroll": 1, "dp_hist_deep": 1}])
def test_trees_identical_with_and_without_pairs(dp, device, extra):
    """C3's layout (features 96-127 take 16 values: tiles 6 and 7 pair) at 200,000 rows:
    the booster's root pass (feature-major partial slots, reduced and evaluated in one
    launch) and its gathered levels with pairs give the trees of the unpaired build."""
    from dpgbdt import ops

    n, f = 200_000, 128
    print(f"[pairs] C3 trees {n} x {f}, {extra}", flush=True)
    values, labels, _, _ = ops.synth(3, n, 20261202, device=device)
    with_pairs = _train(dp, values, labels, 1, 3, extra)
    assert with_pairs.tuning()["paired_tiles"] == 1 << 6
    without = _train(dp, values, labels, 0, 3, extra)
    assert without.tuning()["paired_tiles"] == 0
    a = json.loads(with_pairs.save_raw())
    b = json.loads(without.save_raw())
    assert a["learner"]["gradient_booster"] == b["learner"]["gradient_booster"]


def test_multiclass_sampled_trees_identical_with_and_without_pairs(dp, device):
    """Softprob over 3 classes (three trees per round on concurrent streams, each with its
    own grower and the shared row-major copy) with row and column sampling, on 50,000 rows:
    tiles 0 and 1 take 16 values and pair, tile 2 has 256 bins.  The saved models with and
    without pairs are identical."""
    import torch

    g = torch.Generator(device="cpu").manual_seed(11)
    n = 50000
    narrow = torch.randint(0, 16, (n, 32), generator=g).to(torch.float32)
    wide = torch.randn((n, 16), generator=g)
    values = torch.cat([narrow, wide], dim=1).contiguous().to(device)
    score = torch.stack([values[:, 3] - 7.5, values[:, 20] - 7.5, 4 * values[:, 40]], dim=1)
    labels = (score + torch.randn((n, 3), generator=g).to(device)).argmax(dim=1)
    labels = labels.to(torch.float32).contiguous()
    extra = {"objective": "multi:softprob", "num_class": 3, "max_depth": 6, "subsample": 0.8,
             "colsample_bynode": 0.5, "seed": 5}
    with_pairs = _train(dp, values, labels, 1, 3, extra)
    assert with_pairs.tuning()["paired_tiles"] == 1
    without = _train(dp, values, labels, 0, 3, extra)
    a = json.loads(with_pairs.save_raw())
    b = json.loads(without.save_raw())
    assert a["learner"]["gradient_booster"] == b["learner"]["gradient_booster"]


def test_boosters_sharing_a_matrix_keep_their_row_copies(dp, device):
    """Three boosters on one matrix, their rounds interleaved (each returns with its round in
    flight): one-tile items (the row-major copy with the pair's joint tile in place), two-tile
    items (the pair is an item's two tiles: the same copy) and no pairs (the plain copy).  Each
    copy is made once and kept, and the three models are identical."""
    import torch
    from dpgbdt import ops

    n = 60000
    values, labels, _, _ = ops.synth(3, n, 20261203, device=device)
    d = dp.DMatrix(values, labels)
    base = {"objective": "binary:logistic", "max_depth": 6, "eta": 0.3, "max_bin": 256}
    shapes = [{"dp_hist_tiles": 1}, {"dp_hist_tiles": 2}, {"dp_hist_pair": 0}]
    boosters = [dp.Booster(dict(base, **s), [d]) for s in shapes]
    for r in range(3):
        for b in boosters:
            b.update(d, r)
    torch.cuda.synchronize()
    assert [b.tuning()["paired_tiles"] for b in boosters] == [1 << 6, 1 << 6, 0]
    models = [json.loads(b.save_raw())["learner"]["gradient_booster"] for b in boosters]
    assert models[0] == models[1] == models[2]
