"""dp_evaluate_splits_noalloc: the split evaluation that allocates nothing.

Its per-(node, feature) candidates live in a library-owned device array shared
by every call on the GPU.  Through the C ABI it must return, byte for byte, the
split records dp_evaluate_splits returns on the same histograms -- on two calls
in a row, the second smaller (the array still holds the first call's
candidates), on each evaluation kernel (more than 64 bins, at most 64 bins, at
most 16 features) -- and refuse a call larger than its array with an error.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _inputs(rng, n_nodes, f, stride, device):
    import torch

    n_bins = rng.integers(2, stride + 1, size=f).astype(np.int32)
    n_bins[rng.integers(0, f)] = stride
    g = rng.integers(-(1 << 24), 1 << 24, size=(n_nodes, f, stride)).astype(np.int64)
    h = rng.integers(1, 1 << 22, size=(n_nodes, f, stride)).astype(np.int64)
    mask = np.arange(stride)[None, None, :] < n_bins[None, :, None]
    g *= mask
    h *= mask
    hist = np.stack([g, h], axis=-1)
    # node totals: feature 0's bins plus some missing rows' sums
    sums = np.stack([g[:, 0].sum(1) + rng.integers(-(1 << 26), 1 << 26, size=n_nodes),
                     h[:, 0].sum(1) + rng.integers(0, 1 << 26, size=n_nodes)], axis=1)
    # every other feature holds the same node total (missing = the difference)
    for k in range(1, f):
        short_g = sums[:, 0] - g[:, k].sum(1)
        short_h = sums[:, 1] - h[:, k].sum(1)
        assert np.all(np.abs(short_g) < (1 << 60)) and np.all(np.abs(short_h) < (1 << 60))
    return (torch.as_tensor(hist, device=device), torch.as_tensor(n_bins, device=device),
            torch.as_tensor(sums.astype(np.int64), device=device))


def _noalloc(dp, hist, n_bins, sums, exp_g, exp_h, param):
    import torch
    from dpgbdt import SplitRecord, ops

    lib = dp.load()
    n_nodes, f, stride, _ = hist.shape
    out = torch.empty((n_nodes, ctypes.sizeof(SplitRecord)), dtype=torch.uint8,
                      device=hist.device)
    rc = lib.dp_evaluate_splits_noalloc(ops._ptr(hist), n_nodes, f, stride, ops._ptr(n_bins),
                                        ops._ptr(sums), exp_g, exp_h, ctypes.byref(param),
                                        ops._ptr(out), ops._stream())
    return rc, out


@pytest.mark.parametrize("order", ["large_then_small", "small_then_large"])
def test_noalloc_matches_workspace_entry(dp, ws, device, order):
    import torch
    from dpgbdt import ops

    cases = [(300, 200, 256), (37, 90, 64)]  # >64 bins (one feature per wave), <=64 bins
    if order == "small_then_large":
        cases = cases[::-1]
    cases.append((50, 12, 200))  # at most 16 features: no scratch used
    rng = np.random.default_rng(11)
    valid_seen = {c: False for c in cases}
    for prm in [dict(), dict(lam=0.0, alpha=0.5, gamma=1.0, min_child_weight=3.0)]:
        param = ops.train_param(**prm)
        for case in cases:
            n_nodes, f, stride = case
            print(f"noalloc case nodes={n_nodes} features={f} bins={stride} {prm}", flush=True)
            hist, n_bins, sums = _inputs(rng, n_nodes, f, stride, device)
            want = ops.splits_to_numpy(ops.evaluate_splits(ws, hist, n_bins, sums, 26, 24, param))
            rc, out = _noalloc(dp, hist, n_bins, sums, 26, 24, param)
            assert rc == 0, dp.load().XGBGetLastError().decode()
            torch.cuda.synchronize()
            got = ops.splits_to_numpy(out)
            assert got.tobytes() == want.tobytes()
            valid_seen[case] |= bool(np.any(got["valid"] == 1))
    assert all(valid_seen.values()), valid_seen  # the records compared hold real splits


def test_noalloc_refuses_beyond_its_array(dp, device):
    import torch
    from dpgbdt import ops

    # 2,049 nodes x 256 features x 32 bytes of candidates > 16 MiB: refused on
    # the host before any launch (the inputs are never read).
    hist = torch.zeros((1, 1, 1, 2), dtype=torch.int64, device=device)
    n_bins = torch.ones(256, dtype=torch.int32, device=device)
    sums = torch.zeros((2049, 2), dtype=torch.int64, device=device)
    lib = dp.load()
    from dpgbdt import SplitRecord

    out = torch.empty((2049, ctypes.sizeof(SplitRecord)), dtype=torch.uint8, device=device)
    rc = lib.dp_evaluate_splits_noalloc(ops._ptr(hist), 2049, 256, 256, ops._ptr(n_bins),
                                        ops._ptr(sums), 26, 28, ctypes.byref(ops.train_param()),
                                        ops._ptr(out), ops._stream())
    assert rc == -1
    assert "exceeds" in lib.XGBGetLastError().decode()


def test_noalloc_inside_graph_capture(dp, ws, device):
    """The callers it is for: one warm call (the per-device array address is looked up
    then), then the call captured into a HIP graph with torch.cuda.graph and replayed on new
    histograms copied into the captured input buffers.  Every replay, with eager work and
    synchronisations between replays, must equal dp_evaluate_splits on the same inputs."""
    import torch
    from dpgbdt import SplitRecord, ops

    lib = dp.load()
    rng = np.random.default_rng(23)
    n_nodes, f, stride = 40, 120, 256
    param = ops.train_param()
    hist, n_bins, sums = _inputs(rng, n_nodes, f, stride, device)
    out = torch.empty((n_nodes, ctypes.sizeof(SplitRecord)), dtype=torch.uint8, device=device)

    def call():
        return lib.dp_evaluate_splits_noalloc(ops._ptr(hist), n_nodes, f, stride,
                                              ops._ptr(n_bins), ops._ptr(sums), 26, 24,
                                              ctypes.byref(param), ops._ptr(out), ops._stream())

    assert call() == 0  # warm: the array's device address is known from here on
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert call() == 0, lib.XGBGetLastError().decode()
    valid = 0
    for replay in range(4):
        h2, b2, s2 = _inputs(rng, n_nodes, f, stride, device)
        torch.cuda.synchronize()
        hist.copy_(h2)
        n_bins.copy_(b2)
        sums.copy_(s2)
        want = ops.splits_to_numpy(ops.evaluate_splits(ws, hist, n_bins, sums, 26, 24, param))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = ops.splits_to_numpy(out)
        print(f"noalloc graph replay {replay}", flush=True)
        assert got.tobytes() == want.tobytes(), f"replay {replay}"
        valid += int(np.sum(got["valid"] == 1))
    assert valid > 0
