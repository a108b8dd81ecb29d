#!/usr/bin/env python3
"""Benchmark of the gradient-boosting training hot path on one MI355X.

Headline (`value`): histogram build throughput in rows*features/s on the C3
workload -- 10,000,000 rows x 128 features, 256 quantile bins, uint8 bins,
fixed-point (g, h) -- with everything resident in HBM.  One step is one
histogram pass over all 10M rows (one launch of the histogram kernel).  The
layout pairs the two tiles of C3's 16-value features (dp_layout_pair_tiles, as
the booster does); the unpaired pass is timed beside it.

The same JSON line carries
  roofline      the histogram operation's algorithmic bytes per launch over
                its average duration (HIP events on the launch stream around
                dp_hist_accumulate, i.e. hist_kernel + hist_reduce_kernel),
                against the 8 TB/s HBM3E peak, and beside it the LDS atomic roof
                (libdp_roof.so: the same LDS addressing with no global loads);
  trees_per_s   full boosting rounds on every configuration: C1 (10k x 8,
                depth 6, 10 trees, logistic), C2 (1M x 28, depth 8, 100 trees,
                logistic), C3 (10M x 128, depth 8, 20 trees, injected
                gradients), C4 (60k x 784, softprob K=10, depth 6, 50 rounds =
                500 trees), C5 (2M x 1000, 95 % missing, 64 bins, squared
                error, depth 10, 50 trees), each with its histogram layout,
                algorithmic bytes per tree (from the trees' node row counts)
                and the resulting share of the HBM peak;
  cpu_baseline  the CPU restatement (oracle, OpenMP) of the same histogram
                pass on a bounded row sample, on this box's host cores; in
                full mode also the oracle's single-threaded booster on C1 (10
                trees) and C2 (2 trees) as trees/s.

Data are synthetic (dp_synth, fixed seeds); nothing is read from disk.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for sub in ("decision-programs_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "histogram build rows·features/s + % HBM peak; trees/s (1M×28, depth 8)"
HBM_PEAK_GBS = 8000.0
SEED = 20261201
# Idle seconds before each tree leg.  Right after a heavy leg (the C3 passes)
# the GPU runs C2 about 6 % slower; measured: back to its fresh rate within 4 s.
# The gap makes every leg start from the same state, whatever ran before it.
LEG_GAP_S = 5.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def algorithmic_hist_bytes(n_rows, n_features, n_bins, gathered=False):
    """u8 bins + 8 B (g, h) per row (+4 B row id when gathered) + F*B*8 B output."""
    return n_rows * n_features + 8 * n_rows + (4 * n_rows if gathered else 0) + \
        n_features * n_bins * 8


def read_traffic():
    """HBM bytes per C3 root histogram call (hist_kernel + hist_reduce_kernel) from the
    committed PMC summary, and where they come from: the summary's path and the commit
    whose kernels its counter runs measured (its `measured_at_commit:` line), so that a
    figure older than the kernels shows as such."""
    rel = os.path.join("profiles", "hist_c3_root_pmc.md")
    value, commit = None, "unknown"
    try:
        for line in open(os.path.join(ROOT, rel)):
            if line.startswith("traffic_bytes_per_launch:"):
                value = float(line.split(":", 1)[1])
            elif line.startswith("measured_at_commit:"):
                commit = line.split(":", 1)[1].strip()
    except OSError:
        return None, None
    return value, f"{rel}@{commit}"


def hist_leg(args, torch, dp, ops):
    """C3 root-pass histogram: K timed launches, events around each launch."""
    n, f = args.rows, 128
    dev = torch.device("cuda:0")
    log(f"C3 data: {n} x {f} synth + quantile cuts + bins")
    values, _, g, h = ops.synth(3, n, SEED + 3, device=dev, want_grad=True)
    ws = ops.Workspace()
    cut_ptr, cuts, _, missing = ops.sketch_cuts(ws, values, 256)
    import numpy as np

    # features 96-127 take 16 values: tiles 6 and 7 are paired (their joint tile, one
    # byte per feature pair, follows the 8 tiles), as the booster pairs them; the
    # unpaired layout is timed beside it on the same buffer
    lay = ops.layout_pair_tiles(ops.layout(n, f, 0, -1), cut_ptr)
    plain = ops.layout(n, f, 0, -1)
    bins = ops.bin_values(values, lay, cut_ptr, cuts)
    del values
    n_bins = np.diff(cut_ptr)
    stride = int(n_bins.max())
    exps, gpair, sums = ops.quantise(ws, g, h)
    gp = gpair[0].contiguous()
    hist = torch.zeros((1, f, stride, 2), dtype=torch.int64, device=dev)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        ops.hist_accumulate(ws, bins, lay, gp, [(0, n)], hist)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev[0].record(stream)
    for k in range(args.steps):
        ops.hist_accumulate(ws, bins, lay, gp, [(0, n)], hist)
        ev[k + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launch_ms = [ev[k].elapsed_time(ev[k + 1]) for k in range(args.steps)]
    avg_ms = sum(launch_ms) / len(launch_ms)
    # the same pass without paired tiles (tuned on first use), for comparison
    ku = args.steps if args.unpaired_steps is None else args.unpaired_steps
    unpaired_ms = None
    if ku > 0:
        unpaired = torch.zeros_like(hist)
        ops.hist_accumulate(ws, bins, plain, gp, [(0, n)], unpaired)
        torch.cuda.synchronize()
        ev_u = [torch.cuda.Event(enable_timing=True) for _ in range(ku + 1)]
        ev_u[0].record(stream)
        for k in range(ku):
            ops.hist_accumulate(ws, bins, plain, gp, [(0, n)], unpaired)
            ev_u[k + 1].record(stream)
        torch.cuda.synchronize()
        unpaired_ms = sum(ev_u[k].elapsed_time(ev_u[k + 1]) for k in range(ku)) / ku
        assert bool((unpaired[0] * (args.warmup + args.steps) == hist[0] * (ku + 1)).all()), \
            "paired and unpaired histograms differ"
        del unpaired
    # size-independent check: every feature's bins sum to the root totals
    h0 = hist[0].sum(dim=1)  # [F, 2]
    reps = args.warmup + args.steps
    tot = sums[0].to(torch.int64) * reps
    assert bool((h0 == tot).all()), "histogram totals differ from the gradient sums"
    abytes = algorithmic_hist_bytes(n, f, 256)
    achieved = abytes / (avg_ms * 1e-3) / 1e9
    out = {
        "n": n, "f": f, "stride": stride, "avg_ms": avg_ms, "wall_s": wall,
        "ms_per_step": wall / args.steps * 1e3,
        "rows_features_per_s": n * f / (avg_ms * 1e-3),
        "achieved_gbs": achieved, "algorithmic_bytes": abytes,
        "min_ms": min(launch_ms), "max_ms": max(launch_ms),
        "tuning": ops.hist_tuning(lay, stride),  # the autotuner's launch shape for this pass
        "paired_tiles": int(lay.paired_tiles),
        "issued_elements": n * (f - 16 * bin(int(lay.paired_tiles)).count("1")),
        "unpaired_avg_ms": unpaired_ms,
        "unpaired_launch_shape": (ops.hist_tuning(plain, stride).get("chosen", {}).get("root")
                                  if unpaired_ms is not None else None),
    }
    sample = None
    if not args.skip_cpu:
        rows = min(n, args.cpu_rows)
        tiles = bins[: ops.layout_bytes(plain)].view(lay.n_tiles, n, lay.tile_width)[:, :rows, :]
        sample_bins = tiles.permute(1, 0, 2).reshape(rows, -1)[:, :f].contiguous().cpu().numpy()
        gq = gp[:rows].cpu().numpy()
        sample = (sample_bins, np.ascontiguousarray(gq[:, 0]), np.ascontiguousarray(gq[:, 1]),
                  stride, hist, exps, sums)
    return out, sample, ws, bins, lay, gp, stride


def lds_roof_leg(torch, elements):
    """LDS atomic roof (libdp_roof.so): the histogram kernel's LDS addressing with no
    global loads, timed per mode and scaled to `elements` row-features.  Mode 0 (two
    64-bit atomics per element) is the exact accumulation the histogram kernel does."""
    import ctypes

    path = os.path.join(ROOT, "decision-programs_amd", "lib", "libdp_roof.so")
    if not os.path.exists(path):
        log("libdp_roof.so not built; LDS roof not measured")
        return None
    lib = ctypes.CDLL(path)
    lib.dp_roof_lds_atomics.argtypes = [ctypes.c_int] * 4 + [ctypes.c_void_p,
                                                            ctypes.POINTER(ctypes.c_float),
                                                            ctypes.c_void_p]
    grid, rows = 4096, 20
    probe_elements = grid * 1024 * rows * 16
    out = torch.empty(grid * 1024, dtype=torch.int64, device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    # modes 5-9: lane aggregation (xor-32 partner) on conflict-free, 16-value and
    # 80 %-zero bins, beside the same bins without it
    names = ["two_u64", "one_u64", "two_u32", "one_u32", "no_lds", "two_u64_16bins",
             "two_u64_16bins_agg", "two_u64_agg", "two_u64_zeros", "two_u64_zeros_agg"]
    res = {}
    for mode, name in enumerate(names):
        ms = ctypes.c_float()
        rc = lib.dp_roof_lds_atomics(mode, grid, rows, 4, out.data_ptr(), ctypes.byref(ms),
                                     stream)
        if rc != 0:
            raise RuntimeError(f"dp_roof_lds_atomics failed ({rc})")
        res[name + "_ms"] = ms.value * elements / probe_elements
    torch.cuda.synchronize()
    return res


def cpu_leg(sample, args):
    import numpy as np
    import pyoracle

    bins, qg, qh, stride = sample[:4]
    threads = host_threads()
    rows, f = bins.shape
    pyoracle.hist_parallel(bins[: min(rows, 4096)], qg[:4096], qh[:4096], stride, -1, threads)
    t0 = time.perf_counter()
    reps = 0
    while True:
        res = pyoracle.hist_parallel(bins, qg, qh, stride, -1, threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= args.cpu_seconds or reps >= 5000:
            break
    per_pass = el / reps
    # the sample histogram must equal the sum over its rows (exact integers)
    assert int(res[0, :, 0].sum()) == int(qg.astype(np.int64).sum())
    return {"value": rows * f / per_pass, "unit": "rows·features/s", "cores": threads,
            "affinity_cores": len(os.sched_getaffinity(0)),
            "hardware_concurrency": os.cpu_count(),
            "kind": "port",
            "sample": f"oracle dpo_hist_parallel root pass over the first {rows} rows x {f} "
                      f"features of the C3 matrix (a bounded sample of its 10M rows), "
                      f"{reps} passes, {el:.1f} s",
            "sample_rows": rows,
            "gbs": algorithmic_hist_bytes(rows, f, 256) / per_pass / 1e9}


def host_threads():
    """Threads of the CPU legs: OMP_NUM_THREADS when set, else the affinity count."""
    env = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return env or len(os.sched_getaffinity(0))


def cpu_trees_leg(torch, ops, name, max_rounds, threads):
    """The oracle's booster (same cuts, bins, sampling and tree rules as the GPU path,
    OpenMP over `threads` host threads; results identical for any count) on the
    configuration's data: trees/s over at most `max_rounds` rounds.  The cuts and uint8
    bins come from the GPU (bit-identical to the oracle's, which the GPU tests pin) so
    the timed CPU work is the boosting rounds, as on the GPU side."""
    import numpy as np
    import pyoracle

    config, n, rounds, depth, eta, objective, max_bin, injected = TREE_CONFIGS[name]
    rounds = min(rounds, max_rounds)
    values, labels, g, h = ops.synth(config, n, SEED + config, want_grad=injected)
    f = values.shape[1]
    ws = ops.Workspace()
    has_missing = bool(torch.isnan(values).any().item())
    # the CPU legs read the device's uint8 bins: byte 255 marks missing values
    eff = min(max_bin, 255) if has_missing else min(max_bin, 256)
    cut_ptr, cuts, _, _ = ops.sketch_cuts(ws, values, eff)
    mb = 255 if has_missing else -1
    lay = ops.layout(n, f, 0, mb)
    bins = ops.from_tiles(ops.bin_values(values, lay, cut_ptr, cuts).cpu().numpy(), lay)
    y = labels.cpu().numpy()
    inj = None
    if injected:
        gn, hn = g.cpu().numpy(), h.cpu().numpy()
        inj = lambda r: (np.roll(gn, r)[:, None], np.roll(hn, r)[:, None])  # noqa: E731
    del values, labels, g, h
    torch.cuda.empty_cache()
    obj = {"binary:logistic": 0, "multi:softprob": 1, "reg:squarederror": 2}[objective]
    k = 10 if obj == 1 else 1
    p = pyoracle.params(eta=eta, max_depth=depth)
    pyoracle.set_threads(threads)
    try:
        t0 = time.perf_counter()
        trees, _, _ = pyoracle.train(bins, cut_ptr, cuts, mb, obj, y, k, p, rounds,
                                     bin_stride=int(np.diff(cut_ptr).max()), injected=inj)
        el = time.perf_counter() - t0
    finally:
        pyoracle.set_threads(1)
    return {"value": len(trees) / el, "unit": "trees/s", "cores": threads, "kind": "port",
            "sample": f"oracle booster, {len(trees)} trees ({rounds} rounds) of {name} "
                      f"({n} x {f}, depth {depth}), {el:.1f} s, {threads} threads"}


# name: (config, rows, rounds, depth, eta, objective, max_bin, injected gradients)
TREE_CONFIGS = {
    "C1": (1, 10_000, 10, 6, 0.3, "binary:logistic", 256, False),
    "C2": (2, 1_000_000, 100, 8, 0.1, "binary:logistic", 256, False),
    "C3": (3, 10_000_000, 20, 8, 0.3, "reg:squarederror", 256, True),
    "C4": (4, 60_000, 50, 6, 0.3, "multi:softprob", 256, False),
    "C5": (5, 2_000_000, 50, 10, 0.3, "reg:squarederror", 64, False),
}


# Rounds of each configuration the CPU baseline times (bounded: about 10-30 s in all).
CPU_TREE_ROUNDS = (("C1", 10), ("C2", 5), ("C3", 2), ("C4", 2), ("C5", 3))


def tree_algorithmic_bytes(t, n_rows, n_features, n_bins, depth, density=None):
    """Minimal HBM bytes of one tree from its node row counts, with the unit figures of
    the build's measurement plan: histogram of a node with n rows n*F (u8 bins) + 8n (g, h)
    + 4n if its rows are gathered + F*B*8 out (present-value layout: 3 B per present value
    + 4 B row pointer + 8 B (g, h) per row instead of the bins and (g, h)); subtraction
    3*F*B*8 per built pair; split scan F*B*8 per node evaluated; partition 9 B per row of
    a split node; gradients 16 B per row."""
    left, right, rows = t["left"], t["right"], t["rows"]
    fb8 = n_features * n_bins * 8

    def hist(n, gathered):
        if density is None:
            return n * n_features + 8 * n + (4 * n if gathered else 0) + fb8
        return int(n * n_features * density) * 3 + 12 * n + (4 * n if gathered else 0) + fb8

    dep = [0] * len(left)
    total = hist(int(rows[0]), False) + 16 * n_rows
    for v in range(len(left)):
        if dep[v] < depth:
            total += fb8  # split scan
        if left[v] < 0:
            continue
        a, b = int(left[v]), int(right[v])
        dep[a] = dep[b] = dep[v] + 1
        total += 9 * int(rows[v])  # partition
        if dep[v] + 1 < depth:  # the children get histograms: build the smaller, subtract
            total += hist(min(int(rows[a]), int(rows[b])), True) + 3 * fb8
    return total


def tree_hist_elements(t, n_rows, n_features, depth):
    """(row, feature) elements the dense histogram passes of one tree accumulate: the root
    over all rows, then the smaller child of every pair that gets a histogram (its sibling
    comes from subtraction).  Two 64-bit LDS atomics each: with the LDS roof's rate this
    gives the tree's histogram time at the roof."""
    left, right, rows = t["left"], t["right"], t["rows"]
    dep = [0] * len(left)
    total = n_rows * n_features
    for v in range(len(left)):
        if left[v] < 0:
            continue
        a, b = int(left[v]), int(right[v])
        dep[a] = dep[b] = dep[v] + 1
        if dep[v] + 1 < depth:
            total += min(int(rows[a]), int(rows[b])) * n_features
    return total


def quantum_ratio(g, h, exps):
    """log2 of this build's per-item fixed-point step over upstream's, per output, for one
    round's gradients.  Here the step is 2^-exps (exps = 30 - the frexp exponent of max|x|).
    Upstream's GradientQuantiser (XGBoost 3.4.1, as published; not checkable here) rounds
    max(sum of positive x, sum of |negative x|) / (1 - 2 n eps) up to a power of two R and
    uses the step R / 2^62.  A ratio of k means the step here is 2^k times upstream's."""
    import math
    import numpy as np

    n = g.shape[0]
    out = {"g": [], "h": []}
    for k in range(g.shape[1]):
        for key, x, e in (("g", g[:, k], exps[k][0]), ("h", h[:, k], exps[k][1])):
            x = x.astype(np.float64)
            big = max(float(x[x > 0].sum()), float(-x[x < 0].sum()))
            if big <= 0.0:
                continue
            rounding_exp = math.frexp(big / (1.0 - 2.0 * n * np.finfo(np.float64).eps))[1]
            out[key].append(62 - int(e) - rounding_exp)
    return {key: (v[0] if len(set(v)) == 1 else [min(v), max(v)]) for key, v in out.items() if v}


def trees_leg(torch, dp, ops, name, rows=None, warm_rounds=4):
    """Wall time of the configuration's boosting rounds on a fresh booster (the
    matrix is quantised and the kernels warmed by a previous booster).  The warm
    booster runs four rounds: the first replay of a captured round in a process
    takes a one-off 6-8 ms, paid by the third round's wait."""
    config, n, rounds, depth, eta, objective, max_bin, injected = TREE_CONFIGS[name]
    n = rows or n
    f = ops.SYNTH_FEATURES[config]
    values, labels, g, h = ops.synth(config, n, SEED + config, want_grad=injected)
    dtrain = dp.DMatrix(values, labels)
    present = float((~torch.isnan(values)).sum().item()) / (n * f)
    # the booster's rule for the present-value layout (dp_sparse_hist=1)
    density = present if present <= 0.25 else None
    layout = ("present-value (sparse) histograms, {:.1%} present".format(present) if density
              else "dense 16-feature tiles")
    del values
    params = {"objective": objective, "tree_method": "hist", "device": "cuda:0",
              "max_depth": depth, "eta": eta, "lambda": 1.0, "min_child_weight": 1.0,
              "max_bin": max_bin}
    if objective == "multi:softprob":
        params["num_class"] = 10
    g1 = g.reshape(-1, 1).contiguous() if injected else None
    h1 = h.reshape(-1, 1).contiguous() if injected else None
    k_out = 10 if objective == "multi:softprob" else 1
    warm = dp.Booster(params, [dtrain])  # quantises the matrix, warms kernels
    quantum = {}
    for r in range(warm_rounds):
        warm.boost(dtrain, r, g1, h1) if injected else warm.update(dtrain, r)
        if r == 0 and not injected:  # the first round's gradients (untimed)
            quantum["round_0"] = quantum_ratio(*warm.last_gradients(n, k_out))
    del warm
    bst = dp.Booster(params, [dtrain])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for r in range(rounds):
        bst.boost(dtrain, r, g1, h1) if injected else bst.update(dtrain, r)
    assert bst.num_boosted_rounds() == rounds  # collects the last round's trees
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    trees = bst.num_trees()
    tuning = bst.tuning()  # the autotuner's launch shapes for this matrix
    if injected:  # the caller's gradients, the same every round
        import math

        gi, hi = g1.cpu().numpy(), h1.cpu().numpy()
        exps = [[30 - math.frexp(float(abs(x).max()))[1] for x in (gi[:, 0], hi[:, 0])]]
        quantum["every_round"] = quantum_ratio(gi, hi, exps)
    else:
        quantum["last_round"] = quantum_ratio(*bst.last_gradients(n, k_out))
    nodes, abytes, helems = 0, 0, 0
    for t in range(trees):
        tr = bst.tree(t)
        nodes += len(tr["left"])
        abytes += tree_algorithmic_bytes(tr, n, f, max_bin, depth, density)
        helems += tree_hist_elements(tr, n, f, depth)
    del bst, dtrain
    torch.cuda.empty_cache()
    gbs = abytes / el / 1e9
    return {"trees": trees, "rounds": rounds, "seconds": el, "value": trees / el,
            "unit": "trees/s", "rows": n, "features": f, "depth": depth, "objective": objective,
            "nodes": nodes, "layout": layout, "algorithmic_bytes_per_tree": abytes / trees,
            # dense layouts: (row, feature) elements of the histogram passes per tree
            "hist_elements_per_tree": None if density else helems / trees,
            "gbs": gbs, "pct_hbm_peak": 100.0 * gbs / HBM_PEAK_GBS,
            "hist_config": tuning.get("chosen", tuning),
            # log2 (this build's fixed-point step / upstream's) for g and h (a [min, max]
            # range over the outputs of multi-output rounds)
            "quantum_log2_ratio": quantum}


def paper_shape_leg(torch, dp, ops):
    """A synthetic run shaped like the only training timing the reference
    publishes (docs/paper/decision-programs-paper.tex:1198: a firewall 4-class
    model, depth 16, 64 rounds, about 52k rows x 2 features, "about 2 seconds").
    Not comparable (other data and GPU); reported for scale only."""
    n = 52_000
    values, _, _, _ = ops.synth(1, n, SEED + 11, n_features=2)
    labels = ((values[:, 0] * 2).floor() * 2 + (values[:, 1] * 2).floor()).clamp(0, 3)
    dtrain = dp.DMatrix(values, labels.to(torch.float32).contiguous())
    params = {"objective": "multi:softmax", "num_class": 4, "max_depth": 16, "eta": 0.3}
    warm = dp.Booster(params, [dtrain])
    for r in range(4):
        warm.update(dtrain, r)
    del warm
    time.sleep(LEG_GAP_S)
    bst = dp.Booster(params, [dtrain])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for r in range(64):
        bst.update(dtrain, r)
    assert bst.num_boosted_rounds() == 64
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    nodes = sum(len(bst.tree(t)["left"]) for t in range(bst.num_trees()))
    return {"workload": "52,000 x 2 synthetic, multi:softmax K=4, depth 16, 64 rounds",
            "trees": bst.num_trees(), "nodes": nodes, "seconds": el,
            "trees_per_s": bst.num_trees() / el,
            "reference_paper": "about 2 s on an RTX A5000 laptop GPU (not comparable)"}


def copy_leg(torch, args):
    """Plain device copy of a known size (counter calibration for PMC runs)."""
    nbytes = 1 << 30
    a = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda:0").fill_(1.0)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(args.steps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes,
                      "launches": args.steps}))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--rows", type=int, default=10_000_000)
    ap.add_argument("--mode", choices=["full", "hist", "copy", "c2", "trees", "paper", "cpu"],
                    default="full")
    ap.add_argument("--configs", default="C1,C2,C3,C4,C5",
                    help="tree configurations timed in full/trees mode")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--unpaired-steps", type=int, default=None,
                    help="timed launches of the unpaired comparison pass (default: --steps; "
                         "0 skips it, e.g. so that a profile's last launches are the paired ones)")
    ap.add_argument("--cpu-rows", type=int, default=1_000_000)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the multi-GPU "
              "row-sharded path is a design that this build does not run.", file=sys.stderr)
        sys.exit(2)
    import torch

    import dpgbdt as dp
    from dpgbdt import ops

    dp.load()
    if args.mode == "copy":
        copy_leg(torch, args)
        return
    if args.mode == "paper":
        print(json.dumps(paper_shape_leg(torch, dp, ops)), flush=True)
        return
    if args.mode == "cpu":  # the CPU baseline's boosters only
        threads = host_threads()
        for name, cap in CPU_TREE_ROUNDS:
            if name in args.configs.split(","):
                print(json.dumps({name: cpu_trees_leg(torch, ops, name, cap, threads)}),
                      flush=True)
        return
    names = [c.strip() for c in args.configs.split(",") if c.strip()]
    if args.mode in ("c2", "trees"):  # boosting rounds only (for kernel-trace profiles)
        for name in (["C2"] if args.mode == "c2" else names):
            time.sleep(LEG_GAP_S)
            print(json.dumps({name: trees_leg(torch, dp, ops, name)}), flush=True)
        return
    hist, sample, *_ = hist_leg(args, torch, dp, ops)
    log(f"hist: {hist['avg_ms']:.3f} ms/launch, {hist['achieved_gbs']:.0f} GB/s algorithmic")
    cands = sorted(hist["tuning"].get("root", []), key=lambda c: c["ms"])
    log("autotuner, fastest root shapes (hist + reduce ms): " + ", ".join(
        f"{c['tiles']}t/{c['unroll']}u/{c['items']}i/s{c['split']} {c['ms']:.3f}" for c in cands[:8]))
    issued = hist["issued_elements"]
    roof = lds_roof_leg(torch, issued)
    if roof:
        roof["frac"] = roof["two_u64_ms"] / hist["avg_ms"]
        roof["elements"] = issued
        roof["note"] = ("LDS atomic roof at the elements this pass accumulates (rows x "
                        "features, a paired tile pair counting once): the histogram's exact "
                        "accumulation (two 64-bit LDS atomics per element) with no global "
                        "loads; frac = roof time / measured launch time")
        log(f"LDS roof (two 64-bit atomics): {roof['two_u64_ms']:.3f} ms, "
            f"{100 * roof['frac']:.0f}% reached")
    trees = {}
    if args.mode == "full":
        for name in names:
            log(f"{name} trees: {TREE_CONFIGS[name]} (after {LEG_GAP_S:.0f} s idle)")
            time.sleep(LEG_GAP_S)
            trees[name] = trees_leg(torch, dp, ops, name,
                                    rows=args.rows if name == "C3" else None)
            el = trees[name]["hist_elements_per_tree"]
            if roof and el:  # the tree's histogram passes at the LDS roof's rate
                trees[name]["hist_lds_roof_ms_per_tree"] = roof["two_u64_ms"] * el / issued
            log(f"{name}: {trees[name]['value']:.1f} trees/s")
    cpu = None
    if sample is not None:
        log(f"CPU baseline: oracle histogram, {args.cpu_seconds:.0f} s budget")
        cpu = cpu_leg(sample, args)
        if args.mode == "full":
            threads = host_threads()
            cpu["trees_per_s"] = {}
            for name, cap in CPU_TREE_ROUNDS:
                log(f"CPU baseline: oracle booster on {name}, {threads} threads")
                cpu["trees_per_s"][name] = cpu_trees_leg(torch, ops, name, cap, threads)
            cpu["trees_per_s_one_thread"] = {}
            for name, cap in (("C1", 10), ("C2", 2)):
                log(f"CPU baseline: oracle booster on {name}, one thread")
                cpu["trees_per_s_one_thread"][name] = cpu_trees_leg(torch, ops, name, cap, 1)
    traffic, traffic_source = read_traffic()
    line = {
        "metric": METRIC,
        "value": hist["rows_features_per_s"],
        "unit": "rows·features/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": hist["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int64",
        "data": "synthetic (dp_synth C3: 64 N(0,1), 32 lognormal, 32 U{0..15} features; "
                "g ~ N(0,1), h ~ U(0.01,0.25)); uint8 quantile bins",
        "config": {"workload": f"C3 histogram root pass: {hist['n']} rows x {hist['f']} "
                               f"features x 256 bins, one launch per step",
                   "rows": hist["n"], "features": hist["f"], "max_bin": 256,
                   "bin_stride": hist["stride"], "parallelism": "single GPU"},
        "pct_hbm_peak": 100.0 * hist["achieved_gbs"] / HBM_PEAK_GBS,
        "roofline": {"bound": "lds", "achieved": hist["achieved_gbs"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": hist["achieved_gbs"] / HBM_PEAK_GBS,
                     "bound_note": "the kernel is bound by its LDS atomics (two exact int64 "
                                   "adds per element; lds_atomic_roof below); achieved, peak "
                                   "and frac are its HBM figures",
                     "traffic": traffic,
                     "traffic_source": traffic_source,
                     "kernel": "dp_hist_accumulate = dp::hist_kernel<false, 0, tiles, unroll, "
                               "split> + dp::hist_reduce_kernel",
                     "algorithmic_bytes_per_launch": hist["algorithmic_bytes"],
                     "lds_atomic_roof": roof,
                     "avg_launch_ms": hist["avg_ms"],
                     "launch_shape": hist["tuning"].get("chosen", {}).get("root"),
                     "paired_tiles": hist["paired_tiles"],
                     "unpaired_avg_launch_ms": hist["unpaired_avg_ms"],
                     "unpaired_launch_shape": hist["unpaired_launch_shape"]},
        "trees_per_s": trees,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
