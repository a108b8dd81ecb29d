// Histogram autotuner: the launch shape of the histogram passes of one matrix
// shape, chosen by timing the candidates on the matrix itself.
//
// The reference has no autotuner (its histograms run inside XGBoost); this one
// re-derives, per (rows, features, bins, layout), the choices the histogram
// kernel leaves open on gfx950:
//   tiles per work item   1 (64 KiB of LDS, two workgroups per CU) or 2
//                         (128 KiB, one per CU; each row's gradient pair is
//                         read once for 32 features instead of 16);
//   rows per lane per pipeline step   1 or 2;
//   with two tiles, the lane bit (4, 5 or none) that swaps a lane's tile
//                         order (fewer lanes per (feature, bin) per atomic);
//   without that swap, on the contiguous (root) pass, the prefetch depth: none
//                         or three blocks of rows in flight per workgroup (more
//                         registers, possibly fewer resident workgroups);
//   work items per pass   512, 1024 or 2048 (fewer, longer row chunks write
//                         fewer partial tiles; more balance the CUs better).
// A layout with paired tiles (tiles whose features all have at most 16 bins)
// is tuned as such: one-tile candidates use every pair, two-tile candidates
// the pairs that are one item's two tiles.
// The contiguous (root) pass is timed over the whole matrix; the gathered pass
// through the row-major copy, as the levels below the root read it, over 12
// nodes whose rows are strided over the matrix (node k: rows k, k + 32, ...),
// 3/8 of the rows in all: a level below the root histograms about that share
// in nodes whose rows are spread over the whole matrix.  Every candidate is
// timed in two sweeps, the second in reverse order, and keeps its faster
// time, so that one disturbed measurement (or drift over the sweep) does not
// pick the shape.  Present-value histograms time their work-item count only.
// Every candidate computes the same exact sums, so the choice changes speed,
// never results.  Choices are cached per process; the timings are kept as a
// JSON report.
#include <algorithm>
#include <cstdio>
#include <map>
#include <mutex>
#include <tuple>

#include "tune.hpp"

namespace dp {
namespace {

using Key = std::tuple<int64_t, int32_t, int32_t, int32_t, int32_t, int32_t, uint64_t>;

std::mutex g_lock;
std::map<Key, HistTuning> g_cache;

// contiguous: the root pass's candidates, which include the three-block
// prefetch; the gathered passes' do not (it was slower on C2's levels, whose
// small items the timed pass does not have, and tied on C3's).
std::vector<HistConfig> dense_candidates(int32_t n_tiles, bool contiguous) {
  std::vector<HistConfig> c;
  for (int32_t tiles : {1, 2}) {
    if (tiles > n_tiles) continue;
    for (int32_t split : {0, 4, 5}) {
      if (tiles == 1 && split) continue;
      for (int32_t deep : {0, 1}) {
        if (deep && (split || !contiguous)) continue;
        for (int32_t unroll : {1, 2})
          for (int32_t items : {512, 1024, 2048})
            c.push_back(HistConfig{tiles, unroll, items, split, deep});
      }
    }
  }
  return c;
}

std::string config_json(const HistConfig& c) {
  char b[128];
  std::snprintf(b, sizeof b,
                "{\"tiles\":%d,\"unroll\":%d,\"items\":%d,\"split\":%d,\"deep\":%d}", c.tiles,
                c.unroll, c.items, c.split, c.deep);
  return b;
}

// Average milliseconds of `run` over three launches after one warm launch.
template <class Run>
double time_ms(Run&& run, hipStream_t s) {
  hipEvent_t a, b;
  DP_HIP(hipEventCreate(&a));
  DP_HIP(hipEventCreate(&b));
  run();
  DP_HIP(hipEventRecord(a, s));
  for (int r = 0; r < 3; ++r) run();
  DP_HIP(hipEventRecord(b, s));
  DP_HIP(hipEventSynchronize(b));
  float ms = 0.0f;
  DP_HIP(hipEventElapsedTime(&ms, a, b));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  return double(ms) / 3.0;
}

// One timed pass: work lists of `nodes` nodes of `rows` positions each
// (node i: [i * rows, (i + 1) * rows) of ridx) for cfg, hist + reduce.
struct Pass {
  const dp_bin_layout* L;
  const uint8_t* bins;
  const uint8_t* rows_major;  // gathered pass: row-major copy and ridx
  const uint8_t* skip;        // skip bins per tile, or null
  const uint32_t* ridx;
  int64_t rows;
  int32_t nodes;
  int32_t bin_stride;
  const int32_t* gpair;
  int64_t* out;  // `nodes` node histograms
  bool fmaj;     // the levels' feature-major partial slots (launch_hist's fmaj)
};

double time_dense(const Pass& p, const HistConfig& cfg, hipStream_t s) {
  std::vector<int64_t> b(size_t(p.nodes)), e(size_t(p.nodes));
  for (int32_t i = 0; i < p.nodes; ++i) {
    b[size_t(i)] = int64_t(i) * p.rows;
    e[size_t(i)] = b[size_t(i)] + p.rows;
  }
  std::vector<HistWork> w;
  std::vector<HistReduce> j;
  const int32_t slots =
      make_hist_work(*p.L, b.data(), e.data(), nullptr, p.nodes, true, w, j, 0, cfg);
  DeviceBuffer<HistWork> dw(w.size());
  DeviceBuffer<HistReduce> dj(j.size());
  DeviceBuffer<int64_t> partial(size_t(std::max(slots, 1)) * size_t(p.bin_stride) * 32);
  DP_HIP(hipMemcpyAsync(dw.p, w.data(), dw.bytes(), hipMemcpyHostToDevice, s));
  DP_HIP(hipMemcpyAsync(dj.p, j.data(), dj.bytes(), hipMemcpyHostToDevice, s));
  const double ms = time_ms(
      [&] {
        // With fmaj the reduce below reads the slots in the other layout: its
        // sums are discarded, its time stands for the levels' reduce.
        launch_hist(p.bins, *p.L, p.gpair, p.ridx, dw.p, int32_t(w.size()), nullptr,
                    p.bin_stride, p.out, partial.p, s, p.rows_major, cfg, p.skip, p.fmaj);
        launch_hist_reduce(partial.p, dj.p, p.nodes, nullptr, p.L->n_tiles, p.L->n_features,
                           p.bin_stride, nullptr, p.out, false, s);
      },
      s);
  DP_HIP(hipStreamSynchronize(s));  // before the buffers are freed
  return ms;
}

// Near-tie bands: the root and present-value passes, and the gathered passes,
// whose timed pass ranks the item counts of a tree's levels less faithfully
// (measured on C3: its two-tile gathered shapes with 1,024 items timed 2.7-3.2 %
// faster than the 512-item ones, so the pick flipped between runs, and trained
// at 468-471 trees/s against 485-487 with 512 items).
constexpr double kTieShare = 0.03;
constexpr double kTieShareGathered = 0.05;

template <class Time>
HistConfig pick(const std::vector<HistConfig>& cands, Time&& time, std::string& report,
                const char* name, double tie = kTieShare) {
  // Two sweeps, the second in reverse order; each candidate keeps its best.
  std::vector<double> ms(cands.size());
  for (size_t i = 0; i < cands.size(); ++i) ms[i] = time(cands[i]);
  for (size_t i = cands.size(); i-- > 0;) ms[i] = std::min(ms[i], time(cands[i]));
  report += std::string("\"") + name + "\":[";
  for (size_t i = 0; i < cands.size(); ++i) {
    char b[64];
    std::snprintf(b, sizeof b, ",\"ms\":%.5f}", ms[i]);
    std::string c = config_json(cands[i]);
    c.pop_back();
    report += (i ? "," : "") + c + b;
  }
  report += "]";
  // Near-ties (within `tie` of the fastest) go to the fewest work items,
  // then to one row per lane per step, then the faster: fewer items write
  // fewer partial slots, which a tree's levels pay for in their reduce more
  // than the timed passes show (measured on C3: the gathered shapes within 2 %
  // of each other here trained at 438 to 469 trees/s, the fewer items
  // faster); two rows per step were slower on the small items of C2's levels
  // (about 1 us per level), which the timed pass's larger items do not show.
  const double fastest = *std::min_element(ms.begin(), ms.end());
  size_t best = 0;
  bool have = false;
  for (size_t i = 0; i < cands.size(); ++i) {
    if (ms[i] > fastest * (1.0 + tie)) continue;
    const HistConfig &c = cands[i], &b = cands[best];
    const auto rank = [](const HistConfig& x) { return std::tuple(x.items, x.unroll); };
    if (!have || rank(c) < rank(b) || (rank(c) == rank(b) && ms[i] < ms[best])) best = i;
    have = true;
  }
  return cands[best];
}

}  // namespace

const HistTuning& tune_dense_hist(const dp_bin_layout& L, const uint8_t* bins, bool gathered,
                                  int32_t bin_stride, const int32_t* gpair, hipStream_t s,
                                  const uint8_t* skip) {
  const Key key{L.n_rows, L.n_features, bin_stride, L.missing_bin, gathered ? 1 : 0,
                skip ? 1 : 0, L.paired_tiles};
  std::lock_guard<std::mutex> hold(g_lock);
  auto it = g_cache.find(key);
  if (it != g_cache.end()) return it->second;
  HistTuning t;
  const auto cands = dense_candidates(L.n_tiles, true);
  constexpr int32_t kStride = 32, kNodes = 12;  // the gathered pass's nodes (see above)
  DeviceBuffer<int64_t> out(size_t(kNodes) * size_t(L.n_features) * size_t(bin_stride) * 2);
  Pass root{&L, bins, nullptr, skip, nullptr, L.n_rows, 1, bin_stride, gpair, out.p, false};
  std::string report = "{";
  t.root = pick(cands, [&](const HistConfig& c) { return time_dense(root, c, s); }, report,
                "root");
  t.level = t.root;
  if (gathered && L.n_rows >= kStride) {
    // node k: rows k, k + kStride, k + 2 kStride, ... (k < kNodes)
    const int64_t per = L.n_rows / kStride;
    std::vector<uint32_t> ids(size_t(per) * kNodes);
    for (int32_t k = 0; k < kNodes; ++k)
      for (int64_t i = 0; i < per; ++i)
        ids[size_t(k) * size_t(per) + size_t(i)] = uint32_t(i * kStride + k);
    DeviceBuffer<uint32_t> ridx(ids.size());
    DP_HIP(hipMemcpyAsync(ridx.p, ids.data(), ridx.bytes(), hipMemcpyHostToDevice, s));
    // The row-major copy a candidate reads: the pairs it uses (hist_pairs)
    // hold their joint tiles in place of their first tiles; one copy per set.
    std::map<uint64_t, DeviceBuffer<uint8_t>> copies;
    auto rows_for = [&](const HistConfig& c) -> const uint8_t* {
      const uint64_t used = hist_pairs(L.paired_tiles, c.tiles);
      auto it = copies.find(used);
      if (it == copies.end()) {
        dp_bin_layout rl = L;
        rl.paired_tiles = used;
        it = copies.emplace(used, DeviceBuffer<uint8_t>(size_t(L.n_rows) * size_t(L.n_tiles) * 16))
                 .first;
        launch_tiles_to_rows(bins, rl, it->second.p, s);
      }
      return it->second.p;
    };
    // The levels' flush layout: feature-major where the booster fuses the
    // reduce and the evaluation (it costs more per item than the LDS image).
    const bool fmaj = L.n_features >= kDenseFuseFeatures && bin_stride <= 256;
    report += ",";
    t.level = pick(
        dense_candidates(L.n_tiles, false),
        [&](const HistConfig& c) {
          Pass level{&L,  bins,   rows_for(c), skip, ridx.p, per, kNodes, bin_stride,
                     gpair, out.p, fmaj};
          return time_dense(level, c, s);
        },
        report, "gathered", kTieShareGathered);
    DP_HIP(hipStreamSynchronize(s));
  }
  t.tuned = true;
  report += ",\"chosen\":{\"root\":" + config_json(t.root) + ",\"gathered\":" +
            config_json(t.level) + "}}";
  t.report = report;
  return g_cache.emplace(key, std::move(t)).first->second;
}

const HistTuning* find_dense_tuning(const dp_bin_layout& L, int32_t bin_stride, bool gathered) {
  const Key key{L.n_rows, L.n_features, bin_stride, L.missing_bin, gathered ? 1 : 0, 0,
                L.paired_tiles};
  std::lock_guard<std::mutex> hold(g_lock);
  auto it = g_cache.find(key);
  return it == g_cache.end() ? nullptr : &it->second;
}

const HistTuning& tune_sparse_hist(const SparseBins& sp, int64_t n_rows, int32_t n_features,
                                   int32_t bin_stride, const int32_t* gpair, hipStream_t s) {
  const Key key{n_rows, n_features, bin_stride, sp.tile_features, 2, int32_t(sp.nnz % 1000003),
                0};
  std::lock_guard<std::mutex> hold(g_lock);
  auto it = g_cache.find(key);
  if (it != g_cache.end()) return it->second;
  HistTuning t;
  std::vector<HistConfig> cands;
  for (int32_t items : {512, 1024, 2048}) cands.push_back(HistConfig{1, 2, items});
  DeviceBuffer<int64_t> out(size_t(n_features) * size_t(bin_stride) * 2);
  // The booster sums the root's partial slots in the launch that also
  // evaluates them (reduce_evaluate_flat_kernel) whenever the bins allow it;
  // its reduce runs one workgroup per 16 features, so its time grows with the
  // slots far more than the reduce-only launch's.  The timed pass runs that
  // launch, with node sums of zero (every candidate is refused at once, the
  // same small evaluation for each candidate count).
  const bool fused = bin_stride <= 64 && sp.tile_features % 16 == 0;  // as the booster decides
  DeviceBuffer<int32_t> nbins(fused ? size_t(n_features) : 0);
  DeviceBuffer<int64_t> sums(fused ? 2 : 0);
  DeviceBuffer<int32_t> exps(fused ? 2 : 0);
  DeviceBuffer<FeatCand> feat(fused ? size_t(n_features) : 0);
  std::vector<int32_t> nb;  // alive until the stream has read it (synchronised below)
  if (fused) {
    nb.assign(size_t(n_features), bin_stride);
    DP_HIP(hipMemcpyAsync(nbins.p, nb.data(), nbins.bytes(), hipMemcpyHostToDevice, s));
    DP_HIP(hipMemsetAsync(sums.p, 0, sums.bytes(), s));
    DP_HIP(hipMemsetAsync(exps.p, 0, exps.bytes(), s));
  }
  const dp_train_param zero{};
  dp_bin_layout L{};
  L.n_rows = n_rows;
  L.n_features = n_features;
  L.tile_width = 16;
  L.n_tiles = sp.n_tiles;
  std::string report = "{";
  t.root = pick(
      cands,
      [&](const HistConfig& c) {
        const int64_t b = 0, e = n_rows;
        std::vector<HistWork> w;
        std::vector<HistReduce> j;
        const int32_t slots = make_hist_work(L, &b, &e, nullptr, 1, true, w, j, sp.n_tiles, c);
        DeviceBuffer<HistWork> dw(w.size());
        DeviceBuffer<HistReduce> dj(j.size());
        DeviceBuffer<int64_t> partial(size_t(std::max(slots, 1)) * size_t(sp.tile_features) *
                                      size_t(bin_stride) * 2);
        DP_HIP(hipMemcpyAsync(dw.p, w.data(), dw.bytes(), hipMemcpyHostToDevice, s));
        DP_HIP(hipMemcpyAsync(dj.p, j.data(), dj.bytes(), hipMemcpyHostToDevice, s));
        const double ms = time_ms(
            [&] {
              launch_hist_sparse(sp, n_rows, n_features, gpair, nullptr, dw.p, int32_t(w.size()),
                                 nullptr, bin_stride, out.p, partial.p, s);
              if (fused)
                launch_reduce_evaluate_flat(partial.p, dj.p, 1, nullptr, sp.n_tiles,
                                            sp.tile_features, n_features, bin_stride, nullptr,
                                            out.p, nbins.p, sums.p, exps.p, zero, nullptr,
                                            nullptr, feat.p, true, s);
              else
                launch_hist_reduce_flat(partial.p, dj.p, 1, nullptr, sp.n_tiles,
                                        sp.tile_features, n_features, bin_stride, nullptr, out.p,
                                        s);
            },
            s);
        DP_HIP(hipStreamSynchronize(s));
        return ms;
      },
      report, "present_value");
  t.level = t.root;
  t.tuned = true;
  report += ",\"chosen\":{\"root\":" + config_json(t.root) + ",\"gathered\":" +
            config_json(t.level) + "}}";
  t.report = report;
  return g_cache.emplace(key, std::move(t)).first->second;
}

}  // namespace dp
