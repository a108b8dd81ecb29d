// Split evaluation: per node, per feature, a wavefront prefix scan over the
// bins of the fixed-point histogram, the loss change of every candidate in
// both missing directions, and an argmax with deterministic ties.  One
// wavefront per (node, feature) finds the feature's best candidate.  With up
// to 64 features one workgroup of 16 wavefronts takes a whole node and writes
// its split record (one launch per level); with more, the (node, feature)
// items spread over the chip and a second kernel picks each node's best
// feature.
//
// Semantics (upstream CalcGain/CalcWeight with max_delta_step 0, reached in the
// reference only through XGBoosterUpdateOneIter, class_native_training.cuh:67;
// regularisation parameters whitelisted at class_native_training.cuh:18-27):
//   T(G) = sign(G) max(|G| - alpha, 0);  gain(G,H) = T(G)^2 / (H + lambda),
//   0 when H < min_child_weight or H <= 0.
//   Candidate (f, b): bins <= b left; missing right, then missing left (kept
//   only when strictly better).  Valid iff both children have positive
//   quantised hessian and H >= min_child_weight.  loss = (gain(L) + gain(R)) -
//   gain(P) in double.  Argmax: largest loss, ties to lowest feature, then
//   lowest bin.  expand = valid && loss > 1e-6 && loss >= gamma.
// All double arithmetic is compiled with -ffp-contract=off so each value
// rounds exactly as the CPU restatement computes it.
#include "dp_internal.hpp"
#include "sample.hpp"
#include "select.hpp"
#include "gain.hpp"

#include <algorithm>
#include <cmath>

namespace dp {
namespace {

constexpr int kFeatWaves = 4;  // features per workgroup in evaluate_features_kernel

// The largest value of the wavefront, in lane 63 (the same steps as the scan).
__device__ __forceinline__ double wave_max_to_last(double v) {
  long long b = __double_as_longlong(v);
  auto step = [&](long long o) {
    const double ov = dpp_f64_bits(o), cv = dpp_f64_bits(b);
    if (ov > cv) b = o;
  };
  step(dpp64<0x111>(b, b));
  step(dpp64<0x112>(b, b));
  step(dpp64<0x114>(b, b));
  step(dpp64<0x118>(b, b));
  step(dpp64<0x142, 0xa>(b, b));
  step(dpp64<0x143, 0xc>(b, b));
  return dpp_f64_bits(b);
}


// One feature's histogram of one node as one wavefront holds it: bins
// lane * BPL + j (bins past bin_stride read as zero).
template <int BPL>
struct FeatBins {
  long long g[BPL], h[BPL];
};

template <int BPL>
__device__ __forceinline__ void load_feature(const long long* __restrict__ hist, int32_t node,
                                             int32_t f, int32_t n_features, int32_t bin_stride,
                                             FeatBins<BPL>& d) {
  const int lane = threadIdx.x & 63;
  const long long* hf = hist + (int64_t(node) * n_features + f) * bin_stride * 2;
#pragma unroll
  for (int j = 0; j < BPL; ++j) {
    const int b = lane * BPL + j;
    d.g[j] = b < bin_stride ? hf[2 * b] : 0;
    d.h[j] = b < bin_stride ? hf[2 * b + 1] : 0;
  }
}

// The best candidate of feature f of one node, computed by one wavefront
// (BPL bins per lane, bin_stride <= 64 * BPL): an inclusive prefix scan over
// the bins, both missing directions, and the argmax.  Every lane returns the
// same result; loss is -inf when the feature has no valid candidate.
template <int BPL>
__device__ __forceinline__ Cand feature_best(const FeatBins<BPL>& d, int32_t f, int nb, int skip,
                                             long long gp, long long hp, double parent_gain,
                                             double ug, double uh, const Param& p) {
  const int lane = threadIdx.x & 63;
  long long sg[BPL], sh[BPL];
  long long rg = 0, rh = 0;
#pragma unroll
  for (int j = 0; j < BPL; ++j) {
    rg += d.g[j];
    rh += d.h[j];
    sg[j] = rg;
    sh[j] = rh;
  }
  // inclusive wavefront scan of the lane totals
  const long long ig = wave_inclusive_sum(rg), ih = wave_inclusive_sum(rh);
  const long long total_g = readlane64(ig, 63), total_h = readlane64(ih, 63);
  const long long og = ig - rg, oh = ih - rh;  // exclusive offset of this lane
  // The node's rows the bins do not hold: the missing rows, or (skip >= 0, no
  // missing values) the rows of the skipped bin, which the prefixes from that
  // bin on take back.
  long long mg = gp - total_g, mh = hp - total_h, kg = 0, kh = 0;
  if (skip >= 0) {
    kg = mg;
    kh = mh;
    mg = mh = 0;
  }

  Cand c;
  c.loss = -INFINITY;
  c.gl = c.hl = 0;
  c.feature = f;
  c.bin = -1;
  c.dl = 0;
  if (nb > 0) {  // uniform per wavefront (a feature left out by sampling has none)
    long long lg[BPL], lh[BPL];
    int in = 0;
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
      const int b = lane * BPL + j;
      lg[j] = og + sg[j] + (b >= skip && skip >= 0 ? kg : 0);
      lh[j] = oh + sh[j] + (b >= skip && skip >= 0 ? kh : 0);
      in |= (b < nb ? 1 : 0) << j;
    }
    best_of_bins<BPL>(lg, lh, in, lane * BPL, mg, mh, gp, hp, ug, uh, parent_gain, p, c);
  }
  // Wave argmax: the largest loss, then the lowest lane holding it (lanes hold
  // increasing bins, and each lane kept its lowest bin on ties), so the
  // winner is the lowest bin with the largest loss -- better()'s order within
  // one feature.  Only the loss crosses lanes in the reduction; the winner's
  // fields are then read from its lane.
  const double best = dpp_f64_bits(readlane64(__double_as_longlong(wave_max_to_last(c.loss)), 63));
  const unsigned long long hit = __ballot(c.loss == best);
  const int winner = __builtin_ctzll(hit);
  Cand r;
  r.loss = dpp_f64_bits(readlane64(__double_as_longlong(c.loss), winner));
  r.gl = readlane64(c.gl, winner);
  r.hl = readlane64(c.hl, winner);
  r.feature = f;
  r.bin = __builtin_amdgcn_readlane(c.bin, winner);
  r.dl = __builtin_amdgcn_readlane(c.dl, winner);
  return r;
}

// One wavefront per (node, feature): the feature's best candidate.
// Workgroups loop over (node, feature group) items; the node count may come
// from device memory.
template <int BPL>
__global__ __launch_bounds__(64 * kFeatWaves) void evaluate_features_kernel(
    const long long* __restrict__ hist, int32_t n_nodes_host,
    const int32_t* __restrict__ n_nodes_dev, int32_t n_features, int32_t bin_stride,
    const int32_t* __restrict__ n_bins, const long long* __restrict__ node_sums,
    const int32_t* __restrict__ exps, int32_t exp_g_host, int32_t exp_h_host, Param p,
    const uint32_t* __restrict__ fmask, const uint8_t* __restrict__ skip_bins,
    FeatCand* __restrict__ cand) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int32_t n_nodes = n_nodes_dev ? *n_nodes_dev : n_nodes_host;
  const int32_t groups = (n_features + kFeatWaves - 1) / kFeatWaves;
  const int64_t n_items = int64_t(n_nodes) * groups;
  const int exp_g = exps ? exps[0] : exp_g_host;
  const int exp_h = exps ? exps[1] : exp_h_host;
  const double ug = ldexp(1.0, -exp_g), uh = ldexp(1.0, -exp_h);
  for (int64_t item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int32_t node = int32_t(item / groups);
    const int32_t f = int32_t(item % groups) * kFeatWaves + wave;
    if (f >= n_features) continue;  // wave-uniform; no barriers in this kernel
    FeatBins<BPL> bins;
    load_feature<BPL>(hist, node, f, n_features, bin_stride, bins);
    const long long gp = node_sums[2 * node], hp = node_sums[2 * node + 1];
    const double parent_gain = calc_gain(p, double(gp) * ug, double(hp) * uh);
    // A feature outside the node's sample has no bins to split at: loss -inf.
    const int nb = feature_allowed(fmask, node, f, n_features) ? n_bins[f] : 0;
    const int skip = skip_bins ? int(skip_bins[f]) : -1;
    const Cand c = feature_best<BPL>(bins, f, nb, skip, gp, hp, parent_gain, ug, uh, p);
    if (lane == 0) cand[int64_t(node) * n_features + f] = FeatCand{c.loss, c.gl, c.hl, c.bin, c.dl};
  }
}

// Up to 64 bins: four features per wavefront (seg_evaluate).  Workgroups loop
// over (node, group of 16 features) items.
__global__ __launch_bounds__(256) void evaluate_features_seg_kernel(
    const long long* __restrict__ hist, int32_t n_nodes_host,
    const int32_t* __restrict__ n_nodes_dev, int32_t n_features, int32_t bin_stride,
    const int32_t* __restrict__ n_bins, const long long* __restrict__ node_sums,
    const int32_t* __restrict__ exps, int32_t exp_g_host, int32_t exp_h_host, Param p,
    const uint32_t* __restrict__ fmask, const uint8_t* __restrict__ skip_bins,
    FeatCand* __restrict__ cand) {
  constexpr int BPL = 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int seg = lane >> 4, sub = lane & 15;
  const int32_t n_nodes = n_nodes_dev ? *n_nodes_dev : n_nodes_host;
  const int32_t groups = (n_features + kSegFeatures - 1) / kSegFeatures;
  const int64_t n_items = int64_t(n_nodes) * groups;
  const int exp_g = exps ? exps[0] : exp_g_host;
  const int exp_h = exps ? exps[1] : exp_h_host;
  const double ug = ldexp(1.0, -exp_g), uh = ldexp(1.0, -exp_h);
  for (int64_t item = blockIdx.x; item < n_items; item += gridDim.x) {
    const int32_t node = int32_t(item / groups);
    const int32_t f = int32_t(item % groups) * kSegFeatures + wave * 4 + seg;
    const bool live = f < n_features;  // every lane takes part in the row steps
    long long dg[BPL], dh[BPL];
    const long long* hf = hist + (int64_t(node) * n_features + (live ? f : 0)) * bin_stride * 2;
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
      const int b = sub * BPL + j;
      dg[j] = live && b < bin_stride ? hf[2 * b] : 0;
      dh[j] = live && b < bin_stride ? hf[2 * b + 1] : 0;
    }
    seg_evaluate(dg, dh, node, f, live, n_features, n_bins, node_sums, ug, uh, p, fmask,
                 skip_bins, cand);
  }
}

// Reduce and evaluate in one launch for the present-value layout, whose
// partial slots already hold the node histogram's [feature][bin][g, h] words
// (word e of tile t's slot is word t * tile_features * bin_stride * 2 + e of a
// node histogram).  A 256-thread workgroup per (reduce job, 16 features): each
// lane owns four bins of one feature, as seg_evaluate holds them, sums the
// job's partial slots of its 64 contiguous bytes (or takes what the node's
// only chunk wrote), writes the built and sibling words, and evaluates both
// nodes' feature from its registers.  No barriers, and no second pass over the
// level's histograms: the words and candidates are those of
// hist_reduce_flat_kernel followed by evaluate_features_seg_kernel.  With
// store == 0 (the tree's last split level, whose histograms no later level
// reads) the built and sibling words are evaluated but not written.  With
// skip_direct, jobs whose node was built by its only chunk are left alone:
// the present-value histogram pass evaluated them from LDS.
__global__ __launch_bounds__(256) void reduce_evaluate_flat_kernel(
    const long long* __restrict__ partial, const HistReduce* __restrict__ jobs,
    int32_t n_jobs_host, const int32_t* __restrict__ n_jobs_dev, int32_t n_tiles,
    int32_t tile_features, int32_t n_features, int32_t bin_stride,
    const long long* __restrict__ parent_base, long long* __restrict__ hist,
    const int32_t* __restrict__ n_bins, const long long* __restrict__ node_sums,
    const int32_t* __restrict__ exps, Param p, const uint32_t* __restrict__ fmask,
    const uint8_t* __restrict__ skip_bins, FeatCand* __restrict__ cand, int32_t store,
    int32_t skip_direct) {
  constexpr int BPL = 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int seg = lane >> 4, sub = lane & 15;
  const int32_t f = int32_t(blockIdx.x) * kSegFeatures + wave * 4 + seg;
  const bool live = f < n_features;
  const int32_t fl = live ? f : 0;
  const int32_t t = fl / tile_features;
  const int64_t slot_words = int64_t(tile_features) * bin_stride * 2;
  const int64_t node_elems = int64_t(n_features) * bin_stride * 2;
  const int64_t feat_at = int64_t(fl) * bin_stride * 2 + 2 * (sub * BPL);  // this lane's first bin
  const int64_t slot_at = int64_t(fl - t * tile_features) * bin_stride * 2 + 2 * (sub * BPL);
  // bins of this lane that exist (the lane's bins are sub * 4 + j)
  const int rest = bin_stride - sub * BPL;
  const int nbl = !live || rest < 0 ? 0 : (rest > BPL ? BPL : rest);
  const int32_t n_jobs = n_jobs_dev ? *n_jobs_dev : n_jobs_host;
  const double ug = ldexp(1.0, -exps[0]), uh = ldexp(1.0, -exps[1]);
  for (int32_t jb = blockIdx.y; jb < n_jobs; jb += gridDim.y) {
    const HistReduce j = jobs[jb];
    if (skip_direct && j.nc == 1 && j.p0 < 0) continue;  // uniform per workgroup
    long long bg[BPL] = {0, 0, 0, 0}, bh[BPL] = {0, 0, 0, 0};
    long long* built = hist + int64_t(j.slot) * node_elems + feat_at;
    if (j.nc == 1 && j.p0 < 0) {  // written directly by the node's only chunk
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        if (k < nbl) {
          bg[k] = built[2 * k];
          bh[k] = built[2 * k + 1];
        }
      }
    } else {
      const long long* src = partial + (int64_t(j.p0) * n_tiles + t) * slot_words + slot_at;
      const int64_t step = int64_t(n_tiles) * slot_words;
      for (int32_t c = 0; c < j.nc; ++c) {
#pragma unroll
        for (int k = 0; k < BPL; ++k) {
          if (k < nbl) {
            bg[k] += src[c * step + 2 * k];
            bh[k] += src[c * step + 2 * k + 1];
          }
        }
      }
      if (store) {
#pragma unroll
        for (int k = 0; k < BPL; ++k) {
          if (k < nbl) {
            built[2 * k] = bg[k];
            built[2 * k + 1] = bh[k];
          }
        }
      }
    }
    seg_evaluate(bg, bh, j.slot, f, live, n_features, n_bins, node_sums, ug, uh, p, fmask,
                 skip_bins, cand);
    if (j.sibling >= 0) {  // uniform per workgroup
      long long sg[BPL] = {0, 0, 0, 0}, sh[BPL] = {0, 0, 0, 0};
      const long long* par = parent_base + j.parent + feat_at;
      long long* sib = hist + int64_t(j.sibling) * node_elems + feat_at;
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        if (k < nbl) {
          sg[k] = par[2 * k] - bg[k];
          sh[k] = par[2 * k + 1] - bh[k];
          if (store) {
            sib[2 * k] = sg[k];
            sib[2 * k + 1] = sh[k];
          }
        }
      }
      seg_evaluate(sg, sh, j.sibling, f, live, n_features, n_bins, node_sums, ug, uh, p, fmask,
                   skip_bins, cand);
    }
  }
}

// Reduce and evaluate in one launch for dense levels whose partial slots are
// feature-major ([16 features][bin_stride][g, h] per tile: hist_kernel's fmaj
// flush, so a feature's words in a slot are contiguous), for wide matrices
// (many workgroups per job, nodes of few chunks).  One wavefront per
// feature, four per 256-thread workgroup, lane l holding bins 4l .. 4l + 3 as
// evaluate_features_kernel<4> does: the lane sums the job's partial slots of
// its 64 contiguous bytes (or reads what the node's only chunk wrote), writes
// the built and sibling words (with store), and evaluates both nodes' feature
// from its registers -- the words and candidates of hist_reduce_kernel
// followed by evaluate_features_kernel<4>, with one launch and one pass over
// the level's histograms fewer.  Bins past bin_stride read the feature's last
// bin and are masked (branch-free loads).  No barriers.
constexpr int kDenseEvalFeatures = 4;  // features per workgroup (one per wavefront)
constexpr int64_t kDenseOneRound = 1024;  // four-wave reduce-evaluate workgroups 256 CUs hold at once
__global__ __launch_bounds__(64 * kDenseEvalFeatures) void reduce_evaluate_dense_kernel(
    const long long* __restrict__ partial, const HistReduce* __restrict__ jobs,
    int32_t n_jobs_host, const int32_t* __restrict__ n_jobs_dev, int32_t n_tiles,
    int32_t n_features, int32_t bin_stride, const long long* __restrict__ parent_base,
    long long* __restrict__ hist, const int32_t* __restrict__ n_bins,
    const long long* __restrict__ node_sums, const int32_t* __restrict__ exps, Param p,
    const uint32_t* __restrict__ fmask, const uint8_t* __restrict__ skip_bins,
    FeatCand* __restrict__ cand, int32_t store) {
  constexpr int BPL = 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int32_t f = int32_t(blockIdx.x) * kDenseEvalFeatures + wave;
  if (f >= n_features) return;  // wave-uniform; no barriers in this kernel
  const HistReduce j_first = int32_t(blockIdx.y) < n_jobs_host ? jobs[blockIdx.y] : HistReduce{};
  const int32_t n_jobs = n_jobs_dev ? *n_jobs_dev : n_jobs_host;
  const int32_t tile = f >> 4, fl = f & 15;
  const int64_t slot_words = int64_t(bin_stride) * 32;  // a tile's partial slot
  const int64_t node_elems = int64_t(n_features) * bin_stride * 2;
  bool ok[BPL];
  int64_t at[BPL], pat[BPL];  // word of bin (g; h is + 1): node histogram, partial slot
#pragma unroll
  for (int k = 0; k < BPL; ++k) {
    const int b = lane * BPL + k;
    ok[k] = b < bin_stride;
    const int bc = ok[k] ? b : bin_stride - 1;
    at[k] = (int64_t(f) * bin_stride + bc) * 2;
    pat[k] = (int64_t(fl) * bin_stride + bc) * 2;
  }
  const int nbf = n_bins[f];
  const int skip = skip_bins ? int(skip_bins[f]) : -1;
  const double ug = ldexp(1.0, -exps[0]), uh = ldexp(1.0, -exps[1]);
  auto evaluate = [&](const FeatBins<BPL>& d, int32_t node) {
    const long long gp = node_sums[2 * node], hp = node_sums[2 * node + 1];
    const double parent_gain = calc_gain(p, double(gp) * ug, double(hp) * uh);
    const int nb = feature_allowed(fmask, node, f, n_features) ? nbf : 0;
    const Cand c = feature_best<BPL>(d, f, nb, skip, gp, hp, parent_gain, ug, uh, p);
    if (lane == 0) cand[int64_t(node) * n_features + f] = FeatCand{c.loss, c.gl, c.hl, c.bin, c.dl};
  };
  for (int32_t jb = blockIdx.y; jb < n_jobs; jb += gridDim.y) {
    const HistReduce j = jb == int32_t(blockIdx.y) ? j_first : jobs[jb];
    const bool direct = j.nc == 1 && j.p0 < 0;  // uniform: the node's only chunk wrote it
    FeatBins<BPL> d;
    long long pg[BPL] = {}, ph[BPL] = {};
    if (j.sibling >= 0)  // uniform; issued first, used last
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        pg[k] = parent_base[j.parent + at[k]];
        ph[k] = parent_base[j.parent + at[k] + 1];
      }
    long long* built = hist + int64_t(j.slot) * node_elems;
    if (direct) {
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        const long long g = built[at[k]], h = built[at[k] + 1];
        d.g[k] = ok[k] ? g : 0;
        d.h[k] = ok[k] ? h : 0;
      }
    } else {
#pragma unroll
      for (int k = 0; k < BPL; ++k) d.g[k] = d.h[k] = 0;
      const long long* src = partial + (int64_t(j.p0) * n_tiles + tile) * slot_words;
      const int64_t step = int64_t(n_tiles) * slot_words;
      int32_t c = 0;
      for (; c + 2 <= j.nc; c += 2) {  // two slots' sixteen words in flight
        long long v[2][2 * BPL];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int k = 0; k < BPL; ++k) {
            v[u][2 * k] = src[(c + u) * step + pat[k]];
            v[u][2 * k + 1] = src[(c + u) * step + pat[k] + 1];
          }
#pragma unroll
        for (int k = 0; k < BPL; ++k) {
          d.g[k] += v[0][2 * k] + v[1][2 * k];
          d.h[k] += v[0][2 * k + 1] + v[1][2 * k + 1];
        }
      }
      if (c < j.nc)
#pragma unroll
        for (int k = 0; k < BPL; ++k) {
          d.g[k] += src[c * step + pat[k]];
          d.h[k] += src[c * step + pat[k] + 1];
        }
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        if (!ok[k]) d.g[k] = d.h[k] = 0;
        if (ok[k] && store) {
          built[at[k]] = d.g[k];
          built[at[k] + 1] = d.h[k];
        }
      }
    }
    evaluate(d, j.slot);
    if (j.sibling >= 0) {  // uniform
      long long* sib = hist + int64_t(j.sibling) * node_elems;
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        d.g[k] = ok[k] ? pg[k] - d.g[k] : 0;
        d.h[k] = ok[k] ? ph[k] - d.h[k] : 0;
        if (ok[k] && store) {
          sib[at[k]] = d.g[k];
          sib[at[k] + 1] = d.h[k];
        }
      }
      evaluate(d, j.sibling);
    }
  }
}

// Reduce and evaluate in one launch for dense levels whose partial slots are
// feature-major ([16 features][bin_stride][g, h] per tile: hist_kernel's fmaj
// flush, so a feature's words in a slot are contiguous), for narrower
// matrices (fewer workgroups per job, nodes of many chunks).  One 256-thread
// workgroup per (reduce job, feature); every lane holds bins 4l .. 4l + 3 of
// the feature, as evaluate_features_kernel<4> does.  Wavefront w sums the
// job's partial slots w, w + 4, ... of its lane's 64 contiguous bytes (or
// wavefront 0 reads what the node's only chunk wrote), the sums meet in LDS,
// and then wavefront 0 writes (with store) and evaluates the node while
// wavefront 1 derives, writes and evaluates the sibling from the parent's
// words -- the words and candidates of hist_reduce_kernel followed by
// evaluate_features_kernel<4>, with one launch and one pass over the level's
// histograms fewer.  Bins past bin_stride read the feature's last bin and are
// masked (branch-free loads).  W wavefronts per workgroup: 4, or 2 (the node
// and the sibling only) when the launch has more workgroups than the chip holds
// at once with four wavefronts each (the kernel's registers allow four
// wavefronts per SIMD, 1,024 such workgroups on 256 CUs): two-wave workgroups
// fit twice as many, and such levels have mostly one chunk per node (C2's last
// split level: 12.0 -> 10.0 us; with fewer workgroups two waves measured slower).
template <int W>
__global__ __launch_bounds__(64 * W) void reduce_evaluate_dense_split_kernel(
    const long long* __restrict__ partial, const HistReduce* __restrict__ jobs,
    int32_t n_jobs_host, const int32_t* __restrict__ n_jobs_dev, int32_t n_tiles,
    int32_t n_features, int32_t bin_stride, const long long* __restrict__ parent_base,
    long long* __restrict__ hist, const int32_t* __restrict__ n_bins,
    const long long* __restrict__ node_sums, const int32_t* __restrict__ exps, Param p,
    const uint32_t* __restrict__ fmask, const uint8_t* __restrict__ skip_bins,
    FeatCand* __restrict__ cand, int32_t store) {
  constexpr int BPL = 4;
  __shared__ long long part[W][2 * BPL][64];  // each wavefront's sums; [0] then the node's
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int32_t f = int32_t(blockIdx.x);
  const HistReduce j_first = int32_t(blockIdx.y) < n_jobs_host ? jobs[blockIdx.y] : HistReduce{};
  const int32_t n_jobs = n_jobs_dev ? *n_jobs_dev : n_jobs_host;
  const int32_t tile = f >> 4, fl = f & 15;
  const int64_t slot_words = int64_t(bin_stride) * 32;  // a tile's partial slot
  const int64_t node_elems = int64_t(n_features) * bin_stride * 2;
  bool ok[BPL];
  int64_t at[BPL], pat[BPL];  // word of bin (g; h is + 1): node histogram, partial slot
#pragma unroll
  for (int k = 0; k < BPL; ++k) {
    const int bn = lane * BPL + k;
    ok[k] = bn < bin_stride;
    const int bc = ok[k] ? bn : bin_stride - 1;
    at[k] = (int64_t(f) * bin_stride + bc) * 2;
    pat[k] = (int64_t(fl) * bin_stride + bc) * 2;
  }
  const int nbf = n_bins[f];
  const int skip = skip_bins ? int(skip_bins[f]) : -1;
  const double ug = ldexp(1.0, -exps[0]), uh = ldexp(1.0, -exps[1]);
  for (int32_t jb = blockIdx.y; jb < n_jobs; jb += gridDim.y) {
    const HistReduce j = jb == int32_t(blockIdx.y) ? j_first : jobs[jb];
    const bool direct = j.nc == 1 && j.p0 < 0;  // uniform: the node's only chunk wrote it
    long long s[2 * BPL] = {};                  // g, h of each bin: this wavefront's part
    long long pw[2 * BPL] = {};                 // wavefront 1: the parent's words
    if (wave == 1 && j.sibling >= 0)
#pragma unroll
      for (int k = 0; k < BPL; ++k) {
        pw[2 * k] = parent_base[j.parent + at[k]];
        pw[2 * k + 1] = parent_base[j.parent + at[k] + 1];
      }
    if (direct) {
      if (wave == 0) {
        const long long* built = hist + int64_t(j.slot) * node_elems;
#pragma unroll
        for (int k = 0; k < BPL; ++k) {
          s[2 * k] = built[at[k]];
          s[2 * k + 1] = built[at[k] + 1];
        }
      }
    } else {
      const long long* src = partial + (int64_t(j.p0) * n_tiles + tile) * slot_words;
      const int64_t step = int64_t(n_tiles) * slot_words;
      int32_t c = wave;
      for (; c + W < j.nc; c += 2 * W) {  // two of this wavefront's slots in flight
        long long v[2][2 * BPL];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int k = 0; k < BPL; ++k) {
            v[u][2 * k] = src[(c + u * W) * step + pat[k]];
            v[u][2 * k + 1] = src[(c + u * W) * step + pat[k] + 1];
          }
#pragma unroll
        for (int i = 0; i < 2 * BPL; ++i) s[i] += v[0][i] + v[1][i];
      }
      if (c < j.nc)
#pragma unroll
        for (int k = 0; k < BPL; ++k) {
          s[2 * k] += src[c * step + pat[k]];
          s[2 * k + 1] += src[c * step + pat[k] + 1];
        }
    }
#pragma unroll
    for (int i = 0; i < 2 * BPL; ++i) part[wave][i][lane] = s[i];
    __syncthreads();
    if (wave == 0) {  // the node: the four parts (one, for a direct node)
      if (!direct)
#pragma unroll
        for (int w = 1; w < W; ++w)
#pragma unroll
          for (int i = 0; i < 2 * BPL; ++i) s[i] += part[w][i][lane];
#pragma unroll
      for (int i = 0; i < 2 * BPL; ++i) part[0][i][lane] = s[i];
    }
    __syncthreads();
    if (wave <= 1) {
      const bool sib = wave == 1;
      if (!sib || j.sibling >= 0) {  // wavefront-uniform
        FeatBins<BPL> d;
#pragma unroll
        for (int k = 0; k < BPL; ++k) {
          const long long g = part[0][2 * k][lane], hh = part[0][2 * k + 1][lane];
          d.g[k] = !ok[k] ? 0 : (sib ? pw[2 * k] - g : g);
          d.h[k] = !ok[k] ? 0 : (sib ? pw[2 * k + 1] - hh : hh);
        }
        const int32_t node = sib ? j.sibling : j.slot;
        if (store && (sib || !direct)) {
          long long* o = hist + int64_t(node) * node_elems;
#pragma unroll
          for (int k = 0; k < BPL; ++k)
            if (ok[k]) {
              o[at[k]] = d.g[k];
              o[at[k] + 1] = d.h[k];
            }
        }
        const long long gp = node_sums[2 * node], hp = node_sums[2 * node + 1];
        const double parent_gain = calc_gain(p, double(gp) * ug, double(hp) * uh);
        const int nb = feature_allowed(fmask, node, f, n_features) ? nbf : 0;
        const Cand cd = feature_best<BPL>(d, f, nb, skip, gp, hp, parent_gain, ug, uh, p);
        if (lane == 0)
          cand[int64_t(node) * n_features + f] = FeatCand{cd.loss, cd.gl, cd.hl, cd.bin, cd.dl};
      }
    }
    __syncthreads();  // part is rewritten by the next job
  }
}

constexpr int kNodeWaves = 16;     // wavefronts per node in evaluate_nodes_kernel
constexpr int kNodeFeatures = kEvalNodeFeatures;  // feature counts up to this use evaluate_nodes_kernel

// Few features: one workgroup per node (looping over nodes); wavefront w
// scans features w, w + 16, ..., keeps its best, and the workgroup's best is
// the node's split record -- the whole evaluation in one launch.
template <int BPL>
__global__ __launch_bounds__(64 * kNodeWaves) void evaluate_nodes_kernel(
    const long long* __restrict__ hist, int32_t n_nodes_host,
    const int32_t* __restrict__ n_nodes_dev, int32_t n_features, int32_t bin_stride,
    const int32_t* __restrict__ n_bins, const long long* __restrict__ node_sums,
    const int32_t* __restrict__ exps, int32_t exp_g_host, int32_t exp_h_host, Param p,
    const uint32_t* __restrict__ fmask, const uint8_t* __restrict__ skip_bins,
    dp_split_record* __restrict__ out) {
  __shared__ Cand wave_best[kNodeWaves];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int32_t n_nodes = n_nodes_dev ? *n_nodes_dev : n_nodes_host;
  const int exp_g = exps ? exps[0] : exp_g_host;
  const int exp_h = exps ? exps[1] : exp_h_host;
  const double ug = ldexp(1.0, -exp_g), uh = ldexp(1.0, -exp_h);
  for (int32_t node = blockIdx.x; node < n_nodes; node += gridDim.x) {
    // The wave's next feature is loaded while the current one is evaluated.
    FeatBins<BPL> cur, nxt;
    if (wave < n_features) load_feature<BPL>(hist, node, wave, n_features, bin_stride, cur);
    const long long gp = node_sums[2 * node], hp = node_sums[2 * node + 1];
    const double parent_gain = calc_gain(p, double(gp) * ug, double(hp) * uh);
    Cand best;
    best.loss = -INFINITY;
    best.gl = best.hl = 0;
    best.feature = -1;
    best.bin = -1;
    best.dl = 0;
    for (int32_t f = wave; f < n_features; f += kNodeWaves) {  // wave-uniform
      if (f + kNodeWaves < n_features)
        load_feature<BPL>(hist, node, f + kNodeWaves, n_features, bin_stride, nxt);
      const int nb = feature_allowed(fmask, node, f, n_features) ? n_bins[f] : 0;
      const int skip = skip_bins ? int(skip_bins[f]) : -1;
      const Cand c = feature_best<BPL>(cur, f, nb, skip, gp, hp, parent_gain, ug, uh, p);
      if (c.loss > -INFINITY && better(c, best)) best = c;
      cur = nxt;
    }
    if (lane == 0) wave_best[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
      Cand r = wave_best[0];
      for (int k = 1; k < kNodeWaves; ++k)
        if (better(wave_best[k], r)) r = wave_best[k];
      out[node] = make_record(r, p.gamma);
    }
    __syncthreads();  // wave_best is reused by the next node
  }
}

// ---- column sampling (the draws are defined in sample.hpp) ---------------
constexpr int kColThreads = 256;

// The nth smallest key (nth >= 1, at most the candidate count) among the
// features cand(f) admits: radix selection, eight bits at a time from the top,
// one LDS histogram of the digit per pass.  Keys are distinct, so the result
// is exactly the key of the nth candidate in key order.  Every thread of the
// workgroup calls it and gets the same result.
template <class Cand, class Key>
__device__ uint32_t select_nth_key(int32_t n_features, uint32_t nth, Cand cand, Key key,
                                   uint32_t* hist, uint32_t* pick) {
  const int lane = threadIdx.x & 63;
  uint32_t prefix = 0, pmask = 0, need = nth;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += kColThreads) hist[i] = 0;
    __syncthreads();
    for (int32_t f = threadIdx.x; f < n_features; f += kColThreads) {
      if (!cand(f)) continue;
      const uint32_t k = key(f);
      if ((k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (threadIdx.x < 64) {  // lane l holds digits 4l .. 4l + 3
      uint32_t c[4], tot = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = hist[4 * lane + j];
        tot += c[j];
      }
      uint32_t incl = tot;
      for (int d = 1; d < 64; d <<= 1) {
        const uint32_t v = __shfl_up(incl, d, 64);
        if (lane >= d) incl += v;
      }
      const uint32_t excl = incl - tot;
      if (excl < need && need <= incl) {  // exactly one lane holds the digit
        uint32_t run = excl;
        for (int j = 0; j < 4; ++j) {
          if (run + c[j] >= need) {
            pick[0] = uint32_t(4 * lane + j);
            pick[1] = need - run;
            break;
          }
          run += c[j];
        }
      }
    }
    __syncthreads();
    prefix |= pick[0] << shift;
    pmask |= 0xffu << shift;
    need = pick[1];
    __syncthreads();  // pick and hist are rewritten by the next pass
  }
  return prefix;
}

// One workgroup per node of the level (looping over nodes): the node's
// feature sample as a bit mask, masks[node][ceil(F / 32)].  The tree and level
// stages are the same for every node of the level; each workgroup selects
// them once, then the node stage per node.
__global__ __launch_bounds__(kColThreads) void colsample_kernel(
    const LevelNode* __restrict__ nodes, int32_t n_host, const int32_t* __restrict__ n_dev,
    int32_t n_features, ColSample cs, int32_t depth, uint32_t* __restrict__ masks) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t pick[2];
  const int32_t n_nodes = n_dev ? *n_dev : n_host;
  if (int32_t(blockIdx.x) >= n_nodes) return;  // uniform per workgroup
  const int lane = threadIdx.x & 63;
  const uint64_t round = uint64_t(uint32_t(*cs.round));
  const uint64_t out = uint64_t(uint32_t(cs.output)) << 32;
  const int fbits = feature_bits(n_features);
  const uint64_t p_tree = sample_prefix(cs.seed, kTreeStream, round, out);
  const uint64_t p_level = sample_prefix(cs.seed, kLevelStream, round, out | uint32_t(depth));
  const int32_t n1 = stage_keep(cs.bytree, n_features);
  const int32_t n2 = stage_keep(cs.bylevel, n1);
  const int32_t n3 = stage_keep(cs.bynode, n2);
  auto all = [](int32_t) { return true; };
  const uint32_t t1 =
      n1 < n_features
          ? select_nth_key(n_features, uint32_t(n1), all,
                           [&](int32_t f) { return feature_key(p_tree, f, fbits); }, hist, pick)
          : 0xffffffffu;
  auto in_tree = [&](int32_t f) { return feature_key(p_tree, f, fbits) <= t1; };
  const uint32_t t2 =
      n2 < n1 ? select_nth_key(n_features, uint32_t(n2), in_tree,
                               [&](int32_t f) { return feature_key(p_level, f, fbits); }, hist,
                               pick)
              : 0xffffffffu;
  auto in_level = [&](int32_t f) { return in_tree(f) && feature_key(p_level, f, fbits) <= t2; };
  const int64_t words = (n_features + 31) / 32;
  for (int32_t node = blockIdx.x; node < n_nodes; node += gridDim.x) {
    const uint64_t p_node =
        sample_prefix(cs.seed, kNodeStream, round, out | uint32_t(nodes[node].nid));
    const uint32_t t3 =
        n3 < n2 ? select_nth_key(n_features, uint32_t(n3), in_level,
                                 [&](int32_t f) { return feature_key(p_node, f, fbits); }, hist,
                                 pick)
                : 0xffffffffu;
    uint32_t* m = masks + int64_t(node) * words;
    for (int32_t base = int32_t(threadIdx.x >> 6) * 64; base < n_features; base += kColThreads) {
      const int32_t f = base + lane;
      const bool in = f < n_features && in_level(f) && feature_key(p_node, f, fbits) <= t3;
      const unsigned long long b = __ballot(in);
      if (lane == 0) {
        m[base >> 5] = uint32_t(b);
        if ((base >> 5) + 1 < words) m[(base >> 5) + 1] = uint32_t(b >> 32);
      }
    }
  }
}

constexpr int kSelectThreads = 256;

// One workgroup per node (looping over nodes): argmax over the node's feature
// candidates with ties to the lowest feature, then the split record.
__global__ __launch_bounds__(kSelectThreads) void select_splits_kernel(
    const FeatCand* __restrict__ cand, int32_t n_nodes_host,
    const int32_t* __restrict__ n_nodes_dev, int32_t n_features, double gamma,
    dp_split_record* __restrict__ out) {
  __shared__ Cand wave_best[kSelectThreads / 64];
  __shared__ dp_split_record rec;
  const int32_t n_nodes = n_nodes_dev ? *n_nodes_dev : n_nodes_host;
  for (int32_t node = blockIdx.x; node < n_nodes; node += gridDim.x) {
    const dp_split_record r =
        select_node<kSelectThreads>(cand, node, n_features, gamma, wave_best, &rec);
    if (threadIdx.x == 0) out[node] = r;
  }
}

}  // namespace

size_t evaluate_scratch_bytes(int32_t n_nodes, int32_t n_features) {
  return sizeof(FeatCand) * size_t(n_nodes > 0 ? n_nodes : 0) * size_t(n_features);
}

bool launch_evaluate(const int64_t* hist, int32_t n_nodes, const int32_t* n_nodes_dev,
                     int32_t n_features, int32_t bin_stride, const int32_t* n_bins,
                     const int64_t* node_sums, const int32_t* exps, int32_t exp_g, int32_t exp_h,
                     const dp_train_param& param, void* scratch, dp_split_record* out,
                     hipStream_t s, bool select, const uint32_t* fmask,
                     const uint8_t* skip_bins) {
  if (n_nodes <= 0) return true;
  need(bin_stride >= 1 && bin_stride <= kMaxBins, "split bin stride out of range");
  need(n_features >= 1, "split evaluation needs at least one feature");
  Param p{double(param.lambda), double(param.alpha), double(param.min_child_weight),
          double(param.gamma)};
  const auto* h = reinterpret_cast<const long long*>(hist);
  const auto* sums = reinterpret_cast<const long long*>(node_sums);
  if (n_features <= kNodeFeatures) {
    const dim3 grid(n_nodes < 2048 ? n_nodes : 2048), block(64 * kNodeWaves);
    if (bin_stride <= 64)
      hipLaunchKernelGGL(evaluate_nodes_kernel<1>, grid, block, 0, s, h, n_nodes, n_nodes_dev,
                         n_features, bin_stride, n_bins, sums, exps, exp_g, exp_h, p, fmask, skip_bins, out);
    else if (bin_stride <= 128)
      hipLaunchKernelGGL(evaluate_nodes_kernel<2>, grid, block, 0, s, h, n_nodes, n_nodes_dev,
                         n_features, bin_stride, n_bins, sums, exps, exp_g, exp_h, p, fmask, skip_bins, out);
    else
      hipLaunchKernelGGL(evaluate_nodes_kernel<4>, grid, block, 0, s, h, n_nodes, n_nodes_dev,
                         n_features, bin_stride, n_bins, sums, exps, exp_g, exp_h, p, fmask, skip_bins, out);
    DP_HIP(hipGetLastError());
    return true;
  }
  auto* cand = static_cast<FeatCand*>(scratch);
  if (bin_stride <= 64) {
    const int64_t items = int64_t(n_nodes) * ((n_features + kSegFeatures - 1) / kSegFeatures);
    hipLaunchKernelGGL(evaluate_features_seg_kernel, dim3(items < 2048 ? items : 2048), dim3(256),
                       0, s, h, n_nodes, n_nodes_dev, n_features, bin_stride, n_bins, sums, exps,
                       exp_g, exp_h, p, fmask, skip_bins, cand);
    DP_HIP(hipGetLastError());
    if (!select) return false;
    hipLaunchKernelGGL(select_splits_kernel, dim3(n_nodes < 1024 ? n_nodes : 1024),
                       dim3(kSelectThreads), 0, s, cand, n_nodes, n_nodes_dev, n_features,
                       double(param.gamma), out);
    DP_HIP(hipGetLastError());
    return true;
  }
  const int64_t groups = (n_features + kFeatWaves - 1) / kFeatWaves;
  const int64_t items = int64_t(n_nodes) * groups;
  const int grid = int(items < 2048 ? items : 2048);
  const dim3 block(64 * kFeatWaves);
  if (bin_stride <= 128)
    hipLaunchKernelGGL(evaluate_features_kernel<2>, dim3(grid), block, 0, s, h, n_nodes,
                       n_nodes_dev, n_features, bin_stride, n_bins, sums, exps, exp_g, exp_h, p,
                       fmask, skip_bins, cand);
  else
    hipLaunchKernelGGL(evaluate_features_kernel<4>, dim3(grid), block, 0, s, h, n_nodes,
                       n_nodes_dev, n_features, bin_stride, n_bins, sums, exps, exp_g, exp_h, p,
                       fmask, skip_bins, cand);
  DP_HIP(hipGetLastError());
  if (!select) return false;
  hipLaunchKernelGGL(select_splits_kernel, dim3(n_nodes < 1024 ? n_nodes : 1024),
                     dim3(kSelectThreads), 0, s, cand, n_nodes, n_nodes_dev, n_features,
                     double(param.gamma), out);
  DP_HIP(hipGetLastError());
  return true;
}

void launch_reduce_evaluate_flat(const int64_t* partial, const HistReduce* jobs, int32_t n_jobs,
                                 const int32_t* n_jobs_dev, int32_t n_tiles, int32_t tile_features,
                                 int32_t n_features, int32_t bin_stride,
                                 const int64_t* parent_base, int64_t* hist, const int32_t* n_bins,
                                 const int64_t* node_sums, const int32_t* exps,
                                 const dp_train_param& param, const uint32_t* fmask,
                                 const uint8_t* skip_bins, void* scratch, bool store,
                                 hipStream_t s, bool skip_direct) {
  if (n_jobs <= 0) return;
  need(bin_stride >= 1 && bin_stride <= 64, "the present-value reduce-evaluate takes <= 64 bins");
  need(tile_features >= kSegFeatures && tile_features % kSegFeatures == 0,
       "present-value tiles must hold whole groups of 16 features");
  need(n_tiles == (n_features + tile_features - 1) / tile_features, "tile count");
  need(exps && scratch, "reduce-evaluate needs the quantiser exponents and candidate scratch");
  Param p{double(param.lambda), double(param.alpha), double(param.min_child_weight),
          double(param.gamma)};
  const dim3 grid(unsigned((n_features + kSegFeatures - 1) / kSegFeatures),
                  unsigned(n_jobs < 256 ? n_jobs : 256));
  hipLaunchKernelGGL(reduce_evaluate_flat_kernel, grid, dim3(256), 0, s,
                     reinterpret_cast<const long long*>(partial), jobs, n_jobs, n_jobs_dev,
                     n_tiles, tile_features, n_features, bin_stride,
                     reinterpret_cast<const long long*>(parent_base),
                     reinterpret_cast<long long*>(hist), n_bins,
                     reinterpret_cast<const long long*>(node_sums), exps, p, fmask, skip_bins,
                     static_cast<FeatCand*>(scratch), store ? 1 : 0,
                     skip_direct ? 1 : 0);
  DP_HIP(hipGetLastError());
}

void launch_reduce_evaluate_dense(const int64_t* partial, const HistReduce* jobs, int32_t n_jobs,
                                  const int32_t* n_jobs_dev, int32_t n_tiles, int32_t n_features,
                                  int32_t bin_stride, const int64_t* parent_base, int64_t* hist,
                                  const int32_t* n_bins, const int64_t* node_sums,
                                  const int32_t* exps, const dp_train_param& param,
                                  const uint32_t* fmask, const uint8_t* skip_bins, void* scratch,
                                  bool store, hipStream_t s) {
  if (n_jobs <= 0 || n_features <= 0) return;
  need(bin_stride >= 1 && bin_stride <= 64 * 4, "dense reduce-evaluate needs at most 256 bins");
  need(exps && scratch && n_bins && node_sums,
       "reduce-evaluate needs the quantiser exponents, the bin counts and candidate scratch");
  Param p{double(param.lambda), double(param.alpha), double(param.min_child_weight),
          double(param.gamma)};
  // Wide matrices: four features per workgroup, each wavefront summing its
  // feature's slots alone; narrower ones: a workgroup per feature whose
  // wavefronts split the slots and evaluate the node and the sibling at once
  // (two wavefronts when the grid exceeds kDenseOneRound four-wave workgroups).
  const bool wide = n_features >= kDenseWideFeatures;
  const bool many = !wide && int64_t(n_features) * std::min(n_jobs, 256) > kDenseOneRound;
  const dim3 grid(unsigned(wide ? (n_features + kDenseEvalFeatures - 1) / kDenseEvalFeatures
                                : n_features),
                  unsigned(n_jobs < 256 ? n_jobs : 256));
  hipLaunchKernelGGL(wide   ? reduce_evaluate_dense_kernel
                     : many ? reduce_evaluate_dense_split_kernel<2>
                            : reduce_evaluate_dense_split_kernel<4>,
                     grid, dim3(many ? 128 : 256), 0, s,
                     reinterpret_cast<const long long*>(partial), jobs, n_jobs, n_jobs_dev,
                     n_tiles, n_features, bin_stride,
                     reinterpret_cast<const long long*>(parent_base),
                     reinterpret_cast<long long*>(hist), n_bins,
                     reinterpret_cast<const long long*>(node_sums), exps, p, fmask, skip_bins,
                     static_cast<FeatCand*>(scratch), store ? 1 : 0);
  DP_HIP(hipGetLastError());
}

void launch_colsample(const LevelNode* nodes, int32_t n_host, const int32_t* n_dev,
                      int32_t n_features, const ColSample& cs, int32_t depth, uint32_t* masks,
                      hipStream_t s) {
  if (n_host <= 0 || !cs.active()) return;
  need(n_features >= 1, "column sampling needs at least one feature");
  need(cs.round != nullptr, "column sampling needs the device round index");
  const int grid = n_host < 2048 ? n_host : 2048;
  hipLaunchKernelGGL(colsample_kernel, dim3(grid), dim3(kColThreads), 0, s, nodes, n_host, n_dev,
                     n_features, cs, depth, masks);
  DP_HIP(hipGetLastError());
}

}  // namespace dp
