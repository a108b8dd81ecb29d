// Split gains and the four-features-per-wavefront evaluation, shared by the
// evaluation kernels (split.hip) and by the present-value histogram pass
// (hist.hip), which evaluates the nodes it builds in one chunk straight from
// LDS.  Semantics (upstream CalcGain with max_delta_step 0, reached in the
// reference only through XGBoosterUpdateOneIter,
// class_native_training.cuh:67): T(G) = sign(G) max(|G| - alpha, 0),
// gain(G, H) = T(G)^2 / (H + lambda), 0 when H < min_child_weight or H <= 0;
// loss = (gain(L) + gain(R)) - gain(P) in double, compiled without
// contraction so every value rounds as the CPU restatement computes it.
#pragma once

#include "dp_internal.hpp"
#include "select.hpp"

#include <cmath>

namespace dp {

struct Param {
  double lambda, alpha, mcw, gamma;
};

// The three functions below are branch-free: every value is computed and the
// refused cases are selected afterwards, so a wavefront's bins form one block of
// straight-line code whose divisions the compiler can interleave.  A selected
// value is the one the branching form returns, bit for bit.
__device__ __forceinline__ double threshold_l1(double g, double alpha) {
  const double up = g - alpha, down = g + alpha;
  return g > alpha ? up : (g < -alpha ? down : 0.0);
}

__device__ __forceinline__ double calc_gain(const Param& p, double g, double h) {
  const double t = threshold_l1(g, p.alpha);
  const double q = (t * t) / (h + p.lambda);
  return (h < p.mcw || h <= 0.0) ? 0.0 : q;
}

__device__ __forceinline__ double split_loss(const Param& p, long long qgl, long long qhl,
                                             long long qgr, long long qhr, double ug, double uh,
                                             double parent_gain) {
  const double gl = double(qgl) * ug, hl = double(qhl) * uh;
  const double gr = double(qgr) * ug, hr = double(qhr) * uh;
  const double loss = (calc_gain(p, gl, hl) + calc_gain(p, gr, hr)) - parent_gain;
  return (qhl <= 0 || qhr <= 0 || hl < p.mcw || hr < p.mcw) ? -INFINITY : loss;
}

// The best of a lane's BPL bins, in increasing bin order (ties keep the
// lower): bin b0 + j has left sums (lg[j], lh[j]) and exists where bit j of
// `in` is set; the node's rows the bins do not hold are (mg, mh).  Each bin's
// loss is the better of missing right and missing left (the two are one
// candidate, and compute to the same bits, without missing rows; when no lane
// has any, the second is skipped).  Straight-line code, so that the bins'
// divisions interleave -- or, with SERIAL, one bin after the other behind a
// branch each, which holds fewer registers at once.
template <int BPL, bool SERIAL = false>
__device__ __forceinline__ void best_of_bins(const long long (&lg)[BPL], const long long (&lh)[BPL],
                                             int in, int b0, long long mg, long long mh,
                                             long long gp, long long hp, double ug, double uh,
                                             double parent_gain, const Param& p, Cand& c) {
  auto fold = [&](int j, double l, int d) {
    const bool take = ((in >> j) & 1) && l > c.loss;
    c.loss = take ? l : c.loss;
    c.bin = take ? b0 + j : c.bin;
    c.dl = take ? d : c.dl;
    c.gl = take ? (d ? lg[j] + mg : lg[j]) : c.gl;
    c.hl = take ? (d ? lh[j] + mh : lh[j]) : c.hl;
  };
  if constexpr (SERIAL) {
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
      if ((in >> j) & 1) {
        const double right_missing =
            split_loss(p, lg[j], lh[j], gp - lg[j], hp - lh[j], ug, uh, parent_gain);
        const double left_missing =
            (mg == 0 && mh == 0) ? right_missing
                                 : split_loss(p, lg[j] + mg, lh[j] + mh, gp - lg[j] - mg,
                                              hp - lh[j] - mh, ug, uh, parent_gain);
        const int d = left_missing > right_missing;
        fold(j, d ? left_missing : right_missing, d);
      }
    }
  } else if (__ballot(mg != 0 || mh != 0)) {  // uniform
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
      const double right_missing =
          split_loss(p, lg[j], lh[j], gp - lg[j], hp - lh[j], ug, uh, parent_gain);
      const double left_missing = split_loss(p, lg[j] + mg, lh[j] + mh, gp - lg[j] - mg,
                                             hp - lh[j] - mh, ug, uh, parent_gain);
      const int d = left_missing > right_missing;
      fold(j, d ? left_missing : right_missing, d);
    }
  } else {
#pragma unroll
    for (int j = 0; j < BPL; ++j)
      fold(j, split_loss(p, lg[j], lh[j], gp - lg[j], hp - lh[j], ug, uh, parent_gain), 0);
  }
}

// Column sampling: fmask holds one bit per feature for every node of the
// level ([node][ceil(F / 32)] words); null when every feature is a candidate.
__device__ __forceinline__ bool feature_allowed(const uint32_t* __restrict__ fmask, int32_t node,
                                                int32_t f, int32_t n_features) {
  if (!fmask) return true;
  const int64_t words = (n_features + 31) / 32;
  return (fmask[int64_t(node) * words + (f >> 5)] >> (f & 31)) & 1u;
}

__device__ __forceinline__ double dpp_f64_bits(long long bits) { return __longlong_as_double(bits); }

// Four features per wavefront (seg_evaluate): 16 per 256-thread workgroup.
constexpr int kSegFeatures = 16;

__device__ __forceinline__ long long row_shuffle64(long long v, int src) {
  const int lo = __shfl(int(v), src, 64);
  const int hi = __shfl(int(v >> 32), src, 64);
  return (long long)((uint64_t(uint32_t(hi)) << 32) | uint32_t(lo));
}

// Scratch of the compacted evaluation in seg_evaluate, per wavefront: 64 slots
// of (left g, left h) and the four rows' missing sums (g, h).  16-byte aligned.
constexpr int kSegScratchWords = 2 * 64 + 2 * 4;

// The evaluation of four features per wavefront, one per 16-lane row, four bins
// per lane (bins 4 * (lane % 16) + j in dg, dh): the row's prefix scan and
// argmax take the row_shr steps of the full-wave ones; the row total and the
// winner's fields come by lane permutes.  Same per-bin arithmetic and tie rule
// as feature_best, with a quarter of the wavefronts and of their fixed costs.
// The row's first lane writes feature f's best candidate of `node` (live: the
// row's feature exists; every lane takes part in the row steps).
//
// Empty bins.  A bin b > 0 whose (g, h) words are both zero, and which is not
// the skipped bin, has the left sums of bin b - 1, so its candidate's loss is
// bit for bit that of bin b - 1: with the larger loss winning and ties going
// to the lower bin, it can never be the feature's pick, nor change which lane
// holds the pick.  Only the other bins are needed.  When a wavefront's needed
// bins number at most 64 (a node of few rows: most bins are empty), they are
// packed into consecutive lanes through the per-wavefront LDS scratch `scr`
// (kSegScratchWords words; nullptr: never), their losses are computed there,
// one candidate per lane instead of four bins per lane, and each returns to
// its bin; the empty bins are not candidates.  The gains, and so every pick,
// are those of the in-place evaluation of all bins.  (Packing into two rounds
// of 64 was measured slower than the in-place evaluation.)
template <bool SERIAL = false>
__device__ __forceinline__ void seg_evaluate(const long long (&dg)[4], const long long (&dh)[4],
                                             int32_t node, int32_t f, bool live,
                                             int32_t n_features, const int32_t* __restrict__ n_bins,
                                             const long long* __restrict__ node_sums, double ug,
                                             double uh, const Param& p,
                                             const uint32_t* __restrict__ fmask,
                                             const uint8_t* __restrict__ skip_bins,
                                             FeatCand* __restrict__ cand,
                                             long long* __restrict__ scr = nullptr) {
  constexpr int BPL = 4;
  const int lane = threadIdx.x & 63;
  const int seg = lane >> 4, sub = lane & 15;
  const int row_last = lane | 15;
  const int nb = live && feature_allowed(fmask, node, f, n_features) ? n_bins[f] : 0;
  const long long gp = node_sums[2 * node], hp = node_sums[2 * node + 1];
  const double parent_gain = calc_gain(p, double(gp) * ug, double(hp) * uh);
  long long sg[BPL], sh[BPL];
  long long rg = 0, rh = 0;
#pragma unroll
  for (int j = 0; j < BPL; ++j) {
    rg += dg[j];
    rh += dh[j];
    sg[j] = rg;
    sh[j] = rh;
  }
  // inclusive scan of the lane totals within the 16-lane row
  long long ig = rg, ih = rh;
  ig += dpp64<0x111>(ig, 0);
  ih += dpp64<0x111>(ih, 0);
  ig += dpp64<0x112>(ig, 0);
  ih += dpp64<0x112>(ih, 0);
  ig += dpp64<0x114>(ig, 0);
  ih += dpp64<0x114>(ih, 0);
  ig += dpp64<0x118>(ig, 0);
  ih += dpp64<0x118>(ih, 0);
  const long long total_g = row_shuffle64(ig, row_last), total_h = row_shuffle64(ih, row_last);
  const long long og = ig - rg, oh = ih - rh;
  // as feature_best: a skipped bin's rows return at the prefixes from that bin
  const int skip = live && skip_bins ? int(skip_bins[f]) : -1;
  long long mg = gp - total_g, mh = hp - total_h, kg = 0, kh = 0;
  if (skip >= 0) {
    kg = mg;
    kh = mh;
    mg = mh = 0;
  }
  // Left sums of the lane's bins, and which bins exist (in) and are needed
  // (above), one bit per bin.
  long long lg[BPL], lh[BPL];
  int in = 0, need = 0;
#pragma unroll
  for (int j = 0; j < BPL; ++j) {
    const int b = sub * BPL + j;
    lg[j] = og + sg[j] + (b >= skip && skip >= 0 ? kg : 0);
    lh[j] = oh + sh[j] + (b >= skip && skip >= 0 ? kh : 0);
    if (b < nb) {
      in |= 1 << j;
      if (b == 0 || b == skip || dg[j] != 0 || dh[j] != 0) need |= 1 << j;
    }
  }
  // The lane's best bin, taken in increasing bin order (ties keep the lower).
  Cand c;
  c.loss = -INFINITY;
  c.gl = c.hl = 0;
  c.feature = f;
  c.bin = -1;
  c.dl = 0;
  // Lane-order slots of the needed bins: a lane has fewer than 8, so three
  // bit ballots of its count give the exclusive prefix over the lanes.
  unsigned long long c0 = 0, c1 = 0, c2 = 0;
  int n_need = 65;
  if (scr) {
    const int cnt = __popc(need);
    c0 = __ballot(cnt & 1);
    c1 = __ballot(cnt & 2);
    c2 = __ballot(cnt & 4);
    n_need = __popcll(c0) + 2 * __popcll(c1) + 4 * __popcll(c2);
  }
  if (n_need <= 64) {  // uniform per wavefront: one candidate per lane
    const unsigned long long below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const int base = __popcll(c0 & below) + 2 * __popcll(c1 & below) + 4 * __popcll(c2 & below);
    // Slots of row r start at lane 16 r's base; each row's missing sums sit
    // after the 64 slots.
    const int r1 = __builtin_amdgcn_readlane(base, 16), r2 = __builtin_amdgcn_readlane(base, 32),
              r3 = __builtin_amdgcn_readlane(base, 48);
    if (sub == 0) {
      scr[128 + 2 * seg] = mg;
      scr[128 + 2 * seg + 1] = mh;
    }
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
      const int slot = base + __popc(need & ((1 << j) - 1));
      if ((need >> j) & 1) {
        scr[2 * slot] = lg[j];
        scr[2 * slot + 1] = lh[j];
      }
    }
    __builtin_amdgcn_wave_barrier();
    double l = -INFINITY;
    int d = 0;
    if (lane < n_need) {
      const int r = (lane >= r1 ? 1 : 0) + (lane >= r2 ? 1 : 0) + (lane >= r3 ? 1 : 0);
      const long long xg = scr[2 * lane], xh = scr[2 * lane + 1];
      const long long yg = scr[128 + 2 * r], yh = scr[128 + 2 * r + 1];
      const double right_missing = split_loss(p, xg, xh, gp - xg, hp - xh, ug, uh, parent_gain);
      const double left_missing =
          split_loss(p, xg + yg, xh + yh, gp - xg - yg, hp - xh - yh, ug, uh, parent_gain);
      d = left_missing > right_missing;
      l = d ? left_missing : right_missing;
    }
    const unsigned long long dmask = __ballot(d);
    __builtin_amdgcn_wave_barrier();
    // the slots' (g, h) have been read: their first 64 words take the losses
    if (lane < n_need) scr[lane] = __double_as_longlong(l);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
      const int slot = base + __popc(need & ((1 << j) - 1));
      if ((need >> j) & 1) {
        const double l = __longlong_as_double(scr[slot]);
        const int d = int((dmask >> slot) & 1ull);
        if (l > c.loss) {
          c.loss = l;
          c.bin = sub * BPL + j;
          c.dl = d;
          c.gl = d ? lg[j] + mg : lg[j];
          c.hl = d ? lh[j] + mh : lh[j];
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // the next call rewrites the scratch
  } else if (__ballot(in != 0)) {  // uniform: some row's feature has bins
    best_of_bins<BPL, SERIAL>(lg, lh, in, sub * BPL, mg, mh, gp, hp, ug, uh, parent_gain, p, c);
  }
  // Row argmax: the largest loss, then the lowest lane holding it (lanes hold
  // increasing bins and each kept its lowest bin on ties).
  long long bb = __double_as_longlong(c.loss);
  auto step = [&](long long o) {
    if (dpp_f64_bits(o) > dpp_f64_bits(bb)) bb = o;
  };
  step(dpp64<0x111>(bb, bb));
  step(dpp64<0x112>(bb, bb));
  step(dpp64<0x114>(bb, bb));
  step(dpp64<0x118>(bb, bb));
  const double best = dpp_f64_bits(row_shuffle64(bb, row_last));
  const unsigned long long hit = __ballot(c.loss == best);
  const int winner = seg * 16 + __builtin_ctzll((hit >> (seg * 16)) & 0xffffull);
  const long long w_gl = row_shuffle64(c.gl, winner), w_hl = row_shuffle64(c.hl, winner);
  const int w_bin = __shfl(c.bin, winner, 64), w_dl = __shfl(c.dl, winner, 64);
  if (live && sub == 0)
    cand[int64_t(node) * n_features + f] = FeatCand{best, w_gl, w_hl, w_bin, w_dl};
}

}  // namespace dp
