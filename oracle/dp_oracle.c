/*
 * dp_oracle.c -- CPU restatement of the training hot path.  TEST
 * INFRASTRUCTURE ONLY: the product library never links or calls it.
 *
 * The path is XGBoost 3.4.1 `grow_gpu_hist` as reached from the reference's
 * trainer (native/class_native_training.cuh:47-70, native/class_model_train.cu:48).
 * Where upstream behaviour cannot be checked here (its library is absent) the
 * choice made is stated at the function that makes it.  Every function below is
 * pinned by tests/test_oracle.py against numpy closed forms, brute force or the
 * reference's fixtures; see the header of each test for what it pins.
 *
 * Compile with -ffp-contract=off: every float/double operation here must round
 * exactly as written so the GPU path (built with the same flag) matches bit for
 * bit.
 */
#include "dp_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Threads of the parallel loops below (dpo_set_threads; 1 = serial).  Every */
/* parallel result is identical to the serial one: sums are exact integers, */
/* and every reduction runs in a fixed order.                                */
static int g_threads = 1;

void dpo_set_threads(int32_t n) { g_threads = n > 0 ? n : 1; }
int32_t dpo_get_threads(void) { return g_threads; }

/* Threads for `work` items of which each thread should get at least `grain`. */
static int threads_for(int64_t work, int64_t grain) {
#ifdef _OPENMP
  int64_t t = work / (grain > 0 ? grain : 1);
  if (t > g_threads) t = g_threads;
  return t < 1 ? 1 : (int)t;
#else
  (void)work;
  (void)grain;
  return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* Quantile cuts.                                                            */
/*                                                                           */
/* Upstream builds cuts with a weighted quantile sketch at DMatrix creation  */
/* (XGDMatrixCreateFromCudaArrayInterface, class_native_training.cuh:51).    */
/* This build fixes an exact, order-free definition instead:                 */
/*   v = sorted non-missing values of the feature (-0.0 folded into +0.0),   */
/*   u = distinct values of v, m = |u|;                                      */
/*   m <= max_bin : cuts = u[1..m-1] followed by `last`                      */
/*   m >  max_bin : cuts = strictly increasing subsequence of                */
/*                  v[floor(i*n/max_bin)], i = 1..max_bin-1, each > u[0],    */
/*                  followed by `last`                                       */
/*   last = max + (|max| + 1e-5f)   (upstream's end-cut rule);               */
/*   an all-missing feature gets the single cut 1e-5f.                       */
/* bin(x) = index of the first cut > x, clamped to the last bin; so          */
/* x < cut[b]  <=>  bin(x) <= b, which is what split_conditions encode       */
/* (routing rule of native/class_native_source_contract.hpp:26).             */
/* ------------------------------------------------------------------------ */
static int cmp_float(const void* a, const void* b) {
  float x = *(const float*)a, y = *(const float*)b;
  return (x > y) - (x < y);
}

static float end_cut(float max_value) { return max_value + (fabsf(max_value) + 1e-5f); }

/* Cuts of feature f into out (at most max_bin values); returns their count. */
static int32_t feature_cuts(const float* x, int64_t n, int64_t n_features, int64_t f,
                            int32_t max_bin, float* v, float* out, float* min_value) {
  int32_t count = 0;
  int64_t m_valid = 0;
  for (int64_t r = 0; r < n; ++r) {
    float value = x[r * n_features + f];
    if (isnan(value)) continue;
    v[m_valid++] = value == 0.0f ? 0.0f : value;
  }
  if (m_valid == 0) {
    out[count++] = end_cut(0.0f);
    *min_value = 0.0f;
    return count;
  }
  qsort(v, (size_t)m_valid, sizeof(float), cmp_float);
  int64_t distinct = 1;
  for (int64_t i = 1; i < m_valid; ++i) distinct += v[i] != v[i - 1];
  *min_value = v[0];
  if (distinct <= max_bin) {
    for (int64_t i = 1; i < m_valid; ++i)
      if (v[i] != v[i - 1]) out[count++] = v[i];
  } else {
    float prev = v[0];
    for (int64_t i = 1; i < max_bin; ++i) {
      float c = v[(i * m_valid) / max_bin];
      if (c > prev) { out[count++] = c; prev = c; }
    }
  }
  out[count++] = end_cut(v[m_valid - 1]);
  return count;
}

int dpo_compute_cuts(const float* x, int64_t n, int64_t n_features, int32_t max_bin,
                     int32_t* cut_ptr, float* cut_values, float* min_values) {
  if (max_bin < 2 || max_bin > 256) return -1;
  /* every feature's cuts go to its own max_bin slots, then are packed */
  float* tmp = (float*)malloc(sizeof(float) * (size_t)(n_features > 0 ? n_features : 1) *
                              (size_t)max_bin);
  int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n_features > 0 ? n_features : 1));
  if (!tmp || !counts) { free(tmp); free(counts); return -2; }
  const int threads = threads_for(n_features, 1);
  int failed = 0;
#pragma omp parallel num_threads(threads)
  {
    float* v = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    if (!v) {
#pragma omp atomic write
      failed = 1;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int64_t f = 0; f < n_features; ++f)
        counts[f] = feature_cuts(x, n, n_features, f, max_bin, v, tmp + f * max_bin,
                                 min_values + f);
    }
    free(v);
  }
  if (failed) { free(tmp); free(counts); return -2; }
  int32_t out = 0;
  cut_ptr[0] = 0;
  for (int64_t f = 0; f < n_features; ++f) {
    memcpy(cut_values + out, tmp + f * max_bin, sizeof(float) * (size_t)counts[f]);
    out += counts[f];
    cut_ptr[f + 1] = out;
  }
  free(tmp);
  free(counts);
  return 0;
}

static int32_t upper_bound(const float* cuts, int32_t count, float value) {
  int32_t lo = 0, hi = count;
  while (lo < hi) {
    int32_t mid = (lo + hi) >> 1;
    if (cuts[mid] > value) hi = mid; else lo = mid + 1;
  }
  return lo;
}

/* Bin symbols: uint8, or uint16 when missing_bin > 255 (a matrix with missing  */
/* values some of whose features use all 256 bins: missing is then symbol 256). */
static inline int32_t bin_at(const void* bins, int32_t missing_bin, int64_t i) {
  return missing_bin > 255 ? (int32_t)((const uint16_t*)bins)[i]
                           : (int32_t)((const uint8_t*)bins)[i];
}

void dpo_bin_matrix(const float* x, int64_t n, int64_t n_features, const int32_t* cut_ptr,
                    const float* cut_values, int32_t missing_bin, void* bins) {
  const int threads = threads_for(n * n_features, 1 << 20);
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t r = 0; r < n; ++r)
    for (int64_t f = 0; f < n_features; ++f) {
      float value = x[r * n_features + f];
      int32_t b;
      if (isnan(value)) {
        b = missing_bin;
      } else {
        int32_t count = cut_ptr[f + 1] - cut_ptr[f];
        int32_t idx = upper_bound(cut_values + cut_ptr[f], count, value);
        b = idx < count ? idx : count - 1;
      }
      if (missing_bin > 255)
        ((uint16_t*)bins)[r * n_features + f] = (uint16_t)b;
      else
        ((uint8_t*)bins)[r * n_features + f] = (uint8_t)b;
    }
}

/* ------------------------------------------------------------------------ */
/* exp: Cody & Waite range reduction x = k*ln2 + r, |r| <= ln2/2, with ln2    */
/* split into a float head/tail, then the degree-7 Taylor polynomial of e^r  */
/* (coefficients 1/j!) by Horner with fused multiply-add, scaled by 2^k.     */
/* Only IEEE-exact operations (fma, rint, ldexp) are used so the HIP kernels */
/* and this oracle produce identical bits.  Accuracy about 2 ulp; inputs     */
/* below -87 return 0, so no subnormal result is ever produced.             */
/* ------------------------------------------------------------------------ */
float dpo_expf(float x) {
  if (isnan(x)) return x;
  if (x > 88.72283f) return INFINITY;
  if (x < -87.0f) return 0.0f;
  const float log2e = 1.44269504088896341f;
  const float ln2_hi = 0.693145751953125f;       /* 12 significant bits */
  const float ln2_lo = 1.42860682030941723212e-6f;
  float k = rintf(x * log2e);
  float r = fmaf(-k, ln2_hi, x);
  r = fmaf(-k, ln2_lo, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)k);
}

/* Objective gradients (upstream objective functions; the reference fixes    */
/* multi:softmax at class_native_training.cuh:60 and base margin 0 at :63-64): */
/*   logistic : p = 1/(1+e^-m), g = p - y, h = max(p(1-p), 1e-16)            */
/*   softprob : p = softmax(m), g = p_k - [y==k], h = max(2p(1-p), 1e-16)     */
/*   squared  : g = m - y, h = 1                                              */
void dpo_gradients(int32_t objective, const float* margin, const float* label, int64_t n,
                   int32_t n_classes, float* grad, float* hess) {
  for (int64_t r = 0; r < n; ++r) {
    if (objective == DPO_OBJ_LOGISTIC) {
      float p = 1.0f / (1.0f + dpo_expf(-margin[r]));
      grad[r] = p - label[r];
      hess[r] = fmaxf(p * (1.0f - p), 1e-16f);
    } else if (objective == DPO_OBJ_SQUARED) {
      grad[r] = margin[r] - label[r];
      hess[r] = 1.0f;
    } else if (objective == DPO_OBJ_SOFTPROB) {
      const float* m = margin + r * n_classes;
      float mx = m[0];
      for (int32_t k = 1; k < n_classes; ++k) mx = fmaxf(mx, m[k]);
      float s = 0.0f;
      for (int32_t k = 0; k < n_classes; ++k) s += dpo_expf(m[k] - mx);
      int32_t y = (int32_t)label[r];
      for (int32_t k = 0; k < n_classes; ++k) {
        float p = dpo_expf(m[k] - mx) / s;
        grad[r * n_classes + k] = p - (k == y ? 1.0f : 0.0f);
        hess[r * n_classes + k] = fmaxf(2.0f * p * (1.0f - p), 1e-16f);
      }
    }
  }
}

/* Fixed-point quantiser.  Upstream's GPU hist quantises gradients per round  */
/* with a power-of-two rounding factor so histogram sums are exact integers.  */
/* Here: E = frexp exponent of max|g| (max|g| < 2^E), scale 2^(QBITS-E), so   */
/* every |q| <= 2^QBITS.  exp_q = QBITS - E is what both sides carry.         */
static int32_t quant_exp(float max_abs) {
  if (!(max_abs > 0.0f)) return DPO_QBITS;
  int e;
  frexpf(max_abs, &e);
  return DPO_QBITS - e;
}

void dpo_quantiser(const float* g, const float* h, int64_t n, int64_t stride,
                   int32_t* exp_g, int32_t* exp_h) {
  float mg = 0.0f, mh = 0.0f;
  for (int64_t r = 0; r < n; ++r) {
    mg = fmaxf(mg, fabsf(g[r * stride]));
    mh = fmaxf(mh, fabsf(h[r * stride]));
  }
  *exp_g = quant_exp(mg);
  *exp_h = quant_exp(mh);
}

void dpo_quantise(const float* g, const float* h, int64_t n, int64_t stride, int32_t exp_g,
                  int32_t exp_h, int32_t* qg, int32_t* qh) {
  for (int64_t r = 0; r < n; ++r) {
    qg[r] = (int32_t)rintf(ldexpf(g[r * stride], exp_g));
    qh[r] = (int32_t)rintf(ldexpf(h[r * stride], exp_h));
  }
}

double dpo_unscale(int32_t exp_q) { return ldexp(1.0, -exp_q); }

/* ------------------------------------------------------------------------ */
/* Histogram: hist[f][b] += (qg, qh) for every row of the node whose bin of   */
/* f is b; missing entries are not accumulated (their stats are the node sum */
/* minus the bin total, as upstream derives them).                           */
/* ------------------------------------------------------------------------ */
static void hist_rows(const void* bins, int64_t n_features, const int32_t* qg,
                      const int32_t* qh, const uint32_t* rows, int64_t i0, int64_t i1,
                      int32_t bin_stride, int32_t missing_bin, int64_t* hist) {
  for (int64_t i = i0; i < i1; ++i) {
    int64_t r = rows ? (int64_t)rows[i] : i;
    for (int64_t f = 0; f < n_features; ++f) {
      int32_t b = bin_at(bins, missing_bin, r * n_features + f);
      if (b == missing_bin) continue;
      int64_t* cell = hist + 2 * (f * bin_stride + b);
      cell[0] += qg[r];
      cell[1] += qh[r];
    }
  }
}

void dpo_hist(const void* bins, int64_t n_features, const int32_t* qg, const int32_t* qh,
              const uint32_t* rows, int64_t n_rows, int32_t bin_stride, int32_t missing_bin,
              int64_t* hist) {
  const int64_t cells = 2 * n_features * bin_stride;
  memset(hist, 0, sizeof(int64_t) * (size_t)cells);
  const int threads = threads_for(n_rows * n_features, 1 << 18);
  int64_t* priv = threads > 1 ? (int64_t*)calloc((size_t)(cells * threads), sizeof(int64_t))
                              : NULL;
  if (!priv) {
    hist_rows(bins, n_features, qg, qh, rows, 0, n_rows, bin_stride, missing_bin, hist);
    return;
  }
  /* thread t: rows [n t / T, n (t + 1) / T) into its own histogram, then the */
  /* histograms are added cell by cell (exact integers: any order is equal)  */
#pragma omp parallel num_threads(threads)
  {
#ifdef _OPENMP
    const int t = omp_get_thread_num();
#else
    const int t = 0;
#endif
    hist_rows(bins, n_features, qg, qh, rows, n_rows * t / threads, n_rows * (t + 1) / threads,
              bin_stride, missing_bin, priv + cells * t);
#pragma omp barrier
#pragma omp for schedule(static)
    for (int64_t c = 0; c < cells; ++c) {
      int64_t acc = 0;
      for (int u = 0; u < threads; ++u) acc += priv[cells * u + c];
      hist[c] = acc;
    }
  }
  free(priv);
}

/* Root-pass histogram with OpenMP: thread-private histograms over row blocks */
/* then an exact integer reduction.  Used as the timed CPU baseline.          */
void dpo_hist_parallel(const uint8_t* bins, int64_t n_features, const int32_t* qg,
                       const int32_t* qh, int64_t n_rows, int32_t bin_stride,
                       int32_t missing_bin, int32_t threads, int64_t* hist) {
  const int64_t cells = 2 * n_features * bin_stride;
  memset(hist, 0, sizeof(int64_t) * (size_t)cells);
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#else
  threads = 1;
#endif
  int64_t* priv = (int64_t*)calloc((size_t)(cells * threads), sizeof(int64_t));
  if (!priv) return;
#pragma omp parallel num_threads(threads)
  {
#ifdef _OPENMP
    int t = omp_get_thread_num();
#else
    int t = 0;
#endif
    int64_t* local = priv + cells * t;
#pragma omp for schedule(static)
    for (int64_t r = 0; r < n_rows; ++r) {
      const uint8_t* row = bins + r * n_features;
      const int64_t g = qg[r], h = qh[r];
      for (int64_t f = 0; f < n_features; ++f) {
        uint8_t b = row[f];
        if (b == missing_bin) continue;
        int64_t* cell = local + 2 * (f * bin_stride + b);
        cell[0] += g;
        cell[1] += h;
      }
    }
  }
  for (int t = 0; t < threads; ++t)
    for (int64_t c = 0; c < cells; ++c) hist[c] += priv[cells * t + c];
  free(priv);
}

void dpo_hist_subtract(const int64_t* parent, const int64_t* built, int64_t n, int64_t* sibling) {
  for (int64_t i = 0; i < n; ++i) sibling[i] = parent[i] - built[i];
}

/* ------------------------------------------------------------------------ */
/* Split evaluation (upstream CalcGain / CalcWeight with max_delta_step 0).  */
/*   T(G)   = sign(G) max(|G| - alpha, 0)                                     */
/*   gain   = T(G)^2 / (H + lambda), 0 when H < min_child_weight or H <= 0   */
/*   weight = -T(G) / (H + lambda),  0 in the same cases                     */
/* For every feature f and bin b in [0, n_bins(f)) the candidate sends bins  */
/* <= b left and tries missing right, then missing left; missing-left is kept*/
/* only when strictly better.  A candidate needs both children with H >=     */
/* min_child_weight and positive quantised hessian; its loss change is       */
/* (gain(L) + gain(R)) - gain(P) in double.  The argmax keeps the first      */
/* strictly larger value in (feature, bin) order, i.e. ties go to the lowest */
/* feature, then the lowest bin.                                             */
/* ------------------------------------------------------------------------ */
static double threshold_l1(double g, double alpha) {
  if (g > alpha) return g - alpha;
  if (g < -alpha) return g + alpha;
  return 0.0;
}

double dpo_calc_gain(const dpo_params* p, double g, double h) {
  if (h < (double)p->min_child_weight || h <= 0.0) return 0.0;
  double t = threshold_l1(g, (double)p->alpha);
  return (t * t) / (h + (double)p->lambda);
}

double dpo_calc_weight(const dpo_params* p, double g, double h) {
  if (h < (double)p->min_child_weight || h <= 0.0) return 0.0;
  return -threshold_l1(g, (double)p->alpha) / (h + (double)p->lambda);
}

static double split_loss(const dpo_params* p, int64_t qgl, int64_t qhl, int64_t qgr, int64_t qhr,
                         double ug, double uh, double parent_gain) {
  if (qhl <= 0 || qhr <= 0) return -INFINITY;
  double gl = (double)qgl * ug, hl = (double)qhl * uh;
  double gr = (double)qgr * ug, hr = (double)qhr * uh;
  double mcw = (double)p->min_child_weight;
  if (hl < mcw || hr < mcw) return -INFINITY;
  return (dpo_calc_gain(p, gl, hl) + dpo_calc_gain(p, gr, hr)) - parent_gain;
}

void dpo_evaluate_split(const int64_t* hist, int64_t n_features, int32_t bin_stride,
                        const int32_t* n_bins, int64_t gp, int64_t hp, double unscale_g,
                        double unscale_h, const dpo_params* p, dpo_split* out) {
  dpo_evaluate_split_masked(hist, n_features, bin_stride, n_bins, gp, hp, unscale_g, unscale_h, p,
                            NULL, out);
}

/* Best candidate of one feature: the first bin (then missing right before  */
/* left) with the largest loss; loss -inf when it has none.                  */
static dpo_split feature_split(const int64_t* hf, int64_t f, int32_t nb, int64_t gp, int64_t hp,
                               double unscale_g, double unscale_h, const dpo_params* p,
                               double parent_gain) {
  dpo_split best;
  best.loss_chg = -INFINITY;
  best.feature = (int32_t)f;
  best.bin = -1;
  best.default_left = 0;
  best.valid = 0;
  best.gl = 0;
  best.hl = 0;
  int64_t tg = 0, th = 0;
  for (int32_t b = 0; b < nb; ++b) { tg += hf[2 * b]; th += hf[2 * b + 1]; }
  const int64_t mg = gp - tg, mh = hp - th;
  int64_t lg = 0, lh = 0;
  for (int32_t b = 0; b < nb; ++b) {
    lg += hf[2 * b];
    lh += hf[2 * b + 1];
    double right_missing = split_loss(p, lg, lh, gp - lg, hp - lh, unscale_g, unscale_h, parent_gain);
    double left_missing = split_loss(p, lg + mg, lh + mh, gp - lg - mg, hp - lh - mh,
                                     unscale_g, unscale_h, parent_gain);
    int dl = left_missing > right_missing;
    double c = dl ? left_missing : right_missing;
    if (c > best.loss_chg) {
      best.loss_chg = c;
      best.bin = b;
      best.default_left = dl;
      best.valid = 1;
      best.gl = dl ? lg + mg : lg;
      best.hl = dl ? lh + mh : lh;
    }
  }
  return best;
}

void dpo_evaluate_split_masked(const int64_t* hist, int64_t n_features, int32_t bin_stride,
                               const int32_t* n_bins, int64_t gp, int64_t hp, double unscale_g,
                               double unscale_h, const dpo_params* p, const uint8_t* allowed,
                               dpo_split* out) {
  dpo_split best;
  best.loss_chg = -INFINITY;
  best.feature = -1;
  best.bin = -1;
  best.default_left = 0;
  best.valid = 0;
  best.gl = 0;
  best.hl = 0;
  const double parent_gain = dpo_calc_gain(p, (double)gp * unscale_g, (double)hp * unscale_h);
  dpo_split* each = (dpo_split*)malloc(sizeof(dpo_split) * (size_t)(n_features > 0 ? n_features : 1));
  if (!each) { *out = best; return; }
  const int threads = threads_for(n_features * bin_stride, 1 << 14);
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t f = 0; f < n_features; ++f) {
    if (allowed && !allowed[f]) {  /* outside the node's column sample */
      each[f].valid = 0;
      continue;
    }
    each[f] = feature_split(hist + 2 * f * bin_stride, f, n_bins[f], gp, hp, unscale_g,
                            unscale_h, p, parent_gain);
  }
  /* features in order, strictly larger wins: ties keep the lowest feature */
  /* (and, within a feature, its lowest bin)                               */
  for (int64_t f = 0; f < n_features; ++f)
    if (each[f].valid && each[f].loss_chg > best.loss_chg) best = each[f];
  free(each);
  *out = best;
}

/* Stable partition of ridx[begin, end): rows whose bin <= split_bin (or that */
/* are missing with default_left) first, in their original order.            */
static int row_left(const void* bins, int64_t n_features, uint32_t r, int32_t feature,
                    int32_t split_bin, int32_t default_left, int32_t missing_bin) {
  const int32_t b = bin_at(bins, missing_bin, (int64_t)r * n_features + feature);
  return b == missing_bin ? default_left : b <= split_bin;
}

int64_t dpo_partition(uint32_t* ridx, int64_t begin, int64_t end, const void* bins,
                      int64_t n_features, int32_t feature, int32_t split_bin,
                      int32_t default_left, int32_t missing_bin, uint32_t* scratch) {
  const int64_t n = end - begin;
  const int threads = threads_for(n, 1 << 16);
  if (threads <= 1) {
    int64_t nl = 0, nr = 0;
    for (int64_t i = begin; i < end; ++i) {
      uint32_t r = ridx[i];
      if (row_left(bins, n_features, r, feature, split_bin, default_left, missing_bin))
        ridx[begin + nl++] = r;
      else
        scratch[nr++] = r;
    }
    memcpy(ridx + begin + nl, scratch, sizeof(uint32_t) * (size_t)nr);
    return nl;
  }
  /* blocks of rows: count each block's lefts, then every block writes its    */
  /* lefts and rights after those of the blocks before it (stable)           */
  int64_t* lefts = (int64_t*)calloc((size_t)threads + 1, sizeof(int64_t));
  memcpy(scratch, ridx + begin, sizeof(uint32_t) * (size_t)n);
#pragma omp parallel num_threads(threads)
  {
#ifdef _OPENMP
    const int t = omp_get_thread_num();
#else
    const int t = 0;
#endif
    const int64_t b = n * t / threads, e = n * (t + 1) / threads;
    int64_t c = 0;
    for (int64_t i = b; i < e; ++i)
      c += row_left(bins, n_features, scratch[i], feature, split_bin, default_left, missing_bin);
    lefts[t + 1] = c;
#pragma omp barrier
#pragma omp single
    for (int u = 0; u < threads; ++u) lefts[u + 1] += lefts[u];
    /* implicit barrier after single */
    int64_t pl = begin + lefts[t], pr = begin + lefts[threads] + (b - lefts[t]);
    for (int64_t i = b; i < e; ++i) {
      uint32_t r = scratch[i];
      if (row_left(bins, n_features, r, feature, split_bin, default_left, missing_bin))
        ridx[pl++] = r;
      else
        ridx[pr++] = r;
    }
  }
  const int64_t nl = lefts[threads];
  free(lefts);
  return nl;
}

/* ------------------------------------------------------------------------ */
/* Row and column sampling (subsample, colsample_by{tree,level,node}; the     */
/* reference forwards these keys to the trainer unchanged,                    */
/* native/class_native_training.cuh:30-31, :63).  Upstream draws from a      */
/* global generator that cannot be reproduced here; this build fixes         */
/* counter-based draws instead:                                              */
/*   mix64      SplitMix64's output function (Steele, Lea & Flood 2014)      */
/*   prefix     mix64(mix64(mix64(seed ^ stream << 56) ^ a) ^ b)             */
/*   draw       upper 32 bits of mix64(prefix ^ index)                       */
/* Rows: stream 1, a = round, b = output << 32; row r is kept iff            */
/* draw < floor(subsample * 2^32), and a dropped row's (g, h) are zero for   */
/* that tree (before the quantiser).  Columns: stages tree (stream 2,         */
/* b = output << 32), level (stream 3, b = output << 32 | depth) and node     */
/* (stream 4, b = output << 32 | node id), a = round.  A stage keeps          */
/* n = max(1, (int)(fraction * m)) of its m candidates (the product in float, */
/* as upstream's ColumnSampler forms it), those with the smallest keys,      */
/* key(f) = draw with its low fbits bits replaced by f (fbits: bits of        */
/* n_features - 1).  Each stage chooses among the previous stage's features. */
/* Here the n smallest keys are found by sorting them.                       */
/* ------------------------------------------------------------------------ */
uint64_t dpo_mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t dpo_sample_prefix(uint64_t seed, uint64_t stream, uint64_t a, uint64_t b) {
  return dpo_mix64(dpo_mix64(dpo_mix64(seed ^ (stream << 56)) ^ a) ^ b);
}

uint32_t dpo_sample_draw(uint64_t prefix, uint64_t index) {
  return (uint32_t)(dpo_mix64(prefix ^ index) >> 32);
}

int32_t dpo_stage_keep(float fraction, int32_t m) {
  if (!(fraction < 1.0f)) return m;
  float x = fraction * (float)m;
  int32_t n = (int32_t)x;
  return n < 1 ? 1 : n;
}

void dpo_sample_rows(const dpo_sampling* s, int64_t n, uint8_t* keep) {
  if (!(s->subsample < 1.0f)) {
    memset(keep, 1, (size_t)n);
    return;
  }
  const uint64_t threshold = (uint64_t)ldexp((double)s->subsample, 32);
  const uint64_t prefix = dpo_sample_prefix(s->seed, 1, (uint64_t)(uint32_t)s->round,
                                            (uint64_t)(uint32_t)s->output << 32);
  for (int64_t r = 0; r < n; ++r) keep[r] = (uint64_t)dpo_sample_draw(prefix, (uint64_t)r) < threshold;
}

static int cmp_u32(const void* a, const void* b) {
  uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
  return (x > y) - (x < y);
}

static uint32_t feature_key(uint64_t prefix, int64_t f, int fbits) {
  uint32_t low = fbits >= 32 ? 0xffffffffu : ((1u << fbits) - 1u);
  return (dpo_sample_draw(prefix, (uint64_t)f) & ~low) | (uint32_t)f;
}

/* One stage: among the features allowed[] admits, keep the n smallest keys. */
static void colsample_stage(uint64_t prefix, float fraction, int64_t n_features, int fbits,
                            uint8_t* allowed, uint32_t* keys) {
  int32_t m = 0;
  for (int64_t f = 0; f < n_features; ++f)
    if (allowed[f]) keys[m++] = feature_key(prefix, f, fbits);
  const int32_t n = dpo_stage_keep(fraction, m);
  if (n >= m) return;
  qsort(keys, (size_t)m, sizeof(uint32_t), cmp_u32);
  const uint32_t last = keys[n - 1];
  for (int64_t f = 0; f < n_features; ++f)
    if (allowed[f]) allowed[f] = feature_key(prefix, f, fbits) <= last;
}

void dpo_colsample(const dpo_sampling* s, int32_t depth, int32_t nid, int64_t n_features,
                   uint8_t* allowed) {
  memset(allowed, 1, (size_t)n_features);
  if (!s || !(s->colsample_bytree < 1.0f || s->colsample_bylevel < 1.0f ||
              s->colsample_bynode < 1.0f))
    return;
  int fbits = 0;
  while (fbits < 31 && ((int64_t)1 << fbits) < n_features) ++fbits;
  uint32_t* keys = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(n_features > 0 ? n_features : 1));
  if (!keys) return;
  const uint64_t round = (uint64_t)(uint32_t)s->round;
  const uint64_t out = (uint64_t)(uint32_t)s->output << 32;
  colsample_stage(dpo_sample_prefix(s->seed, 2, round, out), s->colsample_bytree, n_features,
                  fbits, allowed, keys);
  colsample_stage(dpo_sample_prefix(s->seed, 3, round, out | (uint32_t)depth),
                  s->colsample_bylevel, n_features, fbits, allowed, keys);
  colsample_stage(dpo_sample_prefix(s->seed, 4, round, out | (uint32_t)nid), s->colsample_bynode,
                  n_features, fbits, allowed, keys);
  free(keys);
}

/* ------------------------------------------------------------------------ */
/* One depth-wise tree.  Nodes are numbered as upstream's depth-wise driver   */
/* allocates them: level by level, children of the k-th expanded node of a   */
/* level get the next two ids (left, right), so left > node and right =      */
/* left + 1 (native/class_native_source_contract.hpp:24-31).  A node expands */
/* iff its best split is valid, loss_chg > 1e-6, loss_chg >= gamma and depth */
/* < max_depth.  Child histograms: the child with fewer rows is built, its   */
/* sibling is parent - built (ties build the left child).                    */
/* ------------------------------------------------------------------------ */
static void* xcalloc(size_t n, size_t s) { return calloc(n ? n : 1, s); }

int dpo_grow_tree(const void* bins, int64_t n, int64_t n_features, const int32_t* cut_ptr,
                  const float* cut_values, int32_t missing_bin, const int32_t* qg,
                  const int32_t* qh, int32_t exp_g, int32_t exp_h, const dpo_params* p,
                  int32_t bin_stride, uint32_t* ridx, dpo_tree* t) {
  return dpo_grow_tree_sampled(bins, n, n_features, cut_ptr, cut_values, missing_bin, qg, qh,
                               exp_g, exp_h, p, bin_stride, NULL, ridx, t);
}

int dpo_grow_tree_sampled(const void* bins, int64_t n, int64_t n_features,
                          const int32_t* cut_ptr, const float* cut_values, int32_t missing_bin,
                          const int32_t* qg, const int32_t* qh, int32_t exp_g, int32_t exp_h,
                          const dpo_params* p, int32_t bin_stride, const dpo_sampling* smp,
                          uint32_t* ridx, dpo_tree* t) {
  const int32_t depth_cap = p->max_depth;
  if (depth_cap < 0 || depth_cap > 20) return -1;
  const int32_t cap = (int32_t)((1u << (depth_cap + 1)) - 1u);
  const int64_t hsize = 2 * n_features * bin_stride;
  const double ug = dpo_unscale(exp_g), uh = dpo_unscale(exp_h);
  memset(t, 0, sizeof(*t));
  t->left = (int32_t*)xcalloc((size_t)cap, 4);
  t->right = (int32_t*)xcalloc((size_t)cap, 4);
  t->parent = (int32_t*)xcalloc((size_t)cap, 4);
  t->feature = (int32_t*)xcalloc((size_t)cap, 4);
  t->split_bin = (int32_t*)xcalloc((size_t)cap, 4);
  t->default_left = (int32_t*)xcalloc((size_t)cap, 4);
  t->split_condition = (float*)xcalloc((size_t)cap, 4);
  t->base_weight = (float*)xcalloc((size_t)cap, 4);
  t->leaf_value = (float*)xcalloc((size_t)cap, 4);
  t->loss_chg = (float*)xcalloc((size_t)cap, 4);
  t->sum_hess = (float*)xcalloc((size_t)cap, 4);
  t->sum_qg = (int64_t*)xcalloc((size_t)cap, 8);
  t->sum_qh = (int64_t*)xcalloc((size_t)cap, 8);
  t->seg_begin = (int32_t*)xcalloc((size_t)cap, 4);
  t->seg_end = (int32_t*)xcalloc((size_t)cap, 4);
  int32_t* n_bins = (int32_t*)xcalloc((size_t)n_features, 4);
  for (int64_t f = 0; f < n_features; ++f) n_bins[f] = cut_ptr[f + 1] - cut_ptr[f];
  /* histograms of the current level, indexed by node id */
  int64_t** hist = (int64_t**)xcalloc((size_t)cap, sizeof(int64_t*));
  uint32_t* scratch = (uint32_t*)xcalloc((size_t)n, 4);
  int32_t* level = (int32_t*)xcalloc((size_t)cap, 4);
  int32_t* next = (int32_t*)xcalloc((size_t)cap, 4);
  uint8_t* allowed = (uint8_t*)xcalloc((size_t)n_features, 1);

  int64_t g0 = 0, h0 = 0;
  for (int64_t r = 0; r < n; ++r) { g0 += qg[r]; h0 += qh[r]; }
  t->n_nodes = 1;
  t->parent[0] = -1;
  t->seg_begin[0] = 0;
  t->seg_end[0] = (int32_t)n;
  t->sum_qg[0] = g0;
  t->sum_qh[0] = h0;
  if (depth_cap > 0) {
    hist[0] = (int64_t*)xcalloc((size_t)hsize, 8);
    dpo_hist(bins, n_features, qg, qh, ridx, n, bin_stride, missing_bin, hist[0]);
  }
  int32_t n_level = 1;
  level[0] = 0;
  for (int32_t depth = 0; n_level > 0; ++depth) {
    int32_t n_next = 0;
    for (int32_t i = 0; i < n_level; ++i) {
      const int32_t nid = level[i];
      const double G = (double)t->sum_qg[nid] * ug, H = (double)t->sum_qh[nid] * uh;
      const double w = dpo_calc_weight(p, G, H);
      t->base_weight[nid] = (float)w;
      t->sum_hess[nid] = (float)H;
      t->left[nid] = t->right[nid] = -1;
      t->feature[nid] = 0;
      t->split_bin[nid] = -1;
      dpo_split s;
      int expand = 0;
      if (depth < depth_cap) {
        dpo_colsample(smp, depth, nid, n_features, allowed);
        dpo_evaluate_split_masked(hist[nid], n_features, bin_stride, n_bins, t->sum_qg[nid],
                                  t->sum_qh[nid], ug, uh, p, allowed, &s);
        expand = s.valid && s.loss_chg > DPO_RT_EPS && s.loss_chg >= (double)p->gamma;
      }
      if (!expand) {
        t->leaf_value[nid] = (float)(w * (double)p->eta);
        t->split_condition[nid] = t->leaf_value[nid];
        free(hist[nid]);
        hist[nid] = NULL;
        continue;
      }
      const int32_t l = t->n_nodes, r = t->n_nodes + 1;
      t->n_nodes += 2;
      t->left[nid] = l;
      t->right[nid] = r;
      t->feature[nid] = s.feature;
      t->split_bin[nid] = s.bin;
      t->default_left[nid] = s.default_left;
      t->split_condition[nid] = cut_values[cut_ptr[s.feature] + s.bin];
      t->loss_chg[nid] = (float)s.loss_chg;
      const int64_t b = t->seg_begin[nid], e = t->seg_end[nid];
      const int64_t nl = dpo_partition(ridx, b, e, bins, n_features, s.feature, s.bin,
                                       s.default_left, missing_bin, scratch);
      t->parent[l] = t->parent[r] = nid;
      t->seg_begin[l] = (int32_t)b;
      t->seg_end[l] = (int32_t)(b + nl);
      t->seg_begin[r] = (int32_t)(b + nl);
      t->seg_end[r] = (int32_t)e;
      t->sum_qg[l] = s.gl;
      t->sum_qh[l] = s.hl;
      t->sum_qg[r] = t->sum_qg[nid] - s.gl;
      t->sum_qh[r] = t->sum_qh[nid] - s.hl;
      if (depth + 1 < depth_cap) {
        const int32_t small = (e - b - nl) < nl ? r : l, large = small == l ? r : l;
        hist[small] = (int64_t*)xcalloc((size_t)hsize, 8);
        hist[large] = (int64_t*)xcalloc((size_t)hsize, 8);
        dpo_hist(bins, n_features, qg, qh, ridx + t->seg_begin[small],
                 t->seg_end[small] - t->seg_begin[small], bin_stride, missing_bin, hist[small]);
        dpo_hist_subtract(hist[nid], hist[small], hsize, hist[large]);
      }
      free(hist[nid]);
      hist[nid] = NULL;
      next[n_next++] = l;
      next[n_next++] = r;
    }
    int32_t* tmp = level;
    level = next;
    next = tmp;
    n_level = n_next;
  }
  free(hist);
  free(scratch);
  free(level);
  free(next);
  free(n_bins);
  free(allowed);
  return 0;
}

void dpo_tree_free(dpo_tree* t) {
  free(t->left); free(t->right); free(t->parent); free(t->feature); free(t->split_bin);
  free(t->default_left); free(t->split_condition); free(t->base_weight); free(t->leaf_value);
  free(t->loss_chg); free(t->sum_hess); free(t->sum_qg); free(t->sum_qh);
  free(t->seg_begin); free(t->seg_end);
  memset(t, 0, sizeof(*t));
}

void dpo_tree_update_margin(const dpo_tree* t, const uint32_t* ridx, float* margin,
                            int64_t stride) {
  for (int32_t nid = 0; nid < t->n_nodes; ++nid) {
    if (t->left[nid] != -1) continue;
    const float v = t->leaf_value[nid];
    for (int32_t i = t->seg_begin[nid]; i < t->seg_end[nid]; ++i)
      margin[(int64_t)ridx[i] * stride] += v;
  }
}

float dpo_predict_tree(const dpo_tree* t, const float* row) {
  int32_t nid = 0;
  while (t->left[nid] != -1) {
    float x = row[t->feature[nid]];
    if (isnan(x)) nid = t->default_left[nid] ? t->left[nid] : t->right[nid];
    else nid = x < t->split_condition[nid] ? t->left[nid] : t->right[nid];
  }
  return t->leaf_value[nid];
}
