/*
 * dp_oracle.h -- CPU restatement of the gradient-boosting training hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code.  It is the checker that tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg compare the HIP path against.
 *
 * The reference (decision-programs) reaches this path through XGBoost 3.4.1's
 * `grow_gpu_hist` updater (native/class_native_training.cuh:47-70,
 * native/class_model_train.cu:48).  XGBoost is not vendored in the reference
 * and is absent from this image, so the semantics below are a restatement of
 * XGBoost's published hist algorithm with every choice that upstream leaves
 * open fixed explicitly (quantile definition, fixed-point rounding, tie rules).
 *
 * Layout conventions (shared with the HIP library through the C ABI):
 *   bins      : row-major [n_rows][n_features] symbols; `missing_bin` marks NaN.
 *               uint8 (missing_bin -1 or 255), or uint16 with missing_bin 256
 *               for a matrix with missing values some of whose features use
 *               all 256 bins (dpo_hist_parallel takes uint8 only)
 *   cut_ptr   : int32 [n_features + 1]; feature f owns cut_values[cut_ptr[f],
 *               cut_ptr[f+1]); its bin b holds x in [cut[b-1], cut[b])
 *   hist      : int64 [n_features][n_bins_stride][2] = (sum qg, sum qh)
 *   ridx      : uint32 row ids; every tree node owns one contiguous segment
 */
#ifndef DP_ORACLE_H
#define DP_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum dpo_objective {
  DPO_OBJ_LOGISTIC = 0,    /* binary:logistic                     */
  DPO_OBJ_SOFTPROB = 1,    /* multi:softprob and multi:softmax    */
  DPO_OBJ_SQUARED = 2,     /* reg:squarederror                    */
  DPO_OBJ_INJECTED = 3     /* caller-supplied gradients           */
};

/* Fixed-point precision: |q| <= 2^DPO_QBITS for every quantised gradient. */
#define DPO_QBITS 30
#define DPO_RT_EPS 1e-6

typedef struct {
  float eta, lambda, alpha, gamma, min_child_weight;
  int32_t max_depth;
} dpo_params;

typedef struct {
  double loss_chg;         /* -inf when no valid candidate                 */
  int32_t feature, bin;    /* split sends bin <= `bin` to the left          */
  int32_t default_left;    /* missing rows go left                          */
  int32_t valid;           /* a finite candidate was found                  */
  int64_t gl, hl;          /* quantised left-child sums                     */
} dpo_split;

/* ---- threads ----------------------------------------------------------- */
/* OpenMP threads of the cuts, binning, histograms, split search and         */
/* partition (1, the default, runs serially).  Results do not depend on it.  */
void dpo_set_threads(int32_t n);
int32_t dpo_get_threads(void);

/* ---- quantile cuts and binning ---------------------------------------- */
int dpo_compute_cuts(const float* x, int64_t n, int64_t n_features, int32_t max_bin,
                     int32_t* cut_ptr, float* cut_values, float* min_values);
void dpo_bin_matrix(const float* x, int64_t n, int64_t n_features, const int32_t* cut_ptr,
                    const float* cut_values, int32_t missing_bin, void* bins);

/* ---- objective gradients and the fixed-point quantiser ----------------- */
float dpo_expf(float x);
void dpo_gradients(int32_t objective, const float* margin, const float* label, int64_t n,
                   int32_t n_classes, float* grad, float* hess);
void dpo_quantiser(const float* g, const float* h, int64_t n, int64_t stride,
                   int32_t* exp_g, int32_t* exp_h);
void dpo_quantise(const float* g, const float* h, int64_t n, int64_t stride, int32_t exp_g,
                  int32_t exp_h, int32_t* qg, int32_t* qh);
double dpo_unscale(int32_t exp_q);

/* ---- histogram, subtraction ------------------------------------------- */
void dpo_hist(const void* bins, int64_t n_features, const int32_t* qg, const int32_t* qh,
              const uint32_t* rows, int64_t n_rows, int32_t bin_stride, int32_t missing_bin,
              int64_t* hist);
void dpo_hist_parallel(const uint8_t* bins, int64_t n_features, const int32_t* qg,
                       const int32_t* qh, int64_t n_rows, int32_t bin_stride,
                       int32_t missing_bin, int32_t threads, int64_t* hist);
void dpo_hist_subtract(const int64_t* parent, const int64_t* built, int64_t n, int64_t* sibling);

/* ---- split evaluation, partition, leaves ------------------------------- */
double dpo_calc_gain(const dpo_params* p, double g, double h);
double dpo_calc_weight(const dpo_params* p, double g, double h);
void dpo_evaluate_split(const int64_t* hist, int64_t n_features, int32_t bin_stride,
                        const int32_t* n_bins, int64_t gp, int64_t hp, double unscale_g,
                        double unscale_h, const dpo_params* p, dpo_split* out);
/* Only features with allowed[f] != 0 are candidates (allowed NULL: all). */
void dpo_evaluate_split_masked(const int64_t* hist, int64_t n_features, int32_t bin_stride,
                               const int32_t* n_bins, int64_t gp, int64_t hp, double unscale_g,
                               double unscale_h, const dpo_params* p, const uint8_t* allowed,
                               dpo_split* out);
int64_t dpo_partition(uint32_t* ridx, int64_t begin, int64_t end, const void* bins,
                      int64_t n_features, int32_t feature, int32_t split_bin,
                      int32_t default_left, int32_t missing_bin, uint32_t* scratch);

/* ---- row and column sampling ------------------------------------------ */
/* Counter-based draws (see dp_oracle.c): subsample keeps a row of one tree's */
/* gradients iff its draw falls below floor(subsample * 2^32); the column     */
/* stages keep the features with the smallest keys.                          */
typedef struct {
  uint64_t seed;
  int32_t round;           /* boosting round index                          */
  int32_t output;          /* the tree's output (class) index               */
  float subsample, colsample_bytree, colsample_bylevel, colsample_bynode;
} dpo_sampling;

uint64_t dpo_mix64(uint64_t z);
uint64_t dpo_sample_prefix(uint64_t seed, uint64_t stream, uint64_t a, uint64_t b);
uint32_t dpo_sample_draw(uint64_t prefix, uint64_t index);
int32_t dpo_stage_keep(float fraction, int32_t m);
/* keep[r] = 1 when row r's gradient pair is kept for tree (round, output). */
void dpo_sample_rows(const dpo_sampling* s, int64_t n, uint8_t* keep);
/* allowed[f] = 1 when feature f is a split candidate at node `nid` of depth */
/* `depth` (the nested tree, level and node stages).                          */
void dpo_colsample(const dpo_sampling* s, int32_t depth, int32_t nid, int64_t n_features,
                   uint8_t* allowed);

/* ---- one tree ----------------------------------------------------------- */
typedef struct {
  int32_t n_nodes;
  int32_t *left, *right, *parent, *feature, *split_bin, *default_left;
  float *split_condition, *base_weight, *leaf_value, *loss_chg, *sum_hess;
  int64_t *sum_qg, *sum_qh;
  int32_t *seg_begin, *seg_end;   /* row segment of every node in ridx     */
} dpo_tree;

int dpo_grow_tree(const void* bins, int64_t n, int64_t n_features, const int32_t* cut_ptr,
                  const float* cut_values, int32_t missing_bin, const int32_t* qg,
                  const int32_t* qh, int32_t exp_g, int32_t exp_h, const dpo_params* p,
                  int32_t bin_stride, uint32_t* ridx, dpo_tree* out);
/* As dpo_grow_tree with column sampling (s NULL: every feature everywhere). */
int dpo_grow_tree_sampled(const void* bins, int64_t n, int64_t n_features,
                          const int32_t* cut_ptr, const float* cut_values, int32_t missing_bin,
                          const int32_t* qg, const int32_t* qh, int32_t exp_g, int32_t exp_h,
                          const dpo_params* p, int32_t bin_stride, const dpo_sampling* s,
                          uint32_t* ridx, dpo_tree* out);
void dpo_tree_free(dpo_tree* t);
void dpo_tree_update_margin(const dpo_tree* t, const uint32_t* ridx, float* margin,
                            int64_t stride);
float dpo_predict_tree(const dpo_tree* t, const float* row);

#ifdef __cplusplus
}
#endif
#endif
