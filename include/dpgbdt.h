/*
 * dpgbdt.h -- C ABI of libdpgbdt_hip.so, the MI355X (gfx950) implementation of
 * decision-programs' gradient-boosting training hot path.
 *
 * Two layers, both plain C (pointers, sizes, opaque handles; no C++ or torch
 * types):
 *
 *  1. The XGBoost C-API subset that the reference trainer binds with dlopen +
 *     dlsym (native/class_model_native_adapter.cuh:19-31,
 *     native/class_native_training.cuh:47-70, native/class_study_train.cu:84-332).
 *     Same names, argument meaning and status convention: 0 on success, -1 on
 *     failure with the message in XGBGetLastError().  A maintainer points the
 *     reference's `native_library_path` at this library instead of
 *     libxgboost.so.  Extensions beyond the reference's use are marked.
 *
 *  2. The kernel-level operator API (dp_*) that the booster itself is built
 *     from: histogram build, sibling subtraction, split evaluation, row
 *     partition, objective gradients, quantisation, quantile cuts and binning.
 *     These take device pointers and a HIP stream (`void*`, NULL = null
 *     stream).  Upstream has no public counterpart (the reference reaches these
 *     steps only inside XGBoosterUpdateOneIter, class_native_training.cuh:67);
 *     they exist so every step of the path can be driven and checked alone.
 *
 * Data conventions
 *   values     float32 row-major [n_rows][n_features]; NaN = missing
 *   bins       uint8 tile-major: element (r, f) at
 *              bins[(f / tile_width) * n_rows * tile_width + r * tile_width
 *                   + f % tile_width]; `missing_bin` (-1 = none) marks NaN;
 *              a paired layout's joint tiles follow (dp_bin_layout)
 *   gpair      int32 [n_rows][2] = (qg, qh), gradients in fixed point:
 *              q = rint(x * 2^exp), |q| <= 2^30 (see dp_quantise_gradients)
 *   hist       int64 [node][n_features][bin_stride][2] = (sum qg, sum qh)
 *   ridx       uint32 row ids; every tree node owns a contiguous segment
 */
#ifndef DPGBDT_H
#define DPGBDT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* DMatrixHandle;
typedef void* BoosterHandle;
typedef uint64_t bst_ulong;

/* ======================================================================= */
/* 1. XGBoost C-API subset                                                  */
/* ======================================================================= */

/* Reports 3.4.1: the reference refuses any other version
 * (class_model_native_adapter.cuh:24). */
void XGBoostVersion(int* major, int* minor, int* patch);

/* JSON build description; "USE_CUDA": true is what the reference checks
 * (class_model_native_adapter.cuh:24), "USE_HIP" and "GPU_ARCH" name the
 * actual gfx950 build. */
int XGBuildInfo(const char** out);

/* Message of the last failed call on this thread
 * (class_model_native_adapter.cuh:23). */
const char* XGBGetLastError(void);

/* Dense float32 device matrix from an array-interface JSON
 * {"data":[ptr,true],"shape":[N,F],"typestr":"<f4",...} and config
 * {"missing":NaN,...} (class_native_training.cuh:51).  The values are copied;
 * the caller's buffer may be freed afterwards. */
int XGDMatrixCreateFromCudaArrayInterface(const char* data, const char* config,
                                          DMatrixHandle* out);

/* field "label" from a device array interface (class_native_training.cuh:52). */
int XGDMatrixSetInfoFromInterface(DMatrixHandle handle, const char* field, const char* data);

int XGDMatrixNumRow(DMatrixHandle handle, bst_ulong* out);
int XGDMatrixNumCol(DMatrixHandle handle, bst_ulong* out);

/* class_model_native_adapter.cuh:25 */
int XGDMatrixFree(DMatrixHandle handle);

/* class_native_training.cuh:56 */
int XGBoosterCreate(const DMatrixHandle dmats[], bst_ulong len, BoosterHandle* out);

/* class_model_native_adapter.cuh:25 */
int XGBoosterFree(BoosterHandle handle);

/* class_native_training.cuh:57-65; keys objective, num_class, tree_method,
 * device, booster, max_bin, max_depth, eta, lambda, alpha, gamma,
 * min_child_weight, subsample, colsample_*, base_score, boost_from_average,
 * seed, seed_per_iteration, nthread, verbosity, validate_parameters. */
int XGBoosterSetParam(BoosterHandle handle, const char* name, const char* value);

/* One boosting round from the objective's gradients (class_native_training.cuh:67). */
int XGBoosterUpdateOneIter(BoosterHandle handle, int iter, DMatrixHandle dtrain);

/* Extension (upstream's XGBoosterTrainOneIter): one round from caller
 * gradients given as device array interfaces of shape [N] or [N, K]. */
int XGBoosterTrainOneIter(BoosterHandle handle, DMatrixHandle dtrain, int iter,
                          const char* grad, const char* hess);

/* class_model_train.cu:49 */
int XGBoosterBoostedRounds(BoosterHandle handle, int* out);

/* class_native_training.cuh:68; reports updater "grow_gpu_hist", which
 * class_model_train.cu:48 requires. */
int XGBoosterSaveJsonConfig(BoosterHandle handle, bst_ulong* out_len, const char** out_str);

/* class_native_training.cuh:69: XGBoost 3.4.1 JSON model schema. */
int XGBoosterSaveModel(BoosterHandle handle, const char* fname);

/* class_study_train.cu:329; config {"format":"json"}. */
int XGBoosterSaveModelToBuffer(BoosterHandle handle, const char* config, bst_ulong* out_len,
                               const char** out_dptr);

/* Prediction from a dense float32 device array interface [N, F]
 * (class_model_native_adapter.cuh:30, class_study_train.cu:151-163).  config:
 * {"type": 0 value | 1 margin, "iteration_begin", "iteration_end" (rounds, 0 =
 * all), "strict_shape", "missing", "training", "cache_id"}.  Value type applies
 * the objective (logistic probability, softprob probabilities, softmax class
 * id).  *out_result is library-owned device memory valid until the next
 * prediction on this booster; proxy must be NULL. */
int XGBoosterPredictFromCudaArray(BoosterHandle handle, const char* values, const char* config,
                                  DMatrixHandle proxy, const bst_ulong** out_shape,
                                  bst_ulong* out_dim, const float** out_result);

/* XGBoost-3.4.1-schema JSON model from memory / a file (class_study_train.cu:
 * 92-99, class_model_native_adapter.cuh:28).  The booster then predicts and
 * exports; it cannot continue training. */
int XGBoosterLoadModelFromBuffer(BoosterHandle handle, const void* buf, bst_ulong len);
int XGBoosterLoadModel(BoosterHandle handle, const char* fname);

/* Feature count of the booster's model: num_feature of a trained or loaded
 * model, else of the first training matrix it was created with (0 with
 * neither).  The converter's native oracle checks it right after loading a
 * model (native/class_model_convert.cpp:112), as does the RL oracle
 * (native/rl/class_xgboost.hpp:64). */
int XGBoosterGetNumFeature(BoosterHandle handle, bst_ulong* out);

/* Rounds [begin_layer, end_layer) with step as a new booster (end 0 = all),
 * as the reference uses to clone a full-round view (class_study_train.cu:132). */
int XGBoosterSlice(BoosterHandle handle, int begin_layer, int end_layer, int step,
                   BoosterHandle* out);

/* ---- parity hooks on a booster (extensions) ---------------------------- */
typedef struct {
  int32_t n_nodes;
  const int32_t* left_children;
  const int32_t* right_children;
  const int32_t* parents;
  const int32_t* split_indices;
  const int32_t* split_bins;
  const float* split_conditions;
  const uint8_t* default_left;
  const float* base_weights;
  const float* loss_changes;
  const float* sum_hessian;
  const int64_t* sum_qg;
  const int64_t* sum_qh;
  const int64_t* row_counts; /* training rows reaching each node; -1 for loaded models */
} DPTreeView;

int DPBoosterNumTrees(BoosterHandle handle, int* out);
/* Host arrays owned by the booster, valid until the next training call. */
int DPBoosterGetTree(BoosterHandle handle, int tree, DPTreeView* out);
/* Training-cache margins [N][K] copied to host. */
int DPBoosterGetMargins(BoosterHandle handle, float* out, bst_ulong n);
/* Float gradients [N][K] and quantiser exponents [K][2] of the last round. */
int DPBoosterGetLastGradients(BoosterHandle handle, float* grad, float* hess, bst_ulong n,
                              int32_t* exps);
/* Final node id of every row in the last tree (the row partition). */
int DPBoosterGetLastPositions(BoosterHandle handle, int32_t* out, bst_ulong n);
/* JSON of the histogram launch shapes the last round used: the autotuner's
 * per-candidate timings and its choice for the root and gathered passes (or
 * {"forced":true} / {"defaults":true} when dp_hist_* / dp_autotune=0 set
 * them).  Library-owned string, valid until the next call on this booster. */
int DPBoosterGetTuning(BoosterHandle handle, bst_ulong* out_len, const char** out);

/* Validates and defaults a training-hyperparameter object the way the reference
 * does before training (class_native_training.cuh:16-33, via
 * ResidentTrainer::validate_hyperparameters, class_study_train.cu:203-206):
 * only rounds, max_depth, eta, lambda, alpha, gamma, min_child_weight, max_bin,
 * seed, subsample, colsample_by{tree,level,node}; rounds and max_depth required
 * positive integers (rounds <= INT_MAX / classes); max_bin >= 2 (default 256);
 * seed >= 0 (default 0); eta in (0, 1] (0.3); lambda, alpha, gamma,
 * min_child_weight finite >= 0 (1, 0, 0, 1); sampling keys in (0, 1] and kept
 * only when given.  Writes the normalised JSON (library-owned string, valid
 * until the next call on this thread). */
int DPValidateHyperparameters(const char* hyperparameters, uint32_t classes, bst_ulong* out_len,
                              const char** out);

/* Quantile cuts and bins the booster trained on (built at first use).
 * *missing_bin: -1 without missing values, 255 when every feature has at most
 * 255 bins (uint8 symbols, byte 255 = missing), 256 when the matrix has
 * missing values and some feature uses all 256 bins (16-bit symbols, 256 =
 * missing; the booster then builds every histogram from its present values). */
int DPDMatrixGetCuts(DMatrixHandle handle, int32_t max_bin, int32_t* cut_ptr,
                     float* cut_values, bst_ulong capacity, int32_t* missing_bin);

/* ======================================================================= */
/* 2. Kernel-level operator API                                             */
/* ======================================================================= */

typedef struct dp_workspace_s* dp_workspace;

/* Device scratch (work lists, partition counters) reused across calls.  A
 * workspace belongs to one device and must not be used by two streams at
 * once. */
int dp_workspace_create(dp_workspace* out);
int dp_workspace_free(dp_workspace ws);

typedef struct {
  int64_t n_rows;
  int32_t n_features;
  int32_t tile_width;   /* features per tile: 16 */
  int32_t n_tiles;
  int32_t missing_bin;  /* -1 when the matrix holds no NaN, else 255 */
  /* Bit t set: tiles t and t + 1 (t < 63) hold only bins below 16 and are
   * histogrammed together from their joint tile; no two set bits adjacent.
   * The k-th pair's joint tile is tile n_tiles + k of the bins buffer: per row
   * and feature slot i the byte (tile t's bin << 4) | tile t + 1's bin.
   * 0 from dp_layout_init; set by dp_layout_pair_tiles.  Histograms are the
   * same either way. */
  uint64_t paired_tiles;
} dp_bin_layout;

/* Fills `out`; tile_width 0 selects the default (16). */
int dp_layout_init(int64_t n_rows, int32_t n_features, int32_t tile_width, int32_t missing_bin,
                   dp_bin_layout* out);
/* Bytes of the bins buffer: n_tiles tiles of n_rows * 16 bytes (tile-major:
 * tile t holds 16 bytes per row), plus one joint tile per pair. */
size_t dp_layout_bytes(const dp_bin_layout* layout);

/* Sets layout->paired_tiles from the cuts (host cut_ptr [n_features + 1], as
 * dp_sketch_cuts returns): tiles are paired left to right, t with t + 1, when
 * every feature of both has at most 16 bins (pad features count as such); a
 * matrix with missing values gets none.  Call it before sizing the bins buffer
 * (dp_layout_bytes counts the joint tiles); dp_bin_values then writes the
 * joint tiles too.  The bins must come from these cuts (every byte of a paired
 * tile below 16; a larger byte gives wrong sums, never an access out of
 * bounds).  No counterpart in the reference: a layout choice of this library
 * (two tiles' histograms for the LDS atomics of one). */
int dp_layout_pair_tiles(dp_bin_layout* layout, const int32_t* cut_ptr);

/* Writes the joint tiles of layout->paired_tiles from the tiles they pair,
 * for bins made without dp_bin_values.  No counterpart in the reference. */
int dp_join_tiles(uint8_t* bins, const dp_bin_layout* layout, void* stream);

/* Exact quantile cuts of every feature (the definition is stated in the
 * implementation).  Host outputs: cut_ptr [n_features + 1], cut_values
 * [n_features * max_bin], min_values [n_features]; has_missing receives 1 when
 * any value is NaN.  Synchronous. */
int dp_sketch_cuts(dp_workspace ws, const float* values, int64_t n_rows, int32_t n_features,
                   int32_t max_bin, int32_t* cut_ptr, float* cut_values, float* min_values,
                   int32_t* has_missing, void* stream);

/* bins[r][f] = index of the first cut > x (clamped), missing_bin for NaN, in
 * the tile-major layout (and the joint tiles of a paired layout).
 * cut_ptr and cut_values are device arrays.  With missing_bin 255 every
 * feature must have at most 255 bins (byte 255 is the missing marker). */
int dp_bin_values(const float* values, const dp_bin_layout* layout, const int32_t* cut_ptr,
                  const float* cut_values, uint8_t* bins, void* stream);

enum dp_objective { DP_OBJ_LOGISTIC = 0, DP_OBJ_SOFTPROB = 1, DP_OBJ_SQUARED = 2 };

/* grad/hess [n_rows][n_classes] from margins [n_rows][n_classes] and labels. */
int dp_objective_gradients(int32_t objective, const float* margin, const float* label,
                           int64_t n_rows, int32_t n_classes, float* grad, float* hess,
                           void* stream);

/* Per class k: exp_k = 30 - e where max|x| < 2^e (frexp exponent),
 * q = rint(x * 2^exp_k).  Outputs: exps [n_classes][2] (g, h), gpair
 * [n_classes][n_rows][2], sums [n_classes][2] (int64 totals).  grad/hess are
 * [n_rows][n_classes]. */
int dp_quantise_gradients(dp_workspace ws, const float* grad, const float* hess,
                          int64_t n_rows, int32_t n_classes, int32_t* exps, int32_t* gpair,
                          int64_t* sums, void* stream);

/* Histograms of n_nodes row sets: node i covers ridx[begin[i], end[i]) (row
 * ids begin[i]..end[i]-1 when ridx is NULL).  begin/end are host arrays.
 * hist [n_nodes][n_features][bin_stride][2] is overwritten.  bin_stride >= the
 * largest bin index + 1 and <= 256.
 * Launch shape: calls with contiguous rows (ridx NULL) use the shape the
 * autotuner chose for this layout and bin stride.  The first such call of a
 * shape whose nodes hold at least 262,144 rows in all tunes it: once per
 * process, that call allocates device memory, times about 200 passes over the
 * matrix and synchronises `stream` before it returns.  Smaller calls never
 * tune (they take the tuned shape when there is one, else the defaults), nor
 * do gathered calls, so a caller that must not block can make its first large
 * call ahead of time. */
int dp_hist_build(dp_workspace ws, const uint8_t* bins, const dp_bin_layout* layout,
                  const int32_t* gpair, const uint32_t* ridx, const int64_t* begin,
                  const int64_t* end, int32_t n_nodes, int32_t bin_stride, int64_t* hist,
                  void* stream);

/* As dp_hist_build but adds into hist instead of overwriting it (batches of
 * rows, e.g. several device-resident row blocks, summed into one histogram). */
int dp_hist_accumulate(dp_workspace ws, const uint8_t* bins, const dp_bin_layout* layout,
                       const int32_t* gpair, const uint32_t* ridx, const int64_t* begin,
                       const int64_t* end, int32_t n_nodes, int32_t bin_stride, int64_t* hist,
                       void* stream);

/* The launch shape the autotuner chose for contiguous histograms of this
 * layout and bin stride (JSON: every candidate's time and the choice; "{}"
 * before the first contiguous dp_hist_build / dp_hist_accumulate of the
 * shape, which tunes it).  No counterpart in the reference.  Thread-local
 * string, valid until the next call on this thread. */
int dp_hist_tuning(const dp_bin_layout* layout, int32_t bin_stride, bst_ulong* out_len,
                   const char** out);

/* sibling = parent - built, element-wise over n int64 values. */
int dp_hist_subtract(const int64_t* parent, const int64_t* built, int64_t* sibling, int64_t n,
                     void* stream);

typedef struct {
  float eta, lambda, alpha, gamma, min_child_weight;
  int32_t max_depth;
} dp_train_param;

typedef struct {
  double loss_chg;        /* -inf when no valid candidate                  */
  int64_t gl, hl;         /* quantised sums of the left child              */
  int32_t feature, bin;   /* bins <= bin go left                           */
  int32_t default_left;   /* missing rows go left                          */
  int32_t valid;          /* a finite candidate exists                     */
  int32_t expand;         /* valid, loss_chg > 1e-6 and loss_chg >= gamma  */
  int32_t pad;
} dp_split_record;

/* Best split of every node.  node_sums int64 [n_nodes][2], n_bins int32
 * [n_features] (device); exps = (exp_g, exp_h) of the quantiser.  The
 * workspace provides the per-(node, feature) candidate scratch. */
int dp_evaluate_splits(dp_workspace ws, const int64_t* hist, int32_t n_nodes, int32_t n_features,
                       int32_t bin_stride, const int32_t* n_bins, const int64_t* node_sums,
                       int32_t exp_g, int32_t exp_h, const dp_train_param* param,
                       dp_split_record* out, void* stream);

/* As dp_evaluate_splits, but allocates nothing: no workspace, no hipMalloc,
 * no host synchronisation.  No counterpart in the reference; it is for
 * callers that cannot allocate (code under HIP graph capture, serving loops
 * that forbid hipMalloc).  The per-(node, feature) candidates live in a
 * library-owned device array of 16 MiB per GPU, so n_nodes * n_features must
 * not exceed 524,288 when n_features > 16 (with at most 16 features no
 * scratch is used); larger calls fail with an error.  Calls on one GPU share
 * that array: calls that overlap on one GPU (two streams or threads) race. */
int dp_evaluate_splits_noalloc(const int64_t* hist, int32_t n_nodes, int32_t n_features,
                               int32_t bin_stride, const int32_t* n_bins,
                               const int64_t* node_sums, int32_t exp_g, int32_t exp_h,
                               const dp_train_param* param, dp_split_record* out, void* stream);

/* Stable partition: for every node i with splits[i].expand, the rows
 * ridx_in[begin[i], end[i]) are written to ridx_out[begin[i], end[i]) with the
 * left child's rows first.  left_count [n_nodes] (device, int64) receives the
 * left sizes (0 for nodes that do not expand).  begin/end are host arrays. */
int dp_partition(dp_workspace ws, const uint8_t* bins, const dp_bin_layout* layout,
                 const uint32_t* ridx_in, uint32_t* ridx_out, const int64_t* begin,
                 const int64_t* end, const dp_split_record* splits, int32_t n_nodes,
                 int64_t* left_count, void* stream);

/* margin[ridx[i] * stride] += value[j] for i in [begin[j], end[j]); host
 * begin/end/value arrays of n_leaves entries. */
int dp_update_margin(dp_workspace ws, const uint32_t* ridx, const int64_t* begin,
                     const int64_t* end, const float* value, int32_t n_leaves, float* margin,
                     int64_t stride, void* stream);

/* ---- synthetic workloads (benchmark inputs; not part of the path) ------ */
/* config 1..5 as listed in the benchmark definition; writes values
 * [n_rows][n_features], labels [n_rows] and, for config 3, grad/hess [n_rows]
 * (NULL to skip).  Deterministic in (config, seed). */
int dp_synth(int32_t config, uint64_t seed, int64_t n_rows, int32_t n_features, float* values,
             float* labels, float* grad, float* hess, void* stream);

#ifdef __cplusplus
}
#endif
#endif
