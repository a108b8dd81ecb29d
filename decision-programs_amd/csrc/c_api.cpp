// extern "C" entry points declared in include/dpgbdt.h.
//
// Every entry point converts exceptions into status -1 and keeps the message
// for XGBGetLastError(), as the reference's adapter expects
// (native/class_model_native_adapter.cuh:23).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <memory>
#include <string>

#include "booster.hpp"
#include "json.hpp"
#include "tune.hpp"

namespace dp {
void launch_copy_matrix(const float* src, int64_t row_stride, int64_t n_rows, int32_t n_features,
                        float missing, float* dst, int32_t* bad, hipStream_t s);
}

namespace {

thread_local std::string g_last_error;

template <class F>
int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_last_error = e.what();
  } catch (...) {
    g_last_error = "unknown error";
  }
  return -1;
}

// A parsed __cuda_array_interface__-style JSON description (version 3).
struct ArrayInterface {
  uintptr_t data = 0;
  std::vector<int64_t> shape;
  std::vector<int64_t> strides;  // bytes; empty = C-contiguous
  std::string typestr;
};

ArrayInterface parse_array(const char* text) {
  dp::need(text != nullptr, "null array interface");
  dp::json::Value v = dp::json::parse(text);
  ArrayInterface a;
  const auto& data = v.at("data");
  dp::need(data.kind == dp::json::Value::Array && !data.items.empty(),
           "array interface data must be [pointer, readonly]");
  a.data = uintptr_t(data.items[0].u64());
  for (const auto& s : v.at("shape").items) a.shape.push_back(s.i64());
  if (const auto* st = v.find("strides"); st && st->kind == dp::json::Value::Array)
    for (const auto& s : st->items) a.strides.push_back(s.i64());
  a.typestr = v.at("typestr").text;
  return a;
}

struct DMatrixObj {
  dp::DMatrix m;
};

struct BoosterObj {
  std::unique_ptr<dp::Booster> b;
  std::string buffer;  // last returned string (model or config)
  std::vector<bst_ulong> shape;  // last prediction shape
};

dp::DMatrix& dm(DMatrixHandle h) {
  dp::need(h != nullptr, "null DMatrix handle");
  return static_cast<DMatrixObj*>(h)->m;
}

BoosterObj& bo(BoosterHandle h) {
  dp::need(h != nullptr, "null Booster handle");
  return *static_cast<BoosterObj*>(h);
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Kernels read these caller arrays in place, so a host, freed or foreign
// pointer would fault the GPU instead of failing the call: the array must be
// device memory of the current device (or managed memory), and `bytes` from p
// must lie inside its allocation.  The errors the queries leave on a refused
// pointer are cleared, so no later call reports them.
void require_device_array(uintptr_t p, size_t bytes, const char* what) {
  dp::need(p != 0, std::string(what) + " is a null pointer");
  hipPointerAttribute_t attr{};
  const hipError_t e = hipPointerGetAttributes(&attr, reinterpret_cast<const void*>(p));
  if (e != hipSuccess) (void)hipGetLastError();
  const bool managed = e == hipSuccess && (attr.type == hipMemoryTypeManaged || attr.isManaged);
  dp::need(e == hipSuccess && (attr.type == hipMemoryTypeDevice || managed),
           std::string(what) + " must be device memory (a HIP device or managed allocation)");
  if (managed) return;
  int device = 0;
  DP_HIP(hipGetDevice(&device));
  dp::need(attr.device == device, std::string(what) + " belongs to device " +
                                      std::to_string(attr.device) + ", not the current device " +
                                      std::to_string(device));
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  const hipError_t r = hipMemGetAddressRange(&base, &size, reinterpret_cast<hipDeviceptr_t>(p));
  if (r != hipSuccess) (void)hipGetLastError();
  const uintptr_t b = reinterpret_cast<uintptr_t>(base);
  dp::need(r == hipSuccess && p >= b && p - b <= size && bytes <= size - (p - b),
           std::string(what) + ": " + std::to_string(bytes) +
               " bytes from the pointer exceed its device allocation");
}

// Copies a float32 device array interface of shape [n] or [n, k] into dst.
void copy_float_array(const ArrayInterface& a, int64_t n, int64_t k, float* dst) {
  dp::need(a.typestr == "<f4", "array interface must be little-endian float32 (<f4)");
  int64_t elems = 1;
  for (int64_t s : a.shape) elems *= s;
  dp::need(elems == n * k, "array interface shape differs from the matrix");
  // One copy of `elems` floats: the strides, when given, must be the
  // C-contiguous strides of the whole shape (a column slice of a wider array,
  // e.g. [n, 1] with row stride 8, is refused rather than read as contiguous).
  if (!a.strides.empty()) {
    dp::need(a.strides.size() == a.shape.size(), "array interface strides differ from its shape");
    int64_t expect = 4;
    for (size_t d = a.shape.size(); d-- > 0;) {
      dp::need(a.shape[d] == 1 || a.strides[d] == expect, "array interface must be C-contiguous");
      expect *= a.shape[d];
    }
  }
  DP_HIP(hipMemcpy(dst, reinterpret_cast<const void*>(a.data), sizeof(float) * size_t(elems),
                   hipMemcpyDefault));
}

}  // namespace

// ===========================================================================
// Workspace
// ===========================================================================
dp_workspace_s::dp_workspace_s() {
  DP_HIP(hipGetDevice(&device));
  DP_HIP(hipEventCreateWithFlags(&staged_done, hipEventDisableTiming));
}

dp_workspace_s::~dp_workspace_s() {
  if (staged_done) {
    (void)hipEventSynchronize(staged_done);
    (void)hipEventDestroy(staged_done);
  }
}

void dp_workspace_s::begin(size_t staging_bytes) {
  DP_HIP(hipEventSynchronize(staged_done));
  staged_used = 0;
  scratch_used = 0;
  grow_staging(staging_bytes);
}

void dp_workspace_s::grow_staging(size_t bytes) {
  if (bytes <= staged_host.n && bytes <= staged_dev.n) return;
  // Growing would move data already staged in this call: the caller must
  // size the call in begin().
  dp::need(staged_used == 0, "workspace staging exceeded the size given to begin()");
  size_t cap = 1 << 20;
  while (cap < bytes) cap <<= 1;
  staged_host.reserve(cap);
  staged_dev.reserve(cap);
  committed_.clear();  // the device area is new
}

void dp_workspace_s::commit(hipStream_t stream) {
  if (staged_used && !(staged_used == committed_.size() &&
                       std::memcmp(staged_host.p, committed_.data(), staged_used) == 0)) {
    DP_HIP(hipMemcpyAsync(staged_dev.p, staged_host.p, staged_used, hipMemcpyHostToDevice, stream));
    committed_.assign(staged_host.p, staged_host.p + staged_used);
  }
  DP_HIP(hipEventRecord(staged_done, stream));
}

void dp_workspace_s::reserve_scratch(size_t bytes) {
  dp::need(scratch_used == 0, "scratch must be reserved before it is taken");
  if (bytes > scratch.n) {
    size_t cap = 1 << 20;
    while (cap < bytes) cap <<= 1;
    scratch.resize(cap);
  }
}

void dp_workspace_s::need_scratch(size_t bytes) {
  dp::fail("workspace scratch too small: " + std::to_string(bytes) + " bytes needed");
}

extern "C" {

// ===========================================================================
// XGBoost C-API subset
// ===========================================================================
void XGBoostVersion(int* major, int* minor, int* patch) {
  if (major) *major = 3;
  if (minor) *minor = 4;
  if (patch) *patch = 1;
}

int XGBuildInfo(const char** out) {
  static const char* info =
      "{\"USE_CUDA\":true,\"USE_HIP\":true,\"USE_NCCL\":false,\"USE_RCCL\":false,"
      "\"USE_OPENMP\":false,\"GPU_ARCH\":\"gfx950\",\"IMPLEMENTATION\":\"dp-gbdt-mi355x\","
      "\"NOTE\":\"USE_CUDA reports a device (HIP) training path for API compatibility\"}";
  return guarded([&] {
    dp::need(out != nullptr, "null output pointer");
    *out = info;
  });
}

const char* XGBGetLastError(void) { return g_last_error.c_str(); }

int XGDMatrixCreateFromCudaArrayInterface(const char* data, const char* config,
                                          DMatrixHandle* out) {
  return guarded([&] {
    dp::need(out != nullptr, "null output handle");
    ArrayInterface a = parse_array(data);
    dp::need(a.typestr == "<f4", "matrix must be little-endian float32 (<f4)");
    dp::need(a.shape.size() == 2 && a.shape[0] > 0 && a.shape[1] > 0, "matrix shape must be [N, F]");
    float missing = std::nanf("");
    if (config) {
      dp::json::Value c = dp::json::parse(config);
      if (const auto* m = c.find("missing")) missing = float(m->number());
    }
    const int64_t n = a.shape[0], f = a.shape[1];
    dp::need(f <= INT32_MAX && n <= int64_t(UINT32_MAX), "matrix too large for uint32 row ids");
    int64_t row_stride = f;
    if (!a.strides.empty()) {
      dp::need(a.strides.size() == 2 && a.strides[1] == 4 && a.strides[0] % 4 == 0 &&
                   a.strides[0] >= 4 * f,
               "unsupported matrix strides");
      row_stride = a.strides[0] / 4;
    }
    require_device_array(a.data, sizeof(float) * size_t((n - 1) * row_stride + f), "matrix data");
    auto obj = std::make_unique<DMatrixObj>();
    obj->m.n_rows = n;
    obj->m.n_features = int32_t(f);
    obj->m.values.resize(size_t(n * f));
    dp::DeviceBuffer<int32_t> bad(1);
    hipStream_t s = nullptr;
    dp::launch_copy_matrix(reinterpret_cast<const float*>(a.data), row_stride, n, int32_t(f),
                           missing, obj->m.values.p, bad.p, s);
    int32_t flag = 0;
    DP_HIP(hipMemcpy(&flag, bad.p, sizeof flag, hipMemcpyDeviceToHost));
    dp::need(flag == 0, "input data contains inf");
    *out = obj.release();
  });
}

int XGDMatrixSetInfoFromInterface(DMatrixHandle handle, const char* field, const char* data) {
  return guarded([&] {
    dp::DMatrix& m = dm(handle);
    dp::need(field && std::string(field) == "label", "only the label field is supported");
    ArrayInterface a = parse_array(data);
    m.labels.resize(size_t(m.n_rows));
    copy_float_array(a, m.n_rows, 1, m.labels.p);
    m.has_labels = true;
  });
}

int XGDMatrixNumRow(DMatrixHandle handle, bst_ulong* out) {
  return guarded([&] { *out = bst_ulong(dm(handle).n_rows); });
}

int XGDMatrixNumCol(DMatrixHandle handle, bst_ulong* out) {
  return guarded([&] { *out = bst_ulong(dm(handle).n_features); });
}

int XGDMatrixFree(DMatrixHandle handle) {
  return guarded([&] {
    auto* obj = static_cast<DMatrixObj*>(handle);
    if (obj) obj->m.release_pending();  // rounds in flight still read the matrix
    delete obj;
  });
}

int XGBoosterCreate(const DMatrixHandle dmats[], bst_ulong len, BoosterHandle* out) {
  return guarded([&] {
    dp::need(out != nullptr, "null output handle");
    std::vector<dp::DMatrix*> cache;
    for (bst_ulong i = 0; i < len; ++i) cache.push_back(&dm(dmats[i]));
    auto obj = std::make_unique<BoosterObj>();
    obj->b = std::make_unique<dp::Booster>(std::move(cache));
    *out = obj.release();
  });
}

int XGBoosterFree(BoosterHandle handle) {
  return guarded([&] { delete static_cast<BoosterObj*>(handle); });
}

int XGBoosterSetParam(BoosterHandle handle, const char* name, const char* value) {
  return guarded([&] {
    dp::need(name && value, "null parameter");
    bo(handle).b->set_param(name, value);
  });
}

int XGBoosterUpdateOneIter(BoosterHandle handle, int iter, DMatrixHandle dtrain) {
  return guarded([&] { bo(handle).b->update_one_iter(iter, &dm(dtrain)); });
}

int XGBoosterTrainOneIter(BoosterHandle handle, DMatrixHandle dtrain, int iter, const char* grad,
                          const char* hess) {
  return guarded([&] {
    ArrayInterface g = parse_array(grad), h = parse_array(hess);
    dp::need(g.typestr == "<f4" && h.typestr == "<f4", "gradients must be float32");
    dp::need(g.shape == h.shape && !g.shape.empty() && g.shape.size() <= 2,
             "gradient and hessian shapes differ");
    dp::need(g.strides.empty() && h.strides.empty(), "gradients must be C-contiguous");
    const int64_t n = g.shape[0];
    const int32_t k = g.shape.size() == 2 ? int32_t(g.shape[1]) : 1;
    dp::need(n > 0 && k > 0 && n <= INT64_MAX / 4 / k, "gradient shape out of range");
    // The round's quantiser reads both arrays in place.
    require_device_array(g.data, sizeof(float) * size_t(n) * size_t(k), "grad");
    require_device_array(h.data, sizeof(float) * size_t(n) * size_t(k), "hess");
    bo(handle).b->train_one_iter(&dm(dtrain), iter, reinterpret_cast<const float*>(g.data),
                                 reinterpret_cast<const float*>(h.data), n, k);
  });
}

int XGBoosterBoostedRounds(BoosterHandle handle, int* out) {
  return guarded([&] { *out = bo(handle).b->boosted_rounds(); });
}

int XGBoosterSaveJsonConfig(BoosterHandle handle, bst_ulong* out_len, const char** out_str) {
  return guarded([&] {
    BoosterObj& b = bo(handle);
    b.buffer = b.b->save_config();
    *out_len = b.buffer.size();
    *out_str = b.buffer.c_str();
  });
}

int XGBoosterSaveModel(BoosterHandle handle, const char* fname) {
  return guarded([&] {
    dp::need(fname != nullptr, "null file name");
    const std::string text = bo(handle).b->save_model();
    std::ofstream f(fname, std::ios::binary | std::ios::trunc);
    dp::need(bool(f), std::string("cannot open ") + fname);
    f.write(text.data(), std::streamsize(text.size()));
    dp::need(bool(f), std::string("cannot write ") + fname);
  });
}

int XGBoosterSaveModelToBuffer(BoosterHandle handle, const char* config, bst_ulong* out_len,
                               const char** out_dptr) {
  return guarded([&] {
    if (config) {
      dp::json::Value c = dp::json::parse(config);
      if (const auto* f = c.find("format")) dp::need(f->text == "json", "only json format");
    }
    BoosterObj& b = bo(handle);
    b.buffer = b.b->save_model();
    *out_len = b.buffer.size();
    *out_dptr = b.buffer.c_str();
  });
}

int XGBoosterPredictFromCudaArray(BoosterHandle handle, const char* values, const char* config,
                                  DMatrixHandle proxy, const bst_ulong** out_shape,
                                  bst_ulong* out_dim, const float** out_result) {
  return guarded([&] {
    dp::need(out_shape && out_dim && out_result, "null output pointer");
    dp::need(proxy == nullptr, "proxy DMatrix is not supported; pass NULL");
    BoosterObj& b = bo(handle);
    ArrayInterface a = parse_array(values);
    dp::need(a.typestr == "<f4", "prediction input must be float32 (<f4)");
    dp::need(a.shape.size() == 2, "prediction input must be [N, F]");
    dp::PredictRequest req;
    req.values = reinterpret_cast<const float*>(a.data);
    req.rows = a.shape[0];
    req.features = int32_t(a.shape[1]);
    req.row_stride = a.shape[1];
    if (!a.strides.empty()) {
      dp::need(a.strides.size() == 2 && a.strides[1] == 4 && a.strides[0] % 4 == 0,
               "unsupported input strides");
      req.row_stride = a.strides[0] / 4;
    }
    req.missing = std::nanf("");
    if (config) {
      dp::json::Value c = dp::json::parse(config);
      if (const auto* v = c.find("type")) req.type = int32_t(v->i64());
      if (const auto* v = c.find("iteration_begin")) req.iteration_begin = int32_t(v->i64());
      if (const auto* v = c.find("iteration_end")) req.iteration_end = int32_t(v->i64());
      if (const auto* v = c.find("strict_shape")) req.strict_shape = v->boolean;
      if (const auto* v = c.find("missing")) req.missing = float(v->number());
    }
    if (req.rows > 0 && req.features > 0)
      require_device_array(a.data,
                           sizeof(float) * size_t((req.rows - 1) * req.row_stride + req.features),
                           "prediction input");
    std::vector<uint64_t> shape;
    *out_result = b.b->predict(req, shape);
    b.shape.assign(shape.begin(), shape.end());
    *out_shape = b.shape.data();
    *out_dim = b.shape.size();
  });
}

int XGBoosterLoadModelFromBuffer(BoosterHandle handle, const void* buf, bst_ulong len) {
  return guarded([&] {
    dp::need(buf != nullptr, "null model buffer");
    bo(handle).b->load_model(std::string(static_cast<const char*>(buf), size_t(len)));
  });
}

int XGBoosterLoadModel(BoosterHandle handle, const char* fname) {
  return guarded([&] {
    dp::need(fname != nullptr, "null file name");
    std::ifstream f(fname, std::ios::binary);
    dp::need(bool(f), std::string("cannot open ") + fname);
    std::string text((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    bo(handle).b->load_model(text);
  });
}

int XGBoosterGetNumFeature(BoosterHandle handle, bst_ulong* out) {
  return guarded([&] {
    dp::need(out != nullptr, "null output pointer");
    *out = bst_ulong(bo(handle).b->num_features());
  });
}

int XGBoosterSlice(BoosterHandle handle, int begin_layer, int end_layer, int step,
                   BoosterHandle* out) {
  return guarded([&] {
    dp::need(out != nullptr, "null output handle");
    auto obj = std::make_unique<BoosterObj>();
    obj->b = bo(handle).b->slice(begin_layer, end_layer, step);
    *out = obj.release();
  });
}

// ---- parity hooks --------------------------------------------------------
int DPBoosterNumTrees(BoosterHandle handle, int* out) {
  return guarded([&] { *out = int(bo(handle).b->trees().size()); });
}

int DPBoosterGetTree(BoosterHandle handle, int tree, DPTreeView* out) {
  return guarded([&] {
    const auto& trees = bo(handle).b->trees();
    dp::need(tree >= 0 && size_t(tree) < trees.size(), "tree index out of range");
    const dp::Tree& t = trees[size_t(tree)];
    out->n_nodes = t.size();
    out->left_children = t.left.data();
    out->right_children = t.right.data();
    out->parents = t.parent.data();
    out->split_indices = t.feature.data();
    out->split_bins = t.split_bin.data();
    out->split_conditions = t.cond.data();
    out->default_left = t.default_left.data();
    out->base_weights = t.base_weight.data();
    out->loss_changes = t.loss_chg.data();
    out->sum_hessian = t.sum_hess.data();
    out->sum_qg = t.sum_qg.data();
    out->sum_qh = t.sum_qh.data();
    out->row_counts = t.rows.data();
  });
}

int DPBoosterGetMargins(BoosterHandle handle, float* out, bst_ulong n) {
  return guarded([&] { bo(handle).b->margins(out, size_t(n)); });
}

int DPBoosterGetLastGradients(BoosterHandle handle, float* grad, float* hess, bst_ulong n,
                              int32_t* exps) {
  return guarded([&] { bo(handle).b->last_gradients(grad, hess, size_t(n), exps); });
}

int DPBoosterGetLastPositions(BoosterHandle handle, int32_t* out, bst_ulong n) {
  return guarded([&] { bo(handle).b->last_positions(out, size_t(n)); });
}

int DPBoosterGetTuning(BoosterHandle handle, bst_ulong* out_len, const char** out) {
  return guarded([&] {
    dp::need(out_len && out, "null argument");
    BoosterObj& b = bo(handle);
    b.buffer = b.b->tuning();
    *out = b.buffer.c_str();
    *out_len = bst_ulong(b.buffer.size());
  });
}

int DPValidateHyperparameters(const char* hyperparameters, uint32_t classes, bst_ulong* out_len,
                              const char** out) {
  static thread_local std::string result;
  return guarded([&] {
    dp::need(hyperparameters && out_len && out, "null argument");
    dp::need(classes >= 1, "classes must be positive");
    result = dp::validate_hyperparameters(hyperparameters, classes);
    *out_len = result.size();
    *out = result.c_str();
  });
}

int DPDMatrixGetCuts(DMatrixHandle handle, int32_t max_bin, int32_t* cut_ptr, float* cut_values,
                     bst_ulong capacity, int32_t* missing_bin) {
  return guarded([&] {
    dp::DMatrix& m = dm(handle);
    auto it = m.quantized.find(max_bin);
    dp::need(it != m.quantized.end(), "matrix has not been quantised with this max_bin");
    const dp::Quantized& q = *it->second;
    dp::need(capacity >= q.cut_values.size(), "cut buffer too small");
    std::copy(q.cut_ptr.begin(), q.cut_ptr.end(), cut_ptr);
    std::copy(q.cut_values.begin(), q.cut_values.end(), cut_values);
    if (missing_bin) *missing_bin = q.layout.missing_bin;
  });
}

// ===========================================================================
// Kernel-level operator API
// ===========================================================================
int dp_workspace_create(dp_workspace* out) {
  return guarded([&] {
    dp::need(out != nullptr, "null output");
    *out = new dp_workspace_s();
  });
}

int dp_workspace_free(dp_workspace ws) {
  return guarded([&] { delete ws; });
}

int dp_layout_init(int64_t n_rows, int32_t n_features, int32_t tile_width, int32_t missing_bin,
                   dp_bin_layout* out) {
  return guarded([&] {
    dp::need(out != nullptr, "null layout");
    dp::need(n_rows > 0 && n_features > 0, "layout needs rows and features");
    dp::need(missing_bin == -1 || missing_bin == 255, "missing_bin must be -1 or 255");
    if (tile_width == 0) tile_width = 16;
    dp::need(tile_width == 16, "tile_width must be 16");
    out->n_rows = n_rows;
    out->n_features = n_features;
    out->tile_width = tile_width;
    out->n_tiles = (n_features + tile_width - 1) / tile_width;
    out->missing_bin = missing_bin;
    out->paired_tiles = 0;
  });
}

int dp_layout_pair_tiles(dp_bin_layout* layout, const int32_t* cut_ptr) {
  return guarded([&] {
    dp::need(layout && cut_ptr, "null argument");
    dp::need(layout->n_features > 0 && layout->tile_width == 16 &&
                 layout->n_tiles == (layout->n_features + 15) / 16,
             "layout not initialised");
    std::vector<int32_t> n_bins(size_t(layout->n_features));
    for (int32_t f = 0; f < layout->n_features; ++f) {
      n_bins[size_t(f)] = cut_ptr[f + 1] - cut_ptr[f];
      dp::need(n_bins[size_t(f)] >= 0, "cut_ptr must not decrease");
    }
    layout->paired_tiles = dp::pair_tiles(n_bins.data(), layout->n_features, layout->n_tiles,
                                          layout->missing_bin >= 0);
  });
}

size_t dp_layout_bytes(const dp_bin_layout* layout) {
  if (!layout) return 0;
  const size_t tiles = size_t(layout->n_tiles) + size_t(__builtin_popcountll(layout->paired_tiles));
  return tiles * size_t(layout->n_rows) * size_t(layout->tile_width);
}

// A paired layout's buffer holds joint tiles after the matrix's tiles; a
// buffer sized before the layout was paired would be read past its end.
static void require_paired_bins(const uint8_t* bins, const dp_bin_layout& layout) {
  if (!layout.paired_tiles) return;
  dp::check_pairs(layout);
  require_device_array(reinterpret_cast<uintptr_t>(bins), dp_layout_bytes(&layout),
                       "bins of a paired layout (dp_layout_bytes counts its joint tiles; "
                       "pair the layout before sizing the buffer)");
}

int dp_join_tiles(uint8_t* bins, const dp_bin_layout* layout, void* stream) {
  return guarded([&] {
    dp::need(bins && layout, "null argument");
    require_paired_bins(bins, *layout);
    dp::launch_join_tiles(bins, *layout, as_stream(stream));
  });
}

int dp_sketch_cuts(dp_workspace ws, const float* values, int64_t n_rows, int32_t n_features,
                   int32_t max_bin, int32_t* cut_ptr, float* cut_values, float* min_values,
                   int32_t* has_missing, void* stream) {
  return guarded([&] {
    dp::need(ws && values && cut_ptr && cut_values && min_values && has_missing, "null argument");
    dp::sketch_cuts(*ws, values, n_rows, n_features, max_bin, cut_ptr, cut_values, min_values,
                    has_missing, as_stream(stream));
  });
}

int dp_bin_values(const float* values, const dp_bin_layout* layout, const int32_t* cut_ptr,
                  const float* cut_values, uint8_t* bins, void* stream) {
  return guarded([&] {
    dp::need(values && layout && cut_ptr && cut_values && bins, "null argument");
    require_paired_bins(bins, *layout);
    dp::launch_bin_values(values, *layout, cut_ptr, cut_values, bins, as_stream(stream));
    dp::launch_join_tiles(bins, *layout, as_stream(stream));
  });
}

int dp_objective_gradients(int32_t objective, const float* margin, const float* label,
                           int64_t n_rows, int32_t n_classes, float* grad, float* hess,
                           void* stream) {
  return guarded([&] {
    dp::need(margin && label && grad && hess, "null argument");
    dp::need(n_classes >= 1, "n_classes must be positive");
    dp::need(objective != DP_OBJ_SOFTPROB || n_classes >= 2, "softprob needs 2+ classes");
    dp::need(objective == DP_OBJ_SOFTPROB || n_classes == 1, "single-output objective");
    // No leaf values: the margins are only read.
    dp::launch_gradients(objective, const_cast<float*>(margin), label, n_rows, n_classes, grad,
                         hess, nullptr, as_stream(stream));
  });
}

int dp_quantise_gradients(dp_workspace ws, const float* grad, const float* hess, int64_t n_rows,
                          int32_t n_classes, int32_t* exps, int32_t* gpair, int64_t* sums,
                          void* stream) {
  return guarded([&] {
    dp::need(ws && grad && hess && exps && gpair && sums, "null argument");
    dp::need(n_rows >= 1 && n_classes >= 1, "empty gradients");
    ws->begin();
    const size_t bytes = dp::quantise_scratch_bytes(n_rows, n_classes);
    ws->reserve_scratch(bytes + 256);
    void* scratch = ws->take<uint8_t>(bytes);
    dp::launch_quantise(grad, hess, n_rows, n_classes, scratch, false, exps, gpair, sums,
                        as_stream(stream));
    ws->commit(as_stream(stream));
  });
}

namespace {
void hist_call(dp_workspace ws, const uint8_t* bins, const dp_bin_layout* layout,
               const int32_t* gpair, const uint32_t* ridx, const int64_t* begin,
               const int64_t* end, int32_t n_nodes, int32_t bin_stride, int64_t* hist,
               void* stream, bool accumulate) {
  dp::need(ws && bins && layout && gpair && begin && end && hist, "null argument");
  require_paired_bins(bins, *layout);
  dp::need(n_nodes >= 0, "negative node count");
  dp::need(bin_stride >= 1 && bin_stride <= dp::kMaxBins, "bin_stride must be in [1, 256]");
  int64_t total = 0;
  for (int32_t i = 0; i < n_nodes; ++i) {
    dp::need(begin[i] >= 0 && begin[i] <= end[i], "node segment out of order");
    dp::need(ridx != nullptr || end[i] <= layout->n_rows, "row range beyond the matrix");
    total += end[i] - begin[i];
  }
  hipStream_t s = as_stream(stream);
  // Contiguous row ranges take the launch shape the autotuner chose for this
  // matrix shape.  The first such call of a shape that covers at least
  // kTuneMinRows rows times the candidates on these bins (once per process:
  // it allocates, launches about 200 timing passes and synchronises the
  // stream); smaller calls use the shape tuned already, else the defaults.
  // Gathered calls read the tile-major bins and keep the default shape.
  constexpr int64_t kTuneMinRows = int64_t(1) << 18;
  dp::HistConfig cfg;
  if (!ridx) {
    if (const dp::HistTuning* t = dp::find_dense_tuning(*layout, bin_stride, false))
      cfg = t->root;
    else if (total >= kTuneMinRows)
      cfg = dp::tune_dense_hist(*layout, bins, false, bin_stride, gpair, s).root;
  }
  std::vector<dp::HistWork> work;
  std::vector<dp::HistReduce> jobs;
  // Overwriting builds let single-chunk nodes store their histogram directly;
  // accumulating calls route every chunk through a partial slot.
  const int32_t n_partial = dp::make_hist_work(*layout, begin, end, nullptr, n_nodes, !accumulate,
                                               work, jobs, 0, cfg);
  const size_t partial_words = size_t(n_partial) * size_t(bin_stride) * 32;
  ws->begin(sizeof(dp::HistWork) * work.size() + sizeof(dp::HistReduce) * jobs.size() + 512);
  ws->reserve_scratch(sizeof(int64_t) * partial_words + 256);
  dp::HistWork* d_work;
  dp::HistReduce* d_jobs;
  std::copy(work.begin(), work.end(), ws->stage(work.size(), &d_work));
  std::copy(jobs.begin(), jobs.end(), ws->stage(jobs.size(), &d_jobs));
  ws->commit(s);
  int64_t* partial = partial_words ? ws->take<int64_t>(partial_words) : nullptr;
  dp::launch_hist(bins, *layout, gpair, ridx, d_work, int32_t(work.size()), nullptr, bin_stride,
                  hist, partial, s, nullptr, cfg);
  dp::launch_hist_reduce(partial, d_jobs, n_nodes, nullptr, layout->n_tiles, layout->n_features,
                         bin_stride, nullptr, hist, accumulate, s);
}
}  // namespace

int dp_hist_build(dp_workspace ws, const uint8_t* bins, const dp_bin_layout* layout,
                  const int32_t* gpair, const uint32_t* ridx, const int64_t* begin,
                  const int64_t* end, int32_t n_nodes, int32_t bin_stride, int64_t* hist,
                  void* stream) {
  return guarded([&] {
    hist_call(ws, bins, layout, gpair, ridx, begin, end, n_nodes, bin_stride, hist, stream, false);
  });
}

int dp_hist_accumulate(dp_workspace ws, const uint8_t* bins, const dp_bin_layout* layout,
                       const int32_t* gpair, const uint32_t* ridx, const int64_t* begin,
                       const int64_t* end, int32_t n_nodes, int32_t bin_stride, int64_t* hist,
                       void* stream) {
  return guarded([&] {
    hist_call(ws, bins, layout, gpair, ridx, begin, end, n_nodes, bin_stride, hist, stream, true);
  });
}

int dp_hist_tuning(const dp_bin_layout* layout, int32_t bin_stride, bst_ulong* out_len,
                   const char** out) {
  static thread_local std::string result;
  return guarded([&] {
    dp::need(layout && out_len && out, "null argument");
    const dp::HistTuning* t = dp::find_dense_tuning(*layout, bin_stride, false);
    result = t ? t->report : "{}";
    *out = result.c_str();
    *out_len = bst_ulong(result.size());
  });
}

int dp_hist_subtract(const int64_t* parent, const int64_t* built, int64_t* sibling, int64_t n,
                     void* stream) {
  return guarded([&] {
    dp::need(parent && built && sibling, "null argument");
    dp::launch_subtract(parent, built, sibling, n, as_stream(stream));
  });
}

int dp_evaluate_splits(dp_workspace ws, const int64_t* hist, int32_t n_nodes,
                       int32_t n_features, int32_t bin_stride, const int32_t* n_bins,
                       const int64_t* node_sums, int32_t exp_g, int32_t exp_h,
                       const dp_train_param* param, dp_split_record* out, void* stream) {
  return guarded([&] {
    dp::need(ws && hist && n_bins && node_sums && param && out, "null argument");
    dp::need(n_nodes >= 0 && n_features >= 1, "node and feature counts");
    if (n_nodes == 0) return;
    const size_t bytes = dp::evaluate_scratch_bytes(n_nodes, n_features);
    ws->begin(0);
    ws->reserve_scratch(bytes + 256);
    void* scratch = ws->take<uint8_t>(bytes);
    dp::launch_evaluate(hist, n_nodes, nullptr, n_features, bin_stride, n_bins, node_sums, nullptr,
                        exp_g, exp_h, *param, scratch, out, as_stream(stream));
  });
}

int dp_evaluate_splits_noalloc(const int64_t* hist, int32_t n_nodes, int32_t n_features,
                               int32_t bin_stride, const int32_t* n_bins,
                               const int64_t* node_sums, int32_t exp_g, int32_t exp_h,
                               const dp_train_param* param, dp_split_record* out, void* stream) {
  return guarded([&] {
    dp::need(hist && n_bins && node_sums && param && out, "null argument");
    dp::need(n_nodes >= 0 && n_features >= 1, "node and feature counts");
    if (n_nodes == 0) return;
    // The candidates go to the library's device array: no workspace, no
    // allocation, no host synchronisation.
    const size_t bytes =
        n_features > dp::kEvalNodeFeatures ? dp::evaluate_scratch_bytes(n_nodes, n_features) : 0;
    void* scratch = dp::noalloc_scratch(bytes);
    dp::launch_evaluate(hist, n_nodes, nullptr, n_features, bin_stride, n_bins, node_sums, nullptr,
                        exp_g, exp_h, *param, scratch, out, as_stream(stream));
  });
}

int dp_partition(dp_workspace ws, const uint8_t* bins, const dp_bin_layout* layout,
                 const uint32_t* ridx_in, uint32_t* ridx_out, const int64_t* begin,
                 const int64_t* end, const dp_split_record* splits, int32_t n_nodes,
                 int64_t* left_count, void* stream) {
  return guarded([&] {
    dp::need(ws && bins && layout && ridx_in && ridx_out && begin && end && splits && left_count,
             "null argument");
    std::vector<dp::PartWork> work;
    std::vector<int32_t> first(static_cast<size_t>(n_nodes) + 1);
    for (int32_t i = 0; i < n_nodes; ++i) {
      dp::need(begin[i] >= 0 && begin[i] <= end[i], "node segment out of order");
      first[size_t(i)] = int32_t(work.size());
      for (int64_t b = begin[i]; b < end[i]; b += dp::kPartChunk)
        work.push_back({i, 0, b, std::min(b + dp::kPartChunk, end[i])});
    }
    first[size_t(n_nodes)] = int32_t(work.size());
    hipStream_t s = as_stream(stream);
    ws->begin(sizeof(dp::PartWork) * work.size() + sizeof(int64_t) * size_t(n_nodes) +
              sizeof(int32_t) * first.size() + 3 * 256);
    ws->reserve_scratch((sizeof(int64_t) + sizeof(uint64_t) * dp::kPartMasks) * work.size() +
                        2048);
    dp::PartWork* d_work;
    int64_t* d_begin;
    int32_t* d_first;
    std::copy(work.begin(), work.end(), ws->stage(work.size(), &d_work));
    std::copy(begin, begin + n_nodes, ws->stage(size_t(n_nodes), &d_begin));
    std::copy(first.begin(), first.end(), ws->stage(first.size(), &d_first));
    ws->commit(s);
    int64_t* work_left = ws->take<int64_t>(work.size());
    auto* masks = ws->take<unsigned long long>(work.size() * dp::kPartMasks);
    // the records are only read: no SplitSelect is passed
    dp::launch_partition(bins, nullptr, *layout, ridx_in, ridx_out, d_work, int32_t(work.size()),
                         nullptr, d_begin, const_cast<dp_split_record*>(splits), d_first, n_nodes,
                         nullptr, work_left, masks, left_count, false, s);
  });
}

int dp_update_margin(dp_workspace ws, const uint32_t* ridx, const int64_t* begin,
                     const int64_t* end, const float* value, int32_t n_leaves, float* margin,
                     int64_t stride, void* stream) {
  return guarded([&] {
    dp::need(ws && ridx && begin && end && value && margin, "null argument");
    std::vector<dp::LeafWork> work;
    for (int32_t i = 0; i < n_leaves; ++i)
      for (int64_t b = begin[i]; b < end[i]; b += dp::kLeafChunk)
        work.push_back({value[i], i, b, std::min(b + dp::kLeafChunk, end[i])});
    hipStream_t s = as_stream(stream);
    ws->begin(sizeof(dp::LeafWork) * work.size() + 256);
    dp::LeafWork* d_work;
    std::copy(work.begin(), work.end(), ws->stage(work.size(), &d_work));
    ws->commit(s);
    dp::launch_update_margin(ridx, d_work, int32_t(work.size()), nullptr, margin, stride, s);
  });
}

int dp_synth(int32_t config, uint64_t seed, int64_t n_rows, int32_t n_features, float* values,
             float* labels, float* grad, float* hess, void* stream) {
  return guarded([&] {
    dp::launch_synth(config, seed, n_rows, n_features, values, labels, grad, hess,
                     as_stream(stream));
  });
}

}  // extern "C"
