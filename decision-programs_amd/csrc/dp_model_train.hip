// dp_model_train: the FIT-only training process of the reference's
// class_model_train (native/class_model_train.cu:38-86), built for MI355X.
//
//   dp_model_train source-manifest
//   dp_model_train --check-plan PLAN SHA
//   dp_model_train fit PLAN SHA NEW_OUT
//
// A plan (format class-model-training-plan-1) binds a dense FP32 / uint32
// class-label dataset, the numerical library and this executable by SHA-256;
// `fit` checks every pin, stages the FIT rows on the GPU, drives the
// XGBoost-compatible C API of the pinned library (dlopen, as
// native/class_model_native_adapter.cuh:22-24 does) for `rounds` multi:softmax
// rounds, and writes plan.json, source-manifest.json, model.json,
// configuration.json, result.json and result-seal.json into a fresh
// directory, or failure.json when a step fails after the directory exists.
// Exit status 0 on success, 1 with the message on stderr otherwise.
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <charconv>
#include <chrono>
#include <climits>
#include <cstdint>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

#include "json.hpp"
#include "sha256.hpp"

namespace fs = std::filesystem;
using dp::json::Value;
using dp::need;

namespace {

constexpr uint64_t kMaxExactClasses = 16777217ULL;  // labels are exact in FP32 up to 2^24 + 1

// ---- files ------------------------------------------------------------------
void check_path(const fs::path& p) {
  need(p.is_absolute() && p.string().find('\0') == std::string::npos,
       "absolute dataset or output path required");
  (void)fs::weakly_canonical(p);
}

std::string read_file(const fs::path& p) {
  std::ifstream f(p, std::ios::binary | std::ios::ate);
  need(bool(f), "input read failed: " + p.string());
  const auto n = f.tellg();
  need(n >= 0, "input extent");
  std::string s(size_t(n), '\0');
  f.seekg(0);
  if (n) f.read(s.data(), n);
  need(bool(f) && f.peek() == EOF, "input read incomplete: " + p.string());
  return s;
}

// Writes through a temporary file and a rename, so a reader never sees a
// partial receipt.
void atomic_text(const fs::path& p, const std::string& text) {
  const fs::path tmp = p.string() + ".tmp";
  {
    std::ofstream f(tmp, std::ios::binary | std::ios::trunc);
    need(bool(f), "cannot write " + tmp.string());
    f.write(text.data(), std::streamsize(text.size()));
    f.flush();
    need(bool(f), "write failed: " + tmp.string());
  }
  fs::rename(tmp, p);
}

void atomic_json(const fs::path& p, const Value& v) { atomic_text(p, dp::json::dump(v, 2) + "\n"); }

void clean_output(const fs::path& p) {
  need(!fs::exists(p), "output already exists");
  fs::create_directories(p);
}

// ---- JSON helpers -------------------------------------------------------------
uint64_t unsigned_integer(const Value& v, const std::string& message) {
  need(v.kind == Value::Number && v.text.find_first_of(".eEnNI-") == std::string::npos, message);
  uint64_t x = 0;
  const char* b = v.text.data() + (v.text[0] == '+');
  auto r = std::from_chars(b, v.text.data() + v.text.size(), x);
  need(r.ec == std::errc() && r.ptr == v.text.data() + v.text.size(), message);
  return x;
}

bool is_false(const Value* v) { return v && v->kind == Value::Bool && !v->boolean; }
bool is_true(const Value* v) { return v && v->kind == Value::Bool && v->boolean; }

const std::string& text_of(const Value& v, const std::string& message) {
  need(v.kind == Value::String, message);
  return v.text;
}

// ---- dense dataset descriptor (native/class_model_dataset_contract.hpp:23-38) --
struct Dense {
  uint32_t features = 0, classes = 0;
  uint64_t rows = 0, stride = 0, fit_rows = 0, valid_rows = 0;
};

Dense dense(const Value& b, bool fit_only) {
  need(b.kind == Value::Object, "dense format");
  need(b.find("format") && b.at("format").kind == Value::String &&
           b.at("format").text == "dense-fp32-u32-class-labels-1",
       "dense format");
  need(is_false(b.find("TEST_read")), "dense TEST role");
  const uint64_t F = unsigned_integer(b.at("features"), "dense features must be unsigned integer");
  const uint64_t K = unsigned_integer(b.at("classes"), "dense classes must be unsigned integer");
  need(F > 0 && F <= uint64_t(INT32_MAX) && K >= 2 && K <= UINT32_MAX, "dense feature/class range");
  Dense d;
  d.features = uint32_t(F);
  d.classes = uint32_t(K);
  d.rows = unsigned_integer(b.at("rows"), "dense rows must be unsigned integer");
  d.stride = unsigned_integer(b.at("row_stride"), "dense stride must be unsigned integer");
  d.fit_rows = unsigned_integer(b.at("FIT_rows"), "dense FIT must be unsigned integer");
  d.valid_rows = unsigned_integer(b.at("VALID_rows"), "dense VALID must be unsigned integer");
  need(d.rows > 0 && d.stride >= F && d.fit_rows > 0 && d.fit_rows <= d.rows &&
           d.valid_rows == d.rows - d.fit_rows,
       "dense row/split range");
  need(fit_only ? d.fit_rows == d.rows && d.valid_rows == 0 : d.valid_rows > 0,
       "dense FIT-only or evaluation boundary");
  need(d.rows <= UINT64_MAX / d.stride && d.rows * d.stride <= SIZE_MAX / sizeof(float),
       "dense storage extent overflow");
  need(b.find("preprocessing") && b.at("preprocessing").kind == Value::String &&
           !b.at("preprocessing").text.empty(),
       "dense preprocessing identity");
  for (const char* field : {"values_path", "labels_path"})
    need(b.find(field) && b.at(field).kind == Value::String && !b.at(field).text.empty(),
         "dense file path");
  for (const char* field : {"values_sha256", "labels_sha256"})
    need(b.find(field) && b.at(field).kind == Value::String && dp::sha::is_digest(b.at(field).text),
         "dense byte pins must be lowercase SHA256");
  return d;
}

// ---- source manifest (native/class_model_train.cu:14-24) ---------------------
fs::path executable() { return fs::canonical("/proc/self/exe"); }

Value source_manifest() {
  // Sources of this executable, beside the library sources; keys sorted.
  const fs::path dir = executable().parent_path().parent_path() / "csrc";
  static const char* names[] = {"Makefile", "dp_internal.hpp", "dp_model_train.hip", "json.hpp",
                                "sha256.hpp"};
  Value files = dp::json::object();
  for (const char* name : names)
    dp::json::set(files, name, dp::json::string(dp::sha::of_bytes(read_file(dir / name))));
  Value m = dp::json::object();
  dp::json::set(m, "files", files);
  dp::json::set(m, "sha256", dp::json::string(dp::sha::of_bytes(dp::json::dump(files))));
  dp::json::set(m, "role",
                dp::json::string("maintained compilation-source metadata; executable pin is separate"));
  return m;
}

// ---- the numerical library ------------------------------------------------------
struct Library {
  using H = void*;
  void* handle = nullptr;
  H matrix = nullptr, model = nullptr;
  const char* (*error)() = nullptr;
  int (*free_booster)(H) = nullptr;
  int (*free_matrix)(H) = nullptr;

  template <class T>
  T symbol(const char* name) {
    dlerror();
    void* p = dlsym(handle, name);
    const char* e = dlerror();
    need(p && !e, std::string("missing native symbol ") + name);
    return reinterpret_cast<T>(p);
  }
  void check(int status, const std::string& what) {
    if (status) dp::fail(what + ": " + (error ? error() : "native error"));
  }
  explicit Library(const std::string& path) {
    handle = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
    if (!handle) dp::fail(std::string("native dlopen failed: ") + dlerror());
    error = symbol<const char* (*)()>("XGBGetLastError");
    free_booster = symbol<int (*)(H)>("XGBoosterFree");
    free_matrix = symbol<int (*)(H)>("XGDMatrixFree");
    std::array<int, 3> v{};
    symbol<void (*)(int*, int*, int*)>("XGBoostVersion")(&v[0], &v[1], &v[2]);
    need(v == std::array<int, 3>{3, 4, 1}, "native version differs");
    const char* info = nullptr;
    check(symbol<int (*)(const char**)>("XGBuildInfo")(&info), "build info");
    need(info && is_true(dp::json::parse(info).find("USE_CUDA")), "native library has no GPU path");
  }
  ~Library() {
    if (model && free_booster) free_booster(model);
    if (matrix && free_matrix) free_matrix(matrix);
    if (handle) dlclose(handle);
  }
  Library(const Library&) = delete;
  Library& operator=(const Library&) = delete;

  // Normalised hyperparameters (the reference's parameters(),
  // native/class_native_training.cuh:16-33).
  Value parameters(const Value& hp, uint32_t K) {
    auto validate = symbol<int (*)(const char*, uint32_t, uint64_t*, const char**)>(
        "DPValidateHyperparameters");
    uint64_t n = 0;
    const char* out = nullptr;
    check(validate(dp::json::dump(hp).c_str(), K, &n, &out), "hyperparameters");
    return dp::json::parse(std::string(out, n));
  }
  static std::string array(const void* p, uint64_t rows, uint64_t cols, bool labels) {
    std::string s = "{\"data\":[" + std::to_string(reinterpret_cast<uintptr_t>(p)) +
                    ",true],\"shape\":[" + std::to_string(rows);
    if (!labels) s += "," + std::to_string(cols);
    return s + "],\"strides\":null,\"typestr\":\"<f4\",\"version\":3,\"stream\":1}";
  }
};

std::string library_identity(const Value& plan) {
  const std::string& path =
      text_of(plan.at("native_library_path"), "native library path must be a string");
  need(path.find('\0') == std::string::npos && fs::path(path).is_absolute(),
       "native library path must be absolute");
  const std::string& pin =
      text_of(plan.at("native_library_sha256"), "native library SHA must be a string");
  need(pin.size() == 64, "native library SHA must contain 64 lowercase hexadecimal digits");
  need(dp::sha::is_digest(pin), "invalid native library SHA");
  return pin;
}

// ---- staging kernels (native/class_native_training.cuh:36-46) -------------------
__global__ void prepare_values(const float* in, float* out, uint64_t rows, uint64_t stride,
                               uint32_t F, uint32_t* bad) {
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < rows * uint64_t(F);
       i += uint64_t(blockDim.x) * gridDim.x) {
    const float v = in[(i / F) * stride + i % F];
    if (isinf(v)) {
      atomicOr(bad, 2u);
      continue;
    }
    out[i] = v;
  }
}

__global__ void prepare_labels(const uint32_t* in, float* out, uint64_t rows, uint32_t K,
                               uint32_t* bad) {
  for (uint64_t r = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; r < rows;
       r += uint64_t(blockDim.x) * gridDim.x) {
    const uint32_t y = in[r];
    const float v = float(y);
    if (y >= K || double(v) != double(y)) {
      atomicOr(bad, 1u);
      continue;
    }
    out[r] = v;
  }
}

void hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) dp::fail(std::string(what) + ": " + hipGetErrorString(e));
}

template <class T>
struct Dev {
  T* p = nullptr;
  size_t n = 0;
  explicit Dev(size_t count) : n(count) {
    hip_ok(hipMalloc(reinterpret_cast<void**>(&p), (count ? count : 1) * sizeof(T)), "device allocation");
  }
  ~Dev() {
    if (p) (void)hipFree(p);
  }
  Dev(const Dev&) = delete;
  Dev& operator=(const Dev&) = delete;
};

unsigned blocks(uint64_t n) { return unsigned(std::min<uint64_t>((n + 255) / 256, 65536)); }

// ---- plan check (native/class_model_train.cu:25-36) ------------------------------
struct Checked {
  Value plan;
  Dense data;
};

Checked check_plan(const fs::path& path, const std::string& pin, const fs::path& exe) {
  check_path(path);
  const std::string bytes = read_file(path);
  need(dp::sha::of_bytes(bytes) == pin, "training plan SHA differs");
  Value p = dp::json::parse(bytes);
  need(p.kind == Value::Object, "training plan must be an object");
  need(p.find("format") && p.at("format").kind == Value::String &&
           p.at("format").text == "class-model-training-plan-1" && is_false(p.find("TEST_read")) &&
           is_false(p.find("VALID_read")) && is_false(p.find("selection_performed")) &&
           is_true(p.find("training_performed")),
       "FIT-only training protocol");
  const Value& d = p.at("dataset");
  const Dense shape = dense(d, true);
  need(shape.classes <= kMaxExactClasses, "class IDs exceed the exact native FP32 label capacity");
  check_path(d.at("values_path").text);
  check_path(d.at("labels_path").text);
  const std::string lib_pin = library_identity(p);
  const std::string lib = p.at("native_library_path").text;
  need(dp::sha::of_file(lib) == lib_pin, "pinned native library differs");
  need(dp::sha::of_file(exe.string()) ==
           text_of(p.at("executable_sha256"), "executable SHA must be a string"),
       "training executable differs");
  const Value manifest = source_manifest();
  need(p.find("source_manifest_sha256") &&
           dp::json::dump(manifest.at("sha256")) == dp::json::dump(p.at("source_manifest_sha256")),
       "training source manifest differs");
  Library api(lib);
  const Value hp = api.parameters(p.at("hyperparameters"), shape.classes);
  dp::json::set(p, "hyperparameters", hp);
  dp::json::set(p, "checked_source_manifest", manifest);
  return {p, shape};
}

// ---- fit (native/class_model_train.cu:38-64) --------------------------------------
Value train(const fs::path& plan_path, const std::string& pin, const fs::path& out,
            const fs::path& exe, bool& output_owned) {
  Checked c = check_plan(plan_path, pin, exe);
  const Value& p = c.plan;
  const Dense& shape = c.data;
  check_path(out);
  clean_output(out);
  output_owned = true;
  atomic_json(out / "plan.json", dp::json::parse(read_file(plan_path)));
  atomic_json(out / "source-manifest.json", p.at("checked_source_manifest"));
  hip_ok(hipSetDevice(0), "training device");
  const auto start = std::chrono::steady_clock::now();

  const Value& d = p.at("dataset");
  const std::string xb = read_file(d.at("values_path").text);
  const std::string yb = read_file(d.at("labels_path").text);
  need(dp::sha::of_bytes(xb) == d.at("values_sha256").text &&
           dp::sha::of_bytes(yb) == d.at("labels_sha256").text,
       "dense data pins differ");
  const uint64_t rows = shape.rows, stride = shape.stride;
  const uint32_t F = shape.features, K = shape.classes;
  need(xb.size() == rows * stride * 4 && yb.size() == rows * 4, "dense byte extents");
  Dev<float> raw_x(rows * stride), x(rows * F), labels(rows);
  Dev<uint32_t> raw_y(rows), bad(1);
  const uint64_t owned = (raw_x.n + x.n + labels.n) * sizeof(float) + (raw_y.n + 1) * sizeof(uint32_t);
  hip_ok(hipMemcpy(raw_x.p, xb.data(), xb.size(), hipMemcpyHostToDevice), "stage values");
  hip_ok(hipMemcpy(raw_y.p, yb.data(), yb.size(), hipMemcpyHostToDevice), "stage labels");
  hip_ok(hipMemset(bad.p, 0, sizeof(uint32_t)), "clear flags");
  hipLaunchKernelGGL(prepare_values, dim3(blocks(rows * F)), dim3(256), 0, 0, raw_x.p, x.p, rows,
                     stride, F, bad.p);
  hipLaunchKernelGGL(prepare_labels, dim3(blocks(rows)), dim3(256), 0, 0, raw_y.p, labels.p, rows,
                     K, bad.p);
  hip_ok(hipGetLastError(), "staging kernels");
  uint32_t flags = 0;
  hip_ok(hipMemcpy(&flags, bad.p, sizeof flags, hipMemcpyDeviceToHost), "staging flags");
  need(flags == 0, "FIT features must be finite/NaN and labels exact native class IDs");

  const std::string lib_path = p.at("native_library_path").text;
  Library api(lib_path);
  using H = Library::H;
  const std::string xa = Library::array(x.p, rows, F, false), ya = Library::array(labels.p, rows, 0, true);
  api.check(api.symbol<int (*)(const char*, const char*, H*)>("XGDMatrixCreateFromCudaArrayInterface")(
                xa.c_str(), "{\"missing\":NaN,\"nthread\":2}", &api.matrix),
            "create native FIT DMatrix");
  api.check(api.symbol<int (*)(H, const char*, const char*)>("XGDMatrixSetInfoFromInterface")(
                api.matrix, "label", ya.c_str()),
            "assign FIT labels");
  api.check(api.symbol<int (*)(const H*, uint64_t, H*)>("XGBoosterCreate")(&api.matrix, 1, &api.model),
            "create training booster");
  const Value& hp = p.at("hyperparameters");
  auto token = [&](const char* key, const char* dflt) {
    const Value* v = hp.find(key);
    return v ? dp::json::dump(*v) : std::string(dflt);
  };
  std::string zeros = "[";
  for (uint32_t k = 0; k < K; ++k) zeros += k ? ",0" : "0";
  zeros += "]";
  const std::vector<std::pair<std::string, std::string>> params = {
      {"alpha", token("alpha", "0")},
      {"base_score", zeros},
      {"boost_from_average", "0"},
      {"booster", "gbtree"},
      {"colsample_bylevel", token("colsample_bylevel", "1")},
      {"colsample_bynode", token("colsample_bynode", "1")},
      {"colsample_bytree", token("colsample_bytree", "1")},
      {"device", "cuda:0"},
      {"eta", token("eta", "0.3")},
      {"gamma", token("gamma", "0")},
      {"lambda", token("lambda", "1")},
      {"max_bin", token("max_bin", "256")},
      {"max_depth", token("max_depth", "6")},
      {"min_child_weight", token("min_child_weight", "1")},
      {"nthread", "2"},
      {"num_class", std::to_string(K)},
      {"objective", "multi:softmax"},
      {"seed", token("seed", "0")},
      {"seed_per_iteration", "0"},
      {"subsample", token("subsample", "1")},
      {"tree_method", "hist"},
      {"validate_parameters", "1"},
      {"verbosity", "0"}};
  auto set_param = api.symbol<int (*)(H, const char*, const char*)>("XGBoosterSetParam");
  for (const auto& kv : params) api.check(set_param(api.model, kv.first.c_str(), kv.second.c_str()), kv.first);
  const uint64_t rounds = unsigned_integer(hp.at("rounds"), "rounds");
  auto update = api.symbol<int (*)(H, int, H)>("XGBoosterUpdateOneIter");
  for (uint64_t i = 0; i < rounds; ++i) {
    api.check(update(api.model, int(i), api.matrix), "native FIT update");
    hip_ok(hipDeviceSynchronize(), "device synchronisation");
  }
  uint64_t n = 0;
  const char* cfg = nullptr;
  api.check(api.symbol<int (*)(H, uint64_t*, const char**)>("XGBoosterSaveJsonConfig")(api.model, &n, &cfg),
            "save native configuration");
  need(cfg && n, "native configuration missing");
  const Value config = dp::json::parse(std::string(cfg, n));
  const Value& learner = config.at("learner");
  const Value& updaters = learner.at("gradient_booster").at("updater");
  need(learner.at("generic_param").at("device").text == "cuda:0" && updaters.kind == Value::Array &&
           updaters.items.size() == 1 && updaters.items[0].at("name").text == "grow_gpu_hist",
       "native training updater differs from the required GPU updater");
  int done = -1;
  api.check(api.symbol<int (*)(H, int*)>("XGBoosterBoostedRounds")(api.model, &done), "native completed rounds");
  need(done >= 0 && uint64_t(done) == rounds, "native completed round count differs");
  api.check(api.symbol<int (*)(H, const char*)>("XGBoosterSaveModel")(api.model, (out / "model.json").c_str()),
            "save native source model");
  const std::string model_bytes = read_file(out / "model.json");
  const Value model = dp::json::parse(model_bytes);
  const Value& ml = model.at("learner");
  need(ml.at("objective").at("name").text == "multi:softmax" &&
           ml.at("learner_model_param").at("num_feature").text == std::to_string(F) &&
           ml.at("learner_model_param").at("num_class").text == std::to_string(K),
       "saved native objective/shape differs");
  atomic_json(out / "configuration.json", config);
  need(dp::sha::of_file(d.at("values_path").text) == d.at("values_sha256").text &&
           dp::sha::of_file(d.at("labels_path").text) == d.at("labels_sha256").text,
       "dataset changed during evaluation");
  need(dp::json::dump(source_manifest()) == dp::json::dump(p.at("checked_source_manifest")) &&
           dp::sha::of_bytes(read_file(plan_path)) == pin &&
           dp::sha::of_file(exe.string()) == p.at("executable_sha256").text &&
           dp::sha::of_file(lib_path) == p.at("native_library_sha256").text,
       "final training pins differ");

  namespace J = dp::json;
  Value binding = d;
  J::set(binding, "input_dtype", J::string("little-endian FP32"));
  J::set(binding, "label_dtype", J::string("little-endian uint32"));
  J::set(binding, "roles", J::string("All declared rows FIT; no VALID input"));
  J::set(binding, "FIT_only", J::boolean(true));
  Value r = J::object();
  J::set(r, "format", J::string("class-model-training-result-1"));
  J::set(r, "complete", J::boolean(true));
  J::set(r, "CUDA_executed", J::boolean(true));
  J::set(r, "device", J::string("HIP gfx950"));
  J::set(r, "CPU_model_numerical_work", J::boolean(false));
  J::set(r, "FIT_only", J::boolean(true));
  J::set(r, "FIT_rows", J::integer(int64_t(rows)));
  J::set(r, "VALID_read", J::boolean(false));
  J::set(r, "TEST_read", J::boolean(false));
  J::set(r, "selection_performed", J::boolean(false));
  J::set(r, "evaluation_performed", J::boolean(false));
  J::set(r, "features", J::integer(F));
  J::set(r, "classes", J::integer(K));
  J::set(r, "dataset", binding);
  J::set(r, "hyperparameters", hp);
  J::set(r, "native_objective", J::string("multi:softmax"));
  J::set(r, "model_path", J::string((out / "model.json").string()));
  J::set(r, "model_sha256", J::string(dp::sha::of_bytes(model_bytes)));
  J::set(r, "model_bytes", J::integer(int64_t(model_bytes.size())));
  J::set(r, "configuration_sha256", J::string(dp::sha::of_file((out / "configuration.json").string())));
  J::set(r, "plan_sha256", J::string(pin));
  J::set(r, "executable_sha256", p.at("executable_sha256"));
  J::set(r, "source_manifest_sha256", p.at("source_manifest_sha256"));
  J::set(r, "native_library_sha256", p.at("native_library_sha256"));
  J::set(r, "native_class_ID_precision_limit", J::integer(int64_t(kMaxExactClasses)));
  J::set(r, "caller_coordinate_contract", d.at("preprocessing"));
  J::set(r, "consumer_peak_owned_CUDA_bytes_excluding_native_XGBoost", J::integer(int64_t(owned)));
  J::set(r, "seconds_before_receipt",
         J::number(std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count()));
  J::set(r, "scope", J::string("one user-configured FIT-only native GPU classification fit; no "
                               "competitive-quality, conversion-completion or general-scaling claim"));
  atomic_json(out / "result.json", r);
  Value seal = J::object();
  J::set(seal, "sealed", J::boolean(true));
  J::set(seal, "result_sha256", J::string(dp::sha::of_file((out / "result.json").string())));
  J::set(seal, "model_sha256", J::string(dp::sha::of_bytes(model_bytes)));
  J::set(seal, "FIT_only", J::boolean(true));
  J::set(seal, "VALID_read", J::boolean(false));
  J::set(seal, "TEST_read", J::boolean(false));
  atomic_json(out / "result-seal.json", seal);
  return r;
}

}  // namespace

int main(int argc, char** argv) {
  fs::path output;
  bool output_owned = false;
  try {
    static_assert(sizeof(float) == 4 && sizeof(uint32_t) == 4);
    if (argc == 2 && std::string(argv[1]) == "source-manifest") {
      std::cout << dp::json::dump(source_manifest(), 2) << '\n';
      return 0;
    }
    if (argc == 4 && std::string(argv[1]) == "--check-plan") {
      const Checked c = check_plan(argv[2], argv[3], executable());
      Value o = dp::json::object();
      dp::json::set(o, "checked", dp::json::boolean(true));
      dp::json::set(o, "CUDA_executed", dp::json::boolean(false));
      dp::json::set(o, "dataset", c.plan.at("dataset"));
      dp::json::set(o, "hyperparameters", c.plan.at("hyperparameters"));
      std::cout << dp::json::dump(o, 2) << '\n';
      return 0;
    }
    need(argc == 5 && std::string(argv[1]) == "fit",
         "usage: dp_model_train source-manifest | --check-plan PLAN SHA | fit PLAN SHA NEW_OUT");
    output = fs::absolute(argv[4]);
    const Value result = train(argv[2], argv[3], output, executable(), output_owned);
    std::cout << dp::json::dump(result, 2) << '\n';
    return 0;
  } catch (const std::exception& e) {
    if (output_owned && fs::exists(output)) {
      try {
        Value f = dp::json::object();
        dp::json::set(f, "complete", dp::json::boolean(false));
        dp::json::set(f, "error", dp::json::string(e.what()));
        dp::json::set(f, "model_may_be_prepared", dp::json::boolean(fs::exists(output / "model.json")));
        dp::json::set(f, "FIT_only", dp::json::boolean(true));
        dp::json::set(f, "VALID_read", dp::json::boolean(false));
        dp::json::set(f, "TEST_read", dp::json::boolean(false));
        atomic_json(output / "failure.json", f);
      } catch (...) {
      }
    }
    std::cerr << e.what() << '\n';
    return 1;
  }
}
