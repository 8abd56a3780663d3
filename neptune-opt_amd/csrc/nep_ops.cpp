// libneptune_ops: runs neptune fold operators from a launch-plan bundle, without Python.
//
// A fused AOTI package (neptune_opt.compile_best / aoti_compile_and_package) calls neptune
// custom ops by name through the dispatcher.  In a process with the Python package those ops
// exist already (neptune_codegen registers them; their C++ kernels replay recorded plans).  A
// process without it -- a C++ deployment of the package, or Python that never imports
// neptune -- loads this library and a bundle written by neptune_codegen.dispatch.export_bundle:
// the bundle carries, per operator, its schema, the gfx950 code objects of its kernels and one
// launch plan per input layout the exporting process ran.  Each operator is defined and given a
// CUDA kernel that replays the plan of the call's layout; a layout with no plan is an error
// naming the operator.  The reference has no counterpart (its packages embed Triton binaries
// and need the Python op registration, neptune_opt/ab.py:95-255).
//
// Bundle format (little endian), as written by export_bundle:
//   "NEPBNDL1"
//   u32 n_code; n_code x (u32 size, bytes)                          gfx950 code objects
//   u32 n_ops; per op:
//     str qualname ("ns::name"), str arguments ("(Tensor x) -> Tensor"), u32 n_inputs
//     u32 n_plans; per plan:
//       u32 n_key, i64 key[n_key]                                   nep_plan::make_key order
//       u32 n_buffers; per buffer: i32 scalar type, u32 rank, i64 sizes[rank], i64 strides[rank]
//       u32 n_launches; per launch:
//         u32 code index, str kernel name, u32 grid[3], u32 block, u32 lds,
//         u32 image size, bytes image, u32 n_patches, n_patches x (u32 offset, i32 source)
//   str is u32 length + bytes.
#include <ATen/core/dispatch/Dispatcher.h>
#include <torch/library.h>

#include <fstream>
#include <iterator>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "nep_plan.h"

namespace {

using nep_plan::Key;
using nep_plan::KeyHash;
using nep_plan::Plan;

class Reader {
 public:
  Reader(const std::vector<uint8_t>& data) : p_(data.data()), end_(data.data() + data.size()) {}
  template <class T>
  T get() {
    T v{};
    if (static_cast<size_t>(end_ - p_) < sizeof(T)) {
      ok_ = false;
      return v;
    }
    std::memcpy(&v, p_, sizeof(T));
    p_ += sizeof(T);
    return v;
  }
  std::vector<uint8_t> bytes() {
    const uint32_t n = get<uint32_t>();
    if (!ok_ || static_cast<size_t>(end_ - p_) < n) {
      ok_ = false;
      return {};
    }
    std::vector<uint8_t> out(p_, p_ + n);
    p_ += n;
    return out;
  }
  std::string str() {
    const std::vector<uint8_t> b = bytes();
    return std::string(b.begin(), b.end());
  }
  // A count that cannot exceed what is left of the file (each item takes >= `unit` bytes).
  uint32_t count(size_t unit) {
    const uint32_t n = get<uint32_t>();
    if (ok_ && static_cast<size_t>(end_ - p_) / (unit ? unit : 1) < n) ok_ = false;
    return ok_ ? n : 0;
  }
  bool ok() const { return ok_; }
  bool done() const { return p_ == end_; }

 private:
  const uint8_t* p_;
  const uint8_t* end_;
  bool ok_ = true;
};

class ReplayKernel final : public c10::OperatorKernel {
 public:
  ReplayKernel(std::string name, int n_inputs,
               std::unordered_map<Key, Plan, KeyHash> plans)
      : name_(std::move(name)), n_inputs_(n_inputs), plans_(std::move(plans)) {}

  void operator()(const c10::OperatorHandle& /*op*/, c10::DispatchKeySet /*ks*/,
                  torch::jit::Stack* stack) {
    auto args = torch::jit::last(*stack, n_inputs_);
    Key key;
    TORCH_CHECK(nep_plan::make_key(args, c10::DeviceType::CUDA, key), name_,
                ": the inputs have no launch-plan key (a non-CUDA, non-strided or aliased "
                "input)");
    auto it = plans_.find(key);
    TORCH_CHECK(it != plans_.end() && it->second.replayable, name_,
                ": the bundle holds no launch plan for this input layout (dtype, sizes, "
                "strides, alignment); export the bundle from a run with these inputs");
    at::Tensor out = nep_plan::replay(it->second, args);
    torch::jit::drop(*stack, n_inputs_);
    torch::jit::push(*stack, std::move(out));
  }

 private:
  const std::string name_;
  const int n_inputs_;
  const std::unordered_map<Key, Plan, KeyHash> plans_;
};

std::mutex g_mu;

// Parse and register; returns the number of operators defined here (operators that already
// exist in the process, e.g. registered by the Python package, are left as they are).
int64_t load_bundle(const std::string& path) {
  std::ifstream in(path, std::ios::binary);
  TORCH_CHECK(in.good(), "neptune bundle: cannot open ", path);
  const std::vector<uint8_t> data((std::istreambuf_iterator<char>(in)),
                                  std::istreambuf_iterator<char>());
  Reader r(data);
  char magic[8];
  for (char& ch : magic) ch = static_cast<char>(r.get<uint8_t>());
  TORCH_CHECK(r.ok() && std::string(magic, 8) == "NEPBNDL1", "neptune bundle: ", path,
              " is not a bundle (bad magic)");
  std::lock_guard<std::mutex> guard(g_mu);
  const uint32_t n_code = r.count(4);
  std::vector<uint64_t> modules;
  for (uint32_t i = 0; i < n_code && r.ok(); ++i) {
    const std::vector<uint8_t> code = r.bytes();
    uint64_t module = 0;
    TORCH_CHECK(r.ok() && nep_module_load(code.data(), code.size(), &module) == NEP_OK,
                "neptune bundle: code object ", i, " does not load: ", nep_last_error());
    modules.push_back(module);
  }
  int64_t defined = 0;
  const uint32_t n_ops = r.count(12);
  for (uint32_t o = 0; o < n_ops && r.ok(); ++o) {
    const std::string qualname = r.str(), arguments = r.str();
    const int n_inputs = static_cast<int>(r.get<uint32_t>());
    std::unordered_map<Key, Plan, KeyHash> plans;
    const uint32_t n_plans = r.count(12);
    for (uint32_t k = 0; k < n_plans && r.ok(); ++k) {
      Key key(r.count(8));
      for (int64_t& v : key) v = r.get<int64_t>();
      Plan plan;
      const uint32_t n_buffers = r.count(8);
      for (uint32_t b = 0; b < n_buffers && r.ok(); ++b) {
        nep_plan::Buffer buffer;
        buffer.dtype = static_cast<c10::ScalarType>(r.get<int32_t>());
        const uint32_t rank = r.count(16);
        buffer.sizes.resize(rank);
        buffer.strides.resize(rank);
        for (int64_t& v : buffer.sizes) v = r.get<int64_t>();
        for (int64_t& v : buffer.strides) v = r.get<int64_t>();
        plan.buffers.push_back(std::move(buffer));
      }
      const uint32_t n_launches = r.count(32);
      for (uint32_t l = 0; l < n_launches && r.ok(); ++l) {
        nep_plan::Launch launch;
        const uint32_t code = r.get<uint32_t>();
        const std::string kernel_name = r.str();
        for (uint32_t& g : launch.grid) g = r.get<uint32_t>();
        launch.block = r.get<uint32_t>();
        launch.lds = r.get<uint32_t>();
        launch.image = r.bytes();
        const uint32_t n_patches = r.count(8);
        for (uint32_t q = 0; q < n_patches && r.ok(); ++q) {
          const uint32_t offset = r.get<uint32_t>();
          launch.patches.emplace_back(offset, r.get<int32_t>());
        }
        TORCH_CHECK(r.ok() && code < modules.size(), "neptune bundle: ", qualname,
                    " names code object ", code, " of ", modules.size());
        TORCH_CHECK(nep_get_kernel(modules[code], kernel_name.c_str(), &launch.kernel) == NEP_OK,
                    "neptune bundle: ", qualname, ": ", nep_last_error());
        plan.launches.push_back(std::move(launch));
      }
      plan.replayable = nep_plan::plan_consistent(plan, n_inputs);
      plans.emplace(std::move(key), std::move(plan));
    }
    TORCH_CHECK(r.ok(), "neptune bundle: ", path, " is truncated or corrupt (in ", qualname, ")");
    const auto sep = qualname.find("::");
    TORCH_CHECK(sep != std::string::npos && n_inputs >= 1, "neptune bundle: bad operator entry ",
                qualname);
    if (c10::Dispatcher::singleton().findSchema({qualname, ""}).has_value()) continue;
    const std::string ns = qualname.substr(0, sep), name = qualname.substr(sep + 2);
    // Library objects are leaked on purpose: the registrations live as long as the process.
    auto* def = new torch::Library(torch::Library::FRAGMENT, ns, std::nullopt, __FILE__, __LINE__);
    def->def((name + arguments).c_str());
    auto* impl = new torch::Library(torch::Library::IMPL, ns, c10::DispatchKey::CUDA, __FILE__,
                                    __LINE__);
    impl->impl(name.c_str(), torch::CppFunction::makeFromBoxedFunctor(
                                 std::make_unique<ReplayKernel>(qualname, n_inputs,
                                                                std::move(plans))));
    ++defined;
  }
  TORCH_CHECK(r.ok() && r.done(), "neptune bundle: ", path, " is truncated or has trailing data");
  return defined;
}

}  // namespace

TORCH_LIBRARY(neptune_bundle, m) {
  m.def("load(str path) -> int", [](std::string path) { return load_bundle(path); });
}

// C entry point for C++ deployments: the number of operators defined (>= 0), or -1 with the
// message in err (truncated to err_len bytes).  Call it on the device the package will run on.
extern "C" int nep_ops_load_bundle(const char* path, char* err, size_t err_len) {
  try {
    return static_cast<int>(load_bundle(path ? path : ""));
  } catch (const std::exception& e) {
    if (err != nullptr && err_len > 0) {
      std::strncpy(err, e.what(), err_len - 1);
      err[err_len - 1] = '\0';
    }
    return -1;
  }
}
