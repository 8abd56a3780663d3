// _neptune_dispatch: C++ dispatcher kernels for the neptune row-fold operators.
//
// The operators are defined from Python (torch.library.custom_op with a fake impl, as the
// reference does for its Triton ops, neptune_codegen/torch_op.py:16-114), and their Python
// bodies choose a launch configuration, allocate outputs and launch generated HIP kernels.
// Everything those bodies compute is a function of the inputs' dtype, device, sizes, strides
// and 16-byte alignment (no host read of tensor values), so one Python call per such key is
// enough: it runs under a recorder and hands back a *launch plan* -- output/scratch buffer
// shapes plus, per kernel launch, the packed kernarg image with the offsets of its pointer
// arguments.  This file installs, per operator:
//
//   CUDA key          look the key up; on a hit allocate the buffers and replay the launches
//                     on the current stream (no Python, no GIL); on a miss call the Python
//                     body (which validates, launches and records) and keep its plan.
//   AutogradCUDA key  when no input requires grad (or grad mode is off) redispatch below
//                     autograd directly; otherwise hand the call to the operator's original
//                     Python autograd kernel, so gradient behaviour is unchanged.
//
// Calls whose Python body makes a copy of an input, or whose inputs alias one another, leave
// no plan and keep going through Python.
#include <ATen/core/dispatch/Dispatcher.h>
#include <ATen/core/grad_mode.h>
#include <torch/csrc/utils/pybind.h>
#include <torch/library.h>

#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "nep_plan.h"

namespace py = pybind11;

namespace {

using nep_plan::Key;
using nep_plan::KeyHash;
using nep_plan::Launch;
using nep_plan::Plan;

// Python callables are held as leaked references: the dispatcher may destroy kernels after
// the interpreter has finalised, when a Py_DECREF would be unsafe.
PyObject* hold(const py::object& fn) {
  PyObject* raw = fn.ptr();
  Py_INCREF(raw);
  return raw;
}

struct Stats {
  int64_t replays = 0, python_calls = 0, plans = 0;
};

// Plans kept per operator; later layouts keep calling the Python body (correct, slower).
constexpr size_t kMaxPlans = 1024;

class PlanKernel final : public c10::OperatorKernel {
 public:
  PlanKernel(int n_inputs, c10::DeviceType device_type, PyObject* body,
             std::shared_ptr<Stats> stats)
      : n_inputs_(n_inputs), device_type_(device_type), body_(body), stats_(std::move(stats)) {}

  void operator()(const c10::OperatorHandle& /*op*/, c10::DispatchKeySet /*ks*/,
                  torch::jit::Stack* stack) {
    auto args = torch::jit::last(*stack, n_inputs_);
    Key key;
    const bool keyed = make_key(args, key);
    std::shared_ptr<const Plan> plan;
    if (keyed) {
      std::lock_guard<std::mutex> guard(mu_);
      auto it = cache_.find(key);
      if (it != cache_.end()) plan = it->second;
    }
    if (plan && plan->replayable) {
      at::Tensor out = replay(*plan, args);
      torch::jit::drop(*stack, n_inputs_);
      torch::jit::push(*stack, std::move(out));
      return;
    }
    at::Tensor out;
    {
      py::gil_scoped_acquire gil;
      bool full;
      {
        std::lock_guard<std::mutex> guard(mu_);
        full = cache_.size() >= kMaxPlans;
      }
      const bool record = keyed && !plan && !full;
      py::tuple call(n_inputs_ + 1);
      call[0] = py::bool_(record);
      for (int i = 0; i < n_inputs_; ++i) call[i + 1] = py::cast(args[i].toTensor());
      py::object result = py::reinterpret_borrow<py::object>(body_)(*call);
      py::tuple pair = result.cast<py::tuple>();
      out = pair[0].cast<at::Tensor>();
      std::shared_ptr<Plan> parsed;
      if (record) parsed = parse_plan(pair[1]);
      std::lock_guard<std::mutex> guard(mu_);
      stats_->python_calls += 1;
      if (parsed) {
        if (parsed->replayable) stats_->plans += 1;
        cache_.emplace(std::move(key), std::move(parsed));
      }
    }
    torch::jit::drop(*stack, n_inputs_);
    torch::jit::push(*stack, std::move(out));
  }

  void clear() {
    std::lock_guard<std::mutex> guard(mu_);
    cache_.clear();
  }

 private:
  bool make_key(c10::ArrayRef<c10::IValue> args, Key& key) const {
    return nep_plan::make_key(args, device_type_, key);
  }

  std::shared_ptr<Plan> parse_plan(const py::handle& spec) const {
    auto plan = std::make_shared<Plan>();
    if (spec.is_none()) return plan;  // known key, Python only
    py::tuple t = spec.cast<py::tuple>();
    for (py::handle b : t[0].cast<py::tuple>()) {
      py::tuple bt = b.cast<py::tuple>();   // (scalar type code, sizes, strides)
      plan->buffers.push_back({bt[1].cast<std::vector<int64_t>>(),
                               bt[2].cast<std::vector<int64_t>>(),
                               static_cast<c10::ScalarType>(bt[0].cast<int>())});
      if (plan->buffers.back().sizes.size() != plan->buffers.back().strides.size())
        return std::make_shared<Plan>();
    }
    for (py::handle l : t[1].cast<py::tuple>()) {
      py::tuple lt = l.cast<py::tuple>();
      Launch launch;
      launch.kernel = lt[0].cast<uint64_t>();
      py::tuple grid = lt[1].cast<py::tuple>();
      for (int d = 0; d < 3; ++d) launch.grid[d] = grid[d].cast<uint32_t>();
      launch.block = lt[2].cast<uint32_t>();
      launch.lds = lt[3].cast<uint32_t>();
      std::string image = lt[4].cast<std::string>();
      launch.image.assign(image.begin(), image.end());
      for (py::handle p : lt[5].cast<py::tuple>()) {
        py::tuple pt = p.cast<py::tuple>();
        launch.patches.emplace_back(pt[0].cast<uint32_t>(), pt[1].cast<int32_t>());
      }
      plan->launches.push_back(std::move(launch));
    }
    // launches need a HIP stream: only device plans may carry them
    plan->replayable = nep_plan::plan_consistent(*plan, n_inputs_) &&
                       (plan->launches.empty() || device_type_ == c10::DeviceType::CUDA);
    return plan;
  }

  at::Tensor replay(const Plan& plan, c10::ArrayRef<c10::IValue> args) {
    at::Tensor out = nep_plan::replay(plan, args);
    std::lock_guard<std::mutex> guard(mu_);
    stats_->replays += 1;
    return out;
  }

  const int n_inputs_;
  const c10::DeviceType device_type_;
  PyObject* const body_;
  std::shared_ptr<Stats> stats_;
  std::mutex mu_;
  std::unordered_map<Key, std::shared_ptr<const Plan>, KeyHash> cache_;
};

class AutogradKernel final : public c10::OperatorKernel {
 public:
  AutogradKernel(int n_inputs, PyObject* grad_body) : n_inputs_(n_inputs), grad_body_(grad_body) {}

  void operator()(const c10::OperatorHandle& op, c10::DispatchKeySet ks,
                  torch::jit::Stack* stack) {
    auto args = torch::jit::last(*stack, n_inputs_);
    bool needs_grad = false;
    if (at::GradMode::is_enabled())
      for (const c10::IValue& arg : args)
        if (arg.isTensor() && arg.toTensor().defined() && arg.toTensor().requires_grad())
          needs_grad = true;
    if (!needs_grad) {
      op.redispatchBoxed(ks & c10::after_autograd_keyset, stack);
      return;
    }
    at::Tensor out;
    {
      py::gil_scoped_acquire gil;
      py::tuple call(n_inputs_);
      for (int i = 0; i < n_inputs_; ++i) call[i] = py::cast(args[i].toTensor());
      out = py::reinterpret_borrow<py::object>(grad_body_)(*call).cast<at::Tensor>();
    }
    torch::jit::drop(*stack, n_inputs_);
    torch::jit::push(*stack, std::move(out));
  }

 private:
  const int n_inputs_;
  PyObject* const grad_body_;
};

struct Installed {
  std::shared_ptr<Stats> stats;
  PlanKernel* kernel;  // owned by the dispatcher
};

std::mutex g_mu;
std::unordered_map<std::string, Installed>& registry() {
  static auto* r = new std::unordered_map<std::string, Installed>();
  return *r;
}

// Library objects are leaked on purpose: their registrations must outlive every caller.
// `backend` is "CUDA" for the operators; "CPU" exists so that the plan cache, the Python
// round trip and the autograd hand-off can be tested without a GPU (plans without launches).
void install(const std::string& qualname, int n_inputs, const py::object& body,
             const py::object& grad_body, const std::string& backend) {
  TORCH_CHECK(n_inputs >= 1, "install: an operator needs at least one tensor input");
  TORCH_CHECK(backend == "CUDA" || backend == "CPU", "install: backend must be CUDA or CPU");
  const bool cuda = backend == "CUDA";
  const auto sep = qualname.find("::");
  TORCH_CHECK(sep != std::string::npos, "install: qualified name expected, got ", qualname);
  std::lock_guard<std::mutex> guard(g_mu);
  TORCH_CHECK(registry().count(qualname) == 0, "install: ", qualname, " is already installed");
  const std::string ns = qualname.substr(0, sep), name = qualname.substr(sep + 2);
  auto stats = std::make_shared<Stats>();
  auto kernel = std::make_unique<PlanKernel>(
      n_inputs, cuda ? c10::DeviceType::CUDA : c10::DeviceType::CPU, hold(body), stats);
  PlanKernel* raw = kernel.get();
  auto* device = new torch::Library(torch::Library::IMPL, ns,
                                    cuda ? c10::DispatchKey::CUDA : c10::DispatchKey::CPU,
                                    __FILE__, __LINE__);
  device->impl(name.c_str(), torch::CppFunction::makeFromBoxedFunctor(std::move(kernel)));
  auto* autograd = new torch::Library(
      torch::Library::IMPL, ns, cuda ? c10::DispatchKey::AutogradCUDA : c10::DispatchKey::AutogradCPU,
      __FILE__, __LINE__);
  autograd->impl(name.c_str(), torch::CppFunction::makeFromBoxedFunctor(
                                   std::make_unique<AutogradKernel>(n_inputs, hold(grad_body))));
  registry().emplace(qualname, Installed{stats, raw});
}

py::dict stats(const std::string& qualname) {
  std::lock_guard<std::mutex> guard(g_mu);
  auto it = registry().find(qualname);
  TORCH_CHECK(it != registry().end(), "stats: ", qualname, " is not installed");
  py::dict d;
  d["replays"] = it->second.stats->replays;
  d["python_calls"] = it->second.stats->python_calls;
  d["plans"] = it->second.stats->plans;
  return d;
}

void clear() {
  std::lock_guard<std::mutex> guard(g_mu);
  for (auto& [name, entry] : registry()) entry.kernel->clear();
}

// The layout key the CUDA kernels compute for these inputs (None when the call has none).
py::object key_of(const std::vector<at::Tensor>& tensors) {
  std::vector<c10::IValue> args(tensors.begin(), tensors.end());
  Key key;
  if (!nep_plan::make_key(args, c10::DeviceType::CUDA, key)) return py::none();
  return py::cast(key);
}

int64_t dtype_code(const at::Tensor& t) { return static_cast<int64_t>(t.scalar_type()); }

bool installed(const std::string& qualname) {
  std::lock_guard<std::mutex> guard(g_mu);
  return registry().count(qualname) != 0;
}

}  // namespace

PYBIND11_MODULE(_neptune_dispatch, m) {
  m.doc() = "C++ CUDA/AutogradCUDA kernels with launch-plan replay for neptune fold operators";
  m.def("install", &install, py::arg("qualname"), py::arg("n_inputs"), py::arg("body"),
        py::arg("grad_body"), py::arg("backend") = "CUDA");
  m.def("stats", &stats, py::arg("qualname"));
  m.def("clear", &clear);
  m.def("installed", &installed, py::arg("qualname"));
  m.def("key_of", &key_of, py::arg("tensors"));
  m.def("dtype_code", &dtype_code, py::arg("tensor"));
}
