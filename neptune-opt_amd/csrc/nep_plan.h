// nep_plan.h -- launch plans of the neptune fold operators, shared by the Python-side
// dispatcher module (nep_dispatch.cpp) and the Python-free bundle loader (nep_ops.cpp).
//
// A plan is what one operator call did for one input layout: the buffers it allocated (the
// outputs first, then scratch) and, per kernel launch, the packed kernarg image with the
// offsets of its pointer arguments, each tied to an input or a buffer.  The layout key is
// (dtype, device, rank, sizes, strides, address mod 16) per input; inputs sharing an address
// have no key and are never replayed.
#pragma once

#include <ATen/core/ivalue.h>
#include <ATen/ops/empty_strided.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <cstring>
#include <vector>

#include "../../include/neptune_hip.h"

namespace nep_plan {

constexpr size_t kMaxImage = 1024;

struct Launch {
  uint64_t kernel = 0;
  uint32_t grid[3] = {1, 1, 1};
  uint32_t block = 0;
  uint32_t lds = 0;
  std::vector<uint8_t> image;
  // (byte offset in the image, source): source >= 0 is input `source`, source < 0 is
  // buffer (-1 - source); outputs are the first buffers.
  std::vector<std::pair<uint32_t, int32_t>> patches;
};

struct Buffer {
  std::vector<int64_t> sizes, strides;
  c10::ScalarType dtype;
};

struct Plan {
  bool replayable = false;
  std::vector<Buffer> buffers;
  std::vector<Launch> launches;
};

using Key = std::vector<int64_t>;

struct KeyHash {
  size_t operator()(const Key& key) const noexcept {
    uint64_t h = 1469598103934665603ull;
    for (int64_t v : key) {
      h ^= static_cast<uint64_t>(v);
      h *= 1099511628211ull;
    }
    return static_cast<size_t>(h);
  }
};

// The layout key of a call's inputs; false when the call has no key (a non-tensor argument,
// another device type, a non-strided or conjugate/negative view, aliased inputs).
inline bool make_key(c10::ArrayRef<c10::IValue> args, c10::DeviceType device_type, Key& key) {
  std::vector<uintptr_t> ptrs;
  ptrs.reserve(args.size());
  for (const c10::IValue& arg : args) {
    if (!arg.isTensor()) return false;
    const at::Tensor& t = arg.toTensor();
    if (!t.defined() || t.device().type() != device_type || t.layout() != c10::kStrided ||
        t.is_neg() || t.is_conj())
      return false;
    const auto uptr = reinterpret_cast<uintptr_t>(t.data_ptr());
    key.push_back(static_cast<int64_t>(t.scalar_type()));
    key.push_back(t.get_device());
    key.push_back(t.dim());
    for (int64_t s : t.sizes()) key.push_back(s);
    for (int64_t s : t.strides()) key.push_back(s);
    key.push_back(static_cast<int64_t>(uptr % 16));
    ptrs.push_back(uptr);
  }
  for (size_t i = 0; i < ptrs.size(); ++i)
    for (size_t j = i + 1; j < ptrs.size(); ++j)
      if (ptrs[i] == ptrs[j]) return false;
  return true;
}

// Checks a plan's internal consistency against the operator's input count; a plan that fails
// is kept non-replayable.
inline bool plan_consistent(const Plan& plan, int n_inputs) {
  if (plan.buffers.empty()) return false;
  for (const Launch& l : plan.launches) {
    if (l.kernel == 0 || l.image.size() > kMaxImage || l.block == 0 || l.block > 1024) return false;
    for (const auto& [offset, source] : l.patches) {
      if (offset + sizeof(void*) > l.image.size()) return false;
      if (source >= n_inputs || -1 - source >= static_cast<int32_t>(plan.buffers.size()))
        return false;
    }
  }
  return true;
}

// Allocate the plan's buffers on the first input's device and replay its launches on the
// current stream; returns the first buffer (the output).
inline at::Tensor replay(const Plan& plan, c10::ArrayRef<c10::IValue> args) {
  const at::Tensor& first = args[0].toTensor();
  const at::TensorOptions options = at::TensorOptions().device(first.device());
  std::vector<at::Tensor> buffers;
  buffers.reserve(plan.buffers.size());
  for (const Buffer& b : plan.buffers)
    buffers.push_back(at::empty_strided(b.sizes, b.strides, options.dtype(b.dtype)));
  if (!plan.launches.empty()) {
    hipStream_t stream = c10::hip::getCurrentHIPStream(first.get_device()).stream();
    uint8_t image[kMaxImage];
    for (const Launch& l : plan.launches) {
      std::memcpy(image, l.image.data(), l.image.size());
      for (const auto& [offset, source] : l.patches) {
        void* ptr = source >= 0 ? args[source].toTensor().data_ptr()
                                : buffers[-1 - source].data_ptr();
        std::memcpy(image + offset, &ptr, sizeof(ptr));
      }
      const int rc = nep_launch_packed(l.kernel, l.grid[0], l.grid[1], l.grid[2], l.block,
                                       l.lds, stream, image, l.image.size());
      TORCH_CHECK(rc == NEP_OK, "neptune launch failed: ", nep_last_error());
    }
  }
  return buffers[0];
}

}  // namespace nep_plan
