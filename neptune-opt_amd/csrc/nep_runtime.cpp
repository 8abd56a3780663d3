// libneptune_hip: hiprtc compile + code-object cache + module launch for gfx950.
//
// This is the native half of the operator bridge.  The Python emitter hands over complete HIP
// source text; this library turns it into a loaded module (replacing the reference's
// write-file/import/@triton.jit step, neptune_codegen/template.py:198-225) and launches its
// kernels on the caller's stream (replacing kernel[grid](...), template.py:377-390).
#include "../../include/neptune_hip.h"

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include <sys/stat.h>
#include <unistd.h>

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& message) {
  g_last_error = message;
  return code;
}

int hip_fail(hipError_t err, const char* what) {
  std::string msg = std::string(what) + " failed: " + hipGetErrorName(err) + " (" +
                    hipGetErrorString(err) + ")";
  return fail(NEP_ERR_HIP, msg);
}

std::vector<std::string> split_options(const char* options) {
  std::vector<std::string> out;
  if (options == nullptr) return out;
  std::string cur;
  for (const char* p = options;; ++p) {
    if (*p == '\n' || *p == '\0') {
      if (!cur.empty()) out.push_back(cur);
      cur.clear();
      if (*p == '\0') break;
    } else {
      cur.push_back(*p);
    }
  }
  return out;
}

bool read_file(const char* path, std::vector<char>* out) {
  FILE* f = std::fopen(path, "rb");
  if (f == nullptr) return false;
  std::fseek(f, 0, SEEK_END);
  long size = std::ftell(f);
  std::fseek(f, 0, SEEK_SET);
  if (size <= 0) {
    std::fclose(f);
    return false;
  }
  out->resize(static_cast<size_t>(size));
  size_t got = std::fread(out->data(), 1, out->size(), f);
  std::fclose(f);
  return got == out->size();
}

// Write via a temporary file and rename, so a concurrent reader never sees a partial object.
bool write_file_atomic(const char* path, const void* data, size_t size) {
  std::string tmp = std::string(path) + ".tmp" + std::to_string(static_cast<long>(getpid()));
  FILE* f = std::fopen(tmp.c_str(), "wb");
  if (f == nullptr) return false;
  size_t put = std::fwrite(data, 1, size, f);
  bool ok = (put == size) && (std::fclose(f) == 0);
  if (!ok) {
    std::remove(tmp.c_str());
    return false;
  }
  return std::rename(tmp.c_str(), path) == 0;
}

// hiprtc compile of one translation unit to a code object.
int compile_to_code(const char* source, const char* name, const char* options,
                    std::vector<char>* code) {
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, source, name ? name : "neptune_kernel.hip", 0,
                                       nullptr, nullptr);
  if (r != HIPRTC_SUCCESS)
    return fail(NEP_ERR_COMPILE, std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r));
  std::vector<std::string> opts = split_options(options);
  std::vector<const char*> argv;
  argv.reserve(opts.size());
  for (const auto& o : opts) argv.push_back(o.c_str());
  r = hiprtcCompileProgram(prog, static_cast<int>(argv.size()), argv.data());
  size_t log_size = 0;
  hiprtcGetProgramLogSize(prog, &log_size);
  std::string log;
  if (log_size > 1) {
    log.resize(log_size);
    hiprtcGetProgramLog(prog, &log[0]);
  }
  if (r != HIPRTC_SUCCESS) {
    hiprtcDestroyProgram(&prog);
    return fail(NEP_ERR_COMPILE, std::string("hiprtc compile of ") + (name ? name : "?") +
                                     " failed: " + hiprtcGetErrorString(r) + "\n" + log);
  }
  size_t code_size = 0;
  r = hiprtcGetCodeSize(prog, &code_size);
  if (r != HIPRTC_SUCCESS || code_size == 0) {
    hiprtcDestroyProgram(&prog);
    return fail(NEP_ERR_COMPILE, "hiprtc produced no code object");
  }
  code->resize(code_size);
  r = hiprtcGetCode(prog, code->data());
  hiprtcDestroyProgram(&prog);
  if (r != HIPRTC_SUCCESS)
    return fail(NEP_ERR_COMPILE, std::string("hiprtcGetCode: ") + hiprtcGetErrorString(r));
  return NEP_OK;
}

// In-process module cache: exact (device, options, source) identity -> loaded module.  Kept
// for the life of the process, like the reference's generated-module dictionaries.
std::mutex g_mutex;
// Split partial kernels looked up through nep_get_kernel -> the (row, part) pairs one of their
// workgroups covers (the size of the unit's "<kernel>_parts_per_workgroup" marker symbol).
std::map<uint64_t, uint32_t> g_split_parts;
std::mutex g_split_mutex;
std::map<std::tuple<int, std::string, std::string>, hipModule_t> g_modules;

}  // namespace

extern "C" {

int nep_abi_version(void) { return 2; }

const char* nep_last_error(void) { return g_last_error.c_str(); }

int nep_compile_code_object(const char* source, const char* name, const char* options,
                            const char* cache_file, void** code_out, size_t* size_out) {
  if (source == nullptr || code_out == nullptr || size_out == nullptr)
    return fail(NEP_ERR_INVALID, "nep_compile_code_object: null argument");
  std::vector<char> code;
  int rc = compile_to_code(source, name, options, &code);
  if (rc != NEP_OK) return rc;
  if (cache_file != nullptr && !write_file_atomic(cache_file, code.data(), code.size()))
    return fail(NEP_ERR_IO, std::string("cannot write code-object cache ") + cache_file);
  void* buf = std::malloc(code.size());
  if (buf == nullptr) return fail(NEP_ERR_INVALID, "out of host memory");
  std::memcpy(buf, code.data(), code.size());
  *code_out = buf;
  *size_out = code.size();
  g_last_error.clear();
  return NEP_OK;
}

void nep_free(void* buffer) { std::free(buffer); }

int nep_compile(const char* source, const char* name, const char* options,
                const char* cache_file, uint64_t* module_out) {
  if (source == nullptr || module_out == nullptr)
    return fail(NEP_ERR_INVALID, "nep_compile: null argument");
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
  auto key = std::make_tuple(device, std::string(options ? options : ""), std::string(source));
  std::lock_guard<std::mutex> lock(g_mutex);
  auto it = g_modules.find(key);
  if (it != g_modules.end()) {
    *module_out = reinterpret_cast<uint64_t>(it->second);
    return NEP_OK;
  }
  std::vector<char> code;
  bool from_cache = cache_file != nullptr && read_file(cache_file, &code);
  if (!from_cache) {
    int rc = compile_to_code(source, name, options, &code);
    if (rc != NEP_OK) return rc;
    // A cache that cannot be written is not an error: the module is still usable.
    if (cache_file != nullptr) write_file_atomic(cache_file, code.data(), code.size());
  }
  hipModule_t module = nullptr;
  err = hipModuleLoadData(&module, code.data());
  if (err != hipSuccess && from_cache) {
    // A stale or foreign cache entry: rebuild from source once before giving up.
    (void)hipGetLastError();
    int rc = compile_to_code(source, name, options, &code);
    if (rc != NEP_OK) return rc;
    if (cache_file != nullptr) write_file_atomic(cache_file, code.data(), code.size());
    err = hipModuleLoadData(&module, code.data());
  }
  if (err != hipSuccess) return hip_fail(err, "hipModuleLoadData");
  g_modules.emplace(std::move(key), module);
  *module_out = reinterpret_cast<uint64_t>(module);
  g_last_error.clear();
  return NEP_OK;
}

int nep_module_load(const void* image, size_t size, uint64_t* module_out) {
  if (image == nullptr || size == 0 || module_out == nullptr)
    return fail(NEP_ERR_INVALID, "nep_module_load: null or empty code object");
  hipModule_t module = nullptr;
  hipError_t err = hipModuleLoadData(&module, image);
  if (err != hipSuccess) return hip_fail(err, "hipModuleLoadData");
  *module_out = reinterpret_cast<uint64_t>(module);
  return NEP_OK;
}

int nep_get_kernel(uint64_t module, const char* kernel_name, uint64_t* kernel_out) {
  if (module == 0 || kernel_name == nullptr || kernel_out == nullptr)
    return fail(NEP_ERR_INVALID, "nep_get_kernel: null argument");
  hipFunction_t fn = nullptr;
  hipError_t err = hipModuleGetFunction(&fn, reinterpret_cast<hipModule_t>(module), kernel_name);
  if (err != hipSuccess)
    return hip_fail(err, (std::string("hipModuleGetFunction(") + kernel_name + ")").c_str());
  *kernel_out = reinterpret_cast<uint64_t>(fn);
  // A split partial kernel's unit also holds its launch shape as a marker symbol's size.
  const std::string marker = std::string(kernel_name) + "_parts_per_workgroup";
  hipDeviceptr_t sym = nullptr;
  size_t bytes = 0;
  if (hipModuleGetGlobal(&sym, &bytes, reinterpret_cast<hipModule_t>(module), marker.c_str()) ==
          hipSuccess &&
      bytes > 0) {
    std::lock_guard<std::mutex> lock(g_split_mutex);
    g_split_parts[*kernel_out] = static_cast<uint32_t>(bytes);
  } else {
    (void)hipGetLastError();   // most kernels have no marker: leave no error behind
  }
  return NEP_OK;
}

int nep_launch(uint64_t kernel, const uint32_t grid[3], const uint32_t block[3],
               uint32_t lds_bytes, void* stream, void** args, size_t nargs) {
  if (kernel == 0 || grid == nullptr || block == nullptr)
    return fail(NEP_ERR_INVALID, "nep_launch: null kernel, grid or block");
  if (nargs != 0 && args == nullptr)
    return fail(NEP_ERR_INVALID, "nep_launch: nargs > 0 but args is null");
  if (grid[0] == 0 || grid[1] == 0 || grid[2] == 0)
    return fail(NEP_ERR_INVALID, "nep_launch: empty grid");
  if (block[0] * block[1] * block[2] == 0 || block[0] * block[1] * block[2] > 1024)
    return fail(NEP_ERR_INVALID, "nep_launch: workgroup size must be in [1, 1024]");
  hipError_t err = hipModuleLaunchKernel(reinterpret_cast<hipFunction_t>(kernel), grid[0],
                                         grid[1], grid[2], block[0], block[1], block[2],
                                         lds_bytes, reinterpret_cast<hipStream_t>(stream), args,
                                         nullptr);
  if (err != hipSuccess) return hip_fail(err, "hipModuleLaunchKernel");
  return NEP_OK;
}

int nep_launch_packed(uint64_t kernel, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t block,
                      uint32_t lds_bytes, void* stream, const void* args, size_t nbytes) {
  if (kernel == 0) return fail(NEP_ERR_INVALID, "nep_launch_packed: null kernel");
  if (nbytes != 0 && args == nullptr)
    return fail(NEP_ERR_INVALID, "nep_launch_packed: nbytes > 0 but args is null");
  if (gx == 0 || gy == 0 || gz == 0) return fail(NEP_ERR_INVALID, "nep_launch_packed: empty grid");
  if (block == 0 || block > 1024)
    return fail(NEP_ERR_INVALID, "nep_launch_packed: workgroup size must be in [1, 1024]");
  size_t size = nbytes;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(args),
                    HIP_LAUNCH_PARAM_BUFFER_SIZE, &size, HIP_LAUNCH_PARAM_END};
  hipError_t err = hipModuleLaunchKernel(reinterpret_cast<hipFunction_t>(kernel), gx, gy, gz,
                                         block, 1, 1, lds_bytes,
                                         reinterpret_cast<hipStream_t>(stream), nullptr,
                                         nbytes != 0 ? config : nullptr);
  if (err != hipSuccess) return hip_fail(err, "hipModuleLaunchKernel");
  return NEP_OK;
}

int nep_device_arch(char* buf, size_t buf_len) {
  if (buf == nullptr || buf_len == 0) return fail(NEP_ERR_INVALID, "nep_device_arch: no buffer");
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
  hipDeviceProp_t prop;
  err = hipGetDeviceProperties(&prop, device);
  if (err != hipSuccess) return hip_fail(err, "hipGetDeviceProperties");
  std::snprintf(buf, buf_len, "%s", prop.gcnArchName);
  return NEP_OK;
}

}  // extern "C"

// ---------------------------------------------------------------- split plan, typed
// The reference's split branch of launch_reduction (neptune_codegen/template.py:380-390):
// the partial kernel writes one exact chunk state (m, acc, seen, status) per (row, part) into
// scratch, the merge kernel folds each row's states with merge_state and finalises.
namespace {

// argument images of the generated split kernels (emitters.py's _fold_kernel signatures)
struct SplitPartialArgs {
  const void* x;
  float* pm;
  float* pa;
  int* pv;
  int* ps;
  long long rows, ncols, stride_row, stride_col, nparts, block;
};
struct SplitMergeArgs {
  const float* pm;
  const float* pa;
  const int* pv;
  const int* ps;
  void* out;
  long long rows, ncols, nparts;
};

constexpr int64_t kMaxSplitParts = 4096;     // template.py MAX_SPLIT_PARTS
constexpr uint32_t kMergeRowsPerWorkgroup = 4;   // one wave64 per row, 256-lane workgroups

int launch_image(uint64_t kernel, uint32_t grid, uint32_t block, void* stream, void* image,
                 size_t size, const char* what) {
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, image, HIP_LAUNCH_PARAM_BUFFER_SIZE, &size,
                    HIP_LAUNCH_PARAM_END};
  hipError_t err = hipModuleLaunchKernel(reinterpret_cast<hipFunction_t>(kernel), grid, 1, 1,
                                         block, 1, 1, 0, reinterpret_cast<hipStream_t>(stream),
                                         nullptr, config);
  return err == hipSuccess ? NEP_OK : hip_fail(err, what);
}

// Shape checks shared by both entry points; 0 partials (rows == 0) is a valid no-op.
int check_split(const char* who, uint64_t partial_kernel, uint64_t merge_kernel, const void* x,
                void* out, int64_t rows, int64_t ncols, int64_t nparts, int64_t block,
                uint32_t partial_threads, uint32_t parts_per_workgroup) {
  auto bad = [&](const std::string& why) {
    return fail(NEP_ERR_INVALID, std::string(who) + ": " + why);
  };
  if (partial_kernel == 0 || merge_kernel == 0) return bad("null kernel handle");
  if (rows < 0 || ncols <= 0) return bad("rows must be >= 0 and ncols > 0");
  if (rows > 0 && (x == nullptr || out == nullptr)) return bad("null input or output");
  if (block <= 0 || (block & (block - 1)) != 0) return bad("block must be a positive power of two");
  if (nparts != (ncols + block - 1) / block)
    return bad("nparts must be ceil(ncols / block) (split_launch_shape)");
  if (nparts > kMaxSplitParts) return bad("nparts exceeds the split capacity of 4096 partials");
  if (partial_threads == 0 || partial_threads > 1024 || partial_threads % 64 != 0)
    return bad("partial_threads must be a multiple of 64 in [64, 1024]");
  if (parts_per_workgroup == 0 || parts_per_workgroup > partial_threads)
    return bad("parts_per_workgroup must be in [1, partial_threads]");
  if (rows > (int64_t(1) << 40) / nparts) return bad("rows * nparts is too large");
  return NEP_OK;
}

// The partial kernel's lane mapping is compiled for its launch bound and its (row, part)
// pairs per workgroup, and the merge kernel runs 256-lane workgroups: the caller's numbers are
// checked against what the kernels themselves hold (after the argument checks, and only when
// there is work to launch).  A mismatch would leave partials unwritten.
int check_split_kernels(const char* who, uint64_t partial_kernel, uint64_t merge_kernel,
                        uint32_t partial_threads, uint32_t parts_per_workgroup) {
  int bound = 0;
  hipError_t err = hipFuncGetAttribute(&bound, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK,
                                       reinterpret_cast<hipFunction_t>(partial_kernel));
  if (err != hipSuccess) return hip_fail(err, "hipFuncGetAttribute(split partial)");
  if (static_cast<int64_t>(partial_threads) != bound)
    return fail(NEP_ERR_INVALID, std::string(who) + ": partial_threads " +
                                     std::to_string(partial_threads) +
                                     " differs from the partial kernel's workgroup size " +
                                     std::to_string(bound));
  uint32_t parts = 0;
  {
    std::lock_guard<std::mutex> lock(g_split_mutex);
    auto it = g_split_parts.find(partial_kernel);
    if (it != g_split_parts.end()) parts = it->second;
  }
  if (parts == 0)
    return fail(NEP_ERR_INVALID, std::string(who) +
                                     ": partial_kernel is not a split partial kernel looked up "
                                     "through nep_get_kernel");
  if (parts_per_workgroup != parts)
    return fail(NEP_ERR_INVALID, std::string(who) + ": parts_per_workgroup " +
                                     std::to_string(parts_per_workgroup) +
                                     " differs from the partial kernel's " + std::to_string(parts));
  err = hipFuncGetAttribute(&bound, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK,
                            reinterpret_cast<hipFunction_t>(merge_kernel));
  if (err != hipSuccess) return hip_fail(err, "hipFuncGetAttribute(split merge)");
  if (bound < static_cast<int>(64 * kMergeRowsPerWorkgroup))
    return fail(NEP_ERR_INVALID,
                std::string(who) + ": the merge kernel's workgroup bound is below 256 lanes");
  return NEP_OK;
}

int run_split(const char* who, uint64_t partial_kernel, uint64_t merge_kernel, const void* x,
              void* out, int64_t rows, int64_t ncols, int64_t row_stride, int64_t col_stride,
              int64_t nparts, int64_t block, uint32_t partial_threads,
              uint32_t parts_per_workgroup, void* scratch_base, void* stream) {
  if (rows == 0) return NEP_OK;
  int krc = check_split_kernels(who, partial_kernel, merge_kernel, partial_threads,
                                parts_per_workgroup);
  if (krc != NEP_OK) return krc;
  const int64_t count = rows * nparts;
  char* base = static_cast<char*>(scratch_base);
  float* pm = reinterpret_cast<float*>(base);
  float* pa = reinterpret_cast<float*>(base + 4 * count);
  int* pv = reinterpret_cast<int*>(base + 8 * count);
  int* ps = reinterpret_cast<int*>(base + 12 * count);
  const int64_t partial_grid = (count + parts_per_workgroup - 1) / parts_per_workgroup;
  const int64_t merge_grid = (rows + kMergeRowsPerWorkgroup - 1) / kMergeRowsPerWorkgroup;
  if (partial_grid > 0xffffffffLL || merge_grid > 0xffffffffLL)
    return fail(NEP_ERR_INVALID, "split: grid exceeds 2^32 - 1 workgroups");
  SplitPartialArgs pargs{x, pm, pa, pv, ps, rows, ncols, row_stride, col_stride, nparts, block};
  int rc = launch_image(partial_kernel, static_cast<uint32_t>(partial_grid), partial_threads,
                        stream, &pargs, sizeof(pargs), "hipModuleLaunchKernel(split partial)");
  if (rc != NEP_OK) return rc;
  SplitMergeArgs margs{pm, pa, pv, ps, out, rows, ncols, nparts};
  return launch_image(merge_kernel, static_cast<uint32_t>(merge_grid), 64 * kMergeRowsPerWorkgroup,
                      stream, &margs, sizeof(margs), "hipModuleLaunchKernel(split merge)");
}

}  // namespace

extern "C" {

size_t nep_fold_split_workspace_bytes(int64_t rows, int64_t nparts) {
  if (rows <= 0 || nparts <= 0) return 0;
  return static_cast<size_t>(16) * static_cast<size_t>(rows) * static_cast<size_t>(nparts);
}

int nep_fold_split(uint64_t partial_kernel, uint64_t merge_kernel, const void* x, void* out,
                   int64_t rows, int64_t ncols, int64_t row_stride, int64_t col_stride,
                   int64_t nparts, int64_t block, uint32_t partial_threads,
                   uint32_t parts_per_workgroup, void* workspace, size_t workspace_bytes,
                   void* stream) {
  int rc = check_split("nep_fold_split", partial_kernel, merge_kernel, x, out, rows, ncols, nparts,
                       block, partial_threads, parts_per_workgroup);
  if (rc != NEP_OK) return rc;
  const size_t need = nep_fold_split_workspace_bytes(rows, nparts);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(NEP_ERR_INVALID, "nep_fold_split: workspace holds " + std::to_string(workspace_bytes) +
                                     " bytes, the split needs " + std::to_string(need));
  return run_split("nep_fold_split", partial_kernel, merge_kernel, x, out, rows, ncols,
                   row_stride, col_stride, nparts, block, partial_threads, parts_per_workgroup,
                   workspace, stream);
}

}  // extern "C"

// ---------------------------------------------------------------- split plan without allocation
// nep_fold_split_noalloc's scratch: a file-scope device array, one copy per GPU the library
// runs on, held until the process ends.  In host code `scratch` names a host-side stand-in
// symbol, not device memory: every host use goes through the per-device address that
// hipGetSymbolAddress returns (kept in g_scratch_address).  Every call on a GPU shares that
// GPU's copy and overwrites it; calls that overlap on one GPU race.  The split writes every
// partial before the merge reads it, so nothing has to start at zero.
namespace {

constexpr size_t kSplitScratchBytes = size_t(8) << 20;   // 524288 partials of 16 bytes
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kSplitScratchBytes];
std::mutex g_scratch_mutex;
void* g_scratch_address[kMaxDevices] = {};

// The current device's copy of `scratch`, looked up once per device with it current.
int scratch_address(void** out) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
  if (device < 0 || device >= kMaxDevices)
    return fail(NEP_ERR_INVALID, "nep_fold_split_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_address[device] == nullptr) {
    void* address = nullptr;
    err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return hip_fail(err, "hipGetSymbolAddress(scratch)");
    if (address == nullptr)
      return fail(NEP_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address");
    g_scratch_address[device] = address;
  }
  *out = g_scratch_address[device];
  return NEP_OK;
}

}  // namespace

extern "C" {

size_t nep_fold_split_noalloc_capacity(void) { return kSplitScratchBytes; }

int nep_fold_split_noalloc(uint64_t partial_kernel, uint64_t merge_kernel, const void* x,
                           void* out, int64_t rows, int64_t ncols, int64_t row_stride,
                           int64_t col_stride, int64_t nparts, int64_t block,
                           uint32_t partial_threads, uint32_t parts_per_workgroup, void* stream) {
  int rc = check_split("nep_fold_split_noalloc", partial_kernel, merge_kernel, x, out, rows, ncols,
                       nparts, block, partial_threads, parts_per_workgroup);
  if (rc != NEP_OK) return rc;
  const size_t need = nep_fold_split_workspace_bytes(rows, nparts);
  if (need > kSplitScratchBytes)
    return fail(NEP_ERR_INVALID,
                "nep_fold_split_noalloc: " + std::to_string(rows) + " rows x " +
                    std::to_string(nparts) + " partials need " + std::to_string(need) +
                    " bytes of scratch, more than the " + std::to_string(kSplitScratchBytes) +
                    " bytes this library holds per GPU; call nep_fold_split with a workspace");
  if (rows == 0) return NEP_OK;
  void* base = nullptr;
  rc = scratch_address(&base);
  if (rc != NEP_OK) return rc;
  return run_split("nep_fold_split_noalloc", partial_kernel, merge_kernel, x, out, rows, ncols,
                   row_stride, col_stride, nparts, block, partial_threads, parts_per_workgroup,
                   base, stream);
}

}  // extern "C"
