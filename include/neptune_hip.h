/*
 * neptune_hip.h -- C ABI of libneptune_hip.so, the MI355X (gfx950) compile-and-launch
 * boundary behind neptune_codegen's operator bridge.
 *
 * The reference (Defyli/neptune-opt) has no native code: its boundary is Triton's
 * "write generated source -> import -> @triton.jit -> kernel[grid](...)" chain.  Each entry
 * point below replaces one step of that chain, cited as path:line in the reference:
 *
 *   nep_compile              replaces compile_skeleton / compile_state_reduction /
 *                            compile_segment_reduction (neptune_codegen/template.py:198-225,
 *                            template.py:231-264, torch_op.py:309-337): generated source in,
 *                            loaded kernel module out, cached by exact source identity.
 *   nep_compile_code_object  the device-independent half of nep_compile (hiprtc only, no GPU
 *                            needed); used to pre-build the on-disk code-object cache and to
 *                            check that every emitted kernel compiles for gfx950.
 *   nep_module_load          loads a prebuilt code object (a launch-plan bundle's kernels)
 *                            without hiprtc; see its declaration.
 *   nep_get_kernel           replaces getattr(module, name) after the import
 *                            (template.py:219-220, torch_op.py:332).
 *   nep_launch               replaces kernel[grid](args..., BLOCK=, num_warps=)
 *                            (template.py:377-390, template.py:307-319, torch_op.py:406-409):
 *                            asynchronous launch on the caller's stream, no synchronisation.
 *   nep_launch_packed        the same launch with the arguments already packed into one kernarg
 *                            image (what Triton's generated launcher builds per call); the host
 *                            cost per launch is one call, with no per-argument pointer array.
 *   nep_fold_split           replaces the split branch of launch_reduction
 *                            (template.py:380-390, kernels template.py:137-165): a generated
 *                            fold's partial and merge kernels over a caller-owned workspace.
 *   nep_last_error           the text the reference surfaces through Python exceptions; it
 *                            carries the HIP error name so that fatal-error classification by
 *                            message (neptune_opt/ab.py:23-44) keeps working.
 *
 * Conventions: every function returns NEP_OK (0) on success and a nonzero NEP_ERR_* code on
 * failure, with a thread-local message in nep_last_error().  Pointers are plain device or
 * host pointers; no torch types cross this boundary.  Kernels never allocate: the caller owns
 * every input, output and scratch buffer.
 */
#ifndef NEPTUNE_HIP_H
#define NEPTUNE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NEP_OK 0
#define NEP_ERR_INVALID 1   /* bad argument (null pointer, unknown kernel name, ...) */
#define NEP_ERR_COMPILE 2   /* hiprtc rejected the source; message holds the compiler log */
#define NEP_ERR_HIP 3       /* a HIP runtime call failed; message holds hipGetErrorName */
#define NEP_ERR_IO 4        /* code-object cache file could not be read or written */

/* ABI revision of this header; bumped on any signature change. */
int nep_abi_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
const char* nep_last_error(void);

/*
 * Compile `source` (HIP C++, kernels declared extern "C") with hiprtc and load it as a module
 * on the current HIP device.  `options` is a '\n'-separated hiprtc option list (for example
 * "--offload-arch=gfx950\n-O3").  The module is cached in-process by the exact
 * (device, options, source) triple.  If `cache_file` is non-null and names a readable code
 * object it is loaded instead of compiling; after a compile the code object is written there
 * (atomically, via a temporary file and rename).  `*module_out` receives an opaque handle that
 * stays valid until the process ends.
 */
int nep_compile(const char* source, const char* name, const char* options,
                const char* cache_file, uint64_t* module_out);

/*
 * hiprtc only: compile `source` to a gfx950 code object without touching any GPU.  On success
 * `*code_out` points to a malloc'ed buffer of `*size_out` bytes that the caller releases with
 * nep_free().  If `cache_file` is non-null the code object is also written there.
 */
int nep_compile_code_object(const char* source, const char* name, const char* options,
                            const char* cache_file, void** code_out, size_t* size_out);

/* Release a buffer returned by nep_compile_code_object. */
void nep_free(void* buffer);

/*
 * Load a gfx950 code object (the bytes nep_compile_code_object produced) as a module on the
 * current device.  This is how a launch-plan bundle brings its kernels into a process that
 * never compiles: it replaces the reference's load of the Triton binary an AOTI package
 * embeds (neptune_opt/ab.py:95-255 packages it; docs/design.md:283-287).  Not cached.
 */
int nep_module_load(const void* image, size_t size, uint64_t* module_out);

/* Look up an extern "C" kernel in a module returned by nep_compile or nep_module_load. */
int nep_get_kernel(uint64_t module, const char* kernel_name, uint64_t* kernel_out);

/*
 * Launch `kernel` with a grid of grid[0..2] workgroups of block[0..2] work-items and
 * `lds_bytes` of dynamic LDS on `stream` (a hipStream_t; null means the legacy default
 * stream).  `args` holds one pointer per kernel parameter, each pointing at the parameter's
 * value, in declaration order (hipModuleLaunchKernel's kernelParams convention); `nargs` is
 * their count and is checked against nothing but zero-vs-null consistency.
 */
int nep_launch(uint64_t kernel, const uint32_t grid[3], const uint32_t block[3],
               uint32_t lds_bytes, void* stream, void** args, size_t nargs);

/*
 * Launch `kernel` on a grid of (gx, gy, gz) workgroups of `block` work-items (1-D), with
 * `lds_bytes` of dynamic LDS, on `stream`.  `args` is the kernel's explicit-argument image:
 * every parameter at its natural alignment in declaration order (C struct layout), `nbytes`
 * long; the runtime appends the hidden arguments itself.
 */
int nep_launch_packed(uint64_t kernel, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t block,
                      uint32_t lds_bytes, void* stream, const void* args, size_t nbytes);

/*
 * Bytes of workspace nep_fold_split needs for `rows` rows of `nparts` partials: four arrays
 * of rows*nparts 4-byte fields (running max m, accumulator acc, seen flag, status bits).
 */
size_t nep_fold_split_workspace_bytes(int64_t rows, int64_t nparts);

/*
 * The split plan of one scalar fold on `stream`.  `partial_kernel` and `merge_kernel` are the
 * generated unit's "<name>_partial_<variant>" and "<name>_merge_<dtype>" kernels
 * (nep_get_kernel); x is [rows, ncols] with strides (row_stride, col_stride) in elements, out
 * holds `rows` results in x's dtype.  nparts must be ceil(ncols / block) (block a power of
 * two, nparts <= 4096: split_launch_shape, template.py:114-125).  partial_threads and
 * parts_per_workgroup are the partial kernel's workgroup size and the (row, part) pairs one
 * workgroup covers; the generated unit records both (its __launch_bounds__, and the size of
 * the marker symbol "<partial kernel>_parts_per_workgroup", which hipModuleGetGlobal reports),
 * and a call whose numbers differ fails with NEP_ERR_INVALID before any launch.  partial_kernel
 * must have been looked up through nep_get_kernel.  `workspace` is device memory of at
 * least nep_fold_split_workspace_bytes(rows, nparts) bytes, owned by the caller and not read
 * before the partial kernel writes it.  Two launches, no synchronisation, no allocation.
 */
int nep_fold_split(uint64_t partial_kernel, uint64_t merge_kernel, const void* x, void* out,
                   int64_t rows, int64_t ncols, int64_t row_stride, int64_t col_stride,
                   int64_t nparts, int64_t block, uint32_t partial_threads,
                   uint32_t parts_per_workgroup, void* workspace, size_t workspace_bytes,
                   void* stream);

/*
 * nep_fold_split without allocation, for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  Same arguments and results as nep_fold_split minus the workspace: the scratch is
 * a fixed device array inside this library, one per GPU, of nep_fold_split_noalloc_capacity()
 * bytes (8 MiB: rows * nparts <= 524288).  Larger requests fail with NEP_ERR_INVALID before
 * any launch.  Calls no hipMalloc/hipFree.  Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams, other threads) race and must be serialised
 * by the caller.
 */
int nep_fold_split_noalloc(uint64_t partial_kernel, uint64_t merge_kernel, const void* x,
                           void* out, int64_t rows, int64_t ncols, int64_t row_stride,
                           int64_t col_stride, int64_t nparts, int64_t block,
                           uint32_t partial_threads, uint32_t parts_per_workgroup, void* stream);

/* Bytes of the per-GPU scratch array nep_fold_split_noalloc uses. */
size_t nep_fold_split_noalloc_capacity(void);

/* Name of the current device's ISA (e.g. "gfx950:sramecc+:xnack-") into buf. */
int nep_device_arch(char* buf, size_t buf_len);

#ifdef __cplusplus
}
#endif

#endif /* NEPTUNE_HIP_H */
