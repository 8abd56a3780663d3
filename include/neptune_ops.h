/*
 * neptune_ops.h -- C ABI of libneptune_ops.so, the Python-free runner of neptune fold
 * operators from a launch-plan bundle.
 *
 * No counterpart in the reference: its fused AOTI packages embed Triton binaries and need the
 * neptune Python package to register the custom ops before loading (neptune_opt/ab.py:95-255;
 * docs/design.md:283-287).  Here a package and the bundle written next to it by
 * neptune_codegen.dispatch.export_bundle run in a process without Python: load this library,
 * call nep_ops_load_bundle on the device the package runs on, then load the package with
 * torch::inductor::AOTIModelPackageLoader.  From Python the same loader is the operator
 * torch.ops.neptune_bundle.load(path) after torch.ops.load_library(libneptune_ops.so).
 */
#ifndef NEPTUNE_OPS_H
#define NEPTUNE_OPS_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Parse the bundle at `path`, load its gfx950 code objects on the current device, and define
 * each operator it holds that the process does not have yet, with a CUDA kernel that replays
 * the plan of the call's input layout (a layout with no plan raises naming the operator).
 * Returns the number of operators defined (>= 0), or -1 with the reason copied into err
 * (at most err_len bytes, NUL-terminated) for an unreadable, damaged or foreign file or a code
 * object that does not load.
 */
int nep_ops_load_bundle(const char* path, char* err, size_t err_len);

#ifdef __cplusplus
}
#endif

#endif /* NEPTUNE_OPS_H */
