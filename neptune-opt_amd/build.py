"""Build step of the neptune HIP backend (no GPU needed).

1. hipcc builds the C-ABI runtime libneptune_hip.so (host code: hiprtc + module launch) in
   place, next to the Python package, so that it travels with the source tree; g++ builds
   the operators' C++ dispatcher kernels (_neptune_dispatch.so) and the Python-free
   launch-plan bundle loader (libneptune_ops.so) beside it.
2. Every generated kernel unit the benchmark configurations and tests use is compiled with
   hiprtc for gfx950 into the on-disk code-object cache (neptune_codegen/_codeobj).  That both
   proves each emitted unit compiles and spares the GPU host the compile.
"""
from __future__ import annotations

import os
import pathlib
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parent
REPO = ROOT.parent
LIB = ROOT / "neptune_codegen" / "_lib" / "libneptune_hip.so"
SRC = ROOT / "csrc" / "nep_runtime.cpp"
DISPATCH = ROOT / "neptune_codegen" / "_lib" / "_neptune_dispatch.so"
DISPATCH_SRC = ROOT / "csrc" / "nep_dispatch.cpp"


def build_library(verbose: bool = True) -> pathlib.Path:
    LIB.parent.mkdir(parents=True, exist_ok=True)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, "--offload-arch=gfx950", "-O2", "-fPIC", "-shared", "-std=c++17",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           f"-I{REPO / 'include'}", str(SRC), "-o", str(tmp),
           "-L/opt/rocm/lib", "-lhiprtc", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"]
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


def build_dispatch(verbose: bool = True) -> pathlib.Path:
    """g++: the C++ dispatcher kernels (host code only) against torch's headers and
    libraries and libneptune_hip.so, as an importable extension module next to it."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    torch_lib = cpp_extension.library_paths()[0]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = DISPATCH.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-fPIC", "-shared", "-std=c++17",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DTORCH_EXTENSION_NAME=_neptune_dispatch", "-DTORCH_API_INCLUDE_EXTENSION_H",
           *(f"-I{p}" for p in cpp_extension.include_paths()),
           f"-I{sysconfig.get_paths()['include']}", "-I/opt/rocm/include",
           f"-I{REPO / 'include'}", str(DISPATCH_SRC), "-o", str(tmp),
           f"-L{torch_lib}", f"-L{LIB.parent}", "-lneptune_hip", "-lc10", "-lc10_hip",
           "-ltorch", "-ltorch_cpu", "-ltorch_python",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, DISPATCH)
    return DISPATCH


OPS = ROOT / "neptune_codegen" / "_lib" / "libneptune_ops.so"
OPS_SRC = ROOT / "csrc" / "nep_ops.cpp"


def build_ops(verbose: bool = True) -> pathlib.Path:
    """g++: the Python-free bundle loader (libtorch + libneptune_hip only)."""
    import torch
    from torch.utils import cpp_extension

    torch_lib = cpp_extension.library_paths()[0]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = OPS.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-fPIC", "-shared", "-std=c++17",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *(f"-I{p}" for p in cpp_extension.include_paths()), "-I/opt/rocm/include",
           f"-I{REPO / 'include'}", str(OPS_SRC), "-o", str(tmp),
           f"-L{torch_lib}", f"-L{LIB.parent}", "-lneptune_hip", "-lc10", "-lc10_hip",
           "-ltorch", "-ltorch_cpu", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, OPS)
    return OPS


def precompile(verbose: bool = True) -> int:
    """hiprtc-compile the kernel units of the benchmark and test shapes into the cache."""
    sys.path.insert(0, str(ROOT))
    import neptune_codegen as CG

    count = 0
    for program in CG.prebuilt_programs():
        size = program.precompile()
        count += 1
        if verbose:
            print(f"[build] {program.name}: {size} bytes", flush=True)
    return count


def main() -> None:
    build_library()
    build_dispatch()
    build_ops()
    precompile()


if __name__ == "__main__":
    main()
