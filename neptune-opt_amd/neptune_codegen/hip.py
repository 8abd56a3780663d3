"""ctypes binding to libneptune_hip.so (include/neptune_hip.h).

The library is loaded after torch so that it binds to torch's HIP runtime (both carry the
SONAME libamdhip64.so.7): device pointers and streams from torch are then valid in it.  There
is no fallback: without the built library every device entry point raises.
"""
from __future__ import annotations

import ctypes
import hashlib
import os
import pathlib
import struct
import threading

PACKAGE_DIR = pathlib.Path(__file__).resolve().parent
LIB_PATH = PACKAGE_DIR / "_lib" / "libneptune_hip.so"
CACHE_DIR = PACKAGE_DIR / "_codeobj"

NEP_OK = 0
EXPORTED = ("nep_abi_version", "nep_last_error", "nep_compile", "nep_compile_code_object",
            "nep_free", "nep_module_load", "nep_get_kernel", "nep_launch", "nep_launch_packed",
            "nep_device_arch", "nep_fold_split_workspace_bytes", "nep_fold_split",
            "nep_fold_split_noalloc", "nep_fold_split_noalloc_capacity")

_lock = threading.Lock()
_lib = None


class HipError(RuntimeError):
    """A failure reported by libneptune_hip; the message carries the HIP error name."""


def library_path() -> pathlib.Path:
    return LIB_PATH


def load_library(require_torch: bool = True) -> ctypes.CDLL:
    """Load (once) and type the C ABI.  Raises RuntimeError if the library is not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if require_torch:
            import torch  # noqa: F401  -- bind to torch's HIP runtime, see module docstring
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"neptune HIP runtime library is not built ({LIB_PATH}); run "
                "`python -c 'import __graft_entry__ as g; g.build()'` from the repository root")
        lib = ctypes.CDLL(str(LIB_PATH))
        u64p = ctypes.POINTER(ctypes.c_uint64)
        lib.nep_abi_version.restype = ctypes.c_int
        lib.nep_last_error.restype = ctypes.c_char_p
        lib.nep_compile.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
                                    ctypes.c_char_p, u64p]
        lib.nep_compile.restype = ctypes.c_int
        lib.nep_compile_code_object.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
                                                ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p),
                                                ctypes.POINTER(ctypes.c_size_t)]
        lib.nep_compile_code_object.restype = ctypes.c_int
        lib.nep_free.argtypes = [ctypes.c_void_p]
        lib.nep_free.restype = None
        lib.nep_get_kernel.argtypes = [ctypes.c_uint64, ctypes.c_char_p, u64p]
        lib.nep_get_kernel.restype = ctypes.c_int
        lib.nep_launch.argtypes = [ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint32),
                                   ctypes.POINTER(ctypes.c_uint32), ctypes.c_uint32,
                                   ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p),
                                   ctypes.c_size_t]
        lib.nep_launch.restype = ctypes.c_int
        u32 = ctypes.c_uint32
        lib.nep_launch_packed.argtypes = [ctypes.c_uint64, u32, u32, u32, u32, u32,
                                          ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
        lib.nep_launch_packed.restype = ctypes.c_int
        lib.nep_device_arch.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
        lib.nep_device_arch.restype = ctypes.c_int
        i64 = ctypes.c_int64
        lib.nep_fold_split_workspace_bytes.argtypes = [i64, i64]
        lib.nep_fold_split_workspace_bytes.restype = ctypes.c_size_t
        lib.nep_fold_split.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p,
                                       ctypes.c_void_p, i64, i64, i64, i64, i64, i64, u32, u32,
                                       ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.nep_fold_split.restype = ctypes.c_int
        lib.nep_fold_split_noalloc.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p,
                                               ctypes.c_void_p, i64, i64, i64, i64, i64, i64, u32,
                                               u32, ctypes.c_void_p]
        lib.nep_fold_split_noalloc.restype = ctypes.c_int
        lib.nep_fold_split_noalloc_capacity.argtypes = []
        lib.nep_fold_split_noalloc_capacity.restype = ctypes.c_size_t
        if lib.nep_abi_version() != 2:
            raise RuntimeError("libneptune_hip ABI version mismatch; rebuild the library")
        _lib = lib
        return lib


def _check(rc: int, what: str) -> None:
    if rc != NEP_OK:
        msg = _lib.nep_last_error().decode(errors="replace") if _lib is not None else ""
        raise HipError(f"{what}: {msg}")


def runtime_identity() -> str:
    """What a code object depends on besides its source: the hiprtc that compiled it."""
    import torch

    return f"hiprtc-torch-{torch.version.hip}"


def cache_key(source: str, options: tuple[str, ...]) -> str:
    h = hashlib.sha256()
    for part in (runtime_identity(), "\n".join(options), source):
        h.update(part.encode())
        h.update(b"\0")
    return h.hexdigest()


def _cache_file(source: str, options: tuple[str, ...]) -> pathlib.Path:
    return CACHE_DIR / f"{cache_key(source, options)[:40]}.co"


def compile_code_object(source: str, name: str, options: tuple[str, ...],
                        write_cache: bool = True) -> int:
    """hiprtc compile without a GPU; returns the code-object size.  Raises HipError."""
    lib = load_library()
    path = None
    if write_cache:
        CACHE_DIR.mkdir(parents=True, exist_ok=True)
        path = str(_cache_file(source, options)).encode()
    buf = ctypes.c_void_p()
    size = ctypes.c_size_t()
    rc = lib.nep_compile_code_object(source.encode(), name.encode(), "\n".join(options).encode(),
                                     path, ctypes.byref(buf), ctypes.byref(size))
    _check(rc, f"compile {name}")
    lib.nep_free(buf)
    return size.value


def load_module(source: str, name: str, options: tuple[str, ...]) -> int:
    """Compile (or load from the on-disk cache) and load on the current device."""
    lib = load_library()
    CACHE_DIR.mkdir(parents=True, exist_ok=True)
    path = str(_cache_file(source, options)).encode()
    handle = ctypes.c_uint64()
    rc = lib.nep_compile(source.encode(), name.encode(), "\n".join(options).encode(), path,
                         ctypes.byref(handle))
    _check(rc, f"compile/load {name}")
    return handle.value


def get_kernel(module: int, kernel_name: str) -> int:
    lib = load_library()
    handle = ctypes.c_uint64()
    _check(lib.nep_get_kernel(module, kernel_name.encode(), ctypes.byref(handle)),
           f"kernel {kernel_name}")
    return handle.value


# argument kinds of kernel signatures
PTR, I64, I32, F32 = ctypes.c_void_p, ctypes.c_longlong, ctypes.c_int, ctypes.c_float


_ARG_CODES = {ctypes.c_void_p: "P", ctypes.c_longlong: "q", ctypes.c_int: "i",
              ctypes.c_float: "f"}


class Kernel:
    """A loaded extern "C" kernel with a fixed argument signature.

    Arguments are packed into the kernel's explicit-argument image with `struct` in native
    mode ('@': every field at its natural alignment, C struct layout -- the layout the AMDGPU
    kernarg segment uses) and launched in one library call.  Out-of-range values raise
    instead of wrapping."""

    __slots__ = ("handle", "name", "argtypes", "block", "lds", "_packer", "pointer_offsets",
                 "program")

    def __init__(self, handle: int, name: str, argtypes: tuple, block: int, lds: int = 0):
        self.handle, self.name, self.argtypes, self.block, self.lds = handle, name, argtypes, block, lds
        self.program = None     # the Program whose module holds it (set by Program.kernel)
        try:
            codes = "".join(_ARG_CODES[t] for t in argtypes)
        except KeyError as error:
            raise TypeError(f"{name}: unsupported kernel argument type {error}") from None
        self._packer = struct.Struct("@" + codes)
        # byte offset of every pointer argument in the image, by argument index
        self.pointer_offsets = {
            i: struct.calcsize("@" + codes[:i + 1]) - struct.calcsize("@P")
            for i, c in enumerate(codes) if c == "P"}

    def launch(self, grid, args, stream: int) -> None:
        if len(args) != len(self.argtypes):
            raise TypeError(f"{self.name}: expected {len(self.argtypes)} arguments, got {len(args)}")
        try:
            image = self._packer.pack(*args)
        except struct.error as error:
            raise ValueError(f"{self.name}: kernel argument out of range ({error})") from None
        gx = int(grid[0])
        gy = int(grid[1]) if len(grid) > 1 else 1
        gz = int(grid[2]) if len(grid) > 2 else 1
        rc = _lib.nep_launch_packed(self.handle, gx, gy, gz, self.block, self.lds, stream,
                                    image, len(image))
        if rc != NEP_OK:
            _check(rc, f"launch {self.name}")
        recorder = getattr(_recording, "active", None)
        if recorder is not None:
            recorder.launches.append((self, (gx, gy, gz), image, tuple(args)))


class Recorder:
    """What one operator body launched (kernel, grid, image, arguments) and which scratch
    tensors it allocated for those launches; see `recording`."""

    def __init__(self):
        self.launches: list = []
        self.buffers: list = []


_recording = threading.local()


class recording:
    """Context manager: record every Kernel.launch and `scratch` allocation on this thread."""

    def __enter__(self) -> Recorder:
        self._previous = getattr(_recording, "active", None)
        _recording.active = Recorder()
        return _recording.active

    def __exit__(self, *exc) -> None:
        _recording.active = self._previous


def recording_active() -> bool:
    """Whether this thread records launches (hip.recording())."""
    return getattr(_recording, "active", None) is not None


def scratch(tensor):
    """Mark a tensor allocated by a launch path as per-call scratch (recorded when active)."""
    recorder = getattr(_recording, "active", None)
    if recorder is not None:
        recorder.buffers.append(tensor)
    return tensor


class Program:
    """One generated unit: compiled and loaded lazily per device, kernels fetched by name."""

    def __init__(self, source: str, name: str, options: tuple[str, ...]):
        self.source, self.name, self.options = source, name, tuple(options)
        self._modules: dict[int, int] = {}
        self._kernels: dict[tuple, Kernel] = {}

    def kernel(self, kernel_name: str, argtypes: tuple, block: int, device: int) -> Kernel:
        key = (device, kernel_name)
        k = self._kernels.get(key)
        if k is not None:
            return k
        import torch

        with torch.cuda.device(device):
            module = self._modules.get(device)
            if module is None:
                module = load_module(self.source, self.name, self.options)
                self._modules[device] = module
            k = Kernel(get_kernel(module, kernel_name), kernel_name, argtypes, block)
            k.program = self
        self._kernels[key] = k
        return k

    def code_object(self) -> bytes:
        """The unit's gfx950 code object (from the on-disk cache, compiled if absent)."""
        path = _cache_file(self.source, self.options)
        if not (path.exists() and path.stat().st_size > 0):
            compile_code_object(self.source, self.name, self.options)
        return path.read_bytes()

    def precompile(self) -> int:
        """Fill the on-disk code-object cache (no GPU needed)."""
        path = _cache_file(self.source, self.options)
        if path.exists() and path.stat().st_size > 0:
            return path.stat().st_size
        return compile_code_object(self.source, self.name, self.options)


def current_stream(device) -> int:
    """Raw hipStream_t of torch's current stream on `device` (a torch.device or index)."""
    import torch

    index = device.index if isinstance(device, torch.device) else device
    if index is None:
        index = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)
