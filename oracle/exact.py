"""ctypes bindings to the oracle's C restatement (oracle/csrc/neptune_oracle.c).

Test infrastructure; see oracle/__init__.py.  Arrays are numpy; storage dtypes are passed as
raw bit patterns (uint16 for bf16/fp16, float32 for fp32).
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "_build" / "libneptune_oracle.so"
F32, BF16, F16 = 0, 1, 2
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            subprocess.run(["make", "-C", str(HERE)], check=True, capture_output=True)
        L = ctypes.CDLL(str(LIB))
        L.nor_f32_to_bf16.argtypes = [ctypes.c_float]
        L.nor_f32_to_bf16.restype = ctypes.c_uint16
        L.nor_f32_to_f16.argtypes = [ctypes.c_float]
        L.nor_f32_to_f16.restype = ctypes.c_uint16
        L.nor_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.nor_bf16_to_f32.restype = ctypes.c_float
        L.nor_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.nor_f16_to_f32.restype = ctypes.c_float
        L.nor_rsqrt_rn.argtypes = [ctypes.c_float]
        L.nor_rsqrt_rn.restype = ctypes.c_float
        L.nor_rsqrt_is_correctly_rounded.argtypes = [ctypes.c_float, ctypes.c_float]
        L.nor_rsqrt_is_correctly_rounded.restype = ctypes.c_int
        L.nor_check_rsqrt_range.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                            ctypes.POINTER(ctypes.c_uint32)]
        L.nor_check_rsqrt_range.restype = ctypes.c_int64
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        L.nor_rms_norm.argtypes = [vp, vp, vp, i64, i64, ctypes.c_int, ctypes.c_float]
        L.nor_l2_normalize.argtypes = [vp, vp, i64, i64, ctypes.c_int, ctypes.c_float]
        L.nor_segment_pool.argtypes = [vp, vp, vp, i64, i64, i64, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_uint32]
        _lib = L
    return _lib


def _code(dtype: str) -> int:
    return {"float32": F32, "bfloat16": BF16, "float16": F16}[dtype]


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def f32_to_bf16_bits(values) -> np.ndarray:
    return np.array([lib().nor_f32_to_bf16(float(v)) for v in np.asarray(values, np.float32).ravel()],
                    np.uint16)


def f32_to_f16_bits(values) -> np.ndarray:
    return np.array([lib().nor_f32_to_f16(float(v)) for v in np.asarray(values, np.float32).ravel()],
                    np.uint16)


def rsqrt_rn(x: float) -> float:
    return lib().nor_rsqrt_rn(float(x))


def check_rsqrt_range(lo_bits: int, hi_bits: int, stride: int = 1) -> tuple[int, int]:
    first = ctypes.c_uint32(0)
    bad = lib().nor_check_rsqrt_range(lo_bits, hi_bits, stride, ctypes.byref(first))
    return int(bad), int(first.value)


def rms_norm(x_bits: np.ndarray, gamma_bits: np.ndarray, dtype: str, eps: float) -> np.ndarray:
    x_bits, gamma_bits = np.ascontiguousarray(x_bits), np.ascontiguousarray(gamma_bits)
    out = np.empty_like(x_bits)
    rows, ncols = x_bits.shape
    lib().nor_rms_norm(_ptr(x_bits), _ptr(gamma_bits), _ptr(out), rows, ncols, _code(dtype), eps)
    return out


def l2_normalize(x_bits: np.ndarray, dtype: str, eps: float) -> np.ndarray:
    x_bits = np.ascontiguousarray(x_bits)
    out = np.empty_like(x_bits)
    rows, ncols = x_bits.shape
    lib().nor_l2_normalize(_ptr(x_bits), _ptr(out), rows, ncols, _code(dtype), eps)
    return out


def segment_pool(data_bits: np.ndarray, spans, dtype: str, *, mean: bool,
                 initial: float | None) -> np.ndarray:
    import struct

    data_bits = np.ascontiguousarray(data_bits.reshape(data_bits.shape[0], -1))
    spans = np.ascontiguousarray(np.asarray(spans, np.int64))
    nseg, channels = spans.shape[0] - 1, data_bits.shape[1]
    out = np.empty((nseg, channels), dtype=data_bits.dtype)
    value = 0.0 if initial is None else float(initial)
    bits = struct.unpack("I", struct.pack("f", value))[0]
    lib().nor_segment_pool(_ptr(data_bits), _ptr(spans), _ptr(out), data_bits.shape[0], channels,
                           nseg, _code(dtype), int(mean), int(initial is not None), bits)
    return out
