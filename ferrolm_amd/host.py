"""ctypes binding of the load-time host routines (include/ferro_host.h):
synthetic weights, the group-32 quantizer and the AWQ channel statistics and
scales. They run on the CPU."""
from __future__ import annotations

import ctypes as C

import numpy as np

from .gpu import LIB_PATH, check, ptr
from .weights import INT4, INT8, Matrix

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m ferrolm_amd.build`")
        l = C.CDLL(str(LIB_PATH))
        l.fh_random_bf16.restype = C.c_int
        l.fh_random_bf16.argtypes = [C.c_uint64, C.c_uint64, C.c_int64, C.c_int64, C.c_float,
                                     C.POINTER(C.c_uint16)]
        l.fh_stream_seed.restype = C.c_uint64
        l.fh_stream_seed.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        l.fh_quantize.restype = C.c_int
        l.fh_quantize.argtypes = [C.c_int32, C.c_int32, C.c_int32, C.POINTER(C.c_float), C.POINTER(C.c_float),
                                  C.POINTER(C.c_uint8), C.POINTER(C.c_float)]
        l.fh_awq_stats.restype = C.c_int
        l.fh_awq_stats.argtypes = [C.POINTER(C.c_float), C.c_int32, C.c_int32, C.POINTER(C.c_float),
                                   C.POINTER(C.c_float)]
        l.fh_awq_scales.restype = C.c_int
        l.fh_awq_scales.argtypes = [C.POINTER(C.c_float), C.c_int32, C.c_float, C.POINTER(C.c_float)]
        _lib = l
    return _lib


def random_bf16(seed: int, tensor: int, rows: int, cols: int, std: float) -> np.ndarray:
    """N(0, std) weights rounded to bf16 (uint16 bit patterns), rows x cols."""
    out = np.empty((rows, cols), np.uint16)
    check(lib().fh_random_bf16(seed, tensor, rows, cols, std, ptr(out, C.POINTER(C.c_uint16))))
    return out


def stream_seed(seed: int, tensor: int, block: int) -> int:
    return int(lib().fh_stream_seed(seed, tensor, block))


def quantize(kind: int, w: np.ndarray, importance: np.ndarray | None = None) -> Matrix:
    """QMatrix::quantize (src/quant.rs:78-143) of a rows x cols f32 matrix."""
    assert kind in (INT8, INT4)
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    q = np.empty(rows * cols // (1 if kind == INT8 else 2), np.uint8)
    s = np.empty(rows * cols // 32, np.float32)
    imp = None if importance is None else np.ascontiguousarray(importance, np.float32)
    check(lib().fh_quantize(kind, rows, cols, ptr(w, C.POINTER(C.c_float)), ptr(imp, C.POINTER(C.c_float)),
                            ptr(q, C.POINTER(C.c_uint8)), ptr(s, C.POINTER(C.c_float))))
    return Matrix(kind, rows, cols, q=q, s=s)


def awq_stats(cal: np.ndarray):
    """stats (src/awq.rs:128-142): mean |x| and mean x^2 per input channel."""
    cal = np.ascontiguousarray(cal, np.float32)
    m, k = cal.shape
    a = np.zeros(k, np.float32)
    q = np.zeros(k, np.float32)
    fp = C.POINTER(C.c_float)
    check(lib().fh_awq_stats(ptr(cal, fp), m, k, ptr(a, fp), ptr(q, fp)))
    return a, q


def awq_scales(abs_mean: np.ndarray, alpha: float) -> np.ndarray:
    """scales (src/awq.rs:144-150) for one alpha."""
    abs_mean = np.ascontiguousarray(abs_mean, np.float32)
    s = np.zeros(abs_mean.size, np.float32)
    fp = C.POINTER(C.c_float)
    check(lib().fh_awq_scales(ptr(abs_mean, fp), abs_mean.size, alpha, ptr(s, fp)))
    return s
