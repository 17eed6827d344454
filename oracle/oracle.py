"""Python view of the CPU oracle (oracle/mq_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product package never
imports it.

Arrays are numpy: bfloat16 values travel as their raw uint16 bit patterns.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_FAST_PATH = os.path.join(_HERE, "libcpu_baseline.so")
_lib = None
_fast = None

_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i64 = ctypes.c_int64
_int = ctypes.c_int


def build() -> str:
    """Compile oracle/liboracle.so (and the CPU-baseline loop) with its Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def fast_lib():
    """oracle/libcpu_baseline.so: the vectorised float32 loop bench.py times."""
    global _fast
    if _fast is None:
        if not os.path.exists(_FAST_PATH):
            build()
        L = ctypes.CDLL(_FAST_PATH)
        L.cpu_qmm_f32_lanes.argtypes = [_u16p, _u32p, _u16p, _u16p, _i64, _i64, _i64, _int, _int,
                                        _u16p, _int]
        L.cpu_qmm_f32_lanes.restype = _int
        _fast = L
    return _fast


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_quantize.argtypes = [_u16p, _i64, _i64, _int, _int, _u32p, _u16p, _u16p, _f32p, _f32p]
        L.orc_dequantize.argtypes = [_u32p, _u16p, _u16p, _i64, _i64, _int, _int, _u16p, _f64p]
        L.orc_qmm.argtypes = [_u16p, _u32p, _u16p, _u16p, _u16p, _i64, _i64, _i64, _int, _int, _f32p]
        L.orc_qmm_f32.argtypes = [_u16p, _u32p, _u16p, _u16p, _i64, _i64, _i64, _int, _int, _u16p, _int]
        L.orc_gather_qmm.argtypes = [_u16p, _i32p, _i32p, _u32p, _u16p, _u16p,
                                     _i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _f32p]
        for f in ("orc_quantize", "orc_dequantize", "orc_qmm", "orc_qmm_f32", "orc_gather_qmm"):
            getattr(L, f).restype = _int
        L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _p(a: np.ndarray | None, ct):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ct)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments (rc={rc})")


# ----------------------------------------------------------------- bfloat16


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 bits (nearest even); NaN -> quiet NaN."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------------ the ops


def quantize(w_bf16: np.ndarray, group_size: int = 64, bits: int = 4, with_f32: bool = False):
    """mx.quantize on bfloat16 bits w[..., K] -> (wq, scales, biases)[, s32, b32]."""
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    K = w.shape[-1]
    rows = int(np.prod(w.shape[:-1])) if w.ndim > 1 else 1
    lead = w.shape[:-1]
    wq = np.empty(lead + (K * bits // 32,), np.uint32)
    s = np.empty(lead + (K // group_size,), np.uint16)
    b = np.empty_like(s)
    s32 = np.empty(lead + (K // group_size,), np.float32) if with_f32 else None
    b32 = np.empty_like(s32) if with_f32 else None
    _check(lib().orc_quantize(_p(w, _u16p), rows, K, group_size, bits, _p(wq, _u32p),
                              _p(s, _u16p), _p(b, _u16p), _p(s32, _f32p), _p(b32, _f32p)),
           "quantize")
    if with_f32:
        return wq, s, b, s32, b32
    return wq, s, b


def dequantize(wq: np.ndarray, scales: np.ndarray, biases: np.ndarray,
               group_size: int = 64, bits: int = 4, exact: bool = False) -> np.ndarray:
    """mx.dequantize -> bfloat16 bits (or float64 q*s+b when exact=True)."""
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    biases = np.ascontiguousarray(biases, dtype=np.uint16)
    K = wq.shape[-1] * 32 // bits
    rows = int(np.prod(wq.shape[:-1])) if wq.ndim > 1 else 1
    shape = wq.shape[:-1] + (K,)
    if exact:
        out = np.empty(shape, np.float64)
        rc = lib().orc_dequantize(_p(wq, _u32p), _p(scales, _u16p), _p(biases, _u16p), rows, K,
                                  group_size, bits, None, _p(out, _f64p))
    else:
        out = np.empty(shape, np.uint16)
        rc = lib().orc_dequantize(_p(wq, _u32p), _p(scales, _u16p), _p(biases, _u16p), rows, K,
                                  group_size, bits, _p(out, _u16p), None)
    _check(rc, "dequantize")
    return out


def qmm(x_bf16: np.ndarray, wq: np.ndarray, scales: np.ndarray, biases: np.ndarray,
        group_size: int = 64, bits: int = 4, bias: np.ndarray | None = None) -> np.ndarray:
    """quantized_matmul(transpose=True) (+bias) -> float32 [M, N], double accumulation."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    K = x.shape[-1]
    M = int(np.prod(x.shape[:-1])) if x.ndim > 1 else 1
    N = wq.shape[0]
    y = np.empty(x.shape[:-1] + (N,), np.float32)
    bias_c = None if bias is None else np.ascontiguousarray(bias, dtype=np.uint16)
    _check(lib().orc_qmm(_p(x, _u16p), _p(np.ascontiguousarray(wq, np.uint32), _u32p),
                         _p(np.ascontiguousarray(scales, np.uint16), _u16p),
                         _p(np.ascontiguousarray(biases, np.uint16), _u16p),
                         _p(bias_c, _u16p), M, N, K, group_size, bits, _p(y, _f32p)), "qmm")
    return y


def qmm_f32(x_bf16, wq, scales, biases, group_size=64, bits=4, threads=1) -> np.ndarray:
    """MLX-CPU-style float32 quantized_matmul -> bfloat16 bits [M, N]."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    K = x.shape[-1]
    M = int(np.prod(x.shape[:-1])) if x.ndim > 1 else 1
    N = wq.shape[0]
    y = np.empty(x.shape[:-1] + (N,), np.uint16)
    _check(lib().orc_qmm_f32(_p(x, _u16p), _p(np.ascontiguousarray(wq, np.uint32), _u32p),
                             _p(np.ascontiguousarray(scales, np.uint16), _u16p),
                             _p(np.ascontiguousarray(biases, np.uint16), _u16p),
                             M, N, K, group_size, bits, _p(y, _u16p), threads), "qmm_f32")
    return y


def qmm_f32_lanes(x_bf16, wq, scales, biases, group_size=64, bits=4, threads=1) -> np.ndarray:
    """qmm_f32's arithmetic with 16 partial sums per output (vectorised, -O3):
    the CPU baseline's timed loop -> bfloat16 bits [M, N]."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    K = x.shape[-1]
    M = int(np.prod(x.shape[:-1])) if x.ndim > 1 else 1
    N = wq.shape[0]
    y = np.empty(x.shape[:-1] + (N,), np.uint16)
    _check(fast_lib().cpu_qmm_f32_lanes(
        _p(x, _u16p), _p(np.ascontiguousarray(wq, np.uint32), _u32p),
        _p(np.ascontiguousarray(scales, np.uint16), _u16p),
        _p(np.ascontiguousarray(biases, np.uint16), _u16p),
        M, N, K, group_size, bits, _p(y, _u16p), threads), "qmm_f32_lanes")
    return y


def gather_qmm(x_bf16, wq, scales, biases, rhs_indices, lhs_indices=None,
               group_size=64, bits=4) -> np.ndarray:
    """gather_qmm(transpose=True): x [Bx, M, K], wq [E, N, Kw] -> float32 [T, M, N]."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    assert x.ndim == 3
    Bx, M, K = x.shape
    E, N = wq.shape[0], wq.shape[1]
    rhs = np.ascontiguousarray(rhs_indices, dtype=np.int32).reshape(-1)
    lhs = None if lhs_indices is None else np.ascontiguousarray(lhs_indices, np.int32).reshape(-1)
    T = rhs.shape[0]
    y = np.empty((T, M, N), np.float32)
    _check(lib().orc_gather_qmm(_p(x, _u16p), _p(lhs, _i32p), _p(rhs, _i32p),
                                _p(np.ascontiguousarray(wq, np.uint32), _u32p),
                                _p(np.ascontiguousarray(scales, np.uint16), _u16p),
                                _p(np.ascontiguousarray(biases, np.uint16), _u16p),
                                T, M, N, K, E, Bx, group_size, bits, _p(y, _f32p)), "gather_qmm")
    return y
