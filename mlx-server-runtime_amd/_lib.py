"""ctypes binding of libmi355q.so (declarations in include/mq.h, include/mq_measure.h).

The library is loaded from this package directory.  There is no fallback: if
it is missing or cannot be loaded, every op raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
# MQ_LIBRARY_PATH names another build of the same library (the host-side
# sanitizer build of tests/run_host_sanitizers.sh).
LIB_PATH = os.environ.get("MQ_LIBRARY_PATH") or os.path.join(_HERE, "libmi355q.so")

MQ_OK = 0
MQ_ERR_INVALID = -1
MQ_ERR_UNSUPPORTED = -2
MQ_ERR_HIP = -3

# Every symbol include/*.h declares (checked by the CPU test suite).
EXPORTS = (
    "mq_version",
    "mq_last_error",
    "mq_quantize",
    "mq_dequantize",
    "mq_embedding_lookup",
    "mq_repack_codes_u8",
    "mq_quantized_matmul",
    "mq_quantized_matmul_workspace",
    "mq_quantized_matmul_ws",
    "mq_gather_qmm",
    "mq_rms_norm",
    "mq_rope_kv_append",
    "mq_paged_decode_attention_workspace",
    "mq_paged_decode_attention",
    "mq_paged_prefill_attention_supported",
    "mq_paged_prefill_attention",
    "mq_decode_attention_step",
    "mq_silu_mul",
    "mq_moe_route",
    "mq_moe_sort",
    "mq_moe_combine",
    "mq_moe_route_sort",
    "mq_argmax_rows",
    "mq_moe_combine_rms_norm",
    "mq_quantized_matmul_swiglu_supported",
    "mq_quantized_matmul_swiglu",
    "mq_rms_norm_quantized_matmul_supported",
    "mq_rms_norm_quantized_matmul",
    "mq_quantized_matmul_swiglu_workspace",
    "mq_quantized_matmul_swiglu_ws",
    "mq_quantized_matmul_add_rms_norm_supported",
    "mq_quantized_matmul_add_rms_norm_workspace",
    "mq_quantized_matmul_add_rms_norm",
    "mq_gather_qmm_swiglu_supported",
    "mq_gather_qmm_swiglu",
    "mq_quantized_matmul_noalloc",
    "mq_gather_qmm_segments",
    "mq_gather_qmm_segments_supported",
    "mq_hbm_read",          # include/mq_measure.h
    "mq_qmv_trace",         # include/mq_measure.h
)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int


class LibraryNotBuilt(RuntimeError):
    pass


def _declare(L: ctypes.CDLL) -> None:
    L.mq_version.argtypes = []
    L.mq_version.restype = _int
    L.mq_last_error.argtypes = []
    L.mq_last_error.restype = ctypes.c_char_p
    L.mq_quantize.argtypes = [_p, _p, _p, _p, _i64, _i64, _int, _int, _p]
    L.mq_dequantize.argtypes = [_p, _p, _p, _p, _i64, _i64, _int, _int, _p]
    L.mq_embedding_lookup.argtypes = [_p, _i64, _p, _p, _p, _i64, _i64, _int, _int, _p, _p]
    L.mq_repack_codes_u8.argtypes = [_p, _p, _i64, _i64, _int, _p]
    L.mq_quantized_matmul.argtypes = [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _int, _int, _int, _p]
    L.mq_quantized_matmul_workspace.argtypes = [_i64, _i64, _i64, _int, _int]
    L.mq_quantized_matmul_ws.argtypes = [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _int, _int, _int,
                                         _p, ctypes.c_size_t, _p]
    L.mq_gather_qmm.argtypes = [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                _int, _int, _int, _int, _p]
    L.mq_rms_norm.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, ctypes.c_float, _p]
    L.mq_rope_kv_append.argtypes = [_p, _p, _p, _i64, _i64, _i64, _p, _p, _p, _p, ctypes.c_float,
                                    _p, _p, _p, _i64, _int, _int, _int, _p]
    L.mq_paged_decode_attention_workspace.argtypes = [_i64, _int, _int, _int, _i64, _i64]
    L.mq_paged_decode_attention.argtypes = [_p, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _int, _int,
                                            _int, ctypes.c_float, _p, ctypes.c_size_t, _p, _p]
    L.mq_decode_attention_step.argtypes = [_p, _p, _p, _i64, _i64, _i64, _p, _p, _p, _p,
                                           ctypes.c_float, _p, _p, _i64, _int, _int, _int,
                                           ctypes.c_float, _p, ctypes.c_size_t, _p, _p]
    L.mq_paged_prefill_attention_supported.argtypes = [_int, _int, _int, _i64, _i64]
    L.mq_paged_prefill_attention.argtypes = [_p, _p, _p, _p, _i64, _i64, _i64, _p, _p, _i64, _i64,
                                             _int, _int, _int, ctypes.c_float, _p, _p]
    L.mq_silu_mul.argtypes = [_p, _p, _i64, _i64, _p]
    L.mq_moe_route.argtypes = [_p, _p, _i64, _int, _int, _int, _p, _p, _p]
    L.mq_moe_sort.argtypes = [_p, _i64, _int, _int, _p, _p, _p, _p, _p, _p]
    L.mq_moe_combine.argtypes = [_p, _p, _p, _p, _i64, _int, _i64, _p]
    L.mq_moe_route_sort.argtypes = [_p, _p, _i64, _int, _int, _int, _p, _p, _p, _p, _p, _p, _p,
                                    _p]
    L.mq_argmax_rows.argtypes = [_p, _i64, _i64, _p, _p]
    L.mq_quantized_matmul_swiglu_supported.argtypes = [_i64, _i64, _i64, _int, _int]
    L.mq_quantized_matmul_swiglu.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, _i64, _int, _int, _p]
    L.mq_rms_norm_quantized_matmul_supported.argtypes = [_i64, _i64, _i64, _int, _int, _int]
    L.mq_rms_norm_quantized_matmul.argtypes = [_p, _p, _p, _p, ctypes.c_float, _p, _p, _p, _p, _p,
                                               _i64, _i64, _i64, _int, _int, _int, _p]
    L.mq_quantized_matmul_swiglu_workspace.argtypes = [_i64, _i64, _i64, _int, _int]
    L.mq_quantized_matmul_swiglu_ws.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, _i64, _int, _int,
                                                _p, ctypes.c_size_t, _p]
    L.mq_quantized_matmul_add_rms_norm_supported.argtypes = [_i64, _i64, _i64, _int, _int]
    L.mq_quantized_matmul_add_rms_norm_workspace.argtypes = [_i64, _i64, _i64, _int, _int]
    L.mq_quantized_matmul_add_rms_norm.argtypes = [_p, _p, _p, _p, _p, _p, _p, _p,
                                                   ctypes.c_float, _p, _i64, _i64, _i64, _int,
                                                   _int, _p, ctypes.c_size_t, _p]
    L.mq_moe_combine_rms_norm.argtypes = [_p, _p, _p, _p, _p, _p, _p, _i64, _int, _i64,
                                          ctypes.c_float, _p]
    L.mq_gather_qmm_swiglu_supported.argtypes = [_i64, _i64, _i64, _i64, _int, _int]
    L.mq_gather_qmm_swiglu.argtypes = [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                       _i64, _int, _int, _p]
    L.mq_quantized_matmul_noalloc.argtypes = [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _int,
                                              _int, _int, _p]
    L.mq_gather_qmm_segments.argtypes = [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64,
                                         _i64, _i64, _int, _int, _int, _p]
    L.mq_gather_qmm_segments_supported.argtypes = [_i64, _i64, _i64, _i64, _i64, _i64, _int,
                                                   _int, _int]
    L.mq_hbm_read.argtypes = [_p, ctypes.c_size_t, _p, _p]
    L.mq_qmv_trace.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, _p, ctypes.c_size_t, _p]
    for name in EXPORTS[2:]:
        getattr(L, name).restype = _int
    L.mq_quantized_matmul_workspace.restype = ctypes.c_size_t
    L.mq_paged_decode_attention_workspace.restype = ctypes.c_size_t
    L.mq_quantized_matmul_swiglu_workspace.restype = ctypes.c_size_t
    L.mq_quantized_matmul_add_rms_norm_workspace.restype = ctypes.c_size_t


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it is not built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise LibraryNotBuilt(
                        f"{LIB_PATH} is missing: build it with "
                        "`python mlx-server-runtime_amd/build_lib.py` (no CPU fallback exists)")
                L = ctypes.CDLL(LIB_PATH)
                _declare(L)
                _lib = L
    return _lib


def check(rc: int, op: str) -> None:
    """Map a C-ABI return code to the exception MLX raises for the same case."""
    if rc == MQ_OK:
        return
    msg = lib().mq_last_error().decode(errors="replace") or f"[{op}] failed (rc={rc})"
    if rc == MQ_ERR_INVALID:
        raise ValueError(msg)
    if rc == MQ_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)
