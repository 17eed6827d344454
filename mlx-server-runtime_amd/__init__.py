"""MI355X-native affine-quantized matmul path (libmi355q) for the MLX worker graphs.

Import by its directory name (it contains dashes):

    import importlib
    mq = importlib.import_module("mlx-server-runtime_amd")
    y = mq.quantized_matmul(x, wq, scales, biases, transpose=True, group_size=64, bits=4)

Ops (mx.* names): quantize, dequantize, quantized_matmul, gather_qmm,
embedding_lookup; repack_codes_u8 rewrites 2/3/5/6-bit codes one byte each.  Decoder-step ops (decode_ops): rms_norm, rope_kv_append,
paged_decode_attention, silu_mul over a PagedKV cache; qwen2: the Qwen2-shaped
decoder with greedy decode.  Modules (mlx.nn names): nn.QuantizedLinear,
nn.QuantizedEmbedding, nn.QuantizedSwitchLinear, nn.SwitchGLU, nn.quantize.
Everything runs in the gfx950 HIP library libmi355q.so built by build_lib.py;
there is no CPU fallback.
"""

from . import _lib, core, decode_ops, nn
from .core import (dequantize, embedding_lookup, gather_qmm, quantize, quantized_matmul,
                   repack_codes_u8)


def library_path() -> str:
    return _lib.LIB_PATH


def version() -> tuple[int, int]:
    v = _lib.lib().mq_version()
    return v >> 16, v & 0xFFFF


__all__ = ["core", "decode_ops", "nn", "quantize", "dequantize", "quantized_matmul", "gather_qmm",
           "embedding_lookup", "repack_codes_u8", "library_path", "version"]
