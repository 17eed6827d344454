"""mx.* quantization ops on torch tensors, executed by libmi355q on the GPU.

Names, argument order and meaning follow the mlx calls the reference's model
graphs make (python/mlx_worker/native_mlx/models/qwen2.py, lfm2.py):

    quantize(w, group_size=64, bits=4, mode="affine") -> (wq, scales, biases)
    dequantize(wq, scales, biases, group_size=64, bits=4, mode="affine")
    quantized_matmul(x, wq, scales, biases, transpose=True, group_size=64, bits=4)
    gather_qmm(x, wq, scales, biases, lhs_indices=None, rhs_indices=None,
               transpose=True, group_size=64, bits=4, sorted_indices=False)

Tensors live on a ROCm device: activations, scales and biases are bfloat16;
packed weights are uint32 (int32 is accepted as the same bits).  Invalid
arguments raise ValueError like MLX; settings MLX accepts but this backend
does not implement (transpose=False, non-affine modes) raise
NotImplementedError.  Bits 2, 3, 5 and 6 quantize and dequantize natively;
their matmuls run on the 8-bit kernels after the codes are rewritten one byte
each (repack_codes_u8: per call here, once at load time in the model
loader).  There is no CPU or PyTorch fallback.
"""

from __future__ import annotations

import math

import torch

from . import _lib

_CODE_DTYPES = (torch.int32, getattr(torch, "uint32", torch.int32))


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require_gpu(op: str, **tensors: torch.Tensor | None) -> torch.device:
    dev = None
    for name, t in tensors.items():
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"[{op}] {name} must be a torch.Tensor")
        if t.device.type != "cuda":
            raise ValueError(f"[{op}] {name} must be on a ROCm GPU device, got {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"[{op}] all inputs must be on one device ({dev} vs {t.device})")
    return dev


def _check_mode(op: str, mode: str) -> None:
    if mode != "affine":
        raise NotImplementedError(f"[{op}] mode={mode!r} is not implemented (affine only)")


def _check_bf16(op: str, name: str, t: torch.Tensor) -> None:
    if t.dtype != torch.bfloat16:
        raise ValueError(f"[{op}] {name} must be bfloat16, got {t.dtype}")


def _check_codes(op: str, w: torch.Tensor) -> None:
    if w.dtype not in _CODE_DTYPES:
        raise ValueError(f"[{op}] The weight matrix should be uint32 but received {w.dtype}")


def _check_quantized(op: str, w, scales, biases, group_size: int, bits: int) -> int:
    """Validate (w, scales, biases); returns K (unpacked input dimension)."""
    _check_codes(op, w)
    _check_bf16(op, "scales", scales)
    _check_bf16(op, "biases", biases)
    if scales.shape != biases.shape:
        raise ValueError(
            f"[{op}] Scales and biases should have the same shape. Received scales with "
            f"shape {tuple(scales.shape)} and biases with {tuple(biases.shape)}.")
    if w.ndim < 2 or w.shape[:-1] != scales.shape[:-1]:
        raise ValueError(
            f"[{op}] Weight and scales should have the same batch shape. Received weight "
            f"with shape {tuple(w.shape)} and scales with {tuple(scales.shape)}.")
    if bits not in (2, 3, 4, 5, 6, 8):
        raise ValueError(f"[{op}] The requested number of bits {bits} is not supported. "
                         "The supported bits are 2, 3, 4, 5, 6 and 8.")
    if group_size not in (32, 64, 128):
        raise ValueError(f"[{op}] The requested group size {group_size} is not supported. "
                         "The supported group sizes are 32, 64 and 128.")
    K = w.shape[-1] * 32 // bits
    if w.shape[-1] * 32 % bits or scales.shape[-1] * group_size != K:
        raise ValueError(
            f"[{op}] The shapes of the weight and scales are incompatible based on bits and "
            f"group_size. w.shape() == {tuple(w.shape)} and scales.shape() == "
            f"{tuple(scales.shape)} with group_size={group_size} and bits={bits}")
    return K


# --------------------------------------------------------------------- ops


def quantize(w: torch.Tensor, group_size: int = 64, bits: int = 4, mode: str = "affine"):
    """mx.quantize for a bfloat16 matrix w[..., K] -> (wq uint32-bits int32, scales, biases).

    Follows mlx.core.quantize as called at models/lfm2.py:112-117,142-151.
    float32 inputs are rounded to bfloat16 first (scales and biases come out
    in bfloat16, the dtype the quantized kernels consume).
    """
    op = "quantize"
    _check_mode(op, mode)
    _require_gpu(op, w=w)
    if w.ndim < 2:
        raise ValueError(f"[{op}] The matrix to be quantized must have at least 2 dimensions "
                         f"but it has only {w.ndim}.")
    if w.dtype == torch.float32 or w.dtype == torch.float16:
        w = w.to(torch.bfloat16)
    _check_bf16(op, "w", w)
    K = w.shape[-1]
    if K % group_size:
        raise ValueError(
            f"[{op}] The last dimension of the matrix needs to be divisible by the quantization "
            f"group size {group_size}. However the provided matrix has shape {tuple(w.shape)}")
    w = w.contiguous()
    rows = w.numel() // K
    lead = tuple(w.shape[:-1])
    wq = torch.empty(lead + (K * bits // 32,), dtype=torch.int32, device=w.device)
    s = torch.empty(lead + (K // group_size,), dtype=torch.bfloat16, device=w.device)
    b = torch.empty_like(s)
    L = _lib.lib()
    _lib.check(L.mq_quantize(_ptr(w), _ptr(wq), _ptr(s), _ptr(b), rows, K, group_size, bits,
                             _stream(w)), op)
    return wq, s, b


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int = 64,
               bits: int = 4, mode: str = "affine") -> torch.Tensor:
    """mx.dequantize -> bfloat16 [..., K]; out = bf16(bf16(q*scale) + bias)."""
    op = "dequantize"
    _check_mode(op, mode)
    _require_gpu(op, w=w, scales=scales, biases=biases)
    K = _check_quantized(op, w, scales, biases, group_size, bits)
    w, scales, biases = w.contiguous(), scales.contiguous(), biases.contiguous()
    rows = w.numel() // w.shape[-1] if w.shape[-1] else 0
    out = torch.empty(tuple(w.shape[:-1]) + (K,), dtype=torch.bfloat16, device=w.device)
    L = _lib.lib()
    _lib.check(L.mq_dequantize(_ptr(w), _ptr(scales), _ptr(biases), _ptr(out), rows, K,
                               group_size, bits, _stream(w)), op)
    return out


def repack_codes_u8(w: torch.Tensor, bits: int) -> torch.Tensor:
    """2/3/5/6-bit codes [..., K*bits/32] -> the same codes one byte each
    [..., K/4] (the 8-bit layout; with the unchanged scales and biases the
    matrix dequantizes to the same weights and runs on the 8-bit kernels)."""
    op = "repack_codes_u8"
    _require_gpu(op, w=w)
    _check_codes(op, w)
    if bits not in (2, 3, 5, 6):
        raise ValueError(f"[{op}] only 2, 3, 5 and 6-bit codes are repacked, got bits={bits}")
    if w.ndim < 1 or w.shape[-1] * 32 % bits or (w.shape[-1] * 32 // bits) % 32:
        raise ValueError(f"[{op}] {tuple(w.shape)} does not hold a multiple of 32 {bits}-bit "
                         "codes per row")
    K = w.shape[-1] * 32 // bits
    wc = w.contiguous()
    rows = wc.numel() // w.shape[-1]
    out = torch.empty(tuple(w.shape[:-1]) + (K // 4,), dtype=torch.int32, device=w.device)
    _lib.check(_lib.lib().mq_repack_codes_u8(_ptr(wc), _ptr(out), rows, K, bits, _stream(w)), op)
    return out


def embedding_lookup(ids: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: torch.Tensor, group_size: int = 64, bits: int = 4) -> torch.Tensor:
    """Dequantized rows w[ids] -> bfloat16 [*ids.shape, K] (nn.QuantizedEmbedding.__call__)."""
    op = "embedding_lookup"
    _require_gpu(op, ids=ids, w=w, scales=scales, biases=biases)
    K = _check_quantized(op, w, scales, biases, group_size, bits)
    if w.ndim != 2:
        raise ValueError(f"[{op}] the embedding table must be 2-D, got {tuple(w.shape)}")
    flat = ids.reshape(-1).to(torch.int32).contiguous()
    out = torch.empty(tuple(ids.shape) + (K,), dtype=torch.bfloat16, device=w.device)
    L = _lib.lib()
    _lib.check(L.mq_embedding_lookup(_ptr(flat), flat.numel(), _ptr(w.contiguous()),
                                     _ptr(scales.contiguous()), _ptr(biases.contiguous()),
                                     w.shape[0], K, group_size, bits, _ptr(out), _stream(w)), op)
    return out


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: torch.Tensor, transpose: bool = True, group_size: int = 64,
                     bits: int = 4, mode: str = "affine",
                     bias: torch.Tensor | None = None) -> torch.Tensor:
    """mx.quantized_matmul(x, w, scales, biases, transpose=True) -> x @ dequantize(w).T.

    ``bias`` (bfloat16 [N]) fuses QuantizedLinear's "+ bias" into the store.
    """
    op = "quantized_matmul"
    _check_mode(op, mode)
    _require_gpu(op, x=x, w=w, scales=scales, biases=biases, bias=bias)
    K = _check_quantized(op, w, scales, biases, group_size, bits)
    _check_bf16(op, "x", x)
    if w.ndim != 2:
        raise ValueError(f"[{op}] batched weights are not supported here; got {tuple(w.shape)}")
    if not transpose:
        raise NotImplementedError(f"[{op}] transpose=False is not implemented on this backend")
    if x.ndim < 1 or x.shape[-1] != K:
        raise ValueError(
            f"[{op}] Last dimension of first input with shape {tuple(x.shape)} must match "
            f"second input with shape {(w.shape[0], K)}.")
    N = w.shape[0]
    if bias is not None:
        _check_bf16(op, "bias", bias)
        if bias.shape != (N,):
            raise ValueError(f"[{op}] bias must have shape ({N},), got {tuple(bias.shape)}")
        bias = bias.contiguous()
    xc = x.contiguous()
    M = xc.numel() // K
    y = torch.empty(tuple(x.shape[:-1]) + (N,), dtype=torch.bfloat16, device=x.device)
    L = _lib.lib()
    ws_bytes = L.mq_quantized_matmul_workspace(M, N, K, group_size, bits) if M and N else 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    _lib.check(L.mq_quantized_matmul_ws(_ptr(xc), _ptr(w.contiguous()), _ptr(scales.contiguous()),
                                        _ptr(biases.contiguous()), _ptr(bias), _ptr(y), M, N, K,
                                        group_size, bits, 1, _ptr(ws), ws_bytes, _stream(x)), op)
    return y


def swiglu_supported(M: int, N: int, K: int, group_size: int = 64, bits: int = 4) -> bool:
    """Whether quantized_matmul_swiglu takes M rows of x against a [2N, K] gate|up matrix."""
    return bool(_lib.lib().mq_quantized_matmul_swiglu_supported(M, N, K, group_size, bits))


def quantized_matmul_swiglu(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                            biases: torch.Tensor, group_size: int = 64,
                            bits: int = 4) -> torch.Tensor:
    """silu(x @ gate^T) * (x @ up^T) for a fused gate|up matrix w [2N, K] (gate
    rows first), as silu_mul(quantized_matmul(x, w, ...)) computes it, bit for
    bit, in one kernel (decode shapes: see swiglu_supported)."""
    op = "quantized_matmul_swiglu"
    _require_gpu(op, x=x, w=w, scales=scales, biases=biases)
    K = _check_quantized(op, w, scales, biases, group_size, bits)
    _check_bf16(op, "x", x)
    if w.ndim != 2 or w.shape[0] % 2:
        raise ValueError(f"[{op}] w must be [2N, K * bits / 32], got {tuple(w.shape)}")
    if x.shape[-1] != K:
        raise ValueError(f"[{op}] x has {x.shape[-1]} columns, expected {K}")
    N = w.shape[0] // 2
    xc = x.contiguous()
    M = xc.numel() // K
    y = torch.empty(tuple(x.shape[:-1]) + (N,), dtype=torch.bfloat16, device=x.device)
    L = _lib.lib()
    ws_bytes = L.mq_quantized_matmul_swiglu_workspace(M, N, K, group_size, bits) if M else 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    _lib.check(L.mq_quantized_matmul_swiglu_ws(
        _ptr(xc), _ptr(w.contiguous()), _ptr(scales.contiguous()), _ptr(biases.contiguous()),
        _ptr(y), M, N, K, group_size, bits, _ptr(ws), ws_bytes, _stream(x)), op)
    return y


def add_norm_supported(M: int, N: int, K: int, group_size: int = 64, bits: int = 4) -> bool:
    """Whether quantized_matmul_add_rms_norm takes this shape."""
    return bool(_lib.lib().mq_quantized_matmul_add_rms_norm_supported(M, N, K, group_size, bits))


def quantized_matmul_add_rms_norm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                                  biases: torch.Tensor, residual: torch.Tensor,
                                  norm_weight: torch.Tensor, eps: float,
                                  bias: torch.Tensor | None = None, group_size: int = 64,
                                  bits: int = 4):
    """y = quantized_matmul(x, w) (+ bias), h = bf16(y + residual), out =
    rms_norm(h) * norm_weight, in the GEMM and its split-K reduce; equal bit for
    bit to quantized_matmul then decode_ops.rms_norm(y, ..., residual).
    Returns (out, h)."""
    op = "quantized_matmul_add_rms_norm"
    _require_gpu(op, x=x, w=w, scales=scales, biases=biases, residual=residual,
                 norm_weight=norm_weight, bias=bias)
    K = _check_quantized(op, w, scales, biases, group_size, bits)
    _check_bf16(op, "x", x)
    _check_bf16(op, "residual", residual)
    _check_bf16(op, "norm_weight", norm_weight)
    if x.shape[-1] != K:
        raise ValueError(f"[{op}] x has {x.shape[-1]} columns, expected {K}")
    N = w.shape[0]
    xc = x.contiguous()
    M = xc.numel() // K
    out_shape = tuple(x.shape[:-1]) + (N,)
    if tuple(residual.shape) != out_shape:
        raise ValueError(f"[{op}] residual must have shape {out_shape}")
    if norm_weight.shape != (N,):
        raise ValueError(f"[{op}] norm_weight must have shape ({N},)")
    if bias is not None:
        _check_bf16(op, "bias", bias)
        bias = bias.contiguous()
    out = torch.empty(out_shape, dtype=torch.bfloat16, device=x.device)
    h = torch.empty_like(out)
    L = _lib.lib()
    ws_bytes = L.mq_quantized_matmul_add_rms_norm_workspace(M, N, K, group_size, bits) if M else 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
    _lib.check(L.mq_quantized_matmul_add_rms_norm(
        _ptr(xc), _ptr(w.contiguous()), _ptr(scales.contiguous()), _ptr(biases.contiguous()),
        _ptr(bias), _ptr(residual.contiguous()), _ptr(h), _ptr(norm_weight.contiguous()),
        float(eps), _ptr(out), M, N, K, group_size, bits, _ptr(ws), ws_bytes, _stream(x)), op)
    return out, h


def rms_norm_qmm_supported(M: int, N: int, K: int, group_size: int = 64, bits: int = 4,
                           swiglu: bool = False) -> bool:
    """Whether rms_norm_quantized_matmul takes this shape (N outputs)."""
    return bool(_lib.lib().mq_rms_norm_quantized_matmul_supported(M, N, K, group_size, bits,
                                                                  int(swiglu)))


def rms_norm_quantized_matmul(a: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                              w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                              bias: torch.Tensor | None = None,
                              residual: torch.Tensor | None = None, group_size: int = 64,
                              bits: int = 4, swiglu: bool = False):
    """RMSNorm of one row then the quantized linear (or its SwiGLU form), one
    kernel: h = bf16(a + residual) (a without residual), x = rms_norm(h) *
    norm_weight as decode_ops.rms_norm computes it, y = quantized_matmul(x, w)
    (+ bias), or silu(gate) * up of a [2N, K] gate|up w.  Returns (y, h)."""
    op = "rms_norm_quantized_matmul"
    _require_gpu(op, a=a, norm_weight=norm_weight, w=w, scales=scales, biases=biases, bias=bias,
                 residual=residual)
    K = _check_quantized(op, w, scales, biases, group_size, bits)
    _check_bf16(op, "a", a)
    _check_bf16(op, "norm_weight", norm_weight)
    if a.shape[-1] != K or a.numel() != K:
        raise ValueError(f"[{op}] a must be one row of {K}, got {tuple(a.shape)}")
    if norm_weight.shape != (K,):
        raise ValueError(f"[{op}] norm_weight must have shape ({K},)")
    N = w.shape[0] // 2 if swiglu else w.shape[0]
    ac = a.contiguous()
    h = None
    if residual is not None:
        _check_bf16(op, "residual", residual)
        if residual.shape != a.shape:
            raise ValueError(f"[{op}] residual shape {tuple(residual.shape)} != {tuple(a.shape)}")
        residual = residual.contiguous()
        h = torch.empty_like(ac)
    if bias is not None:
        _check_bf16(op, "bias", bias)
        bias = bias.contiguous()
    y = torch.empty(tuple(a.shape[:-1]) + (N,), dtype=torch.bfloat16, device=a.device)
    _lib.check(_lib.lib().mq_rms_norm_quantized_matmul(
        _ptr(ac), _ptr(residual), _ptr(h), _ptr(norm_weight.contiguous()), float(eps),
        _ptr(w.contiguous()), _ptr(scales.contiguous()), _ptr(biases.contiguous()), _ptr(bias),
        _ptr(y), 1, N, K, group_size, bits, int(swiglu), _stream(a)), op)
    return y, (ac if h is None else h)


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               lhs_indices: torch.Tensor | None = None, rhs_indices: torch.Tensor | None = None,
               transpose: bool = True, group_size: int = 64, bits: int = 4, mode: str = "affine",
               sorted_indices: bool = False, expert_offsets: torch.Tensor | None = None
               ) -> torch.Tensor:
    """mx.gather_qmm: out[b] = x[lhs[b]] @ dequantize(w[rhs[b]]).T, b over the index batch.

    x is [..., M, K] (its batch dims flattened are what lhs_indices index), w is
    [..., N, K*bits/32] (batch dims flattened are the experts rhs_indices
    index).  The output shape is broadcast(lhs_indices, rhs_indices) + [M, N];
    a missing lhs_indices means "every x batch in order" and broadcasts the same
    way, as in mlx (models/lfm2.py:176-187, 202-218).  With sorted_indices the
    flat rhs must be non-decreasing (as MLX assumes); expert_offsets (int32
    [E + 1], the segment starts expert_sort / route_sort return) spares the
    kernel deriving the segments.
    """
    op = "gather_qmm"
    _check_mode(op, mode)
    _require_gpu(op, x=x, w=w, scales=scales, biases=biases, lhs_indices=lhs_indices,
                 rhs_indices=rhs_indices)
    K = _check_quantized(op, w, scales, biases, group_size, bits)
    _check_bf16(op, "x", x)
    if not transpose:
        raise NotImplementedError(f"[{op}] transpose=False is not implemented on this backend")
    if x.ndim < 2 or x.shape[-1] != K:
        raise ValueError(f"[{op}] x must be [..., M, {K}], got {tuple(x.shape)}")
    if bits not in (4, 8):  # the expert kernels read word-aligned codes
        w, bits = repack_codes_u8(w, bits), 8
    M = x.shape[-2]
    N = w.shape[-2]
    E = math.prod(w.shape[:-2])
    x_batch = tuple(x.shape[:-2])
    n_xb = math.prod(x_batch)
    dev = x.device
    if rhs_indices is None:
        rhs_indices = torch.arange(E, device=dev).reshape(tuple(w.shape[:-2]))
    for name, t in (("lhs_indices", lhs_indices), ("rhs_indices", rhs_indices)):
        if t is not None and (t.dtype.is_floating_point or t.dtype == torch.bool):
            raise ValueError(f"[{op}] {name} must be an integer array, got {t.dtype}")
    lhs_shape = x_batch if lhs_indices is None else tuple(lhs_indices.shape)
    out_batch = torch.broadcast_shapes(lhs_shape, tuple(rhs_indices.shape))
    T = math.prod(out_batch)
    rhs_flat = rhs_indices.expand(out_batch).reshape(-1).to(torch.int32).contiguous()
    if lhs_indices is None and tuple(out_batch) == x_batch:
        lhs_flat = None  # identity: batch t reads x batch t
    else:
        lhs_full = (torch.arange(n_xb, device=dev).reshape(x_batch) if lhs_indices is None
                    else lhs_indices)
        lhs_flat = lhs_full.expand(out_batch).reshape(-1).to(torch.int32).contiguous()
    xc = x.contiguous()
    y = torch.empty(tuple(out_batch) + (M, N), dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    if expert_offsets is not None and not sorted_indices:
        raise ValueError(f"[{op}] expert_offsets are the segments of expert-sorted rows: pass "
                         "sorted_indices=True with them")
    if expert_offsets is not None:
        if expert_offsets.dtype != torch.int32 or expert_offsets.numel() != E + 1:
            raise ValueError(f"[{op}] expert_offsets must be int32 [{E + 1}]")
        _require_gpu(op, expert_offsets=expert_offsets)
        _lib.check(L.mq_gather_qmm_segments(
            _ptr(xc), _ptr(lhs_flat), _ptr(rhs_flat), _ptr(expert_offsets.contiguous()),
            _ptr(w.contiguous()), _ptr(scales.contiguous()), _ptr(biases.contiguous()), _ptr(y),
            T, M, N, K, E, n_xb, group_size, bits, 0, _stream(x)), op)
        return y
    _lib.check(L.mq_gather_qmm(_ptr(xc), _ptr(lhs_flat), _ptr(rhs_flat), _ptr(w.contiguous()),
                               _ptr(scales.contiguous()), _ptr(biases.contiguous()), _ptr(y), T, M,
                               N, K, E, n_xb, group_size, bits, 1, int(bool(sorted_indices)),
                               _stream(x)), op)
    return y


def gather_swiglu_supported(T: int, M: int, N: int, K: int, group_size: int = 64,
                            bits: int = 4) -> bool:
    """Whether gather_qmm_swiglu takes T (batch, expert) pairs of M rows, N outputs."""
    return bool(_lib.lib().mq_gather_qmm_swiglu_supported(T, M, N, K, group_size, bits))


def gather_segments_supported(T: int, M: int, N: int, K: int, E: int, x_batches: int,
                              group_size: int = 64, bits: int = 4, swiglu: bool = False) -> bool:
    """Whether gather_qmm / gather_qmm_swiglu with expert_offsets take these sizes
    (swiglu: N is the output width of a 2N-row gate|up bank)."""
    return bool(_lib.lib().mq_gather_qmm_segments_supported(T, M, N, K, E, x_batches, group_size,
                                                            bits, int(bool(swiglu))))


def gather_qmm_swiglu(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                      biases: torch.Tensor, lhs_indices: torch.Tensor | None,
                      rhs_indices: torch.Tensor, group_size: int = 64,
                      bits: int = 4, expert_offsets: torch.Tensor | None = None
                      ) -> torch.Tensor:
    """SwitchGLU's gate/up projections and silu(gate) * up (models/lfm2.py:208-214) for
    gathered pairs: w [E, 2N, K*bits/32] holds every expert's gate rows, then its up
    rows; x [n_x, M, K]; rhs_indices [T] (expert per pair), lhs_indices [T] (x batch
    per pair, or None: pair t reads batch t).  Returns bf16 [T, M, N] =
    silu_mul(gather_qmm(x, w, ...)), bit for bit, for the shapes
    gather_swiglu_supported takes."""
    op = "gather_qmm_swiglu"
    _require_gpu(op, x=x, w=w, scales=scales, biases=biases, lhs_indices=lhs_indices,
                 rhs_indices=rhs_indices)
    K = _check_quantized(op, w, scales, biases, group_size, bits)
    _check_bf16(op, "x", x)
    if x.ndim < 2 or x.shape[-1] != K:
        raise ValueError(f"[{op}] x must be [..., M, {K}], got {tuple(x.shape)}")
    if w.ndim != 3 or w.shape[1] % 2:
        raise ValueError(f"[{op}] w must be [E, 2N, K*bits/32], got {tuple(w.shape)}")
    if bits not in (4, 8):  # the expert kernels read word-aligned codes
        w, bits = repack_codes_u8(w, bits), 8
    M, N, E = x.shape[-2], w.shape[1] // 2, w.shape[0]
    n_xb = math.prod(x.shape[:-2])
    rhs = rhs_indices.reshape(-1).to(torch.int32).contiguous()
    T = rhs.numel()
    lhs = None if lhs_indices is None else lhs_indices.reshape(-1).to(torch.int32).contiguous()
    if lhs is not None and lhs.numel() != T:
        raise ValueError(f"[{op}] lhs_indices and rhs_indices differ in length")
    y = torch.empty(T, M, N, dtype=torch.bfloat16, device=x.device)
    L = _lib.lib()
    if expert_offsets is not None:
        # rows sorted by expert with the sort's segment offsets: the segment GEMM
        # with SiLU * up in its epilogue (its GEMV form for decode-sized batches)
        if expert_offsets.dtype != torch.int32 or expert_offsets.numel() != E + 1:
            raise ValueError(f"[{op}] expert_offsets must be int32 [{E + 1}]")
        _require_gpu(op, expert_offsets=expert_offsets)
        _lib.check(L.mq_gather_qmm_segments(
            _ptr(x.contiguous()), _ptr(lhs), _ptr(rhs), _ptr(expert_offsets.contiguous()),
            _ptr(w.contiguous()), _ptr(scales.contiguous()), _ptr(biases.contiguous()), _ptr(y),
            T, M, N, K, E, n_xb, group_size, bits, 1, _stream(x)), op)
        return y
    _lib.check(L.mq_gather_qmm_swiglu(_ptr(x.contiguous()), _ptr(lhs), _ptr(rhs),
                                      _ptr(w.contiguous()), _ptr(scales.contiguous()),
                                      _ptr(biases.contiguous()), _ptr(y), T, M, N, K, E, n_xb,
                                      group_size, bits, _stream(x)), op)
    return y
