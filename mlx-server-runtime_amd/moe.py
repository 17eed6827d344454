"""Mixture-of-experts block on gather_qmm, executed by libmi355q.

Restates the reference's top-k routed SwiGLU expert block
(python/mlx_worker/native_mlx/models/lfm2.py:348-375, SwitchGLU :193-218,
_gather_sort/_scatter_unsort :613-622):

    route(logits, top_k, norm_topk_prob, expert_bias=None) -> (indices, scores)
        softmax(float32(logits)) (+ expert_bias), the top_k experts per token,
        their gates (renormalised to sum 1 when norm_topk_prob), bfloat16
    expert_sort(indices, num_experts) -> (sorted_ids, order, inverse, rows)
        stable sort of the flat expert ids; rows[p] = order[p] // top_k is the
        token whose x feeds sorted pair p (gather_qmm's lhs indices)
    combine(y, inverse, scores) -> out
        out[t] = sum_j bf16(y[inverse[t*k + j]] * scores[t, j])
    route_sort(logits, ...) -> (indices, scores, sorted_ids, order, inverse, rows)
        route then expert_sort, one launch for up to 64 tokens
    combine_rms_norm(y, inverse, scores, residual, weight, eps) -> (out, h)
        h = bf16(combine(...) + residual), out = RMSNorm(h) * weight, one launch

MoEBlock runs them around two gather_qmm calls: the experts' gate and up
projections concatenated per expert (one call, [E, 2I, H]), SiLU * up, and
the down projection.  Rows are sorted by expert when tokens * top_k >= 64,
as in the reference.  MoEBlock.residual_norm also folds the residual add and
the next RMSNorm into the combine.  Every fused form equals its unfused
sequence bit for bit.  There is no CPU fallback.
"""

from __future__ import annotations

import math

import torch

from . import _lib, core
from .core import _check_bf16, _ptr, _require_gpu, _stream
from .decode_ops import silu_mul


def route(logits: torch.Tensor, top_k: int, norm_topk_prob: bool = True,
          expert_bias: torch.Tensor | None = None):
    """logits bf16 [T, E] -> (indices int32 [T, top_k], scores bf16 [T, top_k])."""
    op = "moe_route"
    _require_gpu(op, logits=logits, expert_bias=expert_bias)
    _check_bf16(op, "logits", logits)
    T, E = logits.reshape(-1, logits.shape[-1]).shape
    if expert_bias is not None and (expert_bias.dtype != torch.float32
                                    or expert_bias.shape != (E,)):
        raise ValueError(f"[{op}] expert_bias must be float32 [{E}]")
    idx = torch.empty(T, top_k, dtype=torch.int32, device=logits.device)
    sc = torch.empty(T, top_k, dtype=torch.bfloat16, device=logits.device)
    L = _lib.lib()
    _lib.check(L.mq_moe_route(_ptr(logits.contiguous()), _ptr(expert_bias), T, E, top_k,
                              int(bool(norm_topk_prob)), _ptr(idx), _ptr(sc), _stream(logits)), op)
    return idx, sc


def expert_sort(indices: torch.Tensor, num_experts: int, with_offsets: bool = False):
    """indices int32 [T, k] -> (sorted_ids, order, inverse, rows), each int32 [T*k]
    (+ offsets int32 [num_experts + 1], where each expert's run of sorted_ids
    starts, with_offsets)."""
    op = "moe_sort"
    _require_gpu(op, indices=indices)
    if indices.dtype != torch.int32:
        raise ValueError(f"[{op}] indices must be int32, got {indices.dtype}")
    k = indices.shape[-1]
    flat = indices.contiguous().reshape(-1)
    n = flat.numel()
    outs = [torch.empty(n, dtype=torch.int32, device=flat.device) for _ in range(4)]
    offs = (torch.empty(num_experts + 1, dtype=torch.int32, device=flat.device)
            if with_offsets else None)
    L = _lib.lib()
    _lib.check(L.mq_moe_sort(_ptr(flat), n, k, num_experts, *(_ptr(t) for t in outs),
                             _ptr(offs), _stream(flat)), op)
    return (*outs, offs) if with_offsets else tuple(outs)


def combine(y: torch.Tensor, inverse: torch.Tensor | None, scores: torch.Tensor) -> torch.Tensor:
    """y bf16 [T*k, H] (expert order when inverse is given) -> bf16 [T, H]."""
    op = "moe_combine"
    y2, T, k, H = _combine_args(op, y, inverse, scores)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=y.device)
    L = _lib.lib()
    _lib.check(L.mq_moe_combine(_ptr(y2), _ptr(inverse), _ptr(scores.contiguous()), _ptr(out), T,
                                k, H, _stream(y)), op)
    return out


def route_sort(logits: torch.Tensor, top_k: int, num_experts: int,
               norm_topk_prob: bool = True, expert_bias: torch.Tensor | None = None,
               with_offsets: bool = False):
    """route(...) then expert_sort(indices, num_experts), in one launch when
    logits has at most 64 rows -> (indices, scores, sorted_ids, order, inverse,
    rows) (+ the experts' segment offsets [num_experts + 1], with_offsets)."""
    op = "moe_route_sort"
    _require_gpu(op, logits=logits, expert_bias=expert_bias)
    _check_bf16(op, "logits", logits)
    T, E = logits.reshape(-1, logits.shape[-1]).shape
    if E != num_experts:
        raise ValueError(f"[{op}] logits have {E} experts, expected {num_experts}")
    if expert_bias is not None and (expert_bias.dtype != torch.float32
                                    or expert_bias.shape != (E,)):
        raise ValueError(f"[{op}] expert_bias must be float32 [{E}]")
    dev = logits.device
    idx = torch.empty(T, top_k, dtype=torch.int32, device=dev)
    sc = torch.empty(T, top_k, dtype=torch.bfloat16, device=dev)
    outs = [torch.empty(T * top_k, dtype=torch.int32, device=dev) for _ in range(4)]
    offs = torch.empty(E + 1, dtype=torch.int32, device=dev) if with_offsets else None
    L = _lib.lib()
    _lib.check(L.mq_moe_route_sort(_ptr(logits.contiguous()), _ptr(expert_bias), T, E, top_k,
                                   int(bool(norm_topk_prob)), _ptr(idx), _ptr(sc),
                                   *(_ptr(t) for t in outs), _ptr(offs), _stream(logits)), op)
    return (idx, sc, *outs, offs) if with_offsets else (idx, sc, *outs)


def _combine_args(op, y, inverse, scores):
    _require_gpu(op, y=y, inverse=inverse, scores=scores)
    _check_bf16(op, "y", y)
    _check_bf16(op, "scores", scores)
    T, k = scores.shape
    H = y.shape[-1]
    y2 = y.contiguous().reshape(-1, H)
    if y2.shape[0] != T * k:
        raise ValueError(f"[{op}] y has {y2.shape[0]} rows, expected {T * k}")
    if inverse is not None and (inverse.dtype != torch.int32 or inverse.numel() != T * k):
        raise ValueError(f"[{op}] inverse must be int32 [{T * k}]")
    return y2, T, k, H


def combine_rms_norm(y: torch.Tensor, inverse: torch.Tensor | None, scores: torch.Tensor,
                     residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """h = bf16(combine(y, inverse, scores) + residual); returns
    (bf16(h * rsqrt(mean(h^2) + eps) * weight), h), both bf16 [T, H]."""
    op = "moe_combine_rms_norm"
    y2, T, k, H = _combine_args(op, y, inverse, scores)
    _require_gpu(op, residual=residual, weight=weight)
    _check_bf16(op, "residual", residual)
    _check_bf16(op, "weight", weight)
    if residual.numel() != T * H:
        raise ValueError(f"[{op}] residual has {residual.numel()} elements, expected {T * H}")
    if weight.shape != (H,):
        raise ValueError(f"[{op}] weight must have shape ({H},), got {tuple(weight.shape)}")
    out = torch.empty(T, H, dtype=torch.bfloat16, device=y.device)
    h = torch.empty_like(out)
    L = _lib.lib()
    _lib.check(L.mq_moe_combine_rms_norm(_ptr(y2), _ptr(inverse), _ptr(scores.contiguous()),
                                         _ptr(residual.contiguous()), _ptr(h),
                                         _ptr(weight.contiguous()), _ptr(out), T, k, H,
                                         float(eps), _stream(y)), op)
    return out, h


class QExperts:
    """Quantized expert bank: wq [E, N, K*bits/32], scales/biases [E, N, K/group]."""

    def __init__(self, wq, scales, biases, group_size=64, bits=4):
        self.wq, self.scales, self.biases = wq, scales, biases
        self.group_size, self.bits = group_size, bits

    @property
    def num_experts(self) -> int:
        return self.wq.shape[0]

    def __call__(self, x, lhs=None, rhs=None, sorted_indices=False, offsets=None):
        return core.gather_qmm(x, self.wq, self.scales, self.biases, lhs_indices=lhs,
                               rhs_indices=rhs, transpose=True, group_size=self.group_size,
                               bits=self.bits, sorted_indices=sorted_indices,
                               expert_offsets=offsets)

    def swiglu(self, x, lhs, rhs, sorted_indices=False, offsets=None):
        """silu(gate) * up of a gate|up bank (every expert: gate rows, then up rows)
        for the pairs (lhs, rhs): the fused kernel where it takes the shape, else
        gather_qmm then silu_mul -- the same bits either way."""
        T, M, K = rhs.numel(), x.shape[-2], x.shape[-1]
        N = self.wq.shape[1] // 2
        n_x = math.prod(x.shape[:-2]) if x.ndim > 2 else 1
        if (offsets is not None and sorted_indices and T * M > 64
                and core.gather_segments_supported(T, M, N, K, self.num_experts, n_x,
                                                   self.group_size, self.bits, swiglu=True)):
            # the expert-segment GEMM with SiLU * up in its epilogue (where it
            # takes the shape: an even number of groups per row)
            return core.gather_qmm_swiglu(x, self.wq, self.scales, self.biases, lhs, rhs,
                                          self.group_size, self.bits, expert_offsets=offsets)
        if core.gather_swiglu_supported(T, M, N, K, self.group_size, self.bits):
            return core.gather_qmm_swiglu(x, self.wq, self.scales, self.biases, lhs, rhs,
                                          self.group_size, self.bits)
        return silu_mul(self(x, lhs=lhs, rhs=rhs, sorted_indices=sorted_indices,
                             offsets=offsets if sorted_indices else None))


class MoEBlock:
    """Top-k routed SwiGLU experts (Lfm2MoE.__call__, models/lfm2.py:365-375)."""

    def __init__(self, gate, gate_up: QExperts, down: QExperts, top_k: int,
                 norm_topk_prob: bool = True, expert_bias: torch.Tensor | None = None):
        self.gate, self.gate_up, self.down = gate, gate_up, down
        self.top_k, self.norm_topk_prob, self.expert_bias = top_k, norm_topk_prob, expert_bias
        # A list here receives a copy of every call's routed expert ids
        # (int32 [T, k], token order): the routing trace, for eager calls
        # only (a captured graph's replays do not append).
        self.routing_log: list | None = None

    @property
    def num_experts(self) -> int:
        return self.gate_up.num_experts

    def _experts(self, xt: torch.Tensor):
        """xt bf16 [T, H] -> (y [T*k, H] in expert or token order, inverse, scores)."""
        T, H = xt.shape
        logits = self.gate(xt)
        xb = xt.reshape(T, 1, H)
        if T * self.top_k >= 64:  # the reference sorts at >= 64 pairs (lfm2.py:204)
            # the segment offsets feed the sorted GEMM; decode-sized batches
            # (<= 64 pairs) run per-pair GEMVs that do not read them
            sort = route_sort(logits, self.top_k, self.num_experts, self.norm_topk_prob,
                              self.expert_bias, with_offsets=T * self.top_k > 64)
            idx, sc, sorted_ids, _, inverse, rows = sort[:6]
            offs = sort[6] if len(sort) > 6 else None
            act = self.gate_up.swiglu(xb, rows, sorted_ids, sorted_indices=True, offsets=offs)
            y = self.down(act, rhs=sorted_ids, sorted_indices=True, offsets=offs)
        else:
            idx, sc = route(logits, self.top_k, self.norm_topk_prob, self.expert_bias)
            inverse = None
            rows = torch.arange(T, device=xt.device, dtype=torch.int32).repeat_interleave(
                self.top_k)
            flat = idx.reshape(-1)
            act = self.gate_up.swiglu(xb, rows, flat)
            y = self.down(act, rhs=flat)
        if self.routing_log is not None:
            self.routing_log.append(idx.clone())
        return y.reshape(T * self.top_k, H), inverse, sc

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        """x bf16 [..., H] -> bf16 [..., H]."""
        y, inverse, sc = self._experts(x.reshape(-1, x.shape[-1]))
        return combine(y, inverse, sc).reshape(x.shape)

    def residual_norm(self, x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                      eps: float):
        """The block, the residual add after it and the next RMSNorm
        (lfm2.py:409, then :404 or :436): h = bf16(self(x) + residual) ->
        (bf16(RMSNorm(h) * weight), h), shaped like x."""
        y, inverse, sc = self._experts(x.reshape(-1, x.shape[-1]))
        out, h = combine_rms_norm(y, inverse, sc, residual, weight, eps)
        return out.reshape(x.shape), h.reshape(x.shape)


__all__ = ["route", "expert_sort", "combine", "route_sort", "combine_rms_norm", "QExperts",
           "MoEBlock"]
