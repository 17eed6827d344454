"""Quantized layer modules with the call surface the reference's graphs use.

* QuantizedLinear      -- mlx.nn.QuantizedLinear: weight/scales/biases/bias,
                          group_size, bits, mode; __call__(x) =
                          quantized_matmul(x, ..., transpose=True) + bias
                          (built by nn.quantize at models/qwen2.py:318-324).
* QuantizedEmbedding   -- mlx.nn.QuantizedEmbedding: __call__(ids) returns the
                          dequantized rows, as_linear(x) is the tied LM head
                          (models/qwen2.py:185, 226).
* QuantizedSwitchLinear-- models/lfm2.py:124-190: weight [E, N, K*bits/32],
                          __call__(x, indices, sorted_indices=False) =
                          gather_qmm(...) + bias[indices].
* SwitchGLU            -- models/lfm2.py:193-218 with the expert sort of
                          models/lfm2.py:613-622 (_gather_sort/_scatter_unsort).
* quantize(model, ...) -- nn.quantize: swaps torch Linear/Embedding modules for
                          the quantized ones (class_predicate as in
                          models/qwen2.py:315-316).

Modules are torch.nn.Modules holding buffers; the math runs in libmi355q.
"""

from __future__ import annotations

from typing import Callable

import torch
import torch.nn.functional as F

from . import core


class QuantizedLinear(torch.nn.Module):
    def __init__(self, input_dims: int, output_dims: int, bias: bool = True,
                 group_size: int = 64, bits: int = 4, mode: str = "affine",
                 device: torch.device | str | None = None):
        super().__init__()
        self.group_size, self.bits, self.mode = group_size, bits, mode
        dev = torch.device(device) if device is not None else torch.device("cuda")
        self.register_buffer("weight", torch.zeros(output_dims, input_dims * bits // 32,
                                                   dtype=torch.int32, device=dev))
        self.register_buffer("scales", torch.zeros(output_dims, input_dims // group_size,
                                                   dtype=torch.bfloat16, device=dev))
        self.register_buffer("biases", torch.zeros_like(self.scales))
        if bias:
            self.register_buffer("bias", torch.zeros(output_dims, dtype=torch.bfloat16, device=dev))
        else:
            self.bias = None

    @property
    def input_dims(self) -> int:
        return self.scales.shape[-1] * self.group_size

    @property
    def output_dims(self) -> int:
        return self.weight.shape[0]

    @classmethod
    def from_weights(cls, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                     bias: torch.Tensor | None = None, group_size: int = 64, bits: int = 4,
                     mode: str = "affine") -> "QuantizedLinear":
        """Wrap already-quantized tensors ({path}.weight/.scales/.biases of a checkpoint)."""
        m = cls.__new__(cls)
        torch.nn.Module.__init__(m)
        m.group_size, m.bits, m.mode = group_size, bits, mode
        m.register_buffer("weight", weight)
        m.register_buffer("scales", scales)
        m.register_buffer("biases", biases)
        if bias is not None:
            m.register_buffer("bias", bias)
        else:
            m.bias = None
        return m

    @classmethod
    def from_linear(cls, linear: torch.nn.Linear, group_size: int = 64, bits: int = 4,
                    mode: str = "affine") -> "QuantizedLinear":
        """nn.QuantizedLinear.from_linear: quantize a dense (GPU) linear layer."""
        w = linear.weight.detach().to(torch.bfloat16)
        wq, s, b = core.quantize(w, group_size, bits, mode)
        bias = None if linear.bias is None else linear.bias.detach().to(torch.bfloat16)
        return cls.from_weights(wq, s, b, bias, group_size, bits, mode)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return core.quantized_matmul(x, self.weight, self.scales, self.biases, transpose=True,
                                     group_size=self.group_size, bits=self.bits, mode=self.mode,
                                     bias=self.bias)


class QuantizedEmbedding(torch.nn.Module):
    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 group_size: int = 64, bits: int = 4, mode: str = "affine"):
        super().__init__()
        self.group_size, self.bits, self.mode = group_size, bits, mode
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)

    @classmethod
    def from_embedding(cls, emb: torch.nn.Embedding, group_size: int = 64, bits: int = 4,
                       mode: str = "affine") -> "QuantizedEmbedding":
        wq, s, b = core.quantize(emb.weight.detach().to(torch.bfloat16), group_size, bits, mode)
        return cls(wq, s, b, group_size, bits, mode)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return core.embedding_lookup(ids, self.weight, self.scales, self.biases,
                                     self.group_size, self.bits)

    def as_linear(self, x: torch.Tensor) -> torch.Tensor:
        return core.quantized_matmul(x, self.weight, self.scales, self.biases, transpose=True,
                                     group_size=self.group_size, bits=self.bits, mode=self.mode)


class QuantizedSwitchLinear(torch.nn.Module):
    """Expert-indexed quantized linear (models/lfm2.py:124-190)."""

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 bias: torch.Tensor | None = None, group_size: int = 64, bits: int = 4,
                 mode: str = "affine"):
        super().__init__()
        self.group_size, self.bits, self.mode = group_size, bits, mode
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)
        if bias is not None:
            self.register_buffer("bias", bias)
        else:
            self.bias = None

    @classmethod
    def from_dense(cls, weight: torch.Tensor, bias: torch.Tensor | None = None,
                   group_size: int = 64, bits: int = 4, mode: str = "affine"):
        """SwitchLinear.to_quantized (models/lfm2.py:97-121): quantize [E, N, K] weights."""
        wq, s, b = core.quantize(weight.to(torch.bfloat16), group_size, bits, mode)
        return cls(wq, s, b, bias, group_size, bits, mode)

    @property
    def input_dims(self) -> int:
        return self.scales.shape[-1] * self.group_size

    @property
    def output_dims(self) -> int:
        return self.weight.shape[1]

    @property
    def num_experts(self) -> int:
        return self.weight.shape[0]

    def forward(self, x: torch.Tensor, indices: torch.Tensor, *,
                sorted_indices: bool = False) -> torch.Tensor:
        out = core.gather_qmm(x, self.weight, self.scales, self.biases, rhs_indices=indices,
                              transpose=True, group_size=self.group_size, bits=self.bits,
                              mode=self.mode, sorted_indices=sorted_indices)
        if self.bias is not None:
            out = out + self.bias[indices].unsqueeze(-2)
        return out


def _gather_sort(x: torch.Tensor, indices: torch.Tensor):
    """models/lfm2.py:613-618: sort the flat expert ids, gather x rows to match."""
    width = indices.shape[-1]
    flat = indices.reshape(-1)
    order = torch.argsort(flat, stable=True)
    inverse = torch.argsort(order, stable=True)
    xf = x.reshape((-1,) + tuple(x.shape[-2:]))
    return xf[order // width], flat[order], inverse


def _scatter_unsort(x: torch.Tensor, inverse: torch.Tensor, shape) -> torch.Tensor:
    """models/lfm2.py:621-622."""
    return x[inverse].reshape(tuple(shape) + tuple(x.shape[1:]))


class SwitchGLU(torch.nn.Module):
    """SwiGLU expert bank with top-k routing (models/lfm2.py:193-218)."""

    def __init__(self, gate_proj: QuantizedSwitchLinear, up_proj: QuantizedSwitchLinear,
                 down_proj: QuantizedSwitchLinear):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj

    def forward(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        x = x.unsqueeze(-2).unsqueeze(-2)  # mx.expand_dims(x, (-2, -3))
        do_sort = indices.numel() >= 64
        selected, inverse = indices, None
        if do_sort:
            x, selected, inverse = _gather_sort(x, indices)
        up = self.up_proj(x, selected, sorted_indices=do_sort)
        gate = self.gate_proj(x, selected, sorted_indices=do_sort)
        out = self.down_proj(F.silu(gate) * up, selected, sorted_indices=do_sort)
        if do_sort:
            out = _scatter_unsort(out, inverse, indices.shape)
        return out.squeeze(-2)


def quantize(model: torch.nn.Module, group_size: int = 64, bits: int = 4, mode: str = "affine",
             class_predicate: Callable[[str, torch.nn.Module], bool | dict] | None = None
             ) -> torch.nn.Module:
    """nn.quantize: replace Linear/Embedding submodules in place with quantized ones.

    class_predicate(path, module) may return False (skip), True (use the
    defaults) or a dict with group_size/bits/mode overrides, as in
    models/lfm2.py:579-591.
    """
    for path, module in list(model.named_modules()):
        if not isinstance(module, (torch.nn.Linear, torch.nn.Embedding)):
            continue
        params = {"group_size": group_size, "bits": bits, "mode": mode}
        if class_predicate is not None:
            decision = class_predicate(path, module)
            if not decision:
                continue
            if isinstance(decision, dict):
                params.update(decision)
        if isinstance(module, torch.nn.Linear):
            new = QuantizedLinear.from_linear(module, **params)
        else:
            new = QuantizedEmbedding.from_embedding(module, **params)
        parent_path, _, name = path.rpartition(".")
        parent = model.get_submodule(parent_path) if parent_path else model
        setattr(parent, name, new)
    return model


__all__ = ["QuantizedLinear", "QuantizedEmbedding", "QuantizedSwitchLinear", "SwitchGLU",
           "quantize"]
