"""Qwen2-shaped decoder with 4/8-bit affine-quantized linears, greedy decode.

Restates the reference's native Qwen2 graph
(python/mlx_worker/native_mlx/models/qwen2.py:47-227) on PyTorch-ROCm, with
every linear layer and the token embedding running through libmi355q:

* attention (qwen2.py:47-117): q/k/v projections with bias, non-traditional
  RoPE (theta from the config), grouped-query attention with scale
  head_dim**-0.5 and a causal mask, o_proj without bias;
* MLP (qwen2.py:118-133): down(silu(gate(x)) * up(x)), no biases;
* block (qwen2.py:136-163): pre-norm RMSNorm, residual after attention and
  after the MLP; backbone (qwen2.py:166-196): embedding, layers, final RMSNorm;
* LM head (qwen2.py:199-227): untied quantized linear (or the tied embedding's
  as_linear), greedy argmax over the last position of each row
  (executor.py:406-414).

Two equivalent rearrangements keep the weights MLX's and the arithmetic the
same: q/k/v are concatenated into one quantized matrix (and gate/up into
another) so each is one launch, which is exact because the output columns of
a quantized matmul are independent.  Activations are bfloat16; RMSNorm, RoPE,
the softmax and the KV cache are float32.  The decode step is captured once
in a HIP graph and replayed per token (inputs live in static device buffers).
Weights can be random-initialised at the reference's 7B shape
(Qwen2Config.qwen25_7b) for benchmarking.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import core


@dataclass(frozen=True)
class Qwen2Config:
    hidden_size: int
    intermediate_size: int
    num_attention_heads: int
    num_key_value_heads: int
    num_hidden_layers: int
    vocab_size: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    tie_word_embeddings: bool = False
    group_size: int = 64
    bits: int = 4

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @classmethod
    def qwen25_7b(cls, bits: int = 4) -> "Qwen2Config":
        """Qwen2.5-7B: 28 layers, hidden 3584, 28 Q / 4 KV heads, MLP 18944, vocab 152064."""
        return cls(hidden_size=3584, intermediate_size=18944, num_attention_heads=28,
                   num_key_value_heads=4, num_hidden_layers=28, vocab_size=152064,
                   rms_norm_eps=1e-6, rope_theta=1e6, bits=bits)


class QLinear:
    """Quantized weight triple (+ optional bias) applied with quantized_matmul."""

    def __init__(self, wq, scales, biases, bias=None, group_size=64, bits=4):
        self.wq, self.scales, self.biases, self.bias = wq, scales, biases, bias
        self.group_size, self.bits = group_size, bits

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return core.quantized_matmul(x, self.wq, self.scales, self.biases, True,
                                     self.group_size, self.bits, bias=self.bias)

    @property
    def out_features(self) -> int:
        return self.wq.shape[0]


def _random_qlinear(gen, n_out, n_in, cfg, bias, device, std=0.02) -> QLinear:
    w = (torch.randn(n_out, n_in, generator=gen, device=device) * std).to(torch.bfloat16)
    wq, s, b = core.quantize(w, cfg.group_size, cfg.bits)
    del w
    bv = ((torch.randn(n_out, generator=gen, device=device) * std).to(torch.bfloat16)
          if bias else None)
    return QLinear(wq, s, b, bv, cfg.group_size, cfg.bits)


def _concat(parts: list[QLinear]) -> QLinear:
    """Row-wise concatenation: one launch computes every part's columns."""
    bias = None
    if parts[0].bias is not None:
        bias = torch.cat([p.bias for p in parts])
    return QLinear(torch.cat([p.wq for p in parts]), torch.cat([p.scales for p in parts]),
                   torch.cat([p.biases for p in parts]), bias, parts[0].group_size,
                   parts[0].bits)


@dataclass
class Layer:
    input_norm: torch.Tensor   # bfloat16 [hidden]
    post_norm: torch.Tensor    # bfloat16 [hidden]
    qkv: QLinear               # [(heads + 2 kv_heads) * head_dim, hidden], with bias
    o: QLinear                 # [hidden, heads * head_dim]
    gate_up: QLinear           # [2 * intermediate, hidden]
    down: QLinear              # [hidden, intermediate]


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """nn.RMSNorm: float32 x * rsqrt(mean(x^2) + eps) * weight, stored in x's dtype."""
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * weight.float()
    return y.to(x.dtype)


def rope_tables(cfg: Qwen2Config, max_len: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [max_len, head_dim/2] of mx.fast.rope (traditional=False, base=theta)."""
    half = cfg.head_dim // 2
    inv = cfg.rope_theta ** (-torch.arange(0, half, dtype=torch.float64, device=device) / half)
    ang = torch.arange(max_len, dtype=torch.float64, device=device)[:, None] * inv[None, :]
    return torch.cos(ang).float(), torch.sin(ang).float()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Non-traditional RoPE on the last dim: halves (x1, x2) rotate together.
    x [..., T, D] float32; cos/sin broadcastable to [..., T, D/2]."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)


class KVCache:
    """Dense float32 KV cache [layers][B, kv_heads, max_len, head_dim]."""

    def __init__(self, cfg: Qwen2Config, batch: int, max_len: int, device):
        shape = (batch, cfg.num_key_value_heads, max_len, cfg.head_dim)
        self.k = [torch.zeros(shape, dtype=torch.float32, device=device)
                  for _ in range(cfg.num_hidden_layers)]
        self.v = [torch.zeros(shape, dtype=torch.float32, device=device)
                  for _ in range(cfg.num_hidden_layers)]
        self.max_len = max_len


class Qwen2Model:
    def __init__(self, cfg: Qwen2Config, embed: QLinear, layers: list[Layer],
                 final_norm: torch.Tensor, lm_head: QLinear | None):
        self.cfg, self.embed, self.layers = cfg, embed, layers
        self.final_norm, self.lm_head = final_norm, lm_head
        self._graphs: dict = {}

    # ------------------------------------------------------------ weights
    @classmethod
    def random(cls, cfg: Qwen2Config, seed: int = 0, device="cuda:0") -> "Qwen2Model":
        """Random-init weights (bf16, quantized layer by layer) and unit norms: N(0, 0.02),
        except the two projections that write the residual stream (o_proj, down_proj),
        N(0, 0.02 / sqrt(2 * layers)) as in GPT-2 / Megatron initialisation -- with
        0.02 there too, a deep random stack amplifies bfloat16 rounding chaotically."""
        gen = torch.Generator(device=device).manual_seed(seed)
        h, d = cfg.hidden_size, cfg.head_dim
        res_std = 0.02 / math.sqrt(2 * cfg.num_hidden_layers)
        embed = _random_qlinear(gen, cfg.vocab_size, h, cfg, False, device)
        layers = []
        for _ in range(cfg.num_hidden_layers):
            q = _random_qlinear(gen, cfg.num_attention_heads * d, h, cfg, True, device)
            k = _random_qlinear(gen, cfg.num_key_value_heads * d, h, cfg, True, device)
            v = _random_qlinear(gen, cfg.num_key_value_heads * d, h, cfg, True, device)
            o = _random_qlinear(gen, h, cfg.num_attention_heads * d, cfg, False, device,
                                res_std)
            gate = _random_qlinear(gen, cfg.intermediate_size, h, cfg, False, device)
            up = _random_qlinear(gen, cfg.intermediate_size, h, cfg, False, device)
            down = _random_qlinear(gen, h, cfg.intermediate_size, cfg, False, device, res_std)
            ones = torch.ones(h, dtype=torch.bfloat16, device=device)
            layers.append(Layer(ones, ones.clone(), _concat([q, k, v]), o, _concat([gate, up]),
                                down))
        final_norm = torch.ones(h, dtype=torch.bfloat16, device=device)
        lm_head = None if cfg.tie_word_embeddings else _random_qlinear(
            gen, cfg.vocab_size, h, cfg, False, device)
        return cls(cfg, embed, layers, final_norm, lm_head)

    # ------------------------------------------------------------ pieces
    def _embed(self, ids: torch.Tensor) -> torch.Tensor:
        e = self.embed
        return core.embedding_lookup(ids.to(torch.int32), e.wq, e.scales, e.biases,
                                     e.group_size, e.bits)

    def _logits(self, h: torch.Tensor) -> torch.Tensor:
        h = rms_norm(h, self.final_norm, self.cfg.rms_norm_eps)
        if self.lm_head is None:
            e = self.embed
            return core.quantized_matmul(h, e.wq, e.scales, e.biases, True, e.group_size, e.bits)
        return self.lm_head(h)

    def _split_qkv(self, qkv: torch.Tensor):
        c = self.cfg
        d = c.head_dim
        nq, nkv = c.num_attention_heads * d, c.num_key_value_heads * d
        return qkv[..., :nq], qkv[..., nq:nq + nkv], qkv[..., nq + nkv:]

    def _mlp(self, layer: Layer, x: torch.Tensor) -> torch.Tensor:
        gu = layer.gate_up(x)
        inter = self.cfg.intermediate_size
        return layer.down(F.silu(gu[..., :inter]) * gu[..., inter:])

    # ------------------------------------------------------------ prefill
    def prefill(self, ids: torch.Tensor, cache: KVCache, all_positions: bool = False
                ) -> torch.Tensor:
        """ids [B, T] (positions 0..T-1 of every row) -> logits [B, vocab] of position T-1
        (or [B, T, vocab] with all_positions); fills cache positions 0..T-1."""
        c = self.cfg
        B, T = ids.shape
        d, nh, nkv = c.head_dim, c.num_attention_heads, c.num_key_value_heads
        cos, sin = rope_tables(c, T, ids.device)
        causal = torch.full((T, T), float("-inf"), device=ids.device).triu(1)
        h = self._embed(ids.reshape(-1)).reshape(B, T, c.hidden_size)
        for li, layer in enumerate(self.layers):
            x = rms_norm(h, layer.input_norm, c.rms_norm_eps)
            q, k, v = self._split_qkv(layer.qkv(x))
            q = apply_rope(q.float().reshape(B, T, nh, d).transpose(1, 2), cos, sin)
            k = apply_rope(k.float().reshape(B, T, nkv, d).transpose(1, 2), cos, sin)
            v = v.float().reshape(B, T, nkv, d).transpose(1, 2)
            cache.k[li][:, :, :T] = k
            cache.v[li][:, :, :T] = v
            rep = nh // nkv
            kk = k.repeat_interleave(rep, dim=1)
            vv = v.repeat_interleave(rep, dim=1)
            s = torch.matmul(q, kk.transpose(-1, -2).contiguous()) * (d ** -0.5) + causal
            a = torch.matmul(torch.softmax(s, dim=-1), vv)
            a = a.transpose(1, 2).reshape(B, T, nh * d).to(torch.bfloat16)
            h = h + layer.o(a)
            h = h + self._mlp(layer, rms_norm(h, layer.post_norm, c.rms_norm_eps))
        return self._logits(h if all_positions else h[:, -1])

    # ------------------------------------------------------------ decode
    def decode_step(self, tok: torch.Tensor, pos: torch.Tensor, cache: KVCache,
                    cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        """One token per row: tok [B] int, pos [B] int64 (its position) -> logits [B, vocab].
        Static shapes only (graph-capturable): the cache is read over max_len with a mask."""
        c = self.cfg
        B = tok.shape[0]
        d, nh, nkv = c.head_dim, c.num_attention_heads, c.num_key_value_heads
        rep = nh // nkv
        cs, sn = cos[pos][:, None, None, :], sin[pos][:, None, None, :]  # [B,1,1,D/2]
        idx = pos.view(B, 1, 1, 1).expand(B, nkv, 1, d)
        keep = (torch.arange(cache.max_len, device=tok.device)[None, :] <= pos[:, None])
        mask = torch.where(keep, 0.0, float("-inf"))[:, None, None, :]  # [B,1,1,L]
        h = self._embed(tok)
        for li, layer in enumerate(self.layers):
            x = rms_norm(h, layer.input_norm, c.rms_norm_eps)
            q, k, v = self._split_qkv(layer.qkv(x))
            q = apply_rope(q.float().reshape(B, nh, 1, d), cs, sn)
            k = apply_rope(k.float().reshape(B, nkv, 1, d), cs, sn)
            cache.k[li].scatter_(2, idx, k)
            cache.v[li].scatter_(2, idx, v.float().reshape(B, nkv, 1, d))
            qg = q.reshape(B, nkv, rep, d)
            s = torch.matmul(qg, cache.k[li].transpose(-1, -2)) * (d ** -0.5) + mask
            a = torch.matmul(torch.softmax(s, dim=-1), cache.v[li])  # [B, nkv, rep, d]
            h = h + layer.o(a.reshape(B, nh * d).to(torch.bfloat16))
            h = h + self._mlp(layer, rms_norm(h, layer.post_norm, c.rms_norm_eps))
        return self._logits(h)

    def generate(self, prompt: torch.Tensor, n_new: int, max_len: int | None = None,
                 use_graph: bool = True, logits_out: list | None = None) -> torch.Tensor:
        """Greedy decode: prompt [B, T] -> new tokens [B, n_new] (int64).  With
        logits_out, each step's logits [B, vocab] are appended to it."""
        B, T = prompt.shape
        dev = prompt.device
        max_len = max_len or (T + n_new)
        cache = KVCache(self.cfg, B, max_len, dev)
        cos, sin = rope_tables(self.cfg, max_len, dev)
        out = torch.empty(B, n_new, dtype=torch.int64, device=dev)
        logits = self.prefill(prompt, cache)
        if logits_out is not None:
            logits_out.append(logits.clone())
        out[:, 0] = logits.float().argmax(-1)
        tok = out[:, 0].clone()
        pos = torch.full((B,), T, dtype=torch.int64, device=dev)
        step = lambda: self.decode_step(tok, pos, cache, cos, sin)  # noqa: E731
        if use_graph and n_new > 1:
            g, static_logits = self._capture(step)
        for i in range(1, n_new):
            if use_graph:
                g.replay()
                logits = static_logits
            else:
                logits = step()
            if logits_out is not None:
                logits_out.append(logits.clone())
            nxt = logits.float().argmax(-1)
            out[:, i] = nxt
            tok.copy_(nxt)
            pos.add_(1)
        return out

    @staticmethod
    def _capture(step):
        """Warm up on a side stream, then capture one decode step."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            static_logits = step()
        return g, static_logits


__all__ = ["Qwen2Config", "Qwen2Model", "KVCache", "QLinear", "rms_norm", "rope_tables",
           "apply_rope"]
