"""Qwen2-shaped decoder with 4/8-bit affine-quantized linears, greedy decode.

Restates the reference's native Qwen2 graph
(python/mlx_worker/native_mlx/models/qwen2.py:47-227) on PyTorch-ROCm, with
every linear layer and the token embedding running through libmi355q:

* attention (qwen2.py:47-117): q/k/v projections with bias, non-traditional
  RoPE (theta from the config), grouped-query attention with scale
  head_dim**-0.5 and a causal mask, o_proj without bias;
* MLP (qwen2.py:118-133): down(silu(gate(x)) * up(x)), no biases;
* Qwen3 options (models/qwen3.py:47-117): explicit head_dim, no q/k/v bias,
  per-head RMSNorm of q and k before RoPE; and the reference's top-k routed
  expert MLP (models/lfm2.py:348-375, moe.MoEBlock) for Qwen3-MoE shapes;
* block (qwen2.py:136-163): pre-norm RMSNorm, residual after attention and
  after the MLP; backbone (qwen2.py:166-196): embedding, layers, final RMSNorm;
* LM head (qwen2.py:199-227): untied quantized linear (or the tied embedding's
  as_linear), greedy argmax over the last position of each row
  (executor.py:406-414).

Two equivalent rearrangements keep the weights MLX's and the arithmetic the
same: q/k/v are concatenated into one quantized matrix (and gate/up into
another) so each is one launch, which is exact because the output columns of
a quantized matmul are independent.  Activations and the paged KV cache are
bfloat16 (as in the reference, cache.py:659-695); RMSNorm, RoPE, the softmax
and every accumulation are float32.  A decode step at batch 1 is six
launches per dense layer (residual add + RMSNorm + QKV GEMV; split attention
with RoPE and the KV append inside it; the splits' combine; o GEMV; residual
add + RMSNorm + gate|up GEMV with SiLU * up in its epilogue; down GEMV; the
norms run inside the GEMVs' input staging); batched, the residual adds, the
norms and SiLU * up run in the skinny GEMMs' split-K reduces instead; captured
once in a HIP graph and replayed per token (inputs live in static device
buffers).  Prefill runs the same linears as GEMMs and the paged prefill
attention kernel over the pages (in place of the reference's dense-row gather
and masked scaled_dot_product_attention, attention.py:215-298; head dims it
does not take fall back to a float32 restatement of that), so a prompt may
start after a prefix already in the cache (prefix sharing).
Weights can be random-initialised at the reference's 7B shape
(Qwen2Config.qwen25_7b) for benchmarking.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import core
from .decode_ops import (PagedKV, argmax_rows, attention_step, paged_prefill_attention,
                         prefill_attention_supported, rope_kv_append, silu_mul)
from .moe import MoEBlock, QExperts
from .decode_ops import rms_norm as fused_rms_norm


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
    rope_scale: float = 1.0   # positions are multiplied by it (Qwen3 linear scaling)
    tie_word_embeddings: bool = False
    group_size: int = 64
    bits: int = 4
    # Qwen3 variants (models/qwen3.py:47-66): explicit head_dim, no q/k/v
    # bias, per-head RMSNorm of q and k; mixture-of-experts MLP (the
    # reference's MoE block, models/lfm2.py:348-375) when num_experts > 0.
    head_dim_: int = 0
    attention_bias: bool = True
    qk_norm: bool = False
    num_experts: int = 0
    num_experts_per_tok: int = 0
    moe_intermediate_size: int = 0
    norm_topk_prob: bool = True

    @property
    def head_dim(self) -> int:
        return self.head_dim_ or self.hidden_size // self.num_attention_heads

    @classmethod
    def qwen25_7b(cls, bits: int = 4) -> "Qwen2Config":
        """Qwen2.5-7B: 28 layers, hidden 3584, 28 Q / 4 KV heads, MLP 18944, vocab 152064."""
        return cls(hidden_size=3584, intermediate_size=18944, num_attention_heads=28,
                   num_key_value_heads=4, num_hidden_layers=28, vocab_size=152064,
                   rms_norm_eps=1e-6, rope_theta=1e6, bits=bits)

    @classmethod
    def qwen3_30b_a3b(cls, bits: int = 4) -> "Qwen2Config":
        """Qwen3-30B-A3B: 48 layers, hidden 2048, 32 Q / 4 KV heads of 128, q/k norms,
        128 experts, top 8 (renormalised), expert MLP 768, vocab 151936."""
        return cls(hidden_size=2048, intermediate_size=6144, num_attention_heads=32,
                   num_key_value_heads=4, num_hidden_layers=48, vocab_size=151936,
                   rms_norm_eps=1e-6, rope_theta=1e6, bits=bits, head_dim_=128,
                   attention_bias=False, qk_norm=True, num_experts=128,
                   num_experts_per_tok=8, moe_intermediate_size=768, norm_topk_prob=True)


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


class DenseLinear:
    """A linear layer a checkpoint stores unquantized (no `{path}.scales`):
    the reference keeps such a module an nn.Linear / nn.Embedding
    (models/qwen2.py:316-324 quantizes only paths whose scales are present), so
    it stays bfloat16 here, y = x @ weight^T (+ bias) through torch's GEMM.
    weight bfloat16 [N, K]; as the embedding, its rows are looked up."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None = None):
        if weight.dtype != torch.bfloat16 or weight.dim() != 2:
            raise ValueError("DenseLinear takes a bfloat16 [N, K] weight")
        self.weight, self.bias = weight.contiguous(), bias

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        K = x.shape[-1]
        y = F.linear(x.reshape(-1, K), self.weight, self.bias)
        return y.reshape(*x.shape[:-1], self.weight.shape[0])

    @property
    def out_features(self) -> int:
        return self.weight.shape[0]


def _random_qlinear(gen, n_out, n_in, cfg, bias, device, std=0.02) -> QLinear:
    w = (torch.randn(n_out, n_in, generator=gen, device=device) * std).to(torch.bfloat16)
    wq, s, b = core.quantize(w, cfg.group_size, cfg.bits)
    del w
    bv = ((torch.randn(n_out, generator=gen, device=device) * std).to(torch.bfloat16)
          if bias else None)
    return QLinear(wq, s, b, bv, cfg.group_size, cfg.bits)


def _gate_up_silu(gate_up, x: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up of the fused gate|up projection: one kernel at decode
    shapes (the same bits as the two-kernel path), else the two kernels."""
    K = x.shape[-1]
    if (isinstance(gate_up, QLinear) and gate_up.bias is None
            and core.swiglu_supported(x.numel() // K, gate_up.out_features // 2, K,
                                      gate_up.group_size, gate_up.bits)):
        return core.quantized_matmul_swiglu(x, gate_up.wq, gate_up.scales, gate_up.biases,
                                            gate_up.group_size, gate_up.bits)
    return silu_mul(gate_up(x))


def _concat(parts: list):
    """Row-wise concatenation: one launch computes every part's columns."""
    bias = None
    if parts[0].bias is not None:
        bias = torch.cat([p.bias for p in parts])
    if all(isinstance(p, DenseLinear) for p in parts):
        return DenseLinear(torch.cat([p.weight for p in parts]), bias)
    if not all(isinstance(p, QLinear) for p in parts):
        raise NotImplementedError("a quantized and an unquantized projection cannot be fused")
    return QLinear(torch.cat([p.wq for p in parts]), torch.cat([p.scales for p in parts]),
                   torch.cat([p.biases for p in parts]), bias, parts[0].group_size,
                   parts[0].bits)


@dataclass
class Layer:
    input_norm: torch.Tensor   # bfloat16 [hidden]
    post_norm: torch.Tensor    # bfloat16 [hidden]
    qkv: QLinear               # [(heads + 2 kv_heads) * head_dim, hidden] (+ bias in Qwen2)
    o: QLinear                 # [hidden, heads * head_dim]
    gate_up: QLinear | None = None   # [2 * intermediate, hidden] (dense MLP)
    down: QLinear | None = None      # [hidden, intermediate]
    q_norm: torch.Tensor | None = None   # bfloat16 [head_dim] (Qwen3)
    k_norm: torch.Tensor | None = None
    moe: MoEBlock | None = None          # replaces gate_up / down


def _random_experts(gen, E, n_out, n_in, cfg, device, std=0.02) -> QExperts:
    """E experts of [n_out, n_in], N(0, std), quantized per expert row."""
    w = (torch.randn(E * n_out, n_in, generator=gen, device=device) * std).to(torch.bfloat16)
    wq, s, b = core.quantize(w, cfg.group_size, cfg.bits)
    del w
    return QExperts(wq.reshape(E, n_out, -1), s.reshape(E, n_out, -1), b.reshape(E, n_out, -1),
                    cfg.group_size, cfg.bits)


def greedy_tokens(logits: torch.Tensor) -> torch.Tensor:
    """The next tokens of greedy decoding (executor.py:406-414): the first index
    of each row's largest logit, int64 [...] -- the library's row argmax over the
    bfloat16 logits (torch.argmax's result on the same values) where the
    vocabulary is whole 8-element units."""
    if logits.dtype == torch.bfloat16 and logits.shape[-1] % 8 == 0:
        return argmax_rows(logits)
    return logits.float().argmax(-1)


def rope_tables(cfg: Qwen2Config, max_len: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [max_len, head_dim/2] of mx.fast.rope (traditional=False, base=theta,
    scale): row p, column i holds cos/sin(p * scale * theta^(-2i/head_dim))."""
    half = cfg.head_dim // 2
    inv = cfg.rope_theta ** (-torch.arange(0, half, dtype=torch.float64, device=device) / half)
    pos = torch.arange(max_len, dtype=torch.float64, device=device) * cfg.rope_scale
    ang = pos[:, None] * inv[None, :]
    return torch.cos(ang).float(), torch.sin(ang).float()


def _rope_append_tokens(qkv: torch.Tensor, positions: torch.Tensor, cache: PagedKV, layer: int,
                        cos: torch.Tensor, sin: torch.Tensor, n_heads: int, lyr, eps: float,
                        table: torch.Tensor, step: int = 32768) -> torch.Tensor:
    """rope_kv_append over a prefill chunk's tokens (one row each, with its row's
    page table), at most `step` tokens a call -> q bf16 [tokens, n_heads, head_dim]."""
    n = qkv.shape[0]
    parts = [rope_kv_append(qkv[a:a + step], positions[a:a + step], cache, layer, cos, sin,
                            n_heads, lyr.q_norm, lyr.k_norm, eps, table=table[a:a + step])
             for a in range(0, n, step)]
    return parts[0] if len(parts) == 1 else torch.cat(parts)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Non-traditional RoPE on the last dim: halves (x1, x2) rotate together.
    x [..., T, D] float32; cos/sin broadcastable to [..., T, D/2]."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)


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
        bias = cfg.attention_bias
        layers = []
        for _ in range(cfg.num_hidden_layers):
            q = _random_qlinear(gen, cfg.num_attention_heads * d, h, cfg, bias, device)
            k = _random_qlinear(gen, cfg.num_key_value_heads * d, h, cfg, bias, device)
            v = _random_qlinear(gen, cfg.num_key_value_heads * d, h, cfg, bias, device)
            o = _random_qlinear(gen, h, cfg.num_attention_heads * d, cfg, False, device,
                                res_std)
            ones = torch.ones(h, dtype=torch.bfloat16, device=device)
            layer = Layer(ones, ones.clone(), _concat([q, k, v]), o)
            if cfg.qk_norm:  # non-trivial norm weights, so the tests exercise them
                layer.q_norm, layer.k_norm = (
                    (1 + 0.1 * torch.randn(d, generator=gen, device=device)).to(torch.bfloat16)
                    for _ in range(2))
            if cfg.num_experts:
                E, inter = cfg.num_experts, cfg.moe_intermediate_size
                router = _random_qlinear(gen, E, h, cfg, False, device)
                gate_up = _random_experts(gen, E, 2 * inter, h, cfg, device)  # gate | up rows
                down = _random_experts(gen, E, h, inter, cfg, device, res_std)
                layer.moe = MoEBlock(router, gate_up, down, cfg.num_experts_per_tok,
                                     cfg.norm_topk_prob)
            else:
                gate = _random_qlinear(gen, cfg.intermediate_size, h, cfg, False, device)
                up = _random_qlinear(gen, cfg.intermediate_size, h, cfg, False, device)
                layer.gate_up = _concat([gate, up])
                layer.down = _random_qlinear(gen, h, cfg.intermediate_size, cfg, False, device,
                                             res_std)
            layers.append(layer)
        final_norm = torch.ones(h, dtype=torch.bfloat16, device=device)
        lm_head = None if cfg.tie_word_embeddings else _random_qlinear(
            gen, cfg.vocab_size, h, cfg, False, device)
        return cls(cfg, embed, layers, final_norm, lm_head)

    # ------------------------------------------------------------ pieces
    def new_cache(self, batch: int, max_len: int, prefix_len: int = 0,
                  page_size: int = 16) -> PagedKV:
        """Paged KV for `batch` sequences of up to max_len positions.  With
        prefix_len > 0 (a multiple of page_size) every sequence's first
        prefix_len positions map to the same pages: a shared prompt prefix that
        is prefilled once (the reference's prefix-cache hit, prefix_cache.py:364)."""
        c = self.cfg
        dev = self.final_norm.device
        per = -(-max_len // page_size)
        if prefix_len % page_size or prefix_len > max_len:
            raise ValueError(f"prefix_len {prefix_len} must be a multiple of page_size "
                             f"{page_size} and at most max_len {max_len}")
        shared = prefix_len // page_size
        own = per - shared
        table = torch.empty(batch, per, dtype=torch.int32)
        table[:, :shared] = torch.arange(shared, dtype=torch.int32)
        table[:, shared:] = shared + torch.arange(batch * own, dtype=torch.int32).reshape(batch, own)
        return PagedKV(c.num_hidden_layers, shared + batch * own, page_size,
                       c.num_key_value_heads, c.head_dim, table, dev)

    def _embed(self, ids: torch.Tensor) -> torch.Tensor:
        e = self.embed
        if isinstance(e, DenseLinear):  # an unquantized nn.Embedding
            return e.weight.index_select(0, ids.reshape(-1).long()).reshape(
                *ids.shape, e.weight.shape[1])
        return core.embedding_lookup(ids.to(torch.int32), e.wq, e.scales, e.biases,
                                     e.group_size, e.bits)

    def _head(self, x: torch.Tensor) -> torch.Tensor:
        """LM head on final-normed activations (untied, or the tied embedding's as_linear)."""
        return self._head_linear()(x)

    def _head_linear(self):
        """The LM head as a linear (untied, or the tied embedding's as_linear)."""
        if self.lm_head is not None:
            return self.lm_head
        e = self.embed
        if isinstance(e, DenseLinear):
            return DenseLinear(e.weight)
        return QLinear(e.wq, e.scales, e.biases, None, e.group_size, e.bits)

    def _norm_linear(self, ql: QLinear, a: torch.Tensor, res: torch.Tensor | None,
                     norm_w: torch.Tensor, swiglu: bool = False):
        """ql on rms_norm(a (+ res)) * norm_w -- with silu(gate) * up when swiglu
        -- -> (y, h), h the residual stream after the add (a without res).  One
        kernel for a single row where the shape allows; the same bits either way
        up to the GEMV kernel the unfused path picks."""
        eps = self.cfg.rms_norm_eps
        K = a.shape[-1]
        n_out = ql.out_features // 2 if swiglu else ql.out_features
        if (isinstance(ql, QLinear) and a.numel() == K and not (swiglu and ql.bias is not None)
                and core.rms_norm_qmm_supported(1, n_out, K, ql.group_size, ql.bits, swiglu)):
            return core.rms_norm_quantized_matmul(a, norm_w, eps, ql.wq, ql.scales, ql.biases,
                                                  ql.bias, res, ql.group_size, ql.bits, swiglu)
        if res is None:
            x, h = fused_rms_norm(a, norm_w, eps), a
        else:
            x, h = fused_rms_norm(a, norm_w, eps, residual=res)
        return (_gate_up_silu(ql, x) if swiglu else ql(x)), h

    def _linear_add_norm(self, ql: QLinear, inp: torch.Tensor, h: torch.Tensor,
                         norm_w: torch.Tensor):
        """ql(inp), its residual add and the RMSNorm after it -> (x, h): x the next
        linear's normed input, h the residual stream.  One GEMM plus its reduce
        where the skinny GEMM splits K (batched decode), else the two ops; the
        same bits either way."""
        eps = self.cfg.rms_norm_eps
        K = inp.shape[-1]
        if isinstance(ql, QLinear) and core.add_norm_supported(inp.numel() // K, ql.out_features,
                                                               K, ql.group_size, ql.bits):
            return core.quantized_matmul_add_rms_norm(inp, ql.wq, ql.scales, ql.biases, h, norm_w,
                                                      eps, ql.bias, ql.group_size, ql.bits)
        return fused_rms_norm(ql(inp), norm_w, eps, residual=h)

    def _next_norm(self, li: int) -> torch.Tensor:
        return (self.layers[li + 1].input_norm if li + 1 < len(self.layers)
                else self.final_norm)

    def _ffn(self, li: int, h: torch.Tensor, o: torch.Tensor):
        """Second half of layer li after its o_proj output o: returns (x, h) where
        h is the updated residual stream and x the next layer's normed input
        (the final norm after the last layer)."""
        layer, eps = self.layers[li], self.cfg.rms_norm_eps
        x, h = fused_rms_norm(o, layer.post_norm, eps, residual=h)
        if layer.moe is not None:
            return layer.moe.residual_norm(x, h, self._next_norm(li), eps)
        return self._linear_add_norm(layer.down, _gate_up_silu(layer.gate_up, x), h,
                                     self._next_norm(li))

    # ------------------------------------------------------------ prefill
    def prefill(self, ids: torch.Tensor, cache: PagedKV, start: int | torch.Tensor = 0,
                rows: torch.Tensor | None = None, all_positions: bool = False,
                lengths: torch.Tensor | None = None) -> torch.Tensor:
        """ids [B, T] at positions start..start+T-1 of cache rows `rows` (default
        0..B-1), attending to the cached positions 0..start-1 as well ->
        logits [B, vocab] of the last position (or [B, T, vocab] with all_positions);
        writes K/V of the new positions into the pages.

        Ragged batches (the reference's step layout, executor.py:335-346): start
        may be int64 [B] (each row's cached length) and lengths int64 [B] (each
        row's new tokens, 1..T).  Row b's tokens past lengths[b] are padding: they
        sit at the row's last position (as the reference repeats it), are neither
        written to the pages nor attended to by other tokens, and the logits
        returned are those of each row's last valid token (executor.py:406-414).
        A row with one new token on top of its cache is a decode row, so one call
        also serves a mixed prefill/decode step."""
        if not isinstance(start, int) or lengths is not None:
            return self._prefill_ragged(ids, cache, start, rows, all_positions, lengths)
        c = self.cfg
        B, T = ids.shape
        dev = ids.device
        d, nh, nkv = c.head_dim, c.num_attention_heads, c.num_key_value_heads
        rep = nh // nkv
        S = start + T
        rows = torch.arange(B, device=dev) if rows is None else rows.to(dev).long()
        pos = torch.arange(start, S, device=dev)
        # query i (position start + i) sees keys 0..start + i: RoPE + append and
        # the paged prefill kernel, or (shapes it does not take) a float32
        # restatement
        native = prefill_attention_supported(nh, cache)
        if native:
            cos, sin = rope_tables(c, cache.capacity, dev)
            table = cache.page_table[rows].contiguous()
            tok_table = table.repeat_interleave(T, 0)   # token (b, i): row b's table
            tok_pos = pos.repeat(B)
            starts = torch.full((B,), start, dtype=torch.int64, device=dev)
            lens = torch.full((B,), T, dtype=torch.int64, device=dev)
        else:
            cos, sin = rope_tables(c, S, dev)
            cs, sn = cos[start:], sin[start:]
            slots = cache.slots(rows.repeat_interleave(T), pos.repeat(B))
            causal = torch.full((T, S), float("-inf"), device=dev).triu(start + 1)
        h = self._embed(ids.reshape(-1)).reshape(B, T, c.hidden_size)
        x = fused_rms_norm(h, self.layers[0].input_norm, c.rms_norm_eps)
        for li, layer in enumerate(self.layers):
            qkv = layer.qkv(x)
            if native:
                q = _rope_append_tokens(qkv.reshape(B * T, -1), tok_pos, cache, li, cos, sin, nh,
                                        layer, c.rms_norm_eps, tok_table)
                a = paged_prefill_attention(q.reshape(B, T, nh, d), cache, li, table, starts, lens,
                                            d ** -0.5)
            else:
                q, k, v = (qkv[..., :nh * d], qkv[..., nh * d:(nh + nkv) * d],
                           qkv[..., (nh + nkv) * d:])
                q, k = q.reshape(B, T, nh, d), k.reshape(B, T, nkv, d)
                if layer.q_norm is not None:  # Qwen3: per-head RMSNorm before RoPE
                    q = fused_rms_norm(q, layer.q_norm, c.rms_norm_eps)
                    k = fused_rms_norm(k, layer.k_norm, c.rms_norm_eps)
                q = apply_rope(q.float().transpose(1, 2), cs, sn)
                k = apply_rope(k.float().transpose(1, 2), cs, sn)
                k = k.to(torch.bfloat16)
                v = v.reshape(B, T, nkv, d).transpose(1, 2)
                cache.write(li, slots, k.transpose(1, 2).reshape(B * T, nkv, d),
                            v.transpose(1, 2).reshape(B * T, nkv, d))
                if start:
                    k, v = cache.gather_rows(li, rows, S)
                q = q.to(torch.bfloat16).float()
                kk = k.float().repeat_interleave(rep, dim=1)
                vv = v.float().repeat_interleave(rep, dim=1)
                s = torch.matmul(q, kk.transpose(-1, -2).contiguous()) * (d ** -0.5) + causal
                a = torch.matmul(torch.softmax(s, dim=-1), vv).transpose(1, 2).reshape(
                    B, T, nh * d).to(torch.bfloat16)
            o = layer.o(a)
            x, h = self._ffn(li, h, o)
        return self._head(x if all_positions else x[:, -1])

    def _prefill_ragged(self, ids, cache, start, rows, all_positions, lengths):
        c = self.cfg
        B, T = ids.shape
        dev = ids.device
        d, nh, nkv = c.head_dim, c.num_attention_heads, c.num_key_value_heads
        rep = nh // nkv
        rows = torch.arange(B, device=dev) if rows is None else rows.to(dev).long()
        starts = (torch.full((B,), start, dtype=torch.long) if isinstance(start, int)
                  else torch.as_tensor(start)).to(dev).long().reshape(B)
        lens = (torch.full((B,), T, dtype=torch.long) if lengths is None
                else torch.as_tensor(lengths)).to(dev).long().reshape(B)
        if bool(((lens < 1) | (lens > T) | (starts < 0)).any()):
            raise ValueError(f"lengths must lie in 1..{T} and starts be >= 0")
        S = int((starts + lens).max())
        if S > cache.capacity:
            raise ValueError(f"positions up to {S} exceed the cache capacity {cache.capacity}")
        j = torch.arange(T, device=dev)
        valid = j[None, :] < lens[:, None]                                  # [B, T]
        pos = starts[:, None] + torch.minimum(j[None, :], lens[:, None] - 1)  # [B, T]
        vb, vj = valid.nonzero(as_tuple=True)
        # query (b, j) sees the keys of its row at positions <= pos[b, j]; a
        # padding query repeats the row's last valid one.  Natively only the
        # valid tokens are roped and appended, padding queries are zero (their
        # outputs mean nothing either way)
        native = prefill_attention_supported(nh, cache)
        if native:
            cos, sin = rope_tables(c, cache.capacity, dev)
            table = cache.page_table[rows].contiguous()
            tok_table = table[vb].contiguous()
            tok_pos = pos[vb, vj].contiguous()
        else:
            slots = cache.slots(rows[vb], pos[vb, vj])
            cos, sin = rope_tables(c, S, dev)
            cs, sn = cos[pos][:, None], sin[pos][:, None]                   # [B, 1, T, d/2]
            keyp = torch.arange(S, device=dev)
            mask = torch.zeros(B, 1, T, S, device=dev).masked_fill_(
                (keyp[None, None, :] > pos[:, :, None])[:, None], float("-inf"))
        h = self._embed(ids.reshape(-1)).reshape(B, T, c.hidden_size)
        x = fused_rms_norm(h, self.layers[0].input_norm, c.rms_norm_eps)
        for li, layer in enumerate(self.layers):
            qkv = layer.qkv(x)
            if native:
                qv = _rope_append_tokens(qkv[vb, vj].contiguous(), tok_pos, cache, li, cos, sin,
                                         nh, layer, c.rms_norm_eps, tok_table)
                q = torch.zeros(B, T, nh, d, dtype=torch.bfloat16, device=dev)
                q[vb, vj] = qv
                a = paged_prefill_attention(q, cache, li, table, starts, lens, d ** -0.5)
            else:
                q, k, v = (qkv[..., :nh * d], qkv[..., nh * d:(nh + nkv) * d],
                           qkv[..., (nh + nkv) * d:])
                q, k = q.reshape(B, T, nh, d), k.reshape(B, T, nkv, d)
                if layer.q_norm is not None:  # Qwen3: per-head RMSNorm before RoPE
                    q = fused_rms_norm(q, layer.q_norm, c.rms_norm_eps)
                    k = fused_rms_norm(k, layer.k_norm, c.rms_norm_eps)
                q = apply_rope(q.float().transpose(1, 2), cs, sn)
                k = apply_rope(k.float().transpose(1, 2), cs, sn).to(torch.bfloat16)
                v = v.reshape(B, T, nkv, d)
                cache.write(li, slots, k.transpose(1, 2)[vb, vj], v[vb, vj])
                kk, vv = cache.gather_rows(li, rows, S)
                q = q.to(torch.bfloat16).float()
                kk = kk.float().repeat_interleave(rep, dim=1)
                vv = vv.float().repeat_interleave(rep, dim=1)
                s = torch.matmul(q, kk.transpose(-1, -2).contiguous()) * (d ** -0.5) + mask
                a = torch.matmul(torch.softmax(s, dim=-1), vv).transpose(1, 2).reshape(
                    B, T, nh * d).to(torch.bfloat16)
            o = layer.o(a)
            x, h = self._ffn(li, h, o)
        if all_positions:
            return self._head(x)
        return self._head(x[torch.arange(B, device=dev), lens - 1])

    # ------------------------------------------------------------ decode
    def decode_step(self, tok: torch.Tensor, pos: torch.Tensor, cache: PagedKV,
                    cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        """One token per sequence: tok [B] int, pos [B] int64 (its position, on the
        device) -> logits [B, vocab].  Static shapes only, so it can be captured."""
        c = self.cfg
        d, nh, eps = c.head_dim, c.num_attention_heads, c.rms_norm_eps
        h = self._embed(tok)
        if tok.numel() > 1:  # batched: the norms ride on the GEMMs' split-K reduces
            x = fused_rms_norm(h, self.layers[0].input_norm, eps)
            for li, layer in enumerate(self.layers):
                a = attention_step(layer.qkv(x), pos, cache, li, cos, sin, nh, d ** -0.5,
                                   layer.q_norm, layer.k_norm, eps)
                x, h = self._linear_add_norm(layer.o, a, h, layer.post_norm)
                if layer.moe is not None:
                    x, h = layer.moe.residual_norm(x, h, self._next_norm(li), eps)
                else:
                    x, h = self._linear_add_norm(layer.down, _gate_up_silu(layer.gate_up, x), h,
                                                 self._next_norm(li))
            return self._head(x)
        # One row: the next linear's input is rms_norm(src[0] (+ src[1])) *
        # that layer's norm weight, computed inside the linear's kernel; or x,
        # when an MoE block has already normalised it.
        src, x = (h, None), None
        for li, layer in enumerate(self.layers):
            if x is None:
                qkv, h = self._norm_linear(layer.qkv, *src, layer.input_norm)
            else:
                qkv = layer.qkv(x)
            a = attention_step(qkv, pos, cache, li, cos, sin, nh, d ** -0.5,
                               layer.q_norm, layer.k_norm, eps)
            o = layer.o(a)
            if layer.moe is not None:
                xm, h = fused_rms_norm(o, layer.post_norm, eps, residual=h)
                x, h = layer.moe.residual_norm(xm, h, self._next_norm(li), eps)
            else:
                act, h = self._norm_linear(layer.gate_up, o, h, layer.post_norm, swiglu=True)
                src, x = (layer.down(act), h), None
        if x is None:
            return self._norm_linear(self._head_linear(), *src, self.final_norm)[0]
        return self._head(x)

    def generate(self, prompt: torch.Tensor, n_new: int, max_len: int | None = None,
                 use_graph: bool = True, logits_out: list | None = None,
                 prefix_len: int = 0, page_size: int = 16,
                 lengths: torch.Tensor | None = None) -> torch.Tensor:
        """Greedy decode: prompt [B, T] -> new tokens [B, n_new] (int64).  With
        logits_out, each step's logits [B, vocab] are appended to it.  With
        prefix_len > 0 the rows' first prefix_len prompt tokens are equal (the
        caller's promise): they are prefilled once, from row 0, into pages every
        row shares, and each row prefills only its own suffix.  With lengths
        (int64 [B], prefix_len < lengths[b] <= T) row b's prompt is its first
        lengths[b] tokens (the rest padding); its first new token follows its
        last prompt token and its decode steps continue from there."""
        B, T = prompt.shape
        dev = prompt.device
        max_len = max_len or (T + n_new)
        cache = self.new_cache(B, max_len, prefix_len, page_size)
        cos, sin = rope_tables(self.cfg, cache.capacity, dev)
        out = torch.empty(B, n_new, dtype=torch.int64, device=dev)
        if prefix_len:
            self.prefill(prompt[:1, :prefix_len], cache, rows=torch.zeros(1, dtype=torch.long))
        if lengths is None:
            logits = self.prefill(prompt[:, prefix_len:], cache, start=prefix_len)
            pos = torch.full((B,), T, dtype=torch.int64, device=dev)
        else:
            lens = torch.as_tensor(lengths).to(dev).long().reshape(B)
            if bool(((lens <= prefix_len) | (lens > T)).any()):
                raise ValueError(f"lengths must lie in {prefix_len + 1}..{T}")
            logits = self.prefill(prompt[:, prefix_len:], cache, start=prefix_len,
                                  lengths=lens - prefix_len)
            pos = lens.clone()
        if logits_out is not None:
            logits_out.append(logits.clone())
        out[:, 0] = greedy_tokens(logits)
        tok = out[:, 0].clone()
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
            nxt = greedy_tokens(logits)
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


__all__ = ["Qwen2Config", "Qwen2Model", "QLinear", "DenseLinear", "rope_tables", "apply_rope"]
