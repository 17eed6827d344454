"""Decoder-step ops around the quantized linears, executed by libmi355q.

The reference's Qwen2 graph (python/mlx_worker/native_mlx/models/qwen2.py)
calls these per layer and token:

    rms_norm(x, weight, eps, residual=None)        nn.RMSNorm (qwen2.py:140-145),
                                                   fused with the residual add
                                                   before it (qwen2.py:158-163)
    rope_kv_append(qkv, positions, cache, layer, cos, sin, n_heads)
                                                   mx.fast.rope on q and k
                                                   (qwen2.py:93-108) + the paged
                                                   append (cache.py:485-520)
    paged_decode_attention(q, cache, layer, positions, scale)
                                                   attention over the pages
                                                   (attention.py:206-298)
    attention_step(qkv, positions, cache, layer, cos, sin, n_heads, scale, ...)
                                                   the two above with RoPE + append
                                                   inside the attention kernel
    silu_mul(gate_up)                              silu(gate) * up (qwen2.py:43-44)

PagedKV holds the pages in the reference's layout (cache.py:686-695): per
layer bfloat16 [num_pages, page_size, kv_heads, head_dim], plus an int32 page
table [batch, pages_per_seq] (cache.py:459-471).  There is no CPU fallback.
"""

from __future__ import annotations

import torch

from . import _lib
from .core import _check_bf16, _ptr, _require_gpu, _stream


class PagedKV:
    """Paged bfloat16 KV cache of every layer plus the sequences' page table.

    ``page_table[b, j]`` is the page holding positions [j*page_size,
    (j+1)*page_size) of sequence b; pages may be shared between sequences (a
    common prompt prefix) as long as shared pages are only read.
    """

    def __init__(self, num_layers: int, num_pages: int, page_size: int, kv_heads: int,
                 head_dim: int, page_table: torch.Tensor, device):
        shape = (num_pages, page_size, kv_heads, head_dim)
        self.k = [torch.zeros(shape, dtype=torch.bfloat16, device=device)
                  for _ in range(num_layers)]
        self.v = [torch.zeros(shape, dtype=torch.bfloat16, device=device)
                  for _ in range(num_layers)]
        self.page_table = page_table.to(device=device, dtype=torch.int32).contiguous()
        self.num_pages, self.page_size = num_pages, page_size
        self.kv_heads, self.head_dim = kv_heads, head_dim
        if self.page_table.ndim != 2:
            raise ValueError("page_table must be [batch, pages_per_seq]")

    @classmethod
    def contiguous(cls, num_layers: int, batch: int, max_len: int, kv_heads: int,
                   head_dim: int, device, page_size: int = 16) -> "PagedKV":
        """Each sequence owns ceil(max_len / page_size) consecutive pages."""
        per = -(-max_len // page_size)
        table = torch.arange(batch * per, dtype=torch.int32).reshape(batch, per)
        return cls(num_layers, batch * per, page_size, kv_heads, head_dim, table, device)

    @property
    def batch(self) -> int:
        return self.page_table.shape[0]

    @property
    def pages_per_seq(self) -> int:
        return self.page_table.shape[1]

    @property
    def capacity(self) -> int:
        return self.pages_per_seq * self.page_size

    def slots(self, rows: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """Flat slot of (row, position): page * page_size + position % page_size."""
        pages = self.page_table[rows, positions // self.page_size].long()
        return pages * self.page_size + positions % self.page_size

    def write(self, layer: int, slots: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v [n, kv_heads, head_dim] into flat slots [n] (from slots())."""
        rows = (-1, self.kv_heads, self.head_dim)
        self.k[layer].view(rows).index_copy_(0, slots, k.to(torch.bfloat16))
        self.v[layer].view(rows).index_copy_(0, slots, v.to(torch.bfloat16))

    def gather_rows(self, layer: int, rows: torch.Tensor, length: int
                    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Dense k, v [len(rows), kv_heads, length, head_dim] of positions 0..length-1
        (the reference's _dense_kv_rows, attention.py:264-298)."""
        n = -(-length // self.page_size)
        pages = self.page_table[rows, :n].long()                 # [R, n]
        shape = (pages.shape[0], n * self.page_size, self.kv_heads, self.head_dim)
        k = self.k[layer][pages].reshape(shape)[:, :length]
        v = self.v[layer][pages].reshape(shape)[:, :length]
        return k.transpose(1, 2), v.transpose(1, 2)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float,
             residual: torch.Tensor | None = None):
    """out = bf16(h * rsqrt(mean(h^2) + eps) * weight), h = x, or h = bf16(x + residual).

    Returns out, or (out, h) when residual is given.
    """
    op = "rms_norm"
    _require_gpu(op, x=x, weight=weight, residual=residual)
    _check_bf16(op, "x", x)
    _check_bf16(op, "weight", weight)
    dim = x.shape[-1]
    if weight.shape != (dim,):
        raise ValueError(f"[{op}] weight must have shape ({dim},), got {tuple(weight.shape)}")
    xc = x.contiguous()
    out = torch.empty_like(xc)
    h = None
    if residual is not None:
        _check_bf16(op, "residual", residual)
        if residual.shape != x.shape:
            raise ValueError(f"[{op}] residual shape {tuple(residual.shape)} != {tuple(x.shape)}")
        residual = residual.contiguous()
        h = torch.empty_like(xc)
    L = _lib.lib()
    _lib.check(L.mq_rms_norm(_ptr(xc), _ptr(residual), _ptr(h), _ptr(weight.contiguous()),
                             _ptr(out), xc.numel() // dim, dim, float(eps), _stream(x)), op)
    return out if h is None else (out, h)


def rope_kv_append(qkv: torch.Tensor, positions: torch.Tensor, cache: PagedKV, layer: int,
                   cos: torch.Tensor, sin: torch.Tensor, n_heads: int,
                   q_norm: torch.Tensor | None = None, k_norm: torch.Tensor | None = None,
                   norm_eps: float = 1e-6, table: torch.Tensor | None = None) -> torch.Tensor:
    """qkv bf16 [B, (n_heads + 2 kv_heads) * head_dim] of one token per sequence ->
    q bf16 [B, n_heads, head_dim] after RoPE; rope(k) and v go into the pages at
    each sequence's position (positions int64 [B], on the device).  q_norm /
    k_norm (bf16 [head_dim]): Qwen3's per-head RMSNorm before RoPE.  table (int32
    [B, pages_per_seq], default the cache's own): each token's page-table row --
    a prefill chunk's tokens, one entry per token, each with its row's table."""
    op = "rope_kv_append"
    _require_gpu(op, qkv=qkv, positions=positions, cos=cos, sin=sin)
    _check_bf16(op, "qkv", qkv)
    B = qkv.shape[0]
    d, nkv = cache.head_dim, cache.kv_heads
    if qkv.shape != (B, (n_heads + 2 * nkv) * d):
        raise ValueError(f"[{op}] qkv must be [B, {(n_heads + 2 * nkv) * d}], "
                         f"got {tuple(qkv.shape)}")
    if positions.dtype != torch.int64 or positions.shape != (B,):
        raise ValueError(f"[{op}] positions must be int64 [{B}]")
    if table is None:
        if cache.batch != B:
            raise ValueError(f"[{op}] the page table has {cache.batch} rows, qkv {B}")
        table = cache.page_table
    elif table.dtype != torch.int32 or table.shape != (B, cache.pages_per_seq):
        raise ValueError(f"[{op}] table must be int32 [{B}, {cache.pages_per_seq}], "
                         f"got {tuple(table.shape)}")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape[-1] != d // 2:
        raise ValueError(f"[{op}] cos/sin must be float32 [positions, {d // 2}]")
    if cos.shape[0] < cache.capacity or sin.shape != cos.shape:
        raise ValueError(f"[{op}] cos/sin need {cache.capacity} positions")
    for name, w in (("q_norm", q_norm), ("k_norm", k_norm)):
        if w is not None and (w.dtype != torch.bfloat16 or w.shape != (d,)):
            raise ValueError(f"[{op}] {name} must be bfloat16 [{d}]")
    q = torch.empty(B, n_heads, d, dtype=torch.bfloat16, device=qkv.device)
    L = _lib.lib()
    _lib.check(L.mq_rope_kv_append(
        _ptr(qkv.contiguous()), _ptr(positions), _ptr(table.contiguous()), cache.pages_per_seq,
        cache.page_size, cache.num_pages, _ptr(cos.contiguous()), _ptr(sin.contiguous()),
        _ptr(q_norm), _ptr(k_norm), float(norm_eps), _ptr(q), _ptr(cache.k[layer]),
        _ptr(cache.v[layer]), B, n_heads, nkv, d, _stream(qkv)), op)
    return q


def paged_decode_attention(q: torch.Tensor, cache: PagedKV, layer: int, positions: torch.Tensor,
                           scale: float) -> torch.Tensor:
    """q bf16 [B, n_heads, head_dim] (one token per sequence at positions[b]) ->
    bf16 [B, n_heads * head_dim]: softmax(q k^T * scale) v over positions 0..positions[b]."""
    op = "paged_decode_attention"
    _require_gpu(op, q=q, positions=positions)
    _check_bf16(op, "q", q)
    B, nh, d = q.shape
    if d != cache.head_dim or cache.batch != B:
        raise ValueError(f"[{op}] q {tuple(q.shape)} does not match the cache")
    if positions.dtype != torch.int64 or positions.shape != (B,):
        raise ValueError(f"[{op}] positions must be int64 [{B}]")
    L = _lib.lib()
    ws_bytes = L.mq_paged_decode_attention_workspace(B, nh, cache.kv_heads, d,
                                                     cache.pages_per_seq, cache.page_size)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    out = torch.empty(B, nh * d, dtype=torch.bfloat16, device=q.device)
    _lib.check(L.mq_paged_decode_attention(
        _ptr(q.contiguous()), _ptr(cache.k[layer]), _ptr(cache.v[layer]), _ptr(cache.page_table),
        cache.pages_per_seq, cache.page_size, cache.num_pages, _ptr(positions), B, nh,
        cache.kv_heads, d, float(scale), _ptr(ws), ws_bytes, _ptr(out), _stream(q)), op)
    return out


def prefill_attention_supported(n_heads: int, cache: PagedKV) -> bool:
    """Whether paged_prefill_attention takes this cache's shape."""
    return bool(_lib.lib().mq_paged_prefill_attention_supported(
        n_heads, cache.kv_heads, cache.head_dim, cache.num_pages, cache.page_size))


def argmax_rows(x: torch.Tensor) -> torch.Tensor:
    """Greedy next tokens: x bf16 [..., C] (C % 8 == 0) -> int64 [...], the first
    index of each row's largest value (NaN as the largest), as torch.argmax(-1)
    of the same values."""
    op = "argmax_rows"
    _require_gpu(op, x=x)
    _check_bf16(op, "x", x)
    C = x.shape[-1]
    x2 = x.contiguous().reshape(-1, C)
    out = torch.empty(x2.shape[0], dtype=torch.int64, device=x.device)
    _lib.check(_lib.lib().mq_argmax_rows(_ptr(x2), x2.shape[0], C, _ptr(out), _stream(x)), op)
    return out.reshape(x.shape[:-1])


def paged_prefill_attention(q: torch.Tensor, cache: PagedKV, layer: int, table: torch.Tensor,
                            starts: torch.Tensor, lens: torch.Tensor, scale: float) -> torch.Tensor:
    """Causal attention of a prefill chunk whose k and v are already in the pages
    (attention.py:215-261 gathers the pages and runs scaled_dot_product_attention
    under _dense_causal_mask, :404-425).  q bf16 [B, T, n_heads, head_dim] (roped);
    table int32 [B, pages_per_seq] (the rows' page tables); starts, lens int64 [B]:
    query j of row b sits at position starts[b] + min(j, lens[b] - 1) and attends to
    positions 0..that -> bf16 [B, T, n_heads * head_dim]."""
    op = "paged_prefill_attention"
    _require_gpu(op, q=q, table=table, starts=starts, lens=lens)
    _check_bf16(op, "q", q)
    B, T, nh, d = q.shape
    if d != cache.head_dim:
        raise ValueError(f"[{op}] q {tuple(q.shape)} does not match the cache")
    if table.dtype != torch.int32 or table.shape != (B, cache.pages_per_seq):
        raise ValueError(f"[{op}] table must be int32 [{B}, {cache.pages_per_seq}]")
    for name, t in (("starts", starts), ("lens", lens)):
        if t.dtype != torch.int64 or t.shape != (B,):
            raise ValueError(f"[{op}] {name} must be int64 [{B}]")
    out = torch.empty(B, T, nh * d, dtype=torch.bfloat16, device=q.device)
    L = _lib.lib()
    _lib.check(L.mq_paged_prefill_attention(
        _ptr(q.contiguous()), _ptr(cache.k[layer]), _ptr(cache.v[layer]), _ptr(table.contiguous()),
        cache.pages_per_seq, cache.page_size, cache.num_pages, _ptr(starts.contiguous()),
        _ptr(lens.contiguous()), B, T, nh, cache.kv_heads, d, float(scale), _ptr(out),
        _stream(q)), op)
    return out


def attention_step(qkv: torch.Tensor, positions: torch.Tensor, cache: PagedKV, layer: int,
                   cos: torch.Tensor, sin: torch.Tensor, n_heads: int, scale: float,
                   q_norm: torch.Tensor | None = None, k_norm: torch.Tensor | None = None,
                   norm_eps: float = 1e-6) -> torch.Tensor:
    """rope_kv_append + paged_decode_attention with the RoPE and append inside the
    attention's split kernel (two launches instead of three, the same results):
    qkv bf16 [B, (n_heads + 2 kv_heads) * head_dim] -> bf16 [B, n_heads * head_dim]."""
    op = "decode_attention_step"
    _require_gpu(op, qkv=qkv, positions=positions, cos=cos, sin=sin)
    _check_bf16(op, "qkv", qkv)
    B = qkv.shape[0]
    d, nkv = cache.head_dim, cache.kv_heads
    if qkv.shape != (B, (n_heads + 2 * nkv) * d):
        raise ValueError(f"[{op}] qkv must be [B, {(n_heads + 2 * nkv) * d}], "
                         f"got {tuple(qkv.shape)}")
    if positions.dtype != torch.int64 or positions.shape != (B,) or cache.batch != B:
        raise ValueError(f"[{op}] positions must be int64 [{B}] and match the page table")
    if cos.dtype != torch.float32 or sin.shape != cos.shape or cos.shape[0] < cache.capacity \
            or cos.shape[-1] != d // 2:
        raise ValueError(f"[{op}] cos/sin must be float32 [>= {cache.capacity}, {d // 2}]")
    for name, w in (("q_norm", q_norm), ("k_norm", k_norm)):
        if w is not None and (w.dtype != torch.bfloat16 or w.shape != (d,)):
            raise ValueError(f"[{op}] {name} must be bfloat16 [{d}]")
    L = _lib.lib()
    ws_bytes = L.mq_paged_decode_attention_workspace(B, n_heads, nkv, d, cache.pages_per_seq,
                                                     cache.page_size)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=qkv.device)
    out = torch.empty(B, n_heads * d, dtype=torch.bfloat16, device=qkv.device)
    _lib.check(L.mq_decode_attention_step(
        _ptr(qkv.contiguous()), _ptr(positions), _ptr(cache.page_table), cache.pages_per_seq,
        cache.page_size, cache.num_pages, _ptr(cos.contiguous()), _ptr(sin.contiguous()),
        _ptr(q_norm), _ptr(k_norm), float(norm_eps), _ptr(cache.k[layer]), _ptr(cache.v[layer]),
        B, n_heads, nkv, d, float(scale), _ptr(ws), ws_bytes, _ptr(out), _stream(qkv)), op)
    return out


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """gate_up bf16 [..., 2 * I] -> bf16 [..., I] = bf16(bf16(silu(gate)) * up)."""
    op = "silu_mul"
    _require_gpu(op, gate_up=gate_up)
    _check_bf16(op, "gate_up", gate_up)
    two_i = gate_up.shape[-1]
    if two_i % 2:
        raise ValueError(f"[{op}] the last dimension must be even, got {two_i}")
    g = gate_up.contiguous()
    out = torch.empty(tuple(g.shape[:-1]) + (two_i // 2,), dtype=torch.bfloat16, device=g.device)
    L = _lib.lib()
    _lib.check(L.mq_silu_mul(_ptr(g), _ptr(out), g.numel() // two_i, two_i // 2, _stream(g)), op)
    return out


__all__ = ["PagedKV", "rms_norm", "rope_kv_append", "paged_decode_attention", "attention_step",
           "silu_mul", "argmax_rows"]
