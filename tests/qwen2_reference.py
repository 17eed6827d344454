"""Float32 reference of the Qwen2 decoder for the GPU parity tests.

Test infrastructure only.  It restates the reference's graph
(python/mlx_worker/native_mlx/models/qwen2.py:47-227) in float32 end to end
-- RMSNorm, linears, RoPE, attention, SiLU, residuals -- on the *dequantized*
weights of a mlx-server-runtime_amd.qwen2.Qwen2Model, so it differs from the
model under test only by the latter's bfloat16 activations.  Weights are
dequantized with the library's dequantize (bit-exact with the oracle, checked
by test_gpu_parity.py) one layer at a time.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def _deq(mq, ql) -> torch.Tensor:
    if not hasattr(ql, "wq"):  # an unquantized (bfloat16) linear
        return ql.weight.float()
    return mq.dequantize(ql.wq, ql.scales, ql.biases, ql.group_size, ql.bits).float()


def _rope(x: torch.Tensor, positions: torch.Tensor, theta: float, scale: float) -> torch.Tensor:
    """Non-traditional RoPE (mx.fast.rope, traditional=False) written
    independently of the decoder's tables: element i of the first half and
    element i of the second half form the complex number x_i + j x_(i+d/2),
    multiplied by exp(j * position * scale * theta^(-2i/d)).
    x [..., S, d] float32, positions [S]."""
    d = x.shape[-1]
    half = d // 2
    freq = torch.tensor([math.pow(theta, -2.0 * i / d) for i in range(half)],
                        dtype=torch.float64, device=x.device)
    ang = (positions.double() * scale)[:, None] * freq[None, :]
    rot = torch.polar(torch.ones_like(ang), ang)                      # [S, half] complex128
    z = torch.complex(x[..., :half].double(), x[..., half:].double()) * rot
    return torch.cat([z.real, z.imag], -1).to(x.dtype)


def _linear(mq, ql, x):
    y = x @ _deq(mq, ql).t()
    if ql.bias is not None:
        y = y + ql.bias.float()
    return y


def _rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w.float()


def _deq_experts(mq, qe) -> torch.Tensor:
    E, N = qe.wq.shape[:2]
    return mq.dequantize(qe.wq.reshape(E * N, -1), qe.scales.reshape(E * N, -1),
                         qe.biases.reshape(E * N, -1), qe.group_size, qe.bits
                         ).float().reshape(E, N, -1)


def moe_reference(mq, block, x, r=lambda t: t, indices=None):
    """Float32 restatement of the routed expert MLP (models/lfm2.py:365-375,
    SwitchGLU :193-218): softmax router, top-k, renormalised gates, per
    expert down(silu(gate(x)) * up(x)), gate-weighted sum over the k choices
    in order.  With indices (int [T, k]) the routing choice is taken from there
    (the gates are still recomputed here), which isolates the expert arithmetic
    from near-ties.  Each expert's rows are computed together (one matmul per
    expert), so the weights are never gathered per pair."""
    shape = x.shape
    xt = x.reshape(-1, shape[-1]).float()
    T, H = xt.shape
    gates = torch.softmax(_linear(mq, block.gate, xt), -1)
    if block.expert_bias is not None:
        gates = gates + block.expert_bias.float()
    if indices is None:
        indices = torch.topk(gates, block.top_k, -1).indices
    indices = indices.long()
    sc = gates.gather(-1, indices)
    if block.norm_topk_prob:
        sc = sc / (sc.sum(-1, keepdim=True) + 1e-20)
    sc = r(sc)
    wgu, wd = _deq_experts(mq, block.gate_up), _deq_experts(mq, block.down)
    inter = wd.shape[-1]
    flat = indices.reshape(-1)                       # pair p = (token p // k, choice p % k)
    contrib = torch.zeros(T * block.top_k, H, device=xt.device)
    for e in torch.unique(flat).tolist():
        pairs = (flat == e).nonzero().squeeze(-1)
        xe = xt[pairs // block.top_k]
        gu = r(xe @ wgu[e].t())                                        # [n, 2I]
        act = r(r(F.silu(gu[:, :inter])) * gu[:, inter:])
        y = r(act @ wd[e].t())                                         # [n, H]
        contrib[pairs] = r(y * sc.reshape(-1)[pairs, None])
    contrib = contrib.reshape(T, block.top_k, H)
    out = torch.zeros_like(xt)
    for j in range(block.top_k):
        out = out + contrib[:, j]
    return out.reshape(shape)


def reference_logits(mq, model, tokens: torch.Tensor, bf16_activations: bool = False,
                     head_from: int = 0, routing: dict | None = None) -> torch.Tensor:
    """tokens [B, S] (positions 0..S-1) -> float32 logits [B, S - head_from, vocab]
    of positions head_from..S-1, causal (the LM head on reference_hidden)."""
    h = reference_hidden(mq, model, tokens, bf16_activations, head_from, routing)
    head = model.lm_head if model.lm_head is not None else model.embed
    return h @ _deq(mq, head).t()


def reference_hidden(mq, model, tokens: torch.Tensor, bf16_activations: bool = False,
                     head_from: int = 0, routing: dict | None = None) -> torch.Tensor:
    """tokens [B, S] -> float32 final-normed hidden states [B, S - head_from, hidden]
    of positions head_from..S-1 (the LM head's input), causal.

    routing {layer index: int [B, S, k]} teacher-forces the MoE layers'
    expert choice (moe_reference's indices) to the model's own: the gates are
    still computed here, so only the discrete choice is taken over.

    With bf16_activations, values are rounded to bfloat16 wherever the model
    under test -- and the reference's MLX graph -- stores bfloat16 (norm
    outputs, linear outputs, q and k after RoPE, the KV cache, the residual
    stream, the SiLU product), isolating the kernels' own arithmetic."""
    r = (lambda t: t.to(torch.bfloat16).float()) if bf16_activations else (lambda t: t)

    c = model.cfg
    B, S = tokens.shape
    d, nh, nkv = c.head_dim, c.num_attention_heads, c.num_key_value_heads
    pos = torch.arange(S, device=tokens.device)
    causal = torch.full((S, S), float("-inf"), device=tokens.device).triu(1)
    e = model.embed
    if hasattr(e, "wq"):
        h = mq.embedding_lookup(tokens.reshape(-1).to(torch.int32), e.wq, e.scales, e.biases,
                                e.group_size, e.bits).float().reshape(B, S, c.hidden_size)
    else:
        h = e.weight.float()[tokens.reshape(-1).long()].reshape(B, S, c.hidden_size)
    for li, layer in enumerate(model.layers):
        x = r(_rms(h, layer.input_norm, c.rms_norm_eps))
        qkv = r(_linear(mq, layer.qkv, x))
        q, k, v = qkv[..., :nh * d], qkv[..., nh * d:(nh + nkv) * d], qkv[..., (nh + nkv) * d:]
        q, k = q.reshape(B, S, nh, d), k.reshape(B, S, nkv, d)
        if layer.q_norm is not None:  # Qwen3 per-head RMSNorm (models/qwen3.py:84-85)
            q = r(_rms(q, layer.q_norm, c.rms_norm_eps))
            k = r(_rms(k, layer.k_norm, c.rms_norm_eps))
        q = r(_rope(q.transpose(1, 2), pos, c.rope_theta, c.rope_scale))
        k = r(_rope(k.transpose(1, 2), pos, c.rope_theta, c.rope_scale))
        v = v.reshape(B, S, nkv, d).transpose(1, 2)
        rep = nh // nkv
        k, v = k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1)
        s = q @ k.transpose(-1, -2).contiguous() * d ** -0.5 + causal
        a = r((torch.softmax(s, -1) @ v).transpose(1, 2).reshape(B, S, nh * d))
        h = r(h + r(_linear(mq, layer.o, a)))
        x = r(_rms(h, layer.post_norm, c.rms_norm_eps))
        if layer.moe is not None:
            idx = None if routing is None else routing[li].reshape(B * S, -1)
            h = r(h + r(moe_reference(mq, layer.moe, x, r, indices=idx)))
            continue
        gu = r(_linear(mq, layer.gate_up, x))
        act = r(r(F.silu(gu[..., :c.intermediate_size])) * gu[..., c.intermediate_size:])
        h = r(h + r(_linear(mq, layer.down, act)))
    return r(_rms(h[:, head_from:], model.final_norm, c.rms_norm_eps))


def greedy_agreement(ref_logits: torch.Tensor, prompt_len: int, tokens: torch.Tensor):
    """Teacher-forced check of greedy tokens.  tokens [B, n] were generated after
    a prompt of prompt_len; ref_logits [B, prompt_len + n - 1 (or more), vocab].
    Returns (matches, n, worst), worst = the largest reference margin
    (ref top logit - ref logit of the chosen token) over mismatches, in units
    of that position's logit standard deviation (0 if all match)."""
    B, n = tokens.shape
    lg = ref_logits[:, prompt_len - 1:prompt_len - 1 + n]
    top = lg.argmax(-1)
    match = (top == tokens)
    chosen = lg.gather(-1, tokens.unsqueeze(-1)).squeeze(-1)
    margin = (lg.max(-1).values - chosen) / lg.std(-1)
    worst = float(margin[~match].max()) if (~match).any() else 0.0
    return int(match.sum()), B * n, worst


class RoutingTrace:
    """Records the expert ids every MoE layer of a model routes to, in eager
    calls, and assembles them per layer as [B, S, k] over the positions of a
    generate() call (its prompt prefill, then one position per decode step)
    or of a single prefill: the routing= argument of reference_logits."""

    def __init__(self, model):
        self.layers = [i for i, l in enumerate(model.layers) if l.moe is not None]
        self.model = model
        self.logs = {i: [] for i in self.layers}

    def __enter__(self):
        for i in self.layers:
            self.model.layers[i].moe.routing_log = self.logs[i]
        return self

    def __exit__(self, *exc):
        for i in self.layers:
            self.model.layers[i].moe.routing_log = None

    def per_layer(self, B: int) -> dict:
        """{layer: int [B, S, k]}: the calls' ids in call order, each call's
        rows being B sequences of equal length."""
        out = {}
        for i in self.layers:
            parts = [t.reshape(B, -1, t.shape[-1]) for t in self.logs[i]]
            out[i] = torch.cat(parts, 1)
        return out

