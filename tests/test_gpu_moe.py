"""Mixture-of-experts routing kernels (moe.route / expert_sort / combine) and
the routed expert block (moe.MoEBlock) against PyTorch restatements of the
reference's MoE block (models/lfm2.py:348-375, SwitchGLU :193-218,
_gather_sort/_scatter_unsort :613-622), and a Qwen3-MoE-shaped decoder
against its float32 restatement.

* route: the chosen expert sets equal torch.topk of the float32 softmax; the
  gates (renormalised or not) are within one bfloat16 step.
* expert_sort: bit-equal to torch.argsort(stable=True) and its inverse.
* combine: bit-equal to the sequential float32 sum of bf16(y * score).
* MoEBlock: norm-wise within 2e-2 of a float32 per-expert restatement with the
  same routing choice (the activations in between are bfloat16).
"""

from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from qwen2_reference import _linear, greedy_agreement, moe_reference, reference_logits

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def moe():
    return importlib.import_module("mlx-server-runtime_amd.moe")


@pytest.fixture(scope="module")
def mq():
    return importlib.import_module("mlx-server-runtime_amd")


def _gen(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


@pytest.mark.parametrize("T,E,k,norm", [(37, 128, 8, True), (8, 128, 8, True), (5, 8, 2, False),
                                        (300, 60, 4, True), (3, 512, 16, False), (1, 4, 4, True)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_route(moe, T, E, k, norm, with_bias):
    logits = (torch.randn(T, E, generator=_gen(E + T), device=DEV) * 2).to(torch.bfloat16)
    bias = (torch.randn(E, generator=_gen(1), device=DEV) * 0.01) if with_bias else None
    idx, sc = moe.route(logits, k, norm, bias)
    gates = torch.softmax(logits.float(), -1)
    if bias is not None:
        gates = gates + bias
    top = torch.topk(gates, k, -1)
    assert idx.dtype == torch.int32 and idx.shape == (T, k)
    assert torch.equal(torch.sort(idx.long(), -1).values, torch.sort(top.indices, -1).values)
    ref = gates.gather(-1, idx.long())
    if norm:
        ref = ref / (ref.sum(-1, keepdim=True) + 1e-20)
    assert bool(((sc.float() - ref).abs() <= ref.abs() * 2.0 ** -7 + 1e-7).all())
    # descending gate order
    assert bool((ref[:, :-1] >= ref[:, 1:]).all())


@pytest.mark.parametrize("T,E,k", [(8, 128, 8), (70, 128, 8), (8, 128, 20), (3, 512, 16),
                                   (5, 300, 17), (1, 64, 64), (2, 4, 4)])
def test_route_ties_go_to_the_lower_id(moe, T, E, k):
    """Logits from six values (many equal gates): the picks in the order of
    (descending logit, ascending id) exactly -- the softmax keeps the logits'
    order, equal logits give equal gates -- by moe.route and by the fused
    route_sort (up to 64 tokens one launch), with k rounds of arg-max (k <= 16)
    and with counted ranks (k > 16)."""
    g = torch.Generator().manual_seed(T * E + k)
    lv = torch.randint(0, 6, (T, E), generator=g).float() * 0.5
    logits = lv.to(torch.bfloat16).to(DEV)
    ids = torch.arange(E).expand(T, E)
    ref = torch.from_numpy(np.lexsort((ids.numpy(), -lv.numpy()), axis=-1)[:, :k].copy())
    idx, sc = moe.route(logits, k, True)
    assert torch.equal(idx.cpu().long(), ref)
    got = moe.route_sort(logits, k, E, True, with_offsets=True)
    assert torch.equal(got[0].cpu().long(), ref) and torch.equal(got[1], sc)
    gates = torch.softmax(lv, -1).gather(-1, ref)
    gates = gates / (gates.sum(-1, keepdim=True) + 1e-20)
    assert bool(((sc.cpu().float() - gates).abs() <= gates * 2.0 ** -7 + 1e-7).all())
    flat = ref.reshape(-1)
    offs = got[6].cpu().long()
    assert torch.equal(offs, torch.searchsorted(torch.sort(flat).values, torch.arange(E + 1)))


@pytest.mark.parametrize("T,k,E,bad", [(8, 8, 128, 0), (4096, 8, 128, 0), (77, 3, 17, 0),
                                       (1, 1, 1, 0), (2000, 6, 512, 0),
                                       (20000, 8, 128, 0),   # 157 chunks: 3 to a block
                                       (1500, 3, 60, 40)])   # ids -1 and E in every block
def test_expert_sort(moe, T, k, E, bad):
    """The sort's blocks each place a range of whole 1024-entry chunks (up to
    64 blocks): order, ids, inverse, rows and segment starts against a stable
    argsort, with out-of-range ids (bucket E) spread over several blocks."""
    ids = torch.randint(0, E, (T, k), generator=_gen(T + k), device=DEV, dtype=torch.int32)
    if bad:
        flat_ids = ids.view(-1)
        at = torch.randperm(flat_ids.numel(), generator=_gen(bad), device=DEV)[:bad]
        flat_ids[at[::2]] = -1
        flat_ids[at[1::2]] = E
    sorted_ids, order, inverse, rows, offs = moe.expert_sort(ids, E, with_offsets=True)
    flat = ids.reshape(-1).long()
    # out-of-range ids all sort last, in entry order, kept as they are
    key = torch.where((flat >= 0) & (flat < E), flat, torch.full_like(flat, E))
    ref_order = torch.argsort(key, stable=True)
    assert torch.equal(order.long(), ref_order)
    assert torch.equal(sorted_ids.long(), flat[ref_order])
    assert torch.equal(inverse.long(), torch.argsort(ref_order, stable=True))
    assert torch.equal(rows.long(), ref_order // k)
    # segment starts: expert e's run begins after every smaller valid id
    ref_offs = torch.searchsorted(key[ref_order], torch.arange(E + 1, device=DEV))
    assert torch.equal(offs.long(), ref_offs)


def test_expert_sort_out_of_range_ids_go_last(moe):
    ids = torch.tensor([[3, -1], [7, 0], [8, 3]], dtype=torch.int32, device=DEV)  # E = 8
    sorted_ids, order, inverse, rows, offs = moe.expert_sort(ids, 8, with_offsets=True)
    assert offs.tolist() == [0, 1, 1, 1, 3, 3, 3, 3, 4]  # the ids -1 and 8 follow offs[8]
    assert sorted_ids.tolist() == [0, 3, 3, 7, -1, 8]
    assert order.tolist() == [3, 0, 5, 2, 1, 4]
    assert rows.tolist() == [1, 0, 2, 1, 0, 2]
    assert torch.equal(order[inverse.long()].long(), torch.arange(6, device=DEV))


@pytest.mark.parametrize("T,k,H", [(8, 8, 2048), (3, 2, 256), (513, 8, 2048), (2, 4, 8)])
@pytest.mark.parametrize("sorted_rows", [True, False])
def test_combine(moe, T, k, H, sorted_rows):
    g = _gen(T * H + k)
    y = torch.randn(T * k, H, generator=g, device=DEV).to(torch.bfloat16)
    sc = torch.rand(T, k, generator=g, device=DEV).to(torch.bfloat16)
    inverse = None
    src = torch.arange(T * k, device=DEV)
    if sorted_rows:
        inverse = torch.randperm(T * k, generator=torch.Generator().manual_seed(T)).to(
            device=DEV, dtype=torch.int32)
        src = inverse.long()
    out = moe.combine(y, inverse, sc)
    rows = y[src].float().reshape(T, k, H)
    acc = torch.zeros(T, H, device=DEV)
    for j in range(k):
        acc = acc + (rows[:, j] * sc[:, j:j + 1].float()).to(torch.bfloat16).float()
    assert torch.equal(out, acc.to(torch.bfloat16))


@pytest.mark.parametrize("T,E,k", [(1, 128, 8), (8, 128, 8), (37, 60, 4), (64, 512, 16),
                                   (65, 128, 8), (300, 17, 3)])
def test_route_sort_equals_route_then_sort(moe, T, E, k):
    """One launch up to 64 tokens (else the two kernels): bit-equal outputs."""
    logits = (torch.randn(T, E, generator=_gen(3 * T + E), device=DEV) * 2).to(torch.bfloat16)
    bias = torch.randn(E, generator=_gen(2), device=DEV) * 0.01
    for b in (None, bias):
        idx, sc = moe.route(logits, k, True, b)
        ref = (idx, sc) + moe.expert_sort(idx, E, with_offsets=True)
        got = moe.route_sort(logits, k, E, True, b, with_offsets=True)
        assert len(got) == len(ref) == 7
        for a, r in zip(got, ref):
            assert torch.equal(a, r)


@pytest.mark.parametrize("T,k,H", [(8, 8, 2048), (3, 2, 256), (130, 8, 2048), (2, 4, 8192),
                                   (1, 1, 8)])
@pytest.mark.parametrize("sorted_rows", [True, False])
def test_combine_rms_norm_equals_combine_then_norm(moe, T, k, H, sorted_rows):
    """combine -> residual add -> RMSNorm in one kernel: bit-equal to the
    combine kernel followed by the RMSNorm kernel."""
    dops = importlib.import_module("mlx-server-runtime_amd.decode_ops")
    g = _gen(T * H + 7 * k)
    y = torch.randn(T * k, H, generator=g, device=DEV).to(torch.bfloat16)
    sc = torch.rand(T, k, generator=g, device=DEV).to(torch.bfloat16)
    res = (torch.randn(T, H, generator=g, device=DEV) * 4).to(torch.bfloat16)
    w = (torch.rand(H, generator=g, device=DEV) + 0.5).to(torch.bfloat16)
    inverse = None
    if sorted_rows:
        inverse = torch.randperm(T * k, generator=torch.Generator().manual_seed(T)).to(
            device=DEV, dtype=torch.int32)
    out, h = moe.combine_rms_norm(y, inverse, sc, res, w, 1e-6)
    ref_out, ref_h = dops.rms_norm(moe.combine(y, inverse, sc), w, 1e-6, residual=res)
    assert torch.equal(h, ref_h) and torch.equal(out, ref_out)


def test_fused_entry_errors(moe):
    logits = torch.zeros(4, 16, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="experts"):
        moe.route_sort(logits, 2, 8)
    y = torch.zeros(8, 64, dtype=torch.bfloat16, device=DEV)
    sc = torch.zeros(4, 2, dtype=torch.bfloat16, device=DEV)
    w = torch.ones(64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="residual"):
        moe.combine_rms_norm(y, None, sc, torch.zeros(3, 64, dtype=torch.bfloat16, device=DEV),
                             w, 1e-6)
    with pytest.raises(NotImplementedError, match="not supported"):
        moe.combine_rms_norm(torch.zeros(8, 8200, dtype=torch.bfloat16, device=DEV), None, sc,
                             torch.zeros(4, 8200, dtype=torch.bfloat16, device=DEV),
                             torch.ones(8200, dtype=torch.bfloat16, device=DEV), 1e-6)


@pytest.mark.parametrize("T,E,inter,K,bits,lhs", [(64, 128, 768, 2048, 4, True),
                                                   (64, 128, 768, 2048, 8, True),
                                                   (24, 16, 128, 256, 4, True),
                                                   (5, 8, 256, 512, 4, False)])
def test_gather_qmm_swiglu_equals_gather_then_silu_mul(moe, mq, T, E, inter, K, bits, lhs):
    """The gathered SwiGLU GEMV (every expert: gate rows, then up rows) is bit for
    bit gather_qmm of the 2N-row bank followed by silu_mul; out-of-range expert
    ids give zero rows in both."""
    core = importlib.import_module("mlx-server-runtime_amd.core")
    dops = importlib.import_module("mlx-server-runtime_amd.decode_ops")
    g = _gen(T * 7 + bits)
    w = (torch.randn(E, 2 * inter, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    wq, s, b = mq.quantize(w, 64, bits)
    n_x = 8 if lhs else T
    x = torch.randn(n_x, 1, K, generator=g, device=DEV).to(torch.bfloat16)
    rhs = torch.randint(0, E, (T,), generator=g, device=DEV, dtype=torch.int32)
    rhs[T // 2] = E + 3  # out of the table
    rows = (torch.randint(0, n_x, (T,), generator=g, device=DEV, dtype=torch.int32)
            if lhs else None)
    assert core.gather_swiglu_supported(T, 1, inter, K, 64, bits)
    out = core.gather_qmm_swiglu(x, wq, s, b, rows, rhs, 64, bits)
    gu = core.gather_qmm(x, wq, s, b, lhs_indices=rows, rhs_indices=rhs, group_size=64,
                         bits=bits)
    ref = dops.silu_mul(gu.reshape(T, 2 * inter)).reshape(T, 1, inter)
    assert out.shape == (T, 1, inter)
    assert torch.equal(out, ref)
    assert not out[T // 2].any()


def _block(moe, mq, E, k, H, inter, seed=0):
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    cfg = q2.Qwen2Config(H, 4 * H, 4, 2, 1, 100)
    g = _gen(seed)
    router = q2._random_qlinear(g, E, H, cfg, False, DEV)
    gate_up = q2._random_experts(g, E, 2 * inter, H, cfg, DEV)
    down = q2._random_experts(g, E, H, inter, cfg, DEV)
    return moe.MoEBlock(router, gate_up, down, k, True)


@pytest.mark.parametrize("T", [3, 8, 512])
def test_moe_block_vs_float32(moe, mq, T):
    """T=3: 24 pairs (unsorted path); T=8: 64 pairs (sorted); T=512: 4096 pairs."""
    E, k, H, inter = 16, 8, 256, 128
    block = _block(moe, mq, E, k, H, inter)
    x = torch.randn(T, H, generator=_gen(T), device=DEV).to(torch.bfloat16)
    out = block(x)
    idx, _ = moe.route(block.gate(x), k, True)
    ref = moe_reference(mq, block, x, indices=idx)
    err = float((out.float() - ref).abs().max() / ref.abs().max())
    assert err < 2e-2, err
    # the routing itself: the float32 router's choice matches except at near-ties
    ref_idx = torch.topk(torch.softmax(_linear(mq, block.gate, x.float()), -1), k, -1).indices
    same = (torch.sort(idx.long(), -1).values == torch.sort(ref_idx, -1).values).all(-1)
    assert same.float().mean() >= 0.9


@pytest.mark.parametrize("T", [2, 8, 100])
def test_moe_block_residual_norm_equals_unfused(moe, mq, T):
    """MoEBlock.residual_norm == rms_norm(block(x), residual), bit for bit."""
    dops = importlib.import_module("mlx-server-runtime_amd.decode_ops")
    block = _block(moe, mq, 16, 8, 256, 128, seed=9)
    g = _gen(T + 11)
    x = torch.randn(T, 256, generator=g, device=DEV).to(torch.bfloat16)
    res = torch.randn(T, 256, generator=g, device=DEV).to(torch.bfloat16)
    w = (torch.rand(256, generator=g, device=DEV) + 0.5).to(torch.bfloat16)
    out, h = block.residual_norm(x, res, w, 1e-6)
    ref_out, ref_h = dops.rms_norm(block(x), w, 1e-6, residual=res)
    assert torch.equal(h, ref_h) and torch.equal(out, ref_out)


def test_moe_block_sorted_equals_unsorted(moe, mq):
    """Permutation equivariance (models/lfm2.py:202-218): rows routed through
    the sorted path agree with the same rows through the unsorted path (the
    kernels differ, so to rounding; a wrong permutation would be O(1))."""
    E, k, H, inter = 16, 8, 256, 128
    block = _block(moe, mq, E, k, H, inter, seed=3)
    x = torch.randn(32, H, generator=_gen(4), device=DEV).to(torch.bfloat16)
    full = block(x)                        # 256 pairs: sorted
    parts = torch.cat([block(x[i:i + 2]) for i in range(0, 32, 2)])  # 16 pairs: unsorted
    assert _nrel(full, parts) < 1e-2


def _nrel(a, b):
    return float((a.float() - b.float()).abs().max() / b.float().abs().max())


def _per_position(a, b):
    """Norm-wise relative error of every (row, position) logit vector."""
    d = (a.float() - b.float()).abs().amax(-1)
    return (d / b.float().abs().amax(-1)).flatten()


def _forced_routing_check(mq, m, prompt, n, label, prefill_check=True):
    """Generate n greedy tokens (eager, routing traced; graph replay must give
    the same tokens), then check the logits against the float32 restatement
    with every MoE layer's expert choice teacher-forced to the model's own
    (routing traced per position: the prompt's prefill, then each decode
    step; and, for the prefill check, the model's own prefill over the whole
    sequence).  Bars, per logit vector: decode logits, and prefill logits at
    the same positions, within 2 * e16 + 1e-2 of the restatement, e16 being
    the largest distance between the float32 restatement and the one that
    rounds to bfloat16 wherever the model stores bfloat16 (same routing);
    teacher-forced greedy tokens: where ours differs from the restatement's
    argmax, its top-2 margin is within that position's bfloat16-storage
    error (twice it: the bfloat16 rounding alone could flip such a pair).
    Returns (e_dec max, e16 max)."""
    from qwen2_reference import RoutingTrace
    B, T = prompt.shape
    steps = []
    with RoutingTrace(m) as tr:
        toks = m.generate(prompt, n, use_graph=False, logits_out=steps)
    assert torch.equal(toks, m.generate(prompt, n))
    full = torch.cat([prompt, toks], 1)[:, :-1]
    routing = tr.per_layer(B)
    assert all(r.shape[:2] == full.shape for r in routing.values())
    dec = torch.stack(steps, 1)
    r32 = reference_logits(mq, m, full, head_from=T - 1, routing=routing)
    r16 = reference_logits(mq, m, full, bf16_activations=True, head_from=T - 1,
                           routing=routing)
    e = _per_position(dec, r32)
    e16 = _per_position(r16, r32)
    eps = (dec.float() - r32).abs().amax(-1)
    eps16 = (r16 - r32).abs().amax(-1)
    top2 = r32.topk(2, -1).values
    margin = top2[..., 0] - top2[..., 1]
    differ = r32.argmax(-1) != toks
    print(f"{label}: decode logits err max {e.max():.4f} (bf16-storage {e16.max():.4f}); "
          f"{int(differ.sum())}/{differ.numel()} tokens differ from the restatement's argmax, "
          f"margin/eps16 there {[round(float(v), 2) for v in (margin / eps16)[differ]]}",
          flush=True)
    assert e.max() <= 2 * e16.max() + 1e-2, (float(e.max()), float(e16.max()))
    # disagreements only where the bfloat16 storage alone moves the logits
    # by half the restatement's top-2 margin
    assert bool((margin[differ] <= 2 * eps16[differ]).all()), (margin / eps16)[differ]
    assert bool((eps[differ] <= 2 * eps16[differ] + 1e-2 * r32.abs().amax(-1)[differ]).all())
    if prefill_check:
        with RoutingTrace(m) as tp:
            ours = m.prefill(full, m.new_cache(B, full.shape[1]), all_positions=True)
        pre_routing = tp.per_layer(B)
        flips = sum(int((pre_routing[i].sort(-1).values != routing[i].sort(-1).values)
                        .any(-1).sum()) for i in routing)
        p32 = reference_logits(mq, m, full, head_from=T - 1, routing=pre_routing)
        p16 = reference_logits(mq, m, full, bf16_activations=True, head_from=T - 1,
                               routing=pre_routing)
        ep = _per_position(ours[:, T - 1:], p32)
        ep16 = _per_position(p16, p32)
        print(f"{label}: prefill logits err max {ep.max():.4f} (bf16-storage "
              f"{ep16.max():.4f}); prefill and decode route {flips} of "
              f"{sum(r.shape[0] * r.shape[1] for r in routing.values())} (token, layer) "
              f"pairs differently", flush=True)
        assert ep.max() <= 2 * ep16.max() + 1e-2, (float(ep.max()), float(ep16.max()))
    return float(e.max()), float(e16.max())


def test_qwen3_moe_small_decoder(mq):
    """Qwen3-MoE-shaped (q/k norms, 8 experts top 2, renormalised) decoder:
    graph decode equals eager decode; decode and prefill logits and greedy
    tokens against the float32 restatement with the routing teacher-forced
    (a near-tie between two experts' gates is a discrete choice that the
    bfloat16 model and the float32 restatement can make differently; with the
    model's own choice given, what is left is the arithmetic)."""
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000, head_dim_=64, attention_bias=False,
                         qk_norm=True, num_experts=8, num_experts_per_tok=2,
                         moe_intermediate_size=128)
    m = q2.Qwen2Model.random(cfg, seed=5, device=DEV)
    B, T, n = 4, 24, 16   # 4 * 2 = 8 pairs per decode step; prefill 192 pairs (sorted)
    prompt = torch.randint(0, cfg.vocab_size, (B, T), generator=_gen(6), device=DEV)
    _forced_routing_check(mq, m, prompt, n, "qwen3-moe small")


def test_qwen3_dense_with_qk_norm_small_decoder(mq):
    """The same decoder with a dense MLP (q/k norms only): dense-model bounds."""
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000, head_dim_=64, attention_bias=False,
                         qk_norm=True)
    m = q2.Qwen2Model.random(cfg, seed=5, device=DEV)
    B, T, n = 2, 16, 16
    prompt = torch.randint(0, cfg.vocab_size, (B, T), generator=_gen(7), device=DEV)
    steps = []
    toks = m.generate(prompt, n, use_graph=False, logits_out=steps)
    full = torch.cat([prompt, toks], 1)[:, :-1]
    ref = reference_logits(mq, m, full)
    ours = m.prefill(full, m.new_cache(B, full.shape[1]), all_positions=True)
    assert _per_position(ours, ref).max() <= 4e-2
    assert _per_position(torch.stack(steps, 1), ours[:, T - 1:T - 1 + n]).max() <= 3e-2
    match, total, worst = greedy_agreement(ref, T, toks)
    assert match >= 0.9 * total and worst <= 0.05, (match, total, worst)


def test_qwen3_30b_a3b_shape_decoder_batch_8(mq):
    """The MoE workload at its own widths and batch, 2 layers deep: hidden 2048,
    32/4 heads of 128 with q/k norms, 128 experts top 8 (renormalised), expert
    MLP 768, vocab 151936 (models/lfm2.py:365-375 routing, SwitchGLU
    :193-218); 8 sequences of 512-token prompts (4096 tokens, 32768 expert
    pairs through the sorted gather GEMM at prefill), then 8 greedy decode
    steps (64 pairs per step: route + sort in one launch, the gathered SwiGLU
    GEMV, the gathered down GEMV, combine + residual + norm); the routing
    teacher-forced bars of _forced_routing_check."""
    import dataclasses
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    cfg = dataclasses.replace(q2.Qwen2Config.qwen3_30b_a3b(), num_hidden_layers=2)
    m = q2.Qwen2Model.random(cfg, seed=0, device=DEV)
    B, T, n = 8, 512, 8
    prompt = torch.randint(0, cfg.vocab_size, (B, T), generator=_gen(2), device=DEV)
    _forced_routing_check(mq, m, prompt, n, "config-5 shape (2 layers)")


@pytest.mark.timeout(900)
def test_qwen3_30b_a3b_full_depth_batch_8(mq):
    """The MoE workload at full depth, as the bench decodes it: 48 layers,
    8 sequences of 512-token prompts, then 8 greedy decode steps; graph tokens
    equal eager tokens, and the routing teacher-forced bars of
    _forced_routing_check over all 48 layers (decode and prefill logits)."""
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    cfg = q2.Qwen2Config.qwen3_30b_a3b()
    assert cfg.num_hidden_layers == 48
    m = q2.Qwen2Model.random(cfg, seed=0, device=DEV)
    B, T, n = 8, 512, 8
    prompt = torch.randint(0, cfg.vocab_size, (B, T), generator=_gen(2), device=DEV)
    print("config 5 full depth: 48 layers, batch 8, 512-token prompts, 8 steps", flush=True)
    _forced_routing_check(mq, m, prompt, n, "config-5 shape (48 layers)")


@pytest.mark.parametrize("K", [2048, 768])
def test_gather_segments_equals_gather(moe, mq, K):
    """gather_qmm given the sort's segment offsets (mq_gather_qmm_segments) equals
    gather_qmm deriving the segments itself, bit for bit: 2048 tokens routed to
    8 of 128 experts, the x rows gathered through the sort's rows."""
    E, k, N, T = 128, 8, 512, 2048
    g = _gen(K)
    logits = torch.randn(T, E, generator=g, device=DEV).to(torch.bfloat16)
    _, _, sorted_ids, _, _, rows, offs = moe.route_sort(logits, k, E, with_offsets=True)
    w = (torch.randn(E * N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    wq, sc, bi = (t.reshape(E, N, -1) for t in mq.quantize(w, 64, 4))
    x = torch.randn(T, 1, K, generator=g, device=DEV).to(torch.bfloat16)
    a = mq.gather_qmm(x, wq, sc, bi, lhs_indices=rows, rhs_indices=sorted_ids,
                      sorted_indices=True, expert_offsets=offs)
    b = mq.gather_qmm(x, wq, sc, bi, lhs_indices=rows, rhs_indices=sorted_ids,
                      sorted_indices=True)
    assert torch.equal(a, b)
    c = mq.gather_qmm(x, wq, sc, bi, lhs_indices=rows, rhs_indices=sorted_ids)  # unsorted path
    assert float((a.float() - c.float()).abs().max() / c.float().abs().max()) <= 1e-2
    # the same bank read as gate | up halves: SiLU * up in the GEMM's epilogue
    core = importlib.import_module("mlx-server-runtime_amd.core")
    ops = importlib.import_module("mlx-server-runtime_amd.decode_ops")
    f = core.gather_qmm_swiglu(x, wq, sc, bi, rows, sorted_ids, 64, 4, expert_offsets=offs)
    assert f.shape == (T * k, 1, N // 2)
    assert torch.equal(f.reshape(-1, N // 2), ops.silu_mul(a.reshape(-1, N)))


def test_gather_segments_clamps_caller_offsets(moe, mq):
    """Caller-supplied segment starts outside [0, T] are clamped by the kernel
    (a negative first start, a last start past T): every row and x batch it
    touches stays inside y and lhs, and here the clamped starts are the sort's
    own, so the output is bit-equal to the call with the sort's offsets."""
    E, k, N, K, T = 128, 8, 512, 2048, 256
    g = _gen(91)
    logits = torch.randn(T, E, generator=g, device=DEV).to(torch.bfloat16)
    _, _, sorted_ids, _, _, rows, offs = moe.route_sort(logits, k, E, with_offsets=True)
    P = T * k
    assert int(offs[0]) == 0 and int(offs[-1]) == P
    bad = offs.clone()
    bad[0], bad[-1] = -7, P + 999
    w = (torch.randn(E * N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    wq, sc, bi = (t.reshape(E, N, -1) for t in mq.quantize(w, 64, 4))
    x = torch.randn(T, 1, K, generator=g, device=DEV).to(torch.bfloat16)
    print(f"gather segments: clamped offsets, {P} pairs", flush=True)
    a = mq.gather_qmm(x, wq, sc, bi, lhs_indices=rows, rhs_indices=sorted_ids,
                      sorted_indices=True, expert_offsets=offs)
    b = mq.gather_qmm(x, wq, sc, bi, lhs_indices=rows, rhs_indices=sorted_ids,
                      sorted_indices=True, expert_offsets=bad)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("K,gs", [(2048, 64), (768, 64), (2048, 32), (2048, 128), (768, 128)])
def test_gather_short_tiles_equal_long_tiles(mq, K, gs):
    """An expert segment of at most 64 rows runs the segment GEMM's short-tile
    loop (its own LDS layout and prefetch); the same rows at the head of a
    100-row segment run the masked full-tile loop.  Each output row depends
    only on its own x row, so the two must agree bit for bit: segments of 20
    and 64 rows against the first rows of a 100-row segment of expert 0 (the
    x rows gathered through lhs), expert 1 keeping 100 rows in every call;
    group sizes 32/64/128 (8, 16 or 4 steps a scale chunk; K = 768 ends
    mid-chunk)."""
    E, N, T = 4, 512, 300
    g = _gen(K + gs)
    w = (torch.randn(E * N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    wq, sc, bi = (t.reshape(E, N, -1) for t in mq.quantize(w, gs, 4))
    x = torch.randn(T, 1, K, generator=g, device=DEV).to(torch.bfloat16)
    src = torch.randperm(T, generator=torch.Generator().manual_seed(K))[:200].to(DEV)

    def run(r0):
        lhs = torch.cat([src[:r0], src[100:200]]).to(torch.int32).contiguous()
        rhs = torch.cat([torch.zeros(r0, dtype=torch.int32, device=DEV),
                         torch.ones(100, dtype=torch.int32, device=DEV)]).contiguous()
        offs = torch.tensor([0, r0] + [r0 + 100] * (E - 1), dtype=torch.int32, device=DEV)
        return mq.gather_qmm(x, wq, sc, bi, lhs_indices=lhs, rhs_indices=rhs, group_size=gs,
                             sorted_indices=True, expert_offsets=offs).reshape(-1, N)

    print(f"gather short tiles: K={K}, group {gs}, segments of 100 / 64 / 20 rows", flush=True)
    full = run(100)
    ref = x[src[:100], 0].float() @ mq.dequantize(wq[0], sc[0], bi[0], gs, 4).float().t()
    assert float((full[:100].float() - ref).norm() / ref.norm()) < 1e-2
    for r0 in (64, 20):
        short = run(r0)
        torch.cuda.synchronize()
        assert torch.equal(short[:r0], full[:r0]), r0
        assert torch.equal(short[r0:], full[100:]), r0


def test_moe_block_odd_group_count(moe, mq):
    """hidden 192 (3 groups of 64 per row): the expert-segment GEMM with the
    SiLU*up epilogue does not take an odd group count, so a sorted prefill
    batch (16 tokens x top 8 = 128 pairs) runs gather_qmm then silu_mul --
    against the float32 restatement under the kernel's routing."""
    core = importlib.import_module("mlx-server-runtime_amd.core")
    E, k, H, inter, T = 16, 8, 192, 128, 16
    assert not core.gather_segments_supported(T * k, 1, inter, H, E, T, 64, 4, swiglu=True)
    block = _block(moe, mq, E, k, H, inter, seed=13)
    x = torch.randn(T, H, generator=_gen(14), device=DEV).to(torch.bfloat16)
    out = block(x)
    idx, _ = moe.route(block.gate(x), k, True)
    ref = moe_reference(mq, block, x, indices=idx)
    err = float((out.float() - ref).abs().max() / ref.abs().max())
    assert err < 2e-2, err
