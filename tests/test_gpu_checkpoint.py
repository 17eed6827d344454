"""A model saved in the mlx-community layout and loaded back (checkpoint.py)
computes exactly what the original did: bit-identical logits, on the GPU."""

from __future__ import annotations

import importlib

import pytest
import torch

from qwen2_reference import reference_logits

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("kind,gs", [("qwen2", 64), ("qwen3_moe", 64), ("qwen2", 128),
                                     ("qwen3_moe", 32)])
def test_save_load_round_trip_same_logits(tmp_path, kind, gs):
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    ck = importlib.import_module("mlx-server-runtime_amd.checkpoint")
    if kind == "qwen2":
        cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000, group_size=gs)
    else:
        cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000, attention_bias=False,
                             qk_norm=True, num_experts=8, num_experts_per_tok=2,
                             moe_intermediate_size=128, group_size=gs)
    m = q2.Qwen2Model.random(cfg, seed=3, device=DEV)
    ck.save(m, tmp_path, shard_bytes=1 << 20)
    m2 = ck.load(tmp_path, device=DEV)
    assert m2.cfg == cfg
    ids = torch.randint(0, cfg.vocab_size, (2, 20), generator=torch.Generator(device=DEV)
                        .manual_seed(1), device=DEV)
    a = m.prefill(ids, m.new_cache(2, 20), all_positions=True)
    b = m2.prefill(ids, m2.new_cache(2, 20), all_positions=True)
    assert torch.equal(a, b)
    assert torch.equal(m.generate(ids, 8), m2.generate(ids, 8))


def test_mixed_group_sizes_round_trip(tmp_path):
    """Per-path quantization (config.json["quantization"][path], read at
    models/qwen2.py:279): one o_proj at group size 32 and one MLP down
    projection at 128 / 8 bits in a group-64 4-bit model survive save and load
    (as per-path entries) and decode like the original."""
    mq = importlib.import_module("mlx-server-runtime_amd")
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    ck = importlib.import_module("mlx-server-runtime_amd.checkpoint")
    cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000)
    m = q2.Qwen2Model.random(cfg, seed=5, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(11)
    w_o = (torch.randn(256, 256, generator=gen, device=DEV) * 0.02).to(torch.bfloat16)
    m.layers[0].o = q2.QLinear(*mq.quantize(w_o, 32, 4), None, 32, 4)
    w_d = (torch.randn(256, 512, generator=gen, device=DEV) * 0.02).to(torch.bfloat16)
    m.layers[1].down = q2.QLinear(*mq.quantize(w_d, 128, 8), None, 128, 8)
    ck.save(m, tmp_path)
    m2 = ck.load(tmp_path, device=DEV)
    assert (m2.layers[0].o.group_size, m2.layers[0].o.bits) == (32, 4)
    assert (m2.layers[1].down.group_size, m2.layers[1].down.bits) == (128, 8)
    ids = torch.randint(0, 1000, (2, 20), generator=gen, device=DEV)
    a = m.prefill(ids, m.new_cache(2, 20), all_positions=True)
    b = m2.prefill(ids, m2.new_cache(2, 20), all_positions=True)
    assert torch.equal(a, b)
    assert torch.equal(m.generate(ids, 8), m2.generate(ids, 8))
    ref = reference_logits(mq, m2, ids)
    assert float((b.float() - ref).abs().max() / ref.abs().max()) <= 3e-2


def test_unquantized_modules_decode(tmp_path):
    """A checkpoint whose lm_head and one o_proj are stored unquantized (no
    scales, as models/qwen2.py:316-324 leaves them): the loaded model keeps
    them bfloat16, decodes the same in graph and eager mode, and its logits
    match the float32 restatement on the same weights."""
    mq = importlib.import_module("mlx-server-runtime_amd")
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    ck = importlib.import_module("mlx-server-runtime_amd.checkpoint")
    cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000)
    m = q2.Qwen2Model.random(cfg, seed=4, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(9)
    m.lm_head = q2.DenseLinear((torch.randn(1000, 256, generator=gen, device=DEV) * 0.02)
                               .to(torch.bfloat16))
    m.layers[1].o = q2.DenseLinear((torch.randn(256, 256, generator=gen, device=DEV) * 0.01)
                                   .to(torch.bfloat16))
    ck.save(m, tmp_path)
    m2 = ck.load(tmp_path, device=DEV)
    assert isinstance(m2.lm_head, q2.DenseLinear) and isinstance(m2.layers[1].o, q2.DenseLinear)
    ids = torch.randint(0, 1000, (2, 24), generator=gen, device=DEV)
    steps = []
    toks = m2.generate(ids, 8, use_graph=False, logits_out=steps)
    assert torch.equal(toks, m2.generate(ids, 8))
    full = torch.cat([ids, toks], 1)[:, :-1]
    ref = reference_logits(mq, m2, full)
    ours = m2.prefill(full, m2.new_cache(2, full.shape[1]), all_positions=True)
    err = float((ours.float() - ref).abs().max() / ref.abs().max())
    assert err <= 3e-2, err
