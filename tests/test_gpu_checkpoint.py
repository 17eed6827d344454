"""A model saved in the mlx-community layout and loaded back (checkpoint.py)
computes exactly what the original did: bit-identical logits, on the GPU."""

from __future__ import annotations

import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("kind", ["qwen2", "qwen3_moe"])
def test_save_load_round_trip_same_logits(tmp_path, kind):
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    ck = importlib.import_module("mlx-server-runtime_amd.checkpoint")
    if kind == "qwen2":
        cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000)
    else:
        cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000, attention_bias=False,
                             qk_norm=True, num_experts=8, num_experts_per_tok=2,
                             moe_intermediate_size=128)
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
