"""Ragged batches: rows with different prompt lengths and cached lengths in one
prefill call, as the reference's executor lays a step out (executor.py:335-346:
rows padded with token 0 to the longest, positions padded by repeating the
row's last; executor.py:406-414: each row's next token from its last valid
position; attention.py:406-425: padded queries attend to nothing of other
rows' and write nothing).

What is checked, on a small Qwen2-shaped decoder (and the MoE variant):
* lengths all equal to T and start given per row: bit-identical to the
  uniform prefill;
* each row of a ragged prefill against the same row prefilled alone (the
  kernels may differ with the batch's row count: within 2e-2 norm-wise) and
  against the float32 restatement of that row's tokens (within 3e-2, the
  bound the uniform decoder tests use at 2 layers);
* the pages past a row's valid tokens stay untouched;
* a mixed step (one row decoding one token over its cache, another
  prefilling) against the restatement;
* ragged greedy generation: graph decode equals eager decode, and each row's
  tokens teacher-forced against the restatement of that row.
"""

from __future__ import annotations

import importlib

import pytest
import torch

from qwen2_reference import greedy_agreement, reference_logits

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _nrel(a, b):
    return float((a.float() - b.float()).abs().max() / b.float().abs().max())


def _model(moe: bool, seed: int = 0):
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    if moe:
        cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000, attention_bias=False, qk_norm=True,
                             num_experts=8, num_experts_per_tok=2, moe_intermediate_size=128)
    else:
        cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000)
    return q2.Qwen2Model.random(cfg, seed=seed, device=DEV)


def _prompts(lens, T, vocab, seed=3):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    ids = torch.randint(1, vocab, (len(lens), T), generator=gen, device=DEV)
    for b, n in enumerate(lens):
        ids[b, n:] = 0  # the reference's padding token
    return ids


def test_ragged_equal_lengths_is_uniform():
    m = _model(False)
    ids = _prompts([10, 10, 10], 10, 1000)
    a = m.prefill(ids, m.new_cache(3, 10), all_positions=True)
    b = m.prefill(ids, m.new_cache(3, 10), start=torch.zeros(3, dtype=torch.long),
                  lengths=torch.full((3,), 10), all_positions=True)
    assert torch.equal(a, b)


@pytest.mark.parametrize("moe", [False, True])
def test_ragged_prefill_rows(moe):
    mq = importlib.import_module("mlx-server-runtime_amd")
    m = _model(moe)
    lens = [5, 12, 9, 1]
    T = max(lens)
    ids = _prompts(lens, T, m.cfg.vocab_size)
    cache = m.new_cache(len(lens), 32)
    logits = m.prefill(ids, cache, lengths=torch.tensor(lens))
    assert logits.shape == (len(lens), m.cfg.vocab_size)
    for b, n in enumerate(lens):
        solo = m.prefill(ids[b:b + 1, :n], m.new_cache(1, 32))
        assert _nrel(logits[b], solo[0]) <= 2e-2, (b, _nrel(logits[b], solo[0]))
        ref = reference_logits(mq, m, ids[b:b + 1, :n])[0, -1]
        assert _nrel(logits[b], ref) <= 3e-2, (b, _nrel(logits[b], ref))
        # nothing written past the row's tokens (the cache starts zeroed)
        past = cache.slots(torch.full((32 - n,), b, device=DEV), torch.arange(n, 32, device=DEV))
        flat = cache.k[0].view(-1, cache.kv_heads, cache.head_dim)
        assert not flat[past].any()


@pytest.mark.parametrize("moe", [False, True])
def test_mixed_prefill_decode_step(moe):
    """Row 0 has 20 cached tokens and decodes one; row 1 prefills 12 from
    scratch; row 2 appends 4 tokens to 7 cached ones -- one call."""
    mq = importlib.import_module("mlx-server-runtime_amd")
    m = _model(moe, seed=1)
    full = _prompts([21, 12, 11], 21, m.cfg.vocab_size, seed=5)
    cache = m.new_cache(3, 48)
    # the cached parts: row 0's first 20 tokens, row 2's first 7
    m.prefill(full[0:1, :20], cache, rows=torch.tensor([0]))
    m.prefill(full[2:3, :7], cache, rows=torch.tensor([2]))
    starts = torch.tensor([20, 0, 7])
    lens = torch.tensor([1, 12, 4])
    step = torch.zeros(3, 12, dtype=torch.long, device=DEV)
    step[0, :1] = full[0, 20:21]
    step[1, :12] = full[1, :12]
    step[2, :4] = full[2, 7:11]
    logits = m.prefill(step, cache, start=starts, lengths=lens)
    for b, total in enumerate([21, 12, 11]):
        ref = reference_logits(mq, m, full[b:b + 1, :total])[0, -1]
        assert _nrel(logits[b], ref) <= 3e-2, (b, _nrel(logits[b], ref))


@pytest.mark.parametrize("moe", [False, True])
def test_ragged_generate(moe):
    mq = importlib.import_module("mlx-server-runtime_amd")
    m = _model(moe, seed=2)
    lens = [6, 14, 10]
    T, n = max(lens), 12
    ids = _prompts(lens, T, m.cfg.vocab_size, seed=7)
    L = torch.tensor(lens)
    steps = []
    toks = m.generate(ids, n, use_graph=False, logits_out=steps, lengths=L)
    assert torch.equal(toks, m.generate(ids, n, lengths=L))
    match = total = 0
    worst = 0.0
    for b, p in enumerate(lens):
        full = torch.cat([ids[b, :p], toks[b, :-1]])[None]
        ref = reference_logits(mq, m, full)
        mb, tb, wb = greedy_agreement(ref, p, toks[b:b + 1])
        match, total, worst = match + mb, total + tb, max(worst, wb)
        # the first token follows the row's own last prompt token
        assert _nrel(steps[0][b], ref[0, p - 1]) <= 3e-2
    assert match >= 0.9 * total and worst <= 0.05, (match, total, worst)
