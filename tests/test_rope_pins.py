"""RoPE pinned independently of the code under test (CPU, no GPU).

The decoder's RoPE tables (qwen2.rope_tables) and rotation (qwen2.apply_rope)
feed both the decode kernels and their tests, so they are pinned here by facts
that do not restate their formula: a hand-computed known-answer rotation, the
closed-form structure of the frequencies theta^(-2i/d) of mx.fast.rope
(traditional=False; python/mlx_worker/native_mlx/models/qwen2.py:62-66,93-108)
-- first frequency exactly 1, a constant ratio theta^(-2/d) between
neighbours, freq_i * freq_(half-i) = 1/theta -- and the properties any RoPE
has: norms kept, attention scores depending only on the distance between
positions.  A wrong exponent (-i/d, -2i/(d-2)), a swapped sign or the
interleaved ("traditional") pairing fails at least one of them.
"""

from __future__ import annotations

import importlib
import math

import pytest
import torch

q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")


def _cfg(head_dim, theta, scale=1.0):
    return q2.Qwen2Config(hidden_size=head_dim, intermediate_size=8, num_attention_heads=1,
                          num_key_value_heads=1, num_hidden_layers=1, vocab_size=8,
                          rope_theta=theta, rope_scale=scale)


def test_rotation_known_answer():
    """d = 4, theta = 100, position 1: frequencies (1, 0.1); x = (1, 2, 3, 4)
    rotates the pairs (x0, x2) by 1 rad and (x1, x3) by 0.1 rad, x2 ahead of x0.
    Expected values computed by hand from cos/sin(1) and cos/sin(0.1)."""
    cos, sin = q2.rope_tables(_cfg(4, 100.0), 2, "cpu")
    out = q2.apply_rope(torch.tensor([[1.0, 2.0, 3.0, 4.0]]), cos[1:2], sin[1:2])
    expected = torch.tensor([[-1.984111, 1.590674, 2.462377, 4.179668]])
    assert torch.allclose(out, expected, atol=2e-6), out


def test_frequency_structure():
    d, theta = 128, 1e6
    cos, sin = q2.rope_tables(_cfg(d, theta), 4096, "cpu")
    half = d // 2
    # angle of pair i at position 1, read back from the tables (position 1 < pi)
    ang = torch.atan2(sin[1].double(), cos[1].double())
    assert abs(float(ang[0]) - 1.0) < 1e-7                      # freq_0 = 1
    ratio = ang[1:] / ang[:-1]
    assert torch.allclose(ratio, torch.full_like(ratio, theta ** (-2.0 / d)), rtol=1e-5)
    prod = ang[1:half] * ang[1:half].flip(0)                   # freq_i * freq_(half - i)
    assert torch.allclose(prod, torch.full_like(prod, 1.0 / theta), rtol=1e-5)
    # angle grows linearly with the position: position 4095 of pair 63
    f63 = theta ** (-(half - 1) / half)
    assert abs(float(cos[4095, 63]) - math.cos(4095 * f63)) < 1e-6
    assert abs(float(sin[4095, 63]) - math.sin(4095 * f63)) < 1e-6
    assert torch.equal(cos[0], torch.ones(half)) and torch.equal(sin[0], torch.zeros(half))


def test_linear_scaling_multiplies_positions():
    cos_s, sin_s = q2.rope_tables(_cfg(64, 1e4, scale=0.5), 64, "cpu")
    cos_1, sin_1 = q2.rope_tables(_cfg(64, 1e4), 64, "cpu")
    assert torch.equal(cos_s[2 * torch.arange(32)], cos_1[:32])
    assert torch.equal(sin_s[2 * torch.arange(32)], sin_1[:32])


@pytest.mark.parametrize("d", [64, 128])
def test_norm_and_relative_position(d):
    gen = torch.Generator().manual_seed(0)
    cos, sin = q2.rope_tables(_cfg(d, 1e6), 2048, "cpu")
    q = torch.randn(d, generator=gen, dtype=torch.float64)
    k = torch.randn(d, generator=gen, dtype=torch.float64)
    c, s = cos.double(), sin.double()

    def rot(x, p):
        return q2.apply_rope(x[None], c[p:p + 1], s[p:p + 1])[0]

    # the tables are float32, so cos^2 + sin^2 = 1 holds to ~1e-7
    for p in (0, 5, 1000, 2047):
        assert abs(float(rot(q, p).norm() / q.norm()) - 1) < 1e-6
    # <R(p) q, R(p') k> depends on p - p' only
    qk = float(q.norm() * k.norm())
    for p, pk in ((7, 3), (1503, 1499), (2047, 2043)):
        assert abs(float(rot(q, p) @ rot(k, pk) - rot(q, 4) @ rot(k, 0))) < 1e-5 * qk
    # and on the sign of the offset: the rotation is not symmetric in it
    assert abs(float(rot(q, 7) @ rot(k, 3) - rot(q, 3) @ rot(k, 7))) > 1e-3
