"""Group sizes 32 and 128 (the other values mx.quantize accepts; mlx-community
checkpoints carry them in config.json["quantization"], read per path at
models/qwen2.py:279 and models/lfm2.py:579-589) through the C ABI against the
oracle, as test_gpu_parity.py checks group size 64:

* quantize, dequantize, embedding lookup: bit-exact;
* quantized_matmul at decode rows (the dot2 GEMV, scales indexed per chunk by
  group), at prefill rows (the 128 x 128 MFMA GEMM, group of each thread's
  codes per step) and at the full 7B decode widths; gather_qmm unsorted (per-
  pair GEMV) and sorted (the gathered MFMA rows): norm-wise relative error
  <= 1e-2 (bfloat16 output, float32 accumulation);
* a 2-layer Qwen2-shaped decoder quantized at these group sizes, logits
  against the float32 restatement.
"""

from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from test_gpu_parity import (DEV, assert_close, bf16_dev, bits_host, rand_bf16, u32_dev,
                             u32_host)

pytestmark = pytest.mark.gpu

GROUPS = [32, 128]


def quantized_gs(orc, rng, N, K, gs, bits, std=0.02):
    return orc.quantize(rand_bf16(orc, rng, (N, K), std), gs, bits)


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("shape", [(37, 256), (5, 3584), (3, 128)])
def test_quantize_bit_exact(mq, orc, gs, bits, shape):
    rng = np.random.default_rng(110 + bits + gs)
    w = rand_bf16(orc, rng, shape, 0.02)
    w[0, :gs] = 0                                        # zero group
    w[-1, -gs:] = orc.f32_to_bf16(np.float32(0.0125))   # constant group
    if shape[1] >= 2 * gs:                               # a one-signed group
        w[1 % shape[0], gs:2 * gs] = orc.f32_to_bf16(
            np.abs(rng.normal(0, 1, gs)).astype(np.float32))
    wq, s, b = mq.quantize(bf16_dev(w), gs, bits)
    rq, rs, rb = orc.quantize(w, gs, bits)
    assert s.shape == (shape[0], shape[1] // gs)
    assert np.array_equal(u32_host(wq), rq)
    assert np.array_equal(bits_host(s), rs)
    assert np.array_equal(bits_host(b), rb)


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("shape", [(37, 256), (64, 3584), (1, 128)])
def test_dequantize_bit_exact(mq, orc, gs, bits, shape):
    rng = np.random.default_rng(210 + bits + gs)
    wq, s, b = quantized_gs(orc, rng, *shape, gs, bits)
    out = mq.dequantize(u32_dev(wq), bf16_dev(s), bf16_dev(b), gs, bits)
    assert np.array_equal(bits_host(out), orc.dequantize(wq, s, b, gs, bits))


@pytest.mark.parametrize("gs", GROUPS)
def test_embedding_lookup_bit_exact(mq, orc, gs):
    rng = np.random.default_rng(310 + gs)
    wq, s, b = quantized_gs(orc, rng, 50, 256, gs, 4)
    ids = np.array([[3, 0, 49], [7, 7, 12]], np.int32)
    out = mq.embedding_lookup(torch.from_numpy(ids).to(DEV), u32_dev(wq), bf16_dev(s),
                              bf16_dev(b), gs, 4)
    ref = orc.dequantize(wq, s, b, gs, 4)[ids.reshape(-1)].reshape(2, 3, 256)
    assert np.array_equal(bits_host(out), ref)


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 2, 3, 8, 9, 16, 130])
@pytest.mark.parametrize("KN", [(256, 200), (1024, 384)])
def test_quantized_matmul_parity(mq, orc, gs, bits, M, KN):
    K, N = KN
    rng = np.random.default_rng(1100 * bits + M + K + gs)
    wq, s, b = quantized_gs(orc, rng, N, K, gs, bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    bias = rand_bf16(orc, rng, (N,), 0.5)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, gs, bits,
                            bias=bf16_dev(bias))
    assert y.shape == (M, N)
    assert_close(y, orc.qmm(x, wq, s, b, gs, bits, bias=bias))


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("KN", [(3584, 18944), (18944, 3584)])
def test_decode_shapes_full_size(mq, orc, gs, bits, KN):
    """M = 1 at the 7B widths, the whole output."""
    K, N = KN
    rng = np.random.default_rng(4343 + bits + K + gs)
    wq, s, b = quantized_gs(orc, rng, N, K, gs, bits)
    x = rand_bf16(orc, rng, (1, K), 1.0)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, gs, bits)
    assert_close(y, orc.qmm(x, wq, s, b, gs, bits))


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
def test_prefill_sampled_rows(mq, orc, gs, bits):
    """M = 2048 on the fused-QKV shape (3584 -> 4608): sampled rows."""
    M, K, N = 2048, 3584, 4608
    rng = np.random.default_rng(77 + gs + bits)
    wq, s, b = quantized_gs(orc, rng, N, K, gs, bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, gs, bits)
    rows = np.unique(np.r_[0, 127, 128, M - 1, rng.integers(0, M, 4)])
    assert_close(y[torch.from_numpy(rows).to(DEV)], orc.qmm(x[rows], wq, s, b, gs, bits))


def test_group_32_odd_group_count(mq, orc):
    """K = 192 (six groups of 32) runs; K = 96 (three) does not fit the GEMV's
    4-byte scale words nor the 64-wide GEMM steps, and says so."""
    rng = np.random.default_rng(5)
    for M in (1, 20):
        wq, s, b = quantized_gs(orc, rng, 64, 192, 32, 4)
        x = rand_bf16(orc, rng, (M, 192), 1.0)
        y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 32, 4)
        assert_close(y, orc.qmm(x, wq, s, b, 32, 4))
    wq, s, b = quantized_gs(orc, rng, 64, 96, 32, 4)
    x = rand_bf16(orc, rng, (20, 96), 1.0)
    with pytest.raises(NotImplementedError, match="multiple of 64"):
        mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 32, 4)


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("T,sorted_", [(5, False), (300, True), (300, False)])
def test_gather_qmm_parity(mq, orc, gs, bits, T, sorted_):
    rng = np.random.default_rng(9100 + T + bits + gs)
    E, N, K = 16, 192, 512
    w = rand_bf16(orc, rng, (E * N, K), 0.02)
    wq, s, b = orc.quantize(w, gs, bits)
    wq, s, b = wq.reshape(E, N, -1), s.reshape(E, N, -1), b.reshape(E, N, -1)
    rhs = rng.integers(0, E, T).astype(np.int32)
    if sorted_:
        rhs = np.sort(rhs)
    x = rand_bf16(orc, rng, (T, 1, K), 1.0)
    y = mq.gather_qmm(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b),
                      rhs_indices=torch.from_numpy(rhs).to(DEV), group_size=gs, bits=bits,
                      sorted_indices=sorted_)
    assert y.shape == (T, 1, N)
    assert_close(y, orc.gather_qmm(x, wq, s, b, rhs, group_size=gs, bits=bits))


@pytest.mark.parametrize("gs,bits", [(32, 4), (128, 4), (128, 8)])
def test_decoder_group_sizes(gs, bits):
    """A 2-layer Qwen2-shaped decoder quantized at group size 32 / 128: its
    fused entry points report these group sizes unsupported, so the model runs
    the unfused GEMV / GEMM / SiLU * up / RMSNorm; prefill logits against the
    float32 restatement, graph decode equal to eager decode."""
    from test_gpu_qwen2 import _run

    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000, group_size=gs, bits=bits)
    toks, toks_graph, e_pre, e_dec, (match, total, worst) = _run(cfg, 2, 12, 16)
    m, _ = _run.last
    assert m.layers[0].qkv.group_size == gs
    assert torch.equal(toks, toks_graph)
    assert e_pre <= 3e-2 and e_dec <= 2e-2, (e_pre, e_dec)
    assert match >= 0.9 * total and worst <= 0.05, (match, total, worst)
