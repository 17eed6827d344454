"""Bits 2, 3, 5 and 6 (the other widths mx.quantize accepts; mlx-community
checkpoints carry them in config.json["quantization"], read per path at
models/qwen2.py:279,321 and models/lfm2.py:579-589) through the C ABI against
the oracle:

* quantize and dequantize (the codes as one LSB-first bit stream per row),
  the embedding lookup and the on-grid known-answer fixtures: bit-exact;
* repack_codes_u8: the one-byte codes dequantize at 8 bits to exactly what the
  stream codes dequantize to;
* quantized_matmul at one row (the codes read at their width, no workspace)
  and at skinny and large-M rows (the codes repacked into the call's
  workspace, then the 8-bit kernels), and gather_qmm sorted and unsorted:
  norm-wise relative error <= 1e-2 against the oracle (bfloat16 output,
  float32 accumulation); the one-row kernel also per element;
* a 2-layer Qwen2-shaped decoder and a Qwen3-MoE-shaped one at these widths
  against the float32 restatement, and a 3-bit checkpoint through the loader
  (which keeps linear layers' codes packed and repacks expert banks).
"""

from __future__ import annotations

import ctypes
import importlib

import numpy as np
import pytest
import torch

from test_gpu_parity import (DEV, assert_close, bf16_dev, bits_host, rand_bf16, u32_dev,
                             u32_host)
from test_oracle_pins import load_kat, unpack_stream

pytestmark = pytest.mark.gpu

WIDTHS = [2, 3, 5, 6]


@pytest.mark.parametrize("bits", WIDTHS)
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("shape", [(37, 256), (5, 3584), (3, 128)])
def test_quantize_bit_exact(mq, orc, bits, gs, shape):
    rng = np.random.default_rng(500 + 10 * bits + gs)
    w = rand_bf16(orc, rng, shape, 0.02)
    w[0, :gs] = 0                                        # zero group
    w[-1, -gs:] = orc.f32_to_bf16(np.float32(0.0125))   # constant group
    if shape[1] >= 2 * gs:                               # a one-signed group
        w[1 % shape[0], gs:2 * gs] = orc.f32_to_bf16(
            np.abs(rng.normal(0, 1, gs)).astype(np.float32))
    wq, s, b = mq.quantize(bf16_dev(w), gs, bits)
    rq, rs, rb = orc.quantize(w, gs, bits)
    assert wq.shape == (shape[0], shape[1] * bits // 32)
    assert np.array_equal(u32_host(wq), rq)
    assert np.array_equal(bits_host(s), rs)
    assert np.array_equal(bits_host(b), rb)


@pytest.mark.parametrize("bits", WIDTHS)
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_dequantize_bit_exact(mq, orc, bits, gs):
    rng = np.random.default_rng(600 + 10 * bits + gs)
    wq, s, b = orc.quantize(rand_bf16(orc, rng, (41, 384), 0.02), gs, bits)
    out = mq.dequantize(u32_dev(wq), bf16_dev(s), bf16_dev(b), gs, bits)
    assert np.array_equal(bits_host(out), orc.dequantize(wq, s, b, gs, bits))


@pytest.mark.parametrize("bits", WIDTHS)
def test_kat_fixtures_on_gpu(mq, orc, bits):
    """On-grid weights (tests/golden/make_kat.py): quantize returns the
    constructed codes, scales and biases; dequantize returns w."""
    kat = load_kat(bits)
    wq, s, b = mq.quantize(bf16_dev(kat["w"]), 64, bits)
    assert np.array_equal(u32_host(wq), kat["wq"])
    chk = kat["scale_checked"]
    assert np.array_equal(bits_host(s)[chk], kat["scales"][chk])
    assert np.array_equal(bits_host(b), kat["biases"])
    deq = mq.dequantize(u32_dev(kat["wq"]), bf16_dev(kat["scales"]), bf16_dev(kat["biases"]), 64,
                        bits)
    assert np.array_equal(bits_host(deq), kat["deq"])


@pytest.mark.parametrize("bits", WIDTHS)
def test_embedding_lookup_bit_exact(mq, orc, bits):
    rng = np.random.default_rng(700 + bits)
    wq, s, b = orc.quantize(rand_bf16(orc, rng, (50, 256), 0.02), 64, bits)
    ids = np.array([[3, 0, 49], [7, 7, 12]], np.int32)
    out = mq.embedding_lookup(torch.from_numpy(ids).to(DEV), u32_dev(wq), bf16_dev(s),
                              bf16_dev(b), 64, bits)
    ref = orc.dequantize(wq, s, b, 64, bits)[ids.reshape(-1)].reshape(2, 3, 256)
    assert np.array_equal(bits_host(out), ref)


@pytest.mark.parametrize("bits", WIDTHS)
def test_repack_keeps_codes(mq, orc, bits):
    """One byte per code, the same code values; with the same scales and
    biases the 8-bit matrix dequantizes to the stream matrix's weights."""
    rng = np.random.default_rng(800 + bits)
    wq, s, b = orc.quantize(rand_bf16(orc, rng, (19, 192), 0.02), 64, bits)
    w8 = u32_host(mq.repack_codes_u8(u32_dev(wq), bits))
    assert w8.shape == (19, 48)
    assert np.array_equal(w8.view(np.uint8).reshape(19, 192), unpack_stream(wq, bits))
    assert np.array_equal(orc.dequantize(w8, s, b, 64, 8), orc.dequantize(wq, s, b, 64, bits))


@pytest.mark.parametrize("bits", WIDTHS)
@pytest.mark.parametrize("M", [1, 3, 9, 32, 130, 600])
def test_quantized_matmul_parity(mq, orc, bits, M):
    K, N = 1024, 768
    rng = np.random.default_rng(900 + 10 * bits + M)
    wq, s, b = orc.quantize(rand_bf16(orc, rng, (N, K), 0.02), 64, bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    bias = rand_bf16(orc, rng, (N,), 0.5)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64, bits,
                            bias=bf16_dev(bias))
    assert y.shape == (M, N)
    assert_close(y, orc.qmm(x, wq, s, b, 64, bits, bias=bias))


@pytest.mark.parametrize("bits", WIDTHS)
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("K,N", [(1024, 1000), (3584, 4608), (4096, 600), (18944, 512)])
def test_one_row_at_code_width(mq, orc, bits, gs, K, N):
    """One-row matmuls read the codes at their width -- 32 codes are `bits`
    whole words of the row's bit stream -- with no workspace (K 1024-4096 at
    every group size, the long row K = 18944 at group 64/128; K = 18944 at
    group 32 takes the repacking path): every output against the oracle,
    norm-wise within 1e-2 and each element within its bfloat16 rounding
    (2^-8 relative) plus 2e-3 of the largest output; 1000 and 600 rows leave
    partial blocks."""
    L = mq._lib.lib()
    native = not (K == 18944 and gs == 32)
    assert (L.mq_quantized_matmul_workspace(1, N, K, gs, bits) == 0) == native
    print(f"one row at {bits} bits: K={K}, N={N}, group {gs}", flush=True)
    rng = np.random.default_rng(7000 + 10 * bits + gs + K + N)
    wq, s, b = orc.quantize(rand_bf16(orc, rng, (N, K), 0.02), gs, bits)
    x = rand_bf16(orc, rng, (1, K), 1.0)
    bias = rand_bf16(orc, rng, (N,), 0.5)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, gs, bits,
                            bias=bf16_dev(bias))
    ref = orc.qmm(x, wq, s, b, gs, bits, bias=bias)
    got = orc.bf16_to_f32(bits_host(y))
    scale = float(np.abs(ref).max())
    assert float(np.abs(got - ref).max()) / scale <= 1e-2
    assert bool((np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 2e-3 * scale).all())


@pytest.mark.parametrize("bits,gs", [(3, 32), (6, 128)])
def test_quantized_matmul_group_sizes(mq, orc, bits, gs):
    rng = np.random.default_rng(950 + bits + gs)
    for M, K, N in [(1, 3584, 4608), (20, 512, 256)]:
        wq, s, b = orc.quantize(rand_bf16(orc, rng, (N, K), 0.02), gs, bits)
        x = rand_bf16(orc, rng, (M, K), 1.0)
        y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, gs,
                                bits)
        assert_close(y, orc.qmm(x, wq, s, b, gs, bits))


@pytest.mark.parametrize("bits", [3, 5])
@pytest.mark.parametrize("T,sorted_", [(5, False), (300, True)])
def test_gather_qmm_parity(mq, orc, bits, T, sorted_):
    rng = np.random.default_rng(990 + T + bits)
    E, N, K = 16, 192, 512
    w = rand_bf16(orc, rng, (E * N, K), 0.02)
    wq, s, b = orc.quantize(w, 64, bits)
    wq, s, b = wq.reshape(E, N, -1), s.reshape(E, N, -1), b.reshape(E, N, -1)
    rhs = rng.integers(0, E, T).astype(np.int32)
    if sorted_:
        rhs = np.sort(rhs)
    x = rand_bf16(orc, rng, (T, 1, K), 1.0)
    y = mq.gather_qmm(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b),
                      rhs_indices=torch.from_numpy(rhs).to(DEV), group_size=64, bits=bits,
                      sorted_indices=sorted_)
    assert y.shape == (T, 1, N)
    assert_close(y, orc.gather_qmm(x, wq, s, b, rhs, group_size=64, bits=bits))


@pytest.mark.parametrize("bits", [3, 6])
def test_decoder_bits(bits):
    """A 2-layer Qwen2-shaped decoder quantized at 3 / 6 bits: its fused
    entry points report these widths unsupported, so the model runs the
    unfused kernels on codes repacked per call; prefill logits against the
    float32 restatement, graph decode equal to eager decode."""
    from test_gpu_qwen2 import _run

    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000, bits=bits)
    toks, toks_graph, e_pre, e_dec, (match, total, worst) = _run(cfg, 2, 12, 16)
    m, _ = _run.last
    assert m.layers[0].qkv.bits == bits
    assert torch.equal(toks, toks_graph)
    assert e_pre <= 3e-2 and e_dec <= 2e-2, (e_pre, e_dec)
    assert match >= 0.9 * total and worst <= 0.05, (match, total, worst)


@pytest.mark.parametrize("bits", [3, 6])
@pytest.mark.parametrize("T", [3, 64])
def test_moe_block_bits(mq, bits, T):
    """Routed experts at 3 / 6 bits (banks repacked per call): T=3 is 24
    pairs (per-pair GEMV), T=64 512 pairs (sorted segments, SiLU*up epilogue);
    against the float32 restatement given the kernel's own routing."""
    moe = importlib.import_module("mlx-server-runtime_amd.moe")
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    from qwen2_reference import moe_reference

    E, k, H, inter = 16, 8, 256, 128
    cfg = q2.Qwen2Config(H, 4 * H, 4, 2, 1, 100, bits=bits)
    g = torch.Generator(device=DEV).manual_seed(20 + bits)
    block = moe.MoEBlock(q2._random_qlinear(g, E, H, cfg, False, DEV),
                         q2._random_experts(g, E, 2 * inter, H, cfg, DEV),
                         q2._random_experts(g, E, H, inter, cfg, DEV), k, True)
    assert block.gate_up.bits == bits
    x = torch.randn(T, H, generator=g, device=DEV).to(torch.bfloat16)
    out = block(x)
    idx, _ = moe.route(block.gate(x), k, True)
    ref = moe_reference(mq, block, x, indices=idx)
    err = float((out.float() - ref).abs().max() / ref.abs().max())
    assert err < 2e-2, err


def test_moe_decoder_bits():
    """Qwen3-MoE shape at 3 bits: prefill and decode logits against the float32
    restatement with the routing teacher-forced to the model's own, max
    bounds (test_gpu_moe._forced_routing_check)."""
    mq = importlib.import_module("mlx-server-runtime_amd")
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    from test_gpu_moe import _forced_routing_check

    cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000, attention_bias=False, qk_norm=True,
                         num_experts=8, num_experts_per_tok=2, moe_intermediate_size=128, bits=3)
    m = q2.Qwen2Model.random(cfg, seed=4, device=DEV)
    ids = torch.randint(0, 1000, (3, 24), generator=torch.Generator(device=DEV).manual_seed(6),
                        device=DEV)
    _forced_routing_check(mq, m, ids, 6, "qwen3-moe 3-bit")


def test_three_bit_checkpoint_loads(tmp_path):
    """A checkpoint whose config.json says bits 3 (and one path 6): the loader
    keeps the linear layers' codes packed (decode's one-row matmuls read them
    at their width; prefill repacks them per call); logits against the 3-bit
    model it was saved from and against the float32 restatement."""
    mq = importlib.import_module("mlx-server-runtime_amd")
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    ck = importlib.import_module("mlx-server-runtime_amd.checkpoint")
    from qwen2_reference import reference_logits

    cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000, bits=3)
    m = q2.Qwen2Model.random(cfg, seed=8, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(12)
    w_d = (torch.randn(256, 512, generator=gen, device=DEV) * 0.02).to(torch.bfloat16)
    m.layers[1].down = q2.QLinear(*mq.quantize(w_d, 64, 6), None, 64, 6)
    ck.save(m, tmp_path)
    m2 = ck.load(tmp_path, device=DEV)
    assert m2.layers[0].qkv.bits == 3 and m2.layers[1].down.bits == 6
    ids = torch.randint(0, 1000, (2, 20), generator=gen, device=DEV)
    a = m.prefill(ids, m.new_cache(2, 20), all_positions=True)
    b = m2.prefill(ids, m2.new_cache(2, 20), all_positions=True)
    assert float((a.float() - b.float()).abs().max() / b.float().abs().max()) <= 1e-2
    ref = reference_logits(mq, m2, ids)
    assert float((b.float() - ref).abs().max() / ref.abs().max()) <= 3e-2


def test_noalloc_stream_bits():
    """mq_quantized_matmul_noalloc at 3 bits: the repacked codes (and any
    split-K partial sums) in the per-GPU array, bit-equal to
    mq_quantized_matmul_ws, on two calls in a row (the second smaller); a
    matrix whose repacked codes exceed the array is refused before any launch."""
    from test_zz_no_alloc import SCRATCH_BYTES, _case, _lib

    mq, L = _lib()
    _case(mq, L, 32, 1024, 2048, 3, seed=21, bias=True)
    _case(mq, L, 8, 512, 1024, 3, seed=22, bias=False)
    N, K = 4608, 4096
    assert N * K > SCRATCH_BYTES
    sixteen = ctypes.c_void_p(16)  # never dereferenced: refused before any launch
    rc = L.mq_quantized_matmul_noalloc(sixteen, sixteen, sixteen, sixteen, None, sixteen, 4, N,
                                       K, 64, 3, 1, None)
    assert rc == -1 and b"repacked" in L.mq_last_error()
