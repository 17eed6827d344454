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
* the skinny MFMA GEMM (9..256 rows: unsplit, split-K, wide blocks, 64- and
  128-row tiles) against the oracle, and bit for bit against itself at group
  size 64 on scales that repeat across groups (a group-32 matrix whose pairs
  of groups share a scale and bias is the group-64 matrix of those values; a
  group-128 matrix is the group-64 matrix with every value twice), so a
  misplaced group index shows as a changed bit;
* the fused entry points at these group sizes (SwiGLU: one-row GEMV, dot2
  GEMV, skinny split and direct, large-M epilogue; skinny + residual +
  RMSNorm; RMSNorm + GEMV; gathered SwiGLU; the MoE segment GEMM and its
  SwiGLU form), bit for bit against the unfused calls;
* the large-M GEMM (whole tiles, K splits, stream-K, group counts ending
  mid-chunk) against the oracle on sampled rows, and bit for bit against
  group size 64 on repeated scales where the plans agree;
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


# (M, N, K): split-K 32-row tiles, unsplit ones, 5-wave blocks, 64-row tiles
# split, 128-row tiles split, a 200-row tail of 64-row tiles, 256 rows
SKINNY = [(16, 512, 8192), (32, 16500, 1024), (24, 33000, 512), (64, 640, 4096),
          (128, 640, 8192), (200, 600, 3584), (256, 4608, 3584)]


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("MNK", SKINNY)
def test_skinny_group_sizes_against_oracle(mq, orc, gs, bits, MNK):
    """9..256 rows take the skinny GEMM at every group size, with the plan of
    group size 64 (same workspace); every output against the oracle."""
    M, N, K = MNK
    L = mq._lib.lib()
    assert L.mq_quantized_matmul_workspace(M, N, K, gs, bits) == \
        L.mq_quantized_matmul_workspace(M, N, K, 64, bits)
    print(f"skinny gs={gs} bits={bits} M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + N + K + gs + bits)
    wq, s, b = quantized_gs(orc, rng, N, K, gs, bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    bias = rand_bf16(orc, rng, (N,), 0.5)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, gs, bits,
                            bias=bf16_dev(bias))
    assert_close(y, orc.qmm(x, wq, s, b, gs, bits, bias=bias))


def _expanded(orc, rng, N, K, gs, bits):
    """Codes with scales and biases at group size gs and the same weights at
    group size 64: group 32 from group-64 values repeated, group 128 repeated
    into group 64.  Returns (wq, s_gs, b_gs, s64, b64)."""
    if gs == 32:
        wq, s64, b64 = quantized_gs(orc, rng, N, K, 64, bits)
        return wq, np.repeat(s64, 2, axis=1), np.repeat(b64, 2, axis=1), s64, b64
    wq, s, b = quantized_gs(orc, rng, N, K, 128, bits)
    return wq, s, b, np.repeat(s, 2, axis=1), np.repeat(b, 2, axis=1)


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("MNK", SKINNY)
def test_skinny_repeated_scales_equal_group_64(mq, orc, gs, bits, MNK):
    M, N, K = MNK
    print(f"skinny expand gs={gs} bits={bits} M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(7 * M + N + K + gs + bits)
    wq, sg, bg, s64, b64 = _expanded(orc, rng, N, K, gs, bits)
    x = bf16_dev(rand_bf16(orc, rng, (M, K), 1.0))
    bias = bf16_dev(rand_bf16(orc, rng, (N,), 0.5))
    wd = u32_dev(wq)
    y = mq.quantized_matmul(x, wd, bf16_dev(sg), bf16_dev(bg), True, gs, bits, bias=bias)
    y64 = mq.quantized_matmul(x, wd, bf16_dev(s64), bf16_dev(b64), True, 64, bits, bias=bias)
    assert torch.equal(y.view(torch.int16), y64.view(torch.int16))


def _fused():
    return (importlib.import_module("mlx-server-runtime_amd.core"),
            importlib.import_module("mlx-server-runtime_amd.decode_ops"))


# (M, N out, K): the one-row GEMV (4-bit), the dot2 GEMV, the skinny split
# plan with the SwiGLU reduce, the unsplit one with SwiGLU in its epilogue
SWIGLU = [(1, 9472, 3584), (2, 2304, 3584), (16, 512, 3584), (32, 9472, 3584)]


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("MNK", SWIGLU)
def test_swiglu_group_sizes_equal_unfused(mq, orc, gs, bits, MNK):
    M, N, K = MNK
    core, ops = _fused()
    assert core.swiglu_supported(M, N, K, gs, bits)
    print(f"swiglu gs={gs} bits={bits} M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + N + gs + bits)
    wq, s, b = quantized_gs(orc, rng, 2 * N, K, gs, bits)
    x = bf16_dev(rand_bf16(orc, rng, (M, K), 1.0))
    args = (u32_dev(wq), bf16_dev(s), bf16_dev(b))
    y = core.quantized_matmul_swiglu(x, *args, gs, bits)
    ref = ops.silu_mul(mq.quantized_matmul(x, *args, True, gs, bits))
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
def test_add_rms_norm_group_sizes_equal_unfused(mq, orc, gs, bits):
    """The down projection at 16 rows (split K) with the residual add and
    RMSNorm in the reduce."""
    M, N, K = 16, 3584, 18944
    core, ops = _fused()
    assert core.add_norm_supported(M, N, K, gs, bits)
    rng = np.random.default_rng(99 + gs + bits)
    wq, s, b = quantized_gs(orc, rng, N, K, gs, bits)
    x = bf16_dev(rand_bf16(orc, rng, (M, K), 1.0))
    res = bf16_dev(rand_bf16(orc, rng, (M, N), 1.0))
    nw = bf16_dev(orc.f32_to_bf16((rng.random(N) + 0.5).astype(np.float32)))
    bias = bf16_dev(rand_bf16(orc, rng, (N,), 0.5))
    args = (u32_dev(wq), bf16_dev(s), bf16_dev(b))
    out, h = core.quantized_matmul_add_rms_norm(x, *args, res, nw, 1e-6, bias=bias,
                                              group_size=gs, bits=bits)
    y = mq.quantized_matmul(x, *args, True, gs, bits, bias=bias)
    ref_out, ref_h = ops.rms_norm(y, nw, 1e-6, residual=res)
    assert torch.equal(h.view(torch.int16), ref_h.view(torch.int16))
    assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("NK", [(4608, 3584), (3584, 5120)])
@pytest.mark.parametrize("swiglu", [False, True])
def test_rms_norm_qmm_group_sizes_equal_unfused(mq, orc, gs, bits, NK, swiglu):
    """One row: RMSNorm (with a residual) then the GEMV or its SwiGLU form."""
    N, K = NK
    core, ops = _fused()
    assert core.rms_norm_qmm_supported(1, N, K, gs, bits, swiglu)
    rng = np.random.default_rng(N + K + gs + bits + swiglu)
    wq, s, b = quantized_gs(orc, rng, 2 * N if swiglu else N, K, gs, bits)
    a = bf16_dev(rand_bf16(orc, rng, (1, K), 1.0))
    res = bf16_dev(rand_bf16(orc, rng, (1, K), 1.0))
    nw = bf16_dev(orc.f32_to_bf16((rng.random(K) + 0.5).astype(np.float32)))
    bias = None if swiglu else bf16_dev(rand_bf16(orc, rng, (N,), 0.5))
    args = (u32_dev(wq), bf16_dev(s), bf16_dev(b))
    y, h = core.rms_norm_quantized_matmul(a, nw, 1e-6, *args, bias, res, gs, bits, swiglu)
    xn, ref_h = ops.rms_norm(a, nw, 1e-6, residual=res)
    assert torch.equal(h.view(torch.int16), ref_h.view(torch.int16))
    if swiglu:
        ref = ops.silu_mul(mq.quantized_matmul(xn, *args, True, gs, bits))
    else:
        ref = mq.quantized_matmul(xn, *args, True, gs, bits, bias=bias)
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
def test_gather_swiglu_group_sizes_equal_unfused(mq, orc, gs, bits):
    """A decode step's (token, expert) pairs: 8 tokens x top-4 of 16 experts."""
    core, ops = _fused()
    E, N, K, T = 16, 768, 2048, 32
    assert core.gather_swiglu_supported(T, 1, N, K, gs, bits)
    rng = np.random.default_rng(4242 + gs + bits)
    wq, s, b = quantized_gs(orc, rng, E * 2 * N, K, gs, bits)
    wq, s, b = wq.reshape(E, 2 * N, -1), s.reshape(E, 2 * N, -1), b.reshape(E, 2 * N, -1)
    x = bf16_dev(rand_bf16(orc, rng, (8, 1, K), 1.0))
    lhs = torch.arange(8, device=DEV, dtype=torch.int32).repeat_interleave(4)
    rhs = torch.from_numpy(rng.integers(0, E, T).astype(np.int32)).to(DEV)
    args = (u32_dev(wq), bf16_dev(s), bf16_dev(b))
    y = core.gather_qmm_swiglu(x, *args, lhs, rhs, gs, bits)
    ref = ops.silu_mul(mq.gather_qmm(x, *args, lhs_indices=lhs, rhs_indices=rhs, group_size=gs,
                                     bits=bits))
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


# Large-M GEMM plans that are the same at every group size: every tile whole
# (144 tiles), K split 8 ways (K a multiple of 1024, 32 tiles)
LARGE_SAME_PLAN = [(2048, 4608, 3584), (512, 4096, 8192)]


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("MNK", LARGE_SAME_PLAN)
def test_large_m_repeated_scales_equal_group_64(mq, orc, gs, bits, MNK):
    M, N, K = MNK
    L = mq._lib.lib()
    assert L.mq_quantized_matmul_workspace(M, N, K, gs, bits) == \
        L.mq_quantized_matmul_workspace(M, N, K, 64, bits)
    print(f"large expand gs={gs} bits={bits} M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(3 * M + N + K + gs + bits)
    wq, sg, bg, s64, b64 = _expanded(orc, rng, N, K, gs, bits)
    x = bf16_dev(rand_bf16(orc, rng, (M, K), 1.0))
    bias = bf16_dev(rand_bf16(orc, rng, (N,), 0.5))
    wd = u32_dev(wq)
    y = mq.quantized_matmul(x, wd, bf16_dev(sg), bf16_dev(bg), True, gs, bits, bias=bias)
    y64 = mq.quantized_matmul(x, wd, bf16_dev(s64), bf16_dev(b64), True, 64, bits, bias=bias)
    assert torch.equal(y.view(torch.int16), y64.view(torch.int16))


# (M, N, K): stream-K last round (296 tiles), K split (28 tiles), a ragged
# 600-row launch, group counts that end mid-chunk (K = 2112 at group size 32,
# 66 groups; K = 3584 at 128, 28 groups)
LARGE = [(1024, 18944, 3584), (512, 3584, 18944), (600, 4608, 3584), (1024, 4608, 2112)]


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("MNK", LARGE)
def test_large_m_group_sizes_sampled_rows(mq, orc, gs, bits, MNK):
    M, N, K = MNK
    if K % (2 * gs):
        pytest.skip("K is not an even number of groups of 128")
    print(f"large gs={gs} bits={bits} M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M + 3 * N + K + gs + bits)
    wq, s, b = quantized_gs(orc, rng, N, K, gs, bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    bias = rand_bf16(orc, rng, (N,), 0.5)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, gs, bits,
                            bias=bf16_dev(bias))
    rows = np.unique(np.r_[0, 255, 256, M - 1, rng.integers(0, M, 4)])
    assert_close(y[torch.from_numpy(rows).to(DEV)], orc.qmm(x[rows], wq, s, b, gs, bits,
                                                            bias=bias))


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
def test_large_m_swiglu_group_sizes_equal_unfused(mq, orc, gs, bits):
    """Prefill gate|up (2048 rows, 2 x 4096 x 3584: 256 whole tiles, no
    stream-K round) with SiLU * up in the GEMM's epilogue."""
    M, N, K = 2048, 4096, 3584
    core, ops = _fused()
    assert core.swiglu_supported(M, N, K, gs, bits)
    rng = np.random.default_rng(2048 + gs + bits)
    wq, s, b = quantized_gs(orc, rng, 2 * N, K, gs, bits)
    x = bf16_dev(rand_bf16(orc, rng, (M, K), 1.0))
    args = (u32_dev(wq), bf16_dev(s), bf16_dev(b))
    y = core.quantized_matmul_swiglu(x, *args, gs, bits)
    ref = ops.silu_mul(mq.quantized_matmul(x, *args, True, gs, bits))
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("gs", GROUPS)
@pytest.mark.parametrize("bits", [4, 8])
def test_gather_segments_group_sizes(mq, orc, gs, bits):
    """MoE prefill: 600 (token, expert) rows sorted by expert over 16 experts
    (2 x 768 x 2048 gate|up banks) through the segment GEMM: the plain form
    against the oracle on sampled rows, the SwiGLU form bit for bit against
    silu_mul of the plain one."""
    core, ops = _fused()
    E, N, K, T = 16, 768, 2048, 600
    assert core.gather_segments_supported(T, 1, N, K, E, T, gs, bits, swiglu=True)
    rng = np.random.default_rng(600 + gs + bits)
    wq, s, b = quantized_gs(orc, rng, E * 2 * N, K, gs, bits)
    wq, s, b = wq.reshape(E, 2 * N, -1), s.reshape(E, 2 * N, -1), b.reshape(E, 2 * N, -1)
    rhs = np.sort(rng.integers(0, E, T)).astype(np.int32)
    offs = np.searchsorted(rhs, np.arange(E + 1)).astype(np.int32)
    xh = rand_bf16(orc, rng, (T, 1, K), 1.0)
    x = bf16_dev(xh)
    rhs_d, offs_d = torch.from_numpy(rhs).to(DEV), torch.from_numpy(offs).to(DEV)
    args = (u32_dev(wq), bf16_dev(s), bf16_dev(b))
    y = core.gather_qmm(x, *args, rhs_indices=rhs_d, group_size=gs, bits=bits,
                        sorted_indices=True, expert_offsets=offs_d)
    rows = np.unique(np.r_[0, T - 1, rng.integers(0, T, 6)])
    assert_close(y[torch.from_numpy(rows).to(DEV)],
                 orc.gather_qmm(xh[rows], wq, s, b, rhs[rows], group_size=gs, bits=bits))
    ys = core.gather_qmm_swiglu(x, *args, None, rhs_d, gs, bits, expert_offsets=offs_d)
    assert torch.equal(ys.view(torch.int16), ops.silu_mul(y).view(torch.int16))


@pytest.mark.parametrize("gs,bits", [(32, 4), (128, 4), (128, 8)])
def test_decoder_group_sizes(gs, bits):
    """A 2-layer Qwen2-shaped decoder quantized at group size 32 / 128 (the
    fused decode entry points take these group sizes); prefill logits against
    the float32 restatement, graph decode equal to eager decode."""
    from test_gpu_qwen2 import _run

    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    cfg = q2.Qwen2Config(256, 512, 4, 2, 2, 1000, group_size=gs, bits=bits)
    toks, toks_graph, e_pre, e_dec, (match, total, worst) = _run(cfg, 2, 12, 16)
    m, _ = _run.last
    assert m.layers[0].qkv.group_size == gs
    assert torch.equal(toks, toks_graph)
    assert e_pre <= 3e-2 and e_dec <= 2e-2, (e_pre, e_dec)
    assert match >= 0.9 * total and worst <= 0.05, (match, total, worst)
