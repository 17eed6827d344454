"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Bars:
* quantize, dequantize, embedding lookup: bit-exact (integer codes and
  bfloat16 bit patterns).
* quantized_matmul / gather_qmm: norm-wise relative error
  max|y - ref| / max|ref| <= 1e-2 (bfloat16 output, float32 accumulation),
  where ref is the oracle's double-precision contraction with the exact
  dequantized weights.  TOL below is that bound.
Full-size shapes (the 7B layer widths) are checked directly where the oracle is fast
(M = 1) and on a sample of rows otherwise (rows of the output depend only on
their own row of x).
"""

from __future__ import annotations

import functools
import os

import numpy as np
import pytest
import torch

from conftest import normwise_rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-2
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DEV = "cuda:0"


def bf16_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16)).view(
        torch.bfloat16).to(DEV)


def u32_dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).to(DEV)


def bits_host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def u32_host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy().view(np.uint32)


def rand_bf16(orc, rng, shape, std):
    return orc.f32_to_bf16(rng.normal(0, std, shape).astype(np.float32))


def quantized(orc, rng, N, K, bits, std=0.02):
    w = rand_bf16(orc, rng, (N, K), std)
    return orc.quantize(w, 64, bits)


def assert_close(y_dev, ref, tol=TOL):
    y = bits_host(y_dev)
    from oracle.oracle import bf16_to_f32

    err = normwise_rel_err(bf16_to_f32(y), ref)
    assert err <= tol, f"norm-wise relative error {err:.3e} > {tol}"
    return err


# ----------------------------------------------------------- quantize / deq


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("shape", [(37, 256), (5, 3584), (3, 64)])
def test_quantize_bit_exact(mq, orc, bits, shape):
    rng = np.random.default_rng(100 + bits)
    w = rand_bf16(orc, rng, shape, 0.02)
    w[0, :64] = 0                              # zero group
    w[-1, -64:] = orc.f32_to_bf16(np.float32(0.0125))  # constant group
    if shape[1] >= 128:
        w[0, 64:128] = orc.f32_to_bf16(np.abs(rng.normal(0, 1, 64)).astype(np.float32))
    wq, s, b = mq.quantize(bf16_dev(w), 64, bits)
    rq, rs, rb = orc.quantize(w, 64, bits)
    assert np.array_equal(u32_host(wq), rq)
    assert np.array_equal(bits_host(s), rs)
    assert np.array_equal(bits_host(b), rb)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("shape", [(37, 256), (64, 3584), (1, 64)])
def test_dequantize_bit_exact(mq, orc, bits, shape):
    rng = np.random.default_rng(200 + bits)
    wq, s, b = quantized(orc, rng, *shape, bits)
    out = mq.dequantize(u32_dev(wq), bf16_dev(s), bf16_dev(b), 64, bits)
    assert np.array_equal(bits_host(out), orc.dequantize(wq, s, b, 64, bits))


def test_dequantize_rounds_twice_on_gpu(mq):
    wq = np.full((1, 8), 0x33333333, np.uint32)
    s = np.array([[0x3F81]], np.uint16)   # 1.0078125
    b = np.array([[0xBC00]], np.uint16)   # -0.0078125
    out = bits_host(mq.dequantize(u32_dev(wq), bf16_dev(s), bf16_dev(b), 64, 4))
    assert np.all(out == 0x4042)          # 3.03125


@pytest.mark.parametrize("bits", [4, 8])
def test_embedding_lookup_bit_exact(mq, orc, bits):
    rng = np.random.default_rng(300 + bits)
    wq, s, b = quantized(orc, rng, 50, 256, bits)
    ids = np.array([[3, 0, 49], [7, 7, 12]], np.int32)
    out = mq.embedding_lookup(torch.from_numpy(ids).to(DEV), u32_dev(wq), bf16_dev(s),
                              bf16_dev(b), 64, bits)
    ref = orc.dequantize(wq, s, b, 64, bits)[ids.reshape(-1)].reshape(2, 3, 256)
    assert np.array_equal(bits_host(out), ref)
    bad = mq.embedding_lookup(torch.tensor([50, -1], device=DEV), u32_dev(wq), bf16_dev(s),
                              bf16_dev(b), 64, bits)
    assert np.all(bits_host(bad) == 0)


@pytest.mark.parametrize("bits", [4, 8])
def test_kat_fixtures_on_gpu(mq, orc, bits):
    kat = dict(np.load(os.path.join(GOLDEN, f"kat_affine_b{bits}.npz"), allow_pickle=False))
    wq, s, b = mq.quantize(bf16_dev(kat["w"]), 64, bits)
    assert np.array_equal(u32_host(wq), kat["wq"])
    chk = kat["scale_checked"]
    assert np.array_equal(bits_host(s)[chk], kat["scales"][chk])
    assert np.array_equal(bits_host(b), kat["biases"])
    deq = mq.dequantize(u32_dev(kat["wq"]), bf16_dev(kat["scales"]), bf16_dev(kat["biases"]),
                        64, bits)
    assert np.array_equal(orc.bf16_to_f32(bits_host(deq)), orc.bf16_to_f32(kat["deq"]))
    y = mq.quantized_matmul(bf16_dev(kat["x"]), u32_dev(kat["wq"]), bf16_dev(kat["scales"]),
                            bf16_dev(kat["biases"]), True, 64, bits)
    assert_close(y, kat["y"])
    gy = mq.gather_qmm(bf16_dev(kat["gx"]), u32_dev(kat["gwq"]), bf16_dev(kat["gscales"]),
                       bf16_dev(kat["gbiases"]), rhs_indices=torch.from_numpy(kat["rhs"]).to(DEV),
                       group_size=64, bits=bits)
    assert_close(gy, kat["gy"])


# ------------------------------------------------------------ matmul


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 9, 16, 33, 128, 130])
@pytest.mark.parametrize("KN", [(256, 200), (1024, 384)])
def test_quantized_matmul_parity(mq, orc, bits, M, KN):
    K, N = KN
    rng = np.random.default_rng(1000 * bits + M + K)
    wq, s, b = quantized(orc, rng, N, K, bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    bias = rand_bf16(orc, rng, (N,), 0.5)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64, bits,
                            bias=bf16_dev(bias))
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    assert_close(y, orc.qmm(x, wq, s, b, 64, bits, bias=bias))


@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_matmul_leading_dims_and_stream(mq, orc, bits):
    rng = np.random.default_rng(77)
    wq, s, b = quantized(orc, rng, 96, 192, bits)
    x = rand_bf16(orc, rng, (2, 3, 192), 1.0)
    side = torch.cuda.Stream(device=DEV)
    with torch.cuda.stream(side):
        y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64,
                                bits)
    side.synchronize()
    assert y.shape == (2, 3, 96)
    assert_close(y, orc.qmm(x.reshape(6, 192), wq, s, b, 64, bits).reshape(2, 3, 96))


def test_quantized_matmul_empty_and_errors(mq, orc):
    rng = np.random.default_rng(5)
    wq, s, b = quantized(orc, rng, 64, 128, 4)
    y = mq.quantized_matmul(torch.zeros(0, 128, dtype=torch.bfloat16, device=DEV), u32_dev(wq),
                            bf16_dev(s), bf16_dev(b))
    assert y.shape == (0, 64)
    with pytest.raises(ValueError):
        mq.quantized_matmul(torch.zeros(1, 64, dtype=torch.bfloat16, device=DEV), u32_dev(wq),
                            bf16_dev(s), bf16_dev(b))
    with pytest.raises(NotImplementedError):
        mq.quantized_matmul(torch.zeros(1, 128, dtype=torch.bfloat16, device=DEV), u32_dev(wq),
                            bf16_dev(s), bf16_dev(b), transpose=False)


def test_quantized_matmul_deterministic(mq, orc):
    rng = np.random.default_rng(6)
    wq, s, b = quantized(orc, rng, 512, 1024, 4)
    x = bf16_dev(rand_bf16(orc, rng, (64, 1024), 1.0))
    args = (u32_dev(wq), bf16_dev(s), bf16_dev(b))
    y1 = bits_host(mq.quantized_matmul(x, *args))
    y2 = bits_host(mq.quantized_matmul(x, *args))
    assert np.array_equal(y1, y2)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("MNK", [(9, 512, 8192), (32, 300, 4096), (100, 640, 8192),
                                 (160, 600, 16384), (128, 640, 4096), (250, 300, 3584)])
def test_skinny_split_k(mq, orc, bits, MNK):
    """Few columns and a long K: the skinny kernel splits K over blocks into a
    float32 workspace.  Checked against the oracle, run to run, and against the
    unsplit kernel (the C entry point without a workspace)."""
    import ctypes

    M, N, K = MNK
    L = mq._lib.lib()
    ws_bytes = L.mq_quantized_matmul_workspace(M, N, K, 64, bits)
    assert ws_bytes > 0
    rng = np.random.default_rng(31 * M + bits)
    wq, s, b = quantized(orc, rng, N, K, bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    bias = rand_bf16(orc, rng, (N,), 0.5)
    args = (bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64, bits)
    y = mq.quantized_matmul(*args, bias=bf16_dev(bias))
    assert_close(y, orc.qmm(x, wq, s, b, 64, bits, bias=bias))
    assert torch.equal(mq.quantized_matmul(*args, bias=bf16_dev(bias)).view(torch.int16),
                       y.view(torch.int16))
    xd, wd, sd, bd, biasd = args[0], args[1], args[2], args[3], bf16_dev(bias)
    y1 = torch.empty_like(y)
    torch.cuda.synchronize()
    rc = L.mq_quantized_matmul(xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(),
                               biasd.data_ptr(), y1.data_ptr(), M, N, K, 64, bits, 1,
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert rc == 0
    assert_close(y1, orc.qmm(x, wq, s, b, 64, bits, bias=bias))


@pytest.mark.parametrize("MNKbits", [(24, 33000, 512, 4), (32, 45000, 512, 8),
                                     (17, 60000, 512, 4), (32, 70000, 512, 4)])
def test_skinny_wide_blocks(mq, orc, MNKbits):
    """Unsplit 32-row tiles with more 128-column tiles than CUs: blocks of 5
    (33000 columns, a 40-column last block), 6 (45000) or 8 (60000) waves keep
    the block count within 256; 70000 columns fit no width and keep 4-wave
    blocks.  Checked against the oracle and run to run."""
    M, N, K, bits = MNKbits
    assert mq._lib.lib().mq_quantized_matmul_workspace(M, N, K, 64, bits) == 0  # unsplit
    rng = np.random.default_rng(N + bits)
    wq, s, b = quantized(orc, rng, N, K, bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    bias = rand_bf16(orc, rng, (N,), 0.5)
    args = (bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64, bits)
    y = mq.quantized_matmul(*args, bias=bf16_dev(bias))
    assert_close(y, orc.qmm(x, wq, s, b, 64, bits, bias=bias))
    assert torch.equal(mq.quantized_matmul(*args, bias=bf16_dev(bias)).view(torch.int16),
                       y.view(torch.int16))


@pytest.mark.parametrize("MNK", [(2048, 3584, 18944), (512, 4096, 8192), (1100, 3584, 4096)])
def test_large_tiles_split_k(mq, orc, MNK):
    """Few 256x256 tiles and a long K (the down projection of a 2048-row
    prefill): K is split over blocks into a float32 workspace.  Sampled rows
    against the oracle (rows depend only on their own row of x), bit-identical
    run to run, and the C entry point without a workspace (unsplit) agrees."""
    import ctypes

    M, N, K = MNK
    bits = 4
    L = mq._lib.lib()
    ws_bytes = L.mq_quantized_matmul_workspace(M, N, K, 64, bits)
    assert ws_bytes > 0 and ws_bytes % (M * N * 4) == 0
    rng = np.random.default_rng(M + K)
    wq, s, b = quantized(orc, rng, N, K, bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    bias = rand_bf16(orc, rng, (N,), 0.5)
    args = (bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64, bits)
    y = mq.quantized_matmul(*args, bias=bf16_dev(bias))
    rows = np.array([0, 1, M // 2 + 3, M - 1])
    ref = orc.qmm(x[rows], wq, s, b, 64, bits, bias=bias)
    assert_close(y[rows], ref)
    assert torch.equal(mq.quantized_matmul(*args, bias=bf16_dev(bias)).view(torch.int16),
                       y.view(torch.int16))
    y1 = torch.empty_like(y)
    torch.cuda.synchronize()
    rc = L.mq_quantized_matmul(args[0].data_ptr(), args[1].data_ptr(), args[2].data_ptr(),
                               args[3].data_ptr(), bf16_dev(bias).data_ptr(), y1.data_ptr(), M, N,
                               K, 64, bits, 1,
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert rc == 0
    assert_close(y1[rows], ref)


@pytest.mark.parametrize("bits", [4, 8])
def test_large_tiles_deterministic(mq, orc, bits):
    """The 256x256-tile kernels (DMA staging, register dequantization) give
    bit-identical results run to run: no stage is read before it is filled."""
    rng = np.random.default_rng(17 + bits)
    M, N, K = 2048, 4096, 1024  # 8 x 16 tiles
    wq, s, b = quantized(orc, rng, N, K, bits)
    x = bf16_dev(rand_bf16(orc, rng, (M, K), 1.0))
    args = (u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64, bits)
    first = mq.quantized_matmul(x, *args)
    for _ in range(6):
        assert torch.equal(mq.quantized_matmul(x, *args).view(torch.int16), first.view(torch.int16))
    rows = np.array([0, 777, M - 1])
    assert_close(first[torch.from_numpy(rows).to(DEV)],
                 orc.qmm(bits_host(x)[rows], wq, s, b, 64, bits))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("KN", [(3584, 18944), (18944, 3584), (3584, 4608)])
def test_decode_shapes_full_size(mq, orc, bits, KN):
    """M = 1 at the benchmark shapes (the whole output checked)."""
    K, N = KN
    rng = np.random.default_rng(4242 + bits + K)
    wq, s, b = quantized(orc, rng, N, K, bits)
    x = rand_bf16(orc, rng, (1, K), 1.0)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64, bits)
    assert_close(y, orc.qmm(x, wq, s, b, 64, bits))


@functools.lru_cache(maxsize=6)
def _sweep_weights(orc, K, N, bits):
    """Quantized N(0, 0.02) weights of one sweep shape, shared by its M cases."""
    rng = np.random.default_rng(5151 + K + N + bits)
    return quantized(orc, rng, N, K, bits)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("KN", [(3584, 18944), (18944, 3584), (3584, 4608)])
@pytest.mark.parametrize("M", [16, 128, 2048, 8192])
def test_sweep_shape_sampled_rows(mq, orc, bits, KN, M):
    """Every point of the GEMM sweep above M = 1 (M in 16, 128, 2048, 8192 x
    the three 7B shapes x both widths), each through the kernel and split plan
    it runs at that size: sampled output rows (the first, the last, and rows of
    the first and last row tiles) against the oracle."""
    K, N = KN
    wq, s, b = _sweep_weights(orc, K, N, bits)
    rng = np.random.default_rng(7 + M + K + bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64, bits)
    rows = np.unique(np.r_[0, 1, min(M, 255) - 1, M - 1, rng.integers(0, M, 5)])
    assert_close(y[torch.from_numpy(rows).to(DEV)], orc.qmm(x[rows], wq, s, b, 64, bits))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("KN", [(3584, 4608), (3584, 3584), (18944, 3584), (3584, 18944)])
@pytest.mark.parametrize("M", [300, 512])
def test_mid_m_split_plans_sampled_rows(mq, orc, bits, KN, M):
    """A prefill chunk of 300 / 512 rows at the 7B shapes: few 256 x 256 tiles,
    so the large-M GEMM splits K over blocks (up to 9 splits of the down
    projection) and the fixed-order reduce adds the partial sums; sampled rows
    (the first and last of each row tile among them) against the oracle."""
    K, N = KN
    wq, s, b = _sweep_weights(orc, K, N, bits)
    rng = np.random.default_rng(11 + M + K + bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64, bits)
    rows = np.unique(np.r_[0, 255, min(256, M - 1), M - 1, rng.integers(0, M, 4)])
    assert_close(y[torch.from_numpy(rows).to(DEV)], orc.qmm(x[rows], wq, s, b, 64, bits))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M", [512, 4096])
def test_group_tail_k_sampled_rows(mq, orc, bits, M):
    """K = 11008 (a down projection whose K is not a multiple of 512): the
    LDS-dequantizing GEMMs, 128 x 128 tiles at M = 512 (16 tiles of 256) and
    256 x 256 tiles at M = 4096 (128 tiles)."""
    K, N = 11008, 2048
    rng = np.random.default_rng(99 + M + bits)
    wq, s, b = quantized(orc, rng, N, K, bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    bias = rand_bf16(orc, rng, (N,), 0.5)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64, bits,
                            bias=bf16_dev(bias))
    rows = np.unique(np.r_[0, 255, 256, M - 1, rng.integers(0, M, 5)])
    assert_close(y[torch.from_numpy(rows).to(DEV)],
                 orc.qmm(x[rows], wq, s, b, 64, bits, bias=bias))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("MNK", [(900, 18900, 3584), (1024, 18944, 3712)])
def test_large_tiles_stream_k(mq, orc, bits, MNK):
    """296 tiles of 256 x 256: one full round of the GPU and a last round of
    40 tiles, which run as stream-K pieces whose float32 sums a reduce adds
    (with the bias).  M = 900, N = 18900: the partial last column tile, in
    every row tile, and the 132-row last row tile; K = 3712 (58 groups): the
    last 512-wide chunk holds 2 groups, so pieces end inside a chunk.  Sampled
    rows against the oracle, bit-identical results run to run, and the
    whole-tile plan (no workspace) within one bfloat16 ulp of it (plus the
    float32 reassociation error on sums that cancel)."""
    import ctypes
    M, N, K = MNK
    L = mq._lib.lib()
    need = L.mq_quantized_matmul_workspace(M, N, K, 64, bits)
    assert need >= 40 * 3 * 256 * 256 * 4, need  # the stream-K plan's pieces
    rng = np.random.default_rng(717 + bits + K)
    wq, s, b = quantized(orc, rng, N, K, bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    bias = rand_bf16(orc, rng, (N,), 0.5)
    args = (bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64, bits)
    y = mq.quantized_matmul(*args, bias=bf16_dev(bias))
    for _ in range(3):
        assert torch.equal(mq.quantized_matmul(*args, bias=bf16_dev(bias)).view(torch.int16),
                           y.view(torch.int16))
    rows = np.unique(np.r_[0, 255, 256, 767, 768, M - 1, rng.integers(0, M, 4)])
    assert_close(y[torch.from_numpy(rows).to(DEV)],
                 orc.qmm(x[rows], wq, s, b, 64, bits, bias=bias))
    whole = torch.empty_like(y)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    mq._lib.check(L.mq_quantized_matmul_ws(ptr(args[0]), ptr(args[1]), ptr(args[2]),
                                           ptr(args[3]), ptr(bf16_dev(bias)), ptr(whole), M, N,
                                           K, 64, bits, 1, None, ctypes.c_size_t(0),
                                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                  "ws")
    torch.cuda.synchronize()
    # two roundings of float32 sums that differ only in summation order: one
    # bfloat16 ulp apart, plus the reassociation error of the float32 sums,
    # which shows on results that cancel to near zero (measured: <= 6e-7
    # where max |y| ~ 7)
    mag = torch.maximum(y.float().abs(), whole.float().abs()).clamp_min(1e-30)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    slack = 2.0**-16 * float(whole.float().abs().max())
    assert bool(((y.float() - whole.float()).abs() <= ulp + slack).all())


def _random_shapes(n, seed):
    """Seeded (M, N, K, group size, bits) across every dispatch range: the
    GEMVs (M <= 8), the skinny GEMM (9..256 rows), the large-M GEMM with K
    splits, whole tiles and stream-K tails (300..3100 rows), group sizes
    32 / 64 / 128, N and M off the tile sizes."""
    rng = np.random.default_rng(seed)
    out = []
    m_ranges = [(1, 8), (9, 32), (33, 256), (257, 1100), (1500, 3100)]
    for i in range(n):
        lo, hi = m_ranges[i % len(m_ranges)]
        M = int(rng.integers(lo, hi + 1))
        gs = int(rng.choice([64, 64, 32, 128]))
        bits = int(rng.choice([4, 8]))
        K = int(rng.choice([512, 1024, 2048, 3584, 4096, 5120]))
        N = int(rng.choice([200, 1000, 2304, 4608, 9000, 18944]))
        out.append((M, N, K, gs, bits))
    return out


@pytest.mark.parametrize("M,N,K,gs,bits", _random_shapes(30, 2026))
def test_random_shapes_sampled_rows(mq, orc, M, N, K, gs, bits):
    """Seeded shapes across the dispatch: sampled rows (first, last, the row
    tile edges among them) against the oracle, with a bias."""
    print(f"random shape M={M} N={N} K={K} gs={gs} bits={bits}", flush=True)
    rng = np.random.default_rng(M * 7 + N * 3 + K + gs + bits)
    wq, s, b = orc.quantize(rand_bf16(orc, rng, (N, K), 0.02), gs, bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    bias = rand_bf16(orc, rng, (N,), 0.5)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, gs, bits,
                            bias=bf16_dev(bias))
    assert y.shape == (M, N)
    rows = np.unique(np.r_[0, M - 1, [r for r in (31, 32, 127, 128, 255, 256) if r < M],
                           rng.integers(0, M, 3)]).astype(np.int64)
    assert_close(y[torch.from_numpy(rows).to(DEV)],
                 orc.qmm(x[rows], wq, s, b, gs, bits, bias=bias))


@pytest.mark.parametrize("bits", [4, 8])
def test_large_tiles_ragged_edges(mq, orc, bits):
    """M and N that are not multiples of the 256-row tiles, with enough tiles
    (5 x 26) for the large-tile kernel: rows of the last, partial M tile and
    the last, partial N tile are among those checked."""
    M, N, K = 1100, 6500, 512
    rng = np.random.default_rng(616 + bits)
    wq, s, b = quantized(orc, rng, N, K, bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    bias = rand_bf16(orc, rng, (N,), 0.5)
    y = mq.quantized_matmul(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64, bits,
                            bias=bf16_dev(bias))
    rows = np.unique(np.r_[0, 255, 256, 1023, 1024, M - 1, rng.integers(0, M, 8)])
    assert_close(y[torch.from_numpy(rows).to(DEV)],
                 orc.qmm(x[rows], wq, s, b, 64, bits, bias=bias))


# ------------------------------------------------------------ gather_qmm


def _experts(orc, rng, E, N, K, bits):
    w = rand_bf16(orc, rng, (E, N, K), 0.02)
    return orc.quantize(w, 64, bits)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("T,sorted_", [(5, False), (64, True), (300, True), (300, False)])
def test_gather_qmm_parity(mq, orc, bits, T, sorted_):
    rng = np.random.default_rng(9000 + T + bits)
    E, N, K = 16, 192, 512
    wq, s, b = _experts(orc, rng, E, N, K, bits)
    rhs = rng.integers(0, E, T).astype(np.int32)
    if sorted_:
        rhs = np.sort(rhs)
    x = rand_bf16(orc, rng, (T, 1, K), 1.0)
    y = mq.gather_qmm(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b),
                      rhs_indices=torch.from_numpy(rhs).to(DEV), group_size=64, bits=bits,
                      sorted_indices=sorted_)
    assert y.shape == (T, 1, N)
    assert_close(y, orc.gather_qmm(x, wq, s, b, rhs, group_size=64, bits=bits))


@pytest.mark.parametrize("M", [1, 3, 12])
def test_gather_qmm_lhs_broadcast(mq, orc, M):
    """SwitchGLU's unsorted call: x [B, L, 1, M, K] against indices [B, L, k]."""
    rng = np.random.default_rng(31 + M)
    E, N, K, B, L, k = 8, 128, 256, 2, 3, 4
    wq, s, b = _experts(orc, rng, E, N, K, 4)
    x = rand_bf16(orc, rng, (B, L, 1, M, K), 1.0)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(B * L)]).reshape(B, L, k).astype(np.int32)
    y = mq.gather_qmm(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b),
                      rhs_indices=torch.from_numpy(idx).to(DEV), group_size=64, bits=4)
    assert y.shape == (B, L, k, M, N)
    lhs = np.repeat(np.arange(B * L), k).astype(np.int32)
    ref = orc.gather_qmm(x.reshape(B * L, M, K), wq, s, b, idx.reshape(-1), lhs_indices=lhs)
    assert_close(y.reshape(-1, M, N), ref)


def test_gather_qmm_out_of_range_rows_are_zero(mq, orc):
    rng = np.random.default_rng(44)
    E, N, K = 4, 64, 128
    wq, s, b = _experts(orc, rng, E, N, K, 4)
    for T in (3, 200):
        rhs = np.sort(rng.integers(0, E, T)).astype(np.int32)
        rhs[-1] = E  # out of range
        x = rand_bf16(orc, rng, (T, 1, K), 1.0)
        y = mq.gather_qmm(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b),
                          rhs_indices=torch.from_numpy(rhs).to(DEV), sorted_indices=True)
        yh = bits_host(y)
        assert np.all(yh[-1] == 0)
        ref = orc.gather_qmm(x[:-1], wq, s, b, rhs[:-1])
        assert_close(y[:-1], ref)


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_moe_shape_prefill_sampled(mq, orc, bits):
    """Qwen3-30B-A3B expert shape (E=128, N=768, K=2048), 2048 sorted rows."""
    rng = np.random.default_rng(777 + bits)
    E, N, K, T = 128, 768, 2048, 2048
    wq, s, b = _experts(orc, rng, E, N, K, bits)
    rhs = np.sort(rng.integers(0, E, T)).astype(np.int32)
    x = rand_bf16(orc, rng, (T, 1, K), 1.0)
    y = mq.gather_qmm(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b),
                      rhs_indices=torch.from_numpy(rhs).to(DEV), bits=bits, sorted_indices=True)
    rows = np.unique(np.r_[0, T - 1, rng.integers(0, T, 10)])
    ref = orc.gather_qmm(x[rows], wq, s, b, rhs[rows], bits=bits)
    assert_close(y[torch.from_numpy(rows).to(DEV)], ref)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("K,Mb", [(768, 1), (1024, 1), (768, 3)])
def test_gather_sorted_expert_segments(mq, orc, bits, K, Mb):
    """The expert-segment GEMM behind sorted gather_qmm: segments of 0, 1, 255,
    256, 257, 288, 289 and 700 batches (whole and partial 256-row tiles, empty
    experts),
    ids below 0 first and at or above E last (their rows are zero), x batches
    gathered through lhs (one of them out of range: zero rows), K of 12 groups
    (a partial scale chunk) and 16, and Mb rows per batch."""
    rng = np.random.default_rng(5 + K + Mb + bits)
    sizes = [256, 0, 1, 700, 255, 0, 257, 37, 3, 0, 90, 256, 288, 289]
    E, N = len(sizes), 320
    rhs = np.concatenate([np.full(3, -1)] + [np.full(n, e) for e, n in enumerate(sizes)]
                         + [np.full(4, E)]).astype(np.int32)
    T = rhs.shape[0]
    wq, s, b = _experts(orc, rng, E, N, K, bits)
    xb = 40
    x = rand_bf16(orc, rng, (xb, Mb, K), 1.0)
    lhs = rng.integers(0, xb, T).astype(np.int32)
    lhs[7] = xb  # out of range: its rows are zero
    y = mq.gather_qmm(bf16_dev(x), u32_dev(wq), bf16_dev(s), bf16_dev(b),
                      lhs_indices=torch.from_numpy(lhs).to(DEV),
                      rhs_indices=torch.from_numpy(rhs).to(DEV), group_size=64, bits=bits,
                      sorted_indices=True)
    assert y.shape == (T, Mb, N)
    valid = (rhs >= 0) & (rhs < E) & (lhs < xb)
    yh = bits_host(y)
    assert np.all(yh[~valid] == 0)
    ref = orc.gather_qmm(x, wq, s, b, rhs[valid], lhs_indices=lhs[valid], group_size=64,
                         bits=bits)
    assert_close(y[torch.from_numpy(np.nonzero(valid)[0]).to(DEV)], ref)


# ------------------------------------------------------------ modules


def test_switch_glu_matches_dense_reference(mq, orc):
    """SwitchGLU (models/lfm2.py:193-218) vs a float32 torch reference built from
    the exactly dequantized expert weights; both the sorted (>= 64 rows) and the
    unsorted path."""
    rng = np.random.default_rng(55)
    E, H, I, k = 16, 256, 128, 4
    mods = []
    dense = []
    for (n, kk) in ((I, H), (I, H), (H, I)):
        wq, s, b = _experts(orc, rng, E, n, kk, 4)
        mods.append(mq.nn.QuantizedSwitchLinear(u32_dev(wq), bf16_dev(s), bf16_dev(b)))
        dense.append(torch.from_numpy(orc.dequantize(wq, s, b, 64, 4, exact=True)).float())
    glu = mq.nn.SwitchGLU(*mods)
    for B, L in ((1, 2), (4, 8)):  # 8 and 128 routed rows
        xh = rand_bf16(orc, rng, (B, L, H), 1.0)
        idx = np.stack([rng.permutation(E)[:k] for _ in range(B * L)]).reshape(B, L, k)
        y = glu(bf16_dev(xh), torch.from_numpy(idx.astype(np.int64)).to(DEV))
        assert y.shape == (B, L, k, H)
        xf = torch.from_numpy(orc.bf16_to_f32(xh))
        ref = torch.empty(B, L, k, H)
        for bb in range(B):
            for ll in range(L):
                for j in range(k):
                    e = idx[bb, ll, j]
                    g = dense[0][e] @ xf[bb, ll]
                    u = dense[1][e] @ xf[bb, ll]
                    h = torch.nn.functional.silu(g) * u
                    ref[bb, ll, j] = dense[2][e] @ h
        yf = y.float().cpu()
        err = float((yf - ref).abs().max() / ref.abs().max())
        assert err <= 3 * TOL, err  # three chained bfloat16 matmuls


def test_quantized_linear_module(mq, orc):
    torch.manual_seed(0)
    lin = torch.nn.Linear(256, 96, bias=True).to(DEV)
    ql = mq.nn.QuantizedLinear.from_linear(lin, 64, 4)
    x = torch.randn(3, 256, device=DEV).to(torch.bfloat16)
    y = ql(x)
    wq, s, b = (u32_host(ql.weight), bits_host(ql.scales), bits_host(ql.biases))
    ref = orc.qmm(bits_host(x), wq, s, b, 64, 4, bias=bits_host(ql.bias))
    assert_close(y, ref)
    # nn.quantize swaps modules in place
    seq = torch.nn.Sequential(torch.nn.Linear(128, 64, bias=False), torch.nn.Embedding(10, 128)).to(DEV)
    mq.nn.quantize(seq, 64, 8)
    assert isinstance(seq[0], mq.nn.QuantizedLinear) and seq[0].bits == 8
    assert isinstance(seq[1], mq.nn.QuantizedEmbedding)
    e = seq[1](torch.tensor([1, 2], device=DEV))
    assert e.shape == (2, 128)
    assert seq[1].as_linear(e).shape == (2, 10)


def test_nn_quantize_class_predicate(mq, orc):
    """nn.quantize with the reference's class_predicate forms (models/qwen2.py:318-324,
    models/lfm2.py:579-591): False leaves a module dense, a dict overrides
    group_size/bits per path, True takes the defaults.  Each quantized layer's
    codes equal the oracle's quantization of its bfloat16 weight, and its output
    the oracle's matmul on them; the skipped layer is the original module."""
    torch.manual_seed(1)
    model = torch.nn.ModuleDict({
        "q_proj": torch.nn.Linear(256, 128, bias=True),
        "gate": torch.nn.Linear(256, 16, bias=False),
        "lm_head": torch.nn.Linear(256, 96, bias=False),
        "embed": torch.nn.Embedding(32, 256),
    }).to(DEV).to(torch.bfloat16)
    dense_gate = model["gate"]
    before = {n: model[n].weight.detach().clone() for n in ("q_proj", "lm_head", "embed")}
    seen = []

    def predicate(path, module):
        seen.append(path)
        if path == "gate":
            return False
        if path == "lm_head":
            return {"group_size": 64, "bits": 8}
        return True

    mq.nn.quantize(model, group_size=64, bits=4, class_predicate=predicate)
    assert sorted(seen) == ["embed", "gate", "lm_head", "q_proj"]
    assert model["gate"] is dense_gate
    assert isinstance(model["q_proj"], mq.nn.QuantizedLinear) and model["q_proj"].bits == 4
    assert isinstance(model["lm_head"], mq.nn.QuantizedLinear) and model["lm_head"].bits == 8
    assert isinstance(model["embed"], mq.nn.QuantizedEmbedding) and model["embed"].bits == 4
    x = torch.randn(5, 256, device=DEV).to(torch.bfloat16)
    for name, bits in (("q_proj", 4), ("lm_head", 8), ("embed", 4)):
        ql = model[name]
        wq, s, b = u32_host(ql.weight), bits_host(ql.scales), bits_host(ql.biases)
        ref_q = orc.quantize(bits_host(before[name]), 64, bits)
        assert all(np.array_equal(a, r) for a, r in zip((wq, s, b), ref_q)), name
    for name, bits in (("q_proj", 4), ("lm_head", 8)):
        ql = model[name]
        wq, s, b = u32_host(ql.weight), bits_host(ql.scales), bits_host(ql.biases)
        bias = bits_host(ql.bias) if ql.bias is not None else None
        assert_close(ql(x), orc.qmm(bits_host(x), wq, s, b, 64, bits, bias=bias))
    emb = model["embed"]
    ids = torch.tensor([0, 31, 7], device=DEV)
    wq, s, b = u32_host(emb.weight), bits_host(emb.scales), bits_host(emb.biases)
    assert np.array_equal(bits_host(emb(ids)),
                          orc.dequantize(wq, s, b, 64, 4)[[0, 31, 7]])
