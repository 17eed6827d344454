"""The one-row 4-bit GEMV for 16-lane rows (mq_qmv1.hip) against the general
GEMV kernel it replaces on those shapes, bit for bit.

The general kernel still runs the gathered GEMV: gather_qmm of one expert
(rhs = [0]) at one row takes the same lane layout (16 lanes per row, one row
per lane group, K split into the same chunks) and the same arithmetic, so
its output is the reference for the plain call; gather_qmm_swiglu likewise
for the SwiGLU form.  The RMSNorm-input form must equal rms_norm then the
plain GEMV, bit for bit (the norm is computed in rmsnorm_kernel's element
mapping and order).  Shapes: K from 1024 to 4096 (2 to 8 chunks per lane),
row counts that leave a partial last block, the 7B gate/up shape and its LM
head; all with N * K >= 2^25 (smaller one-row matmuls take the matrix-core
GEMV).
"""

from __future__ import annotations

import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# N * K >= 2^25: smaller one-row matmuls run the matrix-core GEMV
SHAPES = [(3584, 18944), (4096, 14336), (1024, 40000), (2048, 18008), (3072, 12288),
          (2560, 14004)]


def _mods():
    return (importlib.import_module("mlx-server-runtime_amd.core"),
            importlib.import_module("mlx-server-runtime_amd.decode_ops"))


def _weights(core, N, K, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    return (*core.quantize(w, 64, 4), g)


@pytest.mark.parametrize("K,N", SHAPES)
def test_plain_equals_general_kernel(K, N):
    core, _ = _mods()
    print(f"qmv1 plain: K={K}, N={N}", flush=True)
    wq, sc, bi, g = _weights(core, N, K, K + N)
    x = torch.randn(1, K, generator=g, device=DEV).to(torch.bfloat16)
    y = core.quantized_matmul(x, wq, sc, bi, True, 64, 4)
    ref = core.gather_qmm(x.reshape(1, 1, K), wq[None], sc[None], bi[None],
                          rhs_indices=torch.zeros(1, dtype=torch.int32, device=DEV),
                          group_size=64, bits=4)
    assert torch.equal(y, ref.reshape(1, N))


@pytest.mark.parametrize("K,N", [(3584, 18944), (2048, 8192), (4096, 8200)])
def test_swiglu_equals_general_kernel(K, N):
    """The fused gate|up (2N rows) with SiLU * up: equal to the general
    kernel's gathered SwiGLU GEMV and to silu_mul of the plain product."""
    core, ops = _mods()
    print(f"qmv1 swiglu: K={K}, N={N}", flush=True)
    wq, sc, bi, g = _weights(core, 2 * N, K, 3 * K + N)
    x = torch.randn(1, K, generator=g, device=DEV).to(torch.bfloat16)
    assert core.swiglu_supported(1, N, K, 64, 4)
    y = core.quantized_matmul_swiglu(x, wq, sc, bi, 64, 4)
    ref = core.gather_qmm_swiglu(x.reshape(1, 1, K), wq[None], sc[None], bi[None], None,
                                 torch.zeros(1, dtype=torch.int32, device=DEV), 64, 4)
    assert torch.equal(y, ref.reshape(1, N))
    assert torch.equal(y, ops.silu_mul(core.quantized_matmul(x, wq, sc, bi, True, 64, 4)))


@pytest.mark.parametrize("K,N", [(3584, 18944), (3584, 152064), (2048, 18008)])
@pytest.mark.parametrize("with_res", [False, True])
def test_norm_input_equals_norm_then_gemv(K, N, with_res):
    core, ops = _mods()
    print(f"qmv1 norm: K={K}, N={N}, residual={with_res}", flush=True)
    wq, sc, bi, g = _weights(core, N, K, 5 * K + N)
    a = torch.randn(1, K, generator=g, device=DEV).to(torch.bfloat16)
    res = torch.randn(1, K, generator=g, device=DEV).to(torch.bfloat16) if with_res else None
    nw = (torch.rand(K, generator=g, device=DEV) + 0.5).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g, device=DEV) * 0.1).to(torch.bfloat16)
    y, h = core.rms_norm_quantized_matmul(a, nw, 1e-6, wq, sc, bi, bias, res, 64, 4)
    if with_res:
        x, ref_h = ops.rms_norm(a, nw, 1e-6, residual=res)
        assert torch.equal(h, ref_h)
    else:
        x = ops.rms_norm(a, nw, 1e-6)
    assert torch.equal(y, core.quantized_matmul(x, wq, sc, bi, True, 64, 4, bias=bias))


@pytest.mark.parametrize("K,N", [(3584, 4608), (3584, 3584), (3584, 512), (2048, 4096),
                                 (1024, 1000), (4096, 24)])
def test_small_matrices_against_oracle(orc, K, N):
    """Smaller one-row matmuls (where the matrix-core GEMV used to run) take
    the one-row kernel too: against the oracle's float64 contraction with the
    exactly dequantized weights (norm-wise 1e-2), with QuantizedLinear's
    bias; the SwiGLU and RMSNorm forms on the same matrices bit-equal to the
    unfused calls."""
    import numpy as np
    core, ops = _mods()
    print(f"qmv1 small: K={K}, N={N}", flush=True)
    rng = np.random.default_rng(K + 7 * N)
    w = orc.f32_to_bf16(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    wq, s, b = orc.quantize(w, 64, 4)
    x = orc.f32_to_bf16(rng.normal(0, 1, (1, K)).astype(np.float32))
    bias = orc.f32_to_bf16(rng.normal(0, 0.1, (N,)).astype(np.float32))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(DEV)
    wqd = torch.from_numpy(wq.view(np.int32)).to(DEV)
    y = core.quantized_matmul(dev(x), wqd, dev(s), dev(b), True, 64, 4, bias=dev(bias))
    ref = orc.qmm(x, wq, s, b, 64, 4, bias=bias)
    got = orc.bf16_to_f32(y.cpu().view(torch.int16).numpy().view(np.uint16))
    assert float(np.abs(got - ref).max() / np.abs(ref).max()) <= 1e-2
    if N % 16 == 0:  # silu_mul takes widths that are multiples of 8
        h = N // 2
        assert torch.equal(core.quantized_matmul_swiglu(dev(x), wqd, dev(s), dev(b), 64, 4),
                           ops.silu_mul(core.quantized_matmul(dev(x), wqd, dev(s), dev(b), True,
                                                              64, 4)))
        assert core.swiglu_supported(1, h, K, 64, 4)
    nw = dev(orc.f32_to_bf16((rng.random(K) + 0.5).astype(np.float32)))
    yn, _ = core.rms_norm_quantized_matmul(dev(x), nw, 1e-6, wqd, dev(s), dev(b), dev(bias), None,
                                           64, 4)
    xn = ops.rms_norm(dev(x), nw, 1e-6)
    assert torch.equal(yn, core.quantized_matmul(xn, wqd, dev(s), dev(b), True, 64, 4,
                                                 bias=dev(bias)))


@pytest.mark.parametrize("gs", [64, 128])
@pytest.mark.parametrize("K,N", [(18944, 3584), (14336, 4096), (13824, 1000)])
def test_long_rows_against_oracle(orc, gs, K, N):
    """Down projections' long rows (27, 28 and 37 chunks per lane, codes 8
    ahead) in the plain one-row form: every output against the oracle's
    float64 contraction of the exactly dequantized weights -- norm-wise within
    1e-2 and each element within its bfloat16 rounding (2^-8 relative) plus
    2e-3 of the largest output (float32 accumulation over K terms) -- with
    QuantizedLinear's bias; 1000 rows leave a partial last block.  The SwiGLU
    and RMSNorm forms do not take these rows."""
    import numpy as np
    core, _ = _mods()
    print(f"qmv1 long rows: K={K}, N={N}, group {gs}", flush=True)
    rng = np.random.default_rng(K + N + gs)
    w = orc.f32_to_bf16(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    wq, s, b = orc.quantize(w, gs, 4)
    x = orc.f32_to_bf16(rng.normal(0, 1, (1, K)).astype(np.float32))
    bias = orc.f32_to_bf16(rng.normal(0, 0.1, (N,)).astype(np.float32))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(DEV)
    y = core.quantized_matmul(dev(x), torch.from_numpy(wq.view(np.int32)).to(DEV), dev(s), dev(b),
                              True, gs, 4, bias=dev(bias))
    ref = orc.qmm(x, wq, s, b, gs, 4, bias=bias)
    got = orc.bf16_to_f32(y.cpu().view(torch.int16).numpy().view(np.uint16))
    scale = float(np.abs(ref).max())
    assert float(np.abs(got - ref).max()) / scale <= 1e-2
    assert bool((np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 2e-3 * scale).all())
    assert not core.swiglu_supported(1, N // 2, K, gs, 4)
    assert not core.rms_norm_qmm_supported(1, N, K, gs, 4)
