"""Every output element of the large-M GEMMs and of the MoE-prefill gather
GEMMs, against a float32 GEMM (TF32 off) on the exactly dequantized weights
(the oracle's float64 q*s + b, cast to float32: q*s is exact there, + b
rounds once).

The bar is the matmul tolerance (norm-wise relative error <= 1e-2), applied
per 256 x 256 output tile -- every tile the GEMM writes is checked against
its own largest reference value, so one wrong tile (a missed stream-K piece,
a misplaced expert segment, a dropped K split) fails even when the rest of
the output is right.  The fp32 GEMM's own error (fp32 accumulation over at
most 18944 terms) is four orders of magnitude below the bar.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from test_gpu_parity import _sweep_weights, bf16_dev, rand_bf16, u32_dev

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-2
TILE = 256


@pytest.fixture(autouse=True)
def _fp32_gemm():
    prev = torch.backends.cuda.matmul.allow_tf32, torch.get_float32_matmul_precision()
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.set_float32_matmul_precision("highest")
    yield
    torch.backends.cuda.matmul.allow_tf32 = prev[0]
    torch.set_float32_matmul_precision(prev[1])


def _exact_dev(orc, wq, s, b, bits):
    return torch.from_numpy(orc.dequantize(wq, s, b, 64, bits, exact=True).astype(np.float32)).to(DEV)


def tile_errors(y: torch.Tensor, ref: torch.Tensor, tile: int = TILE) -> torch.Tensor:
    """Norm-wise relative error of each tile x tile block of a [M, N] output:
    max|y - ref| / max|ref| within the block (edge blocks partial)."""
    M, N = ref.shape
    tm, tn = -(-M // tile), -(-N // tile)
    d = torch.zeros(tm * tile, tn * tile, device=ref.device)
    r = torch.zeros_like(d)
    d[:M, :N] = (y.float() - ref).abs()
    r[:M, :N] = ref.abs()
    dm = d.reshape(tm, tile, tn, tile).amax((1, 3))
    rm = r.reshape(tm, tile, tn, tile).amax((1, 3))
    return dm / rm.clamp_min(1e-30)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("KN", [(3584, 18944), (18944, 3584), (3584, 4608)])
@pytest.mark.parametrize("M", [2048, 8192])
def test_sweep_large_m_every_tile(mq, orc, bits, KN, M):
    """The large-M sweep points (M = 2048, 8192 x the three 7B shapes x both
    widths), each through the plan it runs at that size (whole tiles,
    stream-K tails): every 256 x 256 output tile within the bar."""
    K, N = KN
    print(f"full output: M={M}, K={K}, N={N}, bits={bits}", flush=True)
    wq, s, b = _sweep_weights(orc, K, N, bits)
    rng = np.random.default_rng(7 + M + K + bits)
    x = rand_bf16(orc, rng, (M, K), 1.0)
    xd = bf16_dev(x)
    y = mq.quantized_matmul(xd, u32_dev(wq), bf16_dev(s), bf16_dev(b), True, 64, bits)
    W = _exact_dev(orc, wq, s, b, bits)
    ref = xd.float() @ W.t()
    del W
    e = tile_errors(y, ref)
    worst = float(e.max())
    print(f"  worst tile error {worst:.2e} over {e.numel()} tiles", flush=True)
    assert worst <= TOL, (worst, (e > TOL).nonzero()[:8].tolist())


@pytest.mark.parametrize("gemm", ["gate|up", "down"])
def test_gather_moe_prefill_every_row(mq, orc, gemm):
    """The MoE-prefill expert GEMMs at the Qwen3-30B-A3B shape, as the bench
    runs them: 8 x 512 tokens routed to 8 of 128 experts, 32768 pairs sorted by
    expert, gather_qmm over the sorted rows given the sort's segment offsets
    (gate|up: 1536 rows, K = 2048, x gathered by token; down: 2048 rows,
    K = 768).  Per expert, its segment's rows against x_rows @ W_e^T in
    float32, tile by tile (256 rows of the segment x 256 columns)."""
    E, k, H, inter, T = 128, 8, 2048, 768, 4096
    N, K = (2 * inter, H) if gemm == "gate|up" else (H, inter)
    print(f"gather full output: {gemm}, {T * k} pairs, N={N}, K={K}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(3)
    ids = torch.rand(T, E, generator=gen, device=DEV).topk(k, -1).indices.reshape(-1)
    order = torch.sort(ids, stable=True).indices
    rhs = ids[order].to(torch.int32).contiguous()
    offs = torch.searchsorted(rhs, torch.arange(E + 1, device=DEV, dtype=torch.int32)
                              ).to(torch.int32)
    if gemm == "gate|up":
        x = torch.randn(T, 1, K, generator=gen, device=DEV).to(torch.bfloat16)
        lhs = (order // k).to(torch.int32).contiguous()
    else:
        x = torch.randn(T * k, 1, K, generator=gen, device=DEV).to(torch.bfloat16)
        lhs = None
    w = (torch.randn(E * N, K, generator=gen, device=DEV) * 0.02).to(torch.bfloat16)
    wq, sc, bi = mq.quantize(w, 64, 4)
    del w
    y = mq.gather_qmm(x, wq.reshape(E, N, -1), sc.reshape(E, N, -1), bi.reshape(E, N, -1),
                      lhs_indices=lhs, rhs_indices=rhs, group_size=64, bits=4,
                      sorted_indices=True, expert_offsets=offs).reshape(T * k, N)
    W = _exact_dev(orc, wq.cpu().numpy().view(np.uint32),
                   sc.cpu().view(torch.int16).numpy().view(np.uint16),
                   bi.cpu().view(torch.int16).numpy().view(np.uint16), 4).reshape(E, N, K)
    xr = x.reshape(-1, K)
    src = lhs.long() if lhs is not None else torch.arange(T * k, device=DEV)
    bounds = offs.cpu().tolist()
    worst, checked = 0.0, 0
    for e in range(E):
        a, z = bounds[e], bounds[e + 1]
        if a == z:
            continue
        ref = xr[src[a:z]].float() @ W[e].t()
        worst = max(worst, float(tile_errors(y[a:z], ref).max()))
        checked += z - a
    assert checked == T * k
    print(f"  worst tile error {worst:.2e} over {checked} rows", flush=True)
    assert worst <= TOL, worst
