"""mq_quantized_matmul_noalloc (split-K partial sums in the library's own
per-GPU device array) against mq_quantized_matmul_ws (a caller workspace),
through the C ABI: bit-identical outputs -- the same kernels, split plan and
fixed-order reduce -- on two calls in a row, the second smaller; shapes
whose plan needs more than the array are refused before any launch."""

from __future__ import annotations

import ctypes
import importlib

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
SCRATCH_BYTES = 16 << 20


def _lib():
    mq = importlib.import_module("mlx-server-runtime_amd")
    return mq, mq._lib.lib()


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _case(mq, L, M, N, K, bits, seed, bias, with_ws=True):
    core = importlib.import_module("mlx-server-runtime_amd.core")
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    wq, sc, bi = core.quantize(w, 64, bits)
    x = torch.randn(M, K, generator=g, device=DEV).to(torch.bfloat16)
    bv = (torch.randn(N, generator=g, device=DEV) * 0.1).to(torch.bfloat16) if bias else None
    need = L.mq_quantized_matmul_workspace(M, N, K, 64, bits) if with_ws else 0
    assert need <= SCRATCH_BYTES, need
    ws = torch.empty(need, dtype=torch.uint8, device=DEV) if need else None
    ref = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    mq._lib.check(L.mq_quantized_matmul_ws(_ptr(x), _ptr(wq), _ptr(sc), _ptr(bi), _ptr(bv),
                                           _ptr(ref), M, N, K, 64, bits, 1, _ptr(ws),
                                           ctypes.c_size_t(need), stream), "ws")
    mq._lib.check(L.mq_quantized_matmul_noalloc(_ptr(x), _ptr(wq), _ptr(sc), _ptr(bi), _ptr(bv),
                                                _ptr(out), M, N, K, 64, bits, 1, stream),
                  "noalloc")
    torch.cuda.synchronize()
    assert torch.equal(out, ref), (M, N, K, bits)


@pytest.mark.parametrize("bits", [4, 8])
def test_noalloc_equals_workspace_entry(bits):
    """The down projection at 128 rows (14 MiB of partial sums), then the same
    matrix at 32 rows (a smaller plan reusing the array), the fused QKV at 16
    rows, each bit-equal to the workspace entry; a GEMV that needs no scratch
    (M = 1) passes through unchanged."""
    mq, L = _lib()
    print(f"noalloc bits={bits}: M=128 then M=32, N=3584, K=18944", flush=True)
    _case(mq, L, 128, 3584, 18944, bits, seed=1, bias=False)
    _case(mq, L, 32, 3584, 18944, bits, seed=2, bias=True)
    _case(mq, L, 16, 4608, 3584, bits, seed=3, bias=True)
    assert L.mq_quantized_matmul_workspace(1, 18944, 3584, 64, bits) == 0
    _case(mq, L, 1, 18944, 3584, bits, seed=4, bias=False)


@pytest.mark.parametrize("bits", [4, 8])
def test_noalloc_stream_k_beyond_the_array_runs_whole_tiles(bits):
    """M = 1024, 3584 -> 18944 (296 tiles of 256 x 256): the workspace entry's
    stream-K plan wants more than the array holds, so the no-allocation entry
    runs every tile whole -- bit-equal to the workspace entry without a
    workspace."""
    mq, L = _lib()
    M, N, K = 1024, 18944, 3584
    print(f"noalloc bits={bits}: M={M}, N={N}, K={K} (stream-K plan beyond the array)", flush=True)
    assert L.mq_quantized_matmul_workspace(M, N, K, 64, bits) > SCRATCH_BYTES
    _case(mq, L, M, N, K, bits, seed=5, bias=True, with_ws=False)


def test_noalloc_refuses_beyond_the_array():
    mq, L = _lib()
    M, N, K = 2048, 3584, 18944
    assert L.mq_quantized_matmul_workspace(M, N, K, 64, 4) > SCRATCH_BYTES
    rc = L.mq_quantized_matmul_noalloc(None, None, None, None, None, None, M, N, K, 64, 4, 1, None)
    assert rc == mq._lib.MQ_ERR_INVALID
    assert b"use mq_quantized_matmul_ws" in L.mq_last_error()


@pytest.mark.parametrize("bits", [4, 8])
def test_noalloc_graph_replay_equals_eager(bits):
    """The entry point's stated use: captured in a HIP graph (after one eager
    call on the device, which resolves the array's address) and replayed
    four times, with eager calls of other shapes -- which overwrite the
    shared array -- and synchronisations between the replays; every replay is
    bit-equal to the workspace entry's output.  M = 32, 3584 -> 18944 splits K
    (partial sums in the array, then the fixed-order reduce)."""
    mq, L = _lib()
    core = importlib.import_module("mlx-server-runtime_amd.core")
    M, N, K = 32, 3584, 18944
    print(f"noalloc graph bits={bits}: M={M}, N={N}, K={K}", flush=True)
    assert 0 < L.mq_quantized_matmul_workspace(M, N, K, 64, bits) <= SCRATCH_BYTES
    g = torch.Generator(device=DEV).manual_seed(11 + bits)
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    wq, sc, bi = core.quantize(w, 64, bits)
    x = torch.randn(M, K, generator=g, device=DEV).to(torch.bfloat16)
    need = L.mq_quantized_matmul_workspace(M, N, K, 64, bits)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    ref = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    cur = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    mq._lib.check(L.mq_quantized_matmul_ws(_ptr(x), _ptr(wq), _ptr(sc), _ptr(bi), None, _ptr(ref),
                                           M, N, K, 64, bits, 1, _ptr(ws), ctypes.c_size_t(need),
                                           cur), "ws")
    out = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    # the eager call that resolves the array before any capture
    mq._lib.check(L.mq_quantized_matmul_noalloc(_ptr(x), _ptr(wq), _ptr(sc), _ptr(bi), None,
                                                _ptr(out), M, N, K, 64, bits, 1, cur), "eager")
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            rc = L.mq_quantized_matmul_noalloc(_ptr(x), _ptr(wq), _ptr(sc), _ptr(bi), None,
                                               _ptr(out), M, N, K, 64, bits, 1, s)
    torch.cuda.current_stream().wait_stream(side)
    assert rc == 0, L.mq_last_error()
    for i in range(4):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}"
        # an eager call of another plan between replays: it rewrites the array
        _case(mq, L, 16, 4608, 3584, bits, seed=20 + i, bias=True)
