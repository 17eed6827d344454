"""Decoder-step kernels (decode_ops: rms_norm, rope_kv_append,
paged_decode_attention, silu_mul) against float32 PyTorch restatements of the
reference's ops on the same inputs.

Bounds: outputs are bfloat16 of a float32 result, so an element may differ from
the float32 restatement by one bfloat16 step (at most 2^-7 relative) where the
two float32 values straddle a rounding boundary; the residual sum and the
appended V rows are exact.
"""

from __future__ import annotations

import importlib

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    return importlib.import_module("mlx-server-runtime_amd.decode_ops")


def _gen(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


def _within_one_step(out, ref_f32):
    """Every element of out (bf16) is within one bf16 step of the float32
    reference, plus 1e-5 of the largest |ref| for results that cancel to near
    zero (there float32 rounding order, e.g. fused multiply-adds, dominates)."""
    ref = ref_f32.float()
    tol = ref.abs() * 2.0 ** -7 + 1e-5 * ref.abs().max()
    return bool(((out.float() - ref).abs() <= tol).all())


@pytest.mark.parametrize("rows,dim", [(1, 256), (7, 3584), (32, 3584), (3, 8192), (2, 8)])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rms_norm(ops, rows, dim, with_residual):
    g = _gen(rows * 131 + dim)
    x = (torch.randn(rows, dim, generator=g, device=DEV) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(dim, generator=g, device=DEV)).to(torch.bfloat16)
    eps = 1e-6
    if with_residual:
        r = torch.randn(rows, dim, generator=g, device=DEV).to(torch.bfloat16)
        out, h = ops.rms_norm(x, w, eps, residual=r)
        h_ref = (x.float() + r.float()).to(torch.bfloat16)
        assert torch.equal(h, h_ref)
    else:
        out = ops.rms_norm(x, w, eps)
        h_ref = x
    hf = h_ref.float()
    ref = hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + eps) * w.float()
    assert _within_one_step(out, ref)


def test_rms_norm_batched_shape(ops):
    x = torch.randn(2, 5, 512, generator=_gen(3), device=DEV).to(torch.bfloat16)
    w = torch.ones(512, dtype=torch.bfloat16, device=DEV)
    out = ops.rms_norm(x, w, 1e-5)
    assert out.shape == x.shape
    ref = ops.rms_norm(x.reshape(10, 512), w, 1e-5).reshape(2, 5, 512)
    assert torch.equal(out, ref)


def _qmm_whole_tiles(x, wq, sc, bi, bits):
    """mq_quantized_matmul_ws without a workspace: the large-M GEMM runs every
    tile whole."""
    import ctypes
    mq = importlib.import_module("mlx-server-runtime_amd")
    L = mq._lib.lib()
    M, K = x.shape
    N = wq.shape[0]
    y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    mq._lib.check(L.mq_quantized_matmul_ws(ptr(x), ptr(wq), ptr(sc), ptr(bi), None, ptr(y), M, N,
                                           K, 64, bits, 1, None, ctypes.c_size_t(0),
                                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                  "ws")
    return y


@pytest.mark.parametrize("M,N,K,bits", [(1, 18944, 3584, 4), (2, 18944, 3584, 8),
                                        (1, 18948, 3584, 4), (1, 1025, 16384, 4),
                                        (2, 2049, 8192, 8), (32, 18944, 3584, 4),
                                        (32, 18944, 3584, 8), (16, 9475, 3584, 4),
                                        (16, 4739, 3584, 4), (32, 14336, 4096, 4),
                                        (16, 24000, 512, 4), (32, 20000, 1024, 8),
                                        (16, 4739, 3584, 8), (16, 18944, 3584, 8),
                                        (12, 9475, 3584, 8), (512, 18944, 3584, 4),
                                        (2048, 4739, 3584, 8), (300, 9476, 2048, 4)])
def test_quantized_matmul_swiglu_equals_two_kernels(ops, M, N, K, bits):
    """The gate|up GEMV with silu(gate) * up in its epilogue: bit-equal to the
    GEMV followed by silu_mul.  N = 18948, 1025 and 2049 leave a partial last
    block (8 and 2 output rows per block; 16 and 64 lanes per row).  At 16 and
    32 rows the skinny GEMM: K split with the SwiGLU in the reduce (4739) or
    unsplit with it in the GEMM's epilogue (9475 ends in a 3-column tile;
    24000 and 20000 take blocks of 6 and 5 waves).  8-bit batches of 9-16 rows
    take the skinny GEMM's 32-row tile too.  Prefill-sized M (300, 512, 2048)
    take the large-M GEMM with SiLU * up in its epilogue (4739 and 9476 leave
    partial 128-column tiles, 300 a partial row tile), against that GEMM with
    every tile whole."""
    core = importlib.import_module("mlx-server-runtime_amd.core")
    assert core.swiglu_supported(M, N, K, 64, bits)
    g = _gen(N + K + bits)
    w = (torch.randn(2 * N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    wq, sc, bi = core.quantize(w, 64, bits)
    x = torch.randn(M, K, generator=g, device=DEV).to(torch.bfloat16)
    out = core.quantized_matmul_swiglu(x, wq, sc, bi, 64, bits)
    if M <= 256:
        gu = core.quantized_matmul(x, wq, sc, bi, True, 64, bits)
    else:
        # the large-M GEMM with every tile whole, as the fused form runs it
        # (with a workspace a short last round of tiles may run as stream-K
        # pieces, summed in another order)
        gu = _qmm_whole_tiles(x, wq, sc, bi, bits)
    pad = -N % 8  # silu_mul takes widths of whole 8-element units; it is elementwise
    g, u = (F.pad(t, (0, pad)) for t in (gu[:, :N], gu[:, N:]))
    ref = ops.silu_mul(torch.cat([g, u], -1))[:, :N]
    assert out.shape == (M, N) and torch.equal(out, ref)


@pytest.mark.parametrize("N,K,bits,swiglu,with_res", [
    (18944, 3584, 4, True, True), (18944, 3584, 8, True, False), (37888, 3584, 4, False, True),
    (4096, 8192, 4, False, True), (4096, 8192, 8, False, False), (9475, 3584, 4, True, True)])
def test_rms_norm_quantized_matmul_equals_two_kernels(ops, N, K, bits, swiglu, with_res):
    """RMSNorm inside the GEMV's input staging: bit-equal to rms_norm followed by
    the dot2 GEMV (these shapes are large enough that quantized_matmul runs it),
    and the residual stream h bit-equal to rms_norm's."""
    core = importlib.import_module("mlx-server-runtime_amd.core")
    assert core.rms_norm_qmm_supported(1, N, K, 64, bits, swiglu)
    g = _gen(N + K + bits + swiglu)
    rows = 2 * N if swiglu else N
    w = (torch.randn(rows, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    wq, sc, bi = core.quantize(w, 64, bits)
    a = (torch.randn(1, K, generator=g, device=DEV) * 3).to(torch.bfloat16)
    res = torch.randn(1, K, generator=g, device=DEV).to(torch.bfloat16) if with_res else None
    nw = (torch.rand(K, generator=g, device=DEV) + 0.5).to(torch.bfloat16)
    y, h = core.rms_norm_quantized_matmul(a, nw, 1e-6, wq, sc, bi, None, res, 64, bits, swiglu)
    if with_res:
        x, ref_h = ops.rms_norm(a, nw, 1e-6, residual=res)
    else:
        x, ref_h = ops.rms_norm(a, nw, 1e-6), a
    if swiglu:
        gu = core.quantized_matmul(x, wq, sc, bi, True, 64, bits)
        pad = -N % 8
        ref = ops.silu_mul(torch.cat([F.pad(gu[:, :N], (0, pad)), F.pad(gu[:, N:], (0, pad))],
                                     -1))[:, :N]
    else:
        ref = core.quantized_matmul(x, wq, sc, bi, True, 64, bits)
    assert torch.equal(h, ref_h) and torch.equal(y, ref)


def test_rms_norm_quantized_matmul_small_matrix_with_bias(ops):
    """The Qwen2-7B QKV shape (quantized_matmul picks the matrix-core GEMV for
    it, so the rounding differs): within 1e-2 norm-wise of rms_norm + the
    unfused linear with its bias; h exact."""
    core = importlib.import_module("mlx-server-runtime_amd.core")
    N, K = 4608, 3584
    g = _gen(11)
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    wq, sc, bi = core.quantize(w, 64, 4)
    bias = (torch.randn(N, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    a = torch.randn(1, K, generator=g, device=DEV).to(torch.bfloat16)
    res = torch.randn(1, K, generator=g, device=DEV).to(torch.bfloat16)
    nw = (torch.rand(K, generator=g, device=DEV) + 0.5).to(torch.bfloat16)
    y, h = core.rms_norm_quantized_matmul(a, nw, 1e-6, wq, sc, bi, bias, res, 64, 4)
    x, ref_h = ops.rms_norm(a, nw, 1e-6, residual=res)
    ref = core.quantized_matmul(x, wq, sc, bi, True, 64, 4, bias=bias)
    assert torch.equal(h, ref_h)
    assert float((y.float() - ref.float()).abs().max() / ref.float().abs().max()) < 1e-2


@pytest.mark.parametrize("M,N,K,bits,with_bias", [
    (32, 3584, 18944, 4, False), (32, 3584, 3584, 4, True), (32, 4096, 4096, 8, False),
    (27, 3584, 18944, 4, True), (16, 3584, 18944, 8, False), (16, 3584, 3584, 8, True),
    (128, 3584, 18944, 4, False), (128, 3584, 18944, 8, True),
    # rows of fewer than 256 8-element units (N < 2048): Qwen3-0.6B's o and
    # down projections at decode batch sizes
    (32, 1024, 3072, 4, False), (16, 1024, 2048, 4, True), (32, 1024, 2048, 8, False)])
def test_quantized_matmul_add_rms_norm_equals_two_kernels(ops, M, N, K, bits, with_bias):
    """The skinny GEMM whose split-K reduce adds the residual and applies the
    RMSNorm: bit-equal to quantized_matmul (its workspace, the same split plan)
    followed by rms_norm, the residual stream included; 27 rows leave a
    partial row tile; 8-bit at 16 rows and 128-row plans (uneven last split)
    too."""
    core = importlib.import_module("mlx-server-runtime_amd.core")
    assert core.add_norm_supported(M, N, K, 64, bits)
    g = _gen(M + N + K + bits)
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    wq, sc, bi = core.quantize(w, 64, bits)
    x = torch.randn(M, K, generator=g, device=DEV).to(torch.bfloat16)
    res = torch.randn(M, N, generator=g, device=DEV).to(torch.bfloat16)
    nw = (torch.rand(N, generator=g, device=DEV) + 0.5).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g, device=DEV) * 0.1).to(torch.bfloat16) if with_bias else None
    out, h = core.quantized_matmul_add_rms_norm(x, wq, sc, bi, res, nw, 1e-6, bias, 64, bits)
    y = core.quantized_matmul(x, wq, sc, bi, True, 64, bits, bias=bias)
    ref_out, ref_h = ops.rms_norm(y, nw, 1e-6, residual=res)
    assert torch.equal(h, ref_h) and torch.equal(out, ref_out)


def test_quantized_matmul_swiglu_refuses_other_shapes(ops):
    core = importlib.import_module("mlx-server-runtime_amd.core")
    w = torch.zeros(2 * 1792, 18944 // 8, dtype=torch.int32, device=DEV)
    sc = torch.zeros(2 * 1792, 18944 // 64, dtype=torch.bfloat16, device=DEV)
    assert not core.swiglu_supported(1, 1792, 18944, 64, 4)  # rows of 128 lanes
    assert not core.swiglu_supported(1, 4864, 768, 64, 4)    # small: the matrix-core GEMV
    # K = 896 (14 groups, not a multiple of the matrix-core GEMV's 4-group
    # scale loads): quantized_matmul runs the dot2 GEMV there, so the fused
    # form takes it
    assert core.swiglu_supported(1, 4864, 896, 64, 4)
    x = (torch.randn(1, 896, generator=_gen(896), device=DEV)).to(torch.bfloat16)
    wt = (torch.randn(2 * 4864, 896, generator=_gen(4864), device=DEV) * 0.02).to(torch.bfloat16)
    wq, s, b = core.quantize(wt, 64, 4)
    assert torch.equal(core.quantized_matmul_swiglu(x, wq, s, b, 64, 4),
                       ops.silu_mul(core.quantized_matmul(x, wq, s, b, True, 64, 4)))
    with pytest.raises(NotImplementedError, match="not a fused shape"):
        core.quantized_matmul_swiglu(torch.zeros(1, 18944, dtype=torch.bfloat16, device=DEV),
                                     w, sc, sc, 64, 4)


@pytest.mark.parametrize("rows,inter", [(1, 18944), (32, 18944), (5, 8), (3, 768)])
def test_silu_mul(ops, rows, inter):
    gu = (torch.randn(rows, 2 * inter, generator=_gen(inter + rows), device=DEV) * 4
          ).to(torch.bfloat16)
    out = ops.silu_mul(gu)
    g, u = gu[:, :inter].float(), gu[:, inter:].float()
    act = F.silu(g).to(torch.bfloat16).float()
    assert out.shape == (rows, inter)
    ref = (act * u).to(torch.bfloat16)
    # bf16(silu(g)) may land on the neighbouring bf16 value (exp differs in the
    # last float32 bits), moving the product by at most two bf16 steps
    d = (out.float() - ref.float()).abs()
    assert bool((d <= ref.float().abs() * 2.0 ** -6 + 1e-30).all())
    assert (out == ref).float().mean() > 0.99


def _rope_ref(x, cos, sin):
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], -1)


def _tables(d, n, theta=1e6):
    q2 = importlib.import_module("mlx-server-runtime_amd.qwen2")
    cfg = q2.Qwen2Config(d * 4, 8, 4, 1, 1, 8, rope_theta=theta)
    return q2.rope_tables(cfg, n, DEV)


def _shuffled_cache(ops, layers, B, pages_per_seq, page_size, nkv, d, seed):
    """Every row gets its own pages in a random order across the pool."""
    perm = torch.randperm(B * pages_per_seq, generator=torch.Generator().manual_seed(seed))
    table = perm.reshape(B, pages_per_seq).to(torch.int32)
    return ops.PagedKV(layers, B * pages_per_seq, page_size, nkv, d, table, DEV)


@pytest.mark.parametrize("B,nh,nkv,d", [(1, 28, 4, 128), (5, 28, 4, 128), (3, 8, 8, 128),
                                        (2, 32, 4, 128), (3, 14, 2, 64)])
def test_rope_kv_append(ops, B, nh, nkv, d):
    ps, per = 16, 5
    cache = _shuffled_cache(ops, 2, B, per, ps, nkv, d, seed=B)
    cos, sin = _tables(d, cache.capacity)
    g = _gen(7 + B)
    qkv = torch.randn(B, (nh + 2 * nkv) * d, generator=g, device=DEV).to(torch.bfloat16)
    pos = torch.randint(0, cache.capacity, (B,), generator=g, device=DEV)
    pos[0] = cache.capacity - 1
    q = ops.rope_kv_append(qkv, pos, cache, 1, cos, sin, nh)
    qf = qkv.float()
    cs, sn = cos[pos][:, None, :], sin[pos][:, None, :]
    q_ref = _rope_ref(qf[:, :nh * d].reshape(B, nh, d), cs, sn)
    k_ref = _rope_ref(qf[:, nh * d:(nh + nkv) * d].reshape(B, nkv, d), cs, sn)
    v_ref = qkv[:, (nh + nkv) * d:].reshape(B, nkv, d)
    assert _within_one_step(q, q_ref)
    slots = cache.slots(torch.arange(B, device=DEV), pos)
    flat_k = cache.k[1].view(-1, nkv, d)
    flat_v = cache.v[1].view(-1, nkv, d)
    assert _within_one_step(flat_k[slots], k_ref)
    assert torch.equal(flat_v[slots], v_ref)
    # nothing else written: layer 0 untouched, and only B slots of layer 1 nonzero
    assert not cache.k[0].any() and not cache.v[0].any()
    assert int((flat_v.abs().sum((1, 2)) > 0).sum()) == B


def test_rope_kv_append_prefill_tokens(ops):
    """A prefill chunk's tokens in one call, each with its row's page-table row
    (the table argument): q roped, k roped and v written at each token's
    position of its row, nothing else written."""
    B, T, nh, nkv, d, ps, per = 2, 5, 28, 4, 128, 16, 4
    cache = _shuffled_cache(ops, 1, B, per, ps, nkv, d, seed=77)
    cos, sin = _tables(d, cache.capacity)
    g = _gen(78)
    qkv = torch.randn(B * T, (nh + 2 * nkv) * d, generator=g, device=DEV).to(torch.bfloat16)
    starts = torch.tensor([3, 40], device=DEV)
    pos = (starts[:, None] + torch.arange(T, device=DEV)[None, :]).reshape(-1)
    rows = torch.arange(B, device=DEV).repeat_interleave(T)
    table = cache.page_table[rows].contiguous()
    q = ops.rope_kv_append(qkv, pos, cache, 0, cos, sin, nh, table=table)
    qf = qkv.float()
    cs, sn = cos[pos][:, None, :], sin[pos][:, None, :]
    assert _within_one_step(q, _rope_ref(qf[:, :nh * d].reshape(-1, nh, d), cs, sn))
    slots = cache.slots(rows, pos)
    flat_k = cache.k[0].view(-1, nkv, d)
    flat_v = cache.v[0].view(-1, nkv, d)
    k_ref = _rope_ref(qf[:, nh * d:(nh + nkv) * d].reshape(-1, nkv, d), cs, sn)
    assert _within_one_step(flat_k[slots], k_ref)
    assert torch.equal(flat_v[slots], qkv[:, (nh + nkv) * d:].reshape(-1, nkv, d))
    assert int((flat_v.abs().sum((1, 2)) > 0).sum()) == B * T


@pytest.mark.parametrize("d,norms,ps", [(128, False, 16), (128, True, 16), (64, True, 16),
                                        (128, True, 24)])
def test_rope_kv_append_many_rows_equal_row_chunks(ops, d, norms, ps):
    """1027 rows in one call take the row-batched grid (4 rows a block, the
    last block partial); the same rows appended in chunks of under 1024 take
    one row a block.  q, the k pages and the v pages agree bit for bit, with
    and without the q/k norms."""
    nh, nkv = 16, 2
    per = -(-400 // ps)  # at least 400 positions a row
    lens = [300, 300, 300, 127]
    starts = [0, 50, 99, 200]
    R = len(lens)
    g = _gen(901 + d + norms)
    qkv = torch.randn(sum(lens), (nh + 2 * nkv) * d, generator=g, device=DEV).to(torch.bfloat16)
    pos = torch.cat([torch.arange(s0, s0 + n, device=DEV) for s0, n in zip(starts, lens)])
    rows = torch.cat([torch.full((n,), r, device=DEV) for r, n in enumerate(lens)])
    qn = kn = None
    if norms:
        qn = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(torch.bfloat16)
        kn = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(torch.bfloat16)
    caches = [_shuffled_cache(ops, 1, R, per, ps, nkv, d, seed=5) for _ in range(2)]
    cos, sin = _tables(d, caches[0].capacity)
    table = caches[0].page_table[rows].contiguous()
    q_all = ops.rope_kv_append(qkv, pos, caches[0], 0, cos, sin, nh, q_norm=qn, k_norm=kn,
                               table=table)
    parts = []
    for a in range(0, qkv.shape[0], 500):
        b = min(a + 500, qkv.shape[0])
        parts.append(ops.rope_kv_append(qkv[a:b].contiguous(), pos[a:b].contiguous(), caches[1],
                                        0, cos, sin, nh, q_norm=qn, k_norm=kn,
                                        table=table[a:b].contiguous()))
    assert torch.equal(q_all, torch.cat(parts))
    assert torch.equal(caches[0].k[0], caches[1].k[0])
    assert torch.equal(caches[0].v[0], caches[1].v[0])
    assert int((caches[0].v[0].abs().sum((2, 3)) > 0).sum()) == sum(lens)


@pytest.mark.parametrize("rows,cols", [(1, 152064), (32, 152064), (5, 8), (6, 1000)])
def test_argmax_rows_equals_torch_argmax(ops, rows, cols):
    """The greedy next token: the first index of each row's largest bfloat16
    value, as torch.argmax over the same values -- random rows, a row of ties
    (the first of two maxima), -0 before +0 among -inf, a NaN (the largest)."""
    g = _gen(rows * 7 + cols)
    x = torch.randn(rows, cols, generator=g, device=DEV).to(torch.bfloat16)
    if rows >= 2:
        x[1] = 0.5
        x[1, cols // 3] = 2.0
        x[1, cols - 1] = 2.0
    if rows >= 3:
        x[2] = -float("inf")
        x[2, cols // 2] = -0.0
        x[2, cols // 2 + 1] = 0.0
    if rows >= 4:
        x[3, cols // 2 - 1] = float("nan")
    got = ops.argmax_rows(x)
    ref = x.float().argmax(-1)
    assert got.dtype == torch.int64 and got.shape == (rows,)
    assert torch.equal(got, ref), (got, ref)
    if rows >= 3:
        assert int(got[1]) == cols // 3 and int(got[2]) == cols // 2
    if rows >= 4:
        assert int(got[3]) == cols // 2 - 1


def _attention_ref(q, cache, layer, pos, scale):
    """float32 softmax(q k^T scale) v per row over its positions 0..pos."""
    B, nh, d = q.shape
    rep = nh // cache.kv_heads
    outs = []
    for b in range(B):
        L = int(pos[b]) + 1
        k, v = cache.gather_rows(layer, torch.tensor([b], device=DEV), L)
        k = k[0].float().repeat_interleave(rep, 0)  # [nh, L, d]
        v = v[0].float().repeat_interleave(rep, 0)
        s = torch.matmul(k, q[b].float().unsqueeze(-1)).squeeze(-1) * scale   # [nh, L]
        p = torch.softmax(s, -1).unsqueeze(1)                                 # [nh, 1, L]
        outs.append(torch.matmul(p, v).reshape(nh * d))
    return torch.stack(outs)


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("B,nh,nkv,per,positions", [
    (1, 28, 4, 40, [639]),                      # 7B heads, batch 1, a full 640-slot row
    (1, 28, 4, 40, [0]),                        # one cached position
    (4, 28, 4, 80, [1279, 17, 640, 1000]),     # ragged rows, several splits each
    (3, 8, 8, 4, [63, 5, 33]),                 # no grouping
    (2, 32, 4, 7, [100, 111]),                 # 8 query heads per KV head
    (2, 12, 4, 3, [47, 16]),                   # 3 per KV head
    (32, 28, 4, 80, None),                     # batch 32 decode at ~1.2K context
    (20, 16, 4, 3, [47, 0, 30] * 6 + [1, 2]),  # many pairs, short rows: one 4-wave split
])
def test_paged_decode_attention(ops, B, nh, nkv, per, positions, d):
    ps = 16
    cache = _shuffled_cache(ops, 1, B, per, ps, nkv, d, seed=per + B)
    g = _gen(11 + B + nh + d)
    cache.k[0].copy_(torch.randn(cache.k[0].shape, generator=g, device=DEV).to(torch.bfloat16))
    cache.v[0].copy_(torch.randn(cache.v[0].shape, generator=g, device=DEV).to(torch.bfloat16))
    if positions is None:
        pos = torch.randint(1000, cache.capacity, (B,), generator=g, device=DEV)
    else:
        pos = torch.tensor(positions, dtype=torch.int64, device=DEV)
    q = (torch.randn(B, nh, d, generator=g, device=DEV) * 2).to(torch.bfloat16)
    scale = d ** -0.5
    out = ops.paged_decode_attention(q, cache, 0, pos, scale)
    ref = _attention_ref(q, cache, 0, pos, scale)
    err = (out.float() - ref).abs().max() / ref.abs().max()
    assert out.shape == (B, nh * d)
    assert err < 2.0 ** -7, float(err)
    again = ops.paged_decode_attention(q, cache, 0, pos, scale)
    assert torch.equal(out, again)


def _prefill_ref(q, cache, layer, starts, lens, scale):
    """float32 causal attention per row: query j of row b at position
    starts[b] + min(j, lens[b] - 1) over the row's positions 0..that."""
    B, T, nh, d = q.shape
    rep = nh // cache.kv_heads
    out = torch.empty(B, T, nh * d, device=DEV)
    for b in range(B):
        pos = int(starts[b]) + torch.clamp(torch.arange(T, device=DEV), max=int(lens[b]) - 1)
        S = int(pos.max()) + 1
        k, v = cache.gather_rows(layer, torch.tensor([b], device=DEV), S)
        k = k[0].float().repeat_interleave(rep, 0)                      # [nh, S, d]
        v = v[0].float().repeat_interleave(rep, 0)
        s = torch.matmul(q[b].float().transpose(0, 1), k.transpose(1, 2).contiguous()) * scale
        masked = torch.arange(S, device=DEV)[None, :] > pos[:, None]  # [T, S]
        p = torch.softmax(s.masked_fill(masked[None], float("-inf")), -1)
        out[b] = torch.matmul(p, v).transpose(0, 1).reshape(T, nh * d)
    return out


@pytest.mark.parametrize("B,T,nh,nkv,per,starts,lens,ps", [
    (1, 64, 28, 4, 4, [0], [64], 16),                        # one tile, no cache before it
    (2, 100, 28, 4, 40, [256, 0], [100, 37], 16),            # a cached prefix; a ragged row
    (3, 200, 32, 4, 50, [0, 500, 17], [200, 150, 1], 16),    # 8 per KV head; a one-token row
    (1, 256, 8, 8, 80, [1000], [256], 16),                   # no grouping, 1000 cached positions
    (4, 33, 16, 2, 10, [7, 64, 100, 0], [33, 20, 1, 9], 16),  # short chunks
    (2, 70, 28, 4, 13, [0, 33], [70, 71 - 33], 8),           # page size 8, 104 positions: the
                                                             # last key block runs past the table
    (1, 130, 28, 4, 3, [61], [130], 64),                     # page size 64, a chunk over 3 pages
    (2, 90, 28, 4, 8, [0, 50], [90, 77], 24),                # page size 24 (not a power of two)
    # 512+ blocks of 128 queries: two query tiles a wave (a row alone: one)
    (8, 256, 32, 4, 30, [0, 100, 7, 200, 0, 33, 64, 150],
     [256, 256, 200, 56, 1, 256, 129, 17], 16),
    (4, 640, 28, 4, 60, [0, 300, 0, 17], [640, 600, 333, 640], 16),
])
def test_paged_prefill_attention(ops, B, T, nh, nkv, per, starts, lens, ps):
    """Prefill-chunk attention over shuffled pages against the float32
    restatement (the probabilities are bfloat16 in the kernel's P.V, as in
    the decode kernel: within 2^-7 of the largest output); each row alone
    gives the same bits as in the batch -- also where the batch runs two
    query tiles a wave and the row alone one."""
    d = 128
    cache = _shuffled_cache(ops, 1, B, per, ps, nkv, d, seed=per + B + T)
    g = _gen(31 + B + T + nh)
    cache.k[0].copy_(torch.randn(cache.k[0].shape, generator=g, device=DEV).to(torch.bfloat16))
    cache.v[0].copy_(torch.randn(cache.v[0].shape, generator=g, device=DEV).to(torch.bfloat16))
    st = torch.tensor(starts, dtype=torch.int64, device=DEV)
    ln = torch.tensor(lens, dtype=torch.int64, device=DEV)
    q = (torch.randn(B, T, nh, d, generator=g, device=DEV) * 2).to(torch.bfloat16)
    scale = d ** -0.5
    print(f"prefill attention B={B} T={T} nh={nh} nkv={nkv} starts={starts} lens={lens}",
          flush=True)
    assert ops.prefill_attention_supported(nh, cache)
    out = ops.paged_prefill_attention(q, cache, 0, cache.page_table, st, ln, scale)
    ref = _prefill_ref(q, cache, 0, st, ln, scale)
    err = (out.float() - ref).abs().max() / ref.abs().max()
    assert out.shape == (B, T, nh * d)
    assert err < 2.0 ** -7, float(err)
    assert torch.equal(out, ops.paged_prefill_attention(q, cache, 0, cache.page_table, st, ln,
                                                        scale))
    for b in range(B):
        n = int(lens[b])
        one = ops.paged_prefill_attention(q[b:b + 1, :n].contiguous(), cache, 0,
                                          cache.page_table[b:b + 1].contiguous(), st[b:b + 1],
                                          ln[b:b + 1], scale)
        assert torch.equal(one[0], out[b, :n]), b


def test_paged_prefill_attention_refusals(ops):
    """head_dim 64 is not taken (the query says so and the call raises)."""
    cache = _shuffled_cache(ops, 1, 1, 2, 16, 2, 64, seed=1)
    assert not ops.prefill_attention_supported(8, cache)
    q = torch.zeros(1, 4, 8, 64, dtype=torch.bfloat16, device=DEV)
    one = torch.zeros(1, dtype=torch.int64, device=DEV)
    with pytest.raises(NotImplementedError):
        ops.paged_prefill_attention(q, cache, 0, cache.page_table, one, one + 4, 0.125)


def test_paged_decode_attention_shared_prefix_pages(ops):
    """Rows that share their first pages (a cached prompt prefix) read them
    through the table: equal to a cache holding private copies."""
    d, ps, nkv, nh, B = 128, 16, 4, 28, 3
    shared, own = 4, 3
    table = torch.empty(B, shared + own, dtype=torch.int32)
    table[:, :shared] = torch.arange(shared, dtype=torch.int32)
    table[:, shared:] = shared + torch.arange(B * own, dtype=torch.int32).reshape(B, own)
    c1 = ops.PagedKV(1, shared + B * own, ps, nkv, d, table, DEV)
    g = _gen(5)
    c1.k[0].copy_(torch.randn(c1.k[0].shape, generator=g, device=DEV).to(torch.bfloat16))
    c1.v[0].copy_(torch.randn(c1.v[0].shape, generator=g, device=DEV).to(torch.bfloat16))
    c2 = ops.PagedKV.contiguous(1, B, (shared + own) * ps, nkv, d, DEV, ps)
    for b in range(B):
        k, v = c1.gather_rows(0, torch.tensor([b], device=DEV), c1.capacity)
        n = c1.capacity
        slots = c2.slots(torch.full((n,), b, device=DEV), torch.arange(n, device=DEV))
        c2.write(0, slots, k[0].transpose(0, 1), v[0].transpose(0, 1))
    pos = torch.tensor([70, 111, 64], device=DEV)
    q = torch.randn(B, nh, d, generator=g, device=DEV).to(torch.bfloat16)
    a1 = ops.paged_decode_attention(q, c1, 0, pos, 0.1)
    a2 = ops.paged_decode_attention(q, c2, 0, pos, 0.1)
    assert torch.equal(a1, a2)


def test_decode_ops_in_graph_replays(ops):
    """A captured rope-append + attention step replays correctly as positions
    advance (positions live on the device)."""
    d, nkv, nh, B, ps, per = 128, 4, 28, 2, 16, 4
    cache = _shuffled_cache(ops, 1, B, per, ps, nkv, d, seed=9)
    cos, sin = _tables(d, cache.capacity)
    g = _gen(21)
    qkv = torch.randn(B, (nh + 2 * nkv) * d, generator=g, device=DEV).to(torch.bfloat16)
    pos = torch.zeros(B, dtype=torch.int64, device=DEV)

    def step():
        q = ops.rope_kv_append(qkv, pos, cache, 0, cos, sin, nh)
        return ops.paged_decode_attention(q, cache, 0, pos, d ** -0.5), q

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, q_static = step()
    for i in range(1, 20):
        pos.fill_(i)
        qkv.copy_(torch.randn(qkv.shape, generator=g, device=DEV).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        ref = _attention_ref(q_static, cache, 0, pos, d ** -0.5)
        err = (out.float() - ref).abs().max() / ref.abs().max()
        assert err < 2.0 ** -7, (i, float(err))


def test_errors(ops):
    d, nkv = 128, 4
    cache = ops.PagedKV.contiguous(1, 2, 32, nkv, d, DEV)
    pos = torch.zeros(2, dtype=torch.int64, device=DEV)
    with pytest.raises(NotImplementedError):
        q = torch.zeros(2, 36, d, dtype=torch.bfloat16, device=DEV)  # 9 per KV head
        ops.paged_decode_attention(q, cache, 0, pos, 1.0)
    with pytest.raises(ValueError):
        q = torch.zeros(2, 28, d, dtype=torch.float32, device=DEV)
        ops.paged_decode_attention(q, cache, 0, pos, 1.0)
    with pytest.raises(NotImplementedError):
        ops.rms_norm(torch.zeros(2, 12, dtype=torch.bfloat16, device=DEV),
                     torch.ones(12, dtype=torch.bfloat16, device=DEV), 1e-6)
    with pytest.raises(ValueError):
        ops.silu_mul(torch.zeros(2, 7, dtype=torch.bfloat16, device=DEV))


@pytest.mark.parametrize("B,nh,nkv,d,per,qk_norm", [
    (1, 28, 4, 128, 40, False), (4, 28, 4, 128, 80, False), (8, 32, 4, 128, 36, True),
    (3, 14, 2, 64, 5, True), (2, 8, 8, 128, 3, False), (32, 28, 4, 128, 80, False)])
def test_attention_step_equals_rope_then_attention(ops, B, nh, nkv, d, per, qk_norm):
    """The fused step (RoPE + append inside the split attention kernel) gives
    the unfused path's results bit for bit and leaves the same pages, across
    HIP-graph replays."""
    ps = 16
    c1 = _shuffled_cache(ops, 1, B, per, ps, nkv, d, seed=B + per)
    c2 = ops.PagedKV(1, c1.num_pages, ps, nkv, d, c1.page_table.cpu(), DEV)
    g = _gen(B * 7 + nh)
    fill = torch.randn(c1.k[0].shape, generator=g, device=DEV).to(torch.bfloat16)
    for c in (c1, c2):
        c.k[0].copy_(fill)
        c.v[0].copy_(fill.flip(0))
    cos, sin = _tables(d, c1.capacity)
    qn = kn = None
    if qk_norm:
        qn = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(torch.bfloat16)
        kn = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(torch.bfloat16)
    qkv = torch.randn(B, (nh + 2 * nkv) * d, generator=g, device=DEV).to(torch.bfloat16)
    pos = torch.randint(0, c1.capacity, (B,), generator=g, device=DEV)
    pos[0] = c1.capacity - 1
    scale = d ** -0.5
    q = ops.rope_kv_append(qkv, pos, c1, 0, cos, sin, nh, qn, kn, 1e-6)
    ref = ops.paged_decode_attention(q, c1, 0, pos, scale)
    out = ops.attention_step(qkv, pos, c2, 0, cos, sin, nh, scale, qn, kn, 1e-6)
    assert torch.equal(out, ref)
    assert torch.equal(c1.k[0], c2.k[0]) and torch.equal(c1.v[0], c2.v[0])
    # captured and replayed with advancing positions
    step = lambda: ops.attention_step(qkv, pos, c2, 0, cos, sin, nh, scale, qn, kn, 1e-6)  # noqa
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    for _ in range(3):
        pos.sub_(1).clamp_(min=0)
        graph.replay()
        torch.cuda.synchronize()
        q = ops.rope_kv_append(qkv, pos, c1, 0, cos, sin, nh, qn, kn, 1e-6)
        assert torch.equal(static, ops.paged_decode_attention(q, c1, 0, pos, scale))
