"""Host-side checks that need no GPU.

* libmi355q.so loads and exports every function include/*.h declares;
* the C ABI rejects what MLX rejects (MQ_ERR_INVALID), flags what this backend
  does not implement (MQ_ERR_UNSUPPORTED), and returns before any launch, so
  these calls run without a device (null pointers are never dereferenced);
* the Python layer maps the codes to ValueError / NotImplementedError and
  refuses CPU tensors instead of falling back to a CPU path.
"""

from __future__ import annotations

import ctypes
import glob
import os
import re

import pytest
import torch

from conftest import ROOT

HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_functions():
    names = set()
    for path in HEADERS:
        text = open(path).read()
        names |= set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(mq_\w+)\s*\(", text, re.M))
    return sorted(names)


def test_header_declares_the_abi():
    assert declared_functions() == sorted([
        "mq_version", "mq_last_error", "mq_quantize", "mq_dequantize", "mq_embedding_lookup",
        "mq_repack_codes_u8", "mq_quantized_matmul", "mq_quantized_matmul_workspace", "mq_quantized_matmul_ws",
        "mq_gather_qmm", "mq_rms_norm", "mq_rope_kv_append",
        "mq_paged_decode_attention_workspace", "mq_paged_decode_attention",
        "mq_decode_attention_step", "mq_silu_mul",
        "mq_moe_route", "mq_moe_sort", "mq_moe_combine", "mq_moe_route_sort",
        "mq_moe_combine_rms_norm", "mq_quantized_matmul_swiglu_supported",
        "mq_quantized_matmul_swiglu", "mq_rms_norm_quantized_matmul_supported",
        "mq_rms_norm_quantized_matmul", "mq_quantized_matmul_swiglu_workspace",
        "mq_quantized_matmul_swiglu_ws", "mq_quantized_matmul_add_rms_norm_supported",
        "mq_quantized_matmul_add_rms_norm_workspace", "mq_quantized_matmul_add_rms_norm",
        "mq_gather_qmm_swiglu_supported", "mq_gather_qmm_swiglu", "mq_hbm_read", "mq_qmv_trace",
        "mq_quantized_matmul_noalloc", "mq_gather_qmm_segments",
        "mq_gather_qmm_segments_supported", "mq_paged_prefill_attention_supported",
        "mq_paged_prefill_attention", "mq_argmax_rows"])


def test_library_exports_every_declared_symbol(mq):
    L = mq._lib.lib()
    for name in declared_functions():
        assert hasattr(L, name), name
    assert set(mq._lib.EXPORTS) == set(declared_functions())
    assert mq.version() == (2, 2)


def _L(mq):
    return mq._lib.lib()


def test_workspace_query(mq):
    """Workspace sizes are pure host arithmetic: float32 partials for split-K
    shapes (few columns, long K), none for wide or GEMV shapes."""
    L = _L(mq)
    q = L.mq_quantized_matmul_workspace
    down = q(64, 3584, 18944, 64, 4)          # 28 column tiles: K is split
    assert down > 0 and down % (64 * 3584 * 4) == 0
    assert q(128, 18944, 3584, 64, 4) == 0    # 148 column tiles: no split
    assert q(1, 3584, 18944, 64, 4) == 0      # GEMV
    assert q(4096, 3584, 18944, 64, 4) == 0   # large-M kernels, 224 tiles: no split
    assert q(2048, 3584, 18944, 64, 4) == 2 * 2048 * 3584 * 4   # 112 tiles: K in 2
    # 3-bit codes: their one-byte repack (rounded to 256 bytes) ahead of the
    # 8-bit plan's own workspace
    assert q(64, 3584, 18944, 64, 3) == (3584 * 18944 + 255) // 256 * 256 + q(64, 3584, 18944, 64, 8)
    assert q(1, 100, 96, 32, 5) == 9728 + q(1, 100, 96, 32, 8)
    assert q(64, 3584, 18900, 64, 4) == 0     # K not a group multiple
    assert q(0, 3584, 18944, 64, 4) == 0


def test_attention_workspace_query(mq):
    """Float32 partials (max, sum, 128 weighted values per query head) per
    (sequence, KV head, split of the positions)."""
    q = _L(mq).mq_paged_decode_attention_workspace
    per_split = 7 * (128 + 2) * 4                # one KV head's 7 query heads
    bs1 = q(1, 28, 4, 128, 40, 16)             # 640 positions
    assert bs1 > 0 and bs1 % (4 * per_split) == 0
    splits = bs1 // (4 * per_split)
    assert 1 < splits <= 10                      # split over blocks, >= 64 positions each
    bs32 = q(32, 28, 4, 128, 80, 16)
    assert bs32 > 0 and bs32 % (32 * 4 * per_split) == 0
    d64 = q(1, 28, 4, 64, 40, 16)                # head_dim 64: 64 + 2 floats per head
    assert d64 > 0 and d64 % (4 * 7 * 66 * 4) == 0
    assert q(1, 28, 4, 96, 40, 16) == 0          # head_dim 96: unsupported
    assert q(1, 36, 4, 128, 40, 16) == 0         # 9 query heads per KV head
    assert q(0, 28, 4, 128, 40, 16) == 0
    assert q(1, 28, 4, 128, 0, 16) == 0


def test_decoder_entry_validation(mq):
    """Argument checks run before any device access (null pointers are fine)."""
    L = _L(mq)
    null = None
    assert L.mq_rms_norm(null, null, null, null, null, 4, 12, 1e-6, null) == -2   # dim % 8
    assert L.mq_rms_norm(null, null, null, null, null, 4, 8200, 1e-6, null) == -2
    assert L.mq_rms_norm(null, 1, null, null, null, 4, 64, 1e-6, null) == -1     # residual pair
    assert L.mq_rms_norm(null, null, null, null, null, 0, 64, 1e-6, null) == 0
    assert L.mq_silu_mul(null, null, 4, 12, null) == -2
    assert L.mq_silu_mul(null, null, 0, 16, null) == 0
    att = L.mq_paged_decode_attention
    assert att(null, null, null, null, 4, 16, 8, null, 2, 30, 4, 128, 1.0, null, 0, null,
               null) == -1                                                      # 30 % 4
    assert att(null, null, null, null, 4, 16, 8, null, 2, 28, 4, 96, 1.0, null, 0, null,
               null) == -2                                                      # head_dim
    assert att(null, null, null, null, 4, 16, 8, null, 2, 28, 4, 128, 1.0, null, 0, null,
               null) == -1                                                      # no workspace
    assert b"workspace" in L.mq_last_error()
    assert att(null, null, null, null, 0, 16, 8, null, 2, 28, 4, 128, 1.0, null, 0, null,
               null) == -1                                                      # no pages
    rope = L.mq_rope_kv_append
    assert rope(null, null, null, 4, 16, 8, null, null, null, null, 1e-6, null, null, null, 2,
                28, 4, 127, null) == -1                                         # odd head_dim
    assert rope(null, null, null, 4, 16, 8, null, null, 1, null, 1e-6, null, null, null, 2,
                28, 4, 256, null) == -2                                         # norm, d > 128
    assert rope(null, null, null, 4, 16, 8, null, null, null, null, 1e-6, null, null, null, 0,
                28, 4, 128, null) == 0
    assert L.mq_moe_route(null, null, 4, 128, 8, 1, null, null, null) == -1    # null pointers
    assert L.mq_moe_route(null, null, 4, 600, 8, 1, null, null, null) == -2    # too many experts
    assert L.mq_moe_route(null, null, 4, 8, 9, 1, null, null, null) == -2      # k > E
    assert L.mq_moe_route(null, null, 0, 128, 8, 1, null, null, null) == 0
    assert L.mq_moe_sort(null, 64, 8, 128, null, null, null, null, null, null) == -1
    assert L.mq_moe_sort(null, 64, 0, 128, null, null, null, null, null, null) == -1
    assert L.mq_moe_sort(null, 0, 8, 128, null, null, null, null, null, null) == 0
    assert L.mq_moe_combine(null, null, null, null, 4, 8, 2044, null) == -2    # hidden % 8
    assert L.mq_moe_combine(null, null, null, null, 0, 8, 2048, null) == 0
    rs = L.mq_moe_route_sort
    assert rs(null, null, 4, 128, 8, 1, null, null, null, null, null, null, null, null) == -1
    assert rs(null, null, 4, 600, 8, 1, null, null, null, null, null, null, null, null) == -2
    assert rs(null, null, 0, 128, 8, 1, null, null, null, null, null, null, null, null) == 0
    seg = L.mq_gather_qmm_segments
    assert seg(null, null, null, null, null, null, null, null, 300, 1, 64, 512, 8, 300, 64, 4,
               0, null) == -1                                                   # no offsets
    one = ctypes.c_void_p(16)  # never dereferenced: validation fails before any launch
    assert seg(null, null, null, one, null, null, null, null, 300, 1, 64, 512, 8, 300, 64, 4,
               0, null) == -1                                                   # null pointers
    assert seg(one, null, one, one, one, one, one, one, 300, 1, 64, 512, 8, 300, 64, 3,
               1, null) == -2                      # SiLU * up epilogue: 4- and 8-bit codes
    assert seg(null, null, null, one, null, null, null, null, 0, 1, 64, 512, 8, 0, 64, 4,
               1, null) == 0
    sup = L.mq_quantized_matmul_swiglu_supported
    assert sup(1, 18944, 3584, 64, 4) == 1 and sup(2, 18944, 3584, 64, 8) == 1
    assert sup(4, 18944, 3584, 64, 4) == 0                                      # M > 2
    assert sup(1, 1792, 18944, 64, 4) == 0                                      # 128-lane rows
    assert sup(1, 18944, 3584, 32, 4) == 1 and sup(1, 18944, 3584, 128, 8) == 1  # group sizes
    assert sup(1, 18944, 3584, 64, 3) == 0 and sup(1, 18944, 3584, 16, 4) == 0
    sw = L.mq_quantized_matmul_swiglu
    assert sw(null, null, null, null, null, 4, 18944, 3584, 64, 4, null) == -2   # not fused
    assert sw(null, null, null, null, null, 1, 18944, 3584, 64, 4, null) == -1   # null pointers
    assert sw(null, null, null, null, null, 0, 18944, 3584, 64, 4, null) == 0
    # batch-32 gate|up: the skinny GEMM runs unsplit with SiLU * up in its epilogue
    assert sup(32, 18944, 3584, 64, 4) == 1
    assert L.mq_quantized_matmul_swiglu_workspace(32, 18944, 3584, 64, 4) == 0
    assert L.mq_quantized_matmul_workspace(32, 2 * 18944, 3584, 64, 4) == 0
    # 2 * 9475 rows are 149 column tiles, under one block per CU, yet no
    # second split fits: unsplit, with the epilogue
    assert sup(16, 9475, 3584, 64, 4) == 1
    assert L.mq_quantized_matmul_swiglu_workspace(16, 9475, 3584, 64, 4) == 0
    # batch 16, 2 * 4739 rows (75 tiles): three K splits with the fused reduce
    assert sup(16, 4739, 3584, 64, 4) == 1
    assert L.mq_quantized_matmul_swiglu_workspace(16, 4739, 3584, 64, 4) == \
        L.mq_quantized_matmul_workspace(16, 2 * 4739, 3584, 64, 4) == 3 * 16 * 2 * 4739 * 4
    assert L.mq_quantized_matmul_swiglu_workspace(1, 18944, 3584, 64, 4) == 0  # the GEMV path
    assert sw(null, null, null, null, null, 32, 18944, 3584, 64, 4, null) == -1  # null pointers
    an = L.mq_quantized_matmul_add_rms_norm_supported
    assert an(32, 3584, 18944, 64, 4) == 1 and an(32, 3584, 3584, 64, 4) == 1
    assert an(1, 3584, 18944, 64, 4) == 0                                       # a GEMV
    assert L.mq_quantized_matmul_add_rms_norm_workspace(32, 3584, 18944, 64, 4) == \
        L.mq_quantized_matmul_workspace(32, 3584, 18944, 64, 4) > 0
    buf = ctypes.create_string_buffer(64)
    p16 = ctypes.addressof(buf) + (-ctypes.addressof(buf) % 16)
    assert L.mq_quantized_matmul_add_rms_norm(p16, p16, p16, p16, None, p16, p16, p16, 1e-6, p16,
                                              32, 3584, 18944, 64, 4, None, 0, null) == -1
    assert b"workspace" in L.mq_last_error()
    ns = L.mq_rms_norm_quantized_matmul_supported
    assert ns(1, 4608, 3584, 64, 4, 0) == 1 and ns(1, 18944, 3584, 64, 4, 1) == 1
    assert ns(2, 4608, 3584, 64, 4, 0) == 0                                     # one row only
    assert ns(1, 3584, 18944, 64, 4, 0) == 0                                    # K > 8192
    nq = L.mq_rms_norm_quantized_matmul
    assert nq(null, null, null, null, 1e-6, null, null, null, null, null, 1, 4608, 3584, 64, 4, 0,
              null) == -1                                                        # null pointers
    assert nq(null, null, null, null, 1e-6, null, null, null, null, null, 2, 4608, 3584, 64, 4, 0,
              null) == -2                                                        # not fused
    buf = ctypes.create_string_buffer(8192)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf) % 16)
    assert nq(p, p, p, p, 1e-6, p, p, p, None, p, 1, 4608, 1024, 64, 4, 0,
              null) == -1                                                        # out overlaps
    assert b"overlap" in L.mq_last_error()
    cn = L.mq_moe_combine_rms_norm
    assert cn(null, null, null, null, null, null, null, 4, 8, 2048, 1e-6, null) == -1
    assert cn(null, null, null, null, null, null, null, 4, 8, 8200, 1e-6, null) == -2  # > 8192
    assert cn(null, null, null, null, null, null, null, 4, 0, 2048, 1e-6, null) == -1  # top_k
    assert cn(null, null, null, null, null, null, null, 0, 8, 2048, 1e-6, null) == 0


def test_argmax_rows_entry_validation(mq):
    """Rows of whole 8-element units only; null pointers and a misaligned x
    refused; no rows a no-op."""
    L = _L(mq)
    f = L.mq_argmax_rows
    assert f(None, 2, 12, None, None) == -2      # cols % 8
    assert f(None, 2, 0, None, None) == -1       # no columns
    assert f(None, 2, (1 << 28) + 8, None, None) == -1   # past 32-bit row offsets
    assert f(None, 0, 16, None, None) == 0
    assert f(None, 2, 16, None, None) == -1      # null
    assert f(8, 2, 16, 64, None) == -1           # x not 16-byte aligned


def test_prefill_attention_entry_validation(mq):
    """The prefill attention entry: its support query and the argument checks,
    all before any device access (null pointers are fine)."""
    L = _L(mq)
    null = None
    sup = L.mq_paged_prefill_attention_supported
    assert sup(28, 4, 128, 4096, 16) == 1
    assert sup(32, 4, 128, 4096, 16) == 1
    assert sup(28, 4, 64, 4096, 16) == 0                   # head_dim 128 only
    assert sup(30, 4, 128, 4096, 16) == 0                  # heads not a multiple of KV heads
    assert sup(28, 0, 128, 4096, 16) == 0
    assert sup(28, 4, 128, 1 << 20, 16) == 0               # a layer's pages past 2 GiB
    assert sup(28, 4, 128, 0, 16) == 0
    pf = L.mq_paged_prefill_attention
    #        q     k     v     table pps ps  pages starts lens B  T    nh  nkv d    scale
    assert pf(null, null, null, null, 4, 16, 8, null, null, 2, 64, 30, 4, 128, 1.0, null,
              null) == -1                                                   # 30 % 4
    assert pf(null, null, null, null, 4, 16, 8, null, null, 2, 64, 28, 4, 64, 1.0, null,
              null) == -2                                                   # head_dim
    assert b"head_dim" in L.mq_last_error()
    assert pf(null, null, null, null, 4, 16, 8, null, null, 2, 64, 28, 4, 128, 1.0, null,
              null) == -1                                                   # null pointers
    assert pf(null, null, null, null, 0, 16, 8, null, null, 2, 64, 28, 4, 128, 1.0, null,
              null) == -1                                                   # no pages
    assert pf(null, null, null, null, 4, 16, 8, null, null, 0, 64, 28, 4, 128, 1.0, null,
              null) == 0                                                    # empty batch
    assert pf(null, null, null, null, 4, 16, 8, null, null, 2, 0, 28, 4, 128, 1.0, null,
              null) == 0                                                    # no tokens
    assert pf(null, null, null, null, 4, 16, 8, null, null, 2, -1, 28, 4, 128, 1.0, null,
              null) == -1                                                   # negative tokens


def test_capi_invalid_and_unsupported_codes(mq):
    L = _L(mq)
    null = None
    qmm = L.mq_quantized_matmul
    # bits MLX does not know -> invalid; 2/3/5/6 bits without the workspace
    # their repacked codes need -> unsupported
    assert qmm(null, null, null, null, null, null, 1, 8, 64, 64, 7, 1, null) == -1
    assert b"supported bits" in L.mq_last_error()
    sixteen = ctypes.c_void_p(16)  # never dereferenced: validation fails before any launch
    assert qmm(sixteen, sixteen, sixteen, sixteen, null, sixteen, 1, 8, 64, 64, 2, 1, null) == -2
    assert b"workspace" in L.mq_last_error()
    ws = L.mq_quantized_matmul_ws
    assert ws(sixteen, sixteen, sixteen, sixteen, null, sixteen, 1, 8, 64, 64, 3, 1, sixteen, 255,
              null) == -2
    # group 32 with K = 96 beyond the GEMV's rows: refused before the repack
    assert ws(sixteen, sixteen, sixteen, sixteen, null, sixteen, 16, 8, 96, 32, 3, 1, sixteen,
              1 << 20, null) == -2 and b"multiple of 64" in L.mq_last_error()
    assert qmm(null, null, null, null, null, null, 1, 8, 64, 48, 4, 1, null) == -1
    # group sizes 32 and 128 pass the checks (null pointers are then the error)
    assert qmm(null, null, null, null, null, null, 1, 8, 64, 32, 4, 1, null) == -1
    assert b"null" in L.mq_last_error()
    assert qmm(null, null, null, null, null, null, 1, 8, 128, 128, 8, 1, null) == -1
    assert qmm(null, null, null, null, null, null, 1, 8, 96, 128, 4, 1, null) == -1
    assert b"divisible" in L.mq_last_error()
    # group size 32 with K = 96: the GEMV takes it, the 64-step GEMMs do not
    one = ctypes.c_void_p(16)  # never dereferenced: validation fails before any launch
    assert qmm(one, one, one, one, null, one, 16, 8, 96, 32, 4, 1, null) == -2
    assert b"multiple of 64" in L.mq_last_error()
    assert qmm(null, null, null, null, null, null, 1, 8, 96, 64, 4, 1, null) == -1
    assert b"divisible" in L.mq_last_error()
    assert qmm(null, null, null, null, null, null, 1, 8, 64, 64, 4, 0, null) == -2
    assert qmm(null, null, null, null, null, null, -1, 8, 64, 64, 4, 1, null) == -1
    # empty problems succeed without touching memory
    assert qmm(null, null, null, null, null, null, 0, 8, 64, 64, 4, 1, null) == 0
    assert L.mq_last_error() == b""
    # non-empty with null pointers -> invalid, nothing launched
    assert qmm(null, null, null, null, null, null, 2, 8, 64, 64, 4, 1, null) == -1
    assert b"null pointer" in L.mq_last_error()
    # misaligned x
    buf = ctypes.create_string_buffer(4096)
    base = (ctypes.addressof(buf) + 15) & ~15
    assert qmm(base + 2, base, base, base, null, base, 1, 8, 64, 64, 4, 1, null) == -1
    assert b"aligned" in L.mq_last_error()


def test_capi_gather_validation(mq):
    L = _L(mq)
    g = L.mq_gather_qmm
    null = None
    # without lhs the x batch count must equal T
    assert g(null, null, null, null, null, null, null, 4, 1, 8, 64, 2, 3, 64, 4, 1, 0, null) == -1
    assert g(null, null, null, null, null, null, null, 0, 1, 8, 64, 2, 0, 64, 4, 1, 0, null) == 0
    assert g(null, null, null, null, null, null, null, 2, 1, 8, 64, 0, 2, 64, 4, 1, 0, null) == -1
    assert g(null, null, null, null, null, null, null, 2, 1, 8, 64, 1, 2, 64, 8, 0, 0, null) == -2


def test_capi_quantize_dequantize_validation(mq):
    L = _L(mq)
    null = None
    assert L.mq_quantize(null, null, null, null, 4, 100, 64, 4, null) == -1
    assert L.mq_quantize(null, null, null, null, 0, 128, 64, 4, null) == 0
    assert L.mq_dequantize(null, null, null, null, 4, 128, 64, 6, null) == -1  # 6-bit: null ptrs
    assert b"null" in L.mq_last_error()
    rp = L.mq_repack_codes_u8
    assert rp(null, null, 4, 128, 4, null) == -1      # 4-bit codes are not repacked
    assert rp(null, null, 4, 100, 3, null) == -1      # K not a multiple of 32
    assert rp(null, null, 0, 128, 3, null) == 0       # empty
    assert rp(null, null, 2, 128, 5, null) == -1 and b"null" in L.mq_last_error()
    assert L.mq_embedding_lookup(null, 3, null, null, null, 10, 128, 64, 4, null, null) == -1


def test_python_layer_refuses_cpu_tensors(mq):
    x = torch.zeros(1, 64, dtype=torch.bfloat16)
    w = torch.zeros(8, 8, dtype=torch.int32)
    s = torch.zeros(8, 1, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        mq.quantized_matmul(x, w, s, s)
    with pytest.raises(ValueError, match="GPU"):
        mq.quantize(torch.zeros(8, 64, dtype=torch.bfloat16))


def test_python_layer_error_mapping(mq):
    with pytest.raises(ValueError):
        mq._lib.check(-1, "x")
    with pytest.raises(NotImplementedError):
        mq._lib.check(-2, "x")
    with pytest.raises(RuntimeError):
        mq._lib.check(-3, "x")
    mq._lib.check(0, "x")


def test_gather_swiglu_queries_and_validation(mq):
    """Which gathered SwiGLU shapes the fused kernel takes, and its argument errors
    (no GPU work: every call here returns before a launch)."""
    L = _L(mq)
    sup = L.mq_gather_qmm_swiglu_supported
    assert sup(64, 1, 768, 2048, 64, 4) == 1 and sup(64, 1, 768, 2048, 64, 8) == 1
    assert sup(64, 4, 768, 2048, 64, 4) == 0       # more than 2 rows per pair
    assert sup(4096, 1, 768, 2048, 64, 4) == 0     # prefill: the sorted gather GEMM
    assert sup(64, 1, 768, 2048, 32, 4) == 1 and sup(64, 1, 768, 2048, 128, 8) == 1
    assert sup(64, 1, 768, 2048, 16, 4) == 0       # group size
    assert sup(64, 1, 768, 2000, 64, 4) == 0       # K not a multiple of the group
    null = None
    f = L.mq_gather_qmm_swiglu
    assert f(null, null, null, null, null, null, null, 0, 1, 768, 2048, 128, 0, 64, 4, null) == 0
    assert f(null, null, null, null, null, null, null, 64, 1, 768, 2048, 128, 64, 64, 4,
             null) == -1                           # null pointers
    assert b"null" in L.mq_last_error()
    assert f(null, null, null, null, null, null, null, 64, 1, 768, 2048, 128, 8, 64, 4,
             null) == -1                           # no lhs: x must have T batches
    assert f(null, null, null, null, null, null, null, 64, 4, 768, 2048, 128, 64, 64, 4,
             null) == -2                           # a shape the kernel does not take


def test_plan_queries_over_a_shape_grid(mq):
    """Every host-side plan and support query over a grid of shapes -- row
    counts from 0 to 65536 around the plan boundaries, the model widths and
    odd ones, every width and group size -- answers without error and
    consistently: support queries say 0 or 1; workspaces are whole float32
    words (past any repacked codes); a fused entry that needs a workspace
    asks for no more than the plain matmul of the same product plus that
    product's repack.  (Run under tests/run_host_sanitizers.sh this sweeps
    the plan arithmetic under ASan and UBSan.)"""
    L = _L(mq)
    rows = [0, 1, 2, 3, 8, 9, 16, 17, 31, 32, 33, 64, 127, 128, 129, 255, 256, 257, 300, 512,
            1023, 1024, 2048, 4096, 8192, 65536]
    shapes = [(3584, 18944), (18944, 3584), (3584, 4608), (2048, 768), (768, 2048), (4096, 14336),
              (1024, 1000), (96, 24), (11008, 2048), (2048, 151936)]
    checked = 0
    for bits in (2, 3, 4, 5, 6, 8):
        for gs in (32, 64, 128):
            for K, N in shapes:
                for M in rows:
                    ws = L.mq_quantized_matmul_workspace(M, N, K, gs, bits)
                    assert ws >= 0
                    if bits in (4, 8):
                        assert ws % 4 == 0
                    sw = L.mq_quantized_matmul_swiglu_supported(M, N // 2, K, gs, bits)
                    assert sw in (0, 1)
                    sww = L.mq_quantized_matmul_swiglu_workspace(M, N // 2, K, gs, bits)
                    if sw and sww:
                        assert sww <= L.mq_quantized_matmul_workspace(M, 2 * (N // 2), K, gs, bits)
                    an = L.mq_quantized_matmul_add_rms_norm_supported(M, N, K, gs, bits)
                    assert an in (0, 1)
                    anw = L.mq_quantized_matmul_add_rms_norm_workspace(M, N, K, gs, bits)
                    assert (anw == 0) or an == 1
                    for swg in (0, 1):
                        assert L.mq_rms_norm_quantized_matmul_supported(M, N, K, gs, bits,
                                                                        swg) in (0, 1)
                    gq = L.mq_gather_qmm_swiglu_supported(max(M, 1), 1, N // 2, K, gs, bits)
                    assert gq in (0, 1)
                    for sg in (0, 1):
                        assert L.mq_gather_qmm_segments_supported(M, 1, N // 2 if sg else N, K,
                                                                  128, max(M, 1), gs, bits,
                                                                  sg) in (0, 1)
                    checked += 1
    assert checked == 6 * 3 * len(shapes) * len(rows)
