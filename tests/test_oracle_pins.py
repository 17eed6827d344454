"""Pins for the CPU oracle (oracle/mq_oracle.c).

MLX (the library the reference delegates this path to) cannot be imported
here, and the reference's own tests never quantize, so the oracle is pinned by
known answers and mathematics that a plausible mistake would break:

* packing: hand-written words whose codes are known;
* dequantize: hand-derived values, including one case where one rounding and
  two roundings give different bfloat16 results;
* quantize: on-grid fixtures (tests/golden/make_kat.py) for both scale signs,
  zero and constant groups; brute-force nearest-code search on random data;
  exactness of 0.0 after the edge refit;
* quantized_matmul: one-hot inputs, all-zero codes, numpy matmul of the
  dequantized matrix, the float32 MLX-CPU-style variant;
* gather_qmm: reduction to per-expert matmuls, permutation equivariance.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import normwise_rel_err

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bf16_bits(x: float) -> int:
    """bfloat16 bits of a value that is exactly representable (asserted)."""
    u = int(np.array([x], np.float32).view(np.uint32)[0])
    assert u & 0xFFFF == 0
    return u >> 16


def load_kat(bits):
    return dict(np.load(os.path.join(GOLDEN, f"kat_affine_b{bits}.npz"), allow_pickle=False))


# ----------------------------------------------------------------- packing


def test_pack_known_word_4bit(orc):
    wq = np.full((1, 8), 0x76543210, np.uint32)  # one group of 64 codes
    s = np.array([[bf16_bits(1.0)]], np.uint16)
    b = np.array([[0]], np.uint16)
    out = orc.bf16_to_f32(orc.dequantize(wq, s, b, 64, 4))
    assert out.tolist() == [list(range(8)) * 8]


def test_pack_known_word_8bit(orc):
    wq = np.full((1, 16), 0xFE020100, np.uint32)
    s = np.array([[bf16_bits(1.0)]], np.uint16)
    b = np.array([[0]], np.uint16)
    out = orc.bf16_to_f32(orc.dequantize(wq, s, b, 64, 8))
    assert out.tolist() == [[0.0, 1.0, 2.0, 254.0] * 16]


# Widths that do not divide 32 continue the LSB-first stream across words
# (MLX: 8 3-bit codes in 3 bytes, 4 6-bit codes in 3 bytes, 8 5-bit codes in
# 5 bytes).  Words below are written out by hand from those byte patterns.
STREAM_KATS = {
    # 3-bit codes 0..7 -> octal 76543210 = bytes 88 C6 FA, repeated
    3: ([0x88FAC688, 0xC688FAC6, 0xFAC688FA] * 2, list(range(8)) * 8),
    # 6-bit codes 1..4 -> octal 04030201 = bytes 81 30 10, repeated
    6: ([0x81103081, 0x30811030, 0x10308110] * 4, [1, 2, 3, 4] * 16),
    # 5-bit: a 1 every 8th code sets stream bits 0, 40, 80, 120 of each 160
    5: ([0x1, 0x100, 0x10000, 0x1000000, 0x0] * 2, ([1] + [0] * 7) * 8),
    # 2-bit: byte E4 = codes 0, 1, 2, 3
    2: ([0xE4E4E4E4] * 4, [0, 1, 2, 3] * 16),
}


@pytest.mark.parametrize("bits", sorted(STREAM_KATS))
def test_pack_known_words_stream(orc, bits):
    words, codes = STREAM_KATS[bits]
    wq = np.array([words], np.uint32)
    s = np.array([[bf16_bits(1.0)]], np.uint16)
    b = np.array([[0]], np.uint16)
    out = orc.bf16_to_f32(orc.dequantize(wq, s, b, 64, bits))
    assert out.tolist() == [[float(c) for c in codes]]


def test_pack_straddling_code(orc):
    # 3-bit code 10 holds bits 30..32: two bits in word 0, one in word 1
    wq = np.array([[0xC0000000, 0x1, 0, 0, 0, 0]], np.uint32)
    s = np.array([[bf16_bits(1.0)]], np.uint16)
    b = np.array([[0]], np.uint16)
    out = orc.bf16_to_f32(orc.dequantize(wq, s, b, 64, 3))[0]
    assert out[10] == 7.0 and np.count_nonzero(out) == 1
    # quantize through the same boundary: zeros with 1.75 at k = 10 refit to
    # scale -0.25 and bias 1.75 (the larger-magnitude edge), so the zeros are
    # code 7 and k = 10 is code 0: every bit set but 30, 31 and 32
    w = np.zeros((1, 64), np.uint16)
    w[0, 10] = bf16_bits(1.75)
    wq2, s2, b2 = orc.quantize(w, 64, 3)
    assert wq2.tolist() == [[0x3FFFFFFF, 0xFFFFFFFE] + [0xFFFFFFFF] * 4]
    assert s2[0, 0] == bf16_bits(-0.25) and b2[0, 0] == bf16_bits(1.75)
    assert orc.bf16_to_f32(orc.dequantize(wq2, s2, b2, 64, 3)).tolist() == \
        orc.bf16_to_f32(w).tolist()


def unpack_stream(wq: np.ndarray, bits: int) -> np.ndarray:
    """Codes [rows, K] of LSB-first stream-packed rows, through Python integers."""
    rows = wq.reshape(-1, wq.shape[-1])
    K = wq.shape[-1] * 32 // bits
    out = np.empty((rows.shape[0], K), np.int64)
    for r, row in enumerate(rows):
        stream = int.from_bytes(row.astype("<u4").tobytes(), "little")
        out[r] = [(stream >> (k * bits)) & ((1 << bits) - 1) for k in range(K)]
    return out


# -------------------------------------------------------------- dequantize


def test_dequantize_exact_grid(orc):
    # s = 1/16, b = -0.5: every q*s + b is exact, so the output is q/16 - 1/2.
    wq = np.full((1, 8), 0xFEDCBA98, np.uint32)
    s = np.array([[bf16_bits(0.0625)]], np.uint16)
    b = np.array([[bf16_bits(-0.5)]], np.uint16)
    out = orc.bf16_to_f32(orc.dequantize(wq, s, b, 64, 4))[0]
    assert out[:8].tolist() == [q / 16 - 0.5 for q in range(8, 16)]


def test_dequantize_rounds_twice(orc):
    # q=3, s=1+2^-7, b=-2^-7.  q*s = 3.0234375 is a bfloat16 tie that rounds to
    # even (3.03125); adding b gives 3.0234375 again, which rounds to 3.03125.
    # A single rounding of q*s+b = 3.015625 (exact) would give 3.015625.
    wq = np.full((1, 8), 0x33333333, np.uint32)
    s = np.array([[bf16_bits(1.0078125)]], np.uint16)
    b = np.array([[bf16_bits(-0.0078125)]], np.uint16)
    out = orc.dequantize(wq, s, b, 64, 4)
    assert np.all(out == bf16_bits(3.03125))
    exact = orc.dequantize(wq, s, b, 64, 4, exact=True)
    assert np.all(exact == 3.015625)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_dequantize_kat_fixture(orc, bits):
    kat = load_kat(bits)
    out = orc.dequantize(kat["wq"], kat["scales"], kat["biases"], 64, bits)
    assert np.array_equal(orc.bf16_to_f32(out), orc.bf16_to_f32(kat["deq"]))


# ---------------------------------------------------------------- quantize


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_quantize_on_grid_fixture(orc, bits):
    kat = load_kat(bits)
    wq, s, b = orc.quantize(kat["w"], 64, bits)
    assert np.array_equal(wq, kat["wq"])
    chk = kat["scale_checked"]
    assert np.array_equal(s[chk], kat["scales"][chk])
    assert np.array_equal(b, kat["biases"])
    # zero groups: negative eps-sized scale; every group dequantizes exactly
    assert np.all(orc.bf16_to_f32(s[~chk]) < 0)
    deq = orc.dequantize(wq, s, b, 64, bits)
    assert np.array_equal(orc.bf16_to_f32(deq), orc.bf16_to_f32(kat["w"]))


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_quantize_codes_are_nearest(orc, bits):
    rng = np.random.default_rng(7)
    w = orc.f32_to_bf16(rng.normal(0, 0.02, (33, 256)).astype(np.float32))
    wq, s, b, s32, b32 = orc.quantize(w, 64, bits, with_f32=True)
    codes = unpack_stream(wq, bits).astype(np.float64)
    wf = orc.bf16_to_f32(w).astype(np.float64).reshape(33, 4, 64)
    sg = s32.astype(np.float64)[..., None]
    bg = b32.astype(np.float64)[..., None]
    grid = np.arange(1 << bits, dtype=np.float64)
    # brute force: distance of every element to every representable value
    dist = np.abs(wf[..., None] - (sg[..., None] * grid + bg[..., None]))
    best = dist.min(-1)
    got = np.abs(wf - (sg * codes.reshape(33, 4, 64) + bg))
    # (w - b) / s is a float32 division: near-ties may land on either side,
    # so allow 1e-4 of a code step; floor/ceil/clamp mistakes cost up to 1.
    assert np.all(got <= best + 1e-4 * np.abs(sg))
    # the stored scale/bias are the float32 values rounded to bfloat16
    assert np.array_equal(s, orc.f32_to_bf16(s32))
    assert np.array_equal(b, orc.f32_to_bf16(b32))
    # every group spans (close to) the full code range
    assert np.all(np.abs(s32) > 0)


def test_quantize_zero_is_exact(orc):
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, (16, 128)).astype(np.float32)
    w[:, ::5] = 0.0
    wb = orc.f32_to_bf16(w)
    wq, s, b, s32, b32 = orc.quantize(wb, 64, 4, with_f32=True)
    codes = np.stack([(wq >> np.uint32(j * 4)) & np.uint32(15) for j in range(8)], -1).reshape(16, 128)
    val = s32.repeat(64, 1).astype(np.float64) * codes + b32.repeat(64, 1)
    zero = orc.bf16_to_f32(wb) == 0
    assert np.all(np.abs(val[zero]) <= 16 * np.abs(s32.repeat(64, 1)[zero]) * 2.0 ** -23)


def test_quantize_rejects_bad_params(orc):
    w = np.zeros((2, 64), np.uint16)
    with pytest.raises(ValueError):
        orc.quantize(w, 64, 7)
    with pytest.raises(ValueError):
        orc.quantize(w, 48, 4)
    with pytest.raises(ValueError):
        orc.quantize(np.zeros((2, 96), np.uint16), 64, 4)


# ---------------------------------------------------------- quantized_matmul


def _rand_quantized(orc, rng, N, K, bits):
    w = orc.f32_to_bf16(rng.normal(0, 0.02, (N, K)).astype(np.float32))
    return orc.quantize(w, 64, bits)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_qmm_kat_fixture(orc, bits):
    kat = load_kat(bits)
    y = orc.qmm(kat["x"], kat["wq"], kat["scales"], kat["biases"], 64, bits)
    assert np.allclose(y, kat["y"], rtol=2e-7, atol=1e-6)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_qmm_one_hot_reads_dequantized_column(orc, bits):
    rng = np.random.default_rng(11)
    wq, s, b = _rand_quantized(orc, rng, 24, 192, bits)
    ex = orc.dequantize(wq, s, b, 64, bits, exact=True)
    for k in (0, 63, 64, 191):
        x = np.zeros((1, 192), np.uint16)
        x[0, k] = bf16_bits(1.0)
        y = orc.qmm(x, wq, s, b, 64, bits)
        assert np.array_equal(y[0], ex[:, k].astype(np.float32))


def test_qmm_zero_codes_sum_biases(orc):
    rng = np.random.default_rng(12)
    N, K = 10, 256
    wq = np.zeros((N, K // 8), np.uint32)
    s = orc.f32_to_bf16(rng.normal(0, 1, (N, K // 64)).astype(np.float32))
    b = orc.f32_to_bf16(rng.normal(0, 1, (N, K // 64)).astype(np.float32))
    x = orc.f32_to_bf16(rng.normal(0, 1, (3, K)).astype(np.float32))
    y = orc.qmm(x, wq, s, b, 64, 4)
    xs = orc.bf16_to_f32(x).astype(np.float64).reshape(3, K // 64, 64).sum(-1)
    ref = xs @ orc.bf16_to_f32(b).astype(np.float64).T
    assert np.allclose(y, ref, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_qmm_matches_numpy_matmul(orc, bits):
    rng = np.random.default_rng(13)
    wq, s, b = _rand_quantized(orc, rng, 40, 320, bits)
    x = orc.f32_to_bf16(rng.normal(0, 1, (5, 320)).astype(np.float32))
    bias = orc.f32_to_bf16(rng.normal(0, 1, (40,)).astype(np.float32))
    ex = orc.dequantize(wq, s, b, 64, bits, exact=True)
    ref = orc.bf16_to_f32(x).astype(np.float64) @ ex.T + orc.bf16_to_f32(bias)
    y = orc.qmm(x, wq, s, b, 64, bits, bias=bias)
    assert np.allclose(y, ref, rtol=1e-6, atol=1e-7)
    # each row alone gives the same result (M-invariance)
    for m in range(5):
        assert np.array_equal(orc.qmm(x[m:m + 1], wq, s, b, 64, bits, bias=bias)[0], y[m])


@pytest.mark.parametrize("bits", [4, 8])
def test_qmm_f32_variant_close_to_double(orc, bits):
    rng = np.random.default_rng(14)
    wq, s, b = _rand_quantized(orc, rng, 64, 512, bits)
    x = orc.f32_to_bf16(rng.normal(0, 1, (3, 512)).astype(np.float32))
    ref = orc.qmm(x, wq, s, b, 64, bits)
    y = orc.bf16_to_f32(orc.qmm_f32(x, wq, s, b, 64, bits, threads=2))
    assert normwise_rel_err(y, ref) < 5e-3  # bfloat16 output rounding dominates
    y1 = orc.qmm_f32(x, wq, s, b, 64, bits, threads=1)
    assert np.array_equal(orc.bf16_to_f32(y1), y)
    # the vectorised loop the CPU baseline times: same products, 16 partial sums
    yl = orc.bf16_to_f32(orc.qmm_f32_lanes(x, wq, s, b, 64, bits, threads=2))
    assert normwise_rel_err(yl, ref) < 5e-3
    assert np.array_equal(orc.qmm_f32_lanes(x, wq, s, b, 64, bits, threads=1),
                          orc.f32_to_bf16(yl))


# ---------------------------------------------------------------- gather_qmm


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_gather_kat_fixture(orc, bits):
    kat = load_kat(bits)
    y = orc.gather_qmm(kat["gx"], kat["gwq"], kat["gscales"], kat["gbiases"], kat["rhs"],
                       group_size=64, bits=bits)
    assert np.allclose(y, kat["gy"], rtol=2e-7, atol=1e-6)


def test_gather_reduces_to_per_expert_qmm(orc):
    rng = np.random.default_rng(15)
    E, N, K, T = 4, 16, 128, 9
    w = orc.f32_to_bf16(rng.normal(0, 0.02, (E, N, K)).astype(np.float32))
    wq, s, b = orc.quantize(w, 64, 4)
    x = orc.f32_to_bf16(rng.normal(0, 1, (3, 2, K)).astype(np.float32))
    rhs = rng.integers(0, E, T).astype(np.int32)
    lhs = rng.integers(0, 3, T).astype(np.int32)
    y = orc.gather_qmm(x, wq, s, b, rhs, lhs_indices=lhs)
    for t in range(T):
        ref = orc.qmm(x[lhs[t]], wq[rhs[t]], s[rhs[t]], b[rhs[t]])
        assert np.array_equal(y[t], ref)
    # sorting the rows (models/lfm2.py:613-618) permutes the output rows only
    order = np.argsort(rhs, kind="stable")
    ys = orc.gather_qmm(x, wq, s, b, rhs[order], lhs_indices=lhs[order])
    assert np.array_equal(ys, y[order])
    with pytest.raises(ValueError):
        orc.gather_qmm(x, wq, s, b, np.array([E], np.int32), lhs_indices=np.array([0], np.int32))
