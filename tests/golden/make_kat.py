"""Write known-answer fixtures for MLX affine quantization
(tests/golden/kat_affine_b{2,3,4,5,6,8}.npz).

Every expected value here is fixed by construction, not computed by the oracle
or the HIP library:

* Weights are built ON the quantization grid: per group a bfloat16-exact scale
  s and integer codes q that attain both 0 and 2^bits-1, with w = s*(q - c)
  for an offset c.  For c chosen so that |min| > |max| ("pos" groups) MLX's
  quantize must return exactly (q, s, bias=-c*s); for c chosen so that
  |max| > |min| ("neg" groups) it must return (2^bits-1-q, -s, bias=max(w)).
  All-zero and constant groups have codes 0 and bias 0 / the constant.
* Every product and sum of the on-grid weights is exact in bfloat16, so
  mx.dequantize must reproduce w bit for bit.
* x holds small dyadic bfloat16 values (k/8), so x @ w^T is exact in float64.
* Codes are packed as one LSB-first bit stream per row (code k at bits
  [k*bits, (k+1)*bits) of the row's little-endian uint32 words), built here as
  a Python integer per row: for 2, 4 and 8 bits that is 32/bits codes per
  word; for 3, 5 and 6 bits it is MLX's 8, 8 and 4 codes per 3, 5 and 3 bytes.

MLX itself is not available offline, so these pin the restatement's algorithm
(sign/edge choice, refit, packing order, dequantize, matmul orientation) from
first principles.  Run: python tests/golden/make_kat.py
"""

from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GS = 64


def exact_bf16_bits(v: np.ndarray) -> np.ndarray:
    f = np.asarray(v, dtype=np.float64).astype(np.float32)
    assert np.array_equal(f.astype(np.float64), np.asarray(v, dtype=np.float64)), "not float32-exact"
    u = f.view(np.uint32)
    assert not np.any(u & 0xFFFF), "value is not bfloat16-exact"
    return (u >> 16).astype(np.uint16)


def pack(codes: np.ndarray, bits: int) -> np.ndarray:
    lead, K = codes.shape[:-1], codes.shape[-1]
    rows = []
    for r in codes.reshape(-1, K):
        stream = 0
        for k, q in enumerate(r.tolist()):
            assert 0 <= q < (1 << bits)
            stream |= q << (k * bits)
        rows.append(np.frombuffer(stream.to_bytes(K * bits // 8, "little"), "<u4"))
    return np.stack(rows).astype(np.uint32).reshape(lead + (K * bits // 32,))


# Per width: (scale exponents drawn from [lo, hi), significant fractional
# steps of the scale, c_pos, c_neg).  c_pos > nmax/2 > c_neg, and |q - c| times
# the scale's significand stays within bfloat16's 8 bits.
SCALE_RULES = {2: (4, 7, 8, 2, 1), 3: (5, 8, 8, 5, 2), 4: (5, 8, 8, 9, 6),
               5: (6, 9, 4, 18, 13), 6: (7, 10, 2, 36, 27), 8: (8, 11, 1, 130, 125)}


def build_matrix(rng, rows: int, K: int, bits: int):
    nmax = (1 << bits) - 1
    groups = K // GS
    w = np.zeros((rows, K), np.float64)
    codes = np.zeros((rows, K), np.int64)
    scales = np.zeros((rows, groups), np.float64)
    biases = np.zeros((rows, groups), np.float64)
    checked = np.zeros((rows, groups), bool)
    kinds = ["pos", "neg", "pos", "neg", "zero", "const"]
    for r in range(rows):
        for g in range(groups):
            kind = kinds[(r * groups + g) % len(kinds)] if (r + g) % 7 else "pos"
            sl = slice(g * GS, (g + 1) * GS)
            if kind in ("pos", "neg"):
                lo, hi, steps, c_pos, c_neg = SCALE_RULES[bits]
                if bits == 8:
                    s = 2.0 ** -int(rng.integers(lo, hi))
                else:
                    s = 2.0 ** -int(rng.integers(lo, hi)) * (1 + int(rng.integers(0, steps)) / steps)
                q = rng.integers(0, nmax + 1, GS)
                q[rng.integers(0, GS)] = 0
                q[(rng.integers(1, GS) + 0) % GS] = nmax
                if not (q == 0).any():
                    q[0] = 0
                if not (q == nmax).any():
                    q[1] = nmax
                if kind == "pos":
                    w[r, sl] = s * (q - c_pos)
                    codes[r, sl] = q
                    scales[r, g], biases[r, g] = s, -c_pos * s
                else:
                    w[r, sl] = s * (q - c_neg)
                    codes[r, sl] = nmax - q
                    scales[r, g], biases[r, g] = -s, (nmax - c_neg) * s
                checked[r, g] = True
            elif kind == "zero":
                w[r, sl] = 0.0
            else:
                cval = float(rng.integers(-64, 64) or 1) / 256.0
                w[r, sl] = cval
                biases[r, g] = cval
    return w, codes, scales, biases, checked


def main() -> None:
    rng = np.random.default_rng(1234)
    # 4 and 8 first: the random stream (and so their fixtures) is unchanged
    # by the widths added after them
    for bits in (4, 8, 2, 3, 5, 6):
        rows, K, M = 12, 256, 3
        w, codes, scales, biases, checked = build_matrix(rng, rows, K, bits)
        x = rng.integers(-16, 17, (M, K)) / 8.0
        y = x @ w.T
        E, Ng, T = 3, 8, 5
        gw = np.zeros((E, Ng, K))
        gcodes = np.zeros((E, Ng, K), np.int64)
        gs_ = np.zeros((E, Ng, K // GS))
        gb_ = np.zeros((E, Ng, K // GS))
        for e in range(E):
            gw[e], gcodes[e], gs_[e], gb_[e], _ = build_matrix(rng, Ng, K, bits)
        rhs = np.array([2, 0, 2, 1, 0], np.int32)
        gx = rng.integers(-16, 17, (T, 1, K)) / 8.0
        gy = np.stack([gx[t] @ gw[rhs[t]].T for t in range(T)])
        np.savez(
            os.path.join(HERE, f"kat_affine_b{bits}.npz"),
            bits=np.int32(bits), group_size=np.int32(GS),
            w=exact_bf16_bits(w), wq=pack(codes, bits),
            scales=exact_bf16_bits(scales), biases=exact_bf16_bits(biases),
            scale_checked=checked, deq=exact_bf16_bits(w),
            x=exact_bf16_bits(x), y=y,
            gw=exact_bf16_bits(gw), gwq=pack(gcodes, bits),
            gscales=exact_bf16_bits(gs_), gbiases=exact_bf16_bits(gb_),
            rhs=rhs, gx=exact_bf16_bits(gx), gy=gy,
        )
        print(f"wrote kat_affine_b{bits}.npz")


if __name__ == "__main__":
    main()
