/*
 * mq_oracle.c -- CPU restatement of MLX affine group-wise quantization.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP library:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it.  Nothing in the product path (mlx-server-runtime_amd/) may import,
 * link or call it.
 *
 * The reference (huydt84/mlx-server-runtime) delegates every op on this path
 * to the third-party package mlx 0.31.2 (python/uv.lock:939-941), which is not
 * vendored under the reference tree and cannot be installed offline.  The
 * functions below restate MLX's published affine-quantization algorithm; the
 * reference call sites they stand behind are:
 *   - mx.quantize:           models/lfm2.py:112-117,142-151; nn.quantize at
 *                            models/qwen2.py:318-324
 *   - mx.dequantize:         quantized embedding lookup (models/qwen2.py:185,
 *                            reached through nn.QuantizedEmbedding)
 *   - mx.quantized_matmul:   every QuantizedLinear (models/qwen2.py:76-78,115,
 *                            134,227)
 *   - mx.gather_qmm:         QuantizedSwitchLinear.__call__ at
 *                            models/lfm2.py:176-187
 * (paths relative to python/mlx_worker/native_mlx/).
 *
 * Format (MLX "affine" mode): a row of K weights is split into K/group_size
 * groups.  Each group has one scale s and one bias b (stored in the weight
 * dtype, bfloat16 here) and the weight is w = s*q + b with an integer code q
 * in [0, 2^bits).  Codes are packed LSB-first as one bit stream per row: code
 * k of a row occupies bits [k*bits, (k+1)*bits) of the row's uint32 words
 * read as a little-endian stream.  For 2, 4 and 8 bits that is 32/bits codes
 * per word (code j of a word at bits [j*bits, (j+1)*bits)); for 3, 5 and 6
 * bits MLX packs 8, 8 and 4 codes into 3, 5 and 3 bytes, which is the same
 * stream, a code possibly straddling two words.  A group (>= 32 codes) always
 * fills whole words.
 *
 * Pins (tests/test_oracle_pins.py): packing known-answer words (every width,
 * including codes that straddle a word boundary), hand-derived
 * dequantize values that separate one rounding from two, on-grid round trips
 * through quantize for both scale signs, brute-force nearest-code search, the
 * zero-exactness property of the edge refit, one-hot and all-zero-code
 * matmul identities, and numpy matmul of the dequantized matrix.
 *
 * Parity unpinned against MLX itself (only an import of mlx could pin these,
 * and mlx is absent): the rounding sequence of mx.dequantize (restated here
 * as bf16(bf16(q*s) + b), MLX's op-graph order), the tie-breaking and refit
 * of mx.quantize on weights that are not on the quantization grid, and the
 * accumulation order of MLX's CPU quantized_matmul.  The restatement itself
 * is pinned by the checks above.
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off so no multiply-add is fused:
 * every float operation below rounds exactly once, as written).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_OK 0
#define ORC_EINVAL -1

static inline float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* float -> bfloat16, round to nearest even (the conversion MLX's bfloat16
 * type performs on every store). NaN stays a quiet NaN. */
static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

uint16_t orc_f32_to_bf16(float f) { return f32_to_bf16(f); }
float orc_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }

static int check_params(int64_t rows, int64_t K, int group_size, int bits) {
  if (rows < 0 || K <= 0) return ORC_EINVAL;
  if (bits != 2 && bits != 3 && bits != 4 && bits != 5 && bits != 6 && bits != 8)
    return ORC_EINVAL;
  if (group_size != 32 && group_size != 64 && group_size != 128) return ORC_EINVAL;
  if (K % group_size) return ORC_EINVAL;
  return ORC_OK;
}

/*
 * mx.quantize(w, group_size, bits, mode="affine") for bfloat16 w[rows, K].
 * Per group (all arithmetic in float32):
 *   w_min, w_max over the group
 *   mask  = |w_min| > |w_max|
 *   scale = max((w_max - w_min) / (2^bits - 1), 1e-7), negated unless mask
 *   edge  = mask ? w_min : w_max
 *   q0    = rint(edge / scale)
 *   if q0 != 0: scale = edge / q0, bias = edge        (makes 0.0 exact)
 *   else:       bias = 0
 *   q     = clamp(rint((w - bias) / scale), 0, 2^bits - 1)
 * scale and bias are then stored rounded to bfloat16; the codes are computed
 * from the float32 values.  rint rounds half to even.
 * scales_f32/biases_f32 (nullable) receive the float32 values before the
 * bfloat16 store, for the brute-force code check in the tests.
 */
int orc_quantize(const uint16_t* w, int64_t rows, int64_t K, int group_size, int bits,
                 uint32_t* wq, uint16_t* scales, uint16_t* biases,
                 float* scales_f32, float* biases_f32) {
  if (check_params(rows, K, group_size, bits)) return ORC_EINVAL;
  const float n_bins = (float)((1 << bits) - 1);
  const float eps = 1e-7f;
  const int64_t groups = K / group_size;
  const int64_t words_per_row = K * bits / 32;
  const int group_words = group_size * bits / 32;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < groups; ++g) {
      const uint16_t* src = w + r * K + g * group_size;
      float w_min = INFINITY, w_max = -INFINITY;
      for (int j = 0; j < group_size; ++j) {
        float v = bf16_to_f32(src[j]);
        w_max = (w_max < v) ? v : w_max;
        w_min = (v < w_min) ? v : w_min;
      }
      int mask = fabsf(w_min) > fabsf(w_max);
      float scale = (w_max - w_min) / n_bins;
      scale = (scale < eps) ? eps : scale;
      scale = mask ? scale : -scale;
      float edge = mask ? w_min : w_max;
      float q0 = rintf(edge / scale);
      float bias = 0.0f;
      if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
      }
      uint32_t* dst = wq + r * words_per_row + g * group_words;
      for (int wd = 0; wd < group_words; ++wd) dst[wd] = 0;
      for (int j = 0; j < group_size; ++j) {
        float v = bf16_to_f32(src[j]);
        float q = rintf((v - bias) / scale);
        q = (q < 0.0f) ? 0.0f : q;
        q = (q > n_bins) ? n_bins : q;
        /* bit p of the group's stream; the high part of a straddling code
         * goes to the next word */
        const int p = j * bits;
        dst[p >> 5] |= (uint32_t)q << (p & 31);
        if ((p & 31) + bits > 32) dst[(p >> 5) + 1] |= (uint32_t)q >> (32 - (p & 31));
      }
      scales[r * groups + g] = f32_to_bf16(scale);
      biases[r * groups + g] = f32_to_bf16(bias);
      if (scales_f32) scales_f32[r * groups + g] = scale;
      if (biases_f32) biases_f32[r * groups + g] = bias;
    }
  }
  return ORC_OK;
}

/* code k of a row: bits [k*bits, (k+1)*bits) of the row's word stream */
static inline uint32_t code_at(const uint32_t* row_words, int64_t k, int bits) {
  const int64_t p = k * bits;
  uint64_t v = row_words[p >> 5];
  if ((p & 31) + bits > 32) v |= (uint64_t)row_words[(p >> 5) + 1] << 32;
  return (uint32_t)(v >> (p & 31)) & ((1u << bits) - 1u);
}

/*
 * mx.dequantize(wq, scales, biases, group_size, bits) for bfloat16 scales.
 * MLX evaluates it as two element-wise ops in the output dtype: the unpacked
 * codes are multiplied by the scale, then the bias is added, and each op
 * rounds to bfloat16:  out = bf16(bf16(q * s) + b).
 * out_exact (nullable) receives the unrounded value q*s + b in double, which
 * is the weight the matmul reference below contracts with.
 */
int orc_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                   int64_t rows, int64_t K, int group_size, int bits,
                   uint16_t* out, double* out_exact) {
  if (check_params(rows, K, group_size, bits)) return ORC_EINVAL;
  const int64_t groups = K / group_size;
  const int64_t words_per_row = K * bits / 32;
  for (int64_t r = 0; r < rows; ++r) {
    const uint32_t* rw = wq + r * words_per_row;
    for (int64_t k = 0; k < K; ++k) {
      const int64_t gi = r * groups + k / group_size;
      const float s = bf16_to_f32(scales[gi]);
      const float b = bf16_to_f32(biases[gi]);
      const uint32_t q = code_at(rw, k, bits);
      if (out) {
        const float t = bf16_to_f32(f32_to_bf16((float)q * s));
        out[r * K + k] = f32_to_bf16(t + b);
      }
      if (out_exact) out_exact[r * K + k] = (double)q * (double)s + (double)b;
    }
  }
  return ORC_OK;
}

/*
 * mx.quantized_matmul(x, wq, scales, biases, transpose=True, group_size, bits)
 * followed by QuantizedLinear's optional "+ bias":
 *   y[m, n] = sum_k x[m, k] * (s[n, k/gs] * q[n, k] + b[n, k/gs])  (+ bias[n])
 * x is bfloat16 [M, K], wq is [N, K*bits/32].  Accumulated in double from the
 * exact dequantized weight; the float32 result is what a bfloat16 output is
 * compared against (within a tolerance).
 */
int orc_qmm(const uint16_t* x, const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
            const uint16_t* bias, int64_t M, int64_t N, int64_t K, int group_size, int bits,
            float* y) {
  if (M < 0 || check_params(N, K, group_size, bits)) return ORC_EINVAL;
  const int64_t groups = K / group_size;
  const int64_t words_per_row = K * bits / 32;
  double* wrow = (double*)malloc(sizeof(double) * (size_t)K);
  double* xd = (double*)malloc(sizeof(double) * (size_t)(M * K + 1));
  if (!wrow || !xd) { free(wrow); free(xd); return ORC_EINVAL; }
  for (int64_t i = 0; i < M * K; ++i) xd[i] = bf16_to_f32(x[i]);
  for (int64_t n = 0; n < N; ++n) {
    const uint32_t* rw = wq + n * words_per_row;
    for (int64_t k = 0; k < K; ++k) {
      const int64_t gi = n * groups + k / group_size;
      wrow[k] = (double)code_at(rw, k, bits) * (double)bf16_to_f32(scales[gi]) +
                (double)bf16_to_f32(biases[gi]);
    }
    const double add = bias ? (double)bf16_to_f32(bias[n]) : 0.0;
    for (int64_t m = 0; m < M; ++m) {
      double acc = 0.0;
      const double* xr = xd + m * K;
      for (int64_t k = 0; k < K; ++k) acc += xr[k] * wrow[k];
      y[m * N + n] = (float)(acc + add);
    }
  }
  free(wrow);
  free(xd);
  return ORC_OK;
}

/*
 * MLX CPU-backend style quantized_matmul (transpose=True): the weight is
 * dequantized to float32 one group at a time (w = q*s, then + b, each a
 * float32 op) and accumulated in float32 per output, then rounded to bfloat16.
 * Rows n are split across `threads` OpenMP threads.  This is the function the
 * CPU baseline times; the tests check it against orc_qmm.
 */
int orc_qmm_f32(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                const uint16_t* biases, int64_t M, int64_t N, int64_t K, int group_size,
                int bits, uint16_t* y, int threads) {
  if (M < 0 || check_params(N, K, group_size, bits)) return ORC_EINVAL;
  const int64_t groups = K / group_size;
  const int64_t words_per_row = K * bits / 32;
  const int per_word = 32 % bits ? 1 : 32 / bits;  /* word-aligned widths only */
  const uint32_t mask = (1u << bits) - 1u;
  float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K + 1));
  if (!xf) return ORC_EINVAL;
  for (int64_t i = 0; i < M * K; ++i) xf[i] = bf16_to_f32(x[i]);
#ifdef _OPENMP
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
  for (int64_t n = 0; n < N; ++n) {
    const uint32_t* rw = wq + n * words_per_row;
    for (int64_t m = 0; m < M; ++m) {
      const float* xr = xf + m * K;
      float acc = 0.0f;
      for (int64_t g = 0; g < groups; ++g) {
        const float s = bf16_to_f32(scales[n * groups + g]);
        const float b = bf16_to_f32(biases[n * groups + g]);
        const float* gx = xr + g * group_size;
        if (32 % bits) {  /* 3, 5, 6 bits: codes from the stream */
          for (int j = 0; j < group_size; ++j) {
            float wv = (float)code_at(rw, g * group_size + j, bits) * s;
            wv = wv + b;
            acc = acc + gx[j] * wv;
          }
          continue;
        }
        const uint32_t* gw = rw + g * (group_size / per_word);
        for (int wd = 0; wd < group_size / per_word; ++wd) {
          uint32_t word = gw[wd];
          for (int p = 0; p < per_word; ++p) {
            float wv = (float)(word & mask) * s;
            wv = wv + b;
            acc = acc + gx[wd * per_word + p] * wv;
            word >>= bits;
          }
        }
      }
      y[m * N + n] = f32_to_bf16(acc);
    }
  }
  free(xf);
  return ORC_OK;
}

/*
 * mx.gather_qmm(x, wq, scales, biases, lhs_indices, rhs_indices,
 *               transpose=True, group_size, bits, sorted_indices):
 *   y[t] = x[lhs[t]] @ dequantize(wq[rhs[t]])^T    for t in [0, T)
 * x is bfloat16 [x_batches, M, K]; wq is [E, N, K*bits/32]; scales and biases
 * are [E, N, K/gs]; y is float32 [T, M, N].  lhs == NULL means lhs[t] = t.
 * sorted_indices is a performance hint only; the result does not depend on
 * it (models/lfm2.py:202-218 uses it after an argsort of the expert ids).
 */
int orc_gather_qmm(const uint16_t* x, const int32_t* lhs, const int32_t* rhs,
                   const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                   int64_t T, int64_t M, int64_t N, int64_t K, int64_t E, int64_t x_batches,
                   int group_size, int bits, float* y) {
  if (T < 0 || E <= 0 || x_batches < 0 || check_params(N, K, group_size, bits)) return ORC_EINVAL;
  if (!lhs && x_batches != T) return ORC_EINVAL;
  const int64_t w_stride = N * (K * bits / 32);
  const int64_t s_stride = N * (K / group_size);
  for (int64_t t = 0; t < T; ++t) {
    const int64_t xb = lhs ? lhs[t] : t;
    const int64_t e = rhs[t];
    if (xb < 0 || xb >= x_batches || e < 0 || e >= E) return ORC_EINVAL;
    int rc = orc_qmm(x + xb * M * K, wq + e * w_stride, scales + e * s_stride,
                     biases + e * s_stride, NULL, M, N, K, group_size, bits, y + t * M * N);
    if (rc) return rc;
  }
  return ORC_OK;
}
