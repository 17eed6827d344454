/*
 * mq_cpu_baseline.c -- vectorisable float32 restatement of MLX's CPU
 * quantized_matmul loop, for bench.py's cpu_baseline leg only.
 *
 * TEST INFRASTRUCTURE (a timed baseline, not a checker and not the product):
 * only bench.py's cpu_baseline leg and the oracle's own tests load it.
 *
 * Same arithmetic per weight as orc_qmm_f32 in mq_oracle.c -- w = s*q + b in
 * float32, then x*w accumulated in float32 -- but every output keeps 16
 * partial sums (lane j takes the elements k = j mod 16 of a group) in two
 * 8-wide vectors, as MLX's CPU backend vectorises with its SIMD types (the reference's call sites: every QuantizedLinear,
 * python/mlx_worker/native_mlx/models/qwen2.py:76-78,115,134,227, which MLX
 * 0.31.2 runs on the CPU when mx.cpu is the default device).  The summation
 * order differs from orc_qmm_f32's, so it is checked against orc_qmm within
 * the matmul tolerance (tests/test_oracle_pins.py), not bit for bit.
 *
 * Build: oracle/Makefile, -O3 -mavx2 -mfma (x86-64-v3: every host here and on
 * the GPU boxes has it) with OpenMP over output rows.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define LANES 16  /* partial sums per output */

static inline float bf16f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f32_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

typedef float v8f __attribute__((vector_size(32)));
typedef uint32_t v8u __attribute__((vector_size(32)));

static inline v8f load8(const float* p) {
  v8f v;
  memcpy(&v, p, sizeof(v));
  return v;
}

/* One output: x row . dequantized weight row, in two 8-wide partial sums
 * (GCC vector extensions; AVX2 shifts, converts and FMAs).  Lane j of a
 * 16-element step holds k = k0 + j. */
static inline __attribute__((always_inline)) float row_dot(const float* xr, const uint32_t* rw,
                                                           const uint16_t* sc, const uint16_t* bi,
                                                           int64_t groups, int group_size,
                                                           const int BITS) {
  const int per_word = 32 / BITS;
  const v8u mask = (v8u){0, 0, 0, 0, 0, 0, 0, 0} + ((1u << BITS) - 1u);
  const v8u sh4 = {0, 4, 8, 12, 16, 20, 24, 28};
  const v8u sh8 = {0, 8, 16, 24, 0, 8, 16, 24};
  v8f acc0 = {0}, acc1 = {0};
  for (int64_t g = 0; g < groups; ++g) {
    const v8f s = (v8f){0} + bf16f(sc[g]);
    const v8f b = (v8f){0} + bf16f(bi[g]);
    for (int c = 0; c < group_size; c += 16) {
      const int64_t k0 = g * group_size + c;
      const uint32_t* w = rw + k0 / per_word;
      v8u c0, c1;
      if (BITS == 4) {
        c0 = (((v8u){0} + w[0]) >> sh4) & mask;
        c1 = (((v8u){0} + w[1]) >> sh4) & mask;
      } else {
        c0 = ((v8u){w[0], w[0], w[0], w[0], w[1], w[1], w[1], w[1]} >> sh8) & mask;
        c1 = ((v8u){w[2], w[2], w[2], w[2], w[3], w[3], w[3], w[3]} >> sh8) & mask;
      }
      const v8f q0 = __builtin_convertvector(c0, v8f), q1 = __builtin_convertvector(c1, v8f);
      acc0 += load8(xr + k0) * (q0 * s + b);
      acc1 += load8(xr + k0 + 8) * (q1 * s + b);
    }
  }
  float tot = 0.0f;
  for (int j = 0; j < 8; ++j) tot += acc0[j];
  for (int j = 0; j < 8; ++j) tot += acc1[j];
  return tot;
}

/* y[M, N] (bfloat16 bits) = x[M, K] @ dequantize(wq)^T; bits 4 or 8,
 * group_size a multiple of 16.  Returns 0, or -1 on bad arguments. */
int cpu_qmm_f32_lanes(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                      const uint16_t* biases, int64_t M, int64_t N, int64_t K, int group_size,
                      int bits, uint16_t* y, int threads) {
  if (M < 0 || N < 0 || K <= 0 || (bits != 4 && bits != 8) || group_size % LANES ||
      K % group_size)
    return -1;
  const int64_t groups = K / group_size;
  const int64_t words_per_row = K * bits / 32;
  float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K + 1));
  if (!xf) return -1;
  for (int64_t i = 0; i < M * K; ++i) xf[i] = bf16f(x[i]);
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(static) num_threads(threads)
  for (int64_t n = 0; n < N; ++n) {
    const uint32_t* rw = wq + n * words_per_row;
    const uint16_t* sc = scales + n * groups;
    const uint16_t* bi = biases + n * groups;
    for (int64_t m = 0; m < M; ++m) {
      const float* xr = xf + m * K;
      const float tot = bits == 4 ? row_dot(xr, rw, sc, bi, groups, group_size, 4)
                                  : row_dot(xr, rw, sc, bi, groups, group_size, 8);
      y[m * N + n] = f32_bf16(tot);
    }
  }
  free(xf);
  return 0;
}
