// Decode-shaped quantized matmul (qmv): y[m, n] = sum_k x[m, k] * (s*q + b)[n, k]
// for a few activation rows (M <= 8).  This is mx.quantized_matmul(x, w, scales,
// biases, transpose=True) as called by every QuantizedLinear at decode
// (python/mlx_worker/native_mlx/models/qwen2.py:76-78,115,134,227), and, with a
// per-batch expert index, mx.gather_qmm for unsorted / few-row MoE calls
// (models/lfm2.py:176-187).
//
// HBM-bound: every weight byte is read once.  Design for gfx950:
//  * a row of W is TPR lanes wide; lane i reads 16-byte chunks i, i+TPR, ...
//    (32 4-bit or 16 8-bit codes per chunk), R rows per lane slot, all loads
//    of a slot issued before any math;
//  * x is staged once per block in LDS, structure-of-arrays by 16-byte block
//    so that consecutive lanes read consecutive LDS addresses; for 4-bit it is
//    stored in "pair order" (x0,x4),(x1,x5),(x2,x6),(x3,x7) per 8 elements,
//    together with the sum of x over every chunk;
//  * 4-bit: (word >> 4t) & 0x000F000F | 0x43004300 is a pair of bfloat16
//    numbers 128+q (exact), fed to v_dot2_f32_bf16 against the x pair; per
//    chunk the result d = sum x*(128+q) turns into the group contribution
//    s*d + (b - 128*s)*sum(x), the same value as sum x*(s*q+b);
//  * 8-bit: v_cvt_f32_ubyte{0..3} + fma in float32, then s*d + b*sum(x);
//  * partial sums are reduced across the TPR lanes of a row with lane
//    shuffles; float32 accumulation throughout, one bfloat16 rounding at the
//    store (+ optional bias, QuantizedLinear's "+ bias" fused).
#include "mq_common.h"
#include "mq_internal.h"

namespace mq {
namespace {

constexpr int kBlock = 256;
constexpr int kQmvLdsBudget = 48 * 1024;

template <int BITS, int TPR, int R, int MT>
__global__ __launch_bounds__(kBlock) void qmv_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K,
    const int32_t* __restrict__ lhs, const int32_t* __restrict__ rhs, int64_t E,
    int64_t x_batches) {
  constexpr int EPC = 128 / BITS;  // elements per 16-byte chunk
  constexpr int UPC = EPC / 8;     // 8-element units per chunk (4 or 2)
  constexpr int SLOTS = kBlock / TPR;
  extern __shared__ u32x4_t smem[];

  const int C = K / EPC;  // chunks per row
  const int G = K / kGroup;
  const int64_t t = blockIdx.y;
  int64_t xb = t, e = 0;
  if (lhs) xb = lhs[t];
  if (rhs) e = rhs[t];
  const int slot = threadIdx.x / TPR;
  const int lane = threadIdx.x % TPR;
  const int row0 = (blockIdx.x * SLOTS + slot) * R;
  y += t * (int64_t)M * N;
  if (xb < 0 || xb >= x_batches || e < 0 || e >= E) {  // index outside the tables: zeros
    if (lane == 0)
      for (int r = 0; r < R; ++r)
        for (int m = 0; m < M; ++m)
          if (row0 + r < N) y[(int64_t)m * N + row0 + r] = 0;
    return;
  }
  x += xb * (int64_t)M * K;
  wq += e * (int64_t)N * (K * BITS / 32);
  scales += e * (int64_t)N * G;
  biases += e * (int64_t)N * G;

  // ---- issue the first slot's weight loads before staging x
  int rowc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rowc[r] = min(row0 + r, N - 1);  // clamp: loads stay in bounds
  const u32x4_t* wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    wrow[r] = reinterpret_cast<const u32x4_t*>(wq + (int64_t)rowc[r] * (C * 4));

  // ---- stage x: unit u (8 elements) of row m -> smem[(m*UPC + u%UPC)*C + u/UPC]
  float* xsum = reinterpret_cast<float*>(smem + MT * UPC * C);
  for (int i = threadIdx.x; i < MT * (K / 8); i += kBlock) {
    const int m = i / (K / 8);
    const int u = i - m * (K / 8);
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (m < M) v = *reinterpret_cast<const u32x4_t*>(x + (int64_t)m * K + u * 8);
    float s8 = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) s8 += lo_bf16(v[j]) + hi_bf16(v[j]);
    if constexpr (BITS == 4) {
      const u32x4_t p = {(v[0] & 0xffffu) | (v[2] << 16), (v[0] >> 16) | (v[2] & 0xffff0000u),
                         (v[1] & 0xffffu) | (v[3] << 16), (v[1] >> 16) | (v[3] & 0xffff0000u)};
      v = p;
    }
    smem[(m * UPC + u % UPC) * C + u / UPC] = v;
    s8 = lane_group_sum<UPC>(s8);
    if (u % UPC == 0) xsum[m * C + u / UPC] = s8;
  }
  __syncthreads();

  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

  const int n_slots = (C + TPR - 1) / TPR;
  for (int j = 0; j < n_slots; ++j) {
    const int c = lane + j * TPR;
    const bool valid = c < C;
    const int cc = valid ? c : C - 1;
    u32x4_t wv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wv[r] = load_stream_u4(wrow[r] + cc);
    const int g = (cc * EPC) / kGroup;
    float sc[R], bi[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      sc[r] = bf16_bits_to_f32(scales[(int64_t)rowc[r] * G + g]);
      bi[r] = bf16_bits_to_f32(biases[(int64_t)rowc[r] * G + g]);
      if (!valid) sc[r] = bi[r] = 0.f;
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m >= M) break;
      const float xs = xsum[m * C + cc];
      u32x4_t xv[UPC];
#pragma unroll
      for (int h = 0; h < UPC; ++h) xv[h] = smem[(m * UPC + h) * C + cc];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float d = 0.f;
        if constexpr (BITS == 4) {
#pragma unroll
          for (int wi = 0; wi < 4; ++wi) {
            const uint32_t wd = wv[r][wi];
#pragma unroll
            for (int sh = 0; sh < 4; ++sh) {
              const uint32_t p = ((wd >> (4 * sh)) & 0x000F000Fu) | 0x43004300u;
              d = dot2_bf16(p, xv[wi][sh], d);
            }
          }
          acc[r][m] = fmaf(sc[r], d, acc[r][m]);
          acc[r][m] = fmaf(fmaf(-128.f, sc[r], bi[r]), xs, acc[r][m]);
        } else {
#pragma unroll
          for (int wi = 0; wi < 4; ++wi) {
            const uint32_t wd = wv[r][wi];
            const uint32_t xa = xv[wi / 2][(wi % 2) * 2];
            const uint32_t xb2 = xv[wi / 2][(wi % 2) * 2 + 1];
            d = fmaf(lo_bf16(xa), ubyte_f32<0>(wd), d);
            d = fmaf(hi_bf16(xa), ubyte_f32<1>(wd), d);
            d = fmaf(lo_bf16(xb2), ubyte_f32<2>(wd), d);
            d = fmaf(hi_bf16(xb2), ubyte_f32<3>(wd), d);
          }
          acc[r][m] = fmaf(sc[r], d, acc[r][m]);
          acc[r][m] = fmaf(bi[r], xs, acc[r][m]);
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
    const float add = (bias && row < N) ? bf16_bits_to_f32(bias[row]) : 0.f;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float v = lane_group_sum<TPR>(acc[r][m]);
      if (lane == 0 && m < M && row < N)
        y[(int64_t)m * N + row] = (uint16_t)f32_to_bf16_bits(v + add);
    }
  }
}

template <int BITS, int TPR, int R, int MT>
hipError_t run(const uint16_t* x, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
               const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K,
               const GatherMap& g, hipStream_t stream) {
  constexpr int EPC = 128 / BITS;
  const int64_t C = K / EPC;
  const size_t lds = (size_t)MT * K * 2 + (size_t)MT * C * 4;
  const int64_t rows_per_block = (kBlock / TPR) * R;
  const dim3 grid((unsigned)((N + rows_per_block - 1) / rows_per_block), (unsigned)g.T);
  hipLaunchKernelGGL((qmv_kernel<BITS, TPR, R, MT>), grid, dim3(kBlock), lds, stream, x, wq, s, b,
                     bias, y, (int)M, (int)N, (int)K, g.lhs, g.rhs, g.E, g.x_batches);
  return hipGetLastError();
}

template <int BITS, int TPR, int R>
hipError_t run_mt(const uint16_t* x, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                  const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K,
                  const GatherMap& g, hipStream_t stream) {
  if (M <= 1) return run<BITS, TPR, R, 1>(x, wq, s, b, bias, y, M, N, K, g, stream);
  if (M <= 2) return run<BITS, TPR, R, 2>(x, wq, s, b, bias, y, M, N, K, g, stream);
  if (M <= 4) return run<BITS, TPR, R, 4>(x, wq, s, b, bias, y, M, N, K, g, stream);
  return run<BITS, TPR, R, 8>(x, wq, s, b, bias, y, M, N, K, g, stream);
}

template <int BITS>
hipError_t run_bits(const uint16_t* x, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                    const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K,
                    const GatherMap& g, hipStream_t stream) {
  constexpr int EPC = 128 / BITS;
  const int64_t C = K / EPC;
  // Lane-per-row shapes tried in order: enough chunks per lane to keep loads
  // in flight, enough blocks (x output batches) to fill 256 CUs.
  auto blocks = [&](int tpr, int r) { return ((N * tpr) / (kBlock * r)) * g.T; };
  if ((C + 15) / 16 <= 8 && blocks(16, 2) >= 1024)
    return run_mt<BITS, 16, 2>(x, wq, s, b, bias, y, M, N, K, g, stream);
  if ((C + 31) / 32 <= 8 && blocks(32, 2) >= 1024)
    return run_mt<BITS, 32, 2>(x, wq, s, b, bias, y, M, N, K, g, stream);
  if ((C + 63) / 64 <= 8 && blocks(64, 2) >= 1024)
    return run_mt<BITS, 64, 2>(x, wq, s, b, bias, y, M, N, K, g, stream);
  return run_mt<BITS, 64, 1>(x, wq, s, b, bias, y, M, N, K, g, stream);
}

}  // namespace

int qmv_max_rows(int64_t K, int bits) {
  const int64_t per_row = K * 2 + (K / (128 / bits)) * 4;  // staged x + chunk sums
  for (int mt = 8; mt >= 1; mt >>= 1)
    if (mt * per_row <= kQmvLdsBudget) return mt;
  return 0;
}

hipError_t launch_qmv(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                      const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                      int64_t N, int64_t K, int bits, const GatherMap& g, hipStream_t stream) {
  if (N == 0 || M == 0 || g.T == 0) return hipSuccess;
  if (bits == 4) return run_bits<4>(x, wq, scales, biases, bias, y, M, N, K, g, stream);
  return run_bits<8>(x, wq, scales, biases, bias, y, M, N, K, g, stream);
}

}  // namespace mq
