// Prefill / batched quantized matmul (qmm) on the gfx950 matrix cores, and its
// expert-gathered form.
//
//   qmm:        y[m, n] = sum_k x[m, k] * w[n, k] (+ bias[n]),   w = s*q + b
//               mx.quantized_matmul(..., transpose=True) as called by every
//               QuantizedLinear with M = batch * tokens > 8
//               (python/mlx_worker/native_mlx/models/qwen2.py:76-78,115,134,227).
//   gather rows: y[r, n] = sum_k x[lhs(r), k] * w[rhs(r)][n, k]
//               mx.gather_qmm(..., transpose=True, sorted_indices) as called by
//               QuantizedSwitchLinear (models/lfm2.py:176-187) after the expert
//               sort of models/lfm2.py:613-618.
//
// Tiling: a 256-thread block owns a 128x128 output tile; K advances 64 at a time.
// A thread's codes for a step (32 4-bit or 16 8-bit: half or a quarter of the
// step) lie in one quantization group at group sizes 32, 64 and 128, so each
// takes one scale/bias, group (64 kt + its offset in the step) >> lgs.  Each
// step the packed codes of the 128 weight rows (4 KiB at 4-bit) are dequantized
// to bfloat16 (fma(s, q, b), one rounding) straight into LDS next to the
// activation tile; the four waves (2x2) each run 2x2 v_mfma_f32_32x32x16_bf16
// per 16-wide k step with float32 accumulators.  LDS rows are 128 bytes; the
// 16-byte chunk index is XOR-swizzled with (row & 7) so that the fragment reads
// (32 rows, same chunk) hit distinct banks.  The next step's global loads are
// issued before the current step's MFMAs.
//
// Gather: a tile's rows may use several experts.  The block walks the distinct
// experts of its rows in increasing order; for each it runs the K loop with the
// rows of other experts zeroed, accumulating into the same registers (rows are
// disjoint, so the sum is exact).  Sorted rows give 1-2 experts per tile.
#include <climits>

#include "mq_common.h"
#include "mq_internal.h"

namespace mq {
namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kThreads = 256;

__device__ __forceinline__ int swz(int row, int chunk) { return row * 8 + (chunk ^ (row & 7)); }

template <int BITS, bool GATHER>
__global__ __launch_bounds__(kThreads) void qmm_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K,
    const int32_t* __restrict__ lhs, const int32_t* __restrict__ rhs, int rows_per_batch,
    int64_t E, int64_t x_rows, int lgs) {
  __shared__ u32x4_t As[BM * 8];
  __shared__ u32x4_t Bs[BN * 8];
  __shared__ int tile_expert[BM];
  __shared__ int tile_xrow[BM];
  __shared__ int red[kThreads / 64];

  const int tid = threadIdx.x;
  const int l = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int n0 = blockIdx.x * BN;
  const int m0 = blockIdx.y * BM;
  const int G = K >> lgs;  // groups per row (group size 1 << lgs)
  const int Kw = K * BITS / 32;  // words per weight row
  const int KT = K / BK;

  // ---- rows of this tile: source row of x and expert (GATHER) ----
  if (tid < BM) {
    const int r = m0 + tid;
    int xr = -1, ex = INT_MAX;
    if (r < M) {
      if constexpr (GATHER) {
        const int tb = r / rows_per_batch, mr = r - tb * rows_per_batch;
        const int64_t xb = lhs ? (int64_t)lhs[tb] : (int64_t)tb;
        const int64_t e = rhs[tb];
        if (e >= 0 && e < E && xb >= 0 && xb * rows_per_batch + mr < x_rows) {
          xr = (int)(xb * rows_per_batch + mr);
          ex = (int)e;
        }
      } else {
        xr = r;
        ex = 0;
      }
    }
    tile_xrow[tid] = xr;
    tile_expert[tid] = ex;
  }
  __syncthreads();

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  int prev_expert = -1;
  for (;;) {
    // ---- next expert: smallest expert id above the previous one ----
    int cand = INT_MAX;
    if (tid < BM) {
      const int ex = tile_expert[tid];
      cand = (ex > prev_expert) ? ex : INT_MAX;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) cand = min(cand, __shfl_xor(cand, off, 64));
    if (l == 0) red[wave] = cand;
    __syncthreads();
    int e = red[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) e = min(e, red[w]);
    __syncthreads();  // red[] is rewritten next round
    if (e == INT_MAX) break;
    prev_expert = e;

    const uint32_t* we = wq + (int64_t)e * N * Kw;
    const uint16_t* se = scales + (int64_t)e * N * G;
    const uint16_t* be = biases + (int64_t)e * N * G;

    // ---- per-thread load assignments ----
    // x: 4 chunks of 16 B: tile row (tid + 256*i) / 8, chunk tid % 8
    const int xch = tid & 7;
    const u32x4_t* xsrc[4];
    bool xon[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = (tid + kThreads * i) >> 3;
      const int xr = tile_xrow[row];
      xon[i] = xr >= 0 && tile_expert[row] == e;
      xsrc[i] = reinterpret_cast<const u32x4_t*>(x + (int64_t)(xon[i] ? xr : 0) * K) + xch;
    }
    // w: 4-bit: row tid/2, half tid%2 (16 B = 32 codes); 8-bit: two of row q/4, quarter q%4
    constexpr int WPT = BITS == 4 ? 1 : 2;  // 16-byte weight chunks per thread
    const u32x4_t* wsrc[WPT];
    const uint16_t* ssrc[WPT];
    const uint16_t* bsrc[WPT];
    bool won[WPT];
    int wrow[WPT], wpart[WPT];
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const int q = tid + kThreads * i;
      wrow[i] = BITS == 4 ? (q >> 1) : (q >> 2);
      wpart[i] = BITS == 4 ? (q & 1) : (q & 3);
      const int n = n0 + wrow[i];
      won[i] = n < N;
      const int nc = won[i] ? n : 0;
      wsrc[i] = reinterpret_cast<const u32x4_t*>(we + (int64_t)nc * Kw) + wpart[i];
      ssrc[i] = se + (int64_t)nc * G;
      bsrc[i] = be + (int64_t)nc * G;
    }

    u32x4_t xr_[4], wr_[WPT];
    uint16_t sr_[WPT], br_[WPT];
    auto load_step = [&](int kt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xr_[i] = u32x4_t{0u, 0u, 0u, 0u};
        if (xon[i]) xr_[i] = xsrc[i][kt * 8];
      }
#pragma unroll
      for (int i = 0; i < WPT; ++i) {
        wr_[i] = u32x4_t{0u, 0u, 0u, 0u};
        sr_[i] = 0;
        br_[i] = 0;
        if (won[i]) {
          wr_[i] = load_stream_u4(wsrc[i] + kt * (BK * BITS / 128));
          const int grp = (kt * BK + wpart[i] * (128 / BITS)) >> lgs;
          sr_[i] = ssrc[i][grp];
          br_[i] = bsrc[i][grp];
        }
      }
    };

    load_step(0);
    for (int kt = 0; kt < KT; ++kt) {
      __syncthreads();  // previous step's fragment reads are done
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = (tid + kThreads * i) >> 3;
        As[swz(row, xch)] = xr_[i];
      }
#pragma unroll
      for (int i = 0; i < WPT; ++i) {
        const float s = bf16_bits_to_f32(sr_[i]);
        const float b = bf16_bits_to_f32(br_[i]);
        if constexpr (BITS == 4) {
#pragma unroll
          for (int wi = 0; wi < 4; ++wi) {
            const uint32_t wd = wr_[i][wi];
            u32x4_t o;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
              const float q0 = (float)((wd >> (8 * p)) & 15u);
              const float q1 = (float)((wd >> (8 * p + 4)) & 15u);
              o[p] = pack_bf16x2(fmaf(s, q0, b), fmaf(s, q1, b));
            }
            Bs[swz(wrow[i], wpart[i] * 4 + wi)] = o;
          }
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            u32x4_t o;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
              const uint32_t wd = wr_[i][2 * h + p / 2];
              const float q0 = (p & 1) ? ubyte_f32<2>(wd)
                                       : ubyte_f32<0>(wd);
              const float q1 = (p & 1) ? ubyte_f32<3>(wd)
                                       : ubyte_f32<1>(wd);
              o[p] = pack_bf16x2(fmaf(s, q0, b), fmaf(s, q1, b));
            }
            Bs[swz(wrow[i], wpart[i] * 2 + h)] = o;
          }
        }
      }
      __syncthreads();
      if (kt + 1 < KT) load_step(kt + 1);
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        const int ch = ks * 2 + (l >> 5);
        bf16x8_t a[2], bfr[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int row = wm * 64 + i * 32 + (l & 31);
          a[i] = __builtin_bit_cast(bf16x8_t, As[swz(row, ch)]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int row = wn * 64 + j * 32 + (l & 31);
          bfr[j] = __builtin_bit_cast(bf16x8_t, Bs[swz(row, ch)]);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bfr[j], acc[i][j], 0, 0, 0);
      }
    }
    if constexpr (!GATHER) break;
  }

  // ---- epilogue: D[m][n], lane holds n = l%32, m = 8*(v/4) + 4*(l/32) + v%4 ----
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn * 64 + j * 32 + (l & 31);
    if (n >= N) continue;
    const float add = bias ? bf16_bits_to_f32(bias[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * (l >> 5) + (v & 3);
        if (m < M) y[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_bits(acc[i][j][v] + add);
      }
    }
  }
}

}  // namespace

hipError_t launch_qmm(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                      const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                      int64_t N, int64_t K, int group_size, int bits, hipStream_t stream) {
  if (M == 0 || N == 0) return hipSuccess;
  if (K % BK) return hipErrorInvalidValue;  // whole 64-wide steps (checked by the caller)
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  const int lgs = __builtin_ctz((unsigned)group_size);
  if (bits == 4)
    hipLaunchKernelGGL((qmm_kernel<4, false>), grid, dim3(kThreads), 0, stream, x, wq, scales,
                       biases, bias, y, (int)M, (int)N, (int)K, nullptr, nullptr, 1, 1, M, lgs);
  else
    hipLaunchKernelGGL((qmm_kernel<8, false>), grid, dim3(kThreads), 0, stream, x, wq, scales,
                       biases, bias, y, (int)M, (int)N, (int)K, nullptr, nullptr, 1, 1, M, lgs);
  return hipGetLastError();
}

hipError_t launch_gather_qmm_rows(const uint16_t* x, const int32_t* lhs, const int32_t* rhs,
                                  const uint32_t* wq, const uint16_t* scales,
                                  const uint16_t* biases, uint16_t* y, int64_t rows, int64_t N,
                                  int64_t K, int64_t E, int64_t x_rows, int rows_per_batch,
                                  int group_size, int bits, hipStream_t stream) {
  if (rows == 0 || N == 0) return hipSuccess;
  if (K % BK) return hipErrorInvalidValue;  // whole 64-wide steps (checked by the caller)
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((rows + BM - 1) / BM));
  const int lgs = __builtin_ctz((unsigned)group_size);
  if (bits == 4)
    hipLaunchKernelGGL((qmm_kernel<4, true>), grid, dim3(kThreads), 0, stream, x, wq, scales,
                       biases, nullptr, y, (int)rows, (int)N, (int)K, lhs, rhs, rows_per_batch,
                       E, x_rows, lgs);
  else
    hipLaunchKernelGGL((qmm_kernel<8, true>), grid, dim3(kThreads), 0, stream, x, wq, scales,
                       biases, nullptr, y, (int)rows, (int)N, (int)K, lhs, rhs, rows_per_batch,
                       E, x_rows, lgs);
  return hipGetLastError();
}

}  // namespace mq
