// Large-M quantized matmul on the gfx950 matrix cores:
//   y[m, n] = sum_k x[m, k] * (s*q + b)[n, k]  (+ bias[n])
// mx.quantized_matmul(x, w, scales, biases, transpose=True) for prefill-sized
// M (python/mlx_worker/native_mlx/models/qwen2.py:76-78,115,134,227).
//
// MFMA-bound.  A 512-thread block owns a 256x256 output tile and walks K in
// steps of 64 (one quantization group: one scale and bias per weight row per
// step).  LDS holds two stages, each an x tile and a dequantized weight tile
// (256 x 64 bfloat16 apiece, rows of 128 bytes, 16-byte chunk index XOR-ed with
// (row >> 1) & 7 so that the 16 rows one ds_read_b128 cycle serves -- 8 even
// rows on banks 0-31, 8 odd rows on banks 32-63 -- hit distinct banks): 128 KiB.
// Per step, each of the 8 waves (2 along M x 4 along N) runs 4 k-slices x 4x2
// v_mfma_f32_32x32x16_bf16 on its 128x64 sub-tile from the current stage while
// the next step's x and packed codes are in flight; the codes are then
// dequantized (fma(s, q, b), one bfloat16 rounding) into the other stage, and
// a single barrier ends the step.
//
// Blocks are numbered so that each XCD (blocks are dealt to the 8 XCDs round
// robin) works through a contiguous run of tiles that share weight columns,
// which keeps a weight tile's codes in that XCD's L2 while the M tiles pass.
#include "mq_common.h"
#include "mq_internal.h"

namespace mq {
namespace {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int kThreads = 512;
constexpr int kStageBytes = (BM + BN) * BK * 2;  // 64 KiB

__device__ __forceinline__ int swz(int row, int chunk) { return row * 8 + (chunk ^ ((row >> 1) & 7)); }

template <int BITS>
__global__ __launch_bounds__(kThreads) void qmm2_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K,
    int tiles_m, int tiles_n) {
  extern __shared__ u32x4_t smem[];  // [stage][A: BM*8 | B: BN*8] 16-byte chunks
  const int tid = threadIdx.x;
  const int l = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;  // 2 x 4 waves: 128 x 64 each

  // ---- tile order: XCD-contiguous runs, M fastest within a weight column ----
  const int nblk = gridDim.x;
  const int per_xcd = nblk / 8, rem = nblk % 8;
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
  const int tile = (xcd < rem ? xcd * (per_xcd + 1) : rem * (per_xcd + 1) + (xcd - rem) * per_xcd) + slot;
  const int bm = tile % tiles_m, bn = tile / tiles_m;
  const int m0 = bm * BM, n0 = bn * BN;

  const int G = K / kGroup;
  const int KT = K / BK;
  const rsrc_t xrs = make_rsrc(x, (uint64_t)M * K * 2);
  const rsrc_t wrs = make_rsrc(wq, (uint64_t)N * K * BITS / 8);
  const rsrc_t srs = make_rsrc(scales, (uint64_t)N * G * 2);
  const rsrc_t brs = make_rsrc(biases, (uint64_t)N * G * 2);

  // ---- per-thread load assignments ----
  // x: 4 chunks of 16 B: tile row (tid + 512 i) / 8, chunk tid % 8.  Rows past
  // M get an out-of-range offset and read as zeros.
  const int xch = tid & 7;
  uint32_t xoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = (tid + kThreads * i) >> 3;
    xoff[i] = (m0 + row < M) ? (uint32_t)((m0 + row) * K + xch * 8) * 2 : kOutOfRange;
  }
  // w: 4-bit: row tid/2, 32 codes at k-half tid%2; 8-bit: rows (tid+512i)/4, quarter %4
  constexpr int WPT = BITS == 4 ? 1 : 2;
  int wrow[WPT], wpart[WPT];
  uint32_t woff[WPT], soff[WPT];
#pragma unroll
  for (int i = 0; i < WPT; ++i) {
    const int q = tid + kThreads * i;
    wrow[i] = BITS == 4 ? (q >> 1) : (q >> 2);
    wpart[i] = BITS == 4 ? (q & 1) : (q & 3);
    const int n = n0 + wrow[i];
    woff[i] = n < N ? (uint32_t)(((int64_t)n * K * BITS / 8) + wpart[i] * 16) : kOutOfRange;
    soff[i] = n < N ? (uint32_t)(n * G) * 2 : kOutOfRange;
  }

  u32x4_t xr[4], wr[WPT];
  uint32_t sr[WPT], br[WPT];
  auto load_step = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) xr[i] = buf_load16(xrs, xoff[i] + kt * BK * 2);
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      wr[i] = buf_load16<kBufNT>(wrs, woff[i] + kt * (BK * BITS / 8));
      sr[i] = buf_load2(srs, soff[i] + kt * 2);
      br[i] = buf_load2(brs, soff[i] + kt * 2);
    }
  };
  auto store_step = [&](int stage) {
    u32x4_t* As = smem + stage * (kStageBytes / 16);
    u32x4_t* Bs = As + BM * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) As[swz((tid + kThreads * i) >> 3, xch)] = xr[i];
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const float s = bf16_bits_to_f32(sr[i]);
      const float b = bf16_bits_to_f32(br[i]);
      if constexpr (BITS == 4) {
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
          const uint32_t wd = wr[i][wi];
          u32x4_t o;
#pragma unroll
          for (int p = 0; p < 4; ++p)
            o[p] = pack_bf16x2(fmaf(s, (float)((wd >> (8 * p)) & 15u), b),
                               fmaf(s, (float)((wd >> (8 * p + 4)) & 15u), b));
          Bs[swz(wrow[i], wpart[i] * 4 + wi)] = o;
        }
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t w0 = wr[i][2 * h], w1 = wr[i][2 * h + 1];
          u32x4_t o;
          o[0] = pack_bf16x2(fmaf(s, ubyte_f32<0>(w0), b), fmaf(s, ubyte_f32<1>(w0), b));
          o[1] = pack_bf16x2(fmaf(s, ubyte_f32<2>(w0), b), fmaf(s, ubyte_f32<3>(w0), b));
          o[2] = pack_bf16x2(fmaf(s, ubyte_f32<0>(w1), b), fmaf(s, ubyte_f32<1>(w1), b));
          o[3] = pack_bf16x2(fmaf(s, ubyte_f32<2>(w1), b), fmaf(s, ubyte_f32<3>(w1), b));
          Bs[swz(wrow[i], wpart[i] * 2 + h)] = o;
        }
      }
    }
  };

  f32x16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  load_step(0);
  store_step(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load_step(kt + 1);
    const u32x4_t* As = smem + cur * (kStageBytes / 16);
    const u32x4_t* Bs = As + BM * 8;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int ch = ks * 2 + (l >> 5);
      bf16x8_t a[4], b[2];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = __builtin_bit_cast(bf16x8_t, As[swz(wm * 128 + i * 32 + (l & 31), ch)]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = __builtin_bit_cast(bf16x8_t, Bs[swz(wn * 64 + j * 32 + (l & 31), ch)]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) store_step(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: D[m][n], lane holds n = l%32, m = 8*(v/4) + 4*(l/32) + v%4 ----
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn * 64 + j * 32 + (l & 31);
    if (n >= N) continue;
    const float add = bias ? bf16_bits_to_f32(bias[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * 128 + i * 32 + 8 * (v >> 2) + 4 * (l >> 5) + (v & 3);
        if (m < M) y[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_bits(acc[i][j][v] + add);
      }
    }
  }
}

}  // namespace

bool qmm2_fits(int64_t M, int64_t N, int64_t K, int bits) {
  (void)bits;
  // 32-bit buffer offsets for x and the codes.  Below about 128 tiles (half of
  // the 256 CUs) the 128x128-tile kernel, with four times the blocks, is faster
  // (measured on MI355X: 112 tiles lose, 144 win).
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  return M * K * 2 < ((int64_t)1 << 31) && N * K < ((int64_t)1 << 32) && tiles >= 128 &&
         tiles < ((int64_t)1 << 31);
}

hipError_t launch_qmm2(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                       int64_t N, int64_t K, int bits, hipStream_t stream) {
  if (M == 0 || N == 0) return hipSuccess;
  const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
  const dim3 grid((unsigned)(tiles_m * tiles_n));
  const int lds = 2 * kStageBytes;
  auto kern = bits == 4 ? qmm2_kernel<4> : qmm2_kernel<8>;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), lds, stream, x, wq, scales, biases, bias, y,
                     (int)M, (int)N, (int)K, tiles_m, tiles_n);
  return hipGetLastError();
}

}  // namespace mq
