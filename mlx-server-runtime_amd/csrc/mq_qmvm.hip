// Decode-shaped quantized matmul on the matrix cores (qmv-mfma):
//   y[m, n] = sum_k x[m, k] * (s*q + b)[n, k]   for M <= 8 (4-bit) / 16 (8-bit)
// mx.quantized_matmul(x, w, scales, biases, transpose=True) at decode batch
// sizes (python/mlx_worker/native_mlx/models/qwen2.py:76-78,115,134,227), and
// mx.gather_qmm with a per-batch expert (models/lfm2.py:176-187).
//
// The weight stream is the cost (HBM-bound); the point of this kernel is to
// spend as few vector-ALU cycles per weight byte as possible so the math hides
// under the stream:
//  * a block owns 16 weight rows and all of K; its NW waves split K.  Lane l
//    serves row n = l % 16 and k-slice g = l / 16 of v_mfma_f32_16x16x32_bf16:
//    per "superstep" each lane loads one 16-byte chunk (chunk 4t+g of its row,
//    32 4-bit / 16 8-bit codes), all of a lane's chunks issued up front;
//  * 4-bit: ((word >> 4j) & 0x000F000F) | 0x43004300 are bfloat16 pairs
//    128+q (exact) -- one v_and_or_b32 (+ shift) per pair -- used directly as
//    the B operand; 8-bit: v_cvt_f32_ubyte + v_cvt_pk_bf16_f32 (exact);
//  * the A operand is x from LDS.  A 4-bit superstep spans two quantization
//    groups (chunks 4t,4t+1 | 4t+2,4t+3); A rows 2m and 2m+1 carry x row m for
//    the first and second group (zeros elsewhere), so the MFMA returns both
//    group partial sums d separately, for up to 8 x rows;
//  * per group: acc += s*d + c*sum(x), c = b - 128*s (4-bit) or b (8-bit),
//    with (s, c) precomputed in float32 per block in LDS and the group sums of
//    x next to it;
//  * partial sums over the waves' K ranges are added through LDS; one
//    bfloat16 rounding at the store, QuantizedLinear's "+ bias" fused.
#include "mq_common.h"
#include "mq_internal.h"

namespace mq {
namespace {

constexpr int kRows = 16;  // weight rows per block (the MFMA N dimension)

struct NibbleM {
  uint32_t mask, magic;
  __device__ __forceinline__ NibbleM() {
    __asm__ volatile("s_mov_b32 %0, 0xf000f" : "=s"(mask));
    __asm__ volatile("v_mov_b32 %0, 0x43004300" : "=v"(magic));
  }
  __device__ __forceinline__ uint32_t pair(uint32_t w) const { return (w & mask) | magic; }
};

template <int BITS>
struct Geo {
  static constexpr int EPC = 128 / BITS;        // codes per 16-byte chunk
  static constexpr int XCB = EPC * 2;           // bytes of x per chunk
  static constexpr int KSTEP = EPC / 8;         // MFMAs (8 codes per lane each) per chunk
  static constexpr int GPS = BITS == 4 ? 2 : 1; // groups per superstep (4 chunks)
  static constexpr int SSB = 4 * XCB;           // x bytes per superstep
};

struct Layout {  // LDS byte offsets, all multiples of 16
  int xrs;       // bytes per x row (padded chunks + 16 to spread banks)
  int x, xs, sc, zero, red, total;
};

constexpr int kMaxS = 12;  // chunks per lane, upper bound (zero region sized for it)

__host__ __device__ inline Layout layout(int bits, int nw, int mt, int K) {
  const int epc = 128 / bits, xcb = 2 * epc, gps = bits == 4 ? 2 : 1;
  Layout L;
  const int C = K / epc;
  const int T = (C + 3) / 4;
  const int TS = (T + nw - 1) / nw;
  const int CP = TS * nw * 4;  // padded chunks per row
  const int GP = TS * nw * gps;
  L.xrs = CP * xcb + 16;
  L.x = 0;
  L.xs = L.x + mt * L.xrs;
  L.sc = L.xs + ((mt * GP * 4 + 15) / 16) * 16;
  L.zero = L.sc + kRows * GP * 8;
  L.red = L.zero + kMaxS * 4 * xcb + 64;  // covers every superstep offset of a zero lane
  L.total = L.red + nw * kRows * mt * 4;
  return L;
}

template <int BITS, int NW, int S, int MT>
__global__ __launch_bounds__(NW * 64) void qmvm_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K,
    const int32_t* __restrict__ lhs, const int32_t* __restrict__ rhs, int64_t E,
    int64_t x_batches) {
  using Gm = Geo<BITS>;
  constexpr int NT = NW * 64;
  constexpr int UPC = Gm::EPC / 8;             // x units (8 elements) per chunk
  constexpr int XPM = (S * UPC + 15) / 16;     // x units per thread per x row
  constexpr int LPR = NT / kRows;              // threads per weight row (scale staging)
  extern __shared__ u32x4_t smem[];
  char* lds = reinterpret_cast<char*>(smem);

  const int C = K / Gm::EPC;       // chunks per row
  const int G = K / kGroup;        // groups per row (multiple of 4 here)
  const int T = (C + 3) / 4;       // supersteps per row
  const int TS = (T + NW - 1) / NW;  // supersteps per wave (<= S)
  const int CP = TS * NW * 4;
  const int GP = TS * NW * Gm::GPS;
  const Layout L = layout(BITS, NW, MT, K);

  const int64_t t = blockIdx.y;
  int64_t xb = t, e = 0;
  if (lhs) xb = lhs[t];
  if (rhs) e = rhs[t];
  const int n0 = blockIdx.x * kRows;
  y += t * (int64_t)M * N;
  const int tid = threadIdx.x;
  if (xb < 0 || xb >= x_batches || e < 0 || e >= E) {  // index outside the tables: zeros
    if (tid < kRows * M) {
      const int m = tid / kRows, n = n0 + tid % kRows;
      if (n < N) y[(int64_t)m * N + n] = 0;
    }
    return;
  }
  const int rows_here = min(kRows, N - n0);
  const rsrc_t xrs = make_rsrc(x + xb * (int64_t)M * K, (uint64_t)M * K * 2);
  const rsrc_t wrs = make_rsrc(wq + (e * (int64_t)N + n0) * (C * 4), (uint64_t)rows_here * C * 16);
  const int64_t sb0 = (e * (int64_t)N + n0) * G;
  const rsrc_t srs = make_rsrc(scales + sb0, (uint64_t)rows_here * G * 2);
  const rsrc_t brs = make_rsrc(biases + sb0, (uint64_t)rows_here * G * 2);

  // ---- 1. loads: x units, the block's scales/biases (4 groups per load),
  // then this lane's weight chunks.  vmcnt counts in issue order, so waiting
  // for x / scales never waits for the weights.
  u32x4_t xr[MT][XPM];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int k = 0; k < XPM; ++k) {
      const int u = tid + k * NT;  // unit within the row
      const bool real = m < M && u < C * UPC;
      xr[m][k] = buf_load16(xrs, real ? (uint32_t)(m * K + u * 8) * 2 : kOutOfRange);
    }
  const int srow = tid / LPR, su = tid % LPR;  // scale staging: row, 4-group unit
  u32x2_t sv[2], bv[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int u4 = su + k * LPR;
    const bool real = u4 < G / 4;  // rows past rows_here fall outside the descriptor
    const uint32_t off = real ? (uint32_t)(srow * G + u4 * 4) * 2 : kOutOfRange;
    sv[k] = buf_load8(srs, off);
    bv[k] = buf_load8(brs, off);
  }
  __asm__ volatile("" ::: "memory");  // keep the weight loads after these

  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  u32x4_t wv[S];
#pragma unroll
  for (int s = 0; s < S; ++s)  // chunks past the row end meet zero x
    wv[s] = buf_load16<kBufNT>(wrs, (uint32_t)((n * C + (wave * TS + s) * 4 + g) * 16));

  // ---- 2. LDS: x rows (4-bit pair-permuted) with zeros past C; group sums
  // of x; (s, c) per row and group in float32; a zero region for idle A lanes.
  uint32_t ones;
  __asm__ volatile("v_mov_b32 %0, 0x3f803f80" : "=v"(ones));  // bfloat16 (1, 1)
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int k = 0; k < XPM; ++k) {
      const int u = tid + k * NT;
      u32x4_t v = xr[m][k];
      float s8 = dot2_bf16(v[0], ones, 0.f);
      s8 = dot2_bf16(v[1], ones, s8);
      s8 = dot2_bf16(v[2], ones, s8);
      s8 = dot2_bf16(v[3], ones, s8);
      if constexpr (BITS == 4) {
        v = u32x4_t{(v[0] & 0xffffu) | (v[2] << 16), (v[0] >> 16) | (v[2] & 0xffff0000u),
                    (v[1] & 0xffffu) | (v[3] << 16), (v[1] >> 16) | (v[3] & 0xffff0000u)};
      }
      s8 += dpp_f32<0xb1>(s8);  // 8 consecutive units = one group of 64
      s8 += dpp_f32<0x4e>(s8);
      s8 += dpp_f32<0x141>(s8);
      if (u < CP * UPC) {
        *reinterpret_cast<u32x4_t*>(lds + L.x + m * L.xrs + u * 16) = v;
        if ((u & 7) == 0) reinterpret_cast<float*>(lds + L.xs)[m * GP + (u >> 3)] = s8;
      }
    }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int u4 = su + k * LPR;
    if (u4 < GP / 4) {  // groups past G were read as zeros: s = c = 0
      float4 out[2];
      float* o = reinterpret_cast<float*>(out);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t sw = sv[k][q >> 1], bw = bv[k][q >> 1];
        const float sc = (q & 1) ? hi_bf16(sw) : lo_bf16(sw);
        const float bi = (q & 1) ? hi_bf16(bw) : lo_bf16(bw);
        o[2 * q] = sc;
        o[2 * q + 1] = BITS == 4 ? fmaf(-128.f, sc, bi) : bi;
      }
      float4* dst = reinterpret_cast<float4*>(lds + L.sc + (srow * GP + u4 * 4) * 8);
      dst[0] = out[0];
      dst[1] = out[1];
    }
  }
  for (int i = tid * 16; i < L.red - L.zero; i += NT * 16)
    *reinterpret_cast<u32x4_t*>(lds + L.zero + i) = u32x4_t{0u, 0u, 0u, 0u};
  lds_barrier();

  // ---- 3. contract ----
  // A row a = lane % 16 reads x row m = a/2 (4-bit; group half a%2, only from
  // the two k-slices of that half) or m = a (8-bit); other lanes read zeros.
  const int a = lane & 15;
  int a_off;
  if constexpr (BITS == 4) {
    const int m = a >> 1;
    const bool real = m < M && (g >> 1) == (a & 1);
    a_off = real ? L.x + m * L.xrs + (wave * TS * 4 + g) * Gm::XCB : L.zero;
  } else {
    a_off = a < M ? L.x + a * L.xrs + (wave * TS * 4 + g) * Gm::XCB : L.zero;
  }
  const char* a_ptr = lds + a_off;
  const float2* scp = reinterpret_cast<const float2*>(lds + L.sc) + n * GP;
  const float* xsp = reinterpret_cast<const float*>(lds + L.xs);
  const int G4 = lane >> 4;  // D rows 4*G4 .. 4*G4+3 live in this lane
  const NibbleM nib;

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if (s < TS) {  // uniform
    const int tt = wave * TS + s;  // superstep index along the row
    f32x4_t d = {0.f, 0.f, 0.f, 0.f};
    if constexpr (BITS == 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t wd = wv[s][i];
        const u32x4_t bq = {nib.pair(wd), nib.pair(wd >> 4), nib.pair(wd >> 8), nib.pair(wd >> 12)};
        const u32x4_t av = *reinterpret_cast<const u32x4_t*>(a_ptr + s * Gm::SSB + i * 16);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av),
                                                    __builtin_bit_cast(bf16x8_t, bq), d, 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t w0 = wv[s][2 * i], w1 = wv[s][2 * i + 1];
        const u32x4_t bq = {pack_bf16x2(ubyte_f32<0>(w0), ubyte_f32<1>(w0)),
                            pack_bf16x2(ubyte_f32<2>(w0), ubyte_f32<3>(w0)),
                            pack_bf16x2(ubyte_f32<0>(w1), ubyte_f32<1>(w1)),
                            pack_bf16x2(ubyte_f32<2>(w1), ubyte_f32<3>(w1))};
        const u32x4_t av = *reinterpret_cast<const u32x4_t*>(a_ptr + s * Gm::SSB + i * 16);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av),
                                                    __builtin_bit_cast(bf16x8_t, bq), d, 0, 0, 0);
      }
    }
    // epilogue: D row 4*G4 + r -> (x row, group)
    if constexpr (BITS == 4) {
      const float4 sc2 = *reinterpret_cast<const float4*>(scp + 2 * tt);  // groups 2tt, 2tt+1
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (MT == 1 && r >= 2) continue;  // x row 1 does not exist
        const int m = 2 * G4 + (r >> 1);
        const float xs = xsp[(m < MT ? m : 0) * GP + 2 * tt + (r & 1)];
        const float sc = (r & 1) ? sc2.z : sc2.x;
        const float cc = (r & 1) ? sc2.w : sc2.y;
        acc[r] = fmaf(sc, d[r], fmaf(cc, xs, acc[r]));
      }
    } else {
      const float2 sc2 = scp[tt];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * G4 + r;
        const float xs = xsp[(m < MT ? m : 0) * GP + tt];
        acc[r] = fmaf(sc2.x, d[r], fmaf(sc2.y, xs, acc[r]));
      }
    }
    }
  }

  // ---- 4. add the waves' partial sums, store ----
  float* red = reinterpret_cast<float*>(lds + L.red);
  if constexpr (BITS == 4) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int m = 2 * G4 + h;
      if (m < MT) red[(wave * MT + m) * kRows + n] = acc[2 * h] + acc[2 * h + 1];
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * G4 + r;
      if (m < MT) red[(wave * MT + m) * kRows + n] = acc[r];
    }
  }
  __syncthreads();
  if (tid < kRows * MT) {
    const int m = tid / kRows, nn = tid % kRows, row = n0 + nn;
    if (m < M && row < N) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) v += red[(w * MT + m) * kRows + nn];
      if (bias) v += bf16_bits_to_f32(bias[row]);
      y[(int64_t)m * N + row] = (uint16_t)f32_to_bf16_bits(v);
    }
  }
}

template <int BITS, int NW, int S, int MT>
hipError_t run(const uint16_t* x, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
               const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K,
               const GatherMap& g, hipStream_t stream) {
  const Layout L = layout(BITS, NW, MT, (int)K);
  const dim3 grid((unsigned)((N + kRows - 1) / kRows), (unsigned)g.T);
  auto kern = qmvm_kernel<BITS, NW, S, MT>;
  if (L.total > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, L.total);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, grid, dim3(NW * 64), L.total, stream, x, wq, s, b, bias, y, (int)M,
                     (int)N, (int)K, g.lhs, g.rhs, g.E, g.x_batches);
  return hipGetLastError();
}

// Waves per block: enough that each lane owns at most 8 chunks (12 past 64 supersteps).
int pick_nw(int64_t K, int bits) {
  const int64_t T = (K / (128 / bits) + 3) / 4;
  return T <= 32 ? 4 : T <= 64 ? 8 : 16;
}

// x registers a lane holds (16-byte units) and the most a block of NW waves
// affords: 1024-thread blocks have 128 VGPRs.  Past it the kernel spills.
constexpr int x_regs(int bits, int s, int mt) { return mt * ((s * (16 / bits) + 15) / 16); }
constexpr int x_regs_max(int nw) { return nw == 16 ? 6 : 16; }

// Instantiates only the row counts whose x registers fit (the rest would
// spill and qmvm_fits refuses them).
template <int BITS, int NW, int S, int MT>
hipError_t run_fit(const uint16_t* x, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                   const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K,
                   const GatherMap& g, hipStream_t stream) {
  if constexpr (x_regs(BITS, S, MT) <= x_regs_max(NW))
    return run<BITS, NW, S, MT>(x, wq, s, b, bias, y, M, N, K, g, stream);
  return hipErrorInvalidValue;
}

template <int BITS, int NW, int S>
hipError_t run_s(const uint16_t* x, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                 const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K,
                 const GatherMap& g, hipStream_t stream) {
  if (M <= 1) return run_fit<BITS, NW, S, 1>(x, wq, s, b, bias, y, M, N, K, g, stream);
  if (M <= 2) return run_fit<BITS, NW, S, 2>(x, wq, s, b, bias, y, M, N, K, g, stream);
  if (M <= 4) return run_fit<BITS, NW, S, 4>(x, wq, s, b, bias, y, M, N, K, g, stream);
  if (M <= 8) return run_fit<BITS, NW, S, 8>(x, wq, s, b, bias, y, M, N, K, g, stream);
  if constexpr (BITS == 8) return run_fit<BITS, NW, S, 16>(x, wq, s, b, bias, y, M, N, K, g, stream);
  return hipErrorInvalidValue;
}

template <int BITS, int NW>
hipError_t run_nw(const uint16_t* x, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                  const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K,
                  const GatherMap& g, hipStream_t stream) {
  const int64_t TS = ((K / (128 / BITS) + 3) / 4 + NW - 1) / NW;
  if (TS <= 8) return run_s<BITS, NW, 8>(x, wq, s, b, bias, y, M, N, K, g, stream);
  return run_s<BITS, NW, kMaxS>(x, wq, s, b, bias, y, M, N, K, g, stream);
}

}  // namespace

bool qmvm_fits(int64_t M, int64_t N, int64_t K, int bits, int64_t T) {
  (void)N;
  if (M < 1 || M > (bits == 4 ? 8 : 16) || T > 65535 || K > (1 << 20)) return false;
  if ((K / kGroup) % 4 != 0) return false;  // scales are loaded 4 groups at a time
  const int nw = pick_nw(K, bits);
  const int64_t Tn = (K / (128 / bits) + 3) / 4;
  const int64_t TS = (Tn + nw - 1) / nw;
  if (TS > kMaxS) return false;                                   // chunks per lane
  if ((K / kGroup) / 4 > 2 * (nw * 64 / kRows)) return false;     // scale loads per thread
  const int mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16;
  if (x_regs(bits, TS <= 8 ? 8 : kMaxS, mt) > x_regs_max(nw)) return false;
  return layout(bits, nw, mt, (int)K).total <= 160 * 1024;
}

hipError_t launch_qmvm(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                       int64_t N, int64_t K, int bits, const GatherMap& g, hipStream_t stream) {
  if (N == 0 || M == 0 || g.T == 0) return hipSuccess;
  const int nw = pick_nw(K, bits);
  if (bits == 4) {
    if (nw == 4) return run_nw<4, 4>(x, wq, scales, biases, bias, y, M, N, K, g, stream);
    if (nw == 8) return run_nw<4, 8>(x, wq, scales, biases, bias, y, M, N, K, g, stream);
    return run_nw<4, 16>(x, wq, scales, biases, bias, y, M, N, K, g, stream);
  }
  if (nw == 4) return run_nw<8, 4>(x, wq, scales, biases, bias, y, M, N, K, g, stream);
  if (nw == 8) return run_nw<8, 8>(x, wq, scales, biases, bias, y, M, N, K, g, stream);
  return run_nw<8, 16>(x, wq, scales, biases, bias, y, M, N, K, g, stream);
}

}  // namespace mq
