// Affine quantize / dequantize kernels for gfx950.
//
// quantize: mx.quantize(w, group_size, bits, mode="affine") as called by
//   QuantizedSwitchLinear (python/mlx_worker/native_mlx/models/lfm2.py:142-151)
//   and by nn.quantize (models/qwen2.py:318-324).  Bit-exact with the float32
//   algorithm: min/max per group, scale = max((max-min)/(2^b-1), 1e-7) signed
//   toward the larger-magnitude edge, edge refit so that 0.0 is exact, codes
//   rint((w-bias)/scale) clamped to [0, 2^b-1].
// dequantize: mx.dequantize -- out = bf16(bf16(q*s) + b), the two rounded
//   element-wise ops MLX evaluates in the bfloat16 output dtype.  With a row
//   index list it is the quantized embedding lookup (models/qwen2.py:185).
//
// Group sizes 32, 64 and 128 (the values MLX accepts).  Layout: a group of GS
// bf16 weights is 2*GS contiguous bytes.  4- and 8-bit: quantize gives each
// group to GS/8 lanes (16 bytes each, one coalesced segment per group);
// dequantize gives each lane one 16-byte chunk of packed codes (32 4-bit or
// 16 8-bit codes: never more than one group).
// 2, 3, 5 and 6 bits: codes form one LSB-first bit stream per row (code k at
// bits [k*bits, (k+1)*bits) of the row's words; MLX packs 16, 8, 8 and 4 codes
// into 4, 3, 5 and 3 bytes), so 32 codes are exactly `bits` whole words: each
// lane quantizes, dequantizes or repacks 32 codes.  repack_u8 rewrites such
// codes one byte each (the 8-bit layout, same scales and biases, so the
// dequantized weights are identical) for the 8-bit matmul kernels.
#include "mq_common.h"
#include "mq_internal.h"

namespace mq {
namespace {

template <int BITS, int GS>
__global__ __launch_bounds__(256) void quantize_kernel(const uint16_t* __restrict__ w,
                                                       uint32_t* __restrict__ wq,
                                                       uint16_t* __restrict__ scales,
                                                       uint16_t* __restrict__ biases,
                                                       int64_t n_groups) {
  constexpr int LPG = GS / 8;  // lanes per group
  const int64_t gid = (int64_t)blockIdx.x * (256 / LPG) + threadIdx.x / LPG;
  const int sub = threadIdx.x % LPG;
  const bool ok = gid < n_groups;
  u32x4_t v = {0u, 0u, 0u, 0u};
  if (ok) v = *reinterpret_cast<const u32x4_t*>(w + gid * GS + sub * 8);
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = lo_bf16(v[i]);
    f[2 * i + 1] = hi_bf16(v[i]);
  }
  float w_max = f[0], w_min = f[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    w_max = (w_max < f[i]) ? f[i] : w_max;
    w_min = (f[i] < w_min) ? f[i] : w_min;
  }
#pragma unroll
  for (int off = 1; off < LPG; off <<= 1) {
    const float omax = __shfl_xor(w_max, off, 64);
    const float omin = __shfl_xor(w_min, off, 64);
    w_max = (w_max < omax) ? omax : w_max;
    w_min = (omin < w_min) ? omin : w_min;
  }
  const float n_bins = (float)((1 << BITS) - 1);
  const bool mask = fabsf(w_min) > fabsf(w_max);
  float scale = (w_max - w_min) / n_bins;
  scale = (scale < 1e-7f) ? 1e-7f : scale;
  scale = mask ? scale : -scale;
  const float edge = mask ? w_min : w_max;
  const float q0 = __builtin_rintf(edge / scale);
  float bias = 0.0f;
  if (q0 != 0.0f) {
    scale = edge / q0;
    bias = edge;
  }
  uint32_t code[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float q = __builtin_rintf((f[i] - bias) / scale);
    q = (q < 0.0f) ? 0.0f : q;
    q = (q > n_bins) ? n_bins : q;
    code[i] = (uint32_t)q;
  }
  if (!ok) return;
  if constexpr (BITS == 4) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) word |= code[i] << (4 * i);
    wq[gid * (GS / 8) + sub] = word;
  } else {
    u32x2_t words;
    words[0] = code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
    words[1] = code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24);
    *reinterpret_cast<u32x2_t*>(wq + gid * (GS / 4) + sub * 2) = words;
  }
  if (sub == 0) {
    scales[gid] = (uint16_t)f32_to_bf16_bits(scale);
    biases[gid] = (uint16_t)f32_to_bf16_bits(bias);
  }
}

// Code j (0..31) of a lane's 32-code run of BITS words (compile-time j after
// unrolling: a shift, or two for a code that straddles a word boundary).
template <int BITS>
__device__ __forceinline__ uint32_t stream_code(const uint32_t (&wd)[BITS], int j) {
  const int p = j * BITS;
  uint32_t v = wd[p >> 5] >> (p & 31);
  if ((p & 31) + BITS > 32) v |= wd[(p >> 5) + 1] << (32 - (p & 31));
  return v & ((1u << BITS) - 1u);
}

// Stream widths (2, 3, 5, 6): GS/32 lanes per group, 32 weights each, the same
// float32 steps as quantize_kernel.
template <int BITS, int GS>
__global__ __launch_bounds__(256) void quantize_stream_kernel(const uint16_t* __restrict__ w,
                                                              uint32_t* __restrict__ wq,
                                                              uint16_t* __restrict__ scales,
                                                              uint16_t* __restrict__ biases,
                                                              int64_t n_groups) {
  constexpr int LPG = GS / 32;  // lanes per group
  const int64_t gid = (int64_t)blockIdx.x * (256 / LPG) + threadIdx.x / LPG;
  const int sub = threadIdx.x % LPG;
  const bool ok = gid < n_groups;
  float f[32];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (ok) v = *reinterpret_cast<const u32x4_t*>(w + gid * GS + sub * 32 + c * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[8 * c + 2 * i] = lo_bf16(v[i]);
      f[8 * c + 2 * i + 1] = hi_bf16(v[i]);
    }
  }
  float w_max = f[0], w_min = f[0];
#pragma unroll
  for (int i = 1; i < 32; ++i) {
    w_max = (w_max < f[i]) ? f[i] : w_max;
    w_min = (f[i] < w_min) ? f[i] : w_min;
  }
#pragma unroll
  for (int off = 1; off < LPG; off <<= 1) {
    const float omax = __shfl_xor(w_max, off, 64);
    const float omin = __shfl_xor(w_min, off, 64);
    w_max = (w_max < omax) ? omax : w_max;
    w_min = (omin < w_min) ? omin : w_min;
  }
  const float n_bins = (float)((1 << BITS) - 1);
  const bool mask = fabsf(w_min) > fabsf(w_max);
  float scale = (w_max - w_min) / n_bins;
  scale = (scale < 1e-7f) ? 1e-7f : scale;
  scale = mask ? scale : -scale;
  const float edge = mask ? w_min : w_max;
  const float q0 = __builtin_rintf(edge / scale);
  float bias = 0.0f;
  if (q0 != 0.0f) {
    scale = edge / q0;
    bias = edge;
  }
  uint32_t out[BITS];
#pragma unroll
  for (int i = 0; i < BITS; ++i) out[i] = 0u;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    float q = __builtin_rintf((f[j] - bias) / scale);
    q = (q < 0.0f) ? 0.0f : q;
    q = (q > n_bins) ? n_bins : q;
    const uint32_t c = (uint32_t)q;
    const int p = j * BITS;
    out[p >> 5] |= c << (p & 31);
    if ((p & 31) + BITS > 32) out[(p >> 5) + 1] |= c >> (32 - (p & 31));
  }
  if (!ok) return;
#pragma unroll
  for (int i = 0; i < BITS; ++i) wq[gid * (GS * BITS / 32) + sub * BITS + i] = out[i];
  if (sub == 0) {
    scales[gid] = (uint16_t)f32_to_bf16_bits(scale);
    biases[gid] = (uint16_t)f32_to_bf16_bits(bias);
  }
}

// bf16(bf16(q*s) + b)
__device__ __forceinline__ float deq_two_round(uint32_t q, float s, float b) {
  const float t = (float)(__bf16)((float)q * s);
  return t + b;
}

template <int BITS>
__global__ __launch_bounds__(256) void dequantize_kernel(
    const uint32_t* __restrict__ wq, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, const int32_t* __restrict__ row_ids, int64_t n_out_rows,
    int64_t n_rows, uint16_t* __restrict__ out, int64_t K, int lgs) {
  constexpr int EPC = 128 / BITS;  // elements per 16-byte chunk
  const int64_t cpr = K / EPC;     // chunks per row
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= n_out_rows * cpr) return;
  const int64_t orow = idx / cpr;
  const int64_t c = idx - orow * cpr;
  int64_t srow = orow;
  if (row_ids) srow = row_ids[orow];
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(out + orow * K + c * EPC);
  if (srow < 0 || srow >= n_rows) {  // an id outside the table reads as zeros
#pragma unroll
    for (int i = 0; i < EPC / 8; ++i) dst[i] = u32x4_t{0u, 0u, 0u, 0u};
    return;
  }
  const u32x4_t v = *reinterpret_cast<const u32x4_t*>(wq + srow * (K * BITS / 32) + c * 4);
  const int64_t g = srow * (K >> lgs) + ((c * EPC) >> lgs);  // group size 1 << lgs
  const float s = bf16_bits_to_f32(scales[g]);
  const float b = bf16_bits_to_f32(biases[g]);
  uint32_t packed[EPC / 2];
#pragma unroll
  for (int i = 0; i < EPC / 2; ++i) {
    const int e0 = 2 * i;
    const uint32_t word0 = v[(e0 * BITS) / 32];
    const uint32_t q0 = (word0 >> ((e0 * BITS) % 32)) & ((1u << BITS) - 1u);
    const uint32_t q1 = (word0 >> ((e0 * BITS) % 32 + BITS)) & ((1u << BITS) - 1u);
    packed[i] = pack_bf16x2(deq_two_round(q0, s, b), deq_two_round(q1, s, b));
  }
#pragma unroll
  for (int i = 0; i < EPC / 8; ++i)
    dst[i] = u32x4_t{packed[4 * i], packed[4 * i + 1], packed[4 * i + 2], packed[4 * i + 3]};
}

// Stream widths: one lane per 32 codes (one group never splits a run).
template <int BITS>
__global__ __launch_bounds__(256) void dequantize_stream_kernel(
    const uint32_t* __restrict__ wq, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, const int32_t* __restrict__ row_ids, int64_t n_out_rows,
    int64_t n_rows, uint16_t* __restrict__ out, int64_t K, int lgs) {
  const int64_t upr = K / 32;  // 32-code runs per row
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= n_out_rows * upr) return;
  const int64_t orow = idx / upr;
  const int64_t u = idx - orow * upr;
  int64_t srow = orow;
  if (row_ids) srow = row_ids[orow];
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(out + orow * K + u * 32);
  if (srow < 0 || srow >= n_rows) {  // an id outside the table reads as zeros
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = u32x4_t{0u, 0u, 0u, 0u};
    return;
  }
  uint32_t wd[BITS];
  const uint32_t* src = wq + srow * (K * BITS / 32) + u * BITS;
#pragma unroll
  for (int i = 0; i < BITS; ++i) wd[i] = src[i];
  const int64_t g = srow * (K >> lgs) + ((u * 32) >> lgs);
  const float s = bf16_bits_to_f32(scales[g]);
  const float b = bf16_bits_to_f32(biases[g]);
  uint32_t packed[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    packed[i] = pack_bf16x2(deq_two_round(stream_code<BITS>(wd, 2 * i), s, b),
                            deq_two_round(stream_code<BITS>(wd, 2 * i + 1), s, b));
#pragma unroll
  for (int i = 0; i < 4; ++i)
    dst[i] = u32x4_t{packed[4 * i], packed[4 * i + 1], packed[4 * i + 2], packed[4 * i + 3]};
}

// Stream-width codes [units of 32] -> one byte per code (8-bit words).
template <int BITS>
__global__ __launch_bounds__(256) void repack_u8_kernel(const uint32_t* __restrict__ wq,
                                                        uint32_t* __restrict__ wq8,
                                                        int64_t units) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= units) return;
  uint32_t wd[BITS];
#pragma unroll
  for (int i = 0; i < BITS; ++i) wd[i] = wq[idx * BITS + i];
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    o[i] = stream_code<BITS>(wd, 4 * i) | stream_code<BITS>(wd, 4 * i + 1) << 8 |
           stream_code<BITS>(wd, 4 * i + 2) << 16 | stream_code<BITS>(wd, 4 * i + 3) << 24;
  u32x4_t* dst = reinterpret_cast<u32x4_t*>(wq8 + idx * 8);
  dst[0] = u32x4_t{o[0], o[1], o[2], o[3]};
  dst[1] = u32x4_t{o[4], o[5], o[6], o[7]};
}

template <int BITS>
void (*quantize_for(int group_size))(const uint16_t*, uint32_t*, uint16_t*, uint16_t*, int64_t) {
  if constexpr (BITS == 4 || BITS == 8)
    return group_size == 32 ? quantize_kernel<BITS, 32>
                            : group_size == 64 ? quantize_kernel<BITS, 64> : quantize_kernel<BITS, 128>;
  else
    return group_size == 32 ? quantize_stream_kernel<BITS, 32>
                            : group_size == 64 ? quantize_stream_kernel<BITS, 64>
                                               : quantize_stream_kernel<BITS, 128>;
}

}  // namespace

hipError_t launch_quantize(const uint16_t* w, uint32_t* wq, uint16_t* scales, uint16_t* biases,
                           int64_t rows, int64_t K, int group_size, int bits, hipStream_t stream) {
  const int64_t n_groups = rows * (K / group_size);
  if (n_groups == 0) return hipSuccess;
  const bool word_aligned = bits == 4 || bits == 8;
  const int64_t per_block = 256 / (group_size / (word_aligned ? 8 : 32));
  const dim3 grid((unsigned)((n_groups + per_block - 1) / per_block));
  void (*kern)(const uint16_t*, uint32_t*, uint16_t*, uint16_t*, int64_t);
  switch (bits) {
    case 2: kern = quantize_for<2>(group_size); break;
    case 3: kern = quantize_for<3>(group_size); break;
    case 4: kern = quantize_for<4>(group_size); break;
    case 5: kern = quantize_for<5>(group_size); break;
    case 6: kern = quantize_for<6>(group_size); break;
    default: kern = quantize_for<8>(group_size); break;
  }
  hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, w, wq, scales, biases, n_groups);
  return hipGetLastError();
}

hipError_t launch_dequantize(const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
                             const int32_t* row_ids, int64_t n_out_rows, int64_t n_rows,
                             uint16_t* out, int64_t K, int group_size, int bits,
                             hipStream_t stream) {
  const int lgs = group_size == 32 ? 5 : group_size == 64 ? 6 : 7;
  if (bits != 4 && bits != 8) {
    const int64_t units = n_out_rows * (K / 32);
    if (units == 0) return hipSuccess;
    const dim3 g((unsigned)((units + 255) / 256));
    auto kern = bits == 2 ? dequantize_stream_kernel<2>
                          : bits == 3 ? dequantize_stream_kernel<3>
                                      : bits == 5 ? dequantize_stream_kernel<5>
                                                  : dequantize_stream_kernel<6>;
    hipLaunchKernelGGL(kern, g, dim3(256), 0, stream, wq, scales, biases, row_ids, n_out_rows,
                       n_rows, out, K, lgs);
    return hipGetLastError();
  }
  const int64_t total = n_out_rows * (K * bits / 128);
  if (total == 0) return hipSuccess;
  const dim3 grid((unsigned)((total + 255) / 256));
  if (bits == 4)
    hipLaunchKernelGGL(dequantize_kernel<4>, grid, dim3(256), 0, stream, wq, scales, biases,
                       row_ids, n_out_rows, n_rows, out, K, lgs);
  else
    hipLaunchKernelGGL(dequantize_kernel<8>, grid, dim3(256), 0, stream, wq, scales, biases,
                       row_ids, n_out_rows, n_rows, out, K, lgs);
  return hipGetLastError();
}

hipError_t launch_repack_u8(const uint32_t* wq, uint32_t* wq8, int64_t rows, int64_t K, int bits,
                            hipStream_t stream) {
  const int64_t units = rows * (K / 32);
  if (units == 0) return hipSuccess;
  const dim3 grid((unsigned)((units + 255) / 256));
  auto kern = bits == 2 ? repack_u8_kernel<2>
                        : bits == 3 ? repack_u8_kernel<3>
                                    : bits == 5 ? repack_u8_kernel<5> : repack_u8_kernel<6>;
  hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, wq, wq8, units);
  return hipGetLastError();
}

}  // namespace mq
