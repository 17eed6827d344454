// Shared device helpers for the gfx950 affine-quantization kernels.
//
// Weight format (MLX "affine"): wq uint32 [rows, K*bits/32], codes packed
// LSB-first (code j of a word at bits [j*bits, (j+1)*bits)); scales and biases
// bfloat16 [rows, K/group_size]; w = scale*q + bias.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mq {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kGroup = 64;  // elements per (scale, bias) group

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __builtin_bit_cast(float, h << 16);
}

// float -> bfloat16 bits, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two floats -> packed bfloat16 pair (lo in bits 0..15).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Low / high bfloat16 of a packed pair as float.
__device__ __forceinline__ float lo_bf16(uint32_t p) { return __builtin_bit_cast(float, p << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t p) {
  return __builtin_bit_cast(float, p & 0xffff0000u);
}

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Byte n of a word as float (selects v_cvt_f32_ubyte<n>).
template <int N>
__device__ __forceinline__ float ubyte_f32(uint32_t w) {
  return (float)((w >> (8 * N)) & 0xffu);
}

// Sum over groups of `width` consecutive lanes (width a power of two <= 64);
// every lane of the group receives the total.
template <int WIDTH>
__device__ __forceinline__ float lane_group_sum(float v) {
#pragma unroll
  for (int off = 1; off < WIDTH; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Non-temporal 16-byte load (weights are streamed once per call).
__device__ __forceinline__ u32x4_t load_stream_u4(const u32x4_t* p) {
  return __builtin_nontemporal_load(p);
}

}  // namespace mq
