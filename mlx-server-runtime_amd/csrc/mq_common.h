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

// SwiGLU on bfloat16 values (models/qwen2.py:43-44, 132-133): silu(g) rounded
// to bfloat16 as nn.silu stores it, times u, rounded -> bfloat16 bits.  One
// definition for every kernel that computes it, so they agree bit for bit.
__device__ __forceinline__ uint16_t silu_mul_bf16(float g, float u) {
  const float s = bf16_bits_to_f32(f32_to_bf16_bits(g / (1.f + __expf(-g))));
  return (uint16_t)f32_to_bf16_bits(s * u);
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

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, true));
}

// Sum over aligned groups of WIDTH consecutive lanes with DPP (no LDS traffic).
// WIDTH <= 16: every lane of the group holds the total.  WIDTH 32: lanes 16-31
// of each 32-lane half hold it.  WIDTH 64: lane 63 holds it.
template <int WIDTH>
__device__ __forceinline__ float dpp_group_sum(float v) {
  if constexpr (WIDTH >= 2) v += dpp_f32<0xb1>(v);   // quad_perm [1,0,3,2]
  if constexpr (WIDTH >= 4) v += dpp_f32<0x4e>(v);   // quad_perm [2,3,0,1]
  if constexpr (WIDTH >= 8) v += dpp_f32<0x141>(v);  // row_half_mirror
  if constexpr (WIDTH >= 16) v += dpp_f32<0x140>(v); // row_mirror
  if constexpr (WIDTH >= 32) v += dpp_f32<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
  if constexpr (WIDTH >= 64) v += dpp_f32<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
  return v;
}

// Lane (within its WIDTH group) that holds dpp_group_sum's result.
template <int WIDTH>
constexpr int dpp_sum_lane() {
  return WIDTH <= 16 ? 0 : WIDTH - 1;
}

// LDS-only barrier: waits for this wave's LDS operations, not its global loads.
__device__ __forceinline__ void lds_barrier() {
  __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Raw buffer access (gfx9 descriptor: 32-bit byte range, stride 0).  A load
// whose offset lies outside [0, bytes) returns zeros without touching memory,
// so tails need no clamping; all addressing is a 32-bit lane offset plus
// compile-time immediates off an SGPR base.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kBufNT = 2;  // cache policy bit: non-temporal (streamed once)

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint64_t bytes) {
  const uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)n, 0x00020000);
}
template <int AUX = 0>
__device__ __forceinline__ u32x4_t buf_load16(rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, AUX));
}
__device__ __forceinline__ u32x2_t buf_load8(rsrc_t r, uint32_t voff) {
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 0));
}
__device__ __forceinline__ uint32_t buf_load2(rsrc_t r, uint32_t voff) {
  return (uint32_t)__builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(r, voff, 0, 0));
}
constexpr uint32_t kOutOfRange = 0x80000000u;  // an offset no descriptor here covers

// Non-temporal 16-byte load (weights are streamed once per call).
__device__ __forceinline__ u32x4_t load_stream_u4(const u32x4_t* p) {
  return __builtin_nontemporal_load(p);
}

}  // namespace mq
