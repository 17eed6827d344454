// Decoder-step kernels around the quantized linears of the Qwen2 graph
// (python/mlx_worker/native_mlx/models/qwen2.py:47-163), fused so that a
// decode step is a handful of launches instead of dozens of elementwise ones:
//
//  * rmsnorm_kernel      nn.RMSNorm (qwen2.py:140-145, 187), optionally after
//                        the residual add before it (qwen2.py:158-163):
//                        h = bf16(x + r) is written out, and
//                        out = bf16(h * rsqrt(mean(h^2) + eps) * w) in float32;
//  * rope_append_kernel  mx.fast.rope (traditional=False) on q and k of one
//                        token per sequence (qwen2.py:93-108), q rounded to
//                        bfloat16, k and v written into the paged cache at the
//                        token's slot (cache.py:459-471: slot = page * page_size
//                        + pos % page_size);
//  * attn_split_kernel   attention of one query token per sequence over its
//    + attn_combine      cached positions 0..pos (attention.py:206-298: the
//                        reference gathers the pages into dense rows and calls
//                        scaled_dot_product_attention).  Query heads that share
//                        a KV head are scored together; the positions are split
//                        over blocks (partial max, sum and weighted values per
//                        split, float32), and a second kernel combines them;
//  * silu_mul_kernel     silu(gate) * up (qwen2.py:43-44, 132-133).
//
// KV pages are the reference's layout (cache.py:686-695): per layer
// bfloat16 [num_pages, page_size, kv_heads, head_dim]; a sequence's pages are
// listed in its row of an int32 page table [B, pages_per_seq].
#include <algorithm>

#include "mq_common.h"
#include "mq_internal.h"

namespace mq {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float bf16r(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// Positions and page ids come from device memory the host does not inspect;
// clamping them keeps a bad table or position inside the cache (wrong values
// in, wrong values out, never an access outside the buffers).
__device__ __forceinline__ int64_t clamp_index(int64_t v, int64_t n) {
  return v < 0 ? 0 : (v >= n ? n - 1 : v);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---------------------------------------------------------------- RMSNorm
// One row per block, 8 elements (16 bytes) per thread and pass; dim <= 8192.
constexpr int kNormMaxUnits = 4;

__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res_in,
    uint16_t* __restrict__ res_out, const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
    int dim, float eps) {
  __shared__ float red[kThreads / 64];
  const int64_t row = blockIdx.x;
  const int units = dim / 8;
  u32x4_t hv[kNormMaxUnits], wv[kNormMaxUnits];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNormMaxUnits; ++k) {
    const int u = threadIdx.x + k * kThreads;
    if (u < units) {
      // the weights now, not after the reduction's barrier: one memory round
      // trip less on the kernel's critical path
      wv[k] = reinterpret_cast<const u32x4_t*>(w)[u];
      u32x4_t v = reinterpret_cast<const u32x4_t*>(x + row * dim)[u];
      if (res_in) {
        const u32x4_t r = reinterpret_cast<const u32x4_t*>(res_in + row * dim)[u];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          v[q] = pack_bf16x2(lo_bf16(v[q]) + lo_bf16(r[q]), hi_bf16(v[q]) + hi_bf16(r[q]));
        reinterpret_cast<u32x4_t*>(res_out + row * dim)[u] = v;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float a = lo_bf16(v[q]), b = hi_bf16(v[q]);
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
      hv[k] = v;
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = 0.f;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) ss += red[i];
  const float inv = rsqrtf(ss / (float)dim + eps);
#pragma unroll
  for (int k = 0; k < kNormMaxUnits; ++k) {
    const int u = threadIdx.x + k * kThreads;
    if (u < units) {
      u32x4_t o;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = pack_bf16x2(lo_bf16(hv[k][q]) * inv * lo_bf16(wv[k][q]),
                           hi_bf16(hv[k][q]) * inv * hi_bf16(wv[k][q]));
      reinterpret_cast<u32x4_t*>(out + row * dim)[u] = o;
    }
  }
}

// ---------------------------------------------------------------- RoPE + append
// Grid (B, ceil((nh + nkv) / 4) + 1), 256 threads.  Block (b, y) takes heads
// 4y .. 4y+3 (q heads, then k heads), one wave per head, lane i < d/2 holding
// the rotated pair (i, i + d/2); the last y copies the v heads.  qkv bf16
// [B, (nh + 2 nkv) * d] (q heads, k heads, v heads); q_out bf16 [B, nh, d];
// cos/sin float32 [positions, d/2].  With q_norm / k_norm (Qwen3,
// qwen3.py:61-62,84-85) each head is first RMS-normalised over d with that
// weight and rounded to bfloat16, as nn.RMSNorm stores it.
constexpr int kRopeHeadsPerBlock = kThreads / 64;

// The rotated pair (x1 c - x2 s, x2 c + x1 s), each with one product rounded
// and the other fused, spelled out so that every kernel rounds it alike.
__device__ __forceinline__ float rope_lo(float x1, float x2, float c, float s) {
  return fmaf(x1, c, -(x2 * s));
}
__device__ __forceinline__ float rope_hi(float x1, float x2, float c, float s) {
  return fmaf(x2, c, x1 * s);
}

__global__ __launch_bounds__(kThreads) void rope_append_kernel(
    const uint16_t* __restrict__ qkv, const int64_t* __restrict__ pos,
    const int32_t* __restrict__ page_table, int pages_per_seq, int page_size, int num_pages,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm, float eps,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_pages, uint16_t* __restrict__ v_pages,
    int nh, int nkv, int d) {
  const int64_t b = blockIdx.x;
  const int64_t p = clamp_index(pos[b], (int64_t)pages_per_seq * page_size);
  const int64_t page = clamp_index(page_table[b * pages_per_seq + p / page_size], num_pages);
  const int64_t slot = page * page_size + p % page_size;
  const uint16_t* row = qkv + b * (int64_t)(nh + 2 * nkv) * d;
  if ((int)blockIdx.y * kRopeHeadsPerBlock >= nh + nkv) {  // the v heads
    for (int e = threadIdx.x; e < nkv * d; e += kThreads)
      v_pages[slot * nkv * (int64_t)d + e] = row[(nh + nkv) * d + e];
    return;
  }
  const int half = d / 2;
  const int lane = threadIdx.x & 63;
  const int hh = blockIdx.y * kRopeHeadsPerBlock + (threadIdx.x >> 6);
  if (hh >= nh + nkv) return;  // whole waves
  const uint16_t* norm = hh < nh ? q_norm : k_norm;
  uint16_t* dst = hh < nh ? q_out + (b * nh + hh) * (int64_t)d
                          : k_pages + (slot * nkv + (hh - nh)) * (int64_t)d;
  for (int i0 = 0; i0 < half; i0 += 64) {  // one pass for d <= 128
    const int i = i0 + lane;
    float x1 = 0.f, x2 = 0.f;
    if (i < half) {
      x1 = bf16_bits_to_f32(row[hh * d + i]);
      x2 = bf16_bits_to_f32(row[hh * d + i + half]);
    }
    if (norm) {  // uniform per wave; d <= 128 so the head is this one pass
      const float inv = rsqrtf(wave_sum(fmaf(x1, x1, x2 * x2)) / (float)d + eps);
      if (i < half) {
        x1 = bf16r(x1 * inv * bf16_bits_to_f32(norm[i]));
        x2 = bf16r(x2 * inv * bf16_bits_to_f32(norm[i + half]));
      }
    }
    if (i < half) {
      const float c = cos_t[p * half + i], sn = sin_t[p * half + i];
      dst[i] = (uint16_t)f32_to_bf16_bits(rope_lo(x1, x2, c, sn));
      dst[i + half] = (uint16_t)f32_to_bf16_bits(rope_hi(x1, x2, c, sn));
    }
  }
}

// The same for many rows at once (a prefill chunk's tokens), head_dim 32, 64
// or 128 and 16-byte aligned operands: every (row, q/k head) pair is taken by
// H = d / 16 adjacent lanes, lane j holding the rotated pairs 8j .. 8j + 7
// (16-byte loads and stores of both halves; cos/sin 32 bytes each).  The
// blocks after the pairs' copy the v heads, 16 bytes a lane.  The norm's sum
// of squares is wave_sum's: its xor butterfly over lanes 0 .. d/2 - 1 (the
// lanes past d/2 add exact zeros) is a balanced tree in lane order, which the
// lane's own 8 pairs (three levels) and shuffles across the H lanes (xor 1, 2,
// 4) reproduce -- so each (row, head) gets rope_append_kernel's bits.
constexpr int64_t kRopeRowsMin = 1024;  // rows from which this grid is used

__global__ __launch_bounds__(kThreads) void rope_append_rows_kernel(
    const uint16_t* __restrict__ qkv, const int64_t* __restrict__ pos,
    const int32_t* __restrict__ page_table, int pages_per_seq, int page_size, int num_pages,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm, float eps,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_pages, uint16_t* __restrict__ v_pages,
    int64_t B, int nh, int nkv, int d, int64_t pair_blocks) {
  const int H = d / 16, half = d / 2;
  const int64_t row_elems = (int64_t)(nh + 2 * nkv) * d;
  auto slot_of = [&](int64_t b, int64_t p) {
    const int64_t page = clamp_index(page_table[b * pages_per_seq + p / page_size], num_pages);
    return page * page_size + p % page_size;
  };
  if ((int64_t)blockIdx.x >= pair_blocks) {  // v rows: nkv * d / 8 lanes a row
    const int per_row = nkv * d / 8;
    const int64_t u = ((int64_t)blockIdx.x - pair_blocks) * kThreads + threadIdx.x;
    const int64_t b = u / per_row;
    if (b >= B) return;
    const int e = (int)(u % per_row) * 8;
    const int64_t p = clamp_index(pos[b], (int64_t)pages_per_seq * page_size);
    *reinterpret_cast<u32x4_t*>(v_pages + slot_of(b, p) * nkv * (int64_t)d + e) =
        *reinterpret_cast<const u32x4_t*>(qkv + b * row_elems + (int64_t)(nh + nkv) * d + e);
    return;
  }
  const int64_t pair = (int64_t)blockIdx.x * (kThreads / H) + threadIdx.x / H;
  const int j = threadIdx.x % H;
  const int64_t npairs = B * (nh + nkv);
  const bool live = pair < npairs;
  const int64_t pr = live ? pair : npairs - 1;  // past the end: repeat the last (not stored)
  const int64_t b = pr / (nh + nkv);
  const int hh = (int)(pr % (nh + nkv));
  const int64_t p = clamp_index(pos[b], (int64_t)pages_per_seq * page_size);
  const uint16_t* src = qkv + b * row_elems + (int64_t)hh * d + 8 * j;
  const u32x4_t v1 = *reinterpret_cast<const u32x4_t*>(src);
  const u32x4_t v2 = *reinterpret_cast<const u32x4_t*>(src + half);
  const float* cp = cos_t + p * half + 8 * j;
  const float* sp = sin_t + p * half + 8 * j;
  const f32x4_t c0 = *reinterpret_cast<const f32x4_t*>(cp), c1 = *reinterpret_cast<const f32x4_t*>(cp + 4);
  const f32x4_t s0 = *reinterpret_cast<const f32x4_t*>(sp), s1 = *reinterpret_cast<const f32x4_t*>(sp + 4);
  const uint16_t* norm = hh < nh ? q_norm : k_norm;
  float x1[8], x2[8];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    x1[2 * q] = lo_bf16(v1[q]), x1[2 * q + 1] = hi_bf16(v1[q]);
    x2[2 * q] = lo_bf16(v2[q]), x2[2 * q + 1] = hi_bf16(v2[q]);
  }
  if (norm) {  // uniform per pair (a pair's lanes are adjacent; the shuffles stay inside it)
    const u32x4_t w1 = *reinterpret_cast<const u32x4_t*>(norm + 8 * j);
    const u32x4_t w2 = *reinterpret_cast<const u32x4_t*>(norm + half + 8 * j);
    float e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = fmaf(x1[i], x1[i], x2[i] * x2[i]);
    float ss = ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
    for (int off = 1; off < H; off <<= 1) ss += __shfl_xor(ss, off, 64);
    const float inv = rsqrtf(ss / (float)d + eps);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      x1[2 * q] = bf16r(x1[2 * q] * inv * lo_bf16(w1[q]));
      x1[2 * q + 1] = bf16r(x1[2 * q + 1] * inv * hi_bf16(w1[q]));
      x2[2 * q] = bf16r(x2[2 * q] * inv * lo_bf16(w2[q]));
      x2[2 * q + 1] = bf16r(x2[2 * q + 1] * inv * hi_bf16(w2[q]));
    }
  }
  if (!live) return;
  const float c[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  const float sn[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  u32x4_t o1, o2;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = 2 * q;
    o1[q] = pack_bf16x2(rope_lo(x1[i], x2[i], c[i], sn[i]),
                        rope_lo(x1[i + 1], x2[i + 1], c[i + 1], sn[i + 1]));
    o2[q] = pack_bf16x2(rope_hi(x1[i], x2[i], c[i], sn[i]),
                        rope_hi(x1[i + 1], x2[i + 1], c[i + 1], sn[i + 1]));
  }
  uint16_t* dst = hh < nh ? q_out + (b * nh + hh) * (int64_t)d
                          : k_pages + (slot_of(b, p) * nkv + (hh - nh)) * (int64_t)d;
  *reinterpret_cast<u32x4_t*>(dst + 8 * j) = o1;
  *reinterpret_cast<u32x4_t*>(dst + half + 8 * j) = o2;
}

// ---------------------------------------------------------------- attention
// Grid (splits, nkv, B), 256 threads (4 waves).  A split block takes its
// positions in passes of 64; wave w takes positions t0 + 16w + [0, 16) of the
// pass t0:
//  * scores S^T = K Q^T by v_mfma_f32_16x16x32_bf16: A = the wave's 16 K
//    rows (lane l holds dims 32s + 8(l/16) .. +7 of position l % 16 for
//    k-step s, 16 contiguous bytes of the cached row), B = the KV head's REP
//    query heads (columns >= REP zero).  Lane l gets the scores of head l % 16
//    at positions 4(l/16) .. +3;
//  * an online softmax per wave over its positions: a head's max and sum
//    over the wave's 16 positions from the lane's 4 and two lane shuffles;
//  * P V by v_mfma_f32_16x16x16_bf16: A = P in bfloat16, exactly as the
//    scores sit in the lanes; B = V, whose rows the wave stages through a
//    private LDS tile so that a lane can read 4 positions of one dim; the
//    output tile t holds heads 4(l/16) .. +3 at dim 16t + l % 16 (no block
//    barrier inside the loop);
//  * the four waves' (max, sum, weighted values) merged through LDS at the
//    end.
// Scores are kept in log2 units (q.k * scale * log2 e), so every exponential
// is exp2.
//
// Partials per (b, kv head, split), float32: m[REP], s[REP], acc[REP][D];
// splits past the sequence's end are neither written nor read.  A grid of
// one split per sequence writes the normalised output itself (no combine).
constexpr int kMaxChunk = 512;
constexpr int kPass = 64;  // positions per pass: 16 per wave
// Waves per SIMD (= blocks per CU: a 4-wave block puts one wave on each SIMD)
// the split kernels are held to, by query heads per KV head.
constexpr int kAttnWaves[9] = {0, 4, 4, 4, 4, 4, 4, 4, 4};
constexpr float kNoScore = -1e30f;  // running max before the first position

// Shared memory of one split block.
template <int REP, int D>
struct AttnShared {
  __align__(16) uint16_t fresh[2][D];  // the new position's K and V rows (attn_step)
  int32_t slot_of[kMaxChunk];
  // per wave: its 16 V rows of the pass, rows padded to D + 4 elements so that
  // a column read by the 4 lane groups spreads over distinct banks
  __align__(16) uint16_t v_tile[kThreads / 64][16][D + 4];
  __align__(16) float f_tile[kThreads / 64][16];  // per wave: the pass's rescale per head
  float mrg_m[kThreads / 64][REP], mrg_s[kThreads / 64][REP];
  float mrg_a[kThreads / 64][REP][D];
};

template <int WIDTH>
__device__ __forceinline__ float dpp_group_max(float v) {
  static_assert(WIDTH == 16, "rows of 16 lanes");
  v = fmaxf(v, dpp_f32<0xb1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4e>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_f32<0x140>(v));  // row_mirror
  return v;
}

// One pass's rows of a wave, as this lane holds them: the MFMA B operand
// (its slice of the K row of position l % 16) and its dims of the wave's 16
// V rows (D = 128: a bf16 pair; D = 64: one bf16 in the low half).
template <int D>
struct AttnPass {
  u32x4_t k[D / 32];
  uint32_t v[16];
};

// Loads a pass's rows: `slot` is the cache slot of this lane's position
// (l % 16 of the wave's 16); kb / vb point at the KV head's dim 0 of slot 0.
template <int D>
__device__ __forceinline__ void attn_load_pass(AttnPass<D>& ps, const uint16_t* kb,
                                               const uint16_t* vb, int64_t row_elems, int slot) {
  const int lane = threadIdx.x & 63, g = lane >> 4;
  const uint16_t* kr = kb + slot * row_elems + 8 * g;
#pragma unroll
  for (int s = 0; s < D / 32; ++s) ps.k[s] = *reinterpret_cast<const u32x4_t*>(kr + 32 * s);
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint16_t* vr = vb + __builtin_amdgcn_readlane(slot, j) * row_elems;  // lane j: position j
    if constexpr (D == 128)
      ps.v[j] = reinterpret_cast<const uint32_t*>(vr)[lane];
    else
      ps.v[j] = vr[lane];
  }
}

// The split's partials over positions l0 + [0, n) of the KV head whose rows
// start at kb / vb (row r at r * row_elems).  qa: this lane's query operand
// (head l % 16, dims 32s + 8(l/16) .. +7).  Position `fresh` of the split (or
// -1) takes its K / V row from sh.fresh instead of the cache.  `first` holds
// the first pass's rows, loaded before n was known; sh.slot_of the slots of
// positions [0, n) (read from the second pass on).  Writes pm[REP], ps[REP],
// pa[REP][D] -- or, with `direct` (the sequence's only split), its REP heads'
// output rows bf16(pa / ps), which is what the combine makes of one split.
template <int REP, int D>
__device__ __forceinline__ void attn_block(const u32x4_t (&qa)[D / 32], AttnShared<REP, D>& sh,
                                           int n, const uint16_t* kb, const uint16_t* vb,
                                           int64_t row_elems, float scale_log2, int fresh,
                                           const AttnPass<D>& first, float* pm, float* ps,
                                           float* pa, uint16_t* direct) {
  constexpr int NS = D / 32, NT = D / 16, VS = D + 4, WAVES = kThreads / 64;
  static_assert(REP <= 16 && (D == 64 || D == 128), "one MFMA column per query head");
  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  float m = kNoScore, s = 0.f;  // running max / sum of head c over the wave's positions
  f32x4_t acc[NT];              // tile t: heads 4g + r at dim 16t + c
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  uint16_t* vt = &sh.v_tile[wave][0][0];
  float* fw = sh.f_tile[wave];
  AttnPass<D> cur = first;
  for (int t0 = 0; t0 < n; t0 += kPass) {
    const int base = t0 + 16 * wave;  // the wave's first position of the pass
    if (t0 > 0) attn_load_pass<D>(cur, kb, vb, row_elems, sh.slot_of[min(base + c, n - 1)]);
    if (fresh >= base && fresh < base + 16) {  // uniform
      if (c == fresh - base) {
#pragma unroll
        for (int k = 0; k < NS; ++k)
          cur.k[k] = *reinterpret_cast<const u32x4_t*>(sh.fresh[0] + 32 * k + 8 * g);
      }
      const uint32_t fv = D == 128 ? reinterpret_cast<const uint32_t*>(sh.fresh[1])[lane]
                                   : (uint32_t)sh.fresh[1][lane];
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (base + j == fresh) cur.v[j] = fv;
    }
    // the V rows to the wave's tile; rows past the end may hold anything: zeros
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t v = base + j < n ? cur.v[j] : 0u;
      if constexpr (D == 128)
        *reinterpret_cast<uint32_t*>(vt + j * VS + 2 * lane) = v;
      else
        vt[j * VS + lane] = (uint16_t)v;
    }

    f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < NS; ++k)
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, cur.k[k]),
                                                  __builtin_bit_cast(bf16x8_t, qa[k]), d, 0, 0,
                                                  0);
    // d[r]: head c at position base + 4g + r
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = base + 4 * g + r < n ? d[r] * scale_log2 : -INFINITY;
    float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m, mx);
    const float f = __builtin_amdgcn_exp2f(m - mn);  // arguments <= 0: no range fix-up needed
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(x[r] - mn);
    float psum = (p[0] + p[1]) + (p[2] + p[3]);
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    s = fmaf(s, f, psum);
    m = mn;
    if (g == 0) fw[c] = f;
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's tiles are written

    const f32x4_t fr = *reinterpret_cast<const f32x4_t*>(fw + 4 * g);  // heads 4g + r
    const u32x2_t pp = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};
    const s16x4_t pa16 = __builtin_bit_cast(s16x4_t, pp);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint16_t* col = vt + 4 * g * VS + 16 * t + c;
      const s16x4_t vb16 = {(short)col[0], (short)col[VS], (short)col[2 * VS],
                            (short)col[3 * VS]};
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa16, vb16, acc[t] * fr, 0, 0, 0);
    }
    __asm__ volatile("" ::: "memory");  // this pass's tile reads stay ahead of the next writes
  }

  // merge the waves through LDS
  if (g == 0 && c < REP) {
    sh.mrg_m[wave][c] = m;
    sh.mrg_s[wave][c] = s;
  }
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (4 * g + r < REP) sh.mrg_a[wave][4 * g + r][16 * t + c] = acc[t][r];
  __syncthreads();
  for (int e = threadIdx.x; e < REP * D; e += kThreads) {
    const int r = e / D, dd = e % D;
    float mx = sh.mrg_m[0][r];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) mx = fmaxf(mx, sh.mrg_m[w][r]);
    float v = 0.f, sum = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float fw2 = exp2f(sh.mrg_m[w][r] - mx);
      v = fmaf(sh.mrg_a[w][r][dd], fw2, v);
      sum = fmaf(sh.mrg_s[w][r], fw2, sum);
    }
    if (direct) {  // uniform
      direct[e] = (uint16_t)f32_to_bf16_bits(v / sum);
    } else {
      pa[e] = v;
      if (dd == 0) {
        pm[r] = mx;
        ps[r] = sum;
      }
    }
  }
}

// Cache slot (page * page_size + offset) of position l of a sequence whose
// page table is `table`; positions past the table's end map into its last
// page, so that a speculative lookup stays in bounds.
__device__ __forceinline__ int attn_slot(const int32_t* table, int pages_per_seq, int page_size,
                                         int num_pages, int l) {
  return (int)(clamp_index(table[min(l / page_size, pages_per_seq - 1)], num_pages) * page_size +
               l % page_size);
}

// The loads a split block issues before it knows the sequence's length, so
// that none of them waits for the position: the slots of the split's
// positions l0 + threadIdx.x + kThreads * k (for sh.slot_of), and the first
// pass's rows.  Positions past the sequence's end are looked up too and
// masked later.
template <int D>
struct AttnPrefetch {
  static constexpr int kSlots = kMaxChunk / kThreads;
  int slot[kSlots];
  AttnPass<D> first;

  __device__ __forceinline__ void issue(const int32_t* table, int pages_per_seq, int page_size,
                                        int num_pages, int l0, int chunk, const uint16_t* kb,
                                        const uint16_t* vb, int64_t row_elems) {
    const int wave = threadIdx.x >> 6, c = threadIdx.x & 15;
    attn_load_pass<D>(first, kb, vb, row_elems,
                      attn_slot(table, pages_per_seq, page_size, num_pages,
                                l0 + min(16 * wave + c, chunk - 1)));
#pragma unroll
    for (int k = 0; k < kSlots; ++k)
      slot[k] = attn_slot(table, pages_per_seq, page_size, num_pages,
                          l0 + min((int)threadIdx.x + kThreads * k, chunk - 1));
  }

  // sh.slot_of[i] for the split's first n positions
  __device__ __forceinline__ void store_slots(int32_t* slot_of, int n) const {
#pragma unroll
    for (int k = 0; k < kSlots; ++k)
      if ((int)threadIdx.x + kThreads * k < n) slot_of[threadIdx.x + kThreads * k] = slot[k];
  }
};

// This lane's A operand from the KV head's REP query heads (q: head 0, dim 0,
// heads `head_stride` elements apart): head l % 16, dims 32s + 8(l/16) .. +7.
template <int REP, int D>
__device__ __forceinline__ void attn_load_q(u32x4_t (&qa)[D / 32], const uint16_t* q,
                                            int64_t head_stride) {
  const int c = threadIdx.x & 15, g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int s = 0; s < D / 32; ++s)
    qa[s] = c < REP ? *reinterpret_cast<const u32x4_t*>(q + c * head_stride + 32 * s + 8 * g)
                    : u32x4_t{0u, 0u, 0u, 0u};
}

// (The pointers the speculative loads read are not __restrict__: with it the
// compiler may sink those loads below the asm barrier that orders them ahead
// of the first wait.)
template <int REP, int D>
__global__ __launch_bounds__(kThreads, kAttnWaves[REP]) void attn_split_kernel(
    const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages, const int32_t* page_table,
    int pages_per_seq, int page_size, int num_pages, const int64_t* pos,
    float* __restrict__ part, uint16_t* __restrict__ out, int nkv, int chunk,
    float scale_log2) {
  __shared__ AttnShared<REP, D> sh;
  const int split = blockIdx.x, kvh = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int splits = gridDim.x;
  const int l0 = split * chunk;
  const int nh = nkv * REP;
  const int64_t pos_b = pos[b];
  asm volatile("" ::: "memory");  // the position's load goes out first
  u32x4_t qa[D / 32];
  attn_load_q<REP, D>(qa, q + (b * nh + kvh * REP) * (int64_t)D, D);
  AttnPrefetch<D> pf;
  pf.issue(page_table + b * pages_per_seq, pages_per_seq, page_size, num_pages, l0, chunk,
           k_pages + kvh * D, v_pages + kvh * D, (int64_t)nkv * D);
  asm volatile("" ::: "memory");  // every load above is issued before the first wait
  const int L = (int)clamp_index(pos_b, (int64_t)pages_per_seq * page_size) + 1;
  const int n = min(L - l0, chunk);
  if (n <= 0) return;  // past the sequence's end
  float* pm = part + ((b * nkv + kvh) * splits + split) * (int64_t)(REP * (D + 2));
  pf.store_slots(sh.slot_of, n);
  __syncthreads();
  attn_block<REP, D>(qa, sh, n, k_pages + kvh * D, v_pages + kvh * D, (int64_t)nkv * D,
                     scale_log2, -1, pf.first, pm, pm + REP, pm + 2 * REP,
                     splits == 1 ? out + (b * nh + kvh * REP) * (int64_t)D : nullptr);
}

// The split kernel of one decode step of a layer's attention, straight from
// the QKV projection: every split block ropes (and q-norms) the query heads of
// its KV head from qkv; the split holding the new position also ropes k, and
// writes k and v into the pages (using them from registers for that
// position).  The partials go to `part` for attn_combine_kernel.  (Combining
// in the last split to finish would save that launch, but publishing the
// partials to a block on another XCD takes an agent-scope release -- an L2
// write-back per block -- which costs far more than the launch.)
template <int REP, int D>
__global__ __launch_bounds__(kThreads, kAttnWaves[REP]) void attn_step_kernel(
    const uint16_t* __restrict__ qkv, const int64_t* pos, const int32_t* page_table,
    int pages_per_seq, int page_size, int num_pages, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, const uint16_t* __restrict__ q_norm,
    const uint16_t* __restrict__ k_norm, float eps, uint16_t* k_pages, uint16_t* v_pages,
    float* __restrict__ part, uint16_t* __restrict__ out, int nkv, int chunk, float scale_log2) {
  constexpr int LANES = D / 8, HALF = D / 2, WAVES = kThreads / 64;
  static_assert(HALF <= 64, "one rotated pair per lane");
  __shared__ AttnShared<REP, D> sh;
  __shared__ __align__(16) uint16_t qs[REP][D];  // the roped query heads
  const int split = blockIdx.x, kvh = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int splits = gridDim.x;
  const int l0 = split * chunk;
  const int64_t pos_b = pos[b];
  asm volatile("" ::: "memory");  // the position's load goes out first
  AttnPrefetch<D> pf;
  pf.issue(page_table + b * pages_per_seq, pages_per_seq, page_size, num_pages, l0, chunk,
           k_pages + kvh * D, v_pages + kvh * D, (int64_t)nkv * D);
  asm volatile("" ::: "memory");  // every load above is issued before the first wait
  const int p = (int)clamp_index(pos_b, (int64_t)pages_per_seq * page_size);
  const int L = p + 1;
  const int n = min(L - l0, chunk);
  if (n <= 0) return;  // past the sequence's end
  const bool owner = p < l0 + n;  // this split holds the new position
  const int nh = nkv * REP;
  const uint16_t* row = qkv + b * (int64_t)(nh + 2 * nkv) * D;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, sub = threadIdx.x % LANES;
  for (int hh = wave; hh < REP + (owner ? 1 : 0); hh += WAVES) {
    const bool is_k = hh == REP;
    const int src = is_k ? nh + kvh : kvh * REP + hh;
    const uint16_t* norm = is_k ? k_norm : q_norm;
    float x1 = 0.f, x2 = 0.f;
    if (lane < HALF) {
      x1 = bf16_bits_to_f32(row[src * D + lane]);
      x2 = bf16_bits_to_f32(row[src * D + lane + HALF]);
    }
    if (norm) {  // uniform per wave
      const float inv = rsqrtf(wave_sum(fmaf(x1, x1, x2 * x2)) / (float)D + eps);
      if (lane < HALF) {
        x1 = bf16r(x1 * inv * bf16_bits_to_f32(norm[lane]));
        x2 = bf16r(x2 * inv * bf16_bits_to_f32(norm[lane + HALF]));
      }
    }
    if (lane < HALF) {
      const float c = cos_t[(int64_t)p * HALF + lane], sn = sin_t[(int64_t)p * HALF + lane];
      uint16_t* dst = is_k ? sh.fresh[0] : qs[hh];
      dst[lane] = (uint16_t)f32_to_bf16_bits(rope_lo(x1, x2, c, sn));
      dst[lane + HALF] = (uint16_t)f32_to_bf16_bits(rope_hi(x1, x2, c, sn));
    }
  }
  if (owner && threadIdx.x < LANES)  // the new v row, as is
    reinterpret_cast<u32x4_t*>(sh.fresh[1])[threadIdx.x] =
        reinterpret_cast<const u32x4_t*>(row + (nh + nkv + kvh) * D)[threadIdx.x];
  pf.store_slots(sh.slot_of, n);
  __syncthreads();
  const int64_t row_elems = (int64_t)nkv * D;
  if (owner && threadIdx.x < LANES) {  // append the new k and v rows to the pages
    const int64_t at = (int64_t)sh.slot_of[p - l0] * row_elems + kvh * D + sub * 8;
    *reinterpret_cast<u32x4_t*>(k_pages + at) = reinterpret_cast<const u32x4_t*>(sh.fresh[0])[sub];
    *reinterpret_cast<u32x4_t*>(v_pages + at) = reinterpret_cast<const u32x4_t*>(sh.fresh[1])[sub];
  }
  u32x4_t qa[D / 32];
  attn_load_q<REP, D>(qa, &qs[0][0], D);
  float* pm = part + ((b * nkv + kvh) * splits + split) * (int64_t)(REP * (D + 2));
  attn_block<REP, D>(qa, sh, n, k_pages + kvh * D, v_pages + kvh * D, row_elems, scale_log2,
                     owner ? p - l0 : -1, pf.first, pm, pm + REP, pm + 2 * REP,
                     splits == 1 ? out + (b * nh + kvh * REP) * (int64_t)D : nullptr);
}

// Grid (nh, B), D threads: out bf16 [B, nh * D] = sum over the sequence's
// splits of the partials rescaled to their common max, over the rescaled sum.
// The partials of the first kCombineAhead splits are loaded before the
// position (which says how many splits the sequence used) arrives; the pointers
// are not __restrict__ so that the asm barriers keep those loads ahead of the
// wait.
constexpr int kCombineAhead = 16;

template <int REP, int D>
__global__ __launch_bounds__(D) void attn_combine_kernel(const float* part, const int64_t* pos,
                                                         int pages_per_seq, int page_size,
                                                         uint16_t* __restrict__ out, int nkv,
                                                         int splits, int chunk) {
  constexpr int STRIDE = REP * (D + 2);
  const int hh = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int kvh = hh / REP, r = hh % REP;
  const int64_t pos_b = pos[b];
  asm volatile("" ::: "memory");  // the position's load goes out first
  const float* base = part + (b * nkv + kvh) * splits * (int64_t)STRIDE;
  float pm[kCombineAhead], ps[kCombineAhead], pa[kCombineAhead];
#pragma unroll
  for (int sp = 0; sp < kCombineAhead; ++sp)
    if (sp < splits) {  // uniform; splits past the used ones are loaded and ignored
      const float* p = base + sp * STRIDE;
      pm[sp] = p[r];
      ps[sp] = p[REP + r];
      pa[sp] = p[2 * REP + r * D + threadIdx.x];
    }
  asm volatile("" ::: "memory");  // every load above is issued before the first wait
  const int L = (int)clamp_index(pos_b, (int64_t)pages_per_seq * page_size) + 1;
  const int used = min(splits, (L + chunk - 1) / chunk);
  float mx = -INFINITY;
#pragma unroll
  for (int sp = 0; sp < kCombineAhead; ++sp)
    if (sp < used) mx = fmaxf(mx, pm[sp]);
  for (int sp = kCombineAhead; sp < used; ++sp) mx = fmaxf(mx, base[sp * STRIDE + r]);
  float num = 0.f, den = 0.f;
#pragma unroll
  for (int sp = 0; sp < kCombineAhead; ++sp)
    if (sp < used) {
      const float f = exp2f(pm[sp] - mx);
      den = fmaf(f, ps[sp], den);
      num = fmaf(f, pa[sp], num);
    }
  for (int sp = kCombineAhead; sp < used; ++sp) {
    const float* p = base + sp * STRIDE;
    const float f = exp2f(p[r] - mx);
    den = fmaf(f, p[REP + r], den);
    num = fmaf(f, p[2 * REP + r * D + threadIdx.x], num);
  }
  out[(b * nkv * REP + hh) * (int64_t)D + threadIdx.x] = (uint16_t)f32_to_bf16_bits(num / den);
}

// ---------------------------------------------------------------- argmax
// Greedy decoding's argmax over each bfloat16 row (the next token, as the
// reference takes mx.argmax of each row's last logits, executor.py:406-414):
// one block per row, 16-byte loads, every element's (value, index) packed
// into a 64-bit key whose maximum is the first index of the largest value --
// the value as an order-preserving 16-bit key (-0 as +0, NaN above every
// number, as torch.argmax returns the first NaN) over the complemented index.
constexpr int kArgmaxThreads = 1024;

__device__ __forceinline__ uint64_t argmax_key(uint32_t u, uint32_t idx) {
  u &= 0xffffu;
  const uint32_t mag = u & 0x7fffu;
  const uint32_t key = mag > 0x7f80u ? 0xffffu          // NaN
                       : mag == 0     ? 0x8000u         // -0 and +0
                       : (u & 0x8000u) ? (~u & 0xffffu) // negative: larger magnitude lower
                                       : (u | 0x8000u);
  return ((uint64_t)key << 32) | (0xffffffffu - idx);
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const uint16_t* __restrict__ x,
                                                                     int64_t cols,
                                                                     int64_t* __restrict__ out) {
  const int64_t r = blockIdx.x;
  const rsrc_t rs = make_rsrc(x + r * cols, (uint64_t)cols * 2);
  const uint32_t units = (uint32_t)(cols / 8);  // 16-byte units (cols % 8 == 0)
  uint64_t best = 0;                             // below every element's key
#pragma unroll 4
  for (uint32_t u = threadIdx.x; u < units; u += kArgmaxThreads) {
    const u32x4_t v = buf_load16(rs, u * 16u);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint64_t a = argmax_key(v[q], 8u * u + 2u * q);
      const uint64_t b = argmax_key(v[q] >> 16, 8u * u + 2u * q + 1u);
      best = a > best ? a : best;
      best = b > best ? b : best;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)best, off, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(best >> 32), off, 64);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    best = o > best ? o : best;
  }
  __shared__ uint64_t wave_best[kArgmaxThreads / 64];
  if ((threadIdx.x & 63) == 0) wave_best[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 0; w < kArgmaxThreads / 64; ++w) best = wave_best[w] > best ? wave_best[w] : best;
    out[r] = (int64_t)(0xffffffffu - (uint32_t)best);
  }
}

// ---------------------------------------------------------------- SiLU * up
// gu bf16 [rows, 2 * inter] = (gate | up) -> out bf16 [rows, inter]
//   = bf16(bf16(silu(gate)) * up)
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const uint16_t* __restrict__ gu,
                                                            uint16_t* __restrict__ out,
                                                            int64_t rows, int inter) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;  // 8-element unit
  const int upr = inter / 8;
  if (i >= rows * upr) return;
  const int64_t r = i / upr, u = i % upr;
  const u32x4_t g = reinterpret_cast<const u32x4_t*>(gu + r * 2 * inter)[u];
  const u32x4_t up = reinterpret_cast<const u32x4_t*>(gu + r * 2 * inter + inter)[u];
  u32x4_t o;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    o[q] = silu_mul_bf16(lo_bf16(g[q]), lo_bf16(up[q])) |
           (uint32_t)silu_mul_bf16(hi_bf16(g[q]), hi_bf16(up[q])) << 16;
  reinterpret_cast<u32x4_t*>(out + r * inter)[u] = o;
}

// Blocks of attn_split_kernel / attn_step_kernel<REP, D> one CU holds at
// once.
int attn_blocks_per_cu(int rep) { return kAttnWaves[rep < 1 ? 1 : rep > 8 ? 8 : rep]; }

// Positions per split: whole passes (kPass positions), at most kMaxChunk,
// and as many splits as keep every CU busy in one round of blocks (a split is
// latency-bound, so a second round costs a full split).
int attn_chunk(int64_t B, int nkv, int rep, int d, int64_t capacity) {
  const int64_t pass = kPass;
  const int64_t blocks = B * nkv;
  const int64_t target = 256 * (int64_t)attn_blocks_per_cu(rep);
  int64_t splits = std::max<int64_t>(1, target / blocks);
  splits = std::min<int64_t>(splits, (capacity + pass - 1) / pass);
  int64_t chunk = (capacity + splits - 1) / splits;
  chunk = (chunk + pass - 1) / pass * pass;
  return (int)std::min<int64_t>(chunk, kMaxChunk);
}

}  // namespace

bool rmsnorm_supported(int64_t dim) {
  return dim > 0 && dim % 8 == 0 && dim <= 8 * kThreads * kNormMaxUnits;
}

bool decode_attention_supported(int nh, int nkv, int d) {
  return (d == 64 || d == 128) && nkv > 0 && nh % nkv == 0 && nh / nkv >= 1 && nh / nkv <= 8;
}

size_t decode_attention_workspace(int64_t B, int nh, int nkv, int d, int64_t capacity) {
  const int rep = nh / nkv;
  const int64_t chunk = attn_chunk(B, nkv, rep, d, capacity);
  const int64_t splits = (capacity + chunk - 1) / chunk;
  return (size_t)(B * nkv * splits * rep * (d + 2)) * sizeof(float);
}

hipError_t launch_rmsnorm(const uint16_t* x, const uint16_t* res_in, uint16_t* res_out,
                          const uint16_t* w, uint16_t* out, int64_t rows, int64_t dim, float eps,
                          hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(kThreads), 0, stream, x, res_in,
                     res_out, w, out, (int)dim, eps);
  return hipGetLastError();
}

hipError_t launch_rope_append(const uint16_t* qkv, const int64_t* pos, const int32_t* page_table,
                              int64_t pages_per_seq, int64_t page_size, int64_t num_pages,
                              const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                              const float* cos_t,
                              const float* sin_t, uint16_t* q_out, uint16_t* k_pages,
                              uint16_t* v_pages, int64_t B, int nh, int nkv, int d,
                              hipStream_t stream) {
  if (B == 0) return hipSuccess;
  const unsigned head_blocks = (unsigned)((nh + nkv + kRopeHeadsPerBlock - 1) / kRopeHeadsPerBlock);
  auto a16 = [](const void* ptr) { return ((uintptr_t)ptr & 15) == 0; };
  if (B >= kRopeRowsMin && (d == 32 || d == 64 || d == 128) && a16(qkv) && a16(cos_t) &&
      a16(sin_t) && a16(q_out) && a16(k_pages) && a16(v_pages) && (!q_norm || a16(q_norm)) &&
      (!k_norm || a16(k_norm))) {
    const int64_t pairs_per_block = kThreads / (d / 16);
    const int64_t pair_blocks = (B * (nh + nkv) + pairs_per_block - 1) / pairs_per_block;
    const int64_t v_blocks = (B * (nkv * d / 8) + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(rope_append_rows_kernel, dim3((unsigned)(pair_blocks + v_blocks)),
                       dim3(kThreads), 0, stream, qkv, pos, page_table, (int)pages_per_seq,
                       (int)page_size, (int)num_pages, cos_t, sin_t, q_norm, k_norm, eps, q_out,
                       k_pages, v_pages, B, nh, nkv, d, pair_blocks);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(rope_append_kernel, dim3((unsigned)B, head_blocks + 1), dim3(kThreads), 0,
                     stream, qkv, pos,
                     page_table, (int)pages_per_seq, (int)page_size, (int)num_pages, cos_t, sin_t,
                     q_norm, k_norm, eps, q_out, k_pages, v_pages, nh, nkv, d);
  return hipGetLastError();
}

namespace {
template <int D>
hipError_t launch_attention_d(const uint16_t* q, const uint16_t* k_pages, const uint16_t* v_pages,
                              const int32_t* page_table, int pages_per_seq, int page_size,
                              int num_pages, const int64_t* pos, int64_t B, int nh, int nkv,
                              float scale, float* workspace, uint16_t* out, int chunk, int splits,
                              hipStream_t stream) {
  const float scale_log2 = scale * 1.4426950408889634f;  // exp(x) = exp2(x log2 e)
  const dim3 grid((unsigned)splits, (unsigned)nkv, (unsigned)B);
  const dim3 cgrid((unsigned)nh, (unsigned)B);
#define MQ_ATTN(REP)                                                                            \
  case REP:                                                                                     \
    hipLaunchKernelGGL((attn_split_kernel<REP, D>), grid, dim3(kThreads), 0, stream, q,        \
                       k_pages, v_pages, page_table, pages_per_seq, page_size, num_pages, pos,  \
                       workspace, out, nkv, chunk, scale_log2);                                 \
    if (splits > 1) /* one split writes the output itself */                                   \
      hipLaunchKernelGGL((attn_combine_kernel<REP, D>), cgrid, dim3(D), 0, stream, workspace,  \
                         pos, pages_per_seq, page_size, out, nkv, splits, chunk);               \
    break;
  switch (nh / nkv) {
    MQ_ATTN(1)
    MQ_ATTN(2)
    MQ_ATTN(3)
    MQ_ATTN(4)
    MQ_ATTN(5)
    MQ_ATTN(6)
    MQ_ATTN(7)
    MQ_ATTN(8)
    default:
      return hipErrorInvalidValue;
  }
#undef MQ_ATTN
  return hipGetLastError();
}
}  // namespace

hipError_t launch_decode_attention(const uint16_t* q, const uint16_t* k_pages,
                                   const uint16_t* v_pages, const int32_t* page_table,
                                   int64_t pages_per_seq, int64_t page_size, int64_t num_pages,
                                   const int64_t* pos, int64_t B, int nh, int nkv, int d,
                                   float scale, float* workspace, uint16_t* out,
                                   hipStream_t stream) {
  if (B == 0) return hipSuccess;
  const int64_t capacity = pages_per_seq * page_size;
  const int chunk = attn_chunk(B, nkv, nh / nkv, d, capacity);
  const int splits = (int)((capacity + chunk - 1) / chunk);
  if (d == 64)
    return launch_attention_d<64>(q, k_pages, v_pages, page_table, (int)pages_per_seq,
                                  (int)page_size, (int)num_pages, pos, B, nh, nkv, scale,
                                  workspace, out, chunk, splits, stream);
  if (d == 128)
    return launch_attention_d<128>(q, k_pages, v_pages, page_table, (int)pages_per_seq,
                                   (int)page_size, (int)num_pages, pos, B, nh, nkv, scale,
                                   workspace, out, chunk, splits, stream);
  return hipErrorInvalidValue;
}

namespace {
template <int D>
hipError_t launch_step_d(const uint16_t* qkv, const int64_t* pos, const int32_t* page_table,
                         int pages_per_seq, int page_size, int num_pages, const float* cos_t,
                         const float* sin_t, const uint16_t* q_norm, const uint16_t* k_norm,
                         float eps, uint16_t* k_pages, uint16_t* v_pages, int64_t B, int nh,
                         int nkv, float scale, float* workspace, uint16_t* out, int chunk,
                         int splits, hipStream_t stream) {
  const float scale_log2 = scale * 1.4426950408889634f;
  const dim3 grid((unsigned)splits, (unsigned)nkv, (unsigned)B);
  const dim3 cgrid((unsigned)nh, (unsigned)B);
#define MQ_STEP(REP)                                                                            \
  case REP:                                                                                     \
    hipLaunchKernelGGL((attn_step_kernel<REP, D>), grid, dim3(kThreads), 0, stream, qkv, pos,  \
                       page_table, pages_per_seq, page_size, num_pages, cos_t, sin_t, q_norm,  \
                       k_norm, eps, k_pages, v_pages, workspace, out, nkv, chunk, scale_log2); \
    if (splits > 1) /* one split writes the output itself */                                   \
      hipLaunchKernelGGL((attn_combine_kernel<REP, D>), cgrid, dim3(D), 0, stream, workspace,  \
                         pos, pages_per_seq, page_size, out, nkv, splits, chunk);               \
    break;
  switch (nh / nkv) {
    MQ_STEP(1)
    MQ_STEP(2)
    MQ_STEP(3)
    MQ_STEP(4)
    MQ_STEP(5)
    MQ_STEP(6)
    MQ_STEP(7)
    MQ_STEP(8)
    default:
      return hipErrorInvalidValue;
  }
#undef MQ_STEP
  return hipGetLastError();
}
}  // namespace

hipError_t launch_attention_step(const uint16_t* qkv, const int64_t* pos,
                                 const int32_t* page_table, int64_t pages_per_seq,
                                 int64_t page_size, int64_t num_pages, const float* cos_t,
                                 const float* sin_t, const uint16_t* q_norm,
                                 const uint16_t* k_norm, float eps, uint16_t* k_pages,
                                 uint16_t* v_pages, int64_t B, int nh, int nkv, int d,
                                 float scale, float* workspace, uint16_t* out,
                                 hipStream_t stream) {
  if (B == 0) return hipSuccess;
  const int64_t capacity = pages_per_seq * page_size;
  const int chunk = attn_chunk(B, nkv, nh / nkv, d, capacity);
  const int splits = (int)((capacity + chunk - 1) / chunk);
  if (d == 64)
    return launch_step_d<64>(qkv, pos, page_table, (int)pages_per_seq, (int)page_size,
                             (int)num_pages, cos_t, sin_t, q_norm, k_norm, eps, k_pages, v_pages,
                             B, nh, nkv, scale, workspace, out, chunk, splits, stream);
  if (d == 128)
    return launch_step_d<128>(qkv, pos, page_table, (int)pages_per_seq, (int)page_size,
                              (int)num_pages, cos_t, sin_t, q_norm, k_norm, eps, k_pages,
                              v_pages, B, nh, nkv, scale, workspace, out, chunk, splits, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_argmax_rows(const uint16_t* x, int64_t rows, int64_t cols, int64_t* out,
                              hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)rows), dim3(kArgmaxThreads), 0, stream, x,
                     cols, out);
  return hipGetLastError();
}

hipError_t launch_silu_mul(const uint16_t* gu, uint16_t* out, int64_t rows, int64_t inter,
                           hipStream_t stream) {
  const int64_t units = rows * (inter / 8);
  if (units == 0) return hipSuccess;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((units + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, gu, out, rows, (int)inter);
  return hipGetLastError();
}

}  // namespace mq
