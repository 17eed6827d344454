// Paged causal attention for prefill chunks: several new tokens per sequence,
// each attending to its sequence's cached positions up to its own.  The
// reference runs mx.fast.scaled_dot_product_attention with an additive mask
// over the gathered pages for chunks of up to 256 tokens
// (python/mlx_worker/native_mlx/attention.py:206-298, scheduler.py:565-567).
//
// Grid (ceil(T / 64), query heads, batch), 256 threads: a block takes 64
// queries of one head, wave w the queries j0 + 16w .. +15, and walks the keys
// 0 .. (its last query's position) in blocks of 64 staged in LDS:
//  * K rows by buffer_load ... lds (256 bytes a key, 16-byte chunks XOR-ed
//    with a function of the key so a fragment read spreads over the banks);
//    V transposed (d-major, 64 keys a row) through registers, so a P.V B
//    fragment is one 16-byte read.
//  * S^T = K Q^T by v_mfma_f32_16x16x32_bf16: A = 16 keys of the block, B =
//    the wave's 16 queries (lane l: query l % 16).  Within each 32-key step,
//    tile 2s + u's row i is key 8(i / 4) + 4u + i % 4, so that lane l's
//    scores of tiles 2s and 2s + 1 (rows 4(l / 16) + r) are the 8 keys
//    8(l / 16) .. +7 of the step: P's A operand for P.V as it sits.
//  * Online softmax per query in log2 units (exp2), keys past the query's
//    position masked; P rounded to bfloat16 for P.V (v_mfma 16x16x32, B = V^T
//    rows), the output tiles rescaled through a per-wave LDS exchange.
// Rows of a ragged batch: query j of row b sits at position starts[b] +
// min(j, lens[b] - 1) (padding queries repeat the row's last one).
#include <algorithm>

#include "mq_common.h"
#include "mq_internal.h"

namespace mq {
namespace {

constexpr int kThreads = 256;
constexpr int kQT = 64;                  // queries per block, 16 per wave
constexpr int kKB = 64;                  // keys per LDS block
constexpr int kD = 128;                  // head dim
constexpr int kVStride = kKB * 2 + 16;   // bytes per V^T row (one d), padded
constexpr float kNoScore = -1e30f;       // running max before the first key

typedef __attribute__((address_space(3))) void lds_t;

struct PrefillShared {
  __align__(16) char k[kKB * kD * 2];       // K rows, 256 bytes a key (swizzled chunks)
  __align__(16) char vt[kD * kVStride];     // V^T: row d holds keys 0..63
  float xch[kThreads / 64][16];             // per wave: a value per query
};

// key (0..63 of the block) of MFMA row i of key tile t
__device__ __forceinline__ int key_of(int t, int i) {
  return 32 * (t >> 1) + 8 * (i >> 2) + 4 * (t & 1) + (i & 3);
}
// 16-byte chunk c of key row r sits at chunk c ^ swz(r): distinct over the 16
// keys one fragment read touches (key_of(t, 0..15) for any t)
__device__ __forceinline__ int swz(int r) { return ((r >> 1) & 12) | (r & 3); }

__device__ __forceinline__ int64_t clampi(int64_t v, int64_t n) {
  return v < 0 ? 0 : (v >= n ? n - 1 : v);
}

__global__ __launch_bounds__(kThreads) void prefill_attn_kernel(
    const uint16_t* __restrict__ q, const uint16_t* k_pages, const uint16_t* __restrict__ v_pages,
    const int32_t* __restrict__ page_table, int pages_per_seq, int page_size, int num_pages,
    const int64_t* __restrict__ starts, const int64_t* __restrict__ lens, int T, int nh, int nkv,
    float scale_log2, uint16_t* __restrict__ out) {
  __shared__ PrefillShared sh;
  const int tid = threadIdx.x, l = tid & 63, c = l & 15, g = l >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = blockIdx.y, kvh = h / (nh / nkv);
  const int64_t b = blockIdx.z;
  const int j0 = blockIdx.x * kQT;
  const int64_t capacity = (int64_t)pages_per_seq * page_size;
  const int64_t start = clampi(starts[b], capacity);
  const int len = (int)std::min<int64_t>(std::max<int64_t>(lens[b], 1), T);
  auto pos_of = [&](int j) {  // position of query j (j < T)
    return (int)std::min<int64_t>(start + std::min(j, len - 1), capacity - 1);
  };
  // this lane's query (column c of the wave's MFMAs) and the block's last
  const int jq = std::min(j0 + 16 * wave + c, T - 1);
  const int pq = pos_of(jq);
  const int pmax = pos_of(std::min(j0 + kQT - 1, T - 1));
  const int wmax = pos_of(std::min(j0 + 16 * wave + 15, T - 1));  // the wave's last
  const int nkb = pmax / kKB + 1;

  const int32_t* table = page_table + b * pages_per_seq;
  auto slot_of = [&](int key) -> int64_t {  // cache slot of position `key`
    const int pg = std::min(key / page_size, pages_per_seq - 1);
    return clampi(table[pg], num_pages) * page_size + key % page_size;
  };
  const int64_t row_elems = (int64_t)nkv * kD;
  const rsrc_t krs = make_rsrc(k_pages, (uint64_t)num_pages * page_size * row_elems * 2);

  // this lane's query operand: dims 32s + 8g .. +7 of query jq
  u32x4_t qa[kD / 32];
  {
    const uint16_t* qr = q + (((int64_t)b * T + jq) * nh + h) * kD + 8 * g;
#pragma unroll
    for (int s = 0; s < kD / 32; ++s) qa[s] = *reinterpret_cast<const u32x4_t*>(qr + 32 * s);
  }

  f32x4_t o[kD / 16];  // tile t: dims 16t + c, queries 4g + r of the wave
#pragma unroll
  for (int t = 0; t < kD / 16; ++t) o[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = kNoScore, lsum = 0.f;  // running max / sum of query c

  for (int kb = 0; kb < nkb; ++kb) {
    const int key0 = kb * kKB;
    __syncthreads();  // the previous block's tiles are read
    // K: wave w's op o fills keys 4o .. 4o + 3 (o = 4w .. 4w + 3); lane l
    // reads logical chunk (l % 16) ^ swz(key) of key 4o + l / 16
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int op = 4 * wave + i, r = 4 * op + g;
      const int64_t slot = slot_of(key0 + r);
      const uint32_t off =
          (uint32_t)((slot * row_elems + kvh * kD) * 2) + 16u * (uint32_t)(c ^ swz(r));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_t*)(sh.k + op * 1024), 16, off, 0, 0, 0);
    }
    // V^T: thread t takes d-chunk t / 16 (dims 8(t/16) .. +7) of keys
    // 4(t % 16) .. +3, transposed into 8-byte row pieces
    {
      const int dc = tid >> 4, kq = tid & 15;
      u32x4_t v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        v[k] = *reinterpret_cast<const u32x4_t*>(
            v_pages + slot_of(key0 + 4 * kq + k) * row_elems + kvh * kD + 8 * dc);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        const u32x2_t w = {__builtin_amdgcn_perm(v[1][e >> 1], v[0][e >> 1], sel),
                           __builtin_amdgcn_perm(v[3][e >> 1], v[2][e >> 1], sel)};
        *reinterpret_cast<u32x2_t*>(sh.vt + (8 * dc + e) * kVStride + kq * 8) = w;
      }
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (key0 > wmax) continue;  // uniform: every key of the block lies past the wave's queries

    // S^T for the 64 keys: tile t's rows are keys key_of(t, 4g + r)
    f32x4_t sc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = key_of(t, c);  // this lane's A row
      const char* kr = sh.k + r * 256;
      f32x4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < kD / 32; ++s) {
        const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(kr + 16 * ((4 * s + g) ^ swz(r)));
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8_t, qa[s]), d, 0,
                                                    0, 0);
      }
      sc[t] = d;
    }
    float x[4][4], mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kp = key0 + key_of(t, 4 * g + r);
        x[t][r] = kp <= pq ? sc[t][r] * scale_log2 : -INFINITY;
        mx = fmaxf(mx, x[t][r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m, mx);
    const float f = __builtin_amdgcn_exp2f(m - mn);  // argument <= 0
    float p[4][4], ps = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[t][r] = __builtin_amdgcn_exp2f(x[t][r] - mn);
        ps += p[t][r];
      }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    lsum = fmaf(lsum, f, ps);
    m = mn;
    // the output rows are queries 4g + r: their rescale through LDS
    if (g == 0) sh.xch[wave][c] = f;
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const f32x4_t fr = *reinterpret_cast<const f32x4_t*>(&sh.xch[wave][4 * g]);
#pragma unroll
    for (int t = 0; t < kD / 16; ++t) o[t] *= fr;
    // P.V: two 32-key steps; A = P of tiles 2s, 2s + 1 (keys 32s + 8g .. +7)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const u32x4_t pa = {pack_bf16x2(p[2 * s][0], p[2 * s][1]), pack_bf16x2(p[2 * s][2], p[2 * s][3]),
                          pack_bf16x2(p[2 * s + 1][0], p[2 * s + 1][1]),
                          pack_bf16x2(p[2 * s + 1][2], p[2 * s + 1][3])};
      const bf16x8_t pb = __builtin_bit_cast(bf16x8_t, pa);
#pragma unroll
      for (int t = 0; t < kD / 16; ++t) {
        const bf16x8_t vb = *reinterpret_cast<const bf16x8_t*>(
            sh.vt + (16 * t + c) * kVStride + (32 * s + 8 * g) * 2);
        o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pb, vb, o[t], 0, 0, 0);
      }
    }
    __asm__ volatile("" ::: "memory");  // the exchange's read stays ahead of its next write
  }

  // normalise: the sums of queries 4g + r through LDS
  if (g == 0) sh.xch[wave][c] = lsum;
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const f32x4_t ls = *reinterpret_cast<const f32x4_t*>(&sh.xch[wave][4 * g]);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int j = j0 + 16 * wave + 4 * g + r;
    if (j >= T) continue;
    uint16_t* orow = out + (((int64_t)b * T + j) * nh + h) * kD;
    const float inv = 1.f / ls[r];
#pragma unroll
    for (int t = 0; t < kD / 16; ++t) orow[16 * t + c] = (uint16_t)f32_to_bf16_bits(o[t][r] * inv);
  }
}

}  // namespace

bool prefill_attention_supported(int nh, int nkv, int d, int64_t num_pages, int64_t page_size) {
  return d == kD && nkv > 0 && nh % nkv == 0 &&
         num_pages * page_size * nkv * kD * 2 < ((int64_t)1 << 31);
}

hipError_t launch_prefill_attention(const uint16_t* q, const uint16_t* k_pages,
                                    const uint16_t* v_pages, const int32_t* page_table,
                                    int64_t pages_per_seq, int64_t page_size, int64_t num_pages,
                                    const int64_t* starts, const int64_t* lens, int64_t B,
                                    int64_t T, int nh, int nkv, float scale, uint16_t* out,
                                    hipStream_t stream) {
  if (B == 0 || T == 0) return hipSuccess;
  const float scale_log2 = scale * 1.4426950408889634f;  // exp(x) = exp2(x log2 e)
  hipLaunchKernelGGL(prefill_attn_kernel, dim3((unsigned)((T + kQT - 1) / kQT), (unsigned)nh,
                                                (unsigned)B),
                     dim3(kThreads), 0, stream, q, k_pages, v_pages, page_table,
                     (int)pages_per_seq, (int)page_size, (int)num_pages, starts, lens, (int)T, nh,
                     nkv, scale_log2, out);
  return hipGetLastError();
}

}  // namespace mq
