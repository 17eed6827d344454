// Paged causal attention for prefill chunks: several new tokens per sequence,
// each attending to its sequence's cached positions up to its own.  The
// reference runs mx.fast.scaled_dot_product_attention with an additive mask
// over the gathered pages for chunks of up to 256 tokens
// (python/mlx_worker/native_mlx/attention.py:206-298, scheduler.py:565-567).
//
// Grid (ceil(T / 64QW), query heads, batch), 256 threads: a block takes 64QW
// queries of one head, wave w QW tiles of 16 (queries j0 + 16QWw ..), and
// walks the keys 0 .. (its last query's position) in blocks of 64 staged in
// LDS, block kb + 1 loading while block kb is computed:
//  * K rows by buffer_load ... lds into one of two buffers (256 bytes a key,
//    16-byte chunks XOR-ed with a function of the key so a fragment read
//    spreads over the banks); V pieces into registers, written transposed
//    (d-major, 64 keys a row) at the top of their block, so a P.V B fragment
//    is one 16-byte read.  The rows' page offsets are computed once per key
//    (one wave, a block ahead) and read from LDS.
//  * S^T = K Q^T by v_mfma_f32_16x16x32_bf16: A = 16 keys of the block, B =
//    a tile's 16 queries (lane l: query l % 16); each K or V fragment read
//    feeds the wave's QW tiles.  Within each 32-key step, tile 2s + u's row
//    i is key 8(i / 4) + 4u + i % 4, so that lane l's scores of tiles 2s and
//    2s + 1 (rows 4(l / 16) + r) are the 8 keys 8(l / 16) .. +7 of the step:
//    P's A operand for P.V as it sits.
//  * Online softmax per query in log2 units (exp2 of fma(score, scale, -m)),
//    keys past the query's position masked; the running max m rises only
//    past 8 (log2) of headroom, so P = exp2(x - m) <= 2^8 and most blocks
//    skip the output rescale (a per-wave LDS exchange); P rounded to
//    bfloat16 for P.V (v_mfma 16x16x32, B = V^T rows).
// Rows of a ragged batch: query j of row b sits at position starts[b] +
// min(j, lens[b] - 1) (padding queries repeat the row's last one).
#include <algorithm>

#include "mq_common.h"
#include "mq_internal.h"

namespace mq {
namespace {

constexpr int kThreads = 256;
constexpr int kKB = 64;                  // keys per LDS block
constexpr int kD = 128;                  // head dim
constexpr int kVStride = kKB * 2 + 16;   // bytes per V^T row (one d), padded
constexpr float kNoScore = -1e30f;       // running max before the first key
constexpr float kLazy = 8.f;             // log2 headroom of the running max

typedef __attribute__((address_space(3))) void lds_t;

struct PrefillShared {
  __align__(16) char k[2][kKB * kD * 2];  // K rows of two key blocks, 256 bytes a key
  __align__(16) char vt[kD * kVStride];   // V^T of the current block: row d holds keys 0..63
  float xch[kThreads / 64][2][16];        // per wave and query tile: a value per query
  uint32_t row[2][kKB];                   // byte offsets of two key blocks' rows in the pages
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

// QW query tiles of 16 per wave (64 QW queries a block): each K and V
// fragment read from LDS feeds QW MFMAs.  Every query sees the same
// operations in the same order for either QW.
template <int QW>
__global__ __launch_bounds__(kThreads, QW == 1 ? 3 : 2) void prefill_attn_kernel(
    const uint16_t* __restrict__ q, const uint16_t* k_pages, const uint16_t* v_pages,
    const int32_t* __restrict__ page_table, int pages_per_seq, int page_size, int num_pages,
    const int64_t* __restrict__ starts, const int64_t* __restrict__ lens, int T, int nh, int nkv,
    float scale_log2, uint16_t* __restrict__ out) {
  constexpr int QT = 64 * QW;  // queries per block
  __shared__ PrefillShared sh;
  const int tid = threadIdx.x, l = tid & 63, c = l & 15, g = l >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = blockIdx.y, kvh = h / (nh / nkv);
  const int64_t b = blockIdx.z;
  const int j0 = blockIdx.x * QT;
  const int jw = j0 + 16 * QW * wave;  // the wave's first query
  const int64_t capacity = (int64_t)pages_per_seq * page_size;
  const int64_t start = clampi(starts[b], capacity);
  const int len = (int)std::min<int64_t>(std::max<int64_t>(lens[b], 1), T);
  auto pos_of = [&](int j) {  // position of query j (j < T)
    return (int)std::min<int64_t>(start + std::min(j, len - 1), capacity - 1);
  };
  // this lane's queries (column c of tile u's MFMAs), the wave's first and
  // last, and the block's last
  int pq[QW];
#pragma unroll
  for (int u = 0; u < QW; ++u) pq[u] = pos_of(std::min(jw + 16 * u + c, T - 1));
  const int pmax = pos_of(std::min(j0 + QT - 1, T - 1));
  const int wmin = pos_of(std::min(jw, T - 1));
  const int wmax = pos_of(std::min(jw + 16 * QW - 1, T - 1));
  const int nkb = pmax / kKB + 1;

  // Byte offset of position `key`'s row of KV head kvh in the pages (positions
  // past the table's last page read its last page; every offset lies below
  // 2^31, which the entry point checks).  The first wave computes a key
  // block's 64 offsets one block ahead, so the other loads index LDS.
  const int32_t* table = page_table + b * pages_per_seq;
  const uint32_t row_bytes = (uint32_t)nkv * kD * 2, head_bytes = (uint32_t)kvh * kD * 2;
  auto row_of = [&](int key) -> uint32_t {
    const int pg = std::min(key / page_size, pages_per_seq - 1);
    const uint32_t slot =
        (uint32_t)clampi(table[pg], num_pages) * (uint32_t)page_size + (uint32_t)(key % page_size);
    return slot * row_bytes + head_bytes;
  };
  const uint64_t page_bytes = (uint64_t)num_pages * page_size * row_bytes;
  const rsrc_t krs = make_rsrc(k_pages, page_bytes);
  const rsrc_t vrs = make_rsrc(v_pages, page_bytes);

  // this lane's query operands: dims 32s + 8g .. +7 of tile u's query c
  u32x4_t qa[QW][kD / 32];
#pragma unroll
  for (int u = 0; u < QW; ++u) {
    const int jq = std::min(jw + 16 * u + c, T - 1);
    const uint16_t* qr = q + (((int64_t)b * T + jq) * nh + h) * kD + 8 * g;
#pragma unroll
    for (int s = 0; s < kD / 32; ++s) qa[u][s] = *reinterpret_cast<const u32x4_t*>(qr + 32 * s);
  }

  // Staging of key block kb (keys 64kb ..): K rows by DMA into sh.k[kb & 1]
  // -- wave w's op i fills keys 4(4w + i) .. +3, lane l reading logical
  // chunk (l % 16) ^ swz(key) of key 4(4w + i) + l / 16 -- and this thread's
  // V pieces, dims 8(t / 16) .. +7 of keys 4(t % 16) .. +3, into registers.
  const int dc = tid >> 4, kq = tid & 15;
  auto stage = [&](int kb, u32x4_t (&v)[4]) {
    const uint32_t* rows = sh.row[kb & 1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int op = 4 * wave + i, r = 4 * op + g;
      const uint32_t off = rows[r] + 16u * (uint32_t)(c ^ swz(r));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_t*)(sh.k[kb & 1] + op * 1024), 16, off,
                                               0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = buf_load16(vrs, rows[4 * kq + k] + 16u * (uint32_t)dc);
  };

  f32x4_t o[QW][kD / 16];  // tile u, t: dims 16t + c, queries 4g + r of query tile u
#pragma unroll
  for (int u = 0; u < QW; ++u)
#pragma unroll
    for (int t = 0; t < kD / 16; ++t) o[u][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m[QW], lsum[QW];  // running max / sum of tile u's query c
#pragma unroll
  for (int u = 0; u < QW; ++u) m[u] = kNoScore, lsum[u] = 0.f;

  // Pipeline: block kb + 1's K rows and V pieces load while block kb is
  // computed; the row offsets run one block further ahead (the first wave's
  // table reads, in a register until the top of the next iteration).
  u32x4_t v[4];
  uint32_t ahead = 0;  // first wave: the row offset of key 64(kb + 2) + l
  if (wave == 0) {
    sh.row[0][l] = row_of(l);
    if (nkb > 1) ahead = row_of(kKB + l);
  }
  __syncthreads();
  stage(0, v);
  for (int kb = 0; kb < nkb; ++kb) {
    const int key0 = kb * kKB;
    // block kb's K rows and V pieces (and the offsets of block kb + 1) have
    // landed: every load in flight was issued before block kb - 1's compute
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (wave == 0 && kb + 1 < nkb) sh.row[(kb + 1) & 1][l] = ahead;
    __syncthreads();  // block kb - 1's tiles are read; block kb's K and offsets visible
    // V^T of block kb, in 8-byte row pieces; keys past the block's last query
    // position as zeros (a never-written slot may hold any bits, and P is 0
    // there, but 0 times a NaN is not)
    {
      if (key0 + kKB - 1 > pmax) {  // uniform: only the last block reaches past pmax
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (key0 + 4 * kq + k > pmax) v[k] = u32x4_t{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        const u32x2_t w = {__builtin_amdgcn_perm(v[1][e >> 1], v[0][e >> 1], sel),
                           __builtin_amdgcn_perm(v[3][e >> 1], v[2][e >> 1], sel)};
        *reinterpret_cast<u32x2_t*>(sh.vt + (8 * dc + e) * kVStride + kq * 8) = w;
      }
    }
    if (kb + 1 < nkb) {
      stage(kb + 1, v);
      if (wave == 0 && kb + 2 < nkb) ahead = row_of(key0 + 2 * kKB + l);
    }
    __syncthreads();  // V^T visible
    if (key0 > wmax) continue;  // uniform: every key of the block lies past the wave's queries

    // S^T for the 64 keys: tile t's rows are keys key_of(t, 4g + r)
    f32x4_t sc[QW][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = key_of(t, c);  // this lane's A row
      const char* kr = sh.k[kb & 1] + r * 256;
      f32x4_t d[QW];
#pragma unroll
      for (int u = 0; u < QW; ++u) d[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < kD / 32; ++s) {
        const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(kr + 16 * ((4 * s + g) ^ swz(r)));
#pragma unroll
        for (int u = 0; u < QW; ++u)
          d[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8_t, qa[u][s]),
                                                         d[u], 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < QW; ++u) sc[u][t] = d[u];
    }
    // keys past query c's position masked (none where the whole block lies
    // at or before the wave's first query); key_of(t, 4g + r) is 8g plus a
    // constant of (t, r).  A tile's running max m is raised only when one of
    // its 16 queries sees a score above m + kLazy (log2 units): P = exp2(x -
    // m) then stays below 2^kLazy, and most blocks skip the output rescale.
    // The decision is per 16-query tile, so each query's arithmetic is the
    // same for either QW.
    const bool full = key0 + kKB - 1 <= wmin;  // uniform
    float y[QW][4][4], mxs[QW];
    bool rescale[QW];
#pragma unroll
    for (int u = 0; u < QW; ++u) {
      float mx = -INFINITY;
      if (full) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            y[u][t][r] = sc[u][t][r];
            mx = fmaxf(mx, y[u][t][r]);
          }
      } else {
        const int lim = pq[u] - key0 - 8 * g;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            y[u][t][r] = key_of(t, r) <= lim ? sc[u][t][r] : -INFINITY;
            mx = fmaxf(mx, y[u][t][r]);
          }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      mxs[u] = mx * scale_log2;  // the scale is positive: the max of the scaled scores
      rescale[u] = __ballot(mxs[u] > m[u] + kLazy) != 0ull;  // uniform
    }
    float p[QW][4][4], f[QW];
#pragma unroll
    for (int u = 0; u < QW; ++u) {
      f[u] = 1.f;
      if (rescale[u]) {
        const float mn = fmaxf(m[u], mxs[u]);
        f[u] = __builtin_amdgcn_exp2f(m[u] - mn);  // argument <= 0
        m[u] = mn;
      }
      float ps = 0.f;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[u][t][r] = __builtin_amdgcn_exp2f(fmaf(y[u][t][r], scale_log2, -m[u]));
          ps += p[u][t][r];
        }
      ps += __shfl_xor(ps, 16, 64);
      ps += __shfl_xor(ps, 32, 64);
      lsum[u] = fmaf(lsum[u], f[u], ps);
    }
#pragma unroll
    for (int u = 0; u < QW; ++u) {
      if (!rescale[u]) continue;
      // the output rows are queries 4g + r: their factors through LDS
      if (g == 0) sh.xch[wave][u][c] = f[u];
      __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      const f32x4_t fr = *reinterpret_cast<const f32x4_t*>(&sh.xch[wave][u][4 * g]);
#pragma unroll
      for (int t = 0; t < kD / 16; ++t) o[u][t] *= fr;
      __asm__ volatile("" ::: "memory");  // the exchange's read stays ahead of its next write
    }
    // P.V: two 32-key steps; A = P of tiles 2s, 2s + 1 (keys 32s + 8g .. +7)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      bf16x8_t pb[QW];
#pragma unroll
      for (int u = 0; u < QW; ++u) {
        const u32x4_t pa = {pack_bf16x2(p[u][2 * s][0], p[u][2 * s][1]),
                            pack_bf16x2(p[u][2 * s][2], p[u][2 * s][3]),
                            pack_bf16x2(p[u][2 * s + 1][0], p[u][2 * s + 1][1]),
                            pack_bf16x2(p[u][2 * s + 1][2], p[u][2 * s + 1][3])};
        pb[u] = __builtin_bit_cast(bf16x8_t, pa);
      }
#pragma unroll
      for (int t = 0; t < kD / 16; ++t) {
        const bf16x8_t vb = *reinterpret_cast<const bf16x8_t*>(
            sh.vt + (16 * t + c) * kVStride + (32 * s + 8 * g) * 2);
#pragma unroll
        for (int u = 0; u < QW; ++u)
          o[u][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pb[u], vb, o[u][t], 0, 0, 0);
      }
    }
    __asm__ volatile("" ::: "memory");  // the exchange's read stays ahead of its next write
  }

  // normalise: the sums of queries 4g + r through LDS
  if (g == 0) {
#pragma unroll
    for (int u = 0; u < QW; ++u) sh.xch[wave][u][c] = lsum[u];
  }
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int u = 0; u < QW; ++u) {
    const f32x4_t ls = *reinterpret_cast<const f32x4_t*>(&sh.xch[wave][u][4 * g]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = jw + 16 * u + 4 * g + r;
      if (j >= T) continue;
      uint16_t* orow = out + (((int64_t)b * T + j) * nh + h) * kD;
      const float inv = 1.f / ls[r];
#pragma unroll
      for (int t = 0; t < kD / 16; ++t)
        orow[16 * t + c] = (uint16_t)f32_to_bf16_bits(o[u][t][r] * inv);
    }
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
  // 128-query blocks (two query tiles a wave, two blocks a CU) where they
  // still give two rounds of the 256 CUs, else 64-query blocks
  const int64_t tiles2 = (T + 127) / 128;
  if (tiles2 * nh * B >= 512) {
    hipLaunchKernelGGL(prefill_attn_kernel<2>, dim3((unsigned)tiles2, (unsigned)nh, (unsigned)B),
                       dim3(kThreads), 0, stream, q, k_pages, v_pages, page_table,
                       (int)pages_per_seq, (int)page_size, (int)num_pages, starts, lens, (int)T,
                       nh, nkv, scale_log2, out);
  } else {
    hipLaunchKernelGGL(prefill_attn_kernel<1>,
                       dim3((unsigned)((T + 63) / 64), (unsigned)nh, (unsigned)B), dim3(kThreads),
                       0, stream, q, k_pages, v_pages, page_table, (int)pages_per_seq,
                       (int)page_size, (int)num_pages, starts, lens, (int)T, nh, nkv, scale_log2,
                       out);
  }
  return hipGetLastError();
}

}  // namespace mq
