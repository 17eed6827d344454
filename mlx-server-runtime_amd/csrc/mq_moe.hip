// Mixture-of-experts routing around mx.gather_qmm, as the reference's MoE
// block runs it (python/mlx_worker/native_mlx/models/lfm2.py:348-375 and
// SwitchGLU, lfm2.py:193-218, 613-622):
//
//  * moe_route_kernel    gates = softmax(float32(router logits)) (+ expert
//                        bias), the top-k experts per token (argpartition:
//                        here in descending gate order, ties to the lower
//                        expert id), their gates, optionally renormalised to
//                        sum 1 (+1e-20), rounded to the activation dtype;
//  * moe_sort_kernel     the flat (token, slot) pairs ordered by expert
//                        (_gather_sort: argsort of the flat ids), stable, as
//                        one counting sort: sorted ids, the order, its
//                        inverse, and the x row of every sorted pair, which
//                        gather_qmm takes as lhs indices (so the sorted copy
//                        of x is never materialised);
//  * moe_combine_kernel  _scatter_unsort plus the weighting of lfm2.py:375:
//                        out[t] = sum_j bf16(y[inverse[t*k + j]] * score[t, j]),
//                        float32 sum, one rounding;
//  * moe_route_sort_kernel  both of the first two in one block, for a decode
//                        step's few tokens;
//  * moe_combine_norm_kernel  the combine, the residual add and the next
//                        RMSNorm in one kernel per token.
#include <algorithm>

#include "mq_common.h"
#include "mq_internal.h"

namespace mq {
namespace {

// ---------------------------------------------------------------- router
// One wave per token; E <= kMaxExperts (E / 64 values per lane).
constexpr int kMaxExperts = 512;
constexpr int kRouteWaves = 4;

constexpr int kMaxTopK = 64;  // one output lane per pick

// A routing wave's LDS: the token's gate keys, then its picks in rank order.
struct RouteScratch {
  uint64_t key[kMaxExperts];
  float pick_gate[kMaxTopK];
  int pick_id[kMaxTopK];
};

// A 64-bit key ordered as the routing order: larger gate first, then the
// smaller expert id.  The high word is the gate's bits made monotonic as
// unsigned (negative floats flipped, the sign bit set on the rest; -0 taken
// as +0, which float comparison treats as equal), the low word ~id.
__device__ __forceinline__ uint64_t route_key(float gate, int id) {
  const uint32_t u = __float_as_uint(gate + 0.f);
  const uint32_t m = (u >> 31) ? ~u : (u | 0x80000000u);
  return (uint64_t)m << 32 | (uint32_t)~(uint32_t)id;
}

// The gate whose route_key has high word m (route_key's map inverted; -0 comes
// back as +0, which no gate is: a softmax term plus a bias rounds -0 to +0).
__device__ __forceinline__ float key_gate(uint32_t m) {
  return __uint_as_float((m >> 31) ? (m & 0x7fffffffu) : ~m);
}

// A 64-bit value moved by DPP, as two 32-bit moves; lanes the pattern leaves
// out read 0, below every key.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, ROW_MASK, 0xf, true);
  const uint32_t hi =
      (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, ROW_MASK, 0xf, true);
  return (uint64_t)hi << 32 | lo;
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// The largest key of the wave, the same in every lane: DPP within rows of 16,
// the row broadcasts into lane 63, then read from it.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t v) {
  v = max_u64(v, dpp_u64<0xb1>(v));        // quad_perm [1,0,3,2]
  v = max_u64(v, dpp_u64<0x4e>(v));        // quad_perm [2,3,0,1]
  v = max_u64(v, dpp_u64<0x141>(v));       // row_half_mirror
  v = max_u64(v, dpp_u64<0x140>(v));       // row_mirror
  v = max_u64(v, dpp_u64<0x142, 0xa>(v));  // row_bcast:15 into rows 1, 3
  v = max_u64(v, dpp_u64<0x143, 0xc>(v));  // row_bcast:31 into rows 2, 3
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
  return (uint64_t)hi << 32 | lo;
}

// Up to this many picks, top-k takes k rounds of the wave arg-max; beyond,
// each expert's rank is counted against every key (one pass over the LDS).
constexpr int kArgmaxTopK = 16;

// Token t's top-k by one whole wave: the arg-max order taken k times
// (descending gates, ties to the lower expert id: the largest route_key
// first).  Up to kArgmaxTopK picks, k rounds of a wave maximum over the keys,
// the winning key removed after each; beyond, the picks are the experts of
// rank < k, rank = the number of larger keys.  PER = experts per lane
// (E <= 64 * PER).
template <int PER>
__device__ __forceinline__ void route_token(const uint16_t* __restrict__ logits,
                                            const float* __restrict__ expert_bias, int64_t t,
                                            int E, int k, int normalize, int32_t* indices,
                                            uint16_t* __restrict__ scores, RouteScratch& rs,
                                            int* flat) {
  static_assert(64 * PER <= kMaxExperts, "the LDS holds kMaxExperts gates");
  const int lane = threadIdx.x & 63;
  const uint16_t* row = logits + t * E;
  float v[PER];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? bf16_bits_to_f32(row[e]) : -INFINITY;
    mx = fmaxf(mx, v[j]);
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    v[j] = lane + 64 * j < E ? __expf(v[j] - mx) : 0.f;
    sum += v[j];
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) sum += __shfl_xor(sum, off, 64);
  const float inv = 1.f / sum;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? v[j] * inv + (expert_bias ? expert_bias[e] : 0.f) : -INFINITY;
  }
  uint64_t key[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j)
    key[j] = lane + 64 * j < E ? route_key(v[j], lane + 64 * j) : 0ull;  // 0: below all
  if (k <= kArgmaxTopK) {
    // round r's winner goes to lane r; the total adds the picks in rank order
    float total = 0.f, mine = 0.f;
    int mine_id = 0;
    for (int r = 0; r < k; ++r) {
      uint64_t best = key[0];
#pragma unroll
      for (int j = 1; j < PER; ++j) best = max_u64(best, key[j]);
      const uint64_t m = wave_max_key(best);
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (key[j] == m) key[j] = 0ull;  // keys are distinct (the id is in them)
      const float g = key_gate((uint32_t)(m >> 32));
      total += g;
      if (lane == r) {
        mine = g;
        mine_id = (int)~(uint32_t)m;
      }
    }
    if (lane < k) {
      const float sc = normalize ? mine / (total + 1e-20f) : mine;
      indices[t * k + lane] = mine_id;
      if (flat) flat[t * k + lane] = mine_id;
      scores[t * k + lane] = (uint16_t)f32_to_bf16_bits(sc);
    }
    return;
  }
  // ranks against every gate of the token, staged in the wave's LDS as keys
  const int EP = (E + 1) & ~1;
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if (lane + 64 * j < EP) rs.key[lane + 64 * j] = key[j];
  if (lane < kMaxTopK) {
    rs.pick_gate[lane] = -INFINITY;
    rs.pick_id[lane] = 0x7fffffff;
  }
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's stores are visible
  int rank[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) rank[j] = 0;
  for (int e0 = 0; e0 < EP; e0 += 2) {
    const uint64_t w0 = rs.key[e0], w1 = rs.key[e0 + 1];
#pragma unroll
    for (int j = 0; j < PER; ++j) rank[j] += (int)(w0 > key[j]) + (int)(w1 > key[j]);
  }
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if (lane + 64 * j < E && rank[j] < k) {
      rs.pick_gate[rank[j]] = v[j];
      rs.pick_id[rank[j]] = lane + 64 * j;
    }
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if (lane < k) {
    float total = 0.f;  // in rank order, as k arg-max rounds add them
    for (int r = 0; r < k; ++r) total += rs.pick_gate[r];
    float sc = rs.pick_gate[lane];
    if (normalize) sc = sc / (total + 1e-20f);
    indices[t * k + lane] = rs.pick_id[lane];
    if (flat) flat[t * k + lane] = rs.pick_id[lane];
    scores[t * k + lane] = (uint16_t)f32_to_bf16_bits(sc);
  }
  __asm__ volatile("" ::: "memory");  // the reads above stay ahead of the next token's stores
}

__device__ __forceinline__ void route_token_any(const uint16_t* __restrict__ logits,
                                                const float* __restrict__ expert_bias, int64_t t,
                                                int E, int k, int normalize, int32_t* indices,
                                                uint16_t* __restrict__ scores, RouteScratch& rs,
                                                int* flat = nullptr) {
  if (E <= 64)
    route_token<1>(logits, expert_bias, t, E, k, normalize, indices, scores, rs, flat);
  else if (E <= 128)
    route_token<2>(logits, expert_bias, t, E, k, normalize, indices, scores, rs, flat);
  else if (E <= 256)
    route_token<4>(logits, expert_bias, t, E, k, normalize, indices, scores, rs, flat);
  else
    route_token<8>(logits, expert_bias, t, E, k, normalize, indices, scores, rs, flat);
}

__global__ __launch_bounds__(64 * kRouteWaves) void moe_route_kernel(
    const uint16_t* __restrict__ logits, const float* __restrict__ expert_bias, int64_t T, int E,
    int k, int normalize, int32_t* __restrict__ indices, uint16_t* __restrict__ scores) {
  __shared__ RouteScratch rs[kRouteWaves];
  const int64_t t = (int64_t)blockIdx.x * kRouteWaves + (threadIdx.x >> 6);
  if (t >= T) return;  // whole waves
  route_token_any(logits, expert_bias, t, E, k, normalize, indices, scores, rs[threadIdx.x >> 6]);
}

// ---------------------------------------------------------------- sort
// Blocks of kSortThreads, each placing one range of the entries.  An entry's
// place is its expert's offset, plus the entries of that expert before the
// block's range, in earlier chunks of the range, in earlier waves of its
// chunk and in earlier lanes of its wave (a match mask built from one ballot
// per id bit).  Every block counts all n ids itself -- the totals give the
// experts' offsets, the ids before its range its start within each expert --
// so the sort needs no memory beyond its outputs and one launch.  Ids outside
// [0, E) go to a last bucket E, kept as they are (gather_qmm gives such rows
// zeros).
constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / 64;
constexpr int kMaxBuckets = kMaxExperts + 1;
constexpr int kSortBlocks = 64;  // at most; a block's range is whole chunks

// Entries [lo, hi) of the sort of ids[0, n), by one block of kSortThreads;
// the block with lo = 0 writes the segment offsets.
__device__ __forceinline__ void sort_block(const int32_t* ids, int n, int lo, int hi, int k,
                                           int E, int32_t* __restrict__ sorted_ids,
                                           int32_t* __restrict__ order,
                                           int32_t* __restrict__ inverse,
                                           int32_t* __restrict__ rows,
                                           int32_t* __restrict__ expert_offsets) {
  __shared__ int offset[kMaxBuckets];
  __shared__ int prior[kMaxBuckets];  // entries of each expert before lo
  __shared__ int wave_count[kSortWaves][kMaxBuckets];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int buckets = E + 1;
  int bits = 0;
  while ((1 << bits) < buckets) ++bits;
  for (int e = tid; e < buckets; e += kSortThreads) offset[e] = prior[e] = 0;
  __syncthreads();
  for (int i = tid; i < n; i += kSortThreads) {
    const int id = ids[i];
    const int b = (id >= 0 && id < E) ? id : E;
    atomicAdd(&offset[b], 1);
    if (i < lo) atomicAdd(&prior[b], 1);
  }
  __syncthreads();
  if (tid < 64) {  // exclusive scan over at most 513 buckets: one wave, PB per lane
    constexpr int PB = (kMaxBuckets + 63) / 64;
    int cnt[PB], local = 0;
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      const int e = tid * PB + q;
      cnt[q] = e < buckets ? offset[e] : 0;
      local += cnt[q];
    }
    int incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(incl, off, 64);
      if (tid >= off) incl += o;
    }
    int run = incl - local;
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      const int e = tid * PB + q;
      if (e < buckets) offset[e] = run;
      run += cnt[q];
    }
  }
  __syncthreads();
  // segment starts: expert e's pairs are sorted positions offset[e] ..
  // offset[e + 1] - 1; offset[E] counts the pairs with a valid id.  Then the
  // block's own start within each expert (the chunk loop's first barrier
  // orders these updates before any read of another bucket).
  for (int e = tid; e < buckets; e += kSortThreads) {
    if (expert_offsets && lo == 0) expert_offsets[e] = offset[e];
    offset[e] += prior[e];
  }
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
  for (int c0 = lo; c0 < hi; c0 += kSortThreads) {
    for (int e = lane; e < buckets; e += 64) wave_count[wave][e] = 0;
    const int i = c0 + tid;
    const bool valid = i < hi;
    int bucket = E;
    int id = 0;
    if (valid) {
      id = ids[i];
      bucket = (id >= 0 && id < E) ? id : E;
    }
    uint64_t match = __ballot(valid);
    for (int bit = 0; bit < bits; ++bit) {
      const uint64_t ones = __ballot(valid && ((bucket >> bit) & 1));
      match &= ((bucket >> bit) & 1) ? ones : ~ones;
    }
    const int rank = __popcll(match & below);
    __syncthreads();  // wave_count cleared by every wave
    if (valid && rank == __popcll(match) - 1) wave_count[wave][bucket] = rank + 1;
    __syncthreads();
    int before = 0;
    if (valid)
      for (int w = 0; w < wave; ++w) before += wave_count[w][bucket];
    if (valid) {
      const int p = offset[bucket] + before + rank;
      sorted_ids[p] = id;
      order[p] = i;
      inverse[i] = p;
      if (rows) rows[p] = i / k;
    }
    __syncthreads();  // every read of offset / wave_count for this chunk done
    for (int e = tid; e < buckets; e += kSortThreads) {
      int add = 0;
      for (int w = 0; w < kSortWaves; ++w) add += wave_count[w][e];
      offset[e] += add;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void zero_i32_kernel(int32_t* __restrict__ p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Block b places entries [b * per, min(n, (b + 1) * per)), per a multiple of
// kSortThreads.
__global__ __launch_bounds__(kSortThreads) void moe_sort_kernel(
    const int32_t* __restrict__ ids, int n, int per, int k, int E,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ order,
    int32_t* __restrict__ inverse, int32_t* __restrict__ rows,
    int32_t* __restrict__ expert_offsets) {
  const int lo = blockIdx.x * per;
  sort_block(ids, n, lo, min(n, lo + per), k, E, sorted_ids, order, inverse, rows,
             expert_offsets);
}

// Route (one wave per token) and then sort, in one block: a decode step's
// few tokens need no more, and a launch in between costs more than both.
// The block's index stores are visible to its own loads after the barrier.
constexpr int kRouteSortMaxTokens = 64;

__global__ __launch_bounds__(kSortThreads) void moe_route_sort_kernel(
    const uint16_t* __restrict__ logits, const float* __restrict__ expert_bias, int T, int E,
    int k, int normalize, int32_t* indices, uint16_t* __restrict__ scores,
    int32_t* __restrict__ sorted_ids, int32_t* __restrict__ order,
    int32_t* __restrict__ inverse, int32_t* __restrict__ rows,
    int32_t* __restrict__ expert_offsets) {
  __shared__ RouteScratch rs[kSortWaves];
  __shared__ int flat[64];  // the picks, for the one-wave sort
  __shared__ int bucket_at[64];  // the sorted pairs' buckets
  __shared__ __align__(16) int sort_key[64];  // the pairs' keys, for their ranks
  const int n = T * k;
  for (int t = threadIdx.x >> 6; t < T; t += kSortWaves)
    route_token_any(logits, expert_bias, t, E, k, normalize, indices, scores,
                    rs[threadIdx.x >> 6], n <= 64 ? flat : nullptr);
  __syncthreads();
  if (n > 64) {
    sort_block(indices, n, 0, n, k, E, sorted_ids, order, inverse, rows, expert_offsets);
    return;
  }
  // At most 64 pairs: one wave places each at its rank among the keys
  // (bucket, index) -- the counting sort's stable order, with no histogram,
  // scan or further barrier.  The keys go through the wave's LDS and come
  // back as broadcast 16-byte reads (a readlane per key cost ~60 cycles each,
  // 1.9 us for 64).
  if (threadIdx.x < 64) {
    const int i = threadIdx.x;
    int id = 0, key = 0x7fffffff;
    if (i < n) {
      id = flat[i];
      key = ((id >= 0 && id < E) ? id : E) << 6 | i;
    }
    sort_key[i] = key;  // lanes past n: above every pair's key
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's stores are visible
    int pos = 0;
    for (int j = 0; j < n; j += 4) {  // keys past n, in the last four, are above all
      const int4 q = *reinterpret_cast<const int4*>(sort_key + j);
      pos += (int)(q.x < key) + (int)(q.y < key) + (int)(q.z < key) + (int)(q.w < key);
    }
    if (i < n) {
      sorted_ids[pos] = id;
      order[pos] = i;
      inverse[i] = pos;
      if (rows) rows[pos] = i / k;
    }
    if (expert_offsets) {
      // segment starts: expert e's pairs begin at the first sorted position
      // whose bucket is >= e, so the pair at sorted position p starts the
      // experts in (bucket[p - 1], bucket[p]], and the experts past the last
      // pair's bucket start at n
      if (i < n) bucket_at[pos] = key >> 6;
      __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's stores are visible
      if (i < n) {
        const int b = bucket_at[i], prev = i > 0 ? bucket_at[i - 1] : -1;
        for (int e = prev + 1; e <= b; ++e) expert_offsets[e] = i;
      }
      const int last = n > 0 ? bucket_at[n - 1] : -1;
      for (int e = last + 1 + i; e <= E; e += 64) expert_offsets[e] = n;
    }
  }
}

// ---------------------------------------------------------------- combine
// acc[0..8) += bf16(y[row_j][8u .. 8u+8) * score_j) over token t's k slots j
// in slot order, row_j = inverse[t*k + j] (or t*k + j), clamped to y's rows.
// The slots go 8 at a time: their rows and scores are loaded, then their y
// units, before any is added, so a group costs two memory round trips, not
// two per slot (slots past k reload slot k - 1 and are not added).
__device__ __forceinline__ void combine_unit(const uint16_t* __restrict__ y,
                                             const int32_t* __restrict__ inverse,
                                             const uint16_t* __restrict__ scores, int64_t t, int k,
                                             int H, int64_t y_rows, int u, float* acc) {
  for (int j0 = 0; j0 < k; j0 += 8) {
    int64_t r[8];
    float sc[8];
    u32x4_t v[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int j = min(j0 + jj, k - 1);
      int64_t rr = t * k + j;
      if (inverse) rr = inverse[rr];
      r[jj] = rr < 0 ? 0 : (rr >= y_rows ? y_rows - 1 : rr);
      sc[jj] = bf16_bits_to_f32(scores[t * k + j]);
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) v[jj] = reinterpret_cast<const u32x4_t*>(y + r[jj] * H)[u];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      if (j0 + jj < k) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] += bf16_bits_to_f32(f32_to_bf16_bits(lo_bf16(v[jj][q]) * sc[jj]));
          acc[2 * q + 1] += bf16_bits_to_f32(f32_to_bf16_bits(hi_bf16(v[jj][q]) * sc[jj]));
        }
      }
    }
  }
}

// Grid (T, ceil(H / (8 * 256))), 256 threads, 8 elements per thread.
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const uint16_t* __restrict__ y, const int32_t* __restrict__ inverse,
    const uint16_t* __restrict__ scores, uint16_t* __restrict__ out, int64_t T, int k, int H,
    int64_t y_rows) {
  const int64_t t = blockIdx.x;
  const int u = blockIdx.y * 256 + threadIdx.x;  // 8-element unit of the row
  if (u >= H / 8) return;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  combine_unit(y, inverse, scores, t, k, H, y_rows, u, acc);
  u32x4_t o;
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
  reinterpret_cast<u32x4_t*>(out + t * H)[u] = o;
}

// moe_combine_kernel followed by the residual add and the RMSNorm that the
// next layer applies, per token: h = bf16(out + residual) -> residual_out,
// normed = bf16(h * rsqrt(mean(h^2) + eps) * w).  The element mapping and the
// reduction order are the RMSNorm kernel's (256 threads, 8 elements per
// thread and pass, four passes), so the outputs equal those of the combine
// then the norm bit for bit.  Grid T; H / 8 <= 1024.
constexpr int kNormThreads = 256;
constexpr int kNormUnits = 4;

__global__ __launch_bounds__(kNormThreads) void moe_combine_norm_kernel(
    const uint16_t* __restrict__ y, const int32_t* __restrict__ inverse,
    const uint16_t* __restrict__ scores, const uint16_t* __restrict__ residual,
    uint16_t* __restrict__ residual_out, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ normed, int k, int H, int64_t y_rows, float eps) {
  __shared__ float red[kNormThreads / 64];
  const int64_t t = blockIdx.x;
  const int units = H / 8;
  u32x4_t hv[kNormUnits], rvs[kNormUnits], wvs[kNormUnits];
  // the residual and the norm weights first: their loads overlap the expert
  // rows' instead of following them (and the reduction's barrier)
#pragma unroll
  for (int pass = 0; pass < kNormUnits; ++pass) {
    const int u = threadIdx.x + pass * kNormThreads;
    if (u < units) {
      rvs[pass] = reinterpret_cast<const u32x4_t*>(residual + t * H)[u];
      wvs[pass] = reinterpret_cast<const u32x4_t*>(w)[u];
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int pass = 0; pass < kNormUnits; ++pass) {
    const int u = threadIdx.x + pass * kNormThreads;
    if (u < units) {
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      combine_unit(y, inverse, scores, t, k, H, y_rows, u, acc);
      const u32x4_t rv = rvs[pass];
      u32x4_t h;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t c = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
        h[q] = pack_bf16x2(lo_bf16(c) + lo_bf16(rv[q]), hi_bf16(c) + hi_bf16(rv[q]));
      }
      reinterpret_cast<u32x4_t*>(residual_out + t * H)[u] = h;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float a = lo_bf16(h[q]), b = hi_bf16(h[q]);
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
      hv[pass] = h;
    }
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) ss += __shfl_xor(ss, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) ss += red[i];
  const float inv = rsqrtf(ss / (float)H + eps);
#pragma unroll
  for (int pass = 0; pass < kNormUnits; ++pass) {
    const int u = threadIdx.x + pass * kNormThreads;
    if (u < units) {
      const u32x4_t wv = wvs[pass];
      u32x4_t o;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = pack_bf16x2(lo_bf16(hv[pass][q]) * inv * lo_bf16(wv[q]),
                           hi_bf16(hv[pass][q]) * inv * hi_bf16(wv[q]));
      reinterpret_cast<u32x4_t*>(normed + t * H)[u] = o;
    }
  }
}

}  // namespace

hipError_t launch_moe_route_sort(const uint16_t* logits, const float* expert_bias, int64_t T,
                                 int E, int k, bool normalize, int32_t* indices, uint16_t* scores,
                                 int32_t* sorted_ids, int32_t* order, int32_t* inverse,
                                 int32_t* rows, int32_t* expert_offsets, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  if (T > kRouteSortMaxTokens) {
    const hipError_t e =
        launch_moe_route(logits, expert_bias, T, E, k, normalize, indices, scores, stream);
    if (e != hipSuccess) return e;
    return launch_moe_sort(indices, T * k, k, E, sorted_ids, order, inverse, rows,
                           expert_offsets, stream);
  }
  hipLaunchKernelGGL(moe_route_sort_kernel, dim3(1), dim3(kSortThreads), 0, stream, logits,
                     expert_bias, (int)T, E, k, normalize ? 1 : 0, indices, scores, sorted_ids,
                     order, inverse, rows, expert_offsets);
  return hipGetLastError();
}

bool moe_combine_norm_supported(int64_t H) {
  return H > 0 && H % 8 == 0 && H / 8 <= (int64_t)kNormThreads * kNormUnits;
}

hipError_t launch_moe_combine_norm(const uint16_t* y, const int32_t* inverse,
                                   const uint16_t* scores, const uint16_t* residual,
                                   uint16_t* residual_out, const uint16_t* w, uint16_t* normed,
                                   int64_t T, int k, int64_t H, float eps, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  hipLaunchKernelGGL(moe_combine_norm_kernel, dim3((unsigned)T), dim3(kNormThreads), 0, stream,
                     y, inverse, scores, residual, residual_out, w, normed, k, (int)H, T * k, eps);
  return hipGetLastError();
}

bool moe_route_supported(int E, int k) {
  return E >= 1 && E <= kMaxExperts && k >= 1 && k <= 64 && k <= E;
}

hipError_t launch_moe_route(const uint16_t* logits, const float* expert_bias, int64_t T, int E,
                            int k, bool normalize, int32_t* indices, uint16_t* scores,
                            hipStream_t stream) {
  if (T == 0) return hipSuccess;
  const unsigned blocks = (unsigned)((T + kRouteWaves - 1) / kRouteWaves);
  hipLaunchKernelGGL(moe_route_kernel, dim3(blocks), dim3(64 * kRouteWaves), 0, stream, logits,
                     expert_bias, T, E, k, normalize ? 1 : 0, indices, scores);
  return hipGetLastError();
}

bool moe_sort_supported(int64_t n, int E) { return E >= 1 && E <= kMaxExperts && n < (1 << 30); }

hipError_t launch_moe_sort(const int32_t* ids, int64_t n, int k, int E, int32_t* sorted_ids,
                           int32_t* order, int32_t* inverse, int32_t* rows,
                           int32_t* expert_offsets, hipStream_t stream) {
  if (n == 0) {
    // no pairs: every segment is empty (a kernel, not a memset node, so that
    // the call can be captured in a graph)
    if (!expert_offsets) return hipSuccess;
    hipLaunchKernelGGL(zero_i32_kernel, dim3((E + 256) / 256), dim3(256), 0, stream,
                       expert_offsets, E + 1);
    return hipGetLastError();
  }
  // whole chunks per block, at most kSortBlocks blocks, none empty
  const int64_t chunks = (n + kSortThreads - 1) / kSortThreads;
  const int64_t per_chunks = (chunks + kSortBlocks - 1) / kSortBlocks;
  const unsigned blocks = (unsigned)((chunks + per_chunks - 1) / per_chunks);
  hipLaunchKernelGGL(moe_sort_kernel, dim3(blocks), dim3(kSortThreads), 0, stream, ids, (int)n,
                     (int)(per_chunks * kSortThreads), k, E, sorted_ids, order, inverse, rows,
                     expert_offsets);
  return hipGetLastError();
}

hipError_t launch_moe_combine(const uint16_t* y, const int32_t* inverse, const uint16_t* scores,
                              uint16_t* out, int64_t T, int k, int64_t H, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  const dim3 grid((unsigned)T, (unsigned)((H / 8 + 255) / 256));
  hipLaunchKernelGGL(moe_combine_kernel, grid, dim3(256), 0, stream, y, inverse, scores, out, T,
                     k, (int)H, T * k);
  return hipGetLastError();
}

}  // namespace mq
