// Large-M quantized matmul, one wave per SIMD:
//   y[m, n] = sum_k x[m, k] * (s*q + b)[n, k]  (+ bias[n])
// mx.quantized_matmul(x, w, scales, biases, transpose=True) for prefill-sized
// M (python/mlx_worker/native_mlx/models/qwen2.py:76-78,115,134,227).
//
// MFMA-bound.  A 256-thread block owns a 256x256 output tile and walks K in
// steps of 64 (one quantization group).  Each of its 4 waves -- one per SIMD --
// computes the whole 256-row M tile for 64 columns: 8x2
// v_mfma_f32_32x32x16_bf16 per 16-wide k slice, 256 float32 accumulators per
// lane.  So every code of the block's 256 columns is dequantized exactly once
// per block (256 MACs per dequantized weight): the weights' VALU work per MFMA
// is half what a 2x4 wave grid (128 rows per wave, each column dequantized by
// two waves) spends.
//
// With one wave per SIMD nothing else hides a stall, so every load is issued
// well ahead of its use:
// * x never passes through registers on its way in: each step's 256x64 tile is
//   copied HBM -> LDS by buffer_load_dwordx4 ... lds (every lane writes 16
//   bytes at M0 + 16*lane), three steps ahead, into one of four 32 KiB stages.
//   Rows are 128 bytes with the 16-byte chunk index XOR-ed with (row >> 1) & 7,
//   so a fragment read of 32 rows hits 16 distinct 4-bank groups per half wave.
// * Weights never pass through LDS: for the MFMA B operand, lane l holds the
//   8 codes of column l % 32 for k-slice ks of its half (l / 32).  The k order
//   inside a group is permuted (A and B agree on it, so the product is
//   unchanged): half h takes k = 32h + 8ks .. 32h + 8ks + 7, which makes a
//   lane's codes for the whole step one contiguous 16-byte (4-bit) or 32-byte
//   (8-bit) load.  Codes are loaded two steps ahead (a ring of four) and
//   dequantized (fma(s, q, b), one bfloat16 rounding) one k-slice ahead of
//   their MFMAs.
// * Scales and biases for 8 groups of the block's 256 columns (16 bytes per
//   column and array) are DMA-ed into LDS four steps before they are needed.
// * Tiles run in groups of 4 row blocks x every column block, the row blocks
//   fastest: the 32 blocks an XCD runs at once cover 4 row blocks x 8 column
//   blocks, so they share x rows and codes in that XCD's L2.
// One barrier per step; the wait before it covers the DMAs of two steps ago
// and earlier (the next step's x tile), never those of this step or the
// previous one.
#include <algorithm>

#include "mq_common.h"
#include "mq_internal.h"

namespace mq {
namespace {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int kThreads = 256;
constexpr int kRowTiles = BM / 32;               // 8 MFMA row tiles per wave
constexpr int kXStage = BM * BK * 2;             // 32 KiB of x per step
constexpr int kXOps = kXStage / (kThreads * 16); // 8 DMA operations per lane per step
constexpr int kSbChunk = 8;                      // groups per scale/bias chunk
constexpr int kSbArray = BN * kSbChunk * 2;      // 4 KiB: one array, one chunk
constexpr int kSbBytes = 2 * kSbArray;           // scales + biases of a chunk
constexpr int kXStages = 4;                      // x three steps ahead
constexpr int kCodeRing = 4;                     // codes two steps ahead
constexpr int kGroupM = 4;                       // row blocks per tile group
constexpr int kSbBase = kXStages * kXStage;      // after the x stages
constexpr int kLds = kSbBase + 2 * kSbBytes;     // 144 KiB

typedef __attribute__((address_space(3))) void lds_t;

__device__ __forceinline__ void dma16(rsrc_t r, lds_t* dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, 0, 0, 0);
}

// End of a step: wait until at most N memory operations are outstanding, N
// being the number of DMA operations issued in this step, then sync the
// block.  vmcnt retires in issue order and the DMAs (LDS writes) never move
// across this asm, so every DMA of earlier steps -- in particular the next
// step's x tile -- has landed whatever the compiler did with the register
// loads (it may move those across the asm: they read __restrict__ memory).
template <int N>
__device__ __forceinline__ void step_barrier() {
  static_assert(N < 64, "vmcnt holds 6 bits");
  __asm__ volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// 8 codes (one MFMA B fragment) -> bf16(fma(s, q, b)), k order preserved.
template <int BITS>
__device__ __forceinline__ bf16x8_t dequant8(uint32_t w0, uint32_t w1, float s, float b) {
  u32x4_t o;
  if constexpr (BITS == 4) {
    // byte t of w0 = q[2t] | q[2t+1] << 4.  The empty asm keeps the two masks
    // as two instructions (otherwise each code becomes its own bit-field
    // extract).
    uint32_t lo = w0 & 0x0F0F0F0Fu, hi = (w0 >> 4) & 0x0F0F0F0Fu;
    __asm__("" : "+v"(lo), "+v"(hi));
    o[0] = pack_bf16x2(fmaf(s, ubyte_f32<0>(lo), b), fmaf(s, ubyte_f32<0>(hi), b));
    o[1] = pack_bf16x2(fmaf(s, ubyte_f32<1>(lo), b), fmaf(s, ubyte_f32<1>(hi), b));
    o[2] = pack_bf16x2(fmaf(s, ubyte_f32<2>(lo), b), fmaf(s, ubyte_f32<2>(hi), b));
    o[3] = pack_bf16x2(fmaf(s, ubyte_f32<3>(lo), b), fmaf(s, ubyte_f32<3>(hi), b));
    (void)w1;
  } else {
    o[0] = pack_bf16x2(fmaf(s, ubyte_f32<0>(w0), b), fmaf(s, ubyte_f32<1>(w0), b));
    o[1] = pack_bf16x2(fmaf(s, ubyte_f32<2>(w0), b), fmaf(s, ubyte_f32<3>(w0), b));
    o[2] = pack_bf16x2(fmaf(s, ubyte_f32<0>(w1), b), fmaf(s, ubyte_f32<1>(w1), b));
    o[3] = pack_bf16x2(fmaf(s, ubyte_f32<2>(w1), b), fmaf(s, ubyte_f32<3>(w1), b));
  }
  return __builtin_bit_cast(bf16x8_t, o);
}

struct GroupAffine {
  float s, b;
};

template <int BITS>
__global__ __launch_bounds__(kThreads, 1) void qmm4_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ wq,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, float* __restrict__ partial,
    int M, int N, int K, int tiles_m, int tiles, int chunks_per_split) {
  extern __shared__ u32x4_t smem[];
  char* const lds = reinterpret_cast<char*>(smem);
  const int tid = threadIdx.x;
  const int l = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = l >> 5;

  // ---- tile order: XCD-contiguous runs of tile groups ----
  const int nblk = gridDim.x;
  const int per_xcd = nblk / 8, rem = nblk % 8;
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
  const int idx = (xcd < rem ? xcd * (per_xcd + 1) : rem * (per_xcd + 1) + (xcd - rem) * per_xcd) + slot;
  // With K split, idx = split * tiles + tile: a split's blocks are contiguous.
  const int tile = idx % tiles, split = idx / tiles;
  // group g: row blocks g*kGroupM .. +gm-1 x every column block, row fastest
  const int tiles_n = tiles / tiles_m;
  const int g = tile / (kGroupM * tiles_n), r = tile % (kGroupM * tiles_n);
  const int gm = min(kGroupM, tiles_m - g * kGroupM);
  const int bm = g * kGroupM + r % gm, bn = r / gm;
  const int m0 = bm * BM, n0 = bn * BN;

  const int G = K / kGroup;
  const int KT = K / BK;
  const int c_begin = split * chunks_per_split;
  const int c_end = min(KT / kSbChunk, c_begin + chunks_per_split);
  const int kt0 = c_begin * kSbChunk;
  const rsrc_t xrs = make_rsrc(x, (uint64_t)M * K * 2);
  const rsrc_t wrs = make_rsrc(wq, (uint64_t)N * K * BITS / 8);
  const rsrc_t srs = make_rsrc(scales, (uint64_t)N * G * 2);
  const rsrc_t brs = make_rsrc(biases, (uint64_t)N * G * 2);

  // x DMA: wave w, op i fills rows (8w + i)*8 .. +7 of a stage (1 KiB); lane l
  // writes physical chunk l % 8 of row l / 8, i.e. logical chunk (l%8) ^ f(row)
  // with f(row) = (row >> 1) & 7.  Rows past M, and steps past K on the last
  // row, lie beyond the descriptor's M*K*2 bytes and read as zeros.
  uint32_t xoff[kXOps];
#pragma unroll
  for (int i = 0; i < kXOps; ++i) {
    const int row = (wave * kXOps + i) * 8 + (l >> 3);
    xoff[i] = (uint32_t)((m0 + row) * K + (((l & 7) ^ ((row >> 1) & 7)) * 8)) * 2;
  }
  // Codes: column n0 + 64*wave + 32j + l%32, half h of each group.
  constexpr int CB = BITS * 4;  // code bytes per lane per step: 16 (4-bit) / 32 (8-bit)
  constexpr int NC = BITS == 4 ? 2 : 4;  // 16-byte code loads per lane per step
  uint32_t coff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wave * 64 + j * 32 + (l & 31);
    coff[j] = n < N ? (uint32_t)(n * (K * BITS / 8) + h * CB) : kOutOfRange;
  }
  // Scale/bias DMA: wave w loads both arrays for columns 64w + l.
  uint32_t soff;
  {
    const int n = n0 + wave * 64 + l;
    soff = n < N ? (uint32_t)(n * G) * 2 : kOutOfRange;
  }
  const int sb_dst = kSbBase + wave * 1024;
  // A fragment rows 32i + l%32; logical chunk 4h + ks, stored at (4h + ks) ^ f
  // with f = (l >> 1) & 7 for every row tile: only bits 4-5 of the byte offset
  // depend on ks, so the k-slice ks reads at aoff ^ (ks << 4).
  const uint32_t aoff = (uint32_t)((l & 31) * 128 + ((h * 4) ^ ((l >> 1) & 7)) * 16);
  uint32_t sbr[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) sbr[j] = kSbBase + (wave * 64 + j * 32 + (l & 31)) * 16;

  auto dma_x = [&](int kt, int stage) {
#pragma unroll
    for (int i = 0; i < kXOps; ++i)
      dma16(xrs, (lds_t*)(lds + stage * kXStage + (wave * kXOps + i) * 1024),
            xoff[i] + kt * (BK * 2));
  };
  auto dma_sb = [&](int chunk, int buf) {
    dma16(srs, (lds_t*)(lds + sb_dst + buf * kSbBytes), soff + chunk * (kSbChunk * 2));
    dma16(brs, (lds_t*)(lds + sb_dst + buf * kSbBytes + kSbArray), soff + chunk * (kSbChunk * 2));
  };
  auto load_codes = [&](u32x4_t (&cw)[2][NC / 2], int kt) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int p = 0; p < NC / 2; ++p) cw[j][p] = buf_load16(wrs, coff[j] + kt * (BK * BITS / 8) + p * 16);
  };

  f32x16_t acc[kRowTiles][2];
#pragma unroll
  for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  u32x4_t cw[kCodeRing][2][NC / 2];
  auto dequant_frag = [&](const u32x4_t (&q)[2][NC / 2], int j, int ks, const GroupAffine& g) {
    const u32x4_t& w = q[j][BITS == 4 ? 0 : ks >> 1];
    if constexpr (BITS == 4) return dequant8<4>(w[ks], 0u, g.s, g.b);
    else return dequant8<8>(w[(ks & 1) * 2], w[(ks & 1) * 2 + 1], g.s, g.b);
  };
  auto read_sb = [&](int buf, int grp, GroupAffine (&g)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const char* p = lds + sbr[j] + buf * kSbBytes + grp * 2;
      g[j].s = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(p));
      g[j].b = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(p + kSbArray));
    }
  };

  // ---- prologue: codes of this split's first two steps, its first scale
  // chunk, x of its first three steps ----
  load_codes(cw[0], kt0);
  load_codes(cw[1], kt0 + 1);
  dma_sb(c_begin, c_begin & 1);
  dma_x(kt0, 0);
  dma_x(kt0 + 1, 1);
  dma_x(kt0 + 2, 2);
  step_barrier<2 * kXOps>();
  // B fragments of k-slice 0 are always dequantized one step early, at the end
  // of the previous step, so each step opens with MFMAs instead of VALU.
  GroupAffine ga[2];
  read_sb(c_begin & 1, 0, ga);
  bf16x8_t b0[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) b0[j] = dequant_frag(cw[0], j, 0, ga[j]);

  int st = 0;  // stage holding x of the current step
  for (int c = c_begin; c < c_end; ++c) {
#pragma unroll
    for (int u = 0; u < kSbChunk; ++u) {
      const int kt = c * kSbChunk + u;
      const uint32_t xa = st * kXStage + aoff;
      bf16x8_t a[kRowTiles];
#pragma unroll
      for (int i = 0; i < kRowTiles; ++i)
        a[i] = *reinterpret_cast<const bf16x8_t*>(lds + xa + i * 4096);
      load_codes(cw[(u + 2) % kCodeRing], kt + 2);
      dma_x(kt + 3, (st + 3) % kXStages);
      if (u == kSbChunk - 4) dma_sb(c + 1, (c + 1) & 1);

#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        bf16x8_t bq[2], an[kRowTiles];
        if (ks < 3) {
#pragma unroll
          for (int i = 0; i < kRowTiles; ++i)
            an[i] = *reinterpret_cast<const bf16x8_t*>(lds + (xa ^ ((ks + 1) << 4)) + i * 4096);
        }
#pragma unroll
        for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b0[j], acc[i][j], 0, 0, 0);
        if (ks < 3) {
#pragma unroll
          for (int j = 0; j < 2; ++j) bq[j] = dequant_frag(cw[u % kCodeRing], j, ks + 1, ga[j]);
        } else {
          // next step: its scales (the next chunk's buffer after the last
          // step of a chunk, DMA-ed four steps ago) and its first k-slice
          if (u == kSbChunk - 1) read_sb((c + 1) & 1, 0, ga);
          else read_sb(c & 1, u + 1, ga);
#pragma unroll
          for (int j = 0; j < 2; ++j) bq[j] = dequant_frag(cw[(u + 1) % kCodeRing], j, 0, ga[j]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) b0[j] = bq[j];
        if (ks < 3) {
#pragma unroll
          for (int i = 0; i < kRowTiles; ++i) a[i] = an[i];
        }
      }
      // the DMAs of this step and the previous one may still be in flight
      // (two more in the steps that load scales); x of the next step, issued
      // two steps ago, and the scales read next step have landed
      if (u == kSbChunk - 4 || u == kSbChunk - 3) step_barrier<2 * kXOps + 2>();
      else step_barrier<2 * kXOps>();
      st = (st + 1) % kXStages;
    }
  }
  // The prefetches of the last steps (past K, unused) must land before the
  // block's LDS is released.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- epilogue: D[m][n], lane holds n = l%32, m = 8*(v/4) + 4*(l/32) + v%4;
  // a split of K writes float32 partial sums instead ----
  const bool full_rows = m0 + BM <= M;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wave * 64 + j * 32 + (l & 31);
    if (n >= N) continue;
    if (partial) {
      float* pc = partial + (int64_t)split * M * N + n;
#pragma unroll
      for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int mb = m0 + i * 32 + 8 * r + 4 * h;
          float* p = pc + (int64_t)mb * N;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (full_rows || mb + e < M) p[(int64_t)e * N] = acc[i][j][4 * r + e];
        }
    } else {
      const float add = bias ? bf16_bits_to_f32(bias[n]) : 0.f;
      uint16_t* yc = y + n;
#pragma unroll
      for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int mb = m0 + i * 32 + 8 * r + 4 * h;
          uint16_t* p = yc + (int64_t)mb * N;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (full_rows || mb + e < M)
              p[(int64_t)e * N] = (uint16_t)f32_to_bf16_bits(acc[i][j][4 * r + e] + add);
        }
    }
  }
}

// K splits for a launch: 1 when the tiles fill one round of the GPU (one
// block per CU); otherwise the most splits that keep the grid within one
// round, each at least 4 scale chunks (2048 K) long.
int qmm4_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  constexpr int64_t kRound = 256;
  if (tiles >= kRound / 2) return 1;
  const int64_t chunks = K / (kSbChunk * kGroup);
  return (int)std::max<int64_t>(1, std::min(kRound / tiles, chunks / 4));
}

}  // namespace

bool qmm4_fits(int64_t M, int64_t N, int64_t K, int bits) {
  // 32-bit buffer offsets (with room for the kOutOfRange marker) for x, the
  // codes and the scales; whole 8-group scale chunks; >= 128 tiles, or >= 32
  // when K is long enough to split over blocks.
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const int64_t lim = (int64_t)1 << 31;
  return K % (kSbChunk * kGroup) == 0 && (M + BM) * K * 2 < lim && N * K * bits / 8 < lim &&
         N * (K / kGroup) * 2 < lim && tiles < lim &&
         (tiles >= 128 || (tiles >= 32 && qmm4_splits(M, N, K) * tiles >= 128));
}

size_t qmm4_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  const int S = qmm4_splits(M, N, K);
  return S > 1 ? (size_t)S * M * N * sizeof(float) : 0;
}

hipError_t launch_qmm4(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                       int64_t N, int64_t K, int bits, void* workspace, size_t workspace_bytes,
                       hipStream_t stream) {
  if (M == 0 || N == 0) return hipSuccess;
  const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
  const int tiles = tiles_m * tiles_n;
  const int chunks = (int)(K / (kSbChunk * kGroup));
  int S = qmm4_splits(M, N, K);
  if (S > 1 && (!workspace || workspace_bytes < qmm4_workspace_bytes(M, N, K))) S = 1;
  const int per = (chunks + S - 1) / S;
  S = (chunks + per - 1) / per;
  float* part = S > 1 ? static_cast<float*>(workspace) : nullptr;
  const dim3 grid((unsigned)(tiles * S));
  auto kern = bits == 4 ? qmm4_kernel<4> : qmm4_kernel<8>;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), kLds, stream, x, wq, scales, biases, bias, y,
                     part, (int)M, (int)N, (int)K, tiles_m, tiles, per);
  if (S == 1) return hipGetLastError();
  return launch_splitk_reduce(part, S, bias, y, M * N, N, stream);
}

}  // namespace mq
