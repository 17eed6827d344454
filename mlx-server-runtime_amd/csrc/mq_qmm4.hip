// Large-M quantized matmul, two waves per SIMD:
//   y[m, n] = sum_k x[m, k] * (s*q + b)[n, k]  (+ bias[n])
// mx.quantized_matmul(x, w, scales, biases, transpose=True) for prefill-sized
// M (python/mlx_worker/native_mlx/models/qwen2.py:76-78,115,134,227), and
// gather_qmm over experts' row segments (mx.gather_qmm with sorted_indices, as
// python/mlx_worker/native_mlx/models/lfm2.py:176-187 calls it).
//
// MFMA-bound.  A 512-thread block owns a 256x256 output tile and walks K in
// steps of 64 (one quantization group).  Each of its 8 waves -- two per SIMD --
// computes the whole 256-row M tile for 32 columns: 8
// v_mfma_f32_32x32x16_bf16 per 16-wide k slice, 128 float32 accumulators per
// lane.  So every code of the block's 256 columns is dequantized exactly once
// per block (256 MACs per dequantized weight): the weights' VALU work per MFMA
// is half what a 2x4 wave grid (128 rows per wave, each column dequantized by
// two waves) spends; the price is that every wave reads the whole x tile from
// LDS (256 rows x 64 k per step), which the LDS's read bandwidth carries.
// The second wave per SIMD covers the other's stalls (dequantization, LDS
// reads, the barrier); 8 waves measured 4-11% faster than 4 waves of 64
// columns on every shape this kernel serves.
//
// Every load is still issued well ahead of its use:
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
//   Group sizes 32, 64 and 128: a chunk of 8 groups spans 4, 8 or 16 steps; in
//   step u of a chunk lane half h reads group 2u + h, u or u / 2 of it.
// * Tiles run in groups of 4 row blocks x every column block, the row blocks
//   fastest: the 32 blocks an XCD runs at once cover 4 row blocks x 8 column
//   blocks, so they share x rows and codes in that XCD's L2.
// * The output tile is staged through LDS as bfloat16 and written as 16-byte
//   row chunks.
// * Few tiles and a long K split K evenly over blocks; a short last round of
//   tiles (at most a third of the CUs) runs as stream-K pieces (qmm4_plan).
//   Both write float32 partial sums that a reduce adds in a fixed order.
// One barrier per step; the wait before it covers the DMAs of two steps ago
// and earlier (the next step's x tile), never those of this step or the
// previous one.
#include <algorithm>
#include <climits>
#include <type_traits>

#include "mq_common.h"
#include "mq_internal.h"

namespace mq {
namespace {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int kRowTiles = BM / 32;               // 8 MFMA row tiles per wave
constexpr int kXStage = BM * BK * 2;             // 32 KiB of x per step
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

// Arguments of one launch.  Dense: y[M, N] = x[M, K] @ W^T over tiles_m x
// tiles_n tiles (K maybe split).  Gather (mx.gather_qmm over rows sorted by
// expert): rows = T * Mb, row p = (batch t = p / Mb, row m = p % Mb) reads x row
// lhs[t] * Mb + m (t * Mb + m without lhs) and expert rhs[t]'s matrix, and
// writes y row p; tiles are whole 256-row pieces of one expert's segment.
struct Qmm4Args {
  const uint16_t* x;
  const uint32_t* wq;
  const uint16_t* scales;
  const uint16_t* biases;
  const uint16_t* bias;
  uint16_t* y;
  float* partial;
  int M, N, K;  // M: dense rows (gather: T * Mb)
  int tiles_m, tiles_n, tiles, chunks_per_split;
  int chunks;  // scale/bias chunks (8 groups) along K
  // Dense K split: blocks below dp_blocks take (split, tile) pairs of
  // dp_tiles x (K / chunks_per_split) (partial != null: their float32 sums go
  // to partial[split][M][N]).  Blocks from dp_blocks on are stream-K blocks
  // over the tiles from dp_tiles on: block b takes chunks [b sk_w, (b + 1)
  // sk_w) of the flattened (tile, chunk) order of those tiles, a piece of at
  // most two tiles, and writes each piece's float32 sums to
  // sk_partial[(s * sk_pieces + p) * BM * BN] (stream-K tile s's piece p,
  // 256 x 256, row-major); qmm4_sk_reduce adds a tile's pieces in order.
  int dp_blocks, dp_tiles, sk_w, sk_units, sk_pieces;
  float* sk_partial;
  // gather only
  const int32_t* lhs;
  const int32_t* rhs;
  const int32_t* seg;  // E + 1 batch offsets of the expert segments, or null
  int T, Mb, E, x_batches;
};

// Gather tile map, computed by each block from the expert segments: segment e
// holds batches [start_e, start_(e+1)), i.e. ceil((start_(e+1) - start_e) * Mb
// / BM) row tiles, R in all; row tile rt is the (rt - pre_e)-th tile of the
// expert e with pre_e <= rt < pre_(e+1) (exclusive prefix sums).  XCD x
// takes the contiguous row tiles [x P, (x + 1) P), P = ceil(R / 8), in
// expert order, so an expert's tiles share one L2 (its bank fetched once)
// unless they straddle two ranges; the block is its XCD's row-tile slot
// `slot`.  Out: e (-1 for a slot past its range), first row, valid rows,
// and lo/hi: the batches outside [lo, hi) name no expert (ids < 0 sort
// first, ids >= E last) and give zeros, written by XCD 0's slot P (`zero`).
struct GatherTile {
  int e, row0, rows, lo, hi;
  bool zero;
};

template <int kThreads>
__device__ GatherTile gather_tile(const Qmm4Args& a, int xcd, int slot, int* sh) {
  // sh: LDS ints, 2 * (E + 1) + 10 of them; E <= 4 * kThreads
  int* start = sh;              // [E + 1] segment starts (batches)
  int* pre = sh + a.E + 1;      // [E + 1] exclusive tile prefix
  int* misc = pre + a.E + 1;    // [10]: lo, wave totals, the tile's expert
  const int tid = threadIdx.x;
  if (a.seg) {
    // Caller-supplied starts are clamped to [0, T], so every row and x batch
    // a tile touches stays inside y and lhs; a start below its predecessor
    // gives the predecessor an empty segment (rows = max(0, ...) below).
    for (int e = tid; e <= a.E; e += kThreads) start[e] = min(max(a.seg[e], 0), a.T);
  } else {
    // start[e] = the first batch whose id is >= e: one coalesced pass over the
    // sorted ids, each boundary (ids u < v at batches p - 1, p) giving
    // start[e] = p for u < e <= v; experts past the largest id keep T
    for (int e = tid; e <= a.E; e += kThreads) start[e] = a.T;
    __syncthreads();
    for (int p0 = 0; p0 < a.T; p0 += kThreads * 4) {
      int v[4], u[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int p = p0 + q * kThreads + tid;
        v[q] = p < a.T ? a.rhs[p] : INT_MAX;
        u[q] = (p > 0 && p < a.T) ? a.rhs[p - 1] : INT_MIN;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int p = p0 + q * kThreads + tid;
        if (p < a.T && u[q] < v[q])
          for (int e = max(u[q] + 1, 0); e <= min(v[q], a.E); ++e) start[e] = p;
      }
    }
  }
  __syncthreads();
  if (tid == 0) misc[0] = start[0];  // batches before it have negative ids
  __syncthreads();
  // each thread counts the tiles of up to 4 experts: 4 tid .. 4 tid + 3
  int mine[4], sum = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = 4 * tid + q;
    int t = 0;
    if (e < a.E) {
      const int lo = max(start[e], misc[0]);
      const int rows = max(0, start[e + 1] - lo) * a.Mb;
      t = (rows + BM - 1) / BM;
    }
    mine[q] = t;
    sum += t;
  }
  // block exclusive scan of the per-thread sums (wave scan, then wave totals)
  int incl = sum;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off, 64);
    if ((tid & 63) >= off) incl += v;
  }
  if ((tid & 63) == 63) misc[1 + (tid >> 6)] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < (tid >> 6); ++w) base += misc[1 + w];
  int run = base + incl - sum;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = 4 * tid + q;
    if (e < a.E) pre[e] = run;
    run += mine[q];
  }
  if (tid == kThreads - 1) pre[min(a.E, 4 * kThreads)] = run;
  if (tid == 0) misc[9] = -1;
  __syncthreads();
  const int total = pre[a.E];
  const int per = (total + 7) / 8;  // row tiles per XCD
  const int rt = slot < per ? xcd * per + slot : total;  // total: no tile
  for (int e = tid; e < a.E; e += kThreads)
    if (pre[e] <= rt && rt < pre[e + 1]) misc[9] = e;
  __syncthreads();
  GatherTile g;
  g.e = misc[9];
  g.lo = misc[0];
  g.hi = start[a.E];
  g.zero = xcd == 0 && slot == per;
  g.row0 = 0;
  g.rows = 0;
  if (g.e >= 0) {
    const int lo = max(start[g.e], g.lo);
    const int k = rt - pre[g.e];
    g.row0 = lo * a.Mb + k * BM;
    g.rows = min(BM, start[g.e + 1] * a.Mb - g.row0);
  }
  __syncthreads();  // the map's LDS is reused for x tiles
  return g;
}

// Dense tile order: groups of kGroupM row blocks x every column block, row
// blocks fastest.
__device__ __forceinline__ void dense_tile(const Qmm4Args& a, int tile, int& bm, int& bn) {
  const int g = tile / (kGroupM * a.tiles_n), r = tile % (kGroupM * a.tiles_n);
  const int gm = min(kGroupM, a.tiles_m - g * kGroupM);
  bm = g * kGroupM + r % gm;
  bn = r / gm;
}

// WAVES waves (4: one per SIMD, or 8: two) split the block's 256 columns: each
// owns all 256 rows of 256 / WAVES columns (NJ = 8 / WAVES MFMA column tiles),
// so every code of the block is dequantized once whatever WAVES is.
// SWIGLU: the matrix holds 2N rows, gate rows then up rows (the fused gate|up
// projection); block columns 0..127 are 128 gate columns and 128..255 their up
// columns; the epilogue pairs them and writes y[., N] = silu(gate) * up, each
// rounded to bfloat16 as the unfused kernels round (gate and up, then silu,
// then the product).
// GSH: log2(group size / 32); a scale/bias chunk of 8 groups spans SPC steps.
template <int BITS, bool GATHER, bool SB16, bool SWIGLU, int WAVES, int GSH>
__global__ __launch_bounds__(64 * WAVES, 1) void qmm4_kernel(const Qmm4Args a) {
  constexpr int SPC = 4 << GSH;  // steps per chunk
  constexpr int kRun = SPC < 8 ? SPC : 8;  // steps per unrolled run
  static_assert(SPC >= 4 && kRun % kCodeRing == 0, "the chunk's DMA goes 4 steps ahead");
  constexpr int kThreads = 64 * WAVES;
  constexpr int NJ = 8 / WAVES;                     // 32-column MFMA tiles per wave
  constexpr int kXOps = kXStage / (kThreads * 16);  // x DMA operations per lane per step
  extern __shared__ u32x4_t smem[];
  char* const lds = reinterpret_cast<char*>(smem);
  const int tid = threadIdx.x;
  const int l = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = l >> 5;
  const int N = a.N, K = a.K;  // N output columns
  constexpr int kOutCols = SWIGLU ? BN / 2 : BN;  // output columns per block
  const int NW = SWIGLU ? 2 * N : N;              // rows of the (expert's) matrix

  int bn = 0, out_row0 = 0, rows_valid = 0, c_begin = 0, c_end = 0;
  const uint32_t* wbank = a.wq;
  const uint16_t* sbank = a.scales;
  const uint16_t* bbank = a.biases;
  const int G = K >> (5 + GSH);  // groups per row
  const int KT = K / BK;
  const int chunks = (KT + SPC - 1) / SPC;
  // A K split writes float32 sums: element (m, c) of the tile (row m, block
  // column c) goes to pdst[(prow + m) * pld + pcol + c]; null: bfloat16 output
  float* pdst = nullptr;
  int64_t pld = 0;
  int prow = 0, pcol = 0;
  // stream-K block: chunks [sk_f, sk_end) of the flattened (tile, chunk) order
  const bool sk = !GATHER && (int)blockIdx.x >= a.dp_blocks;
  int sk_f = 0, sk_end = 0;
  if constexpr (GATHER) {
    // Blocks go to the 8 XCDs round-robin: block b runs on XCD b % 8 as its
    // (b / 8)-th block there, i.e. row-tile slot (b / 8) / tiles_n, column
    // tile (b / 8) % tiles_n -- each row tile's column tiles consecutive on
    // one XCD, the XCD's row tiles a contiguous run of the expert order
    // (gather_tile).  The grid reserves at least one slot per XCD past its
    // run.
    const int xcd = (int)blockIdx.x % 8, j = (int)blockIdx.x / 8;
    bn = j % a.tiles_n;
    const GatherTile g =
        gather_tile<kThreads>(a, xcd, j / a.tiles_n, reinterpret_cast<int*>(lds));
    if (g.e < 0) {
      // one spare slot zeroes the rows whose id names no expert
      if (g.zero) {
        const int n = bn * kOutCols + tid;
        if (tid < kOutCols && n < N) {
          for (int p = 0; p < g.lo * a.Mb; ++p) a.y[(int64_t)p * N + n] = 0;
          for (int p = g.hi * a.Mb; p < a.T * a.Mb; ++p) a.y[(int64_t)p * N + n] = 0;
        }
      }
      return;
    }
    out_row0 = g.row0;
    rows_valid = g.rows;
    wbank += (int64_t)g.e * NW * (K * BITS / 32);
    sbank += (int64_t)g.e * NW * G;
    bbank += (int64_t)g.e * NW * G;
    c_end = chunks;
  } else if (!sk) {
    // XCD-contiguous runs of the tile order below: consecutive idx on one XCD
    const int nblk = a.dp_blocks;
    const int per_xcd = nblk / 8, rem = nblk % 8;
    const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
    const int idx = (xcd < rem ? xcd * (per_xcd + 1) : rem * (per_xcd + 1) + (xcd - rem) * per_xcd) + slot;
    // With K split, idx = split * tiles + tile: a split's blocks are contiguous.
    const int tile = idx % a.dp_tiles, split = idx / a.dp_tiles;
    int bm;
    dense_tile(a, tile, bm, bn);
    out_row0 = bm * BM;
    rows_valid = min(BM, a.M - out_row0);
    c_begin = split * a.chunks_per_split;
    c_end = min(chunks, c_begin + a.chunks_per_split);
    if (a.partial) {
      pdst = a.partial + (int64_t)split * a.M * N;
      pld = N, prow = out_row0, pcol = bn * kOutCols;
    }
  } else {
    const int b = (int)blockIdx.x - a.dp_blocks;
    sk_f = b * a.sk_w;
    sk_end = min(a.sk_units, sk_f + a.sk_w);
  }
  for (;;) {  // one segment (a tile's chunk range) per pass; only stream-K blocks loop
    if (sk) {
      const int s = sk_f / chunks;
      c_begin = sk_f - s * chunks;
      c_end = min(chunks, c_begin + (sk_end - sk_f));
      int bm;
      dense_tile(a, a.dp_tiles + s, bm, bn);
      out_row0 = bm * BM;
      rows_valid = min(BM, a.M - out_row0);
      // pieces of tile s come from blocks s*chunks/sk_w, ... in chunk order
      const int piece = (int)blockIdx.x - a.dp_blocks - s * chunks / a.sk_w;
      pdst = a.sk_partial + ((int64_t)s * a.sk_pieces + piece) * (BM * BN);
      pld = BN, prow = 0, pcol = 0;
    }
    const int n0 = bn * kOutCols;
    // matrix row of block column c (0..255): c itself past n0, or for SWIGLU
    // gate row n0 + c for c < 128, else the up row of output column n0 + c - 128
    auto wrow = [&](int c, int& out_col) {
      if constexpr (SWIGLU) {
        out_col = n0 + (c & 127);
        return (c >> 7) * N + out_col;
      } else {
        out_col = n0 + c;
        return out_col;
      }
    };
    // MFMA row tiles holding valid rows (the same for every wave of the block)
    const int live = __builtin_amdgcn_readfirstlane((rows_valid + 31) / 32);

    const int kt0 = c_begin * SPC;
    const int kt_end = min(KT, c_end * SPC);
    const int x_rows = GATHER ? a.x_batches * a.Mb : a.M;
    const rsrc_t xrs = make_rsrc(a.x, (uint64_t)x_rows * K * 2);
    const rsrc_t wrs = make_rsrc(wbank, (uint64_t)NW * K * BITS / 8);
    const rsrc_t srs = make_rsrc(sbank, (uint64_t)NW * G * 2);
    const rsrc_t brs = make_rsrc(bbank, (uint64_t)NW * G * 2);

    // x DMA: wave w, op i fills rows (8w + i)*8 .. +7 of a stage (1 KiB); lane l
    // writes physical chunk l % 8 of row l / 8, i.e. logical chunk (l%8) ^ f(row)
    // with f(row) = (row >> 1) & 7.  Rows past the tile's valid rows read as
    // zeros (an offset past the descriptor).
    uint32_t xoff[kXOps];
#pragma unroll
    for (int i = 0; i < kXOps; ++i) {
      const int row = (wave * kXOps + i) * 8 + (l >> 3);
      const uint32_t chunk = (uint32_t)(((l & 7) ^ ((row >> 1) & 7)) * 8);
      if constexpr (GATHER) {
        xoff[i] = kOutOfRange;
        if (row < rows_valid) {
          const int p = out_row0 + row;
          const int t = p / a.Mb, m = p - t * a.Mb;
          const int xb = a.lhs ? a.lhs[t] : t;
          if (xb >= 0 && xb < a.x_batches)
            xoff[i] = ((uint32_t)(xb * a.Mb + m) * (uint32_t)K + chunk) * 2u;
        }
      } else {
        xoff[i] = row < rows_valid ? (uint32_t)((out_row0 + row) * K + (int)chunk) * 2 : kOutOfRange;
      }
    }
    // Codes: block column 32 NJ wave + 32j + l%32, half h of each group.
    constexpr int CB = BITS * 4;  // code bytes per lane per step: 16 (4-bit) / 32 (8-bit)
    constexpr int NC = BITS == 4 ? 2 : 4;  // 16-byte code loads per lane per step
    uint32_t coff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      int oc;
      const int n = wrow(wave * 32 * NJ + j * 32 + (l & 31), oc);
      coff[j] = oc < N ? (uint32_t)(n * (K * BITS / 8) + h * CB) : kOutOfRange;
    }
    // Scale/bias DMA, as wave operations o of 64 lanes (column block cb of 64
    // columns, lane l taking column 64 cb + l); wave w issues o = w, w + WAVES,
    // ..., all with cb = w % 4.  SB16: 8 operations per chunk, o = 4a + cb, one
    // 16-byte load per lane (8 groups of a column; LDS [array][column][group]);
    // otherwise 32, o = 16a + 4d + cb, dword d of 4 (rows of G groups, G even,
    // are only 4-byte aligned; LDS [array][group pair][column]).
    constexpr int kSbOps = (SB16 ? 8 : 32) / WAVES;  // DMA operations per lane per chunk
    uint32_t soff;
    {
      int oc;
      const int n = wrow((wave & 3) * 64 + l, oc);
      soff = oc < N ? (uint32_t)(n * G) * 2 : kOutOfRange;
    }
    // A fragment rows 32i + l%32; logical chunk 4h + ks, stored at (4h + ks) ^ f
    // with f = (l >> 1) & 7 for every row tile: only bits 4-5 of the byte offset
    // depend on ks, so the k-slice ks reads at aoff ^ (ks << 4).
    const uint32_t aoff = (uint32_t)((l & 31) * 128 + ((h * 4) ^ ((l >> 1) & 7)) * 16);
    uint32_t sbr[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = wave * 32 * NJ + j * 32 + (l & 31);
      sbr[j] = kSbBase + (SB16 ? c * 16 : c * 4);
    }

    auto dma_x = [&](int kt, int stage) {
#pragma unroll
      for (int i = 0; i < kXOps; ++i)
        dma16(xrs, (lds_t*)(lds + stage * kXStage + (wave * kXOps + i) * 1024),
              xoff[i] + kt * (BK * 2));
    };
    auto dma_sb = [&](int chunk, int buf) {
      char* dst = lds + kSbBase + buf * kSbBytes;
      const uint32_t src = soff + chunk * (kSbChunk * 2);
#pragma unroll
      for (int t = 0; t < kSbOps; ++t) {
        const int o = wave + WAVES * t;
        if constexpr (SB16) {
          const int arr = o >> 2, cb = o & 3;
          dma16(arr ? brs : srs, (lds_t*)(dst + arr * kSbArray + cb * 1024), src);
        } else {
          const int arr = o >> 4, d = (o >> 2) & 3, cb = o & 3;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(arr ? brs : srs,
                                                   (lds_t*)(dst + arr * kSbArray + d * 1024 + cb * 256),
                                                   4, src + d * 4, 0, 0, 0);
        }
      }
    };
    auto load_codes = [&](u32x4_t (&cw)[NJ][NC / 2], int kt) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int p = 0; p < NC / 2; ++p) cw[j][p] = buf_load16(wrs, coff[j] + kt * (BK * BITS / 8) + p * 16);
    };

    f32x16_t acc[kRowTiles][NJ];
#pragma unroll
    for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    u32x4_t cw[kCodeRing][NJ][NC / 2];
    auto dequant_frag = [&](const u32x4_t (&q)[NJ][NC / 2], int j, int ks, const GroupAffine& g) {
      const u32x4_t& w = q[j][BITS == 4 ? 0 : ks >> 1];
      if constexpr (BITS == 4) return dequant8<4>(w[ks], 0u, g.s, g.b);
      else return dequant8<8>(w[(ks & 1) * 2], w[(ks & 1) * 2 + 1], g.s, g.b);
    };
    // the chunk's group of step u for this lane (half h of the step's 64 k)
    auto group_of = [&](int u) { return GSH == 0 ? 2 * u + h : GSH == 1 ? u : u >> 1; };
    auto read_sb = [&](int buf, int grp, GroupAffine (&g)[NJ]) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const char* p = lds + sbr[j] + buf * kSbBytes +
                        (SB16 ? grp * 2 : (grp >> 1) * 1024 + (grp & 1) * 2);
        g[j].s = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(p));
        g[j].b = bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(p + kSbArray));
      }
    };

    // ---- short gather tiles: at most 64 valid rows (two MFMA row tiles) ----
    // Such a tile (an expert segment's last few rows) does little MFMA work
    // per step, so its steps wait on memory latency: with the loops below a
    // 32-row tile cost 84 % of a full one.  It lays the LDS out differently:
    // eight 8 KiB x stages of 64 rows, x six steps ahead, and per wave a ring
    // of two 4-step code blocks (its 32 columns x 128 bytes, DMA'd as 8
    // columns x 128 bytes per operation), the next block four steps ahead.
    // Every load is a DMA, so each barrier's count is exact.  Dequantization
    // and MFMA order are those of the loops below: bit-identical results.
    auto short_tile = [&]() {
      constexpr int XS = 8, XA = 6;      // x stages, x DMAs ahead
      constexpr int kShX = 64 * BK * 2;  // an x stage: 64 rows
      constexpr int kShCode = 32 * 128;  // a wave's 4-step code block
      static_assert(XS * kShX + WAVES * 2 * kShCode <= kSbBase, "short-tile LDS");
      char* const cring = lds + XS * kShX + wave * (2 * kShCode);
      // x: wave w fills rows 8w .. 8w + 7 of a stage (the swizzle above)
      uint32_t xo = kOutOfRange;
      {
        const int row = 8 * wave + (l >> 3);
        const uint32_t chunk = (uint32_t)(((l & 7) ^ ((row >> 1) & 7)) * 8);
        if (row < rows_valid) {
          const int p = out_row0 + row;
          const int t = p / a.Mb, m = p - t * a.Mb;
          const int xb = a.lhs ? a.lhs[t] : t;
          if (xb >= 0 && xb < a.x_batches)
            xo = ((uint32_t)(xb * a.Mb + m) * (uint32_t)K + chunk) * 2u;
        }
      }
      // codes: operation j fills columns 8j .. 8j + 7 of the wave's 32; lane l
      // reads piece (l % 8) ^ f(c) of column c = 8j + l / 8, f(c) = (c >> 1) &
      // 7, so column c holds logical piece p at c * 128 + 16 (p ^ f(c)) and 8
      // lanes reading one piece of 8 columns hit 8 distinct bank groups
      uint32_t cdo[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = 8 * j + (l >> 3);
        int oc;
        const int n = wrow(wave * 32 + c, oc);
        cdo[j] = oc < N ? (uint32_t)n * (uint32_t)(K / 2) + 16u * (uint32_t)((l & 7) ^ ((c >> 1) & 7))
                        : kOutOfRange;
      }
      // this lane's 16 bytes of step s of a block: logical piece 2s + h
      const uint32_t cread = (uint32_t)((l & 31) * 128 + 16 * (h ^ ((l >> 1) & 7)));
      auto dma_code_block = [&](int b) {  // steps 4b .. 4b + 3 into slot b & 1
        char* slot = cring + (b & 1) * kShCode;
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16(wrs, (lds_t*)(slot + j * 1024), cdo[j] + (uint32_t)b * 128u);
      };
      auto dma_x_short = [&](int kt) {
        dma16(xrs, (lds_t*)(lds + (kt % XS) * kShX + wave * 1024), xo + kt * (BK * 2));
      };
      // In issue order a step makes: the next code block's 4 DMAs (steps 4b),
      // one x DMA, the next chunk's scale/bias DMAs (a chunk's first step).
      // End of step kt: x of kt + 1 (issued at kt - 5) has at least 9
      // operations after it; at 4b + 3 the block of 4b + 4 (issued at 4b) has
      // 4, and a chunk's scales (issued at its first step) have SPC - 1 or
      // more by the chunk's last step, where the next chunk's are read.
      dma_sb(c_begin, c_begin & 1);
      dma_code_block(kt0 / 4);
#pragma unroll
      for (int p = 0; p < XA; ++p) dma_x_short(kt0 + p);
      step_barrier<XA - 1>();
      for (int c = c_begin; c < c_end; ++c) {
#pragma unroll 1
        for (int u0 = 0; u0 < SPC; u0 += kRun) {
#pragma unroll
          for (int ui = 0; ui < kRun; ++ui) {
            const int u = u0 + ui;
            const int kt = c * SPC + u;
            if (kt >= kt_end) break;
            if (ui % 4 == 0) dma_code_block(kt / 4 + 1);
            dma_x_short(kt + XA);
            if (u == 0) dma_sb(c + 1, (c + 1) & 1);
            GroupAffine g[NJ];
            read_sb(c & 1, group_of(u), g);
            const u32x4_t q = *reinterpret_cast<const u32x4_t*>(
                cring + ((kt / 4) & 1) * kShCode + (cread ^ (32u * (uint32_t)(ui & 3))));
            const uint32_t xa = (uint32_t)(kt % XS) * kShX + aoff;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
              const bf16x8_t bq = dequant8<4>(q[ks], 0u, g[0].s, g[0].b);
#pragma unroll
              for (int i = 0; i < 2; ++i)
                if (i < live)
                  acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                      *reinterpret_cast<const bf16x8_t*>(lds + (xa ^ (ks << 4)) + i * 4096), bq,
                      acc[i][0], 0, 0, 0);
            }
            if ((ui & 3) == 3) step_barrier<SPC == 4 ? 3 : 4>();
            else step_barrier<9>();
          }
        }
      }
    };

    if (GATHER && BITS == 4 && NJ == 1 && live <= 2) {
      if constexpr (GATHER && BITS == 4 && NJ == 1) short_tile();
    } else {
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
    GroupAffine ga[NJ];
    read_sb(c_begin & 1, group_of(0), ga);
    bf16x8_t b0[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) b0[j] = dequant_frag(cw[0], j, 0, ga[j]);

    // The K loop.  MASKED skips the MFMAs (and A reads) of row tiles past the
    // tile's valid rows, at the price of a branch per row tile; full tiles take
    // the branch-free body.
    auto k_loop = [&](auto masked) {
      constexpr bool MASKED = decltype(masked)::value;
      int st = 0;  // stage holding x of the current step
      for (int c = c_begin; c < c_end; ++c) {
        // a 16-step chunk (group size 128) runs as two unrolled runs of 8
        // (the compiler does not unroll 16 of these steps); ui, a multiple
        // of the code ring's length away from u, indexes the ring
#pragma unroll 1
        for (int u0 = 0; u0 < SPC; u0 += kRun) {
#pragma unroll
        for (int ui = 0; ui < kRun; ++ui) {
          const int u = u0 + ui;
          const int kt = c * SPC + u;
          // a K of G % 8 != 0 groups ends mid-chunk; the runs of 16-step
          // chunks keep the test too (without it the compiler spills the
          // SB16 form's registers)
          if constexpr (!SB16 || kRun < SPC) {
            if (kt >= kt_end) break;
          }
          const uint32_t xa = st * kXStage + aoff;
          bf16x8_t a[kRowTiles];
#pragma unroll
          for (int i = 0; i < kRowTiles; ++i)
            if (!MASKED || i < live) a[i] = *reinterpret_cast<const bf16x8_t*>(lds + xa + i * 4096);
          load_codes(cw[(ui + 2) % kCodeRing], kt + 2);
          dma_x(kt + 3, (st + 3) % kXStages);
          if (u == SPC - 4) dma_sb(c + 1, (c + 1) & 1);

#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            bf16x8_t bq[NJ], an[kRowTiles];
            if (ks < 3) {
#pragma unroll
              for (int i = 0; i < kRowTiles; ++i)
                if (!MASKED || i < live)
                  an[i] = *reinterpret_cast<const bf16x8_t*>(lds + (xa ^ ((ks + 1) << 4)) + i * 4096);
            }
#pragma unroll
            for (int i = 0; i < kRowTiles; ++i)
              if (!MASKED || i < live) {
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                  acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b0[j], acc[i][j], 0, 0, 0);
              }
            if (ks < 3) {
#pragma unroll
              for (int j = 0; j < NJ; ++j) bq[j] = dequant_frag(cw[ui % kCodeRing], j, ks + 1, ga[j]);
            } else {
              // next step: its scales (the next chunk's buffer after the last
              // step of a chunk, DMA-ed four steps ago) and its first k-slice
              if (u == SPC - 1) read_sb((c + 1) & 1, group_of(0), ga);
              else read_sb(c & 1, group_of(u + 1), ga);
#pragma unroll
              for (int j = 0; j < NJ; ++j) bq[j] = dequant_frag(cw[(ui + 1) % kCodeRing], j, 0, ga[j]);
            }
#pragma unroll
            for (int j = 0; j < NJ; ++j) b0[j] = bq[j];
            if (ks < 3) {
#pragma unroll
              for (int i = 0; i < kRowTiles; ++i) a[i] = an[i];
            }
          }
          // the DMAs of this step and the previous one may still be in flight
          // (more in the steps that load scales); x of the next step, issued two
          // steps ago, and the scales read next step have landed
          if (u == SPC - 4 || u == SPC - 3) step_barrier<2 * kXOps + kSbOps>();
          else step_barrier<2 * kXOps>();
          st = (st + 1) % kXStages;
        }
        }
      }
    };
    // Tiles of at most 192 valid rows (short expert segments, the last row
    // tile) skip their empty MFMA row tiles; the branches cost more than one
    // row tile's MFMAs (a dense sweep of masked tile heights measured a
    // 224-row masked tile 6 % slower than a full 256-row one).
    if (live <= kRowTiles - 2) k_loop(std::true_type{});
    else k_loop(std::false_type{});
    }
    // The prefetches of the last steps (past K, unused) must land before the
    // block's LDS is released.
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // ---- epilogue: D[m][n], lane holds n = l%32, m = 8*(v/4) + 4*(l/32) + v%4 ----
    const bool full_rows = rows_valid == BM;
    if (pdst) {
      // a K split writes its float32 partial sums straight from registers
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int c = wave * 32 * NJ + j * 32 + (l & 31);
        if (n0 + c >= N) continue;
        float* pc = pdst + pcol + c;
#pragma unroll
        for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int mb = i * 32 + 8 * r + 4 * h;
            float* p = pc + (int64_t)(prow + mb) * pld;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (full_rows || mb + e < rows_valid) p[(int64_t)e * pld] = acc[i][j][4 * r + e];
          }
      }
    } else {
      // bfloat16 output: the 256 x 256 tile of block columns goes through LDS
      // (the x stages; every wave's DMAs have landed once all have passed the
      // barrier) so that rows leave as 16-byte stores instead of 2-byte ones per
      // lane and value.  SWIGLU stages the gate and up columns (rounded to
      // bfloat16, as the unfused GEMM stores them) and pairs them on the way out.
      __syncthreads();
      constexpr int kStageStride = BN * 2 + 16;  // bytes per staged row (padding spreads banks)
      static_assert(BM * kStageStride <= kLds, "the output tile must fit the LDS");
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int c = wave * 32 * NJ + j * 32 + (l & 31);
        float add = 0.f;
        if constexpr (!SWIGLU) {
          const int n = n0 + c;
          add = (a.bias && n < N) ? bf16_bits_to_f32(a.bias[n]) : 0.f;
        }
#pragma unroll
        for (int i = 0; i < kRowTiles; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int m = i * 32 + 8 * r + 4 * h + e;
              *reinterpret_cast<uint16_t*>(lds + m * kStageStride + c * 2) =
                  (uint16_t)f32_to_bf16_bits(acc[i][j][4 * r + e] + add);
            }
      }
      __syncthreads();
      // thread t stores 16-byte chunk t % CPR of rows (kThreads / CPR) q + t / CPR
      constexpr int kOutCols_ = SWIGLU ? BN / 2 : BN;
      constexpr int CPR = kOutCols_ / 8;  // chunks per output row
      const int cc = tid % CPR;
      const int n = n0 + cc * 8;
      const bool vec = (N % 8 == 0) && ((reinterpret_cast<uintptr_t>(a.y) & 15) == 0);
#pragma unroll 4
      for (int q = 0; q < BM * CPR / kThreads; ++q) {
        const int row = q * (kThreads / CPR) + tid / CPR;
        if (row >= rows_valid || n >= N) continue;
        const char* src = lds + row * kStageStride + cc * 16;
        u32x4_t v = *reinterpret_cast<const u32x4_t*>(src);
        if constexpr (SWIGLU) {
          const u32x4_t up = *reinterpret_cast<const u32x4_t*>(src + (BN / 2) * 2);
#pragma unroll
          for (int w = 0; w < 4; ++w)
            v[w] = (uint32_t)silu_mul_bf16(lo_bf16(v[w]), lo_bf16(up[w])) |
                   ((uint32_t)silu_mul_bf16(hi_bf16(v[w]), hi_bf16(up[w])) << 16);
        }
        uint16_t* dst = a.y + (int64_t)(out_row0 + row) * N + n;
        if (vec) {
          // nontemporal: the output streams out once (measured against plain
          // stores: the MoE-prefill down projection 8 % faster, the dense and
          // gate|up GEMMs 1-4 %)
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(dst));
        } else {
          // constant indices into v: no copy of it on the stack
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (n + e < N) dst[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
        }
      }
    }
    if (!sk) break;
    sk_f += c_end - c_begin;
    if (sk_f >= sk_end) break;
    // the next segment's DMAs reuse the LDS: every wave's stores and reads of
    // this one are done
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
}

// Scale/bias chunks (8 groups each) along K.
int64_t sb_chunks(int64_t K, int group_size) {
  return (K / group_size + kSbChunk - 1) / kSbChunk;
}

// K splits for a launch: 1 when the tiles fill half a round of the GPU (one
// block per CU); otherwise the most splits that keep the grid within one
// round, each at least 1024 K long (whole scale chunks).  Measured at M = 512
// (7B prefill of one 512-token prompt, group size 64): the down projection
// 18944 -> 3584 in 28 tiles x 9 splits takes 81 us where the 128 x 128 GEMM
// took 431 us, and q/k/v 3584 -> 4608 in 36 tiles x 3 splits 47 us (85 us).
int qmm4_splits(int64_t M, int64_t N, int64_t K, int group_size) {
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  constexpr int64_t kRound = 256;
  if (tiles >= kRound / 2) return 1;
  const int64_t cap = sb_chunks(K, group_size) * group_size / 128;  // 1024 K per split
  return (int)std::max<int64_t>(1, std::min(kRound / tiles, cap));
}

constexpr int kWaves = 8;  // waves per block: two per SIMD
constexpr int kMaxPieces = 8;  // stream-K pieces per tile

// Stream-K tiles: y = the sum of a tile's pieces in piece order (+ bias),
// rounded to bfloat16 -- the order is fixed by the plan, so results do not
// depend on timing.  Grid (BM / 8, stream-K tiles) of 256 threads; thread t
// adds 8 consecutive columns of tile row 8 * blockIdx.x + t / 32.
__global__ __launch_bounds__(256) void qmm4_sk_reduce(const Qmm4Args a) {
  const int s = blockIdx.y;
  const int chunks = a.chunks;
  const int first = s * chunks / a.sk_w;
  const int pieces = (s * chunks + chunks - 1) / a.sk_w - first + 1;
  int bm, bn;
  dense_tile(a, a.dp_tiles + s, bm, bn);
  const int r = blockIdx.x * 8 + (threadIdx.x >> 5);
  const int c = (threadIdx.x & 31) * 8;
  const int m = bm * BM + r, n = bn * BN + c;
  if (m >= a.M || n >= a.N) return;
  const float* p = a.sk_partial + (int64_t)s * a.sk_pieces * (BM * BN) + r * BN + c;
  f32x4_t v[kMaxPieces][2];
#pragma unroll
  for (int q = 0; q < kMaxPieces; ++q)
    if (q < pieces) {
      v[q][0] = *reinterpret_cast<const f32x4_t*>(p + q * (BM * BN));
      v[q][1] = *reinterpret_cast<const f32x4_t*>(p + q * (BM * BN) + 4);
    }
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
  for (int q = 0; q < kMaxPieces; ++q)
    if (q < pieces) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += v[q][e >> 2][e & 3];
    }
  uint16_t* dst = a.y + (int64_t)m * a.N + n;
  uint16_t o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float b = (a.bias && n + e < a.N) ? bf16_bits_to_f32(a.bias[n + e]) : 0.f;
    o[e] = (uint16_t)f32_to_bf16_bits(acc[e] + b);
  }
  if (n + 8 <= a.N && ((reinterpret_cast<uintptr_t>(dst) & 15) == 0)) {
    *reinterpret_cast<u32x4_t*>(dst) = __builtin_bit_cast(u32x4_t, o);
  } else {
    for (int e = 0; e < 8 && n + e < a.N; ++e) dst[e] = o[e];
  }
}

// How a dense launch covers its tiles.  The uniform plan runs every tile
// whole, or (few tiles) split into S equal K ranges.  When the tiles fill
// whole rounds of the GPU (one block per CU, 256 CUs) and leave a short last
// round -- at most a third of the CUs busy -- the tiles of that last round go
// to stream-K blocks instead: 256 blocks share their chunks equally, so the
// launch takes its full rounds plus sk_w chunks, and a reduce adds the
// pieces.  Measured (4-bit, against every tile whole): 296 tiles (M = 1024,
// 3584 -> 18944) -15 %, 576 (M = 8192, 3584 -> 4608) -4 %, 592 (M = 2048,
// 3584 -> 18944) -2 %, 2368 (M = 8192) +-0.  Longer last rounds, and launches
// of fewer than 256 tiles, were slower (M = 2048, 3584 -> 4608 in 144 tiles
// +17 %; 18944 -> 3584 in 112 tiles +5 %; 448 tiles +1-3 %): the float32
// pieces' round trip through memory costs more than the idle CUs, which the
// short last round runs at a higher clock.
struct Plan {
  int S;          // uniform K splits per tile
  int dp_tiles;   // tiles run whole or uniformly split
  int sk_tiles;   // the last tiles, run by stream-K blocks
  int sk_w;       // chunks per stream-K block
  int sk_blocks, sk_pieces;
};

Plan qmm4_plan(int64_t M, int64_t N, int64_t K, int group_size) {
  constexpr int64_t kRound = 256;
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const int64_t chunks = sb_chunks(K, group_size);
  Plan p{};
  p.S = qmm4_splits(M, N, K, group_size);
  const int64_t cps = (chunks + p.S - 1) / p.S;
  p.S = (int)((chunks + cps - 1) / cps);
  p.dp_tiles = (int)tiles;
  const int64_t makespan = p.S > 1 ? cps : (tiles + kRound - 1) / kRound * chunks;
  const int64_t skt = tiles % kRound;
  if (tiles < kRound || skt == 0 || skt > kRound / 3) return p;
  const int64_t units = skt * chunks, w = (units + kRound - 1) / kRound;
  if (w < 2 || w >= chunks || (tiles - skt) / kRound * chunks + w > makespan - 2) return p;
  int64_t pieces = 0;
  for (int64_t s = 0; s < skt; ++s)
    pieces = std::max(pieces, ((s + 1) * chunks - 1) / w - s * chunks / w + 1);
  if (pieces > kMaxPieces) return p;
  p.S = 1;
  p.dp_tiles = (int)(tiles - skt);
  p.sk_tiles = (int)skt;
  p.sk_w = (int)w;
  p.sk_blocks = (int)((units + w - 1) / w);
  p.sk_pieces = (int)pieces;
  return p;
}

size_t plan_workspace(const Plan& p, int64_t M, int64_t N) {
  if (p.sk_tiles) return (size_t)p.sk_tiles * p.sk_pieces * BM * BN * sizeof(float);
  return p.S > 1 ? (size_t)p.S * M * N * sizeof(float) : 0;
}

template <bool GATHER, bool SWIGLU, int GSH>
void (*pick_kernel(int bits, bool sb16))(Qmm4Args) {
  if (bits == 4)
    return sb16 ? qmm4_kernel<4, GATHER, true, SWIGLU, kWaves, GSH>
                : qmm4_kernel<4, GATHER, false, SWIGLU, kWaves, GSH>;
  return sb16 ? qmm4_kernel<8, GATHER, true, SWIGLU, kWaves, GSH>
              : qmm4_kernel<8, GATHER, false, SWIGLU, kWaves, GSH>;
}

template <bool GATHER, bool SWIGLU>
hipError_t launch(const Qmm4Args& a, int bits, int group_size, dim3 grid, hipStream_t stream) {
  const bool sb16 = (a.K / group_size) % kSbChunk == 0;
  void (*kern)(Qmm4Args) = group_size == 32  ? pick_kernel<GATHER, SWIGLU, 0>(bits, sb16)
                           : group_size == 64 ? pick_kernel<GATHER, SWIGLU, 1>(bits, sb16)
                                              : pick_kernel<GATHER, SWIGLU, 2>(bits, sb16);
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, grid, dim3(64 * kWaves), kLds, stream, a);
  return hipGetLastError();
}

// 32-bit buffer offsets (with room for the kOutOfRange marker) for x, the
// codes and the scales of one matrix; an even number of groups (whole 64-wide
// steps, 4-byte aligned scale rows) of 32, 64 or 128.
bool offsets_fit(int64_t x_rows, int64_t N, int64_t K, int bits, int group_size) {
  const int64_t lim = (int64_t)1 << 31;
  return (group_size == 32 || group_size == 64 || group_size == 128) &&
         K % (2 * group_size) == 0 && (x_rows + BM) * K * 2 < lim && N * K * bits / 8 < lim &&
         N * (K / group_size) * 2 < lim;
}

}  // namespace

bool qmm4_fits(int64_t M, int64_t N, int64_t K, int bits, int group_size) {
  // >= 128 tiles, or >= 8 whose K splits give >= 64 blocks
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  return offsets_fit(M, N, K, bits, group_size) && tiles < ((int64_t)1 << 31) &&
         (tiles >= 128 || (tiles >= 8 && qmm4_splits(M, N, K, group_size) * tiles >= 64));
}

size_t qmm4_workspace_bytes(int64_t M, int64_t N, int64_t K, int group_size) {
  return plan_workspace(qmm4_plan(M, N, K, group_size), M, N);
}

bool qmm4_unsplit(int64_t M, int64_t N, int64_t K, int group_size) {
  return qmm4_splits(M, N, K, group_size) == 1;
}

bool qmm4_stream_k(int64_t M, int64_t N, int64_t K, int group_size) {
  return qmm4_plan(M, N, K, group_size).sk_tiles > 0;
}

hipError_t launch_qmm4(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                       int64_t N, int64_t K, int bits, int group_size, void* workspace,
                       size_t workspace_bytes, hipStream_t stream) {
  if (M == 0 || N == 0) return hipSuccess;
  Qmm4Args a{};
  a.x = x, a.wq = wq, a.scales = scales, a.biases = biases, a.bias = bias, a.y = y;
  a.M = (int)M, a.N = (int)N, a.K = (int)K;
  a.tiles_m = (int)((M + BM - 1) / BM), a.tiles_n = (int)((N + BN - 1) / BN);
  a.tiles = a.tiles_m * a.tiles_n;
  const int chunks = (int)sb_chunks(K, group_size);
  a.chunks = chunks;
  Plan p = qmm4_plan(M, N, K, group_size);
  // without the workspace the plan needs: every tile whole
  if (!workspace || workspace_bytes < plan_workspace(p, M, N)) p = Plan{1, a.tiles, 0, 0, 0, 0};
  a.chunks_per_split = (chunks + p.S - 1) / p.S;
  a.partial = p.S > 1 ? static_cast<float*>(workspace) : nullptr;
  a.dp_tiles = p.dp_tiles;
  a.dp_blocks = p.dp_tiles * p.S;
  a.sk_w = p.sk_w;
  a.sk_units = p.sk_tiles * chunks;
  a.sk_pieces = p.sk_pieces;
  a.sk_partial = p.sk_tiles ? static_cast<float*>(workspace) : nullptr;
  const hipError_t e = launch<false, false>(a, bits, group_size,
                                            dim3((unsigned)(a.dp_blocks + p.sk_blocks)), stream);
  if (e != hipSuccess) return e;
  if (p.sk_tiles) {
    hipLaunchKernelGGL(qmm4_sk_reduce, dim3(BM / 8, (unsigned)p.sk_tiles), dim3(256), 0, stream, a);
    return hipGetLastError();
  }
  if (p.S == 1) return e;
  return launch_splitk_reduce(a.partial, p.S, bias, y, M * N, N, stream);
}

bool qmm4_gather_fits(int64_t T, int64_t Mb, int64_t N, int64_t K, int64_t E,
                      int64_t x_batches, int bits, int group_size) {
  const int64_t lim = (int64_t)1 << 31;
  return E >= 1 && E <= 4 * 64 * kWaves && T * Mb < lim / 2 &&
         offsets_fit(x_batches * Mb, N, K, bits, group_size);
}

hipError_t launch_qmm4_gather(const uint16_t* x, const int32_t* lhs, const int32_t* rhs,
                              const int32_t* seg, const uint32_t* wq, const uint16_t* scales,
                              const uint16_t* biases, uint16_t* y, int64_t T, int64_t Mb,
                              int64_t N, int64_t K, int64_t E, int64_t x_batches, int bits,
                              int group_size, bool swiglu, hipStream_t stream) {
  if (T == 0 || Mb == 0 || N == 0) return hipSuccess;
  Qmm4Args a{};
  a.x = x, a.wq = wq, a.scales = scales, a.biases = biases, a.y = y;
  a.M = (int)(T * Mb), a.N = (int)N, a.K = (int)K;
  const int out_cols = swiglu ? BN / 2 : BN;
  a.tiles_n = (int)((N + out_cols - 1) / out_cols);
  a.chunks = a.chunks_per_split = (int)sb_chunks(K, group_size);
  a.lhs = lhs, a.rhs = rhs, a.seg = seg;
  a.T = (int)T, a.Mb = (int)Mb, a.E = (int)E, a.x_batches = (int)x_batches;
  // every expert's segment adds at most one partial tile: R <= bound row
  // tiles in all; each XCD gets ceil(R / 8) of them and one more slot (the
  // spare that zeroes the rows whose id names no expert)
  const int64_t bound = (T * Mb + BM - 1) / BM + std::min(E, T);
  const int64_t row_tiles = ((bound + 7) / 8 + 1) * 8;
  const dim3 grid((unsigned)(row_tiles * a.tiles_n));
  return swiglu ? launch<true, true>(a, bits, group_size, grid, stream)
                : launch<true, false>(a, bits, group_size, grid, stream);
}

bool qmm4_swiglu_fits(int64_t M, int64_t N, int64_t K, int bits, int group_size) {
  // the gate|up matrix (2N rows) in 128-column output tiles, unsplit
  const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN / 2 - 1) / (BN / 2));
  return offsets_fit(M, 2 * N, K, bits, group_size) && tiles >= 128 &&
         tiles < ((int64_t)1 << 31);
}

hipError_t launch_qmm4_swiglu(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                              const uint16_t* biases, uint16_t* y, int64_t M, int64_t N,
                              int64_t K, int bits, int group_size, hipStream_t stream) {
  if (M == 0 || N == 0) return hipSuccess;
  Qmm4Args a{};
  a.x = x, a.wq = wq, a.scales = scales, a.biases = biases, a.y = y;
  a.M = (int)M, a.N = (int)N, a.K = (int)K;
  a.tiles_m = (int)((M + BM - 1) / BM), a.tiles_n = (int)((N + BN / 2 - 1) / (BN / 2));
  a.tiles = a.tiles_m * a.tiles_n;
  a.chunks = a.chunks_per_split = (int)sb_chunks(K, group_size);
  a.dp_tiles = a.dp_blocks = a.tiles;
  return launch<false, true>(a, bits, group_size, dim3((unsigned)a.tiles), stream);
}

}  // namespace mq
