// Skinny quantized matmul on the matrix cores (M up to a few hundred rows):
//   y[m, n] = sum_k x[m, k] * (s*q + b)[n, k]  (+ bias[n])
// mx.quantized_matmul(x, w, scales, biases, transpose=True) for batched decode
// and short prefill chunks (python/mlx_worker/native_mlx/models/qwen2.py:
// 76-78,115,134,227; the scheduler caps a prefill chunk at 256 rows,
// python/mlx_worker/scheduler.py:567).
//
// Every weight is read from HBM and dequantized exactly once per M tile, so
// for M <= 128 the kernel streams the codes like a GEMV while the matrix
// cores do the arithmetic.  A block of 4 waves owns 128 columns (32 per
// wave; unsplit 32-row plans may take 5, 6 or 8 waves) and an M tile of
// 32*MI rows (MI = 1, 2, 4), and walks K in steps of one quantization group:
// * x tiles (32*MI rows x 64) are copied HBM -> LDS by buffer_load_dwordx4
//   ... lds three steps ahead into four stages, rows of 128 bytes with the
//   16-byte chunk index XOR-ed with (row >> 1) & 7.
// * For v_mfma_f32_32x32x16_bf16's B operand lane l holds column l % 32 and,
//   in k-slice ks, the 8 codes k = 32h + 8ks .. +7 of its half h = l / 32
//   (A reads x with the same k order), so a lane's codes for a step are one
//   contiguous 16-byte (4-bit) or 32-byte (8-bit) range, dequantized
//   (fma(s, q, b), one bfloat16 rounding) in registers.  4-bit codes are
//   loaded into registers four steps ahead (a GEMV-sized M has little work
//   per step, so the loads in flight must cover the memory latency); 8-bit
//   codes come as whole 128-byte lines, DMA'd 4-6 steps ahead into a
//   per-wave LDS ring, and are read from there a step ahead.
// * Scales and biases come 8 groups at a time (16 bytes per column and
//   array), a chunk ahead.
// When the N x M tiles alone cannot fill the GPU (few columns, long K: the
// down projection), K is split over blocks in whole 8-group chunks; each
// split writes float32 partial sums to a caller-provided workspace and
// splitk_reduce adds them in a fixed order (results do not depend on timing).
// Unsplit 32-row plans too wide for one block per CU at 4 waves take blocks of
// 5-8 column groups, each group's K steps split over two waves (4-bit).
#include <algorithm>
#include <type_traits>

#include "mq_common.h"
#include "mq_internal.h"

namespace mq {
namespace {

constexpr int BN = 128;  // columns of a 4-wave block
constexpr int BK = 64;
constexpr int kChunk = 8;     // groups per scale/bias load
// Pipeline depths: codes kPrefetch steps ahead (divides kChunk), x kXAhead
// steps ahead in kXStages LDS stages (a power of two above kXAhead).  Measured
// on the M = 16/32 7B shapes: x 4-7 steps ahead in 8 stages changed nothing
// (+-1 %), codes 8 steps ahead were 5-8 % slower, 2 ahead slower still.
constexpr int kPrefetch = 4;
constexpr int kXAhead = 3;
constexpr int kXStages = 4;

typedef __attribute__((address_space(3))) void lds_t;

template <int AUX = 0>
__device__ __forceinline__ void dma16(rsrc_t r, lds_t* dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, 0, 0, AUX);
}

// 8-bit codes by DMA: a code block is a wave's 32 columns x 128 bytes (2 K
// steps), brought in by 4 DMAs of 8 columns x 128 bytes, so that every 8
// lanes read one whole 128-byte line, where a lane's own 2 x 16 bytes per step
// make each wave instruction read 32 columns x 16 bytes.  Each wave keeps
// kCodeSlots blocks in its own LDS ring.  Measured against the per-lane loads
// (bit-identical results): 8-bit 11-25 % faster (M = 16 down projection
// 26.1 -> 21.2 us, M = 32 3584 x 18944 28.4 -> 21.4 us, M = 128 40.6 ->
// 36.1 us); 4-bit (32 columns x 32 bytes per instruction) 2-14 % slower at
// M = 16..256, so 4-bit codes keep the per-lane register loads -- except in
// the K-sliced 10-wave blocks (qmms_kernel's KS), where the DMA is 5 % faster.
constexpr int kCodeSlots = 4;
constexpr int kCodeBlock = 32 * 128;
template <int BITS>
constexpr bool kCodeDma = BITS == 8;

// End of a step: wait until at most N memory operations are outstanding, then
// sync the block.  vmcnt retires in issue order.  Every memory operation of
// the kernel stays where the program issues it (the streamed inputs are not
// __restrict__, and the loads sit between empty asm statements with memory
// clobbers), so N can count exactly the operations issued after the DMA that
// must have landed: the next step's x tile.
template <int N>
__device__ __forceinline__ void step_barrier() {
  __asm__ volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

template <int BITS>
__device__ __forceinline__ bf16x8_t dequant8(uint32_t w0, uint32_t w1, float s, float b) {
  u32x4_t o;
  if constexpr (BITS == 4) {
    // byte t of w0 = q[2t] | q[2t+1] << 4; the empty asm keeps two masks
    // feeding v_cvt_f32_ubyte0..3 instead of one bit-field extract per code.
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

// W waves per block (4, or 5, 6, 8 for unsplit 32-row tiles: the block count
// then stays within one per CU); waves 0-3 copy the x tiles.
// EPI 1 (SwiGLU; one 32-row tile, no split): the matrix is N = 2*Nout rows,
// gate rows first; wave w of a block takes gate columns n0 + 16w .. +15 in
// lanes l % 32 < 16 and the matching up columns Nout + n0 + 16w .. in lanes
// l % 32 >= 16, and its gate lanes store y[m, n] = bf16(bf16(silu(g)) * u)
// with g, u rounded to bfloat16 as the plain kernel stores them -- silu_mul
// of its output, bit for bit (each column's MFMA sums do not depend on the
// lane that holds it).
// x, wq, scales and biases are deliberately not __restrict__: with it the
// compiler may move their loads across the barriers' inline asm, and the
// barriers' counts assume the issue order below.
// GSH: log2(group size / 32) -- group sizes 32, 64, 128.  A lane's codes for
// a 64-wide step are k = 32h .. 32h + 31 of it (both widths), all in one
// group, (2 step + h) >> GSH within the chunk of 8 steps.
// KS (2: 4-bit, one unsplit 32-row tile): the block's W waves are W / KS
// column groups x KS K slices -- wave w takes column group w % (W / KS) and,
// of every 8-step chunk, the 8 / KS steps of slice w / (W / KS), each slice
// with x stages of its own; at the end the slices' sums meet in LDS and are
// added in slice order.  Each code is still dequantized once, but the work of
// a column group is spread over KS waves (more waves per SIMD, each with less
// serial work).
// CDMA: codes by DMA into the per-wave LDS ring (8-bit always; 4-bit with KS 2).
template <int BITS, int MI, bool PARTIAL, int EPI = 0, int W = 4, int GSH = 1, int KS = 1,
          bool CDMA = kCodeDma<BITS>>
__global__ __launch_bounds__(64 * W) void qmms_kernel(
    const uint16_t* x, const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, float* __restrict__ partial,
    int M, int N, int K, int tiles_n, int tiles_m, int chunks_per_split) {
  constexpr int BM = 32 * MI;
  constexpr int P = kXAhead;   // x DMA steps ahead
  constexpr int S = kXStages;  // x stages
  static_assert(kChunk % kPrefetch == 0 && (S & (S - 1)) == 0 && S > P && P >= 2 && P <= kChunk,
                "pipeline");
  constexpr int kXStage = BM * BK * 2;
  constexpr int CB = BITS * 4;           // code bytes per lane per step
  constexpr int NC = BITS == 4 ? 1 : 2;  // 16-byte code loads per lane per step
  static_assert(EPI == 0 || (MI == 1 && !PARTIAL), "SwiGLU epilogue: one tile, no split");
  static_assert(W == 4 || (MI == 1 && !PARTIAL), "wider blocks: one tile, no split");
  constexpr int C = W / KS;  // column groups of 32 columns (EPI 1: 16 + 16)
  static_assert(W % KS == 0 && C >= 4 && (KS == 1 || (KS == 2 && W > 4 && BITS == 4)),
                "K slices: wide 4-bit plans");
  static_assert(CDMA || BITS == 4, "8-bit codes come by DMA");
  // A slice takes SPI consecutive steps of each 8-step chunk: slice sl the
  // steps 8c + SPI sl .. + SPI - 1 of chunk c.
  constexpr int SPI = kChunk / KS;
  constexpr int CSL = KS > 1 ? 3 : kCodeSlots;  // code blocks in a wave's ring
  extern __shared__ u32x4_t smem[];
  char* const lds = reinterpret_cast<char*>(smem);
  const int l = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cg = KS == 1 ? wave : wave % C;  // column group
  const int sl = KS == 1 ? 0 : wave / C;     // K slice
  const int h = l >> 5;

  int blk = blockIdx.x;
  const int tn = blk % tiles_n;
  blk /= tiles_n;
  const int tm = blk % tiles_m;
  const int split = blk / tiles_m;
  const int Nout = N / 2;  // EPI 1: output columns
  const int n0 = tn * (EPI == 1 ? 16 * C : 32 * C), m0 = tm * BM;
  const int KT = K / BK;
  const int G = K >> (5 + GSH);  // groups per row
  constexpr uint32_t kChunkSB = 32u >> GSH;  // scale (or bias) bytes per chunk of 8 steps
  const int c_begin = split * chunks_per_split;
  const int c_end = min(KT / kChunk, c_begin + chunks_per_split);

  const rsrc_t xrs = make_rsrc(x, (uint64_t)M * K * 2);
  const rsrc_t wrs = make_rsrc(wq, (uint64_t)N * K * BITS / 8);
  const rsrc_t srs = make_rsrc(scales, (uint64_t)N * G * 2);
  const rsrc_t brs = make_rsrc(biases, (uint64_t)N * G * 2);

  // x DMA: op i of column group w < 4 fills rows (4i + w)*8 .. +7 (1 KiB) of
  // its slice's tile; lane l writes physical chunk l % 8 of row l / 8,
  // logical chunk (l % 8) ^ ((row >> 1) & 7).  Rows past M lie beyond the
  // descriptor and read as zeros.
  uint32_t xoff[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int row = (i * 4 + cg) * 8 + (l >> 3);
    xoff[i] = (uint32_t)((m0 + row) * K + (((l & 7) ^ ((row >> 1) & 7)) * 8)) * 2;
  }
  // This lane's column; columns past N lie beyond the descriptors (zeros).
  const int n = EPI == 1 ? ((l & 16) ? Nout : 0) + n0 + cg * 16 + (l & 15)
                         : n0 + cg * 32 + (l & 31);
  const uint32_t coff = (uint32_t)n * (uint32_t)(K * BITS / 8) + h * CB;
  const uint32_t soff = (uint32_t)n * (uint32_t)G * 2;
  // A fragment: row 32i + l % 32, logical chunk 4h + ks at (4h + ks) ^ f(row).
  const uint32_t aoff = (uint32_t)((l & 31) * 128 + ((h * 4) ^ ((l >> 1) & 7)) * 16);
  // Code DMA: op j of a block fills rows 8j .. 8j + 7 of the wave's slot
  // (row c = the B operand's column c); lane l reads piece (l % 8) ^ f(c) of
  // column c = 8j + l / 8, f(c) = (c >> 1) & 7, and lands at physical piece
  // l % 8, so row c holds logical 16-byte piece p at c * 128 + 16 * (p ^ f(c)):
  // 16 consecutive lanes reading one piece of 16 rows hit 16 distinct 16-byte
  // bank groups.  A lane's codes for step s of a block are logical piece
  // 2s + h (4-bit) or pieces 4s + 2h, +1 (8-bit); they are read from the ring
  // at the end of the step before (ahead of its barrier), so no LDS latency
  // sits between a barrier and the next step's dequantization.
  constexpr int QS = 128 / (BK * BITS / 8);  // K steps per code block
  // A slice's code blocks are numbered in its own order, BPC per chunk:
  // slice block b of chunk b / BPC is K block KS b + sl (KS 1: b itself).
  constexpr int BPC = SPI / QS;
  // blocks DMA'd ahead: QS * (DA - 1) > P, so the wait for step kt's x tile
  // (issued P steps before kt) also covers the code block of step kt + 1
  constexpr int DA = 1 + (P + QS) / QS;
  static_assert(!CDMA || (DA < CSL && SPI % QS == 0 && QS * NC == 4), "code ring");
  char* const cring = lds + S * KS * kXStage + wave * (CSL * kCodeBlock);
  uint32_t cdoff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = 8 * j + (l >> 3);
    const int col = EPI == 1 ? ((c & 16) ? Nout : 0) + n0 + cg * 16 + (c & 15) : n0 + cg * 32 + c;
    cdoff[j] = (uint32_t)col * (uint32_t)(K * BITS / 8) + 16u * (uint32_t)((l & 7) ^ ((c >> 1) & 7));
  }
  const uint32_t cread =
      (uint32_t)((l & 31) * 128 + 16 * ((BITS == 4 ? h : 2 * h) ^ ((l >> 1) & 7)));
  auto read_codes = [&](u32x4_t (&q)[NC], int qb, int s) {  // step s of slice block qb
    const char* slot = cring + (qb % CSL) * kCodeBlock;
#pragma unroll
    for (int e = 0; e < NC; ++e)
      q[e] = *reinterpret_cast<const u32x4_t*>(
          slot + (cread ^ (BITS == 4 ? 32 * s : 64 * s + 16 * e)));
  };
  auto dma_codes = [&](int qb, int j0) {  // ops j0 .. j0 + NC - 1 of slice block qb
#pragma unroll
    for (int p = 0; p < NC; ++p)
      dma16<kBufNT>(wrs, (lds_t*)(cring + (qb % CSL) * kCodeBlock + (j0 + p) * 1024),
                    cdoff[j0 + p] + (uint32_t)(KS * qb + sl) * 128u);
  };

  auto dma_x = [&](int kt, int stage) {
    if (W > 4 && cg >= 4) return;  // uniform
#pragma unroll
    for (int i = 0; i < MI; ++i)
      dma16(xrs, (lds_t*)(lds + (stage * KS + sl) * kXStage + (i * 4 + cg) * 1024),
            xoff[i] + kt * (BK * 2));
  };
  auto load_codes = [&](u32x4_t (&cw)[NC], int kt) {
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (int p = 0; p < NC; ++p) cw[p] = buf_load16(wrs, coff + kt * (BK * BITS / 8) + p * 16);
    __asm__ volatile("" ::: "memory");
  };
  // At the end of step kt the x DMA of step kt + 1 (issued in step
  // kt + 1 - P) must have landed; issued after it: the codes of that step,
  // then per step kt + 2 - P .. kt MI DMAs and NC code loads (and, at a
  // chunk's first step, two scale/bias loads, which only add to the count).
  constexpr int kInFlight = NC + (P - 1) * (MI + NC);
  // A split's first P - 1 steps are the exception: x of step j + 1 (j < P - 1)
  // was issued by the prologue, which loads no codes after its x DMAs, so
  // only the prologue's later x DMAs, the first step's scale/bias loads and
  // steps 0..j's x DMAs and codes follow it.
  constexpr auto first_count = [](int u) {
    const int a = (P - 1) * MI + (u + 1) * NC + 2;
    return u <= P - 2 && a < kInFlight ? a : kInFlight;
  };
  // Waves past the fourth issue no x DMA: their barrier waits for their own
  // code blocks.  The block read at the end of step kt (for step kt + 1) had
  // its last op in step kt - QS * (DA - 1), so the barrier of step kt - 1
  // leaves at most the QS * (DA - 1) - 1 steps of NC ops after it in flight
  // (the prologue's blocks are followed by more).
  constexpr int kCodeOnly = (QS * (DA - 1) - 1) * NC;
  static_assert(!CDMA || W <= 4 || (P - 1) * MI <= (DA - 1) * 4,
                "prologue wait covers block 0");
  // the barrier of step u of a split's first chunk (u is a constant after
  // the unrolling, so the switch folds away)
  auto first_barrier = [&](int u) {
    switch (u) {
      case 0: step_barrier<first_count(0)>(); break;
      case 1: step_barrier<first_count(1)>(); break;
      case 2: step_barrier<first_count(2)>(); break;
      case 3: step_barrier<first_count(3)>(); break;
      case 4: step_barrier<first_count(4)>(); break;
      case 5: step_barrier<first_count(5)>(); break;
      case 6: step_barrier<first_count(6)>(); break;
      default: step_barrier<first_count(7)>(); break;
    }
  };
  static_assert(kChunk == 8, "first_barrier covers one chunk of 8 steps");

  f32x16_t acc[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[i][v] = 0.f;

  // ---- prologue: codes of the first kPrefetch steps, x of the first P ----
  // a chunk's scales and biases for this lane's column: 16 (GSH 0), 8 or 4
  // entries
  auto load_sb = [&](u32x4_t (&v)[2], const rsrc_t& r, int c) {
    const uint32_t o = soff + (uint32_t)c * kChunkSB;
    if constexpr (GSH == 0) {
      v[0] = buf_load16(r, o);
      v[1] = buf_load16(r, o + 16);
    } else if constexpr (GSH == 1) {
      v[0] = buf_load16(r, o);
    } else {
      const u32x2_t t = buf_load8(r, o);
      v[0] = u32x4_t{t[0], t[1], 0u, 0u};
    }
  };
  // the entry of the slice's step u (a compile-time constant after
  // unrolling) of a chunk -- step e = SPI sl + u of the chunk -- for lane
  // half h: group 2e + h, e or e / 2
  auto sb_entry = [&](const u32x4_t (&v)[2], int u) -> float {
    uint32_t d;
    int half;
    if constexpr (GSH == 0) {
      d = KS > 1 ? (sl ? v[1][u] : v[0][u]) : v[u >> 2][u & 3];
      half = h;
    } else if constexpr (GSH == 1) {
      d = KS > 1 ? (sl ? v[0][2 + (u >> 1)] : v[0][u >> 1]) : v[0][u >> 1];
      half = u & 1;
    } else {
      d = KS > 1 ? (sl ? v[0][1] : v[0][0]) : v[0][u >> 2];
      half = (u >> 1) & 1;
    }
    return half ? hi_bf16(d) : lo_bf16(d);
  };
  // the slice's step u of chunk c (u past the chunk: of the chunks after it)
  auto step_at = [&](int c, int u) { return (c + u / SPI) * kChunk + SPI * sl + u % SPI; };
  u32x4_t sv[2], bv[2];
  load_sb(sv, srs, c_begin);
  load_sb(bv, brs, c_begin);
  u32x4_t cw[CDMA ? 1 : kPrefetch][NC];
  if constexpr (CDMA) {
#pragma unroll
    for (int b = 0; b < DA; ++b)
#pragma unroll
      for (int j = 0; j < 4; j += NC) dma_codes(c_begin * BPC + b, j);
  } else {
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) load_codes(cw[p], step_at(c_begin, p));
  }
#pragma unroll
  for (int p = 0; p < P; ++p) dma_x(step_at(c_begin, p), p);
  step_barrier<(P - 1) * MI>();
  if constexpr (CDMA) read_codes(cw[0], c_begin * BPC, 0);

  int st = 0;  // stage of the current step's x tile
  for (int c = c_begin; c < c_end; ++c) {
    u32x4_t svn[2], bvn[2];
#pragma unroll
    for (int u = 0; u < SPI; ++u) {
      if (u == 0) {
        __asm__ volatile("" ::: "memory");
        load_sb(svn, srs, c + 1);
        load_sb(bvn, brs, c + 1);
        __asm__ volatile("" ::: "memory");
      }
      dma_x(step_at(c, u + P), (st + P) & (S - 1));

      const float s = sb_entry(sv, u);
      const float b = sb_entry(bv, u);
      const uint32_t xa = (st * KS + sl) * kXStage + aoff;
      u32x4_t (&q)[NC] = cw[CDMA ? 0 : u % kPrefetch];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        bf16x8_t a[MI];
#pragma unroll
        for (int i = 0; i < MI; ++i)
          a[i] = *reinterpret_cast<const bf16x8_t*>(lds + (xa ^ (ks << 4)) + i * 4096);
        const u32x4_t& w = q[BITS == 4 ? 0 : ks >> 1];
        bf16x8_t bq;
        if constexpr (BITS == 4) bq = dequant8<4>(w[ks], 0u, s, b);
        else bq = dequant8<8>(w[(ks & 1) * 2], w[(ks & 1) * 2 + 1], s, b);
#pragma unroll
        for (int i = 0; i < MI; ++i)
          acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bq, acc[i], 0, 0, 0);
      }
      // refill the slot just consumed with the codes kPrefetch steps ahead
      // (by DMA: the next step's codes from the ring, then this step's share
      // of the block DA ahead)
      if constexpr (CDMA) {
        read_codes(q, c * BPC + (u + 1) / QS, (u + 1) % QS);
        dma_codes(c * BPC + u / QS + DA, (u % QS) * NC);
      } else {
        load_codes(q, step_at(c, u + kPrefetch));
      }
      if (CDMA && W > 4 && cg >= 4) step_barrier<kCodeOnly>();  // uniform
      else if (c == c_begin) first_barrier(u);
      else step_barrier<kInFlight>();
      st = (st + 1) & (S - 1);
    }
    sv[0] = svn[0];
    bv[0] = bvn[0];
    if constexpr (GSH == 0) {
      sv[1] = svn[1];
      bv[1] = bvn[1];
    }
  }
  // Prefetches past the split's range must land before the LDS is released.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (KS > 1) {
    // slice 1's sums to LDS (over the x stages, read by every wave by now),
    // added to slice 0's in that order; slice 0 stores
    static_assert(C * 16 * 64 * 4 <= kXStages * KS * kXStage, "slice sums fit the x stages");
    float* red = reinterpret_cast<float*>(lds) + cg * 16 * 64 + l;
    __syncthreads();
    if (sl == 1) {
#pragma unroll
      for (int v = 0; v < 16; ++v) red[v * 64] = acc[0][v];
    }
    __syncthreads();
    if (sl != 0) return;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[0][v] += red[v * 64];
  }

  // ---- epilogue: D[m][n], lane holds column l % 32, rows 8(v/4) + 4(l/32) + v%4 ----
  if constexpr (EPI == 1) {
    // lane l ^ 16 holds the up column of gate lane l (same rows)
    const int cl = n0 + cg * 16 + (l & 15);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float g = bf16_bits_to_f32(f32_to_bf16_bits(acc[0][v]));
      const float u = __shfl_xor(g, 16, 64);
      const int r = 8 * (v >> 2) + 4 * (l >> 5) + (v & 3);
      if (!(l & 16) && cl < Nout && m0 + r < M)
        y[(int64_t)(m0 + r) * Nout + cl] = silu_mul_bf16(g, u);
    }
    return;
  }
  if (n >= N) return;
  const float add = (!PARTIAL && bias) ? bf16_bits_to_f32(bias[n]) : 0.f;
#pragma unroll
  for (int i = 0; i < MI; ++i) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int m = m0 + i * 32 + 8 * (v >> 2) + 4 * (l >> 5) + (v & 3);
      if (m < M) {
        if constexpr (PARTIAL)
          partial[((int64_t)split * M + m) * N + n] = acc[i][v];
        else
          y[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_bits(acc[i][v] + add);
      }
    }
  }
}

// y[m, n] = bf16(sum over splits of partial[s, m, n] (in split order) + bias[n])
// acc[e] += the S split-K partials p[s * stride + off[e]] (e < W), added in
// split order.  The loads of B splits go out before the first add, so S
// splits cost ceil(S / B) memory round trips instead of S.
template <int W, int B>
__device__ __forceinline__ void add_splits(const float* p, int S, int64_t stride,
                                           const int (&off)[W], float (&acc)[W]) {
  for (int s0 = 0; s0 < S; s0 += B) {
    float v[B][W];
#pragma unroll
    for (int i = 0; i < B; ++i)
      if (s0 + i < S) {  // uniform
#pragma unroll
        for (int e = 0; e < W; ++e) v[i][e] = p[(s0 + i) * stride + off[e]];
      }
#pragma unroll
    for (int i = 0; i < B; ++i)
      if (s0 + i < S) {
#pragma unroll
        for (int e = 0; e < W; ++e) acc[e] += v[i][e];
      }
  }
}

__global__ __launch_bounds__(256) void splitk_reduce(const float* __restrict__ partial, int S,
                                                     const uint16_t* __restrict__ bias,
                                                     uint16_t* __restrict__ y, int64_t MN, int N) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= MN) return;
  float acc[1] = {0.f};
  add_splits<1, 16>(partial + i, S, MN, {0}, acc);
  if (bias) acc[0] += bf16_bits_to_f32(bias[i % N]);
  y[i] = (uint16_t)f32_to_bf16_bits(acc[0]);
}

// splitk_reduce's sums (same order), then silu_mul on the bf16 results: y
// [M, Nout] from partials of the [M, 2 Nout] gate|up product.
__global__ __launch_bounds__(256) void splitk_reduce_swiglu(const float* __restrict__ partial,
                                                            int S, uint16_t* __restrict__ y,
                                                            int64_t M, int Nout) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= M * Nout) return;
  const int64_t m = i / Nout;
  const int n = (int)(i - m * Nout);
  const int64_t N2 = 2 * (int64_t)Nout, MN2 = M * N2;
  const float* p = partial + m * N2 + n;
  float g = 0.f, u = 0.f;
  for (int s = 0; s < S; ++s) {  // few splits here (the gate|up product is wide)
    g += p[s * MN2];
    u += p[s * MN2 + Nout];
  }
  y[i] = silu_mul_bf16(bf16_bits_to_f32(f32_to_bf16_bits(g)), bf16_bits_to_f32(f32_to_bf16_bits(u)));
}

// splitk_reduce's sums (same order, + bias), rounded to bf16 as it stores
// them, then the RMSNorm kernel's residual add and norm on the row: one block
// (256 threads) per row m, 8-element units t, t + 256, ... (N <= 8192), the
// same reduction order -- equal bit for bit to splitk_reduce + mq_rms_norm.
__global__ __launch_bounds__(256) void splitk_reduce_add_norm(
    const float* __restrict__ partial, int S, const uint16_t* __restrict__ bias,
    const uint16_t* __restrict__ residual, uint16_t* __restrict__ residual_out,
    const uint16_t* __restrict__ w, uint16_t* __restrict__ out, int64_t M, int N, float eps) {
  constexpr int kUnits = 4;
  __shared__ float red[4];
  const int64_t m = blockIdx.x;
  const int units = N / 8;
  const int64_t MN = M * N;
  u32x4_t hv[kUnits], rv[kUnits], wv[kUnits], bv[kUnits];
  // the row's residual, norm weight and bias first: none of them waits for the
  // partial sums
#pragma unroll
  for (int k = 0; k < kUnits; ++k) {
    const int u = threadIdx.x + k * 256;
    if (u < units) {
      rv[k] = reinterpret_cast<const u32x4_t*>(residual + m * N)[u];
      wv[k] = reinterpret_cast<const u32x4_t*>(w)[u];
      if (bias) {
        if ((reinterpret_cast<uintptr_t>(bias) & 15) == 0) {  // uniform
          bv[k] = reinterpret_cast<const u32x4_t*>(bias)[u];
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            bv[k][q] = (uint32_t)bias[u * 8 + 2 * q] | (uint32_t)bias[u * 8 + 2 * q + 1] << 16;
        }
      }
    }
  }
  float ss = 0.f;
  // Rows of at most 512 units (N <= 4096): the partial sums of both of a
  // thread's units are requested before the first add (one round trip); a
  // thread without a second unit reads its first unit's twice.  Threads past
  // the row's units (N < 2048) read nothing: their first unit would lie past
  // the row, and past the workspace on the last row of the last split.
  float acc2[2][8] = {};
  const bool two = units <= 512 && (int)threadIdx.x < units;
  if (two) {
    const int u1 = threadIdx.x + 256 < units ? 256 * 8 : 0;
    float acc16[16] = {};
    add_splits<16, 8>(partial + m * N + threadIdx.x * 8, S, MN,
                      {0, 1, 2, 3, 4, 5, 6, 7, u1, u1 + 1, u1 + 2, u1 + 3, u1 + 4, u1 + 5, u1 + 6,
                       u1 + 7},
                      acc16);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc2[0][e] = acc16[e], acc2[1][e] = acc16[8 + e];
  }
#pragma unroll
  for (int k = 0; k < kUnits; ++k) {
    const int u = threadIdx.x + k * 256;
    if (u < units) {
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (two && k < 2) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = acc2[k][e];
      } else {
        add_splits<8, 16>(partial + m * N + u * 8, S, MN, {0, 1, 2, 3, 4, 5, 6, 7}, acc);
      }
      if (bias) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[2 * q] += lo_bf16(bv[k][q]);
          acc[2 * q + 1] += hi_bf16(bv[k][q]);
        }
      }
      const u32x4_t r = rv[k];
      u32x4_t h;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t yv = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
        h[q] = pack_bf16x2(lo_bf16(yv) + lo_bf16(r[q]), hi_bf16(yv) + hi_bf16(r[q]));
      }
      reinterpret_cast<u32x4_t*>(residual_out + m * N)[u] = h;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float a = lo_bf16(h[q]), b = hi_bf16(h[q]);
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
      hv[k] = h;
    }
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) ss += __shfl_xor(ss, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss += red[i];
  const float inv = rsqrtf(ss / (float)N + eps);
#pragma unroll
  for (int k = 0; k < kUnits; ++k) {
    const int u = threadIdx.x + k * 256;
    if (u < units) {
      u32x4_t o;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = pack_bf16x2(lo_bf16(hv[k][q]) * inv * lo_bf16(wv[k][q]),
                           hi_bf16(hv[k][q]) * inv * hi_bf16(wv[k][q]));
      reinterpret_cast<u32x4_t*>(out + m * N)[u] = o;
    }
  }
}

struct Plan {
  int mi, waves, tiles_n, tiles_m, splits, chunks_per_split;
  int ks;  // K slices per column group (qmms_kernel's KS): waves * ks waves a block
};

Plan plan(int64_t M, int64_t N, int64_t K, int bits, bool can_split) {
  Plan p;
  const int chunks = (int)(K / (BK * kChunk));
  p.tiles_n = (int)((N + BN - 1) / BN);
  // Above 32 rows: 128-row tiles where they alone give >= 128 tiles or K is
  // long enough (>= 16 chunks) to split finely, else 64-row tiles. Measured
  // at M = 128: 18944 x 3584 in 148 unsplit 128-row tiles 33.6 us (64-row:
  // 35.7), 4608 x 3584 in 72 64-row tiles x 3 splits 16.6 us (128-row tiles
  // x 7 splits: 19.2); at M = 256, 4608 x 3584 in 144 unsplit 64-row tiles
  // 20.0 us (128-row x 3 splits: 23.4).
  p.mi = 1;
  if (M > 32) {
    const int64_t tiles4 = (int64_t)p.tiles_n * ((M + 127) / 128);
    p.mi = M > 64 && (tiles4 >= 128 || chunks >= 16) ? 4 : 2;
  }
  p.tiles_m = (int)((M + 32 * p.mi - 1) / (32 * p.mi));
  const int64_t base = (int64_t)p.tiles_n * p.tiles_m;
  int64_t splits = 1;
  // Blocks wanted: at most one per CU (256 CUs), the splits rounded down.
  // Measured at M = 16..32: the down projection 3584 x 18944 at 8 splits
  // (224 blocks) takes 20 us where 13 splits (364 blocks, two on some CUs)
  // take 23 us, and 28672 x 4096 runs unsplit (224 tiles) in 24 us against
  // 34 us in 5 splits. At M = 64..256 the same holds: the 128-row down
  // projection in 28 tiles x 8 splits takes 32.0 us (4 splits: 47.7), and
  // 148 tiles of 18944 x 3584 run unsplit in 33.6 us (2 splits: 42.7).
  if (can_split && base < 256) {
    int64_t cap = chunks;
    if (p.mi == 1) {
      // The partial sums (written once, read once) stay under an eighth of
      // the weight bytes, or 4 MiB, which stays in the Infinity Cache: small
      // matrices (a layer's q/k/v or o at M = 32) then get short blocks,
      // whose serial step latency otherwise sets the kernel time. Taller
      // tiles carry enough work per step that their partials (at most
      // 256 blocks x 128 x 128 floats, 16 MiB) cost less than idle CUs.
      const int64_t weight_bytes = N * K * bits / 8;
      cap = std::max<int64_t>(weight_bytes / (16 * M * N), (4 << 20) / (4 * M * N));
    }
    splits = std::min<int64_t>({256 / base, chunks, cap});
  }
  if (splits < 1) splits = 1;
  p.chunks_per_split = (int)((chunks + splits - 1) / splits);
  p.splits = (chunks + p.chunks_per_split - 1) / p.chunks_per_split;
  // Unsplit 32-row plans with more tiles than CUs take wider blocks (5, 6 or
  // 8 waves of 32 columns) where that brings them within one per CU: at
  // M = 32 the 37888-row gate|up matrix in 296 blocks of 128 columns takes
  // 36.9 us, as 40 CUs run two blocks, where 32768 rows in 256 blocks take
  // 22.2 us.
  p.waves = 4;
  p.ks = 1;
  if (p.mi == 1 && p.splits == 1 && base > 256) {
    for (const int w : {5, 6, 8}) {
      const int t = (int)((N + 32 * w - 1) / (32 * w));
      if (t <= 256) {
        p.waves = w;
        p.tiles_n = t;
        // 4-bit: two waves per column group, each on half of every chunk's
        // K steps, codes by DMA where the per-wave rings fit (5 groups):
        // the 37888-row gate|up at M = 32 29.5 -> 26.5 us (M = 16 29.0 ->
        // 26.2), of which 29.5 -> 27.9 from the slices alone
        p.ks = bits == 4 ? 2 : 1;
        break;
      }
    }
  }
  return p;
}

template <int BITS, int MI, bool PARTIAL, int EPI, int W, int GSH, int KS = 1,
          bool CDMA = kCodeDma<BITS>>
hipError_t run(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
               const uint16_t* biases, const uint16_t* bias, uint16_t* y, float* partial,
               int64_t M, int64_t N, int64_t K, const Plan& p, hipStream_t stream) {
  const dim3 grid((unsigned)(p.tiles_n * p.tiles_m * p.splits));
  const int lds =
      KS * kXStages * 32 * MI * BK * 2 + (CDMA ? W * (KS > 1 ? 3 : kCodeSlots) * kCodeBlock : 0);
  auto kern = qmms_kernel<BITS, MI, PARTIAL, EPI, W, GSH, KS, CDMA>;
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, grid, dim3(64 * W), lds, stream,
                     x, wq, scales, biases, bias, y, partial, (int)M, (int)N, (int)K, p.tiles_n,
                     p.tiles_m, p.chunks_per_split);
  return hipGetLastError();
}

// one unsplit 32-row tile: the plan's block width
template <int BITS, int EPI, int GSH>
hipError_t run_wide(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                    const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                    int64_t N, int64_t K, const Plan& p, hipStream_t stream) {
  if constexpr (BITS == 4) {
    if (p.ks == 2) {
      switch (p.waves) {
        case 5: return run<BITS, 1, false, EPI, 10, GSH, 2, true>(x, wq, scales, biases, bias, y, nullptr, M, N, K, p, stream);
        case 6: return run<BITS, 1, false, EPI, 12, GSH, 2>(x, wq, scales, biases, bias, y, nullptr, M, N, K, p, stream);
        case 8: return run<BITS, 1, false, EPI, 16, GSH, 2>(x, wq, scales, biases, bias, y, nullptr, M, N, K, p, stream);
        default: return hipErrorInvalidValue;
      }
    }
  }
  switch (p.waves) {
    case 5: return run<BITS, 1, false, EPI, 5, GSH>(x, wq, scales, biases, bias, y, nullptr, M, N, K, p, stream);
    case 6: return run<BITS, 1, false, EPI, 6, GSH>(x, wq, scales, biases, bias, y, nullptr, M, N, K, p, stream);
    case 8: return run<BITS, 1, false, EPI, 8, GSH>(x, wq, scales, biases, bias, y, nullptr, M, N, K, p, stream);
    default: return run<BITS, 1, false, EPI, 4, GSH>(x, wq, scales, biases, bias, y, nullptr, M, N, K, p, stream);
  }
}

template <int BITS, bool PARTIAL, int GSH>
hipError_t run_mi(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                  const uint16_t* biases, const uint16_t* bias, uint16_t* y, float* partial,
                  int64_t M, int64_t N, int64_t K, const Plan& p, hipStream_t stream) {
  if constexpr (!PARTIAL)
    if (p.mi == 1) return run_wide<BITS, 0, GSH>(x, wq, scales, biases, bias, y, M, N, K, p, stream);
  switch (p.mi) {
    case 1: return run<BITS, 1, PARTIAL, 0, 4, GSH>(x, wq, scales, biases, bias, y, partial, M, N, K, p, stream);
    case 2: return run<BITS, 2, PARTIAL, 0, 4, GSH>(x, wq, scales, biases, bias, y, partial, M, N, K, p, stream);
    default: return run<BITS, 4, PARTIAL, 0, 4, GSH>(x, wq, scales, biases, bias, y, partial, M, N, K, p, stream);
  }
}

// f(std::integral_constant<int, GSH>) for group size 32 << GSH
template <class F>
hipError_t by_group(int group_size, F&& f) {
  switch (group_size) {
    case 32: return f(std::integral_constant<int, 0>{});
    case 64: return f(std::integral_constant<int, 1>{});
    case 128: return f(std::integral_constant<int, 2>{});
    default: return hipErrorInvalidValue;
  }
}

// the skinny kernel over the plan p (split or not) for 4- or 8-bit codes
template <bool PARTIAL>
hipError_t run_plan(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                    const uint16_t* biases, const uint16_t* bias, uint16_t* y, float* partial,
                    int64_t M, int64_t N, int64_t K, int bits, int group_size, const Plan& p,
                    hipStream_t stream) {
  return by_group(group_size, [&](auto g) {
    constexpr int GSH = decltype(g)::value;
    return bits == 4 ? run_mi<4, PARTIAL, GSH>(x, wq, scales, biases, bias, y, partial, M, N, K, p,
                                               stream)
                     : run_mi<8, PARTIAL, GSH>(x, wq, scales, biases, bias, y, partial, M, N, K, p,
                                               stream);
  });
}

}  // namespace

hipError_t launch_splitk_reduce(const float* partial, int splits, const uint16_t* bias,
                                uint16_t* y, int64_t MN, int64_t N, hipStream_t stream) {
  hipLaunchKernelGGL(splitk_reduce, dim3((unsigned)((MN + 255) / 256)), dim3(256), 0, stream,
                     partial, splits, bias, y, MN, (int)N);
  return hipGetLastError();
}

bool qmms_fits(int64_t M, int64_t N, int64_t K, int bits) {
  const int64_t lim = (int64_t)1 << 31;
  // whole 8-step chunks; 32-bit offsets with room for the tiles' overhang
  // (up to 256 columns for the widest blocks), scales for group size 32
  return K % (BK * kChunk) == 0 && M >= 1 && (M + 128) * K * 2 < lim &&
         (N + 256) * K * bits / 8 < lim && (N + 256) * (K / 32) * 2 < lim;
}

size_t qmms_workspace_bytes(int64_t M, int64_t N, int64_t K, int bits) {
  const Plan p = plan(M, N, K, bits, true);
  return p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
}

// The fused reduces need the split plan (the kernels' partial sums).
bool qmms_split_fusable(int64_t M, int64_t N, int64_t K, int bits) {
  return qmms_fits(M, N, K, bits) && plan(M, N, K, bits, true).splits > 1;
}

// The unsplit one-tile plan of the 2*Nout-row matrix: the SwiGLU in the
// GEMM's own epilogue (no workspace, no reduce).
bool qmms_swiglu_direct(int64_t M, int64_t Nout, int64_t K, int bits) {
  if (!qmms_fits(M, 2 * Nout, K, bits)) return false;
  const Plan p = plan(M, 2 * Nout, K, bits, true);
  return p.splits == 1 && p.mi == 1 && p.tiles_m == 1;
}

hipError_t launch_qmms_swiglu_direct(const uint16_t* x, const uint32_t* wq,
                                     const uint16_t* scales, const uint16_t* biases, uint16_t* y,
                                     int64_t M, int64_t Nout, int64_t K, int bits, int group_size,
                                     hipStream_t stream) {
  if (M == 0 || Nout == 0) return hipSuccess;
  Plan p = plan(M, 2 * Nout, K, bits, true);
  if (p.splits != 1 || p.mi != 1 || p.tiles_m != 1) return hipErrorInvalidValue;
  // 16 gate + 16 up columns per wave
  p.tiles_n = (int)((Nout + 16 * p.waves - 1) / (16 * p.waves));
  return by_group(group_size, [&](auto g) {
    constexpr int GSH = decltype(g)::value;
    return bits == 4
               ? run_wide<4, 1, GSH>(x, wq, scales, biases, nullptr, y, M, 2 * Nout, K, p, stream)
               : run_wide<8, 1, GSH>(x, wq, scales, biases, nullptr, y, M, 2 * Nout, K, p, stream);
  });
}

hipError_t launch_qmms_swiglu(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                              const uint16_t* biases, uint16_t* y, int64_t M, int64_t Nout,
                              int64_t K, int bits, int group_size, void* workspace,
                              size_t workspace_bytes, hipStream_t stream) {
  if (M == 0 || Nout == 0) return hipSuccess;
  const int64_t N = 2 * Nout;
  const Plan p = plan(M, N, K, bits, true);
  if (p.splits < 2 || !workspace || workspace_bytes < (size_t)p.splits * M * N * sizeof(float))
    return hipErrorInvalidValue;  // excluded by the caller's checks
  float* part = static_cast<float*>(workspace);
  const hipError_t e = run_plan<true>(x, wq, scales, biases, nullptr, nullptr, part, M, N, K, bits,
                                      group_size, p, stream);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(splitk_reduce_swiglu, dim3((unsigned)((M * Nout + 255) / 256)), dim3(256), 0,
                     stream, part, p.splits, y, M, (int)Nout);
  return hipGetLastError();
}

hipError_t launch_qmms_add_norm(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                                const uint16_t* biases, const uint16_t* bias,
                                const uint16_t* residual, uint16_t* residual_out,
                                const uint16_t* norm_w, float eps, uint16_t* out, int64_t M,
                                int64_t N, int64_t K, int bits, int group_size, void* workspace,
                                size_t workspace_bytes, hipStream_t stream) {
  if (M == 0 || N == 0) return hipSuccess;
  const Plan p = plan(M, N, K, bits, true);
  if (p.splits < 2 || !workspace || workspace_bytes < (size_t)p.splits * M * N * sizeof(float))
    return hipErrorInvalidValue;  // excluded by the caller's checks
  float* part = static_cast<float*>(workspace);
  const hipError_t e = run_plan<true>(x, wq, scales, biases, nullptr, nullptr, part, M, N, K, bits,
                                      group_size, p, stream);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(splitk_reduce_add_norm, dim3((unsigned)M), dim3(256), 0, stream, part,
                     p.splits, bias, residual, residual_out, norm_w, out, M, (int)N, eps);
  return hipGetLastError();
}

hipError_t launch_qmms(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                       int64_t N, int64_t K, int bits, int group_size, void* workspace,
                       size_t workspace_bytes, hipStream_t stream) {
  if (M == 0 || N == 0) return hipSuccess;
  Plan p = plan(M, N, K, bits, true);
  if (p.splits > 1 && (!workspace || workspace_bytes < (size_t)p.splits * M * N * sizeof(float)))
    p = plan(M, N, K, bits, false);
  if (p.splits == 1)
    return run_plan<false>(x, wq, scales, biases, bias, y, nullptr, M, N, K, bits, group_size, p,
                           stream);
  float* part = static_cast<float*>(workspace);
  hipError_t e = run_plan<true>(x, wq, scales, biases, bias, y, part, M, N, K, bits, group_size,
                                p, stream);
  if (e != hipSuccess) return e;
  return launch_splitk_reduce(part, p.splits, bias, y, M * N, N, stream);
}

}  // namespace mq
