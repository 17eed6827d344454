#pragma once
// Decode-shaped quantized matmul (qmv) kernel and launch templates: y[m, n] = sum_k x[m, k] * (s*q + b)[n, k]
// for a few activation rows (M <= 8).  This is mx.quantized_matmul(x, w, scales,
// biases, transpose=True) as called by every QuantizedLinear at decode
// (python/mlx_worker/native_mlx/models/qwen2.py:76-78,115,134,227), and, with a
// per-batch expert index, mx.gather_qmm for unsorted / few-row MoE calls
// (models/lfm2.py:176-187).
//
// HBM-bound: every weight byte is read once.  Design for gfx950:
//  * a weight row is TPR lanes wide; lane l owns 16-byte chunks l, l+TPR, ...
//    (32 4-bit or 16 8-bit codes per chunk), up to S chunks for each of its R
//    rows.  Loads are issued in the order they are consumed -- x, this block's
//    scales and biases, then the lane's weight chunks, D ahead of the one being
//    contracted -- so waiting for x (vmcnt counts in issue order) never waits
//    for weights, and the contraction of chunk j overlaps the arrival of
//    chunks j+1..j+D.  Every block of a large GEMV is resident at once and
//    the CU's memory queue is full for most of the kernel: issuing all chunks
//    up front would leave each wave stalled in that queue with its first
//    chunks landed, and all the arithmetic would follow the last load;
//  * x is staged once per block in LDS as [m][slot][unit][lane] (16-byte
//    units): consecutive lanes read consecutive addresses, and every slot/unit
//    offset is a compile-time immediate.  Chunk sums of x and the block's
//    scales and biases sit next to it.  Past the end of a row the LDS holds
//    zeros, so padded lanes contribute 0 with no per-lane test;
//  * 4-bit: ((word >> 4t) & 0x000F000F) | 0x43004300 (one v_and_or_b32 after
//    the shift) is a pair of bfloat16 numbers 128+q, exact, contracted with an
//    x pair by v_dot2_f32_bf16 (x stored pair-permuted: (x0,x4),(x1,x5),...);
//    the chunk result d = sum x*(128+q) becomes s*d + (b - 128*s)*sum(x),
//    equal to sum x*(s*q+b), right after the chunk's dot products;
//  * 8-bit: bytes -> float (v_cvt_f32_ubyte) -> bfloat16 pairs (exact for
//    q <= 255) -> v_dot2_f32_bf16 against natural x pairs; then s*d + b*sum(x);
//  * per-row partial sums are reduced across the TPR lanes with DPP (LDS across
//    waves when TPR > 64); float32 throughout, one bfloat16 rounding at the
//    store, where QuantizedLinear's "+ bias" is fused.
#include "mq_common.h"
#include "mq_internal.h"

namespace mq {
namespace qmv {


constexpr int kBlock = 256;
constexpr int kQmvLdsBudget = 48 * 1024;
// Two rows per lane group may use up to 52 KiB: still 3 blocks per CU.
constexpr int kTwoRowLdsBudget = 52 * 1024;
// Four rows per lane group (half the blocks) may use up to 56 KiB, 2 blocks
// per CU: the 4-bit K = 18944 GEMV (53 KiB) takes 11.5 us in 448 blocks of
// 8 rows against 12.1 us in 896 blocks of 4.
constexpr int kFourRowLdsBudget = 56 * 1024;
// Scale + bias DMA operations per wave: 2 arrays of ceil((RPB*G + GP) / 2)
// words in 64-word operations, over 4 waves (an instance issues the most it
// can need, capped here; four rows per lane group at K = 18944 need 11).
constexpr int kSbOpsPerWave = 12;
// Weight chunks a lane keeps in flight ahead of the one it contracts, per
// row count R (measured on the 4-bit K=3584 and K=18944 GEMVs: 2 for one
// row per lane group, 3 for two).
constexpr int lookahead(int rows) { return rows == 1 ? 2 : 3; }

// Opaque register constants: the mask in an SGPR and the bfloat16 magic in a
// VGPR let ((w >> s) & mask) | magic select v_and_or_b32 (gfx9 VOP3 encodings
// take no literal and at most one scalar operand).
struct Nibble {
  uint32_t mask, magic;
  __device__ __forceinline__ Nibble() {
    __asm__ volatile("s_mov_b32 %0, 0xf000f" : "=s"(mask));
    __asm__ volatile("v_mov_b32 %0, 0x43004300" : "=v"(magic));
  }
  __device__ __forceinline__ uint32_t pair(uint32_t w) const { return (w & mask) | magic; }
};

// NORM: x is not the GEMV's input but a row a (M = 1) that the block first
// turns into it, as the RMSNorm kernel (mq_rms_norm) does, bit for bit:
// h = bf16(a + res) (h = a without res), x = bf16(h * rsqrt(mean(h^2) + eps)
// * w), in that kernel's element mapping (thread t: 8-element units t, t+256,
// ...) and reduction order.  Block 0 stores h to res_out.
struct NormIn {
  const uint16_t* res;
  uint16_t* res_out;
  const uint16_t* w;
  float eps;
};

// EPI 0: y[m, n] = (x W^T)[m, n] (+ bias[n]).  EPI 1 (SwiGLU, the gate and up
// projections of a Qwen2 MLP as one matrix of 2N rows, gate rows first;
// with GATHER, every expert's matrix is 2N rows):
// y[m, n] = bf16(bf16(silu(g)) * u) with g, u the bfloat16 results of rows n
// and N + n -- a block computes RPB/2 gate rows and the matching up rows.
template <int BITS, int TPR, int R, int S, int MT, int XU, bool GATHER, int EPI, bool NORM>
// The input pointers are deliberately not __restrict__: with it the compiler
// may move their loads across the inline-asm barriers below (it proves the
// asm cannot touch restrict memory), which breaks the issue order the waits
// rely on.
__global__ __launch_bounds__(kBlock) void qmv_kernel(
    const uint16_t* x, const uint32_t* wq, const uint16_t* scales, const uint16_t* biases,
    const uint16_t* bias, uint16_t* y, int M, int N, int K,
    const int32_t* __restrict__ lhs, const int32_t* __restrict__ rhs, int64_t E,
    int64_t x_batches, NormIn nrm, int lcpg) {
  constexpr int EPC = 128 / BITS;      // elements per 16-byte chunk
  constexpr int UPC = EPC / 8;         // 8-element units per chunk (4 or 2)
  // Chunks per group, 1 << lcpg: 1, 2 or 4 at 4 bits and 2, 4 or 8 at 8 bits
  // for group sizes 32, 64 and 128 (TPR is a multiple of it).
  constexpr int CPG_MIN = 32 / EPC < 1 ? 1 : 32 / EPC;
  constexpr int SLOTS = kBlock / TPR;  // row slots per block
  constexpr int RPB = SLOTS * R;       // rows per block
  constexpr int WPR = TPR > 64 ? TPR / 64 : 1;  // waves per row (TPR > 64)
  constexpr int HALF = RPB / 2;        // SwiGLU: output rows per block
  static_assert(EPI == 0 || (WPR == 1 && RPB % 2 == 0), "SwiGLU epilogue layout");
  static_assert(!NORM || (!GATHER && MT == 1 && XU <= 4), "RMSNorm input: one row of <= 8192");
  extern __shared__ u32x4_t smem[];
  __shared__ float red[WPR > 1 ? kBlock / 64 * R * MT : EPI == 1 ? RPB * MT : 1];

  const int C = K / EPC;                // chunks per row
  const int G = C >> lcpg;              // groups per row
  const int NJ = (C + TPR - 1) / TPR;   // slots used (<= S)
  const int CP = NJ * TPR;              // chunks per row, padded
  const int GP = CP >> lcpg;            // groups per row, padded
  const int64_t t = blockIdx.y;
  int64_t xb = t, e = 0;
  const int slot = threadIdx.x / TPR;
  const int lane = threadIdx.x % TPR;
  // First weight row of the block (EPI 1: first gate row = first output row).
  const int rb0 = blockIdx.x * (EPI == 1 ? HALF : RPB);
  const int row0 = rb0 + slot * R;
  // Without gather tables nothing here waits on memory before the first
  // loads are issued: the index loads, their wait and the test would
  // otherwise precede every address computation.
  if constexpr (GATHER) {
    if (lhs) xb = lhs[t];
    if (rhs) e = rhs[t];
    y += t * (int64_t)M * N;
    if (xb < 0 || xb >= x_batches || e < 0 || e >= E) {  // index outside the tables: zeros
      if constexpr (EPI == 1) {
        const int o = threadIdx.x % HALF, m = threadIdx.x / HALF;
        if (m < M && rb0 + o < N) y[(int64_t)m * N + rb0 + o] = 0;
      } else if (lane == 0) {
        for (int r = 0; r < R; ++r)
          for (int m = 0; m < M; ++m)
            if (row0 + r < N) y[(int64_t)m * N + row0 + r] = 0;
      }
      return;
    }
  }
  // ---- 1. loads through buffer descriptors (out-of-range reads return 0):
  // x, the block's scales/biases (contiguous: the block's rows are
  // consecutive), then the first D weight chunks of this lane.  The rest are
  // issued one per chunk contracted (step 3): a CU's memory queue fills long
  // before every wave has issued all its loads, so a wave that issued them
  // all up front would sit in the queue with its first chunks already
  // landed, and the grid's arithmetic would pile up behind the last loads.
  constexpr int D = S < lookahead(R) ? S : lookahead(R);
  // Local row lr = slot*R + r lies rel(lr) rows past rb0: the block's rows
  // are consecutive, or (EPI 1) HALF gate rows and, N rows further, their up
  // rows.  Rows past the matrix read as zeros (out of the descriptor's range).
  const int rows_here = min(EPI == 1 ? HALF : RPB, N - rb0);
  const int span = EPI == 1 ? N + rows_here : rows_here;  // rows the descriptors cover
  auto rel = [&](int lr) { return EPI == 1 && lr >= HALF ? N - HALF + lr : lr; };
  const rsrc_t xrs = make_rsrc(x + xb * (int64_t)M * K, (uint64_t)M * K * 2);
  const int64_t erows = EPI == 1 ? 2 * (int64_t)N : N;  // rows of one expert's matrix
  const rsrc_t wrs = make_rsrc(wq + (e * erows + rb0) * (C * 4), (uint64_t)span * C * 16);
  const int64_t sb0 = e * erows * G + (int64_t)rb0 * G;
  const rsrc_t srs = make_rsrc(scales + sb0, (uint64_t)span * G * 2);
  const rsrc_t brs = make_rsrc(biases + sb0, (uint64_t)span * G * 2);

  const int x_units = MT * CP * UPC;  // padded 8-element units of x
  u32x4_t xr[XU];
#pragma unroll
  for (int k = 0; k < XU; ++k) {
    const int i = threadIdx.x + k * kBlock;
    const int m = MT == 1 ? 0 : i / (CP * UPC);
    const int u = i - m * (CP * UPC);  // unit within the row
    const bool real = m < M && u < C * UPC;
    xr[k] = buf_load16(xrs, real ? (uint32_t)(m * K + u * 8) * 2 : kOutOfRange);
  }
  u32x4_t rr[NORM ? XU : 1], nw[NORM ? XU : 1];  // residual and norm weight units
  if constexpr (NORM) {
    const rsrc_t rrs = make_rsrc(nrm.res, nrm.res ? (uint64_t)K * 2 : 0);
    const rsrc_t wns = make_rsrc(nrm.w, (uint64_t)K * 2);
#pragma unroll
    for (int k = 0; k < XU; ++k) {
      const int u = threadIdx.x + k * kBlock;
      rr[k] = buf_load16(rrs, u < C * UPC ? (uint32_t)u * 16 : kOutOfRange);
    }
#pragma unroll
    for (int k = 0; k < XU; ++k) {
      const int u = threadIdx.x + k * kBlock;
      nw[k] = buf_load16(wns, u < C * UPC ? (uint32_t)u * 16 : kOutOfRange);
    }
  }
  // Scales and biases go straight to LDS (buffer_load ... lds, 4 bytes per
  // lane).  Entries past the block's rows read as zeros.
  u32x4_t* xl = smem;
  float* xsum = reinterpret_cast<float*>(smem + MT * CP * UPC);
  uint16_t* sl = reinterpret_cast<uint16_t*>(xsum + MT * CP);  // [RPB*G + GP] scales
  const int sb_words = (RPB * G + GP + 1) / 2;                 // 32-bit words per array
  uint16_t* bl = sl + 2 * ((sb_words + 63) / 64 * 64);          // biases, same layout
  {
    // A fixed number of operations per wave, so that every wait below counts
    // exactly: the most this instance can need (a row has at most S*TPR
    // chunks, so RPB*G + GP <= (RPB + 1) * S*TPR/CPG entries, most at the
    // smallest group size); a wave stops after the operations this shape
    // needs, the last of them repeated where the waves' shares differ.  Each
    // is a VMEM instruction in a congested queue.
    constexpr int SB_WORDS_MAX = ((RPB + 1) * (S * TPR / CPG_MIN) + 1) / 2;
    constexpr int OPS_PER_WAVE = (2 * ((SB_WORDS_MAX + 63) / 64) + kBlock / 64 - 1) / (kBlock / 64);
    constexpr int NQ = OPS_PER_WAVE < kSbOpsPerWave ? OPS_PER_WAVE : kSbOpsPerWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), ln = threadIdx.x & 63;
    const int ops = (sb_words + 63) / 64;  // wave-wide 4-byte DMA operations per array
    const int nq = (2 * ops + kBlock / 64 - 1) / (kBlock / 64);  // <= NQ (checked on the host)
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if (q >= nq) break;  // uniform
      const int o = min(wave + q * (kBlock / 64), 2 * ops - 1);
      const bool is_b = o >= ops;
      const int oo = is_b ? o - ops : o;
      uint16_t* dst = (is_b ? bl : sl) + oo * 128;
      // Word w holds entries 2w, 2w+1 of one local row (G is even); EPI 1
      // moves the up half (w >= HALF*G/2, pad words included) N - HALF rows on.
      const int w = oo * 64 + ln;
      const uint32_t src = EPI == 1 && 2 * w >= HALF * G ? (uint32_t)(2 * w + (N - HALF) * G) * 2
                                                          : (uint32_t)w * 4;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(is_b ? brs : srs,
                                               (__attribute__((address_space(3))) void*)dst, 4,
                                               src, 0, 0, 0);
    }
  }
  // Weight chunk j of the lane's R rows; slots past NJ read nothing (out of
  // range: zeros), so every chunk is one straight-line load per row and the
  // waits below count exactly.  The empty asm statements pin the issue
  // order: vmcnt retires in issue order.
  u32x4_t wv[S][R];
  auto issue = [&](int j) {
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (int r = 0; r < R; ++r)
      wv[j][r] = buf_load16<kBufNT>(
          wrs, j < NJ ? (uint32_t)((rel(slot * R + r) * C + lane + j * TPR) * 16) : kOutOfRange);
    __asm__ volatile("" ::: "memory");
  };
#pragma unroll
  for (int j = 0; j < D; ++j) issue(j);
  // x and this wave's scale/bias DMA have landed once at most the D*R weight
  // loads are outstanding; the barrier below then publishes every wave's.
  __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(D * R) : "memory");

  if constexpr (NORM) {
    // ---- 1b. x = RMSNorm(a (+ res)) * w, as rmsnorm_kernel computes it.
    __shared__ float nred[kBlock / 64];
    const bool has_res = nrm.res != nullptr;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < XU; ++k) {
      const int u = threadIdx.x + k * kBlock;
      if (u < C * UPC) {
        u32x4_t v = xr[k];
        if (has_res) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            v[q] = pack_bf16x2(lo_bf16(v[q]) + lo_bf16(rr[k][q]), hi_bf16(v[q]) + hi_bf16(rr[k][q]));
          if (blockIdx.x == 0) reinterpret_cast<u32x4_t*>(nrm.res_out)[u] = v;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float a = lo_bf16(v[q]), b = hi_bf16(v[q]);
          ss = fmaf(a, a, ss);
          ss = fmaf(b, b, ss);
        }
        xr[k] = v;
      }
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) ss += __shfl_xor(ss, off, 64);
    if ((threadIdx.x & 63) == 0) nred[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int i = 0; i < kBlock / 64; ++i) ss += nred[i];
    const float inv = rsqrtf(ss / (float)K + nrm.eps);
#pragma unroll
    for (int k = 0; k < XU; ++k) {
      const int u = threadIdx.x + k * kBlock;
      if (u < C * UPC) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          xr[k][q] = pack_bf16x2(lo_bf16(xr[k][q]) * inv * lo_bf16(nw[k][q]),
                                 hi_bf16(xr[k][q]) * inv * hi_bf16(nw[k][q]));
      }
    }
  }

  // ---- 2. LDS: x as [m][slot j][unit h][lane] (4-bit pair-permuted) and
  // chunk sums [m][chunk]; zeros past the row.
#pragma unroll
  for (int k = 0; k < XU; ++k) {
    const int i = threadIdx.x + k * kBlock;
    if (k * kBlock >= x_units) break;  // uniform
    const int m = MT == 1 ? 0 : i / (CP * UPC);
    const int u = i - m * (CP * UPC);
    const int c = u / UPC, h = u % UPC;
    u32x4_t v = xr[k];
    float s8 = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) s8 += lo_bf16(v[q]) + hi_bf16(v[q]);
    if constexpr (BITS == 4) {
      const u32x4_t p = {(v[0] & 0xffffu) | (v[2] << 16), (v[0] >> 16) | (v[2] & 0xffff0000u),
                         (v[1] & 0xffffu) | (v[3] << 16), (v[1] >> 16) | (v[3] & 0xffff0000u)};
      v = p;
    }
    s8 += dpp_f32<0xb1>(s8);  // the UPC (2 or 4) consecutive units of a chunk
    if constexpr (UPC == 4) s8 += dpp_f32<0x4e>(s8);
    if (i < x_units) {
      xl[((m * NJ + c / TPR) * UPC + h) * TPR + c % TPR] = v;
      if (h == 0) xsum[m * CP + c] = s8;
    }
  }
  lds_barrier();

  // ---- 3. contract: chunk j, then its scale/bias epilogue, after issuing
  // chunk j + D.  Straight-line over all S chunks and MT rows so that the
  // wait before chunk j covers chunks <= j only: rows m >= M are zeros in
  // LDS; chunks past NJ (only when S > NJ) read a valid chunk and are masked
  // out.
  const Nibble nib;
  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

  const u32x4_t* xlane = xl + lane;
  const float* xslane = xsum + lane;
  const uint16_t* slane = sl + slot * R * G + (lane >> lcpg);
  const uint16_t* blane = bl + slot * R * G + (lane >> lcpg);
  const int gstep = TPR >> lcpg;  // groups per chunk slot
#pragma unroll
  for (int j = 0; j < S; ++j) {
    if (j + D < S) issue(j + D);
    const int jj = j < NJ ? j : NJ - 1;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      u32x4_t xv[UPC];
#pragma unroll
      for (int h = 0; h < UPC; ++h) xv[h] = xlane[((m * NJ + jj) * UPC + h) * TPR];
      const float xs = xslane[m * CP + jj * TPR];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float d = 0.f;
        if constexpr (BITS == 4) {
#pragma unroll
          for (int wi = 0; wi < 4; ++wi) {
            const uint32_t wd = wv[j][r][wi];
            d = dot2_bf16(nib.pair(wd), xv[wi][0], d);
            d = dot2_bf16(nib.pair(wd >> 4), xv[wi][1], d);
            d = dot2_bf16(nib.pair(wd >> 8), xv[wi][2], d);
            d = dot2_bf16(nib.pair(wd >> 12), xv[wi][3], d);
          }
        } else {
#pragma unroll
          for (int wi = 0; wi < 4; ++wi) {
            const uint32_t wd = wv[j][r][wi];
            d = dot2_bf16(pack_bf16x2(ubyte_f32<0>(wd), ubyte_f32<1>(wd)),
                          xv[wi / 2][(wi % 2) * 2], d);
            d = dot2_bf16(pack_bf16x2(ubyte_f32<2>(wd), ubyte_f32<3>(wd)),
                          xv[wi / 2][(wi % 2) * 2 + 1], d);
          }
        }
        const float sc = bf16_bits_to_f32(slane[r * G + jj * gstep]);
        const float bi = bf16_bits_to_f32(blane[r * G + jj * gstep]);
        if (j < NJ && m < M) {  // uniform
          if constexpr (BITS == 4) {
            acc[r][m] = fmaf(sc, d, acc[r][m]);
            acc[r][m] = fmaf(fmaf(-128.f, sc, bi), xs, acc[r][m]);
          } else {
            acc[r][m] = fmaf(sc, d, acc[r][m]);
            acc[r][m] = fmaf(bi, xs, acc[r][m]);
          }
        }
      }
    }
  }

  // ---- 4. reduce across the TPR lanes of each row, store ----
  constexpr int W = TPR < 64 ? TPR : 64;
  constexpr int SUM_LANE = dpp_sum_lane<W>();
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = dpp_group_sum<W>(acc[r][m]);

  if constexpr (EPI == 1) {
    // g and u rounded to bfloat16 as the GEMV would store them, then
    // silu_mul's arithmetic on the pair.
    if (lane % W == SUM_LANE) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m)
          red[m * RPB + slot * R + r] = bf16_bits_to_f32(f32_to_bf16_bits(acc[r][m]));
    }
    __syncthreads();
    const int o = threadIdx.x % HALF, m = threadIdx.x / HALF;
    if (m < M && m < MT && o < rows_here)
      y[(int64_t)m * N + rb0 + o] = silu_mul_bf16(red[m * RPB + o], red[m * RPB + HALF + o]);
  } else if constexpr (WPR == 1) {
    if (lane % W == SUM_LANE) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        if (row >= N) continue;
        const float add = bias ? bf16_bits_to_f32(bias[row]) : 0.f;
#pragma unroll
        for (int m = 0; m < MT; ++m)
          if (m < M) y[(int64_t)m * N + row] = (uint16_t)f32_to_bf16_bits(acc[r][m] + add);
      }
    }
  } else {
    const int wave = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 63) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) red[(wave * R + r) * MT + m] = acc[r][m];
    }
    __syncthreads();
    if (lane == 0) {
      const int w0 = slot * WPR;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        if (row >= N) continue;
        const float add = bias ? bf16_bits_to_f32(bias[row]) : 0.f;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          float v = 0.f;
#pragma unroll
          for (int w = 0; w < WPR; ++w) v += red[((w0 + w) * R + r) * MT + m];
          if (m < M) y[(int64_t)m * N + row] = (uint16_t)f32_to_bf16_bits(v + add);
        }
      }
    }
  }
}

// x units, chunk sums, then scales and biases: each array ceil((RPB*G + GP) / 2)
// words rounded up to whole 64-lane DMA operations.
inline int64_t lds_bytes(int bits, int tpr, int64_t MT, int64_t K, int R, int gs) {
  const int epc = 128 / bits;
  const int64_t C = K / epc;
  const int64_t CP = (C + tpr - 1) / tpr * tpr;
  const int64_t G = K / gs;
  const int64_t GP = CP / (gs / epc);
  const int64_t RPB = (kBlock / tpr) * R;
  const int64_t sb_words = (RPB * G + GP + 1) / 2;
  return MT * CP * 16 * (epc / 8) + MT * CP * 4 + 2 * ((sb_words + 63) / 64) * 256;
}

template <int BITS, int TPR, int R, int S, int MT, int XU, bool GATHER, int EPI, bool NORM>
hipError_t run(const uint16_t* x, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
               const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K,
               const GatherMap& g, const NormIn& nrm, int gs, hipStream_t stream) {
  const int64_t rows_per_block = (kBlock / TPR) * R / (EPI == 1 ? 2 : 1);
  const size_t lds = (size_t)lds_bytes(BITS, TPR, MT, K, R, gs);
  const dim3 grid((unsigned)((N + rows_per_block - 1) / rows_per_block), (unsigned)g.T);
  const int lcpg = __builtin_ctz((unsigned)(gs / (128 / BITS)));  // log2 chunks per group
  hipLaunchKernelGGL((qmv_kernel<BITS, TPR, R, S, MT, XU, GATHER, EPI, NORM>), grid, dim3(kBlock),
                     lds, stream, x, wq, s, b, bias, y, (int)M, (int)N, (int)K, g.lhs, g.rhs, g.E,
                     g.x_batches, nrm, lcpg);
  return hipGetLastError();
}

template <int BITS, int TPR, int R, int S, int MT, bool GATHER, int EPI, bool NORM>
hipError_t run_xu(const uint16_t* x, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                  const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K,
                  const GatherMap& g, const NormIn& nrm, int gs, hipStream_t stream) {
  constexpr int EPC = 128 / BITS;
  const int64_t CP = (K / EPC + TPR - 1) / TPR * TPR;
  const int64_t units = (MT * CP * (EPC / 8) + kBlock - 1) / kBlock;  // x units per thread
  if (units <= 2)
    return run<BITS, TPR, R, S, MT, 2, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs,
                                                          stream);
  if (units <= 4)
    return run<BITS, TPR, R, S, MT, 4, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs,
                                                          stream);
  if constexpr (NORM) {
    return hipErrorInvalidValue;  // rows of <= 8192 (excluded by qmv_norm_fits)
  } else {
    if (units <= 12)
      return run<BITS, TPR, R, S, MT, 12, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs,
                                                             stream);
    return hipErrorInvalidValue;  // excluded by qmv_fits
  }
}

template <int BITS, int TPR, int R, int S, bool GATHER, int EPI, bool NORM>
hipError_t run_mt(const uint16_t* x, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                  const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K,
                  const GatherMap& g, const NormIn& nrm, int gs, hipStream_t stream) {
  if (M <= 1)
    return run_xu<BITS, TPR, R, S, 1, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs,
                                                         stream);
  if constexpr (NORM) {
    return hipErrorInvalidValue;  // one row (excluded by qmv_norm_fits)
  } else {
    if (M <= 2)
      return run_xu<BITS, TPR, R, S, 2, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs,
                                                           stream);
    if constexpr (EPI == 1) {
      return hipErrorInvalidValue;  // SwiGLU: M <= 2 (excluded by qmv_swiglu_fits)
    } else {
      if (M <= 4)
        return run_xu<BITS, TPR, R, S, 4, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g,
                                                             nrm, gs, stream);
      return run_xu<BITS, TPR, R, S, 8, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs,
                                                           stream);
    }
  }
}

inline constexpr int kTprs[] = {8, 16, 32, 64, 128, 256};

// Lanes per row: the narrowest whose lanes own at most 8 chunks each, widened
// while the grid has fewer than 2 blocks per CU.  8 lanes only for short rows
// (<= 24 chunks: 3 slots), where 16 lanes would leave a quarter of the slots
// empty (an expert's down projection, K = 768).
inline int pick_tpr(int64_t C, int64_t N, int64_t T) {
  int pick = C <= 24 ? 0 : 1;
  while (pick < 5 && (C + kTprs[pick] - 1) / kTprs[pick] > 8) ++pick;
  while (pick < 5 && ((N * kTprs[pick]) / kBlock) * T < 512) ++pick;
  return kTprs[pick];
}

// R rows per lane group needs the scales to fit the block's LDS DMA budget
// (RPB * G + GP entries per array, kSbOpsPerWave operations per wave), the
// LDS budget, and at least min_blocks blocks.
inline bool rows_fit(int R, int bits, int tpr, int64_t M, int64_t N, int64_t K, int64_t T,
                     int64_t min_blocks, int gs) {
  const int epc = 128 / bits;
  const int64_t C = K / epc, G = K / gs;
  const int64_t CP = (C + tpr - 1) / tpr * tpr, GP = CP / (gs / epc);
  const int64_t rpb = (kBlock / tpr) * R;
  const int64_t mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  const int64_t sb_words = (rpb * G + GP + 1) / 2;
  return 2 * ((sb_words + 63) / 64) <= kSbOpsPerWave * (kBlock / 64) &&
         lds_bytes(bits, tpr, mt, K, R, gs) <= (R >= 4 ? kFourRowLdsBudget : kTwoRowLdsBudget) &&
         (N + rpb - 1) / rpb * T >= min_blocks;
}

// Launches the GEMV for one code width; GATHER selects the kernels that
// read per-batch x / expert indices, EPI the SwiGLU epilogue (N output rows
// of a 2N-row matrix), NORM the RMSNorm input (see NormIn).  Each
// instantiation lives in a translation unit of its own (mq_qmv*.hip), so that
// they compile in parallel.
template <int BITS, bool GATHER, int EPI, bool NORM>
hipError_t run_bits(const uint16_t* x, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
                    const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K,
                    const GatherMap& g, const NormIn& nrm, int gs, hipStream_t stream) {
  constexpr int EPC = 128 / BITS;
  const int64_t C = K / EPC;
  const int tpr = pick_tpr(C, EPI == 1 ? 2 * N : N, g.T);
  const int slots = (int)((C + tpr - 1) / tpr);
  switch (tpr) {
    case 8:
      return run_mt<BITS, 8, 1, 3, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
    // Chunk slots per lane S: the instantiated S >= NJ closest to it (slots
    // past NJ cost arithmetic on zeros, not memory traffic).  The S values
    // cover the model shapes exactly: K = 3584 / 18944 / 2048 / 768 at 4 and
    // 8 bits.
    case 16:
      if (slots <= 2) return run_mt<BITS, 16, 1, 2, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
      if (slots <= 3) return run_mt<BITS, 16, 1, 3, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
      if (slots <= 4) return run_mt<BITS, 16, 1, 4, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
      if (slots <= 7) return run_mt<BITS, 16, 1, 7, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
      return run_mt<BITS, 16, 1, 8, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
    case 32:
      if (slots <= 4) return run_mt<BITS, 32, 1, 4, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
      if (slots <= 7) return run_mt<BITS, 32, 1, 7, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
      return run_mt<BITS, 32, 1, 8, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
    case 64:
      if (slots <= 5) return run_mt<BITS, 64, 1, 5, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
      return run_mt<BITS, 64, 1, 8, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
    default:
      if constexpr (EPI == 1) {
        return hipErrorInvalidValue;  // SwiGLU: one wave per row at most
      } else {
        if (tpr == 128) {
          // More rows per lane group while the blocks still fill the GPU: a
          // block stages all of x (long rows: up to 40 KB), so rows per block
          // divide that L2 traffic, and fewer blocks fit one round of
          // residency (2 or 3 per CU at these LDS sizes).
          if (slots <= 5 && M == 1 && rows_fit(4, BITS, 128, M, N, K, g.T, 256, gs))
            return run_mt<BITS, 128, 4, 5, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
          if (slots <= 5 && rows_fit(2, BITS, 128, M, N, K, g.T, 512, gs))
            return run_mt<BITS, 128, 2, 5, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
          if (slots <= 5) return run_mt<BITS, 128, 1, 5, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
          return run_mt<BITS, 128, 1, 8, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
        }
        if (slots <= 3) return run_mt<BITS, 256, 1, 3, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
        if (slots <= 5) return run_mt<BITS, 256, 1, 5, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
        if (slots <= 8) return run_mt<BITS, 256, 1, 8, GATHER, EPI, NORM>(x, wq, s, b, bias, y, M, N, K, g, nrm, gs, stream);
        return hipErrorInvalidValue;  // excluded by qmv_fits
      }
  }
}

}  // namespace qmv
}  // namespace mq

// Explicit instantiation (or, after `extern`, its declaration) of one
// run_bits launch, inside namespace mq.
#define MQ_QMV_INSTANCE(BITS, GATHER, EPI, NORM)                                             \
  template hipError_t qmv::run_bits<BITS, GATHER, EPI, NORM>(                               \
      const uint16_t*, const uint32_t*, const uint16_t*, const uint16_t*, const uint16_t*, \
      uint16_t*, int64_t, int64_t, int64_t, const GatherMap&, const qmv::NormIn&, int,     \
      hipStream_t)
