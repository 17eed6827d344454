// One-row 4-bit GEMV, 16 lanes per row (K a multiple of 512, at most 4096, or
// the long rows of down projections), group sizes 32, 64 and 128:
// y[n] = x . (s*q + b)[n], as every decode-time
// QuantizedLinear calls mx.quantized_matmul(x, w, scales, biases,
// transpose=True) with one activation row
// (python/mlx_worker/native_mlx/models/qwen2.py:76-78,115,134,227) -- gate and
// up projections of the 7B shape are each this call (K = 3584, N = 18944).
//
// The arithmetic is qmv_kernel's for 16 lanes per row (mq_qmv_kernel.h), term
// for term and in the same order, so the results are bit-identical to it; the
// kernel differs in when the scales and biases arrive:
//  * qmv_kernel requests a block's scale/bias DMA before its code loads, and a
//    vector-memory counter retires in issue order, so the first chunk's wait
//    also waits for the DMA.  Blocks that start later on a CU find their DMA
//    queued behind the earlier blocks' code loads (a per-wave timestamp trace
//    of the 7B gate GEMV: the prologue of a CU's fifth block ends ~2.3 us
//    after its first block's).  Here the DMA is issued after the lane's last
//    code load and the chunk contractions keep the raw dot products
//    d_j = sum x * (128 + q); s*d_j + (b - 128 s)*sum(x) is added at the end,
//    in chunk order, once the scales have landed.  Only x gates the first
//    contraction;
//  * every size that the general kernel takes at run time (lanes per row,
//    rows per lane group, group size, activation rows, the DMA operation
//    count) is a compile-time constant here.
// EPI 1: SiLU(gate) * up of a 2N-row gate|up matrix (qmv_kernel's EPI 1);
// NORM: x = RMSNorm(a (+ res)) * w computed by every block (qmv_kernel's
// NormIn).
#pragma once
#include <type_traits>

#include "mq_qmv_kernel.h"

namespace mq {
namespace qmv1 {

constexpr int kBlock = 256, TPR = 16, RPB = kBlock / TPR;

// Code loads a lane keeps in flight ahead of its contraction.  Rows of up to
// 8 chunks per lane run 4-19 blocks per CU, whose loads together fill the
// memory queue at 2; a down projection's long rows (K = 18944: 37 chunks per
// lane, 224 blocks, at most one per CU) need more per lane: measured on
// 3584 x 18944, 2 ahead 12.4 us, 4 ahead 10.1, 8 ahead 9.5, 12 ahead 9.9.
constexpr int lookahead(int S) { return S > 8 ? 8 : 2; }

template <int N_>
__device__ __forceinline__ void wait_vm() {
  __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N_) : "memory");
}

// vmcnt at the wait for chunk j: codes issued after it, plus the scale/bias
// DMA once it is issued (right after the last code load).
// (vmcnt holds 6 bits: a larger count waits for 63, more than it must.)
template <int N_>
__device__ __forceinline__ void wait_at_most() {
  wait_vm<(N_ < 63 ? N_ : 63)>();
}

// f(std::integral_constant<int, I>) for I = I0 .. N - 1, in order: the chunk
// loop with every index a compile-time constant (no unroll heuristics).
template <int I0, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I0 < N) {
    f(std::integral_constant<int, I0>{});
    static_for<I0 + 1, N>(f);
  }
}

// 2/3/5/6-bit codes: a chunk of 32 codes is BITS whole words of the row's
// LSB-first bit stream (code c at bits BITS*c .. BITS*c + BITS - 1), loaded
// with as few buffer loads as cover them.
template <int BITS>
constexpr int stream_loads() { return BITS == 5 || BITS == 6 ? 2 : 1; }

template <int BITS>
__device__ __forceinline__ void load_stream_chunk(uint32_t (&w)[BITS], rsrc_t r, uint32_t off) {
  if constexpr (BITS == 2) {
    const u32x2_t v = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kBufNT));
    w[0] = v[0], w[1] = v[1];
  } else if constexpr (BITS == 3) {
    typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
    const u32x3_t v = __builtin_bit_cast(u32x3_t, __builtin_amdgcn_raw_buffer_load_b96(r, off, 0, kBufNT));
    w[0] = v[0], w[1] = v[1], w[2] = v[2];
  } else {
    const u32x4_t a = buf_load16<kBufNT>(r, off);
    w[0] = a[0], w[1] = a[1], w[2] = a[2], w[3] = a[3];
    if constexpr (BITS == 5) {
      w[4] = __builtin_amdgcn_raw_buffer_load_b32(r, off + 16, 0, kBufNT);
    } else {
      const u32x2_t b = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, off + 16, 0, kBufNT));
      w[4] = b[0], w[5] = b[1];
    }
  }
}

// bf16 pair (128 + code c, 128 + code c + 4): the 4-bit kernel's pairing, so
// that x's pair-permuted LDS layout serves every width (c a compile-time
// constant after unrolling: a bit-field extract each, a funnel shift for a
// code that straddles two words).
template <int BITS>
__device__ __forceinline__ uint32_t stream_code(const uint32_t (&w)[BITS], int c) {
  const int bit = BITS * c, wi = bit >> 5, sh = bit & 31;
  if (sh + BITS <= 32) return __builtin_amdgcn_ubfe(w[wi], sh, BITS);
  return __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh), 0, BITS);
}
template <int BITS>
__device__ __forceinline__ uint32_t stream_pair(const uint32_t (&w)[BITS], int c) {
  return (stream_code<BITS>(w, c + 4) << 16) | stream_code<BITS>(w, c) | 0x43004300u;
}

// The four pairs (c, c + 4), c = 8g .. 8g + 3, of 8-code group g.  2 and 3
// bits: the group's 16 / 24 bits are spread so that its upper four codes
// sit 16 bits above the lower four (bits between them are never read), and
// each pair is then one shift and one mask-and-magic, as for 4 bits.  5 and 6
// bits: four codes are too wide for that, a bit-field extract per code.
template <int BITS>
__device__ __forceinline__ void stream_pairs(const uint32_t (&w)[BITS], int g, uint32_t (&p)[4]) {
  if constexpr (BITS == 2) {
    const uint32_t f = (g & 1) ? w[g >> 1] >> 16 : w[g >> 1] & 0xffffu;  // codes at 2i
    const uint32_t v = (f << 8) | f;  // code i + 4 at bit 16 + 2i
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = ((v >> (2 * i)) & 0x00030003u) | 0x43004300u;
  } else if constexpr (BITS == 3) {
    const int bit = 24 * g, wi = bit >> 5, sh = bit & 31;  // the group's 24 bits
    const uint32_t f = sh + 24 <= 32 ? w[wi] >> sh : __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh);
    // bits 0..11: codes 0..3; bits 16..27: codes 4..7 (f << 4's)
    const uint32_t v = (f & 0xfffu) | ((f << 4) & 0xfffff000u);
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = ((v >> (3 * i)) & 0x00070007u) | 0x43004300u;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = stream_pair<BITS>(w, 8 * g + i);
  }
}

// 100 MHz constant clock (s_memrealtime), read into scalar registers.
__device__ __forceinline__ uint64_t realtime() {
  uint64_t t;
  __asm__ volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t));
  return t;
}

// S chunks per lane (C = 16 S), EPI 0 / 1, NORM as in qmv_kernel; 2^GSH
// chunks per group (group sizes 32, 64, 128: GSH 0, 1, 2).  TRACE
// (measurement only, mq_qmv_trace): every wave also records the constant
// clock at entry, after the prologue's barrier and after its store, and the
// CU it ran on, into trace[wave][4].
template <int S, int EPI, bool NORM, int GSH, bool TRACE = false, int BITS = 4>
__global__ __launch_bounds__(kBlock) void qmv1_kernel(const uint16_t* x, const uint32_t* wq,
                                                      const uint16_t* scales,
                                                      const uint16_t* biases,
                                                      const uint16_t* bias, uint16_t* y, int N,
                                                      qmv::NormIn nrm, uint64_t* trace) {
  uint64_t t0 = 0, t1 = 0;
  if constexpr (TRACE) t0 = realtime();
  constexpr int C = 16 * S, G = C >> GSH;       // chunks, groups per row
  constexpr int K = 32 * C;
  constexpr int XU = (4 * C + kBlock - 1) / kBlock;
  constexpr int HALF = RPB / 2;
  // codes issued before the loop; the RMSNorm forms issue every chunk first,
  // so the weight stream runs while the block reduces the norm
  constexpr int D = NORM || lookahead(S) >= S ? S : lookahead(S);
  constexpr int SB_WORDS = (RPB * G + G + 1) / 2;     // qmv_kernel's LDS layout (GP = G)
  constexpr int OPS = (SB_WORDS + 63) / 64;           // DMA operations per array
  constexpr int NQ = (2 * OPS + kBlock / 64 - 1) / (kBlock / 64);  // per wave
  static_assert(BITS == 4 || (EPI == 0 && !NORM), "2/3/5/6 bits: the plain form");
  constexpr int NL = BITS == 4 ? 1 : stream_loads<BITS>();  // code loads per chunk
  constexpr int CB = 4 * BITS;                                // code bytes per chunk
  extern __shared__ u32x4_t smem[];
  __shared__ float red[EPI == 1 ? RPB : 1];

  const int slot = threadIdx.x / TPR;
  const int lane = threadIdx.x % TPR;
  const int rb0 = blockIdx.x * (EPI == 1 ? HALF : RPB);
  const int rows_here = min(EPI == 1 ? HALF : RPB, N - rb0);
  const int span = EPI == 1 ? N + rows_here : rows_here;
  // EPI 1: local rows HALF.. are the up rows, N rows further on
  const int rel = EPI == 1 && slot >= HALF ? N - HALF + slot : slot;
  const rsrc_t xrs = make_rsrc(x, (uint64_t)K * 2);
  const rsrc_t wrs = make_rsrc(wq + (int64_t)rb0 * (C * BITS), (uint64_t)span * C * CB);
  const rsrc_t srs = make_rsrc(scales + (int64_t)rb0 * G, (uint64_t)span * G * 2);
  const rsrc_t brs = make_rsrc(biases + (int64_t)rb0 * G, (uint64_t)span * G * 2);

  u32x4_t xr[XU];
#pragma unroll
  for (int k = 0; k < XU; ++k) {
    const int u = threadIdx.x + k * kBlock;
    xr[k] = buf_load16(xrs, u < 4 * C ? (uint32_t)u * 16 : kOutOfRange);
  }
  u32x4_t rr[NORM ? XU : 1], nw[NORM ? XU : 1];
  if constexpr (NORM) {
    const rsrc_t rrs = make_rsrc(nrm.res, nrm.res ? (uint64_t)K * 2 : 0);
    const rsrc_t wns = make_rsrc(nrm.w, (uint64_t)K * 2);
#pragma unroll
    for (int k = 0; k < XU; ++k) {
      const int u = threadIdx.x + k * kBlock;
      rr[k] = buf_load16(rrs, u < 4 * C ? (uint32_t)u * 16 : kOutOfRange);
    }
#pragma unroll
    for (int k = 0; k < XU; ++k) {
      const int u = threadIdx.x + k * kBlock;
      nw[k] = buf_load16(wns, u < 4 * C ? (uint32_t)u * 16 : kOutOfRange);
    }
  }
  u32x4_t* xl = smem;
  float* xsum = reinterpret_cast<float*>(smem + 4 * C);
  uint16_t* sl = reinterpret_cast<uint16_t*>(xsum + C);
  uint16_t* bl = sl + 2 * (OPS * 64);
  // scale/bias DMA: NQ operations per wave (the last repeated where the
  // waves' shares differ), 4 bytes per lane
  auto dma = [&]() {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), ln = threadIdx.x & 63;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int o = min(wave + q * (kBlock / 64), 2 * OPS - 1);
      const bool is_b = o >= OPS;
      const int oo = is_b ? o - OPS : o;
      uint16_t* dst = (is_b ? bl : sl) + oo * 128;
      const int w = oo * 64 + ln;
      const uint32_t src = EPI == 1 && 2 * w >= HALF * G ? (uint32_t)(2 * w + (N - HALF) * G) * 2
                                                          : (uint32_t)w * 4;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(is_b ? brs : srs,
                                               (__attribute__((address_space(3))) void*)dst, 4,
                                               src, 0, 0, 0);
    }
  };
  u32x4_t wv[BITS == 4 ? S : 1];
  // stream widths: a ring of the D + 1 chunks in flight (chunk j in slot
  // j % RING; chunk j + D is issued before chunk j is read, into another slot)
  constexpr int RING = D + 1;
  uint32_t ws[BITS == 4 ? 1 : RING][BITS == 4 ? 1 : BITS];
  auto issue = [&](int j) {
    __asm__ volatile("" ::: "memory");
    // rows past the matrix lie past the descriptor's range: zeros
    if constexpr (BITS == 4)
      wv[j] = buf_load16<kBufNT>(wrs, (uint32_t)((rel * C + lane + j * TPR) * 16));
    else
      load_stream_chunk<BITS>(ws[j % RING], wrs, (uint32_t)((rel * C + lane + j * TPR) * CB));
    __asm__ volatile("" ::: "memory");
  };
#pragma unroll
  for (int j = 0; j < D; ++j) issue(j);
  if constexpr (D >= S) dma();
  wait_vm<(D >= S ? D * NL + NQ : D * NL)>();  // x (and the norm's inputs) have landed

  if constexpr (NORM) {
    __shared__ float nred[kBlock / 64];
    const bool has_res = nrm.res != nullptr;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < XU; ++k) {
      const int u = threadIdx.x + k * kBlock;
      if (u < 4 * C) {
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
      if (u < 4 * C) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          xr[k][q] = pack_bf16x2(lo_bf16(xr[k][q]) * inv * lo_bf16(nw[k][q]),
                                 hi_bf16(xr[k][q]) * inv * hi_bf16(nw[k][q]));
      }
    }
  }

  // x in LDS as [slot j][unit h][lane], pair-permuted; chunk sums of x
#pragma unroll
  for (int k = 0; k < XU; ++k) {
    const int u = threadIdx.x + k * kBlock;
    const int c = u / 4, h = u % 4;
    const u32x4_t v = xr[k];
    float s8 = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) s8 += lo_bf16(v[q]) + hi_bf16(v[q]);
    const u32x4_t p = {(v[0] & 0xffffu) | (v[2] << 16), (v[0] >> 16) | (v[2] & 0xffff0000u),
                       (v[1] & 0xffffu) | (v[3] << 16), (v[1] >> 16) | (v[3] & 0xffff0000u)};
    s8 += dpp_f32<0xb1>(s8);
    s8 += dpp_f32<0x4e>(s8);
    if (u < 4 * C) {
      xl[((c / TPR) * 4 + h) * TPR + c % TPR] = p;
      if (h == 0) xsum[c] = s8;
    }
  }
  lds_barrier();
  if constexpr (TRACE) t1 = realtime();

  // contract chunk j after issuing chunk j + D; keep the raw dot products
  const qmv::Nibble nib;
  float dd[S];
  const u32x4_t* xlane = xl + lane;
  static_for<0, S>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    if constexpr (j + D < S) {
      issue(j + D);
      if constexpr (j + D == S - 1) dma();
    }
    wait_at_most<((S - 1 - j) < D ? (S - 1 - j) : D) * NL + (j >= S - 1 - D ? NQ : 0)>();
    u32x4_t xv[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) xv[h] = xlane[(j * 4 + h) * TPR];
    float d = 0.f;
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
      if constexpr (BITS == 4) {
        const uint32_t wd = wv[j][wi];
        d = dot2_bf16(nib.pair(wd), xv[wi][0], d);
        d = dot2_bf16(nib.pair(wd >> 4), xv[wi][1], d);
        d = dot2_bf16(nib.pair(wd >> 8), xv[wi][2], d);
        d = dot2_bf16(nib.pair(wd >> 12), xv[wi][3], d);
      } else {
        uint32_t pr[4];
        stream_pairs<BITS>(ws[j % RING], wi, pr);
#pragma unroll
        for (int i = 0; i < 4; ++i) d = dot2_bf16(pr[i], xv[wi][i], d);
      }
    }
    dd[j] = d;
  });
  wait_vm<0>();
  __syncthreads();  // every wave's share of the scales and biases has landed
  const float* xslane = xsum + lane;
  const uint16_t* slane = sl + slot * G + (lane >> GSH);
  const uint16_t* blane = bl + slot * G + (lane >> GSH);
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const float xs = xslane[j * TPR];
    const float sc = bf16_bits_to_f32(slane[j * (TPR >> GSH)]);
    const float bi = bf16_bits_to_f32(blane[j * (TPR >> GSH)]);
    acc = fmaf(sc, dd[j], acc);
    acc = fmaf(fmaf(-128.f, sc, bi), xs, acc);
  }
  acc = dpp_group_sum<TPR>(acc);
  if constexpr (EPI == 1) {
    if (lane == 0) red[slot] = bf16_bits_to_f32(f32_to_bf16_bits(acc));
    __syncthreads();
    const int o = threadIdx.x;
    if (o < rows_here) y[rb0 + o] = silu_mul_bf16(red[o], red[HALF + o]);
  } else {
    const int row = rb0 + slot;
    if (lane == 0 && slot < rows_here) {
      const float add = bias ? bf16_bits_to_f32(bias[row]) : 0.f;
      y[row] = (uint16_t)f32_to_bf16_bits(acc + add);
    }
  }
  if constexpr (TRACE) {
    const uint64_t t2 = realtime();
    uint32_t hw, xcc;
    __asm__ volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    __asm__ volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    const int l = threadIdx.x & 63;
    if (l < 4)
      trace[((uint64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6)) * 4 + l] =
          l == 0 ? t0 : l == 1 ? t1 : l == 2 ? t2 : (((uint64_t)xcc << 32) | hw);
  } else {
    (void)t0, (void)t1, (void)trace;
  }
}

template <int S, int EPI, bool NORM, int GSH, bool TRACE = false, int BITS = 4>
hipError_t run(const uint16_t* x, const uint32_t* wq, const uint16_t* s, const uint16_t* b,
               const uint16_t* bias, uint16_t* y, int64_t N, const qmv::NormIn& nrm,
               hipStream_t stream, uint64_t* trace = nullptr) {
  constexpr int C = 16 * S, G = C >> GSH;
  constexpr int OPS = ((RPB * G + G + 1) / 2 + 63) / 64;
  const size_t lds = (size_t)C * 64 + C * 4 + 2 * OPS * 256;
  const int64_t rows = EPI == 1 ? RPB / 2 : RPB;
  hipLaunchKernelGGL((qmv1_kernel<S, EPI, NORM, GSH, TRACE, BITS>),
                     dim3((unsigned)((N + rows - 1) / rows)), dim3(kBlock), lds, stream, x, wq, s,
                     b, bias, y, (int)N, nrm, trace);
  return hipGetLastError();
}

template <int EPI, bool NORM, int GSH>
hipError_t run_s(int S, const uint16_t* x, const uint32_t* wq, const uint16_t* s,
                 const uint16_t* b, const uint16_t* bias, uint16_t* y, int64_t N,
                 const qmv::NormIn& nrm, hipStream_t stream) {
  switch (S) {
    case 2: return run<2, EPI, NORM, GSH>(x, wq, s, b, bias, y, N, nrm, stream);
    case 3: return run<3, EPI, NORM, GSH>(x, wq, s, b, bias, y, N, nrm, stream);
    case 4: return run<4, EPI, NORM, GSH>(x, wq, s, b, bias, y, N, nrm, stream);
    case 5: return run<5, EPI, NORM, GSH>(x, wq, s, b, bias, y, N, nrm, stream);
    case 6: return run<6, EPI, NORM, GSH>(x, wq, s, b, bias, y, N, nrm, stream);
    case 7: return run<7, EPI, NORM, GSH>(x, wq, s, b, bias, y, N, nrm, stream);
    case 8: return run<8, EPI, NORM, GSH>(x, wq, s, b, bias, y, N, nrm, stream);
    default: break;
  }
  // long rows: the plain form at group size 64 or 128 (qmv1_plain_fits)
  if constexpr (EPI == 0 && !NORM && GSH > 0) {
    switch (S) {
      case 27: return run<27, EPI, NORM, GSH>(x, wq, s, b, bias, y, N, nrm, stream);
      case 28: return run<28, EPI, NORM, GSH>(x, wq, s, b, bias, y, N, nrm, stream);
      case 37: return run<37, EPI, NORM, GSH>(x, wq, s, b, bias, y, N, nrm, stream);
      default: break;
    }
  }
  return hipErrorInvalidValue;  // excluded by qmv1_fits / qmv1_plain_fits
}

template <int EPI, bool NORM>
hipError_t run_gs(int S, int group_size, const uint16_t* x, const uint32_t* wq,
                  const uint16_t* s, const uint16_t* b, const uint16_t* bias, uint16_t* y,
                  int64_t N, const qmv::NormIn& nrm, hipStream_t stream) {
  switch (group_size) {
    case 32: return run_s<EPI, NORM, 0>(S, x, wq, s, b, bias, y, N, nrm, stream);
    case 64: return run_s<EPI, NORM, 1>(S, x, wq, s, b, bias, y, N, nrm, stream);
    case 128: return run_s<EPI, NORM, 2>(S, x, wq, s, b, bias, y, N, nrm, stream);
    default: return hipErrorInvalidValue;  // excluded by qmv1_fits
  }
}

// The plain form at 2/3/5/6 bits: S chunks per lane (2..8, or a down
// projection's 27/28/37 at group size 64/128), group size 32 << GSH.
template <int BITS, int GSH>
hipError_t run_stream_s(int S, const uint16_t* x, const uint32_t* wq, const uint16_t* s,
                        const uint16_t* b, const uint16_t* bias, uint16_t* y, int64_t N,
                        hipStream_t stream) {
  const qmv::NormIn none{};
#define MQ_QMVS_S(SS) \
  case SS: return run<SS, 0, false, GSH, false, BITS>(x, wq, s, b, bias, y, N, none, stream);
  switch (S) {
    MQ_QMVS_S(2) MQ_QMVS_S(3) MQ_QMVS_S(4) MQ_QMVS_S(5) MQ_QMVS_S(6) MQ_QMVS_S(7) MQ_QMVS_S(8)
    default: break;
  }
  if constexpr (GSH > 0) {
    switch (S) {
      MQ_QMVS_S(27) MQ_QMVS_S(28) MQ_QMVS_S(37)
      default: break;
    }
  }
#undef MQ_QMVS_S
  return hipErrorInvalidValue;  // excluded by qmvs_fits
}

template <int BITS>
hipError_t run_stream(int S, int group_size, const uint16_t* x, const uint32_t* wq,
                      const uint16_t* s, const uint16_t* b, const uint16_t* bias, uint16_t* y,
                      int64_t N, hipStream_t stream) {
  switch (group_size) {
    case 32: return run_stream_s<BITS, 0>(S, x, wq, s, b, bias, y, N, stream);
    case 64: return run_stream_s<BITS, 1>(S, x, wq, s, b, bias, y, N, stream);
    case 128: return run_stream_s<BITS, 2>(S, x, wq, s, b, bias, y, N, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qmv1
}  // namespace mq
