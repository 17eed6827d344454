// One-row GEMV dispatch: the shapes the kernel of mq_qmv1_kernel.h takes and
// its 4-bit launches (mq_qmvs_b*.hip instantiate the 2/3/5/6-bit ones).
#include "../../include/mq.h"
#include "../../include/mq_measure.h"
#include "mq_qmv1_kernel.h"

namespace mq {

// One activation row, 4-bit codes, group size 32, 64 or 128, K a multiple of 512 from
// 1024 to 4096 (2 to 8 chunks per lane), 32-bit code offsets: every form.  Where
// qmv_kernel itself would run 16 lanes per row (large matrices) the results
// are its own, bit for bit; on smaller matrices (where the dispatch used to
// take the matrix-core GEMV or qmv_kernel with wider rows) this kernel is the
// faster one too: 3584 -> 4608 5.9 -> 4.7 us, 3584 -> 3584 4.4 -> 4.0 us,
// 3584 -> 9216 7.7 -> 5.6 us.  rows: the rows of the matrix (2N for the
// SwiGLU form).
bool qmv1_fits(int64_t M, int64_t rows, int64_t K, int bits, int group_size) {
  if (M != 1 || bits != 4 || K % 512 || K < 1024 || K > 4096) return false;
  if (group_size != 32 && group_size != 64 && group_size != 128) return false;
  return rows >= 1 && rows * (K / 32) * 16 < (int64_t(1) << 32) && rows < (int64_t(1) << 30);
}

// The plain form also takes the long rows of decoders' down projections --
// K = 13824, 14336, 18944 (27, 28, 37 chunks per lane) -- at group size 64 or
// 128 (at group size 32, or 54 chunks, the kernel spills registers).  Measured on
// 3584 x 18944 (the 7B down projection): 9.5 us against 11.7 for qmv_kernel
// (128 lanes per row), group 128 9.2 against 11.5.
bool qmv1_plain_fits(int64_t M, int64_t rows, int64_t K, int bits, int group_size) {
  if (qmv1_fits(M, rows, K, bits, group_size)) return true;
  const int64_t S = K / 512;
  if (M != 1 || bits != 4 || K % 512 || (group_size != 64 && group_size != 128) ||
      (S != 27 && S != 28 && S != 37))
    return false;
  return rows >= 1 && rows * (K / 32) * 16 < (int64_t(1) << 32) && rows < (int64_t(1) << 30);
}

bool qmvs_fits(int64_t M, int64_t rows, int64_t K, int bits, int group_size) {
  if (bits != 2 && bits != 3 && bits != 5 && bits != 6) return false;
  // the 4-bit shapes, the code bytes of a row at this width
  return qmv1_plain_fits(M, rows, K, 4, group_size) &&
         rows * (K / 32) * 4 * bits < (int64_t(1) << 32);
}

hipError_t launch_qmvs_b2(int S, int group_size, const uint16_t* x, const uint32_t* wq,
                          const uint16_t* scales, const uint16_t* biases, const uint16_t* bias,
                          uint16_t* y, int64_t N, hipStream_t stream);
hipError_t launch_qmvs_b3(int S, int group_size, const uint16_t* x, const uint32_t* wq,
                          const uint16_t* scales, const uint16_t* biases, const uint16_t* bias,
                          uint16_t* y, int64_t N, hipStream_t stream);
hipError_t launch_qmvs_b5(int S, int group_size, const uint16_t* x, const uint32_t* wq,
                          const uint16_t* scales, const uint16_t* biases, const uint16_t* bias,
                          uint16_t* y, int64_t N, hipStream_t stream);
hipError_t launch_qmvs_b6(int S, int group_size, const uint16_t* x, const uint32_t* wq,
                          const uint16_t* scales, const uint16_t* biases, const uint16_t* bias,
                          uint16_t* y, int64_t N, hipStream_t stream);

hipError_t launch_qmvs(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t N,
                       int64_t K, int bits, int group_size, hipStream_t stream) {
  if (N == 0) return hipSuccess;
  const int S = (int)(K / 512);
  switch (bits) {
    case 2: return launch_qmvs_b2(S, group_size, x, wq, scales, biases, bias, y, N, stream);
    case 3: return launch_qmvs_b3(S, group_size, x, wq, scales, biases, bias, y, N, stream);
    case 5: return launch_qmvs_b5(S, group_size, x, wq, scales, biases, bias, y, N, stream);
    case 6: return launch_qmvs_b6(S, group_size, x, wq, scales, biases, bias, y, N, stream);
    default: return hipErrorInvalidValue;  // excluded by qmvs_fits
  }
}

hipError_t launch_qmv1(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                       const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t N,
                       int64_t K, int group_size, bool swiglu, const qmv::NormIn* nrm,
                       hipStream_t stream) {
  if (N == 0) return hipSuccess;
  const int S = (int)(K / 512);
  const qmv::NormIn none{};
  if (nrm)
    return swiglu ? qmv1::run_gs<1, true>(S, group_size, x, wq, scales, biases, nullptr, y, N,
                                          *nrm, stream)
                  : qmv1::run_gs<0, true>(S, group_size, x, wq, scales, biases, bias, y, N, *nrm,
                                          stream);
  return swiglu ? qmv1::run_gs<1, false>(S, group_size, x, wq, scales, biases, nullptr, y, N,
                                         none, stream)
                : qmv1::run_gs<0, false>(S, group_size, x, wq, scales, biases, bias, y, N, none,
                                         stream);
}

// The traced plain form: 4 uint64 per wave (entry, after the prologue's
// barrier, after the store -- constant-clock ticks of 10 ns -- and
// XCC_ID << 32 | HW_ID), waves in block order, four per block.
hipError_t launch_qmv1_trace(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                             const uint16_t* biases, uint16_t* y, int64_t N, int64_t K,
                             uint64_t* trace, hipStream_t stream) {
  const qmv::NormIn none{};
  switch (K / 512) {
    case 7: return qmv1::run<7, 0, false, 1, true>(x, wq, scales, biases, nullptr, y, N, none,
                                                    stream, trace);
    case 8: return qmv1::run<8, 0, false, 1, true>(x, wq, scales, biases, nullptr, y, N, none,
                                                    stream, trace);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mq

extern "C" int mq_qmv_trace(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                            const uint16_t* biases, uint16_t* y, int64_t N, int64_t K,
                            uint64_t* trace, size_t trace_words, hipStream_t stream) {
  const int64_t waves = (N + mq::qmv1::RPB - 1) / mq::qmv1::RPB * (mq::qmv1::kBlock / 64);
  if (!x || !wq || !scales || !biases || !y || !trace || (K != 3584 && K != 4096) ||
      !mq::qmv1_fits(1, N, K, 4, 64) || trace_words < (size_t)waves * 4)
    return mq::set_last_error(MQ_ERR_INVALID,
                              "[qmv_trace] needs a one-row 4-bit group-64 GEMV that the one-row "
                              "kernel takes, K 3584 or 4096, and 4 words of trace per wave.");
  if (hipError_t e = mq::launch_qmv1_trace(x, wq, scales, biases, y, N, K, trace, stream);
      e != hipSuccess)
    return mq::set_last_error(MQ_ERR_HIP, "[qmv_trace] HIP launch failed.");
  return mq::set_last_error(MQ_OK, "");
}
