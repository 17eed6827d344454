// Decode-shaped quantized matmul (qmv): dispatch and the shape test.  The
// kernel and its launch templates are in mq_qmv_kernel.h; this file
// instantiates the plain 4-bit launches, mq_qmv_b8.hip / mq_qmv_g4.hip /
// mq_qmv_g8.hip / mq_qmv_swiglu.hip / mq_qmv_norm*.hip the others.
#include "mq_qmv_kernel.h"

namespace mq {

MQ_QMV_INSTANCE(4, false, 0, false);
extern MQ_QMV_INSTANCE(8, false, 0, false);
extern MQ_QMV_INSTANCE(4, true, 0, false);
extern MQ_QMV_INSTANCE(8, true, 0, false);
extern MQ_QMV_INSTANCE(4, false, 1, false);
extern MQ_QMV_INSTANCE(8, false, 1, false);
extern MQ_QMV_INSTANCE(4, false, 0, true);
extern MQ_QMV_INSTANCE(8, false, 0, true);
extern MQ_QMV_INSTANCE(4, false, 1, true);
extern MQ_QMV_INSTANCE(8, false, 1, true);
extern MQ_QMV_INSTANCE(4, true, 1, false);
extern MQ_QMV_INSTANCE(8, true, 1, false);

using qmv::kBlock;
using qmv::kQmvLdsBudget;

bool qmv_fits(int64_t M, int64_t N, int64_t K, int bits, int64_t T, int group_size) {
  if (M < 1 || M > 8 || T > 65535) return false;
  const int epc = 128 / bits;
  const int64_t C = K / epc;
  if (C > 8 * 256) return false;  // more chunks than one block's lanes can own
  if ((K / group_size) % 2 != 0) return false;  // scales move in 4-byte words
  const int tpr = qmv::pick_tpr(C, N, T);
  const int64_t CP = (C + tpr - 1) / tpr * tpr;
  const int64_t mt = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  const int64_t units = mt * CP * (epc / 8);  // x units staged per block
  // one row per lane group: the scale/bias DMA within its per-wave operations
  const int64_t rpb = kBlock / tpr;
  const int64_t sb_words = (rpb * (K / group_size) + CP / (group_size / epc) + 1) / 2;
  // group size 32 doubles the scale arrays: up to the two-row budget (still
  // three blocks per CU), so the 7B down projection's GEMV fits
  const int64_t budget = group_size < 64 ? qmv::kTwoRowLdsBudget : kQmvLdsBudget;
  return qmv::lds_bytes(bits, tpr, mt, K, 1, group_size) <= budget &&
         units <= 12 * kBlock && 2 * ((sb_words + 63) / 64) <= qmv::kSbOpsPerWave * (kBlock / 64);
}

// The SwiGLU GEMV: N outputs from a 2N-row matrix, M <= 2, at most one wave
// per row (a block pairs RPB/2 gate rows with their up rows), and every byte
// offset of the block's rows within one buffer descriptor.
bool qmv_swiglu_fits(int64_t M, int64_t N, int64_t K, int bits, int group_size) {
  if (M < 1 || M > 2 || N < 1 || !qmv_fits(M, 2 * N, K, bits, 1, group_size)) return false;
  const int64_t C = K / (128 / bits);
  return qmv::pick_tpr(C, 2 * N, 1) <= 64 && 2 * N * C * 16 < (int64_t(1) << 32);
}

hipError_t launch_qmv_swiglu(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                             const uint16_t* biases, uint16_t* y, int64_t M, int64_t N, int64_t K,
                             int bits, int group_size, hipStream_t stream) {
  if (N == 0 || M == 0) return hipSuccess;
  if (qmv1_fits(M, 2 * N, K, bits, group_size))
    return launch_qmv1(x, wq, scales, biases, nullptr, y, N, K, group_size, true, nullptr,
                       stream);
  const GatherMap g1{nullptr, nullptr, 1, 1, 1};
  const qmv::NormIn none{};
  if (bits == 4)
    return qmv::run_bits<4, false, 1, false>(x, wq, scales, biases, nullptr, y, M, N, K, g1, none,
                                             group_size, stream);
  return qmv::run_bits<8, false, 1, false>(x, wq, scales, biases, nullptr, y, M, N, K, g1, none,
                                           group_size, stream);
}

// The SwiGLU GEMV per gathered (batch, expert) pair: every expert's matrix is
// 2N rows (gate rows, then up rows).  The lanes split each row exactly as the
// plain gathered GEMV of the 2N-row matrix does, so the results are those of
// that GEMV followed by silu_mul, bit for bit.
bool gather_qmv_swiglu_fits(int64_t M, int64_t N, int64_t K, int bits, int64_t T,
                            int group_size) {
  if (M < 1 || M > 2 || N < 1 || T < 1 || !qmv_fits(M, 2 * N, K, bits, T, group_size))
    return false;
  const int64_t C = K / (128 / bits);
  return qmv::pick_tpr(C, 2 * N, T) <= 64 && 2 * N * C * 16 < (int64_t(1) << 32);
}

hipError_t launch_gather_qmv_swiglu(const uint16_t* x, const uint32_t* wq,
                                    const uint16_t* scales, const uint16_t* biases, uint16_t* y,
                                    int64_t M, int64_t N, int64_t K, int bits, const GatherMap& g,
                                    int group_size, hipStream_t stream) {
  if (N == 0 || M == 0 || g.T == 0) return hipSuccess;
  const qmv::NormIn none{};
  if (bits == 4)
    return qmv::run_bits<4, true, 1, false>(x, wq, scales, biases, nullptr, y, M, N, K, g, none,
                                            group_size, stream);
  return qmv::run_bits<8, true, 1, false>(x, wq, scales, biases, nullptr, y, M, N, K, g, none,
                                          group_size, stream);
}

// RMSNorm of one row, then the GEMV (or the SwiGLU GEMV over a 2N-row
// matrix): the row's 8-element units must fit the norm's four per thread.
bool qmv_norm_fits(int64_t N, int64_t K, int bits, bool swiglu, int group_size) {
  if (K > 8192) return false;
  return swiglu ? qmv_swiglu_fits(1, N, K, bits, group_size)
                : qmv_fits(1, N, K, bits, 1, group_size);
}

hipError_t launch_qmv_norm(const uint16_t* a, const uint16_t* res, uint16_t* res_out,
                           const uint16_t* norm_w, float eps, const uint32_t* wq,
                           const uint16_t* scales, const uint16_t* biases, const uint16_t* bias,
                           uint16_t* y, int64_t N, int64_t K, int bits, bool swiglu,
                           int group_size, hipStream_t stream) {
  if (N == 0) return hipSuccess;
  const qmv::NormIn nrm{res, res_out, norm_w, eps};
  if (qmv1_fits(1, swiglu ? 2 * N : N, K, bits, group_size))
    return launch_qmv1(a, wq, scales, biases, bias, y, N, K, group_size, swiglu, &nrm, stream);
  const GatherMap g1{nullptr, nullptr, 1, 1, 1};
  if (swiglu)
    return bits == 4 ? qmv::run_bits<4, false, 1, true>(a, wq, scales, biases, nullptr, y, 1, N,
                                                        K, g1, nrm, group_size, stream)
                     : qmv::run_bits<8, false, 1, true>(a, wq, scales, biases, nullptr, y, 1, N,
                                                        K, g1, nrm, group_size, stream);
  return bits == 4 ? qmv::run_bits<4, false, 0, true>(a, wq, scales, biases, bias, y, 1, N, K, g1,
                                                      nrm, group_size, stream)
                   : qmv::run_bits<8, false, 0, true>(a, wq, scales, biases, bias, y, 1, N, K, g1,
                                                      nrm, group_size, stream);
}

hipError_t launch_qmv(const uint16_t* x, const uint32_t* wq, const uint16_t* scales,
                      const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M,
                      int64_t N, int64_t K, int bits, const GatherMap& g, int group_size,
                      hipStream_t stream) {
  if (N == 0 || M == 0 || g.T == 0) return hipSuccess;
  // A plain matmul carries no tables: its kernels skip the index loads.
  const bool gather = g.lhs || g.rhs || g.T != 1;
  if (!gather && qmv1_plain_fits(M, N, K, bits, group_size))
    return launch_qmv1(x, wq, scales, biases, bias, y, N, K, group_size, false, nullptr, stream);
  const qmv::NormIn none{};
  if (bits == 4)
    return gather ? qmv::run_bits<4, true, 0, false>(x, wq, scales, biases, bias, y, M, N, K, g,
                                                     none, group_size, stream)
                  : qmv::run_bits<4, false, 0, false>(x, wq, scales, biases, bias, y, M, N, K, g,
                                                      none, group_size, stream);
  return gather ? qmv::run_bits<8, true, 0, false>(x, wq, scales, biases, bias, y, M, N, K, g,
                                                   none, group_size, stream)
                : qmv::run_bits<8, false, 0, false>(x, wq, scales, biases, bias, y, M, N, K, g,
                                                    none, group_size, stream);
}

}  // namespace mq
