// The one-row GEMV on 2-bit codes read at their width (mq_qmv1_kernel.h).
#include "mq_qmv1_kernel.h"

namespace mq {

hipError_t launch_qmvs_b2(int S, int group_size, const uint16_t* x, const uint32_t* wq,
                          const uint16_t* scales, const uint16_t* biases, const uint16_t* bias,
                          uint16_t* y, int64_t N, hipStream_t stream) {
  return qmv1::run_stream<2>(S, group_size, x, wq, scales, biases, bias, y, N, stream);
}

}  // namespace mq
