// The gathered SwiGLU-epilogue GEMV launches (qmv kernel, mq_qmv_kernel.h):
// an MoE expert's gate and up projections and silu(gate) * up in one kernel,
// per (token, expert) pair.
#include "mq_qmv_kernel.h"

namespace mq {
MQ_QMV_INSTANCE(4, true, 1, false);
MQ_QMV_INSTANCE(8, true, 1, false);
}  // namespace mq
