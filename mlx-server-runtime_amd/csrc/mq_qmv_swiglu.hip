// The SwiGLU-epilogue GEMV launches (qmv kernel, mq_qmv_kernel.h): the gate
// and up projections of an MLP and silu(gate) * up in one kernel.
#include "mq_qmv_kernel.h"

namespace mq {
MQ_QMV_INSTANCE(4, false, 1, false);
MQ_QMV_INSTANCE(8, false, 1, false);
}  // namespace mq
