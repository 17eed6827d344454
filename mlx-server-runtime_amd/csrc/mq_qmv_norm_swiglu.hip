// RMSNorm input and SwiGLU epilogue in one GEMV launch (qmv kernel with NORM
// and EPI 1, mq_qmv_kernel.h): an MLP's norm, gate|up projection and
// silu(gate) * up.
#include "mq_qmv_kernel.h"

namespace mq {
MQ_QMV_INSTANCE(4, false, 1, true);
MQ_QMV_INSTANCE(8, false, 1, true);
}  // namespace mq
