// The GEMV launches that take their input row through an RMSNorm first
// (qmv kernel with NORM, mq_qmv_kernel.h).
#include "mq_qmv_kernel.h"

namespace mq {
MQ_QMV_INSTANCE(4, false, 0, true);
MQ_QMV_INSTANCE(8, false, 0, true);
}  // namespace mq
