// The plain 8-bit GEMV launches (qmv kernel, mq_qmv_kernel.h).
#include "mq_qmv_kernel.h"

namespace mq {
MQ_QMV_INSTANCE(8, false, 0, false);
}  // namespace mq
