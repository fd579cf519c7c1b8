// f16 instances of the 2D / 3D conv's host runs (plain and mixed-boundary).
#include "fftconv_nd_plan.h"

namespace nsq {
NSQ_ND_RUN_INSTANCES(, NSQ_DTYPE_F16, false)
}  // namespace nsq
