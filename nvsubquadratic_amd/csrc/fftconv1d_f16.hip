// Instantiates every causal 1D FFT-conv kernel for f16 I/O.
#include "fftconv1d_impl.h"

namespace nsq {
NSQ_INSTANTIATE_FFTCONV1D(NSQ_DTYPE_F16)
}  // namespace nsq
