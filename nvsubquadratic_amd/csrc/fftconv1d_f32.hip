// Instantiates every causal 1D FFT-conv kernel for f32 I/O.
#include "fftconv1d_impl.h"

namespace nsq {
NSQ_INSTANTIATE_FFTCONV1D(NSQ_DTYPE_F32)
template bool run_col_fwd_rows<0>(int, const float*, int64_t, int64_t, int64_t, float2*, const float2*, hipStream_t);
template bool run_col_inv_rows<0>(int, const float2*, float*, float*, int64_t, int, const float2*, hipStream_t);
}  // namespace nsq
