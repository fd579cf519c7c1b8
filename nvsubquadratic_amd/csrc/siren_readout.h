// The SIREN readout's one-pass gradient (siren_filter.hip) as seen from other
// translation units: gk [nb][H][G] (row stride ldk), the readout input
// act [nb][HD + 1][G] (row stride lda; only rows < HD are read), W_out [H][HD]:
//   gact[s][j][g] = sum_h W_out[h][j] gk[s][h][g],
//   gwout[h][j] = scale * sum_{s,g} gk[s][h][g] act[s][j][g],
//   gbout[h]    = scale * sum_{s,g} gk[s][h][g] bw[g]   (bw == nullptr: weight 1),
// bf16-split matrix products with fp32 accumulation, fixed-order sums.
// HD in {16, 32, 64}, G <= 2^23, ldk <= 2^23; ws: siren_readout_bwd_ws_floats.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace nsq {

size_t siren_readout_bwd_ws_floats(int64_t H, int HD, int64_t G, int64_t nb);

bool siren_readout_bwd_run(const float* gk, int64_t ldk, const float* act, int64_t lda, const float* bw,
                           const float* wout, int64_t H, int HD, int64_t G, int64_t nb, float* gact, float* gwout,
                           float* gbout, float scale, float* ws, hipStream_t st);

}  // namespace nsq
