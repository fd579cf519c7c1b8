// Depthwise causal direct convolution (k = 1..256), forward and backward.
//
// Replaces the native kernel the reference binds at
// nvsubquadratic/ops/causal_conv1d_custom.py:81-98 (subquadratic_ops_torch
// .causal_conv1d(x, w, bias, activation)), used by the Hyena short-conv slot
// through nvsubquadratic/modules/subq_ops_causal_conv1d.py:77-83.
#include "direct_conv.h"

namespace nsq {

// grid = (B*C, ceil(L / kConvTile)).
template <int DT, int ACT>
__global__ __launch_bounds__(kConvThreads) void cconv_fwd_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                                  const float* __restrict__ w,
                                                                  const float* __restrict__ bias,
                                                                  typename Elem<DT>::T* __restrict__ y, int C, int L,
                                                                  int K) {
  __shared__ __align__(16) float xs[conv_tile_floats(kConvMaxK)];
  __shared__ __align__(16) float wl[kConvWeightFloats];
  const int64_t row = blockIdx.x;
  const int c = int(row % C);
  const int64_t n0 = int64_t(blockIdx.y) * kConvTile;
  const typename Elem<DT>::T* xr = x + row * L;
  stage_weights<false>(wl, w + int64_t(c) * K, K);
  stage_row<DT, conv_tile_floats(kConvMaxK)>(xs, xr, n0 - (K - 1), kConvTile + K - 1 + 2 * kConvPer, L);
  const float b0 = bias ? bias[c] : 0.f;
  float acc[kConvPer];
#pragma unroll
  for (int e = 0; e < kConvPer; ++e) acc[e] = b0;
  const int base = threadIdx.x * kConvPer;
  slide_fma(acc, xs, base, K, wl);
  typename Elem<DT>::T* yr = y + row * L;
#pragma unroll
  for (int e = 0; e < kConvPer; e += 2) {
    const int64_t n = n0 + base + e;
    if (n < L) store_pair<DT>(yr, n, L, make_float2(act_fwd<ACT>(acc[e]), act_fwd<ACT>(acc[e + 1])));
  }
}

// gpre = gy * silu'(pre), pre recomputed; fp32 workspace.  grid as forward.
template <int DT>
__global__ __launch_bounds__(kConvThreads) void cconv_gpre_silu_kernel(const typename Elem<DT>::T* __restrict__ gy,
                                                                        const typename Elem<DT>::T* __restrict__ x,
                                                                        const float* __restrict__ w,
                                                                        const float* __restrict__ bias,
                                                                        float* __restrict__ gpre, int C, int L, int K) {
  __shared__ __align__(16) float xs[conv_tile_floats(kConvMaxK)];
  __shared__ __align__(16) float wl[kConvWeightFloats];
  const int64_t row = blockIdx.x;
  const int c = int(row % C);
  const int64_t n0 = int64_t(blockIdx.y) * kConvTile;
  stage_weights<false>(wl, w + int64_t(c) * K, K);
  stage_row<DT, conv_tile_floats(kConvMaxK)>(xs, x + row * L, n0 - (K - 1), kConvTile + K - 1 + 2 * kConvPer, L);
  const float b0 = bias ? bias[c] : 0.f;
  float acc[kConvPer];
#pragma unroll
  for (int e = 0; e < kConvPer; ++e) acc[e] = b0;
  const int base = threadIdx.x * kConvPer;
  slide_fma(acc, xs, base, K, wl);
#pragma unroll
  for (int e = 0; e < kConvPer; ++e) {
    const int64_t n = n0 + base + e;
    if (n < L) gpre[row * L + n] = Elem<DT>::load(gy, row * L + n) * dsilu(acc[e]);
  }
}

template <int DT>
static void launch_fwd(const void* x, const float* w, const float* bias, void* y, int act, int B, int C, int L, int K,
                       hipStream_t st) {
  using ET = typename Elem<DT>::T;
  dim3 grid(B * C, unsigned(ceil_div(L, kConvTile)));
  if (act == NSQ_ACT_SILU)
    hipLaunchKernelGGL((cconv_fwd_kernel<DT, NSQ_ACT_SILU>), grid, dim3(kConvThreads), 0, st, (const ET*)x, w, bias,
                       (ET*)y, C, L, K);
  else
    hipLaunchKernelGGL((cconv_fwd_kernel<DT, NSQ_ACT_IDENTITY>), grid, dim3(kConvThreads), 0, st, (const ET*)x, w,
                       bias, (ET*)y, C, L, K);
}

template <int DT>
static void launch_bwd(const void* gy, const void* x, const float* w, const float* bias, void* gx, float* gw,
                       float* gb, int act, int B, int C, int L, int K, float* ws, hipStream_t st) {
  using ET = typename Elem<DT>::T;
  dim3 grid(B * C, unsigned(ceil_div(L, kConvTile)));
  if (act == NSQ_ACT_SILU) {
    hipLaunchKernelGGL((cconv_gpre_silu_kernel<DT>), grid, dim3(kConvThreads), 0, st, (const ET*)gy, (const ET*)x, w,
                       bias, ws, C, L, K);
    hipLaunchKernelGGL((cconv_gx_kernel<DT, NSQ_DTYPE_F32>), grid, dim3(kConvThreads), 0, st, (const float*)ws, w,
                       (ET*)gx, C, L, K);
    hipLaunchKernelGGL((cconv_wgrad_kernel<DT, NSQ_DTYPE_F32>), dim3(C), dim3(kConvThreads), 0, st, (const float*)ws,
                       (const ET*)x, gw, gb, B, C, L, K);
  } else {
    hipLaunchKernelGGL((cconv_gx_kernel<DT, DT>), grid, dim3(kConvThreads), 0, st, (const ET*)gy, w, (ET*)gx, C, L, K);
    hipLaunchKernelGGL((cconv_wgrad_kernel<DT, DT>), dim3(C), dim3(kConvThreads), 0, st, (const ET*)gy, (const ET*)x,
                       gw, gb, B, C, L, K);
  }
}

static int validate_cconv(const void* a, const void* b, const float* w, int dtype, int act, int64_t B, int64_t C,
                          int64_t L, int64_t K) {
  NSQ_CHECK_ARG(a && b && w, "causal_conv1d: null tensor pointer");
  NSQ_CHECK_ARG(valid_dtype(dtype), "causal_conv1d: unsupported dtype code %d", dtype);
  NSQ_CHECK_ARG(act == NSQ_ACT_IDENTITY || act == NSQ_ACT_SILU, "causal_conv1d: activation code %d not in {0, 1}", act);
  NSQ_CHECK_ARG(B >= 1 && C >= 1 && L >= 1, "causal_conv1d: sizes must be positive");
  NSQ_CHECK_ARG(K >= 1 && K <= kConvMaxK, "causal_conv1d: kernel size %lld outside [1, %d]", (long long)K, kConvMaxK);
  NSQ_CHECK_ARG(B * C <= 0x7fffffff && L < (int64_t(1) << 28), "causal_conv1d: tensor too large (rows are staged through 32-bit byte offsets: L < 2^28)");
  return NSQ_OK;
}

}  // namespace nsq

using namespace nsq;

extern "C" {

size_t nsq_causal_conv1d_bwd_workspace_bytes(int64_t B, int64_t C, int64_t L, int64_t K, int activation) {
  (void)K;
  return activation == NSQ_ACT_SILU ? size_t(B * C * L) * sizeof(float) : 0;
}

int nsq_causal_conv1d_fwd(const void* x, const float* weight, const float* bias, void* y, int dtype, int activation,
                          int64_t B, int64_t C, int64_t L, int64_t K, void* stream) {
  clear_error();
  int rc = validate_cconv(x, y, weight, dtype, activation, B, C, L, K);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case NSQ_DTYPE_F32: launch_fwd<NSQ_DTYPE_F32>(x, weight, bias, y, activation, int(B), int(C), int(L), int(K), st); break;
    case NSQ_DTYPE_BF16: launch_fwd<NSQ_DTYPE_BF16>(x, weight, bias, y, activation, int(B), int(C), int(L), int(K), st); break;
    default: launch_fwd<NSQ_DTYPE_F16>(x, weight, bias, y, activation, int(B), int(C), int(L), int(K), st); break;
  }
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

int nsq_causal_conv1d_bwd(const void* gy, const void* x, const float* weight, const float* bias, void* gx,
                          float* gweight, float* gbias, int dtype, int activation, int64_t B, int64_t C, int64_t L,
                          int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = validate_cconv(gy, x, weight, dtype, activation, B, C, L, K);
  if (rc) return rc;
  NSQ_CHECK_ARG(gx && gweight, "causal_conv1d_bwd: null gradient output pointer");
  const size_t need = nsq_causal_conv1d_bwd_workspace_bytes(B, C, L, K, activation);
  NSQ_CHECK_ARG(need == 0 || (workspace && workspace_bytes >= need),
                "causal_conv1d_bwd: workspace of %zu bytes required, got %zu", need, workspace_bytes);
  hipStream_t st = (hipStream_t)stream;
  float* ws = (float*)workspace;
  switch (dtype) {
    case NSQ_DTYPE_F32:
      launch_bwd<NSQ_DTYPE_F32>(gy, x, weight, bias, gx, gweight, gbias, activation, int(B), int(C), int(L), int(K), ws, st);
      break;
    case NSQ_DTYPE_BF16:
      launch_bwd<NSQ_DTYPE_BF16>(gy, x, weight, bias, gx, gweight, gbias, activation, int(B), int(C), int(L), int(K), ws, st);
      break;
    default:
      launch_bwd<NSQ_DTYPE_F16>(gy, x, weight, bias, gx, gweight, gbias, activation, int(B), int(C), int(L), int(K), ws, st);
      break;
  }
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

}  // extern "C"
