// C ABI of the plain and mixed-boundary 2D / 3D non-causal FFT convolution
// (host plans in fftconv_nd_plan.h, kernels in fftconv_nd_impl.h).
#include "fftconv_nd_plan.h"

namespace nsq {

int nd_fwd(int nd, const void* x, const float* k, const void* shortcut, void* y, int dtype, int64_t B,
                  int64_t H, const int64_t* S, const int64_t* K, int64_t kbatch, unsigned periodic, void* workspace,
                  size_t workspace_bytes, void* stream) {
  clear_error();
  NdPlan p;
  int rc = validate_nd(nd, x, y, k, dtype, B, H, S, K, kbatch, periodic, p);
  if (rc) return rc;
  const size_t need = nd_workspace_bytes(nd, B, H, S, K, kbatch, periodic, NSQ_DIR_FWD);
  NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "fftconv_nd_fwd: workspace of %zu bytes required, got %zu", need,
                workspace_bytes);
  const float2* tw = twiddle_table();
  if (!tw) return NSQ_ERR_HIP;
  hipStream_t st = (hipStream_t)stream;
  float2* ws = (float2*)workspace;
  const bool save = workspace_bytes >= nd_workspace_bytes(nd, B, H, S, K, kbatch, periodic, NSQ_DIR_BWD);
  bool ok;
  switch (dtype) {
    case NSQ_DTYPE_F32: ok = run_nd_fwd<NSQ_DTYPE_F32>(p, x, k, shortcut, y, ws, save, tw, st); break;
    case NSQ_DTYPE_BF16: ok = run_nd_fwd<NSQ_DTYPE_BF16>(p, x, k, shortcut, y, ws, save, tw, st); break;
    default: ok = run_nd_fwd<NSQ_DTYPE_F16>(p, x, k, shortcut, y, ws, save, tw, st); break;
  }
  NSQ_CHECK_ARG(ok, "fftconv_nd_fwd: no kernel instantiated for this shape");
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

int nd_bwd(int nd, const void* g, const void* x, const float* k, const void* shortcut, void* gx, float* gk,
                  float* gs, int dtype, int64_t B, int64_t H, const int64_t* S, const int64_t* K, int64_t kbatch,
                  unsigned periodic, void* workspace, size_t workspace_bytes, int fwd_state, void* stream) {
  clear_error();
  NdPlan p;
  int rc = validate_nd(nd, g, x, k, dtype, B, H, S, K, kbatch, periodic, p);
  if (rc) return rc;
  NSQ_CHECK_ARG(gx && gk, "fftconv_nd_bwd: null gradient output pointer");
  NSQ_CHECK_ARG(!shortcut || gs, "fftconv_nd_bwd: gs required when a shortcut is given");
  const size_t need = nd_workspace_bytes(nd, B, H, S, K, kbatch, periodic, NSQ_DIR_BWD);
  NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "fftconv_nd_bwd: workspace of %zu bytes required, got %zu", need,
                workspace_bytes);
  const float2* tw = twiddle_table();
  if (!tw) return NSQ_ERR_HIP;
  hipStream_t st = (hipStream_t)stream;
  float2* ws = (float2*)workspace;
  bool ok;
  switch (dtype) {
    case NSQ_DTYPE_F32: ok = run_nd_bwd<NSQ_DTYPE_F32>(p, g, x, k, shortcut, gx, gk, gs, ws, fwd_state != 0, tw, st); break;
    case NSQ_DTYPE_BF16: ok = run_nd_bwd<NSQ_DTYPE_BF16>(p, g, x, k, shortcut, gx, gk, gs, ws, fwd_state != 0, tw, st); break;
    default: ok = run_nd_bwd<NSQ_DTYPE_F16>(p, g, x, k, shortcut, gx, gk, gs, ws, fwd_state != 0, tw, st); break;
  }
  NSQ_CHECK_ARG(ok, "fftconv_nd_bwd: no kernel instantiated for this shape");
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

}  // namespace nsq

using namespace nsq;

extern "C" {

size_t nsq_fftconv_nd_workspace_bytes(int nd, int64_t B, int64_t H, const int64_t* S, const int64_t* K,
                                      int64_t kbatch, int direction) {
  return nd_workspace_bytes(nd, B, H, S, K, kbatch, 0u, direction);
}

int nsq_fftconv_nd_fwd(int nd, const void* x, const float* k, const void* shortcut, void* y, int dtype, int64_t B,
                       int64_t H, const int64_t* S, const int64_t* K, int64_t kbatch, void* workspace,
                       size_t workspace_bytes, void* stream) {
  return nd_fwd(nd, x, k, shortcut, y, dtype, B, H, S, K, kbatch, 0u, workspace, workspace_bytes, stream);
}

int nsq_fftconv_nd_bwd(int nd, const void* g, const void* x, const float* k, const void* shortcut, void* gx, float* gk,
                       float* gs, int dtype, int64_t B, int64_t H, const int64_t* S, const int64_t* K, int64_t kbatch,
                       void* workspace, size_t workspace_bytes, int fwd_state, void* stream) {
  return nd_bwd(nd, g, x, k, shortcut, gx, gk, gs, dtype, B, H, S, K, kbatch, 0u, workspace, workspace_bytes,
                fwd_state, stream);
}

size_t nsq_mixed_fftconv_nd_workspace_bytes(int nd, int64_t B, int64_t H, const int64_t* S, const int64_t* K,
                                            int64_t kbatch, unsigned periodic, int direction) {
  return nd_workspace_bytes(nd, B, H, S, K, kbatch, periodic, direction);
}

int nsq_mixed_fftconv_nd_fwd(int nd, const void* x, const float* k, const void* shortcut, void* y, int dtype,
                             int64_t B, int64_t H, const int64_t* S, const int64_t* K, int64_t kbatch,
                             unsigned periodic, void* workspace, size_t workspace_bytes, void* stream) {
  return nd_fwd(nd, x, k, shortcut, y, dtype, B, H, S, K, kbatch, periodic, workspace, workspace_bytes, stream);
}

int nsq_mixed_fftconv_nd_bwd(int nd, const void* g, const void* x, const float* k, const void* shortcut, void* gx,
                             float* gk, float* gs, int dtype, int64_t B, int64_t H, const int64_t* S,
                             const int64_t* K, int64_t kbatch, unsigned periodic, void* workspace,
                             size_t workspace_bytes, int fwd_state, void* stream) {
  return nd_bwd(nd, g, x, k, shortcut, gx, gk, gs, dtype, B, H, S, K, kbatch, periodic, workspace, workspace_bytes,
                fwd_state, stream);
}

}  // extern "C"
