// C ABI of the Hyena-gated 2D / 3D conv: the gates fused into the conv's first
// and last passes (fftconv_nd_plan.h with GATED), or the elementwise gate
// kernels (gate.h) around the plain conv where the plan has no fused variant.
#include "fftconv_nd_plan.h"
#include "gate.h"

#include <cstdlib>
#include <initializer_list>

namespace nsq {

// ---------------------------------------------------------------------------
// Hyena-gated 2D/3D conv.  Workspace: the conv's; for the gate-kernel plan
// rounded up to 256 bytes and followed by I/O-dtype buffers of B*H*prod(S)
// values: forward z and (when the caller keeps none) y1; backward z, dy1, dz.
// ---------------------------------------------------------------------------
static int64_t nd_numel(int nd, int64_t B, int64_t H, const int64_t* S) {
  int64_t n = B * H;
  for (int d = 0; d < nd; ++d) n *= S[d];
  return n;
}

// The gates run inside the conv's first and last passes where those are the
// packed 2D rows with the vector epilogue (the forward's crop offset along the
// last axis even and its length a multiple of 8) or the 3D plane passes; other
// plans, or NSQ_ND_GATES_FUSED=0, run the gate kernels around the conv (same
// results: the fused loaders and epilogues round as gate_ew_kernel does).
static bool gated_fused_ok(const NdPlan& p) {
  const char* e = getenv("NSQ_ND_GATES_FUSED");
  if (e && e[0] == '0') return false;
  if (p.nd == 3) return plane_ok(p);
  return p.pack && p.o[2] % 2 == 0 && p.S[2] % 8 == 0;
}

static size_t gated_nd_workspace_bytes(int nd, int64_t B, int64_t H, const int64_t* S, const int64_t* K,
                                       int64_t kbatch, unsigned periodic, int dtype, int direction) {
  const size_t conv = nd_workspace_bytes(nd, B, H, S, K, kbatch, periodic, direction);
  if (!conv || !valid_dtype(dtype)) return 0;
  NdPlan p;
  if (make_nd_plan(nd, B, H, S, K, kbatch, periodic, p) && gated_fused_ok(p)) return conv;
  const size_t es = dtype == NSQ_DTYPE_F32 ? 4 : 2;
  return round256(conv) + size_t(direction == NSQ_DIR_BWD ? 3 : 2) * round256(size_t(nd_numel(nd, B, H, S)) * es);
}

template <int DT>
static void gate_pass(int op, const GateEw& g, int64_t n, hipStream_t st) {
  switch (op) {
    case GATE_OP_FWD1: launch_gate_ew<DT, GATE_OP_FWD1>(g, n, st); break;
    case GATE_OP_FWD2: launch_gate_ew<DT, GATE_OP_FWD2>(g, n, st); break;
    case GATE_OP_BWD2: launch_gate_ew<DT, GATE_OP_BWD2>(g, n, st); break;
    default: launch_gate_ew<DT, GATE_OP_BWD1>(g, n, st); break;
  }
}

static void gate_pass(int dtype, int op, const GateEw& g, int64_t n, hipStream_t st) {
  switch (dtype) {
    case NSQ_DTYPE_F32: gate_pass<NSQ_DTYPE_F32>(op, g, n, st); break;
    case NSQ_DTYPE_BF16: gate_pass<NSQ_DTYPE_BF16>(op, g, n, st); break;
    default: gate_pass<NSQ_DTYPE_F16>(op, g, n, st); break;
  }
}

static bool aligned16_nd(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (p && (reinterpret_cast<uintptr_t>(p) & 15)) return false;
  return true;
}

static int gated_nd_fwd(int nd, const void* q, const void* kgate, const void* v, const float* k, const void* shortcut,
                        void* y, void* y1, int dtype, int act1, int act2, int64_t B, int64_t H, const int64_t* S,
                        const int64_t* K, int64_t kbatch, unsigned periodic, void* workspace, size_t workspace_bytes,
                        void* stream) {
  clear_error();
  NdPlan p;
  int rc = validate_nd(nd, q, y, k, dtype, B, H, S, K, kbatch, periodic, p);
  if (rc) return rc;
  NSQ_CHECK_ARG(kgate && v, "gated_fftconv_nd_fwd: null gate operand");
  NSQ_CHECK_ARG(act1 >= 0 && act1 <= 2 && act2 >= 0 && act2 <= 2,
                "gated_fftconv_nd: gate codes must be 0 (identity), 1 (sigmoid) or 2 (silu); got %d, %d", act1, act2);
  NSQ_CHECK_ARG(aligned16_nd({q, kgate, v, y, y1, workspace}), "gated_fftconv_nd_fwd: tensors must be 16-byte aligned");
  const size_t need = gated_nd_workspace_bytes(nd, B, H, S, K, kbatch, periodic, dtype, NSQ_DIR_FWD);
  NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "gated_fftconv_nd_fwd: workspace of %zu bytes required, got %zu",
                need, workspace_bytes);
  hipStream_t st = (hipStream_t)stream;
  if (gated_fused_ok(p)) {
    const float2* tw = twiddle_table();
    if (!tw) return NSQ_ERR_HIP;
    const GatedIO gi{q, kgate, v, nullptr, y1, nullptr, nullptr, act1, act2};
    float2* ws = (float2*)workspace;
    bool ok;
    switch (dtype) {
      case NSQ_DTYPE_F32: ok = run_nd_fwd<NSQ_DTYPE_F32, true>(p, q, k, shortcut, y, ws, false, tw, st, &gi); break;
      case NSQ_DTYPE_BF16: ok = run_nd_fwd<NSQ_DTYPE_BF16, true>(p, q, k, shortcut, y, ws, false, tw, st, &gi); break;
      default: ok = run_nd_fwd<NSQ_DTYPE_F16, true>(p, q, k, shortcut, y, ws, false, tw, st, &gi); break;
    }
    NSQ_CHECK_ARG(ok, "gated_fftconv_nd_fwd: no kernel instantiated for this shape");
    NSQ_CHECK_LAUNCH();
    return NSQ_OK;
  }
  const size_t conv = round256(nd_workspace_bytes(nd, B, H, S, K, kbatch, periodic, NSQ_DIR_FWD));
  const int64_t n = nd_numel(nd, B, H, S);
  const size_t es = dtype == NSQ_DTYPE_F32 ? 4 : 2;
  char* z = (char*)workspace + conv;
  void* y1b = y1 ? y1 : (void*)(z + round256(n * es));
  gate_pass(dtype, GATE_OP_FWD1, GateEw{q, kgate, nullptr, z, nullptr, act1}, n, st);
  rc = nd_fwd(nd, z, k, shortcut, y1b, dtype, B, H, S, K, kbatch, periodic, workspace, conv, stream);
  if (rc) return rc;
  gate_pass(dtype, GATE_OP_FWD2, GateEw{y1b, v, nullptr, y, nullptr, act2}, n, st);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

static int gated_nd_bwd(int nd, const void* g, const void* q, const void* kgate, const void* v, const void* y1,
                        const float* k, const void* shortcut, void* dq, void* dkgate, void* dv, float* gk, float* gs,
                        int dtype, int act1, int act2, int64_t B, int64_t H, const int64_t* S, const int64_t* K,
                        int64_t kbatch, unsigned periodic, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  NdPlan p;
  int rc = validate_nd(nd, g, q, k, dtype, B, H, S, K, kbatch, periodic, p);
  if (rc) return rc;
  NSQ_CHECK_ARG(kgate && v && y1 && dq && dkgate && dv && gk, "gated_fftconv_nd_bwd: null tensor pointer");
  NSQ_CHECK_ARG(!shortcut || gs, "gated_fftconv_nd_bwd: gs required when a shortcut is given");
  NSQ_CHECK_ARG(act1 >= 0 && act1 <= 2 && act2 >= 0 && act2 <= 2,
                "gated_fftconv_nd: gate codes must be 0 (identity), 1 (sigmoid) or 2 (silu); got %d, %d", act1, act2);
  NSQ_CHECK_ARG(aligned16_nd({g, q, kgate, v, y1, dq, dkgate, dv, workspace}),
                "gated_fftconv_nd_bwd: tensors must be 16-byte aligned");
  const size_t need = gated_nd_workspace_bytes(nd, B, H, S, K, kbatch, periodic, dtype, NSQ_DIR_BWD);
  NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "gated_fftconv_nd_bwd: workspace of %zu bytes required, got %zu",
                need, workspace_bytes);
  hipStream_t st = (hipStream_t)stream;
  if (gated_fused_ok(p)) {
    const float2* tw = twiddle_table();
    if (!tw) return NSQ_ERR_HIP;
    const GatedIO gi{q, kgate, v, y1, nullptr, dv, dkgate, act1, act2};
    float2* ws = (float2*)workspace;
    bool ok;
    switch (dtype) {
      case NSQ_DTYPE_F32:
        ok = run_nd_bwd<NSQ_DTYPE_F32, true>(p, g, q, k, shortcut, dq, gk, gs, ws, false, tw, st, &gi);
        break;
      case NSQ_DTYPE_BF16:
        ok = run_nd_bwd<NSQ_DTYPE_BF16, true>(p, g, q, k, shortcut, dq, gk, gs, ws, false, tw, st, &gi);
        break;
      default: ok = run_nd_bwd<NSQ_DTYPE_F16, true>(p, g, q, k, shortcut, dq, gk, gs, ws, false, tw, st, &gi); break;
    }
    NSQ_CHECK_ARG(ok, "gated_fftconv_nd_bwd: no kernel instantiated for this shape");
    NSQ_CHECK_LAUNCH();
    return NSQ_OK;
  }
  const size_t conv = round256(nd_workspace_bytes(nd, B, H, S, K, kbatch, periodic, NSQ_DIR_BWD));
  const int64_t n = nd_numel(nd, B, H, S);
  const size_t es = dtype == NSQ_DTYPE_F32 ? 4 : 2;
  char* z = (char*)workspace + conv;
  char* dy1 = z + round256(n * es);
  char* dz = dy1 + round256(n * es);
  gate_pass(dtype, GATE_OP_BWD2, GateEw{g, v, y1, dy1, dv, act2}, n, st);
  gate_pass(dtype, GATE_OP_FWD1, GateEw{q, kgate, nullptr, z, nullptr, act1}, n, st);
  rc = nd_bwd(nd, dy1, z, k, shortcut, dz, gk, gs, dtype, B, H, S, K, kbatch, periodic, workspace, conv, 0, stream);
  if (rc) return rc;
  gate_pass(dtype, GATE_OP_BWD1, GateEw{dz, q, kgate, dq, dkgate, act1}, n, st);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

}  // namespace nsq

using namespace nsq;

extern "C" {

size_t nsq_gated_fftconv_nd_workspace_bytes(int nd, int64_t B, int64_t H, const int64_t* S, const int64_t* K,
                                            int64_t kbatch, unsigned periodic, int dtype, int direction) {
  return gated_nd_workspace_bytes(nd, B, H, S, K, kbatch, periodic, dtype, direction);
}

int nsq_gated_fftconv_nd_fwd(int nd, const void* q, const void* kgate, const void* v, const float* k,
                             const void* shortcut, void* y, void* y1, int dtype, int act1, int act2, int64_t B,
                             int64_t H, const int64_t* S, const int64_t* K, int64_t kbatch, unsigned periodic,
                             void* workspace, size_t workspace_bytes, void* stream) {
  return gated_nd_fwd(nd, q, kgate, v, k, shortcut, y, y1, dtype, act1, act2, B, H, S, K, kbatch, periodic, workspace,
                      workspace_bytes, stream);
}

int nsq_gated_fftconv_nd_bwd(int nd, const void* g, const void* q, const void* kgate, const void* v, const void* y1,
                             const float* k, const void* shortcut, void* dq, void* dkgate, void* dv, float* gk,
                             float* gs, int dtype, int act1, int act2, int64_t B, int64_t H, const int64_t* S,
                             const int64_t* K, int64_t kbatch, unsigned periodic, void* workspace,
                             size_t workspace_bytes, void* stream) {
  return gated_nd_bwd(nd, g, q, kgate, v, y1, k, shortcut, dq, dkgate, dv, gk, gs, dtype, act1, act2, B, H, S, K,
                      kbatch, periodic, workspace, workspace_bytes, stream);
}

}  // extern "C"
