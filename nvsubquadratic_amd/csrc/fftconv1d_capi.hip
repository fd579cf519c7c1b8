// C ABI entry points of the causal 1D FFT convolution (see include/nsq_hip.h).
// Kernels and plans live in fftconv1d_impl.h; the per-dtype instantiations are
// compiled in fftconv1d_f32.hip / fftconv1d_bf16.hip / fftconv1d_f16.hip.
#include <cstdlib>
#include <cstring>
#include <initializer_list>

#include "fftconv1d_impl.h"

namespace nsq {

static int validate(const void* a, const void* b, const float* k, int dtype, int64_t B, int64_t H, int64_t L,
                    int64_t K, int64_t kbatch, Plan1D& p) {
  NSQ_CHECK_ARG(kbatch == 1 || kbatch == B, "fftconv1d_causal: kernel batch must be 1 or B (got %lld, B=%lld)",
                (long long)kbatch, (long long)B);
  NSQ_CHECK_ARG(a && b && k, "fftconv1d_causal: null tensor pointer");
  NSQ_CHECK_ARG(valid_dtype(dtype), "fftconv1d_causal: unsupported dtype code %d", dtype);
  NSQ_CHECK_ARG(B >= 1 && H >= 1 && L >= 1 && K >= 1, "fftconv1d_causal: sizes must be positive (B=%lld H=%lld L=%lld K=%lld)",
                (long long)B, (long long)H, (long long)L, (long long)K);
  NSQ_CHECK_ARG(K <= 2 * L, "fftconv1d_causal: kernel length %lld exceeds 2*seq_len=%lld", (long long)K,
                (long long)(2 * L));
  NSQ_CHECK_ARG(B * H <= 0x7fffffff && L <= (int64_t(1) << 30), "fftconv1d_causal: tensor too large");
  if (!make_plan(L, K, p)) {
    set_error("fftconv1d_causal: unsupported (L=%lld, K=%lld): FFT length beyond 2^24", (long long)L, (long long)K);
    return NSQ_ERR_UNSUPPORTED;
  }
  // 4-step column grids are B*H * (N2 / columns per workgroup) <= B*H * 512 workgroups; the row passes run
  // B*H * N1/2 (N1 <= 2048: up to B*H * 1024) workgroups: both below 2^31.
  NSQ_CHECK_ARG(p.fused || B * H * (int64_t(1) << (p.logN1 - 1 > 9 ? p.logN1 - 1 : 9)) < (int64_t(1) << 31),
                "fftconv1d_causal: B*H=%lld too large for the 4-step plan", (long long)(B * H));
  NSQ_CHECK_ARG(!p.fused || kbatch == 1 || B <= 65535, "fftconv1d_causal: B=%lld too large for per-sample filters",
                (long long)B);
  return NSQ_OK;
}

// The 4-step passes' grids: B*H * max(N1/2, 512) workgroups, below 2^31.
static int check_4step_grid(const char* op, int64_t B, int64_t H, int logN) {
  if (logN <= 13) return NSQ_OK;
  const int l1 = split_log_n1(logN);
  NSQ_CHECK_ARG(B * H * (int64_t(1) << (l1 - 1 > 9 ? l1 - 1 : 9)) < (int64_t(1) << 31),
                "%s: B*H=%lld too large for the 4-step plan", op, (long long)(B * H));
  return NSQ_OK;
}

// Circular 1D: L a power of two <= 16384 (the fused plan at FFT length
// max(L, 16)), 1 <= K <= L, kbatch 1 or B.
// Shifted 1D convs.  zpad = false: circular, K <= L, L a power of two (FFT
// length L; below 16, its periodic extension at 16).  zpad = true: zero-padded
// "same", K <= 2L, FFT length pow2(L + ceil(K/2)).  logN = log2(FFT length) - 1:
// the fused plan up to 13, the 4-step plan (with a workspace) up to max_logn.
static int validate_shifted(const char* op, const void* a, const void* b, const float* k, int dtype, int64_t B,
                            int64_t H, int64_t L, int64_t K, int64_t kbatch, bool zpad, int& logN,
                            int max_logn = kMaxLogN) {
  NSQ_CHECK_ARG(a && b && k, "%s: null tensor pointer", op);
  NSQ_CHECK_ARG(valid_dtype(dtype), "%s: unsupported dtype code %d", op, dtype);
  NSQ_CHECK_ARG(B >= 1 && H >= 1 && L >= 1 && K >= 1, "%s: sizes must be positive (B=%lld H=%lld L=%lld K=%lld)",
                op, (long long)B, (long long)H, (long long)L, (long long)K);
  if (zpad)
    NSQ_CHECK_ARG(K <= 2 * L, "%s: K must be <= 2*L on a zero-padded axis (K=%lld, L=%lld)", op, (long long)K,
                  (long long)L);
  else
    NSQ_CHECK_ARG(K <= L, "%s: K must be <= L (K=%lld, L=%lld)", op, (long long)K, (long long)L);
  NSQ_CHECK_ARG(kbatch == 1 || kbatch == B, "%s: kernel batch must be 1 or B (got %lld, B=%lld)", op,
                (long long)kbatch, (long long)B);
  NSQ_CHECK_ARG(B * H <= 0x7fffffff && B <= 65535, "%s: tensor too large", op);
  const int64_t maxF = int64_t(2) << max_logn;
  if (zpad) {
    const int64_t F = L + (K + 1) / 2;
    if (F > maxF) {
      set_error("%s: zero-padded length L + ceil(K/2) = %lld exceeds the largest FFT length %lld", op, (long long)F,
                (long long)maxF);
      return NSQ_ERR_UNSUPPORTED;
    }
    logN = (F < 16 ? 4 : ilog2_ceil(F)) - 1;
    return check_4step_grid(op, B, H, logN);
  }
  if (L > maxF || (L & (L - 1))) {
    set_error("%s: unsupported length L=%lld: the HIP kernels take powers of two up to %lld", op, (long long)L,
              (long long)maxF);
    return NSQ_ERR_UNSUPPORTED;
  }
  logN = (L < 16 ? 4 : ilog2_ceil(L)) - 1;
  return check_4step_grid(op, B, H, logN);
}

// Workspace of a shifted conv: none on the fused plan; on the 4-step plan the
// 4-step blocks (forward: x and k; backward: x, k and g, N complex values
// each), then the rolled rows (B*H rows of F = 2N I/O-dtype values).
static size_t shifted_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch, int dtype,
                                      bool zpad, int direction) {
  int logN = 0;
  if (!valid_dtype(dtype) || B < 1 || H < 1 || L < 1 || K < 1 || K > (zpad ? 2 * L : L)) return 0;
  const int64_t F = zpad ? L + (K + 1) / 2 : L;
  if (F > (int64_t(2) << kMaxLogN) || (!zpad && (L & (L - 1)))) return 0;
  logN = (F < 16 ? 4 : ilog2_ceil(F)) - 1;
  if (logN <= 13) return 0;
  const int64_t N = int64_t(1) << logN;
  const int64_t nk = kbatch * H;
  const int64_t blocks = direction == NSQ_DIR_BWD ? 2 * B * H + nk : B * H + nk;
  const size_t es = dtype == NSQ_DTYPE_F32 ? 4 : 2;
  return (size_t(blocks * N) * sizeof(float2) + 255) / 256 * 256 + size_t(B * H * 2 * N) * es;
}

static size_t causal_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch, int direction) {
  Plan1D p;
  if (!make_plan(L, K, p) || p.fused) return 0;
  const int64_t N = int64_t(1) << p.logN;
  const int64_t nk = kbatch * H;
  // 4-step blocks of N complex values: x, k (forward: y in place of x, or in a third block kept with x and k for
  // the backward); backward x, k, g.  K > L+1 adds one block for the wrap copy of x or g (fold_rows_kernel).
  const int64_t rows = (direction == NSQ_DIR_BWD) ? (2 * B * H + nk) : (B * H + nk);
  return size_t(rows * N + (p.fold ? B * H * N : 0)) * sizeof(float2);
}

static int causal_fwd(const void* x, const float* k, const void* shortcut, void* y, int dtype, int64_t B, int64_t H,
                      int64_t L, int64_t K, int64_t kbatch, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  Plan1D p;
  int rc = validate(x, y, k, dtype, B, H, L, K, kbatch, p);
  if (rc) return rc;
  const float2* tw = twiddle_table();
  if (!tw) return NSQ_ERR_HIP;
  hipStream_t st = (hipStream_t)stream;
  float2* ws = nullptr;
  bool save = false;
  if (!p.fused) {
    const size_t need = causal_workspace_bytes(B, H, L, K, kbatch, NSQ_DIR_FWD);
    NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "fftconv1d_causal_fwd: workspace of %zu bytes required, got %zu",
                  need, workspace_bytes);
    ws = (float2*)workspace;
    save = workspace_bytes >= causal_workspace_bytes(B, H, L, K, kbatch, NSQ_DIR_BWD);
  }
  const int kf = kbatch != 1;
  bool ok = false;
  switch (dtype) {
    case NSQ_DTYPE_F32:
      ok = run_fwd<NSQ_DTYPE_F32>(p, x, k, shortcut, y, int(B), int(H), int(L), int(K), kf, ws, save, tw, st);
      break;
    case NSQ_DTYPE_BF16:
      ok = run_fwd<NSQ_DTYPE_BF16>(p, x, k, shortcut, y, int(B), int(H), int(L), int(K), kf, ws, save, tw, st);
      break;
    default:
      ok = run_fwd<NSQ_DTYPE_F16>(p, x, k, shortcut, y, int(B), int(H), int(L), int(K), kf, ws, save, tw, st);
      break;
  }
  NSQ_CHECK_ARG(ok, "fftconv1d_causal_fwd: no kernel for logN=%d", p.logN);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

static int causal_bwd(const void* g, const void* x, const float* k, const void* shortcut, void* gx, float* gk,
                      float* gs, int dtype, int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch, void* workspace,
                      size_t workspace_bytes, int fwd_state, void* stream) {
  clear_error();
  Plan1D p;
  int rc = validate(g, x, k, dtype, B, H, L, K, kbatch, p);
  if (rc) return rc;
  NSQ_CHECK_ARG(gx && gk, "fftconv1d_causal_bwd: null gradient output pointer");
  NSQ_CHECK_ARG(!shortcut || gs, "fftconv1d_causal_bwd: gs required when a shortcut is given");
  const float2* tw = twiddle_table();
  if (!tw) return NSQ_ERR_HIP;
  hipStream_t st = (hipStream_t)stream;
  float2* ws = nullptr;
  if (!p.fused) {
    const size_t need = causal_workspace_bytes(B, H, L, K, kbatch, NSQ_DIR_BWD);
    NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "fftconv1d_causal_bwd: workspace of %zu bytes required, got %zu",
                  need, workspace_bytes);
    ws = (float2*)workspace;
  }
  const int kf = kbatch != 1;
  const bool fs = fwd_state != 0;
  bool ok = false;
  switch (dtype) {
    case NSQ_DTYPE_F32:
      ok = run_bwd<NSQ_DTYPE_F32>(p, g, x, k, shortcut, gx, gk, gs, int(B), int(H), int(L), int(K), kf, ws, fs, tw, st);
      break;
    case NSQ_DTYPE_BF16:
      ok = run_bwd<NSQ_DTYPE_BF16>(p, g, x, k, shortcut, gx, gk, gs, int(B), int(H), int(L), int(K), kf, ws, fs, tw, st);
      break;
    default:
      ok = run_bwd<NSQ_DTYPE_F16>(p, g, x, k, shortcut, gx, gk, gs, int(B), int(H), int(L), int(K), kf, ws, fs, tw, st);
      break;
  }
  NSQ_CHECK_ARG(ok, "fftconv1d_causal_bwd: no kernel for logN=%d", p.logN);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

// Gated (Hyena) causal conv: the plain conv's checks plus gate codes and, for
// the elementwise kernels of the multi-kernel plan, 16-byte aligned tensors.
static size_t gated_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch, int dtype,
                                    int direction) {
  Plan1D p;
  if (!make_plan(L, K, p) || !valid_dtype(dtype)) return 0;
  if (gates_fused_1d(p, B * H * L) && direction == NSQ_DIR_FWD) return 0;  // one gated kernel
  const size_t conv = round256(causal_workspace_bytes(B, H, L, K, kbatch, direction));
  const size_t es = dtype == NSQ_DTYPE_F32 ? 4 : 2;
  return conv + size_t(direction == NSQ_DIR_BWD ? 3 : 2) * round256(size_t(B * H * L) * es);
}

static bool aligned16(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (p && (reinterpret_cast<uintptr_t>(p) & 15)) return false;
  return true;
}

static int validate_gate(int act1, int act2) {
  NSQ_CHECK_ARG(act1 >= 0 && act1 <= 2 && act2 >= 0 && act2 <= 2,
                "gated_fftconv1d: gate codes must be 0 (identity), 1 (sigmoid) or 2 (silu); got %d, %d", act1, act2);
  return NSQ_OK;
}

}  // namespace nsq

using namespace nsq;

extern "C" {

size_t nsq_fftconv1d_causal_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t K, int direction) {
  return causal_workspace_bytes(B, H, L, K, 1, direction);
}

int nsq_fftconv1d_causal_fwd(const void* x, const float* k, const void* shortcut, void* y, int dtype, int64_t B,
                             int64_t H, int64_t L, int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
  return causal_fwd(x, k, shortcut, y, dtype, B, H, L, K, 1, workspace, workspace_bytes, stream);
}

int nsq_fftconv1d_causal_bwd(const void* g, const void* x, const float* k, const void* shortcut, void* gx, float* gk,
                             float* gs, int dtype, int64_t B, int64_t H, int64_t L, int64_t K, void* workspace,
                             size_t workspace_bytes, int fwd_state, void* stream) {
  return causal_bwd(g, x, k, shortcut, gx, gk, gs, dtype, B, H, L, K, 1, workspace, workspace_bytes, fwd_state, stream);
}

size_t nsq_fftconv1d_causal_film_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch,
                                                 int direction) {
  return causal_workspace_bytes(B, H, L, K, kbatch, direction);
}

int nsq_fftconv1d_causal_film_fwd(const void* x, const float* k, const void* shortcut, void* y, int dtype, int64_t B,
                                  int64_t H, int64_t L, int64_t K, int64_t kbatch, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  return causal_fwd(x, k, shortcut, y, dtype, B, H, L, K, kbatch, workspace, workspace_bytes, stream);
}

int nsq_fftconv1d_causal_film_bwd(const void* g, const void* x, const float* k, const void* shortcut, void* gx,
                                  float* gk, float* gs, int dtype, int64_t B, int64_t H, int64_t L, int64_t K,
                                  int64_t kbatch, void* workspace, size_t workspace_bytes, int fwd_state,
                                  void* stream) {
  return causal_bwd(g, x, k, shortcut, gx, gk, gs, dtype, B, H, L, K, kbatch, workspace, workspace_bytes, fwd_state,
                    stream);
}

static int shifted_fwd(const char* op, const void* x, const float* k, const void* shortcut, void* y, int dtype,
                       int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch, bool zpad, void* workspace,
                       size_t workspace_bytes, int max_logn, void* stream) {
  clear_error();
  int logN = 0;
  int rc = validate_shifted(op, x, y, k, dtype, B, H, L, K, kbatch, zpad, logN, max_logn);
  if (rc) return rc;
  const float2* tw = twiddle_table();
  if (!tw) return NSQ_ERR_HIP;
  hipStream_t st = (hipStream_t)stream;
  const int kf = kbatch != 1;
  const int c = zpad ? int(K / 2) : int((K - 1) / 2);
  bool ok = false;
  if (logN > 13) {
    const size_t need = shifted_workspace_bytes(B, H, L, K, kbatch, dtype, zpad, NSQ_DIR_FWD);
    NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "%s: workspace of %zu bytes required, got %zu", op, need,
                  workspace_bytes);
    float2* ws = (float2*)workspace;
    void* roll = (char*)workspace + (need - size_t(B * H * (int64_t(2) << logN)) * (dtype == NSQ_DTYPE_F32 ? 4 : 2));
    const int b = int(B), h = int(H), l = int(L), kk = int(K);
    switch (dtype) {
      case NSQ_DTYPE_F32:
        ok = run_shift4_fwd<NSQ_DTYPE_F32>(logN, x, k, shortcut, y, b, h, l, kk, kf, c, zpad, roll, ws, tw, st);
        break;
      case NSQ_DTYPE_BF16:
        ok = run_shift4_fwd<NSQ_DTYPE_BF16>(logN, x, k, shortcut, y, b, h, l, kk, kf, c, zpad, roll, ws, tw, st);
        break;
      default:
        ok = run_shift4_fwd<NSQ_DTYPE_F16>(logN, x, k, shortcut, y, b, h, l, kk, kf, c, zpad, roll, ws, tw, st);
        break;
    }
    NSQ_CHECK_ARG(ok, "%s: no kernel for logN=%d", op, logN);
    NSQ_CHECK_LAUNCH();
    return NSQ_OK;
  }
  switch (dtype) {
    case NSQ_DTYPE_F32:
      ok = run_circ_fwd<NSQ_DTYPE_F32>(logN, x, k, shortcut, y, int(B), int(H), int(L), int(K), kf, c, zpad, tw, st);
      break;
    case NSQ_DTYPE_BF16:
      ok = run_circ_fwd<NSQ_DTYPE_BF16>(logN, x, k, shortcut, y, int(B), int(H), int(L), int(K), kf, c, zpad, tw, st);
      break;
    default:
      ok = run_circ_fwd<NSQ_DTYPE_F16>(logN, x, k, shortcut, y, int(B), int(H), int(L), int(K), kf, c, zpad, tw, st);
      break;
  }
  NSQ_CHECK_ARG(ok, "%s: no kernel for logN=%d", op, logN);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

static int shifted_bwd(const char* op, const void* g, const void* x, const float* k, const void* shortcut, void* gx,
                       float* gk, float* gs, int dtype, int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch,
                       bool zpad, void* workspace, size_t workspace_bytes, int max_logn, void* stream) {
  clear_error();
  int logN = 0;
  int rc = validate_shifted(op, g, x, k, dtype, B, H, L, K, kbatch, zpad, logN, max_logn);
  if (rc) return rc;
  NSQ_CHECK_ARG(gx && gk, "%s: null gradient output pointer", op);
  NSQ_CHECK_ARG(!shortcut || gs, "%s: gs required when a shortcut is given", op);
  const float2* tw = twiddle_table();
  if (!tw) return NSQ_ERR_HIP;
  hipStream_t st = (hipStream_t)stream;
  const int kf = kbatch != 1;
  const int c = zpad ? int(K / 2) : int((K - 1) / 2);
  const int b = int(B), h = int(H), l = int(L), kk = int(K);
  bool ok = false;
  if (logN > 13) {
    const size_t need = shifted_workspace_bytes(B, H, L, K, kbatch, dtype, zpad, NSQ_DIR_BWD);
    NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "%s: workspace of %zu bytes required, got %zu", op, need,
                  workspace_bytes);
    float2* ws = (float2*)workspace;
    void* roll = (char*)workspace + (need - size_t(B * H * (int64_t(2) << logN)) * (dtype == NSQ_DTYPE_F32 ? 4 : 2));
    switch (dtype) {
      case NSQ_DTYPE_F32:
        ok = run_shift4_bwd<NSQ_DTYPE_F32>(logN, g, x, k, shortcut, gx, gk, gs, b, h, l, kk, kf, c, zpad, roll, ws,
                                           tw, st);
        break;
      case NSQ_DTYPE_BF16:
        ok = run_shift4_bwd<NSQ_DTYPE_BF16>(logN, g, x, k, shortcut, gx, gk, gs, b, h, l, kk, kf, c, zpad, roll, ws,
                                            tw, st);
        break;
      default:
        ok = run_shift4_bwd<NSQ_DTYPE_F16>(logN, g, x, k, shortcut, gx, gk, gs, b, h, l, kk, kf, c, zpad, roll, ws,
                                           tw, st);
        break;
    }
    NSQ_CHECK_ARG(ok, "%s: no kernel for logN=%d", op, logN);
    NSQ_CHECK_LAUNCH();
    return NSQ_OK;
  }
  switch (dtype) {
    case NSQ_DTYPE_F32:
      ok = run_circ_bwd<NSQ_DTYPE_F32>(logN, g, x, k, shortcut, gx, gk, gs, b, h, l, kk, kf, c, zpad, tw, st);
      break;
    case NSQ_DTYPE_BF16:
      ok = run_circ_bwd<NSQ_DTYPE_BF16>(logN, g, x, k, shortcut, gx, gk, gs, b, h, l, kk, kf, c, zpad, tw, st);
      break;
    default:
      ok = run_circ_bwd<NSQ_DTYPE_F16>(logN, g, x, k, shortcut, gx, gk, gs, b, h, l, kk, kf, c, zpad, tw, st);
      break;
  }
  NSQ_CHECK_ARG(ok, "%s: no kernel for logN=%d", op, logN);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

int nsq_circular_fftconv1d_fwd(const void* x, const float* k, const void* shortcut, void* y, int dtype, int64_t B,
                               int64_t H, int64_t L, int64_t K, int64_t kbatch, void* stream) {
  return shifted_fwd("circular_fftconv1d_fwd", x, k, shortcut, y, dtype, B, H, L, K, kbatch, false, nullptr, 0, 13,
                     stream);
}

int nsq_circular_fftconv1d_bwd(const void* g, const void* x, const float* k, const void* shortcut, void* gx,
                               float* gk, float* gs, int dtype, int64_t B, int64_t H, int64_t L, int64_t K,
                               int64_t kbatch, void* stream) {
  return shifted_bwd("circular_fftconv1d_bwd", g, x, k, shortcut, gx, gk, gs, dtype, B, H, L, K, kbatch, false,
                     nullptr, 0, 13, stream);
}

size_t nsq_mixed_fftconv1d_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch,
                                           unsigned periodic, int dtype, int direction) {
  if (periodic > 1u) return 0;
  return shifted_workspace_bytes(B, H, L, K, kbatch, dtype, periodic == 0, direction);
}

int nsq_mixed_fftconv1d_fwd(const void* x, const float* k, const void* shortcut, void* y, int dtype, int64_t B,
                            int64_t H, int64_t L, int64_t K, int64_t kbatch, unsigned periodic, void* workspace,
                            size_t workspace_bytes, void* stream) {
  clear_error();
  NSQ_CHECK_ARG(periodic <= 1u, "mixed_fftconv1d_fwd: periodic mask 0x%x names an axis >= 1", periodic);
  return shifted_fwd(periodic ? "mixed_fftconv1d_fwd (periodic)" : "mixed_fftconv1d_fwd (zero-padded)", x, k,
                     shortcut, y, dtype, B, H, L, K, kbatch, periodic == 0, workspace, workspace_bytes, kMaxLogN, stream);
}

int nsq_mixed_fftconv1d_bwd(const void* g, const void* x, const float* k, const void* shortcut, void* gx, float* gk,
                            float* gs, int dtype, int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch,
                            unsigned periodic, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  NSQ_CHECK_ARG(periodic <= 1u, "mixed_fftconv1d_bwd: periodic mask 0x%x names an axis >= 1", periodic);
  return shifted_bwd(periodic ? "mixed_fftconv1d_bwd (periodic)" : "mixed_fftconv1d_bwd (zero-padded)", g, x, k,
                     shortcut, gx, gk, gs, dtype, B, H, L, K, kbatch, periodic == 0, workspace, workspace_bytes, kMaxLogN,
                     stream);
}

size_t nsq_gated_fftconv1d_causal_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t K, int64_t kbatch,
                                                  int dtype, int direction) {
  return gated_workspace_bytes(B, H, L, K, kbatch, dtype, direction);
}

int nsq_gated_fftconv1d_causal_fwd(const void* q, const void* kgate, const void* v, const float* k,
                                   const void* shortcut, void* y, void* y1, int dtype, int act1, int act2, int64_t B,
                                   int64_t H, int64_t L, int64_t K, int64_t kbatch, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  clear_error();
  Plan1D p;
  int rc = validate(q, y, k, dtype, B, H, L, K, kbatch, p);
  if (rc) return rc;
  rc = validate_gate(act1, act2);
  if (rc) return rc;
  NSQ_CHECK_ARG(kgate && v, "gated_fftconv1d_fwd: null gate input pointer");
  const bool one_kernel = gates_fused_1d(p, B * H * L);
  NSQ_CHECK_ARG(one_kernel || aligned16({q, kgate, v, y, y1}), "gated_fftconv1d_fwd: tensors must be 16-byte aligned");
  const float2* tw = twiddle_table();
  if (!tw) return NSQ_ERR_HIP;
  hipStream_t st = (hipStream_t)stream;
  float2* ws = nullptr;
  void* gws = nullptr;
  if (!one_kernel) {
    const size_t need = gated_workspace_bytes(B, H, L, K, kbatch, dtype, NSQ_DIR_FWD);
    NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "gated_fftconv1d_fwd: workspace of %zu bytes required, got %zu",
                  need, workspace_bytes);
    ws = (float2*)workspace;
    gws = (char*)workspace + round256(causal_workspace_bytes(B, H, L, K, kbatch, NSQ_DIR_FWD));
  }
  const GateArgs ga{kgate, v, y1, nullptr, nullptr, act1, act2};
  const int kf = kbatch != 1;
  bool ok = false;
  switch (dtype) {
    case NSQ_DTYPE_F32:
      ok = run_gated_fwd<NSQ_DTYPE_F32>(p, q, k, shortcut, y, int(B), int(H), int(L), int(K), kf, ga, gws, ws, tw, st);
      break;
    case NSQ_DTYPE_BF16:
      ok = run_gated_fwd<NSQ_DTYPE_BF16>(p, q, k, shortcut, y, int(B), int(H), int(L), int(K), kf, ga, gws, ws, tw, st);
      break;
    default:
      ok = run_gated_fwd<NSQ_DTYPE_F16>(p, q, k, shortcut, y, int(B), int(H), int(L), int(K), kf, ga, gws, ws, tw, st);
      break;
  }
  NSQ_CHECK_ARG(ok, "gated_fftconv1d_fwd: no kernel for logN=%d", p.logN);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

int nsq_gated_fftconv1d_causal_bwd(const void* g, const void* q, const void* kgate, const void* v, const void* y1,
                                   const float* k, const void* shortcut, void* dq, void* dkgate, void* dv, float* gk,
                                   float* gs, int dtype, int act1, int act2, int64_t B, int64_t H, int64_t L,
                                   int64_t K, int64_t kbatch, int fuse_gates, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  clear_error();
  Plan1D p;
  int rc = validate(g, q, k, dtype, B, H, L, K, kbatch, p);
  if (rc) return rc;
  rc = validate_gate(act1, act2);
  if (rc) return rc;
  NSQ_CHECK_ARG(kgate && v && y1, "gated_fftconv1d_bwd: null gate input pointer (y1 is required)");
  NSQ_CHECK_ARG(dq && dkgate && dv && gk, "gated_fftconv1d_bwd: null gradient output pointer");
  NSQ_CHECK_ARG(!shortcut || gs, "gated_fftconv1d_bwd: gs required when a shortcut is given");
  NSQ_CHECK_ARG(fuse_gates == 0, "gated_fftconv1d_bwd: fuse_gates is reserved and must be 0");
  NSQ_CHECK_ARG(aligned16({g, q, kgate, v, y1, dq, dkgate, dv}), "gated_fftconv1d_bwd: tensors must be 16-byte aligned");
  const float2* tw = twiddle_table();
  if (!tw) return NSQ_ERR_HIP;
  hipStream_t st = (hipStream_t)stream;
  const size_t need = gated_workspace_bytes(B, H, L, K, kbatch, dtype, NSQ_DIR_BWD);
  NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "gated_fftconv1d_bwd: workspace of %zu bytes required, got %zu",
                need, workspace_bytes);
  float2* ws = (float2*)workspace;
  void* gws = (char*)workspace + round256(causal_workspace_bytes(B, H, L, K, kbatch, NSQ_DIR_BWD));
  const GateArgs ga{kgate, v, const_cast<void*>(y1), dkgate, dv, act1, act2};
  const int kf = kbatch != 1;
  bool ok = false;
  switch (dtype) {
    case NSQ_DTYPE_F32:
      ok = run_gated_bwd<NSQ_DTYPE_F32>(p, g, q, k, shortcut, dq, gk, gs, int(B), int(H), int(L), int(K), kf, ga, gws,
                                        ws, tw, st);
      break;
    case NSQ_DTYPE_BF16:
      ok = run_gated_bwd<NSQ_DTYPE_BF16>(p, g, q, k, shortcut, dq, gk, gs, int(B), int(H), int(L), int(K), kf, ga, gws,
                                         ws, tw, st);
      break;
    default:
      ok = run_gated_bwd<NSQ_DTYPE_F16>(p, g, q, k, shortcut, dq, gk, gs, int(B), int(H), int(L), int(K), kf, ga, gws,
                                        ws, tw, st);
      break;
  }
  NSQ_CHECK_ARG(ok, "gated_fftconv1d_bwd: no kernel for logN=%d", p.logN);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

}  // extern "C"
