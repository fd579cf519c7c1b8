// Causal 1D FFT convolution with a SIREN filter that never reaches HBM (see include/nsq_hip.h).
//
// nvsubquadratic/modules/ckconv_nd.py:1149-1164 generates the filter k = W_out a + b_out from the SIREN
// activations a [HD][K] (kernels_nd.py:1181-1189), crops it to the causal half and hands it to the causal FFT
// conv (ops/fftconv.py:546-600).  On the 4-step plan the column pass C is linear, so the filter's column
// transforms are
//   C(k_h) = sum_j W_out[h][j] C(a_j) + b_out[h] C(1_K):
// the HD + 1 activation rows (the last one is the ones row) are transformed once, A' = C(a) ((HD + 1) x N
// complex), and siren_spectrum_kernel forms every channel's C(k_h) from them straight into the conv's filter
// block.  k [H][K] is never written or read back.
//
// Backward.  The inverse column pass D turns the filter gradient's spectrum P'_h (what the row pass leaves in
// the filter block) into gk_h = D(P'_h)[0:K]; D's adjoint is C / N, so
//   dW_out[h][j] = <gk_h, a_j> = <P'_h, A'_j> / N,    db_out[h] = <P'_h, A'_HD> / N,
//   ga_j = sum_h W_out[h][j] gk_h = D(Q'_j)[0:K],       Q'_j = sum_h W_out[h][j] P'_h,
//   gs[h] = gk_h[0] = (1/N) sum_{k1} Re P'_h[k1][n2 = 0]
// (<u, v> the real inner product of the interleaved (re, im) floats).  The readout's one-pass gradient kernel
// reads P' once, as it reads gk on the unfused path (gk -> P', a -> A', G -> 2N floats, the bias gradient
// weighted by A'_HD, sums scaled by 1/N); the inverse column pass turns the HD rows of Q' into ga.  gk is never
// written.
#include "fftconv1d_impl.h"
#include "siren_readout.h"

namespace nsq {
namespace {

// K'[h][r] = sum_{j < HD} W_out[h][j] A'[j][r] + b_out[h] A'[HD][r] for the r < n floats of a row (n = 2N, a
// multiple of 256), on the matrix cores: v_mfma_f32_16x16x4_f32 (fp32 products, fp32 accumulation) with
// D[m = point][n = channel] = sum_k A[m][k] B[k][n], A[m][k] = A'[k][point], B[k][n] = W~[channel][k], W~ = [W_out |
// b_out | 0] (HD + 1 columns padded to S = 4 KS).  Lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16] and
// receives D[4 (l / 16) + r][l % 16]: four consecutive points of one channel, one 16-byte store.  A wave owns 64
// points (4 tiles of 16) and holds their A operands for the whole channel sweep; W~ comes through LDS in chunks of
// 64 channels, double-buffered (the next chunk's words are loaded while this one's products run).  The B reads
// (rows of S words, S = 20, 36 or 68) hit 64 distinct banks.
typedef float spec_f32x4 __attribute__((ext_vector_type(4)));

template <int HD>
struct SpecCfg {
  static constexpr int KS = (HD + 1 + 3) / 4;  // k-steps of 4
  static constexpr int S = 4 * KS;             // LDS words per channel
  static constexpr int CH = 64;                // channels per LDS chunk
  static constexpr int PT = CH * S / 256;      // chunk words per thread (= KS)
};

template <int HD>
__global__ __launch_bounds__(256) void siren_spectrum_kernel(const float* __restrict__ wout,
                                                             const float* __restrict__ bout,
                                                             const float* __restrict__ A, int64_t n, int H,
                                                             int chunks_per_slice, float* __restrict__ out) {
  using C = SpecCfg<HD>;
  __shared__ float wl[2][C::CH * C::S];
  const int t = int(threadIdx.x), wv = t >> 6, l = t & 63, i = l & 15, kk = l >> 4;
  const int64_t p0 = int64_t(blockIdx.x) * 256 + 64 * wv;  // the wave's first float of every row
  float a[4][C::KS];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      const int j = 4 * ks + kk;
      a[mt][ks] = j <= HD ? A[int64_t(j) * n + p0 + 16 * mt + i] : 0.f;
    }
  const int nch = int((H + C::CH - 1) / C::CH);
  const int c0 = int(blockIdx.y) * chunks_per_slice;
  const int c1 = c0 + chunks_per_slice < nch ? c0 + chunks_per_slice : nch;
  float v[C::PT];
  auto fetch = [&](int c) {  // word e = t + 256 u of chunk c: channel e / S, column e % S
#pragma unroll
    for (int u = 0; u < C::PT; ++u) {
      const int e = t + 256 * u, ch = e / C::S, j = e - ch * C::S, h = c * C::CH + ch;
      v[u] = h >= H ? 0.f : (j < HD ? wout[int64_t(h) * HD + j] : (j == HD && bout ? bout[h] : 0.f));
    }
  };
  if (c0 >= c1) return;  // workgroup-uniform
  fetch(c0);
#pragma unroll
  for (int u = 0; u < C::PT; ++u) wl[0][t + 256 * u] = v[u];
  __syncthreads();
  for (int c = c0; c < c1; ++c) {
    const int buf = (c - c0) & 1;
    if (c + 1 < c1) fetch(c + 1);
    const float* w = wl[buf];
#pragma unroll
    for (int nt = 0; nt < C::CH / 16; ++nt) {
      spec_f32x4 d[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) d[mt] = spec_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) {
        const float b = w[(16 * nt + i) * C::S + 4 * ks + kk];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) d[mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[mt][ks], b, d[mt], 0, 0, 0);
      }
      const int h = c * C::CH + 16 * nt + i;
      if (h < H) {
        float* o = out + int64_t(h) * n + p0 + 4 * kk;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
          *reinterpret_cast<float4*>(o + 16 * mt) = make_float4(d[mt][0], d[mt][1], d[mt][2], d[mt][3]);
      }
    }
    if (c + 1 < c1) {
#pragma unroll
      for (int u = 0; u < C::PT; ++u) wl[buf ^ 1][t + 256 * u] = v[u];
    }
    __syncthreads();
  }
}

// gs[h] = scale * sum_{k1 < N1} Re spec[h][k1 * N2]: one wave per channel, lanes over k1 in order, a fixed
// butterfly across the wave.
__global__ __launch_bounds__(256) void siren_lag0_kernel(const float2* __restrict__ spec, int64_t N, int N1, int N2,
                                                         int H, float scale, float* __restrict__ gs) {
  const int h = int(blockIdx.x) * 4 + int(threadIdx.x >> 6);
  const int l = int(threadIdx.x & 63);
  if (h >= H) return;  // wave-uniform
  const float2* row = spec + int64_t(h) * N;
  float a = 0.f;
  for (int k1 = l; k1 < N1; k1 += 64) a += row[int64_t(k1) * N2].x;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) a += __shfl_xor(a, o);
  if (l == 0) gs[h] = a * scale;
}

constexpr int kSirenConvMaxLogN = 22;  // rows of 2N <= 2^23 floats: the readout gradient kernel's limit

size_t al256(size_t v) { return (v + 255) / 256 * 256; }

// Workspace: the 4-step blocks x, k, g (N complex values each: B*H, H, B*H rows), A' (HD + 1 rows), Q' (HD
// rows), then the readout gradient's partials.  One size for both directions: the forward keeps x's and k's
// column transforms and A' for the backward.
struct SirenConvWs {
  size_t a, q, rb, total;  // byte offsets
};

SirenConvWs siren_conv_ws(int64_t B, int64_t H, int HD, int logN) {
  const int64_t N = int64_t(1) << logN;
  SirenConvWs w{};
  w.a = al256(size_t(2 * B * H + H) * size_t(N) * sizeof(float2));
  w.q = w.a + al256(size_t(HD + 1) * size_t(N) * sizeof(float2));
  w.rb = w.q + al256(size_t(HD) * size_t(N) * sizeof(float2));
  w.total = w.rb + al256(siren_readout_bwd_ws_floats(H, HD, 2 * N, 1) * sizeof(float));
  return w;
}

int validate_siren_conv(const char* op, const void* a, const void* b, const float* act, int64_t lda,
                        const float* wout, int HD, int dtype, int64_t B, int64_t H, int64_t L, int64_t K, Plan1D& p) {
  NSQ_CHECK_ARG(a && b && act && wout, "%s: null tensor pointer", op);
  NSQ_CHECK_ARG(valid_dtype(dtype), "%s: unsupported dtype code %d", op, dtype);
  NSQ_CHECK_ARG(B >= 1 && H >= 1 && L >= 1 && K >= 1, "%s: sizes must be positive (B=%lld H=%lld L=%lld K=%lld)",
                op, (long long)B, (long long)H, (long long)L, (long long)K);
  NSQ_CHECK_ARG(K <= 2 * L, "%s: kernel length %lld exceeds 2*seq_len=%lld", op, (long long)K, (long long)(2 * L));
  NSQ_CHECK_ARG(lda >= K, "%s: activation row stride %lld below the filter length %lld", op, (long long)lda,
                (long long)K);
  NSQ_CHECK_ARG(H <= (int64_t(1) << 20) && B * H <= 0x7fffffff && L <= (int64_t(1) << 30), "%s: tensor too large",
                op);
  if (!(HD == 16 || HD == 32 || HD == 64)) {
    set_error("%s: mlp_hidden_dim %d must be 16, 32 or 64", op, HD);
    return NSQ_ERR_UNSUPPORTED;
  }
  if (!make_plan(L, K, p) || p.fused || p.fold || p.logN > kSirenConvMaxLogN) {
    set_error("%s: unsupported (L=%lld, K=%lld): the filter-free path runs the 4-step plan, FFT lengths 2^15 .. 2^23 "
              "with K <= L + 1; shorter convs read the filter (nsq_siren_readout_fwd, then nsq_fftconv1d_causal_*)",
              op, (long long)L, (long long)K);
    return NSQ_ERR_UNSUPPORTED;
  }
  const int l1 = split_log_n1(p.logN);
  NSQ_CHECK_ARG(B * H * (int64_t(1) << (l1 - 1 > 9 ? l1 - 1 : 9)) < (int64_t(1) << 31),
                "%s: B*H=%lld too large for the 4-step plan", op, (long long)(B * H));
  return NSQ_OK;
}

// A' = C(act rows) into ws + w.a, then K' into the conv's filter block.
bool filter_spectrum(const Plan1D& p, const float* act, int64_t lda, const float* wout, const float* bout, int HD,
                     int64_t B, int64_t H, int64_t K, char* ws, const SirenConvWs& w, const float2* tw,
                     hipStream_t st) {
  const int64_t N = int64_t(1) << p.logN;
  float2* wsa = reinterpret_cast<float2*>(ws + w.a);
  if (!run_col_fwd_rows<0>(p.logN, act, lda, K, HD + 1, wsa, tw, st)) return false;
  const int64_t n = 2 * N;
  const unsigned gx = unsigned(n / 256);
  const int64_t nch = ceil_div(H, int64_t(64));  // 64-channel chunks
  int64_t hs = ceil_div(int64_t(2048), int64_t(gx));  // channel slices so the grid reaches ~2048 workgroups
  hs = hs < 1 ? 1 : (hs > nch ? nch : hs);
  const int cps = int(ceil_div(nch, hs));
  const dim3 grid(gx, unsigned(ceil_div(nch, int64_t(cps))));
  float* wsk = reinterpret_cast<float*>(reinterpret_cast<float2*>(ws) + B * H * N);
  const float* A = reinterpret_cast<const float*>(wsa);
  switch (HD) {
    case 16:
      hipLaunchKernelGGL(siren_spectrum_kernel<16>, grid, dim3(256), 0, st, wout, bout, A, n, int(H), cps, wsk);
      break;
    case 32:
      hipLaunchKernelGGL(siren_spectrum_kernel<32>, grid, dim3(256), 0, st, wout, bout, A, n, int(H), cps, wsk);
      break;
    default:
      hipLaunchKernelGGL(siren_spectrum_kernel<64>, grid, dim3(256), 0, st, wout, bout, A, n, int(H), cps, wsk);
      break;
  }
  return true;
}

}  // namespace
}  // namespace nsq

extern "C" {

size_t nsq_siren_fftconv1d_causal_workspace_bytes(int64_t B, int64_t H, int64_t L, int64_t K, int HD) {
  nsq::Plan1D p;
  if (B < 1 || H < 1 || L < 1 || K < 1 || K > 2 * L || !(HD == 16 || HD == 32 || HD == 64)) return 0;
  if (!nsq::make_plan(L, K, p) || p.fused || p.fold || p.logN > nsq::kSirenConvMaxLogN) return 0;
  return nsq::siren_conv_ws(B, H, HD, p.logN).total;
}

int nsq_siren_fftconv1d_causal_fwd(const void* x, const float* act, int64_t lda, const float* wout,
                                   const float* bout, int HD, const void* shortcut, void* y, int dtype, int64_t B,
                                   int64_t H, int64_t L, int64_t K, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  using namespace nsq;
  clear_error();
  Plan1D p;
  const int rc = validate_siren_conv("siren_fftconv1d_causal_fwd", x, y, act, lda, wout, HD, dtype, B, H, L, K, p);
  if (rc) return rc;
  const SirenConvWs w = siren_conv_ws(B, H, HD, p.logN);
  NSQ_CHECK_ARG(workspace && workspace_bytes >= w.total && (reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
                "siren_fftconv1d_causal_fwd: 256-byte aligned workspace of %zu bytes required, got %zu", w.total,
                workspace_bytes);
  const float2* tw = twiddle_table();
  if (!tw) return NSQ_ERR_HIP;
  hipStream_t st = (hipStream_t)stream;
  char* ws = static_cast<char*>(workspace);
  bool ok = filter_spectrum(p, act, lda, wout, bout, HD, B, H, K, ws, w, tw, st);
  float2* cws = reinterpret_cast<float2*>(ws);
  if (ok) {
    switch (dtype) {
      case NSQ_DTYPE_F32:
        ok = run_fwd<NSQ_DTYPE_F32>(p, x, nullptr, shortcut, y, int(B), int(H), int(L), int(K), 0, cws, true, tw, st);
        break;
      case NSQ_DTYPE_BF16:
        ok = run_fwd<NSQ_DTYPE_BF16>(p, x, nullptr, shortcut, y, int(B), int(H), int(L), int(K), 0, cws, true, tw, st);
        break;
      default:
        ok = run_fwd<NSQ_DTYPE_F16>(p, x, nullptr, shortcut, y, int(B), int(H), int(L), int(K), 0, cws, true, tw, st);
        break;
    }
  }
  NSQ_CHECK_ARG(ok, "siren_fftconv1d_causal_fwd: no kernel for logN=%d", p.logN);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

int nsq_siren_fftconv1d_causal_bwd(const void* g, const void* x, const float* act, int64_t lda, const float* wout,
                                   const float* bout, int HD, const void* shortcut, void* gx, float* gact,
                                   float* gwout, float* gbout, float* gs, int dtype, int64_t B, int64_t H, int64_t L,
                                   int64_t K, void* workspace, size_t workspace_bytes, int fwd_state, void* stream) {
  using namespace nsq;
  clear_error();
  Plan1D p;
  const int rc = validate_siren_conv("siren_fftconv1d_causal_bwd", g, x, act, lda, wout, HD, dtype, B, H, L, K, p);
  if (rc) return rc;
  NSQ_CHECK_ARG(gx && gact && gwout, "siren_fftconv1d_causal_bwd: null gradient output pointer");
  NSQ_CHECK_ARG(!shortcut || gs, "siren_fftconv1d_causal_bwd: gs required when a shortcut is given");
  const SirenConvWs w = siren_conv_ws(B, H, HD, p.logN);
  NSQ_CHECK_ARG(workspace && workspace_bytes >= w.total && (reinterpret_cast<uintptr_t>(workspace) & 255) == 0,
                "siren_fftconv1d_causal_bwd: 256-byte aligned workspace of %zu bytes required, got %zu", w.total,
                workspace_bytes);
  const float2* tw = twiddle_table();
  if (!tw) return NSQ_ERR_HIP;
  hipStream_t st = (hipStream_t)stream;
  char* ws = static_cast<char*>(workspace);
  float2* cws = reinterpret_cast<float2*>(ws);
  const int64_t N = int64_t(1) << p.logN;
  bool ok = fwd_state ? true : filter_spectrum(p, act, lda, wout, bout, HD, B, H, K, ws, w, tw, st);
  if (ok) {
    const bool fs = fwd_state != 0;
    switch (dtype) {
      case NSQ_DTYPE_F32:
        ok = run_bwd<NSQ_DTYPE_F32>(p, g, x, nullptr, shortcut, gx, nullptr, nullptr, int(B), int(H), int(L), int(K),
                                    0, cws, fs, tw, st);
        break;
      case NSQ_DTYPE_BF16:
        ok = run_bwd<NSQ_DTYPE_BF16>(p, g, x, nullptr, shortcut, gx, nullptr, nullptr, int(B), int(H), int(L),
                                     int(K), 0, cws, fs, tw, st);
        break;
      default:
        ok = run_bwd<NSQ_DTYPE_F16>(p, g, x, nullptr, shortcut, gx, nullptr, nullptr, int(B), int(H), int(L), int(K),
                                    0, cws, fs, tw, st);
        break;
    }
  }
  NSQ_CHECK_ARG(ok, "siren_fftconv1d_causal_bwd: no kernel for logN=%d", p.logN);
  const float2* spec = cws + B * H * N;  // the filter gradient's column-pass spectrum P'
  const float scale = 1.f / float(N);
  if (shortcut) {
    const int l1 = split_log_n1(p.logN);
    hipLaunchKernelGGL(siren_lag0_kernel, dim3(unsigned(ceil_div(H, int64_t(4)))), dim3(256), 0, st, spec, N,
                       1 << l1, int(N >> l1), int(H), scale, gs);
  }
  const float* A = reinterpret_cast<const float*>(ws + w.a);
  float* Q = reinterpret_cast<float*>(ws + w.q);
  ok = siren_readout_bwd_run(reinterpret_cast<const float*>(spec), 2 * N, A, 2 * N, gbout ? A + HD * 2 * N : nullptr,
                             wout, H, HD, 2 * N, 1, Q, gwout, gbout, scale, reinterpret_cast<float*>(ws + w.rb), st);
  NSQ_CHECK_ARG(ok, "siren_fftconv1d_causal_bwd: mlp_hidden_dim %d", HD);
  ok = run_col_inv_rows<0>(p.logN, reinterpret_cast<const float2*>(Q), gact, nullptr, HD, int(K), tw, st);
  NSQ_CHECK_ARG(ok, "siren_fftconv1d_causal_bwd: no kernel for logN=%d", p.logN);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

}  // extern "C"
