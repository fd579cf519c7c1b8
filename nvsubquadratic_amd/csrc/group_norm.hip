// Hyena's pixelhyena_norm site with torch.nn.GroupNorm(num_groups, C) (the
// reference's configs use num_groups = 1, e.g. examples/imagenet_classification/
// ccnn_7_512_hyena.py), which hyena_nd.py:548-550 applies channels-first to
// z = q * act(k) (hyena_nd.py:546): per sample b and group g of C / G channels,
// over those channels and every position,
//   mu, var = mean and biased variance of u, r = rsqrt(var + eps),
//   out[b,c,s] = round(u a + h),  a = r w[c],  h = bias[c] - mu a
// (torch's group norm scale / shift form), u = round(y * round(act(v))) or y.
//
// Channels-first, a group is C / G consecutive rows of S values, so the passes
// are plain streams over [B, C, S]:
//   gn_row_stats   one wave per (b, c) row: mean and M2 of the row from sums
//                  of u - u[0] (shifted data, no cancellation for a large mean);
//   gn_finalize    one wave per (b, g): the rows combined in a fixed order
//                  (Chan et al.'s update for equal counts, in double) -> mean,
//                  rstd (kept for the backward);
//   gn_apply       out, 16-byte accesses where rows allow;
// backward, with xhat = (u - mu) r and g = w dout:
//   gn_row_bwd     per row: s1 = sum dout xhat, s2 = sum dout;
//   gn_finalize_bwd per (b, g): mean_g(g xhat) = sum_c w s1 / n, mean_g(g) =
//                  sum_c w s2 / n; per channel dw = sum_b s1, dbias = sum_b s2
//                  (fixed order: deterministic);
//   gn_apply_bwd   du = round(r (g - mean(g) - xhat mean(g xhat))), then the
//                  gate's adjoint as the other norm passes round it.
#include "gate.h"
#include "nsq_common.h"

#include <initializer_list>

namespace nsq {
namespace {

constexpr int kGnT = 256;      // threads per workgroup
constexpr int kGnRowsPerWG = 4;  // row passes: one wave per row
constexpr int kGnVecIter = 4;  // apply passes: vectors per thread

template <int DT, int VW>
__device__ __forceinline__ void gn_load(const typename Elem<DT>::T* p, int64_t i, float (&o)[VW]) {
  using T = typename Elem<DT>::T;
  if constexpr (VW == 1) {
    o[0] = Elem<DT>::load(p, i);
  } else {
    static_assert(VW * sizeof(T) == 16, "16-byte vectors");
    const uint4 u = *reinterpret_cast<const uint4*>(p + i);
    const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
    for (int k = 0; k < VW; ++k) o[k] = Elem<DT>::load(e, k);
  }
}

template <int DT, int VW>
__device__ __forceinline__ void gn_store(typename Elem<DT>::T* p, int64_t i, const float (&o)[VW]) {
  using T = typename Elem<DT>::T;
  if constexpr (VW == 1) {
    Elem<DT>::store(p, i, o[0]);
  } else {
    uint4 u;
    T* e = reinterpret_cast<T*>(&u);
#pragma unroll
    for (int k = 0; k < VW; ++k) Elem<DT>::store(e, k, o[k]);
    *reinterpret_cast<uint4*>(p + i) = u;
  }
}

// u of VW consecutive values (y alone without a gate)
template <int DT, int VW>
__device__ __forceinline__ void gn_u(const typename Elem<DT>::T* y, const typename Elem<DT>::T* v, int act,
                                     int64_t i, float (&u)[VW], float (&yv)[VW], float (&vv)[VW]) {
#pragma clang fp contract(off)
  gn_load<DT, VW>(y, i, yv);
  if (v) {
    gn_load<DT, VW>(v, i, vv);
#pragma unroll
    for (int k = 0; k < VW; ++k) u[k] = Elem<DT>::round(yv[k] * Elem<DT>::round(gate_act(act, vv[k])));
  } else {
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      u[k] = yv[k];
      vv[k] = 0.f;
    }
  }
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

template <int DT, int VW>
__global__ __launch_bounds__(kGnT) void gn_row_stats_kernel(const typename Elem<DT>::T* __restrict__ y,
                                                            const typename Elem<DT>::T* __restrict__ v, int act,
                                                            int64_t rows, int64_t S, float2* __restrict__ rowst) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * kGnRowsPerWG + (threadIdx.x >> 6);
  if (r >= rows) return;  // a whole wave; the kernel has no barrier
  const int64_t base = r * S;
  float u0[1], t0[1], t1[1];
  gn_u<DT, 1>(y, v, act, base, u0, t0, t1);
  const float sh = u0[0];
  float s = 0.f, ss = 0.f;
#pragma unroll 4
  for (int64_t i = int64_t(lane) * VW; i < S; i += 64 * VW) {
    float u[VW], yv[VW], vv[VW];
    gn_u<DT, VW>(y, v, act, base + i, u, yv, vv);
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      const float d = u[k] - sh;
      s += d;
      ss = fmaf(d, d, ss);
    }
  }
  s = wave_sum(s);
  ss = wave_sum(ss);
  if (lane == 0) {
    const float n = float(S);
    rowst[r] = make_float2(sh + s / n, fmaxf(ss - s * (s / n), 0.f));
  }
}

__device__ __forceinline__ double wave_sum_d(double x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

// One wave per (b, g), the group's rows (n = S each) combined in a fixed order:
// mean = the average of the row means, M2 = sum_r (M2_r + S (mean_r - mean)^2)
// (the pairwise update of Chan et al. for equal counts), in double.
__global__ __launch_bounds__(kGnT) void gn_finalize_kernel(const float2* __restrict__ rowst, int64_t BG, int C,
                                                           int G, int64_t S, float eps, float* __restrict__ mean,
                                                           float* __restrict__ rstd) {
  const int lane = threadIdx.x & 63;
  const int64_t i = int64_t(blockIdx.x) * kGnRowsPerWG + (threadIdx.x >> 6);
  if (i >= BG) return;  // a whole wave
  const int cpg = C / G;
  const int64_t b = i / G, g = i - b * G;
  const float2* rs = rowst + b * C + g * cpg;
  double sm = 0.0;
  for (int c = lane; c < cpg; c += 64) sm += double(rs[c].x);
  const double m = wave_sum_d(sm) / double(cpg);
  double m2 = 0.0;
  for (int c = lane; c < cpg; c += 64) {
    const double d = double(rs[c].x) - m;
    m2 += double(rs[c].y) + double(S) * d * d;
  }
  m2 = wave_sum_d(m2);
  if (lane == 0) {
    mean[i] = float(m);
    rstd[i] = float(1.0 / sqrt(m2 / (double(cpg) * double(S)) + double(eps)));
  }
}

// Workgroup w: row w / nch, chunk w % nch of kGnT * VW * kGnVecIter values.
template <int DT, int VW>
__global__ __launch_bounds__(kGnT) void gn_apply_kernel(const typename Elem<DT>::T* __restrict__ y,
                                                        const typename Elem<DT>::T* __restrict__ v, int act,
                                                        const float* __restrict__ w, const float* __restrict__ bias,
                                                        const float* __restrict__ mean,
                                                        const float* __restrict__ rstd,
                                                        typename Elem<DT>::T* __restrict__ out, int C, int G,
                                                        int64_t S, int nch) {
#pragma clang fp contract(off)
  const int64_t r = blockIdx.x / nch;
  const int ch = int(blockIdx.x - r * nch);
  const int c = int(r % C);
  const int64_t bg = (r / C) * G + c / (C / G);
  const float a = rstd[bg] * (w ? w[c] : 1.f);
  const float h = (bias ? bias[c] : 0.f) - mean[bg] * a;
  const int64_t base = r * S;
#pragma unroll
  for (int it = 0; it < kGnVecIter; ++it) {
    const int64_t i = (int64_t(ch) * kGnVecIter + it) * (kGnT * VW) + int64_t(threadIdx.x) * VW;
    if (i >= S) break;
    float u[VW], yv[VW], vv[VW], o[VW];
    gn_u<DT, VW>(y, v, act, base + i, u, yv, vv);
#pragma unroll
    for (int k = 0; k < VW; ++k) o[k] = u[k] * a + h;
    gn_store<DT, VW>(out, base + i, o);
  }
}

template <int DT, int VW>
__global__ __launch_bounds__(kGnT) void gn_row_bwd_kernel(const typename Elem<DT>::T* __restrict__ dout,
                                                          const typename Elem<DT>::T* __restrict__ y,
                                                          const typename Elem<DT>::T* __restrict__ v, int act,
                                                          const float* __restrict__ mean,
                                                          const float* __restrict__ rstd, int64_t rows, int C, int G,
                                                          int64_t S, float2* __restrict__ rowsum) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * kGnRowsPerWG + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int c = int(r % C);
  const int64_t bg = (r / C) * G + c / (C / G);
  const float mu = mean[bg], rs = rstd[bg];
  const int64_t base = r * S;
  float s1 = 0.f, s2 = 0.f;
#pragma unroll 4
  for (int64_t i = int64_t(lane) * VW; i < S; i += 64 * VW) {
    float u[VW], yv[VW], vv[VW], d[VW];
    gn_u<DT, VW>(y, v, act, base + i, u, yv, vv);
    gn_load<DT, VW>(dout, base + i, d);
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      s1 = fmaf(d[k], (u[k] - mu) * rs, s1);
      s2 += d[k];
    }
  }
  s1 = wave_sum(s1);
  s2 = wave_sum(s2);
  if (lane == 0) rowsum[r] = make_float2(s1, s2);
}

// Workgroups [0, nwg_coef): one wave per (b, g), the group coefficients
// coef[bg] = (mean(g xhat), mean(g)) summed over the group's channels in a
// fixed order; the workgroups after them: a thread per channel, dw[c] and
// dbias[c] summed over b in order.
__global__ __launch_bounds__(kGnT) void gn_finalize_bwd_kernel(const float2* __restrict__ rowsum,
                                                               const float* __restrict__ w, int64_t B, int C, int G,
                                                               int64_t S, int nwg_coef, float2* __restrict__ coef,
                                                               float* __restrict__ dw, float* __restrict__ db) {
  const int64_t BG = B * G;
  const int cpg = C / G;
  if (int(blockIdx.x) < nwg_coef) {
    const int lane = threadIdx.x & 63;
    const int64_t i = int64_t(blockIdx.x) * kGnRowsPerWG + (threadIdx.x >> 6);
    if (i >= BG) return;
    const int64_t b = i / G, g = i - b * G;
    double a1 = 0.0, a2 = 0.0;
    for (int k = lane; k < cpg; k += 64) {
      const int c = int(g) * cpg + k;
      const float2 s = rowsum[b * C + c];
      const double wc = w ? double(w[c]) : 1.0;
      a1 += wc * double(s.x);
      a2 += wc * double(s.y);
    }
    a1 = wave_sum_d(a1);
    a2 = wave_sum_d(a2);
    const double n = double(cpg) * double(S);
    if (lane == 0) coef[i] = make_float2(float(a1 / n), float(a2 / n));
  } else {
    const int64_t c = int64_t(int(blockIdx.x) - nwg_coef) * kGnT + threadIdx.x;
    if (c >= C) return;
    float s1 = 0.f, s2 = 0.f;
    for (int64_t b = 0; b < B; ++b) {
      const float2 s = rowsum[b * C + c];
      s1 += s.x;
      s2 += s.y;
    }
    if (dw) dw[c] = s1;
    if (db) db[c] = s2;
  }
}

template <int DT, int VW>
__global__ __launch_bounds__(kGnT) void gn_apply_bwd_kernel(const typename Elem<DT>::T* __restrict__ dout,
                                                            const typename Elem<DT>::T* __restrict__ y,
                                                            const typename Elem<DT>::T* __restrict__ v, int act,
                                                            const float* __restrict__ w,
                                                            const float* __restrict__ mean,
                                                            const float* __restrict__ rstd,
                                                            const float2* __restrict__ coef,
                                                            typename Elem<DT>::T* __restrict__ dy,
                                                            typename Elem<DT>::T* __restrict__ dv, int C, int G,
                                                            int64_t S, int nch) {
#pragma clang fp contract(off)
  const int64_t r = blockIdx.x / nch;
  const int ch = int(blockIdx.x - r * nch);
  const int c = int(r % C);
  const int64_t bg = (r / C) * G + c / (C / G);
  const float mu = mean[bg], rs = rstd[bg], wc = w ? w[c] : 1.f;
  const float2 cf = coef[bg];
  const int64_t base = r * S;
#pragma unroll
  for (int it = 0; it < kGnVecIter; ++it) {
    const int64_t i = (int64_t(ch) * kGnVecIter + it) * (kGnT * VW) + int64_t(threadIdx.x) * VW;
    if (i >= S) break;
    float u[VW], yv[VW], vv[VW], d[VW], o0[VW], o1[VW];
    gn_u<DT, VW>(y, v, act, base + i, u, yv, vv);
    gn_load<DT, VW>(dout, base + i, d);
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      const float xh = (u[k] - mu) * rs;
      const float du = Elem<DT>::round(rs * ((wc * d[k] - cf.y) - xh * cf.x));
      if (v) {
        o0[k] = du * Elem<DT>::round(gate_act(act, vv[k]));
        o1[k] = Elem<DT>::round(du * yv[k]) * gate_dact(act, vv[k]);
      } else {
        o0[k] = du;
        o1[k] = 0.f;
      }
    }
    gn_store<DT, VW>(dy, base + i, o0);
    if (v) gn_store<DT, VW>(dv, base + i, o1);
  }
}

bool gn_vec_ok(int vw, int64_t S, std::initializer_list<const void*> ptrs) {
  if (S % vw) return false;
  for (const void* q : ptrs)
    if (q && (reinterpret_cast<uintptr_t>(q) & 15)) return false;
  return true;
}

template <int DT>
int gn_fwd(const void* y, const void* v, const float* w, const float* bias, void* out, float* mean, float* rstd,
           int64_t B, int C, int64_t S, int G, float eps, int act, float2* rowst, hipStream_t st) {
  using T = typename Elem<DT>::T;
  constexpr int VW = 16 / int(sizeof(T));
  const int64_t rows = B * C;
  const bool vec = gn_vec_ok(VW, S, {y, v, out});
  const dim3 rg(unsigned(ceil_div(rows, kGnRowsPerWG)));
  if (vec)
    hipLaunchKernelGGL((gn_row_stats_kernel<DT, VW>), rg, dim3(kGnT), 0, st, (const T*)y, (const T*)v, act, rows, S,
                       rowst);
  else
    hipLaunchKernelGGL((gn_row_stats_kernel<DT, 1>), rg, dim3(kGnT), 0, st, (const T*)y, (const T*)v, act, rows, S,
                       rowst);
  hipLaunchKernelGGL(gn_finalize_kernel, dim3(unsigned(ceil_div(B * G, kGnRowsPerWG))), dim3(kGnT), 0, st,
                     (const float2*)rowst, B * G, C, G, S, eps, mean, rstd);
  const int vw = vec ? VW : 1;
  const int nch = int(ceil_div(S, int64_t(kGnT) * vw * kGnVecIter));
  const dim3 ag(unsigned(rows * nch));
  if (vec)
    hipLaunchKernelGGL((gn_apply_kernel<DT, VW>), ag, dim3(kGnT), 0, st, (const T*)y, (const T*)v, act, w, bias,
                       (const float*)mean, (const float*)rstd, (T*)out, C, G, S, nch);
  else
    hipLaunchKernelGGL((gn_apply_kernel<DT, 1>), ag, dim3(kGnT), 0, st, (const T*)y, (const T*)v, act, w, bias,
                       (const float*)mean, (const float*)rstd, (T*)out, C, G, S, nch);
  return NSQ_OK;
}

template <int DT>
int gn_bwd(const void* dout, const void* y, const void* v, const float* w, const float* mean, const float* rstd,
           void* dy, void* dv, float* dw, float* db, int64_t B, int C, int64_t S, int G, int act, float2* rowsum,
           float2* coef, hipStream_t st) {
  using T = typename Elem<DT>::T;
  constexpr int VW = 16 / int(sizeof(T));
  const int64_t rows = B * C;
  const bool vec = gn_vec_ok(VW, S, {dout, y, v, dy, dv});
  const dim3 rg(unsigned(ceil_div(rows, kGnRowsPerWG)));
  if (vec)
    hipLaunchKernelGGL((gn_row_bwd_kernel<DT, VW>), rg, dim3(kGnT), 0, st, (const T*)dout, (const T*)y, (const T*)v,
                       act, mean, rstd, rows, C, G, S, rowsum);
  else
    hipLaunchKernelGGL((gn_row_bwd_kernel<DT, 1>), rg, dim3(kGnT), 0, st, (const T*)dout, (const T*)y, (const T*)v,
                       act, mean, rstd, rows, C, G, S, rowsum);
  const int nwg_coef = int(ceil_div(B * G, kGnRowsPerWG));
  hipLaunchKernelGGL(gn_finalize_bwd_kernel, dim3(unsigned(nwg_coef + ceil_div(int64_t(C), kGnT))), dim3(kGnT), 0, st,
                     (const float2*)rowsum, w, B, C, G, S, nwg_coef, coef, dw, db);
  const int vw = vec ? VW : 1;
  const int nch = int(ceil_div(S, int64_t(kGnT) * vw * kGnVecIter));
  const dim3 ag(unsigned(rows * nch));
  if (vec)
    hipLaunchKernelGGL((gn_apply_bwd_kernel<DT, VW>), ag, dim3(kGnT), 0, st, (const T*)dout, (const T*)y,
                       (const T*)v, act, w, mean, rstd, (const float2*)coef, (T*)dy, (T*)dv, C, G, S, nch);
  else
    hipLaunchKernelGGL((gn_apply_bwd_kernel<DT, 1>), ag, dim3(kGnT), 0, st, (const T*)dout, (const T*)y,
                       (const T*)v, act, w, mean, rstd, (const float2*)coef, (T*)dy, (T*)dv, C, G, S, nch);
  return NSQ_OK;
}

int gn_check(const char* who, int dtype, int64_t B, int64_t C, int64_t S, int64_t G, float eps, int act) {
  NSQ_CHECK_ARG(dtype == NSQ_DTYPE_F32 || dtype == NSQ_DTYPE_BF16 || dtype == NSQ_DTYPE_F16, "%s: bad dtype %d", who,
                dtype);
  NSQ_CHECK_ARG(B >= 1 && C >= 1 && S >= 1 && G >= 1, "%s: sizes must be positive (B=%lld C=%lld S=%lld G=%lld)", who,
                (long long)B, (long long)C, (long long)S, (long long)G);
  NSQ_CHECK_ARG(C % G == 0, "%s: num_channels %lld must be divisible by num_groups %lld", who, (long long)C,
                (long long)G);
  NSQ_CHECK_ARG(C <= 0x7fffffff && B * C <= 0x7fffffff, "%s: B*C=%lld too large", who, (long long)(B * C));
  NSQ_CHECK_ARG(eps >= 0.f, "%s: eps must be >= 0", who);
  NSQ_CHECK_ARG(act == NSQ_GATE_IDENTITY || act == NSQ_GATE_SIGMOID || act == NSQ_GATE_SILU, "%s: bad act %d", who,
                act);
  // apply grids: rows * chunks workgroups
  const int64_t nch = ceil_div(S, int64_t(kGnT) * kGnVecIter);
  NSQ_CHECK_ARG(B * C * nch <= 0x7fffffff, "%s: B*C*S too large for the grid", who);
  return NSQ_OK;
}

}  // namespace
}  // namespace nsq

using namespace nsq;

extern "C" size_t nsq_channel_groupnorm_workspace_bytes(int64_t B, int64_t C, int64_t G, int direction) {
  if (B < 1 || C < 1 || G < 1 || C % G) return 0;
  const size_t rows = size_t(B) * size_t(C) * sizeof(float2);
  return direction == NSQ_DIR_BWD ? rows + size_t(B) * size_t(G) * sizeof(float2) : rows;
}

extern "C" int nsq_channel_groupnorm_fwd(const void* y, const void* v, const float* w, const float* b, void* out,
                                         float* mean, float* rstd, int dtype, int64_t B, int64_t C, int64_t S,
                                         int64_t G, float eps, int act, void* workspace, size_t workspace_bytes,
                                         void* stream) {
  clear_error();
  NSQ_CHECK_ARG(y && out && mean && rstd, "channel_groupnorm_fwd: null pointer argument");
  if (int e = gn_check("channel_groupnorm_fwd", dtype, B, C, S, G, eps, act)) return e;
  const size_t need = nsq_channel_groupnorm_workspace_bytes(B, C, G, NSQ_DIR_FWD);
  NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "channel_groupnorm_fwd: workspace of %zu bytes needed", need);
  hipStream_t st = (hipStream_t)stream;
  float2* rowst = (float2*)workspace;
  if (dtype == NSQ_DTYPE_F32)
    gn_fwd<NSQ_DTYPE_F32>(y, v, w, b, out, mean, rstd, B, int(C), S, int(G), eps, act, rowst, st);
  else if (dtype == NSQ_DTYPE_BF16)
    gn_fwd<NSQ_DTYPE_BF16>(y, v, w, b, out, mean, rstd, B, int(C), S, int(G), eps, act, rowst, st);
  else
    gn_fwd<NSQ_DTYPE_F16>(y, v, w, b, out, mean, rstd, B, int(C), S, int(G), eps, act, rowst, st);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

extern "C" int nsq_channel_groupnorm_bwd(const void* dout, const void* y, const void* v, const float* w,
                                         const float* mean, const float* rstd, void* dy, void* dv, float* dw,
                                         float* db, int dtype, int64_t B, int64_t C, int64_t S, int64_t G, int act,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  NSQ_CHECK_ARG(dout && y && mean && rstd && dy, "channel_groupnorm_bwd: null pointer argument");
  NSQ_CHECK_ARG((v == nullptr) == (dv == nullptr), "channel_groupnorm_bwd: v and dv must be given together");
  NSQ_CHECK_ARG(w || !dw, "channel_groupnorm_bwd: dw needs the weight w");
  if (int e = gn_check("channel_groupnorm_bwd", dtype, B, C, S, G, 0.f, act)) return e;
  const size_t need = nsq_channel_groupnorm_workspace_bytes(B, C, G, NSQ_DIR_BWD);
  NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "channel_groupnorm_bwd: workspace of %zu bytes needed", need);
  hipStream_t st = (hipStream_t)stream;
  float2* rowsum = (float2*)workspace;
  float2* coef = rowsum + B * C;
  if (dtype == NSQ_DTYPE_F32)
    gn_bwd<NSQ_DTYPE_F32>(dout, y, v, w, mean, rstd, dy, dv, dw, db, B, int(C), S, int(G), act, rowsum, coef, st);
  else if (dtype == NSQ_DTYPE_BF16)
    gn_bwd<NSQ_DTYPE_BF16>(dout, y, v, w, mean, rstd, dy, dv, dw, db, B, int(C), S, int(G), act, rowsum, coef, st);
  else
    gn_bwd<NSQ_DTYPE_F16>(dout, y, v, w, mean, rstd, dy, dv, dw, db, B, int(C), S, int(G), act, rowsum, coef, st);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}
