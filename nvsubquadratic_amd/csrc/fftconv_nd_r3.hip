// Host passes of the mixed-radix 2D / 3D plan (kernels in fftconv_nd_r3.h): the
// same pass sequence, workspace layout and results as run_nd_fwd /
// run_nd_bwd in fftconv_nd_plan.h, at FFT lengths 3 * 2^m.
#include "fftconv2d_image192.h"
#include "fftconv_nd_plan.h"
#include "fftconv_nd_r3.h"

namespace nsq {

template <int V>
using IC = std::integral_constant<int, V>;

// (N2 = F2 / 2, F1) of the plane kernels.
template <class F>
static bool with_r3_plane(const NdPlan& p, F&& f) {
  const int n2 = p.F[2] / 2, f1 = p.F[1];
  if (n2 == 24 && f1 == 48) f(IC<24>{}, IC<48>{});
  else if (n2 == 24 && f1 == 96) f(IC<24>{}, IC<96>{});
  else if (n2 == 48 && f1 == 48) f(IC<48>{}, IC<48>{});
  else if (n2 == 48 && f1 == 96) f(IC<48>{}, IC<96>{});
  else return false;
  return true;
}

// N2 = F2 / 2 of the 2D row kernels.
template <class F>
static bool with_r3_row(const NdPlan& p, F&& f) {
  switch (p.F[2] / 2) {
    case 24: f(IC<24>{}); return true;
    case 48: f(IC<48>{}); return true;
    case 96: f(IC<96>{}); return true;
    default: return false;
  }
}

template <class F>
static bool with_r3_col(const NdPlan& p, F&& f) {
  switch (p.F[0]) {
    case 48: f(IC<48>{}); return true;
    case 96: f(IC<96>{}); return true;
    case 192: f(IC<192>{}); return true;
    default: return false;
  }
}

// NSQ_R3_PLANE_WAVE=0: the plane passes with workgroup-wide transforms.
static bool r3_plane_wave() {
  static const bool on = [] {
    const char* e = std::getenv("NSQ_R3_PLANE_WAVE");
    return !(e && e[0] == '0');
  }();
  return on;
}

// Forward inner-axis passes of nbh blocks of [n0][n1][len] real values: the
// plane kernels (3D), or the row kernels (2D, n1 = 1).
template <int DT>
static bool r3_inner_fwd(const NdPlan& p, const void* src, int64_t nbh, int n0, int n1, int len, float2* ws,
                         const float2* tw, hipStream_t st) {
  using ET = typename Elem<DT>::T;
  const bool al = pairs_aligned<DT>(src, len, len);
  if (p.nd == 2) {
    const bool third = 3 * len <= 2 * p.F[2];
    const int rows = int(nbh * n0);
    return with_r3_row(p, [&](auto NC) {
      constexpr int N2 = decltype(NC)::value;
      const dim3 grid(unsigned(ceil_div(rows, R3RowCfg<N2>::M)));
      auto go = [&](auto a, auto th) {
        hipLaunchKernelGGL((r3_row_fwd_kernel<N2, DT, decltype(a)::value, decltype(th)::value>), grid,
                           dim3(R3RowCfg<N2>::T), 0, st, (const ET*)src, rows, n0, len, ws, p.spec, tw);
      };
      using T_ = std::true_type;
      using F_ = std::false_type;
      if (al)
        third ? go(T_{}, T_{}) : go(T_{}, F_{});
      else
        third ? go(F_{}, T_{}) : go(F_{}, F_{});
    });
  }
  const bool third = 3 * len <= 2 * p.F[2] && 3 * n1 <= 2 * p.F[1];
  return with_r3_plane(p, [&](auto NC, auto FC) {
    constexpr int N2 = decltype(NC)::value, F1 = decltype(FC)::value;
    const dim3 grid(unsigned(nbh * n0));
    auto go = [&](auto a, auto th) {
      if (r3_plane_wave())
        hipLaunchKernelGGL((r3_plane_fwd_w_kernel<N2, F1, DT, decltype(a)::value, decltype(th)::value>), grid,
                           dim3(256), 0, st, (const ET*)src, n0, n1, len, ws, p.spec, tw);
      else
        hipLaunchKernelGGL((r3_plane_fwd_kernel<N2, F1, DT, decltype(a)::value, decltype(th)::value>), grid,
                           dim3(R3PlaneCfg<N2, F1>::T), 0, st, (const ET*)src, n0, n1, len, ws, p.spec, tw);
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    if (al)
      third ? go(T_{}, T_{}) : go(T_{}, F_{});
    else
      third ? go(F_{}, T_{}) : go(F_{}, F_{});
  });
}

// Inverse plane passes of nbh blocks whose axis-0 extent is n0: rows [off1,
// off1 + n1out) of axis 1, the epilogue and last-axis window of `o`.
template <int DT, int MODE>
static bool r3_inner_inv(const NdPlan& p, const float2* ws, int64_t nbh, int n0, int off1, int n1out, RowInvOut o,
                         const float2* tw, hipStream_t st) {
  const bool has_s = MODE == ND_OUT_Y && o.s;
  if (p.nd == 2) {
    const int rows = int(nbh * n0);
    return with_r3_row(p, [&](auto NC) {
      constexpr int N2 = decltype(NC)::value;
      const dim3 grid(unsigned(ceil_div(rows, R3RowCfg<N2>::M)));
      auto go = [&](auto hs) {
        hipLaunchKernelGGL((r3_row_inv_kernel<N2, DT, MODE, decltype(hs)::value>), grid, dim3(R3RowCfg<N2>::T), 0,
                           st, ws, rows, n0, p.spec, o, tw);
      };
      has_s ? go(std::true_type{}) : go(std::false_type{});
    });
  }
  return with_r3_plane(p, [&](auto NC, auto FC) {
    constexpr int N2 = decltype(NC)::value, F1 = decltype(FC)::value;
    const dim3 grid(unsigned(nbh * n0));
    auto go = [&](auto hs) {
      if (r3_plane_wave())
        hipLaunchKernelGGL((r3_plane_inv_w_kernel<N2, F1, DT, MODE, decltype(hs)::value>), grid, dim3(256), 0, st,
                           ws, p.spec, n0, off1, n1out, o, tw);
      else
        hipLaunchKernelGGL((r3_plane_inv_kernel<N2, F1, DT, MODE, decltype(hs)::value>), grid,
                           dim3(R3PlaneCfg<N2, F1>::T), 0, st, ws, p.spec, n0, off1, n1out, o, tw);
    };
    has_s ? go(std::true_type{}) : go(std::false_type{});
  });
}

// Filter spectrum: kb*H blocks of the [kb*H][K0][K1][K2] float32 kernel.
static bool r3_filter_spectrum(const NdPlan& p, const float* k, float2* wsk, const float2* tw, hipStream_t st) {
  const int64_t nk = p.kb * p.H;
  if (!r3_inner_fwd<NSQ_DTYPE_F32>(p, k, nk, p.K[0], p.K[1], p.K[2], wsk, tw, st)) return false;
  const ColGeom cg = axis0_geom(p);
  const bool third = 3 * p.K[0] <= 2 * p.F[0];
  return with_r3_col(p, [&](auto FC) {
    constexpr int F0 = decltype(FC)::value;
    const dim3 grid(unsigned(nk), unsigned(ceil_div(cg.inner_count, R3ColCfg<F0>::M)));
    if (third)
      hipLaunchKernelGGL((r3_col_fwd_kernel<F0, true>), grid, dim3(R3ColCfg<F0>::T), 0, st, wsk, cg, p.K[0], tw);
    else
      hipLaunchKernelGGL((r3_col_fwd_kernel<F0, false>), grid, dim3(R3ColCfg<F0>::T), 0, st, wsk, cg, p.K[0], tw);
  });
}

template <int DT>
bool run_r3_fwd(const NdPlan& p, const void* x, const float* k, const void* s, void* y, float2* ws, bool save,
                const float2* tw, hipStream_t st) {
  const int64_t BH = p.B * p.H;
  float2* wsx = save ? ws + BH * p.spec : ws;
  float2* wsk = wsx + BH * p.spec;
  float2* wsy = save ? ws : wsx;
  if (!r3_filter_spectrum(p, k, wsk, tw, st)) return false;
  if (!r3_inner_fwd<DT>(p, x, BH, p.S[0], p.S[1], p.S[2], wsx, tw, st)) return false;
  const ColGeom cg = axis0_geom(p);
  const int bsplit = mul_batch_split(p);
  const bool third = 3 * p.S[0] <= 2 * p.F[0];
  const bool ok = with_r3_col(p, [&](auto FC) {
    constexpr int F0 = decltype(FC)::value;
    const dim3 grid(unsigned((p.kb != 1 ? BH : p.H) * bsplit), unsigned(ceil_div(cg.inner_count, R3ColCfg<F0>::M)));
    auto go = [&](auto th) {
      hipLaunchKernelGGL((r3_col_mul_kernel<F0, decltype(th)::value>), grid, dim3(R3ColCfg<F0>::T), 0, st,
                         (const float2*)wsx, wsy, (const float2*)wsk, cg, int(p.B), int(p.H), int(p.kb != 1), p.S[0],
                         p.o[0], bsplit, tw);
    };
    third ? go(std::true_type{}) : go(std::false_type{});
  });
  if (!ok) return false;
  RowInvOut o{y, x, s, nullptr, int(p.H), p.o[2], p.S[2], 0, 0, 0,
              1.f / (float(p.F[0]) * float(p.F[1]) * float(p.F[2] / 2))};
  return r3_inner_inv<DT, ND_OUT_Y>(p, wsy, BH, p.S[0], p.o[1], p.S[1], o, tw, st);
}

template <int DT>
bool run_r3_bwd(const NdPlan& p, const void* g, const void* x, const float* k, const void* s, void* gx, float* gk,
                float* gs, float2* ws, bool fwd_state, const float2* tw, hipStream_t st) {
  const int64_t BH = p.B * p.H, NK = p.kb * p.H;
  float2* wsg = ws;
  float2* wsx = wsg + BH * p.spec;
  float2* wsk = wsx + BH * p.spec;
  float2* wsq = wsk + NK * p.spec;
  if (!fwd_state) {
    if (!r3_filter_spectrum(p, k, wsk, tw, st)) return false;
    if (!r3_inner_fwd<DT>(p, x, BH, p.S[0], p.S[1], p.S[2], wsx, tw, st)) return false;
  }
  if (!r3_inner_fwd<DT>(p, g, BH, p.S[0], p.S[1], p.S[2], wsg, tw, st)) return false;
  const ColGeom cg = axis0_geom(p);
  const R3Ramp rp{p.c[0], p.c[1], p.c[2], p.F[1], p.F[2], p.FH};
  const int nz = bwd_batch_split(p);  // partial Q blocks follow Q in the workspace
  const bool third = 3 * p.S[0] <= 2 * p.F[0];
  const bool ok = with_r3_col(p, [&](auto FC) {
    constexpr int F0 = decltype(FC)::value;
    const dim3 grid(unsigned(NK), unsigned(ceil_div(cg.inner_count, R3ColCfg<F0>::M)), unsigned(nz));
    auto go = [&](auto th) {
      hipLaunchKernelGGL((r3_col_bwd_kernel<F0, decltype(th)::value>), grid, dim3(R3ColCfg<F0>::T), 0, st, wsg,
                         (const float2*)wsx, (const float2*)wsk, wsq, cg, int(p.B), int(p.H), int(p.kb != 1), p.S[0],
                         p.K[0], rp, NK, tw);
    };
    third ? go(std::true_type{}) : go(std::false_type{});
  });
  if (!ok) return false;
  if (nz > 1) {
    const int64_t count = int64_t(p.K[0]) * p.F[1] * p.RS;  // rows [0, K0) of a block
    const int64_t blocks = (NK * count + 255) / 256;
    hipLaunchKernelGGL(nd_q_reduce_kernel, dim3(unsigned(blocks < 8192 ? blocks : 8192)), dim3(256), 0, st, wsq, NK,
                       p.spec, count, nz);
  }
  const float scale = 1.f / (float(p.F[0]) * float(p.F[1]) * float(p.F[2] / 2));
  RowInvOut og{gx, g, s, nullptr, int(p.H), 0, p.S[2], 0, 0, 0, scale};
  if (!r3_inner_inv<DT, ND_OUT_Y>(p, wsg, BH, p.S[0], 0, p.S[1], og, tw, st)) return false;
  RowInvOut ok_{gk, nullptr, nullptr, gs, int(p.H), 0, p.K[2], p.c[0], p.c[1], p.c[2], scale * p.gk_scale};
  return r3_inner_inv<NSQ_DTYPE_F32, ND_OUT_GK>(p, wsq, NK, p.K[0], 0, p.K[1], ok_, tw, st);
}

// The one-kernel image forward on the 192 x 192 plane (fftconv2d_image192.h)
// for a 2D forward that keeps no state: the filter spectrum's rows at the
// workspace's Khat position, its columns transposed into the X region the
// kernel does not use (H * 97 * 192 <= B * H * spec).
inline bool r3_image_ok(const NdPlan& p, const void* x, const void* y) {
  return p.r3 && p.nd == 2 && p.kb == 1 && !p.ramp && p.wm[0] == -1 && p.wm[2] == -1 && p.F[0] == kI3F &&
         p.F[2] == kI3F && p.FH == kI3Bins && p.S[0] <= kI3Rows && p.S[2] <= kI3Rows &&
         p.S[2] % 8 == 0 && p.o[2] % 2 == 0 && p.o[0] + p.S[0] <= kI3F && p.o[2] + p.S[2] <= kI3F &&
         p.spec >= int64_t(kI3Bins) * kI3F && p.B * p.H <= int64_t(1) << 30 &&
         (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
}

inline int image192_threads() {
  static const int t = [] {
    const char* e = std::getenv("NSQ_2D_IMAGE192_T");
    return (e && std::atoi(e) == 512) ? 512 : 1024;
  }();
  return t;
}

template <int DT>
bool run_r3_image_fwd(const NdPlan& p, const void* x, const float* k, const void* s, void* y, float2* ws,
                      const float2* tw, hipStream_t st) {
  if (!r3_image_ok(p, x, y)) return false;
  using ET = typename Elem<DT>::T;
  const int64_t BH = p.B * p.H;
  float2* wsk = ws + BH * p.spec;
  float2* kt = ws;
  // the filter spectrum's row passes into the Khat region, its column pass
  // written transposed into the X region
  if (!r3_inner_fwd<NSQ_DTYPE_F32>(p, k, p.H, p.K[0], p.K[1], p.K[2], wsk, tw, st)) return false;
  const ColGeom cg = axis0_geom(p);
  const dim3 kgrid{unsigned(p.H), unsigned(ceil_div(cg.inner_count, R3ColCfg<kI3F>::M))};
  if (3 * p.K[0] <= 2 * kI3F)
    hipLaunchKernelGGL((r3_col_fwd_t_kernel<kI3F, true>), kgrid, dim3(R3ColCfg<kI3F>::T), 0, st, (const float2*)wsk,
                       cg, p.K[0], kt, tw);
  else
    hipLaunchKernelGGL((r3_col_fwd_t_kernel<kI3F, false>), kgrid, dim3(R3ColCfg<kI3F>::T), 0, st, (const float2*)wsk,
                       cg, p.K[0], kt, tw);
  const float scale = 1.f / (float(kI3F) * float(kI3N2));
  const dim3 grid{unsigned(BH)};
  auto go = [&](auto hs, auto tc) {
    constexpr int T = decltype(tc)::value;
    hipLaunchKernelGGL((nd2_image192_fwd_kernel<DT, decltype(hs)::value, T>), grid, dim3(T), 0, st, (const ET*)x,
                       (const float2*)kt, (const ET*)s, (ET*)y, int(p.B), int(p.H), int(p.S[0]), int(p.S[2]),
                       int(p.o[0]), int(p.o[2]), scale, tw);
  };
  const bool t512 = image192_threads() == 512;
  if (s)
    t512 ? go(std::true_type{}, IC<512>{}) : go(std::true_type{}, IC<1024>{});
  else
    t512 ? go(std::false_type{}, IC<512>{}) : go(std::false_type{}, IC<1024>{});
  return true;
}

NSQ_R3_RUN_INSTANCES(, NSQ_DTYPE_F32)
NSQ_R3_RUN_INSTANCES(, NSQ_DTYPE_BF16)
NSQ_R3_RUN_INSTANCES(, NSQ_DTYPE_F16)

}  // namespace nsq
