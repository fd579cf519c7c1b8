// Team plan of the causal 1D FFT convolution (see fftconv1d_team.h): the
// cooperative forward / backward kernels and their launchers.
#include "fftconv1d_team.h"

namespace nsq {

template <int LOGN1, int LOGN2>
struct TeamGeom {
  static constexpr int LOGN = LOGN1 + LOGN2;
  static constexpr int64_t N = int64_t(1) << LOGN;
  static constexpr int N1 = 1 << LOGN1, N2 = 1 << LOGN2;
  static constexpr int CM = ColCfg<LOGN1>::M;                 // columns per column tile
  static constexpr int NCB = N2 / CM;                          // column tiles per signal
  static constexpr int NRT = (N1 / 2) / TeamRowCfg<LOGN2>::NP;  // row-pair tiles per signal
  static constexpr int COL_LDS = ColCfg<LOGN1>::M * ColCfg<LOGN1>::S;
  static constexpr int ROW_LDS = TeamRowCfg<LOGN2>::M * TeamRowCfg<LOGN2>::N2P;
  static constexpr int LDS = COL_LDS > ROW_LDS ? COL_LDS : ROW_LDS;
};

// Exchange region b (0/1) of team t: NSIG signals of N complex values.
__device__ __forceinline__ float2* team_region(void* ws, int t, int b, int nsig, int64_t N) {
  return reinterpret_cast<float2*>(static_cast<char*>(ws) + kTeamCtlBytes) + (int64_t(t) * 2 + b) * nsig * N;
}

struct TeamFwdArgs {
  const void* x;
  const float* k;
  const void* s;
  void* y;
  int H, L, K;
  const float2* tw;
  void* ws;
  int max_spin;
};

struct TeamBwdArgs {
  const void* g;
  const void* x;
  const float* k;
  const void* s;
  void* gx;
  float* gk;
  float* gs;
  int H, L, K;
  const float2* tw;
  void* ws;
  int max_spin;
};

// Column-forward tile of a real row.  A row of at most N real samples (N =
// F/2) leaves packed samples [N/2, N) zero, and the first pass folds that
// half away (HalfZeroLoad); config 3 (L = K = N) is such a case, a long x with
// a short filter is not.
template <int LOGN1, int LOGN, int DT>
__device__ __forceinline__ void team_col_fwd_any(const typename Elem<DT>::T* row, int valid, bool al, int c0,
                                                 float2* out, const float2* tw, float2* lds) {
  const bool half = int64_t(valid) <= (int64_t(1) << LOGN);
  if (al)
    half ? team_col_fwd<LOGN1, LOGN, DT, true, true>(row, valid, c0, out, tw, lds)
         : team_col_fwd<LOGN1, LOGN, DT, true, false>(row, valid, c0, out, tw, lds);
  else
    half ? team_col_fwd<LOGN1, LOGN, DT, false, true>(row, valid, c0, out, tw, lds)
         : team_col_fwd<LOGN1, LOGN, DT, false, false>(row, valid, c0, out, tw, lds);
}

// Forward: per channel h, A (x, k columns -> X', K'), B (rows, product,
// inverse rows -> Y' over X'), C (inverse columns of Y' -> y).
template <int DT, int LOGN1, int LOGN2>
__global__ __launch_bounds__(kTeamThreads) __attribute__((amdgpu_waves_per_eu(2 * kTeamSub))) void team_fwd_kernel(
    TeamFwdArgs a) {
  using G = TeamGeom<LOGN1, LOGN2>;
  using ET = typename Elem<DT>::T;
  __shared__ float2 lds[G::LDS];
  TeamCtl* ctl = static_cast<TeamCtl*>(a.ws);
  Team tm;
  if (!team_join(ctl, tm, a.max_spin)) return;
  int* cA = &ctl->bar[tm.t][0];
  int* cB = &ctl->bar[tm.t][16];
  int* cC = &ctl->bar[tm.t][32];
  const int S = (a.H - tm.t + tm.n - 1) / tm.n;  // channels of this team
  const ET* x = static_cast<const ET*>(a.x);
  const bool alx = (a.L % 2 == 0) && ((reinterpret_cast<uintptr_t>(x) & (2 * sizeof(ET) - 1)) == 0);
  const bool aly = (a.L % 2 == 0) && ((reinterpret_cast<uintptr_t>(a.y) & (2 * sizeof(ET) - 1)) == 0);
  const bool alk = (a.K % 2 == 0) && ((reinterpret_cast<uintptr_t>(a.k) & 7) == 0);
  const ET* sh = static_cast<const ET*>(a.s);
  const float scale = 1.f / float(G::N);
  for (int s = 0; s <= S; ++s) {
    if (s < S) {  // A(s): needs C(s-2) done (its region)
      if (s >= 2 && !team_wait(cC, (s - 1) * tm.P, ctl, a.max_spin)) return;
      const int h = tm.t + s * tm.n;
      float2* reg = team_region(a.ws, tm.t, s & 1, 2, G::N);
      for (int tile = tm.rank; tile < 2 * G::NCB; tile += tm.P) {
        if (tile < G::NCB)
          team_col_fwd_any<LOGN1, G::LOGN, DT>(x + int64_t(h) * a.L, a.L, alx, tile * G::CM, reg, a.tw, lds);
        else
          team_col_fwd_any<LOGN1, G::LOGN, NSQ_DTYPE_F32>(a.k + int64_t(h) * a.K, a.K, alk, (tile - G::NCB) * G::CM,
                                                           reg + G::N, a.tw, lds);
      }
      team_arrive(cA);
    }
    if (s >= 1) {  // C(s-1): needs B(s-1) done
      if (!team_wait(cB, s * tm.P, ctl, a.max_spin)) return;
      const int h = tm.t + (s - 1) * tm.n;
      const float2* reg = team_region(a.ws, tm.t, (s - 1) & 1, 2, G::N);
      const bool has_s = sh != nullptr;
      const float sv = has_s ? Elem<DT>::round(Elem<DT>::load(sh, h)) : 0.f;
      ET* yrow = static_cast<ET*>(a.y) + int64_t(h) * a.L;
      const ET* xrow = x + int64_t(h) * a.L;
      for (int tile = tm.rank; tile < G::NCB; tile += tm.P) {
        if (alx && aly) {
          const RowBuf<DT, true> orow(yrow, a.L), arow(xrow, has_s ? a.L : 0);
          auto epi = [&](int64_t m, float2 v) {
            const float2 av = arow.load_pair(2 * m);
            orow.store_pair(2 * m, make_float2(epilogue<DT>(v.x * scale, has_s, sv, av.x),
                                               epilogue<DT>(v.y * scale, has_s, sv, av.y)));
          };
          team_col_inv<LOGN1, G::LOGN>(reg, tile * G::CM, epi, a.tw, lds);
        } else {
          const RowBuf<DT, false> orow(yrow, a.L), arow(xrow, has_s ? a.L : 0);
          auto epi = [&](int64_t m, float2 v) {
            const float2 av = arow.load_pair(2 * m);
            orow.store_pair(2 * m, make_float2(epilogue<DT>(v.x * scale, has_s, sv, av.x),
                                               epilogue<DT>(v.y * scale, has_s, sv, av.y)));
          };
          team_col_inv<LOGN1, G::LOGN>(reg, tile * G::CM, epi, a.tw, lds);
        }
      }
      team_arrive(cC);
    }
    if (s < S) {  // B(s): needs A(s) done
      if (!team_wait(cA, (s + 1) * tm.P, ctl, a.max_spin)) return;
      float2* reg = team_region(a.ws, tm.t, s & 1, 2, G::N);
      for (int rt = tm.rank; rt < G::NRT; rt += tm.P)
        team_rows_fwd<LOGN1, LOGN2>(reg, reg + G::N, rt * TeamRowCfg<LOGN2>::NP, a.tw, lds);
      team_arrive(cB);
    }
  }
}

// Backward: per channel h, A (g, x, k columns -> G', X', K'), B (rows: gx
// pre-image over K', gk pre-image over X'), C (inverse columns -> gx, gk, gs).
template <int DT, int LOGN1, int LOGN2>
__global__ __launch_bounds__(kTeamThreads) __attribute__((amdgpu_waves_per_eu(2 * kTeamSub))) void team_bwd_kernel(
    TeamBwdArgs a) {
  using G = TeamGeom<LOGN1, LOGN2>;
  using ET = typename Elem<DT>::T;
  __shared__ float2 lds[G::LDS];
  TeamCtl* ctl = static_cast<TeamCtl*>(a.ws);
  Team tm;
  if (!team_join(ctl, tm, a.max_spin)) return;
  int* cA = &ctl->bar[tm.t][0];
  int* cB = &ctl->bar[tm.t][16];
  int* cC = &ctl->bar[tm.t][32];
  const int S = (a.H - tm.t + tm.n - 1) / tm.n;
  const ET* g = static_cast<const ET*>(a.g);
  const ET* x = static_cast<const ET*>(a.x);
  const bool alg = (a.L % 2 == 0) && ((reinterpret_cast<uintptr_t>(g) & (2 * sizeof(ET) - 1)) == 0);
  const bool alx = (a.L % 2 == 0) && ((reinterpret_cast<uintptr_t>(x) & (2 * sizeof(ET) - 1)) == 0);
  const bool algx = (a.L % 2 == 0) && ((reinterpret_cast<uintptr_t>(a.gx) & (2 * sizeof(ET) - 1)) == 0);
  const bool alk = (a.K % 2 == 0) && ((reinterpret_cast<uintptr_t>(a.k) & 7) == 0);
  const bool algk = (a.K % 2 == 0) && ((reinterpret_cast<uintptr_t>(a.gk) & 7) == 0);
  const ET* sh = static_cast<const ET*>(a.s);
  const float scale = 1.f / float(G::N);
  for (int s = 0; s <= S; ++s) {
    if (s < S) {
      if (s >= 2 && !team_wait(cC, (s - 1) * tm.P, ctl, a.max_spin)) return;
      const int h = tm.t + s * tm.n;
      float2* reg = team_region(a.ws, tm.t, s & 1, 3, G::N);  // G', X', K'
      for (int tile = tm.rank; tile < 3 * G::NCB; tile += tm.P) {
        const int sig = tile / G::NCB, c0 = (tile - sig * G::NCB) * G::CM;
        if (sig == 0)
          team_col_fwd_any<LOGN1, G::LOGN, DT>(g + int64_t(h) * a.L, a.L, alg, c0, reg, a.tw, lds);
        else if (sig == 1)
          team_col_fwd_any<LOGN1, G::LOGN, DT>(x + int64_t(h) * a.L, a.L, alx, c0, reg + G::N, a.tw, lds);
        else
          team_col_fwd_any<LOGN1, G::LOGN, NSQ_DTYPE_F32>(a.k + int64_t(h) * a.K, a.K, alk, c0, reg + 2 * G::N,
                                                           a.tw, lds);
      }
      team_arrive(cA);
    }
    if (s >= 1) {
      if (!team_wait(cB, s * tm.P, ctl, a.max_spin)) return;
      const int h = tm.t + (s - 1) * tm.n;
      const float2* reg = team_region(a.ws, tm.t, (s - 1) & 1, 3, G::N);
      const bool has_s = sh != nullptr;
      const float sv = has_s ? Elem<DT>::round(Elem<DT>::load(sh, h)) : 0.f;
      ET* gxrow = static_cast<ET*>(a.gx) + int64_t(h) * a.L;
      const ET* grow = g + int64_t(h) * a.L;
      float* gkrow = a.gk + int64_t(h) * a.K;
      for (int tile = tm.rank; tile < 2 * G::NCB; tile += tm.P) {
        if (tile < G::NCB) {  // gx = conv^T(g) + s g, from the K' region
          auto run = [&](auto al) {
            constexpr bool AL = decltype(al)::value;
            const RowBuf<DT, AL> orow(gxrow, a.L), arow(grow, has_s ? a.L : 0);
            auto epi = [&](int64_t m, float2 v) {
              const float2 av = arow.load_pair(2 * m);
              orow.store_pair(2 * m, make_float2(epilogue<DT>(v.x * scale, has_s, sv, av.x),
                                                 epilogue<DT>(v.y * scale, has_s, sv, av.y)));
            };
            team_col_inv<LOGN1, G::LOGN>(reg + 2 * G::N, tile * G::CM, epi, a.tw, lds);
          };
          (algx && alg) ? run(std::true_type{}) : run(std::false_type{});
        } else {  // gk = correlation of g and x at lags [0, K), gs = its lag 0, from the X' region
          bool has0 = false;
          float g0 = 0.f;
          auto run = [&](auto al) {
            constexpr bool AL = decltype(al)::value;
            const RowBuf<NSQ_DTYPE_F32, AL> krow(gkrow, a.K);
            auto epi = [&](int64_t m, float2 v) {
              krow.store_pair(2 * m, make_float2(v.x * scale, v.y * scale));
              has0 = has0 || (m == 0);
              g0 = (m == 0) ? v.x * scale : g0;
            };
            team_col_inv<LOGN1, G::LOGN>(reg + G::N, (tile - G::NCB) * G::CM, epi, a.tw, lds);
          };
          algk ? run(std::true_type{}) : run(std::false_type{});
          if (a.gs && has0) a.gs[h] = g0;
        }
      }
      team_arrive(cC);
    }
    if (s < S) {
      if (!team_wait(cA, (s + 1) * tm.P, ctl, a.max_spin)) return;
      float2* reg = team_region(a.ws, tm.t, s & 1, 3, G::N);
      for (int rt = tm.rank; rt < G::NRT; rt += tm.P)
        team_rows_bwd<LOGN1, LOGN2>(reg, reg + G::N, reg + 2 * G::N, rt * TeamRowCfg<LOGN2>::NP, a.tw, lds);
      team_arrive(cB);
    }
  }
}

__global__ void team_ctl_clear_kernel(int* ctl, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) ctl[i] = 0;
}

bool team_plan_ok(const Plan1D& p, int64_t B, int64_t kbatch) {
  return !p.fused && !p.fold && B == 1 && kbatch == 1 && p.logN == 18 && p.logN1 == 8;
}

size_t team_workspace_bytes(const Plan1D& p, int direction) {
  const int nsig = direction == NSQ_DIR_BWD ? 3 : 2;
  return kTeamCtlBytes + size_t(kTeamMaxTeams) * 2 * nsig * (size_t(1) << p.logN) * sizeof(float2);
}

// Grid: kTeamSub workgroups per CU (fewer if they do not fit), launched
// cooperatively so that all of them are resident together (the team barriers
// need every member running).
template <class KERNEL, class ARGS>
static int team_launch(KERNEL kernel, ARGS& args, void* ws, hipStream_t st) {
  int dev = 0, cus = 0, per_cu = 0;
  NSQ_CHECK_HIP(hipGetDevice(&dev));
  NSQ_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  NSQ_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kTeamThreads, 0));
  if (per_cu < 1 || cus < 1) {
    set_error("fftconv1d_causal team plan: kernel does not fit a CU (occupancy %d)", per_cu);
    return NSQ_ERR_HIP;
  }
  hipLaunchKernelGGL(team_ctl_clear_kernel, dim3(1), dim3(256), 0, st, static_cast<int*>(ws),
                     int(sizeof(TeamCtl) / sizeof(int)));
  NSQ_CHECK_LAUNCH();
  void* kargs[] = {&args};
  const int grid = cus * (per_cu < kTeamSub ? per_cu : kTeamSub);
  NSQ_CHECK_HIP(hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kernel), dim3(grid), dim3(kTeamThreads), kargs,
                                           0, st));
  return NSQ_OK;
}

template <int DT>
static int team_fwd_dt(const void* x, const float* k, const void* s, void* y, int H, int L, int K, void* ws,
                       const float2* tw, hipStream_t st) {
  TeamFwdArgs a{x, k, s, y, H, L, K, tw, ws, kTeamMaxSpin};
  return team_launch(team_fwd_kernel<DT, 8, 10>, a, ws, st);
}

template <int DT>
static int team_bwd_dt(const void* g, const void* x, const float* k, const void* s, void* gx, float* gk, float* gs,
                       int H, int L, int K, void* ws, const float2* tw, hipStream_t st) {
  TeamBwdArgs a{g, x, k, s, gx, gk, gs, H, L, K, tw, ws, kTeamMaxSpin};
  return team_launch(team_bwd_kernel<DT, 8, 10>, a, ws, st);
}

int team_fwd(const Plan1D& p, int dtype, const void* x, const float* k, const void* s, void* y, int H, int L, int K,
             void* ws, const float2* tw, hipStream_t st) {
  (void)p;
  switch (dtype) {
    case NSQ_DTYPE_F32: return team_fwd_dt<NSQ_DTYPE_F32>(x, k, s, y, H, L, K, ws, tw, st);
    case NSQ_DTYPE_BF16: return team_fwd_dt<NSQ_DTYPE_BF16>(x, k, s, y, H, L, K, ws, tw, st);
    default: return team_fwd_dt<NSQ_DTYPE_F16>(x, k, s, y, H, L, K, ws, tw, st);
  }
}

int team_bwd(const Plan1D& p, int dtype, const void* g, const void* x, const float* k, const void* s, void* gx,
             float* gk, float* gs, int H, int L, int K, void* ws, const float2* tw, hipStream_t st) {
  (void)p;
  switch (dtype) {
    case NSQ_DTYPE_F32: return team_bwd_dt<NSQ_DTYPE_F32>(g, x, k, s, gx, gk, gs, H, L, K, ws, tw, st);
    case NSQ_DTYPE_BF16: return team_bwd_dt<NSQ_DTYPE_BF16>(g, x, k, s, gx, gk, gs, H, L, K, ws, tw, st);
    default: return team_bwd_dt<NSQ_DTYPE_F16>(g, x, k, s, gx, gk, gs, H, L, K, ws, tw, st);
  }
}

}  // namespace nsq
