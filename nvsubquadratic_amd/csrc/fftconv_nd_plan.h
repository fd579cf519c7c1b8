// Host plans of the 2D / 3D non-causal FFT convolution, shared by the plain
// and mixed-boundary entry points (fftconv_nd.hip) and the gated ones
// (fftconv_nd_gated.hip); see fftconv_nd_impl.h for the kernels and the pass
// structure.
#pragma once

#include <cstdlib>

#include "fftconv2d_image.h"
#include "fftconv_nd_impl.h"

namespace nsq {

// Boundary condition per axis (ops/mixed_fftconv.py:295-343, `_mixed_recipe`):
//   zero-padded ("same"): F_d = 2^ceil(log2(S_d + ceil(K_d/2))) >= 16, output
//     window [K_d/2, K_d/2 + S_d) of the linear conv (crop o_d = K_d/2);
//   periodic (circular):  F_d = S_d (a power of two in [16, 2^kNdMaxLogF]),
//     K_d <= S_d, output = the whole circular conv rolled by -(K_d-1)/2, done
//     as a ramp on the filter spectrum (r_d = (K_d-1)/2, o_d = 0).  A shorter
//     power-of-two period (2, 4, 8) is tiled: F_d = 16 and the first passes read
//     x and g at index n & (S_d - 1) (their periodic extension, of which the
//     period-16 circular conv restricted to [0, S_d) is the period-S_d one;
//     the filter is not extended).  The extension repeats every product
//     F_d / S_d times, so gk and gs are scaled by S_d / F_d.  A period of 1 is
//     the zero-padded 1-tap case.
// Either way y[n] = sum_j k[j] x[n + c_d - j] along the axis, c_d = o_d + r_d,
// which is the shift the backward's ramp and its gs lag use.
struct NdPlan {
  int nd;
  int64_t B, H, kb;      // kb = kernel batch: 1 (shared) or B (per-sample FiLM)
  int S[3], K[3];        // padded to 3 axes: (S0, S1, S2) with S1 = K1 = 1 for 2D
  int lF[3], F[3], c[3];
  int o[3], r[3];        // forward crop offsets and forward ramp shifts (c = o + r)
  bool ramp;             // some r_d != 0
  int wm[3];             // index mask of x / g along the axis: -1, or S_d - 1 for a tiled periodic axis
  float gk_scale;        // 1 / (product of F_d / S_d over tiled axes): gk, gs of the periodic extension
  bool pack;             // 2D: the DC and Nyquist bins share bin 0 (FH = F2/2)
  int FH;        // spectrum columns along the last axis: F2/2 + 1, or F2/2 packed
  int RS;        // spectrum row stride (complex elements), >= FH
  int64_t spec;
  bool r3;       // mixed-radix plan (fftconv_nd_r3.h): F_d in {48, 96, 192}, lF unused
};

// The mixed-radix plan is taken where it applies unless NSQ_ND_R3=0 (read per
// call, so the workspace size and the run agree for a given setting).
inline bool nd_r3_allowed() {
  const char* e = std::getenv("NSQ_ND_R3");
  return !(e && e[0] == '0');
}

// Axis-0 columns per workgroup of the mixed-radix column passes (R3ColCfg::M).
inline int r3_col_m(int F0) { return F0 == 48 ? 32 : 16; }

// `periodic`: bit d set = axis d (of the nd given axes) is periodic.
// allow_r3 = false builds the power-of-two plan whatever the shape.
inline bool make_nd_plan(int nd, int64_t B, int64_t H, const int64_t* S, const int64_t* K, int64_t kb,
                         unsigned periodic, NdPlan& p, bool allow_r3 = true) {
  if (nd != 2 && nd != 3) return false;
  if (periodic >> nd) return false;
  p.nd = nd;
  p.B = B;
  p.H = H;
  p.kb = kb;
  p.r3 = false;
  p.ramp = false;
  p.gk_scale = 1.f;
  int s[3] = {1, 1, 1}, k[3] = {1, 1, 1};
  bool per[3] = {false, false, false};
  if (nd == 2) {
    s[0] = int(S[0]); s[2] = int(S[1]);
    k[0] = int(K[0]); k[2] = int(K[1]);
    per[0] = periodic & 1u; per[2] = (periodic >> 1) & 1u;
  } else {
    for (int d = 0; d < 3; ++d) { s[d] = int(S[d]); k[d] = int(K[d]); per[d] = (periodic >> d) & 1u; }
  }
  for (int d = 0; d < 3; ++d) {
    p.S[d] = s[d];
    p.K[d] = k[d];
    p.wm[d] = -1;
    if (nd == 2 && d == 1) {
      p.lF[d] = 0; p.F[d] = 1; p.c[d] = 0; p.o[d] = 0; p.r[d] = 0;
      continue;
    }
    if (per[d] && s[d] > 1) {
      if (k[d] < 1 || k[d] > s[d] || (s[d] & (s[d] - 1))) return false;
      int lf = ilog2_ceil(s[d]);
      if (lf > kNdMaxLogF) return false;
      if (lf < 4) {  // tiled short period
        p.wm[d] = s[d] - 1;
        p.gk_scale *= float(s[d]) / 16.f;
        lf = 4;
      }
      p.lF[d] = lf;
      p.F[d] = 1 << lf;
      p.c[d] = p.r[d] = (k[d] - 1) / 2;
      p.o[d] = 0;
      p.ramp = p.ramp || p.r[d] != 0;
      continue;
    }
    if (s[d] < 1 || k[d] < 1 || k[d] > 2 * s[d]) return false;
    int lf = ilog2_ceil(int64_t(s[d]) + (k[d] + 1) / 2);
    if (lf < 4) lf = 4;
    if (lf > kNdMaxLogF) return false;
    p.lF[d] = lf;
    p.F[d] = 1 << lf;
    p.c[d] = p.o[d] = k[d] / 2;
    p.r[d] = 0;
  }
  // 2D rows store the real DC and Nyquist bins packed in bin 0 (N columns, a
  // multiple of the axis-0 passes' column tiles, instead of N + 1 with a
  // one-column tail); 3D keeps N + 1 (its axis-1 pass pairs across columns).
  p.pack = nd == 2;
  p.FH = p.pack ? p.F[2] / 2 : p.F[2] / 2 + 1;
  // 2D: rows padded to a multiple of 16 complex values (a pad only for
  // F2 = 16), so the 16-column segments the axis-0 passes move per row start
  // on a 128-byte line.  The pad is never read or written.  3D planes are F1 rows of FH: the axis-0 segments are aligned
  // there already (the plane stride is a multiple of 16) and the plane passes
  // keep their compile-time row stride.
  p.RS = nd == 2 ? (p.FH + 15) / 16 * 16 : p.FH;
  p.spec = int64_t(p.F[0]) * p.F[1] * p.RS;
  // The reference's FFT sizes (ops/fftconv.py:699-702, 774-778: F_d = S_d +
  // ceil(K_d/2), mixed-radix): with every axis zero-padded, the mixed-radix
  // plan runs when each axis fits a length 3 * 2^m it has kernels for (3D:
  // 48 or 96, axis 0 also 192; 2D: 48, 96 or 192) and the spectrum is smaller
  // than the power-of-two one (96^3 against 128^3 at S = K = 64, 192^2
  // against 256^2 at S = K = 128).
  if (periodic == 0 && allow_r3 && nd_r3_allowed()) {
    int f3[3] = {1, 1, 1};
    bool ok = true;
    for (int d = 0; d < 3; ++d) {
      if (nd == 2 && d == 1) continue;
      const int64_t need = int64_t(s[d]) + (k[d] + 1) / 2;
      const bool long_ok = d == 0 || nd == 2;  // 192 on axis 0, and on both axes of a 2D plane
      f3[d] = need <= 48 ? 48 : need <= 96 ? 96 : (long_ok && need <= 192) ? 192 : 0;
      ok = ok && f3[d] != 0;
    }
    const int64_t spec3 = int64_t(f3[0]) * f3[1] * (f3[2] / 2 + 1);
    if (ok && spec3 < p.spec) {
      p.r3 = true;
      for (int d = 0; d < 3; ++d) {
        p.F[d] = f3[d];
        p.lF[d] = 0;
      }
      p.pack = false;
      p.FH = p.RS = f3[2] / 2 + 1;
      p.spec = spec3;
    }
  }
  return true;
}

// ---------------------------------------------------------------------------
// Compile-time dispatch of the row / column passes on their log2 sizes.
// ---------------------------------------------------------------------------
template <int LO, int HI, class F>
bool with_log(int v, F&& f) {
  if constexpr (LO > HI) {
    return false;
  } else {
    if (v == LO) {
      f(std::integral_constant<int, LO>{});
      return true;
    }
    return with_log<LO + 1, HI>(v, f);
  }
}

// wrap: x / g (read through the plan's periodic extension masks); the filter
// is never extended.  GL: gate formed by the loads (GATED_*, packed 2D rows
// only; gi holds its operands).
template <int DT, int GL = GATED_NONE>
bool row_fwd(const NdPlan& p, const void* src, int64_t nbh, int n0, int n1, int len, bool wrap, float2* ws,
             const float2* tw, hipStream_t st, const GatedIO& gi = GatedIO{}) {
  RowGeom rg{nbh * n0 * n1, n0, n1, p.spec, p.F[1], p.RS};
  const int wm = wrap ? p.wm[2] : -1;
  return with_log<3, kNdMaxLogF - 1>(p.lF[2] - 1, [&](auto L) {
    constexpr int LOGN = decltype(L)::value;
    using C = RowNdCfg<LOGN>;
    const dim3 grid{unsigned(ceil_div(rg.rows, C::M))};
    using ET = typename Elem<DT>::T;
    auto go = [&](auto al, auto half) {
      constexpr bool A = decltype(al)::value, H = decltype(half)::value;
      if (p.pack)
        hipLaunchKernelGGL((nd_row_fwd_kernel<LOGN, DT, A, H, true, GL>), grid, dim3(C::T), 0, st, (const ET*)src,
                           len, wm, rg, ws, tw, gi);
      else if constexpr (GL == GATED_NONE)  // gated_fused_ok: gates only on packed rows
        hipLaunchKernelGGL((nd_row_fwd_kernel<LOGN, DT, A, H, false>), grid, dim3(C::T), 0, st, (const ET*)src, len,
                           wm, rg, ws, tw, gi);
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    const bool al = pairs_aligned<DT>(src, len, len);
    if (len <= C::N && wm == -1)  // packed samples [N/2, N) of every row are zero
      al ? go(T_{}, T_{}) : go(F_{}, T_{});
    else
      al ? go(T_{}, F_{}) : go(F_{}, F_{});
  });
}

// Whether row_inv runs the vectorized epilogue (FAST) for `o`: the gated
// epilogues exist only there.
inline bool row_inv_fast(const RowInvOut& o) {
  return o.off2 % 2 == 0 && o.w2 % 8 == 0 && (reinterpret_cast<uintptr_t>(o.out) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(o.aux) & 15) == 0;
}

// GE: gated epilogue (GATED_*; packed rows with row_inv_fast(o) only).
template <int DT, int MODE, int GE = GATED_NONE>
bool row_inv(const NdPlan& p, const float2* ws, int64_t nbh, int n0, int n1, RowInvOut o, const float2* tw,
             hipStream_t st) {
  RowGeom rg{nbh * n0 * n1, n0, n1, p.spec, p.F[1], p.RS};
  return with_log<3, kNdMaxLogF - 1>(p.lF[2] - 1, [&](auto L) {
    constexpr int LOGN = decltype(L)::value;
    using C = RowNdCfg<LOGN>;
    const dim3 grid(unsigned(ceil_div(rg.rows, C::M)));
    const bool fast = MODE == ND_OUT_Y && row_inv_fast(o);
    auto go = [&](auto has_s, auto fst, auto pack) {
      hipLaunchKernelGGL((nd_row_inv_kernel<LOGN, DT, MODE, decltype(has_s)::value, decltype(fst)::value,
                                            decltype(pack)::value>),
                         grid, dim3(C::T), 0, st, ws, rg, o, tw);
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    auto go_pack = [&](auto has_s, auto fst) { p.pack ? go(has_s, fst, T_{}) : go(has_s, fst, F_{}); };
    if constexpr (MODE == ND_OUT_Y && GE != GATED_NONE) {
      auto gated = [&](auto has_s) {  // gated_fused_ok: packed rows, fast epilogue
        hipLaunchKernelGGL((nd_row_inv_kernel<LOGN, DT, MODE, decltype(has_s)::value, true, true, GE>), grid,
                           dim3(C::T), 0, st, ws, rg, o, tw);
      };
      o.s ? gated(T_{}) : gated(F_{});
    } else if constexpr (MODE == ND_OUT_Y) {
      if (fast) {
        o.s ? go_pack(T_{}, T_{}) : go_pack(F_{}, T_{});
        return;
      }
      o.s ? go_pack(T_{}, F_{}) : go_pack(F_{}, F_{});
    } else {
      go_pack(F_{}, F_{});
    }
  });
}

// Column blocks of a pass: full blocks of the kernel's regular width, then the
// remainder in blocks of kNdTailTile's 4 columns at column offset jbase (a
// remainder exists for short 2D rows, FH = F2/2 < 16, and for 3D blocks whose
// F1 * FH is not a multiple of the width).  launch(tile, grid_y, jbase)
// launches one instance.
constexpr int kNdTailTile = 1;  // ColNdCfg clamps this to 4 columns
template <int LOGF, int TARGET, class LAUNCH>
void col_blocks(int inner, LAUNCH&& launch) {
  using CM = ColNdCfg<LOGF, TARGET>;
  using CT = ColNdCfg<LOGF, kNdTailTile>;
  const int full = inner / CM::M, rem = inner - full * CM::M;
  if (full) launch(std::integral_constant<int, TARGET>{}, full, 0);
  if (rem) launch(std::integral_constant<int, kNdTailTile>{}, int(ceil_div(rem, CT::M)), full * CM::M);
}

// Column-block workgroups per channel of an axis-0 pass with tile target
// `target` (col_blocks: full blocks of M columns, then blocks of 4).
inline int64_t axis0_blocks(const NdPlan& p, int target) {
  const int inner = p.F[1] * p.FH;
  if (p.r3) return ceil_div(inner, r3_col_m(p.F[0]));
  int m = target >> p.lF[0];
  m = m < 4 ? 4 : (m > 16 ? 16 : m);
  const int full = inner / m, rem = inner - full * m;
  return full + (rem + 3) / 4;
}

// Batch split of the axis-0 product / adjoint passes for a shared kernel: a
// workgroup per (channel, column block) loops over the batch, so few channels
// and small spectra leave CUs idle.  Below `lo` workgroups the batch is split
// until about `want` are in flight.  The product pass splits for free (each
// share re-reads only its filter columns): lo 4096, want 6144 (24 per CU);
// the adjoint's shares each add a partial filter-gradient block and a reduce:
// lo 1024, want 3072 (measured on MI355X: more shares cost more than they
// hide there).  FiLM kernels already launch B*H workgroups.
inline int axis0_batch_split(const NdPlan& p, int target, int64_t lo, int64_t want_total) {
  if (p.kb != 1) return 1;
  const int64_t wgs = p.H * axis0_blocks(p, target);
  if (wgs >= lo) return 1;
  const int64_t want = (want_total + wgs - 1) / wgs;
  return int(want < p.B ? want : p.B);
}
inline int mul_batch_split(const NdPlan& p) { return axis0_batch_split(p, 8192, 4096, 6144); }
inline int bwd_batch_split(const NdPlan& p) { return axis0_batch_split(p, kNdBwdTile, 1024, 3072); }

// Axis-0 columns: the inner index j runs over a block's F1 rows of the last
// axis; 3D packs them (RS = FH), 2D has one padded row (F1 = 1, j < FH).
inline ColGeom axis0_geom(const NdPlan& p) {
  return ColGeom{1, 0, p.spec, int64_t(p.F[1]) * p.RS, p.F[1] * p.FH};
}

// Column pass along axis d (0 or 1) of `nbh` blocks whose valid extent along
// axis 0 is n_valid0 (used as the middle-row count of axis-1 passes).
template <bool INV>
bool col_pass(const NdPlan& p, float2* ws, int64_t nbh, int axis, int n_valid0, int in_cnt, int out_off,
                     int out_cnt, const float2* tw, hipStream_t st, int wm = -1) {
  ColGeom cg;
  if (axis == 1) {
    cg = ColGeom{n_valid0, int64_t(p.F[1]) * p.RS, p.spec, int64_t(p.RS), p.FH};
  } else {
    cg = axis0_geom(p);
  }
  const int64_t n_outer = nbh * cg.n_mid;
  return with_log<4, kNdMaxLogF>(p.lF[axis], [&](auto L) {
    constexpr int LOGF = decltype(L)::value;
    col_blocks<LOGF, 8192>(cg.inner_count, [&](auto tile, int gy, int jbase) {
      constexpr int TGT = decltype(tile)::value;
      hipLaunchKernelGGL((nd_col_kernel<LOGF, INV, TGT>), dim3(unsigned(n_outer), unsigned(gy)),
                         dim3(ColNdCfg<LOGF, TGT>::T), 0, st, ws, cg, in_cnt, wm, out_off, out_cnt, jbase, tw);
    });
  });
}

// Plane passes (3D, a (b, h, a0) plane fits in LDS): both inner axes in one
// kernel.  plane_ok mirrors PlaneCfg::OK for the plan's sizes.
inline bool plane_ok(const NdPlan& p) {
  if (p.nd != 3 || p.r3) return false;
  const int logn = p.lF[2] - 1, logf1 = p.lF[1];
  if (logn < 4 || logn > 9 || logf1 < 4 || logf1 > kNdMaxLogF) return false;
  const int n = 1 << logn, f1 = 1 << logf1, mr = 4096 >> logn, mc = 4096 >> logf1;
  return mr >= 1 && mr <= f1 && mc >= 1 && mc <= n && int64_t(f1) * (n + n / 16) * 8 <= 80 * 1024;
}

template <class F>
bool with_plane(const NdPlan& p, F&& f) {
  bool launched = false;
  with_log<4, 9>(p.lF[2] - 1, [&](auto LN) {
    constexpr int LOGN = decltype(LN)::value;
    with_log<4, kNdMaxLogF>(p.lF[1], [&](auto LF) {
      constexpr int LOGF1 = decltype(LF)::value;
      if constexpr (PlaneCfg<LOGN, LOGF1>::OK) {
        f(std::integral_constant<int, LOGN>{}, std::integral_constant<int, LOGF1>{});
        launched = true;
      }
    });
  });
  return launched;
}

// Forward inner-axis transforms of nbh blocks of [n0][n1][len] real rows
// (wrap: x / g, read through the periodic extension masks).
// GL: gate formed by the first pass's loads (GATED_*; the packed 2D rows or
// the 3D plane pass only, see gated_fused_ok).
template <int DT, int GL = GATED_NONE>
bool inner_fwd(const NdPlan& p, const void* src, int64_t nbh, int n0, int n1, int len, bool wrap, float2* ws,
               const float2* tw, hipStream_t st, const GatedIO& gi = GatedIO{}) {
  const int wm1 = wrap ? p.wm[1] : -1, wm2 = wrap ? p.wm[2] : -1;
  if (plane_ok(p)) {
    using ET = typename Elem<DT>::T;
    const bool al = pairs_aligned<DT>(src, len, len);
    return with_plane(p, [&](auto LN, auto LF) {
      constexpr int LOGN = decltype(LN)::value, LOGF1 = decltype(LF)::value;
      const dim3 grid(unsigned(nbh * n0));
      auto go = [&](auto alc, auto half) {
        constexpr bool A = decltype(alc)::value, H = decltype(half)::value;
        hipLaunchKernelGGL((nd_plane_fwd_kernel<LOGN, LOGF1, DT, A, H, GL>), grid, dim3(256), 0, st, (const ET*)src,
                           n0, n1, len, wm1, wm2, ws, p.spec, tw, gi);
      };
      using T_ = std::true_type;
      using F_ = std::false_type;
      if (len <= (1 << LOGN) && 2 * n1 <= (1 << LOGF1) && wm1 == -1 && wm2 == -1)  // at least half zero padding
        al ? go(T_{}, T_{}) : go(F_{}, T_{});
      else
        al ? go(T_{}, F_{}) : go(F_{}, F_{});
    });
  }
  if (!row_fwd<DT, GL>(p, src, nbh, n0, n1, len, wrap, ws, tw, st, gi)) return false;
  return p.nd != 3 || col_pass<false>(p, ws, nbh, 1, n0, n1, 0, p.F[1], tw, st, wm1);
}

// Inverse inner-axis transforms, crop (axis 1: [off1, off1 + n1out); axis 2:
// RowInvOut) and epilogue, for nbh blocks whose axis-0 extent is n0.
// GE: gated epilogue (GATED_*; the packed 2D rows with the vector epilogue
// or the 3D plane pass only, see gated_fused_ok).
template <int DT, int MODE, int GE = GATED_NONE>
bool inner_inv(const NdPlan& p, float2* ws, int64_t nbh, int n0, int off1, int n1out, RowInvOut o,
               const float2* tw, hipStream_t st) {
  if (plane_ok(p)) {
    const bool has_s = MODE == ND_OUT_Y && o.s;
    return with_plane(p, [&](auto LN, auto LF) {
      constexpr int LOGN = decltype(LN)::value, LOGF1 = decltype(LF)::value;
      const dim3 grid(unsigned(nbh * n0));
      auto go = [&](auto hs) {
        hipLaunchKernelGGL((nd_plane_inv_kernel<LOGN, LOGF1, DT, MODE, decltype(hs)::value, GE>), grid, dim3(256), 0,
                           st, (const float2*)ws, p.spec, n0, off1, n1out, o, tw);
      };
      has_s ? go(std::true_type{}) : go(std::false_type{});
    });
  }
  if (p.nd == 3 && !col_pass<true>(p, ws, nbh, 1, n0, p.F[1], off1, n1out, tw, st)) return false;
  return row_inv<DT, MODE, GE>(p, ws, nbh, n0, n1out, o, tw, st);
}



// Filter spectrum: kb*H blocks of the [kb*H][K0][K1][K2] float32 kernel.
// Shapes the one-kernel image forward (fftconv2d_image.h) takes; the caller
// also needs a forward that keeps no state, a shared filter and no gates.
inline bool image_fwd_ok(const NdPlan& p, const void* x, const void* y) {
  return p.nd == 2 && p.kb == 1 && !p.ramp && p.wm[0] == -1 && p.wm[2] == -1 && p.F[0] == 256 && p.F[2] == 256 &&
         p.S[0] <= 128 && p.S[2] <= 128 && p.o[0] <= 128 && p.o[2] % 2 == 0 && p.S[2] % 8 == 0 && p.pack &&
         p.RS == 128 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0 &&
         p.B * p.H <= int64_t(1) << 30;
}

template <int DT>
inline void launch_image_fwd(const NdPlan& p, const void* x, const float2* khat, const void* s, void* y,
                             const float2* tw, hipStream_t st) {
  using ET = typename Elem<DT>::T;
  const dim3 grid(unsigned(p.B * p.H));
  const float scale = 1.f / (float(p.F[0]) * float(p.F[2] / 2));
  constexpr int T = kImgThreads;
  if (s)
    hipLaunchKernelGGL((nd2_image_fwd_kernel<DT, true, T>), grid, dim3(T), 0, st, (const ET*)x, khat, p.RS,
                       (const ET*)s, (ET*)y, int(p.B), int(p.H), p.S[0], p.S[2], p.o[0], p.o[2], scale, tw);
  else
    hipLaunchKernelGGL((nd2_image_fwd_kernel<DT, false, T>), grid, dim3(T), 0, st, (const ET*)x, khat, p.RS,
                       (const ET*)s, (ET*)y, int(p.B), int(p.H), p.S[0], p.S[2], p.o[0], p.o[2], scale, tw);
}

// (A template, so that only the units that run the plan instantiate its kernels.)
template <int DT = NSQ_DTYPE_F32>
bool filter_spectrum(const NdPlan& p, const float* k, float2* wsk, const float2* tw, hipStream_t st) {
  const int64_t nk = p.kb * p.H;
  if (!inner_fwd<DT>(p, k, nk, p.K[0], p.K[1], p.K[2], false, wsk, tw, st)) return false;
  return col_pass<false>(p, wsk, nk, 0, 1, p.K[0], 0, p.F[0], tw, st);
}

// A forward that keeps no state for a backward runs whole 2D images in one
// kernel where the shape allows (fftconv2d_image.h); NSQ_2D_IMAGE_FWD=0
// selects the passes of the plan instead.
inline bool image_fwd_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("NSQ_2D_IMAGE_FWD");
    return !(e && e[0] == '0');
  }();
  return on;
}

// NSQ_2D_IMAGE192=0: no one-kernel image forward on the 192 x 192 plane.
inline bool image192_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("NSQ_2D_IMAGE192");
    return !(e && e[0] == '0');
  }();
  return on;
}

// The power-of-two plan of the shape of p (no periodic axes: the mixed-radix
// plan has none).
inline bool pow2_plan_of(const NdPlan& p, NdPlan& p2) {
  const int64_t S[3] = {p.S[0], p.nd == 2 ? p.S[2] : p.S[1], p.S[2]};
  const int64_t K[3] = {p.K[0], p.nd == 2 ? p.K[2] : p.K[1], p.K[2]};
  return make_nd_plan(p.nd, p.B, p.H, S, K, p.kb, 0u, p2, false);
}

// The mixed-radix plan's passes (fftconv_nd_r3.hip, one instance per dtype),
// same arguments, workspace layout and results as run_nd_fwd / run_nd_bwd.
template <int DT>
bool run_r3_fwd(const NdPlan& p, const void* x, const float* k, const void* s, void* y, float2* ws, bool save,
                const float2* tw, hipStream_t st);
template <int DT>
bool run_r3_bwd(const NdPlan& p, const void* g, const void* x, const float* k, const void* s, void* gx, float* gk,
                float* gs, float2* ws, bool fwd_state, const float2* tw, hipStream_t st);
template <int DT>
bool run_r3_image_fwd(const NdPlan& p, const void* x, const float* k, const void* s, void* y, float2* ws,
                      const float2* tw, hipStream_t st);
#define NSQ_R3_RUN_INSTANCES(EXT, DT)                                                                               \
  EXT template bool run_r3_fwd<DT>(const NdPlan&, const void*, const float*, const void*, void*, float2*, bool,    \
                                   const float2*, hipStream_t);                                                  \
  EXT template bool run_r3_image_fwd<DT>(const NdPlan&, const void*, const float*, const void*, void*, float2*,   \
                                         const float2*, hipStream_t);                                            \
  EXT template bool run_r3_bwd<DT>(const NdPlan&, const void*, const void*, const float*, const void*, void*,      \
                                   float*, float*, float2*, bool, const float2*, hipStream_t);
NSQ_R3_RUN_INSTANCES(extern, NSQ_DTYPE_F32)
NSQ_R3_RUN_INSTANCES(extern, NSQ_DTYPE_BF16)
NSQ_R3_RUN_INSTANCES(extern, NSQ_DTYPE_F16)

// Workspace layout (spectrum blocks of p.spec complex64):
//   backward: [G: BH | X: BH | Khat: NK | Q: NK | (nz - 1) * NK partial Q]
//     (nz = bwd_batch_split: the adjoint's batch split, 1 for most shapes)
//   forward with `save` (a backward-sized workspace): X after the inner-axis
//     passes and Khat at the backward's positions, the product in the G region;
//     the backward called with fwd_state then starts from them.
//   forward without `save`: [X (product in place): BH | Khat: NK].
// GATED: the Hyena gates fused into the first and last passes, operands in
// *gate (x is then q; gated_nd_fwd).
template <int DT, bool GATED = false>
bool run_nd_fwd(const NdPlan& p, const void* x, const float* k, const void* s, void* y, float2* ws, bool save,
                const float2* tw, hipStream_t st, const GatedIO* gate = nullptr) {
  constexpr int GM = GATED ? GATED_FWD : GATED_NONE;
  if (p.r3) {  // the gated ops run their gate kernels around the plain conv on this plan
    if constexpr (GATED) {
      return false;
    } else {
      // A 2D forward that keeps no state runs the one-kernel image forward of
      // the power-of-two plan where that applies: 0.82 ms against 1.00 ms for
      // the mixed-radix passes at config 4 (measured).  Its filter spectrum
      // (H blocks of 256 x 128) goes to the workspace start; the mixed-radix
      // forward workspace ((B + 1) H blocks of 192 x 97) holds it.
      if (!save && p.nd == 2 && p.kb == 1 && image192_enabled() && run_r3_image_fwd<DT>(p, x, k, s, y, ws, tw, st))
        return true;
      NdPlan p2;
      if (!save && p.nd == 2 && p.kb == 1 && image_fwd_enabled() && pow2_plan_of(p, p2) && image_fwd_ok(p2, x, y) &&
          p2.H * p2.spec <= (p.B * p.H + p.H) * p.spec) {
        if (!filter_spectrum(p2, k, ws, tw, st)) return false;
        launch_image_fwd<DT>(p2, x, ws, s, y, tw, st);
        return true;
      }
      return run_r3_fwd<DT>(p, x, k, s, y, ws, save, tw, st);
    }
  }
  const int64_t BH = p.B * p.H;
  float2* wsx = save ? ws + BH * p.spec : ws;
  float2* wsk = wsx + BH * p.spec;
  float2* wsy = save ? ws : wsx;
  if (!filter_spectrum(p, k, wsk, tw, st)) return false;
  if (!GATED && !save && image_fwd_enabled() && image_fwd_ok(p, x, y)) {
    launch_image_fwd<DT>(p, x, wsk, s, y, tw, st);
    return true;
  }
  const GatedIO gi = GATED ? *gate : GatedIO{};
  if (!inner_fwd<DT, GM>(p, x, BH, p.S[0], p.S[1], p.S[2], true, wsx, tw, st, gi)) return false;
  const ColGeom cg = axis0_geom(p);
  const Ramp rf{p.r[0], p.r[1], p.r[2], p.lF[0], p.lF[1], p.lF[2], p.FH};
  bool ok = with_log<4, kNdMaxLogF>(p.lF[0], [&](auto L) {
    constexpr int LOGF = decltype(L)::value;
    col_blocks<LOGF, 8192>(cg.inner_count, [&](auto tile, int gy, int jbase) {
      constexpr int TGT = decltype(tile)::value;
      // a narrow tail instance (3D blocks whose F1 * FH is not a multiple of
      // the column tile, or 2D rows shorter than 16 bins) takes one image per
      // workgroup: its work per image is small
      const int bsplit = (TGT == kNdTailTile && p.kb == 1) ? int(p.B) : mul_batch_split(p);
      const dim3 grid(unsigned((p.kb != 1 ? BH : p.H) * bsplit), unsigned(gy));
      auto go = [&](auto half, auto ramp) {
        auto launch = [&](auto pack) {
          hipLaunchKernelGGL(
              (nd_col_mul_kernel<LOGF, TGT, decltype(half)::value, decltype(ramp)::value, decltype(pack)::value>),
              grid, dim3(ColNdCfg<LOGF, TGT>::T), 0, st, (const float2*)wsx, wsy, (const float2*)wsk, cg, int(p.B),
              int(p.H), int(p.kb != 1), p.S[0], p.wm[0], p.o[0], rf, jbase, bsplit, tw);
        };
        p.pack ? launch(std::true_type{}) : launch(std::false_type{});
      };
      using T_ = std::true_type;
      using F_ = std::false_type;
      if (2 * p.S[0] <= p.F[0] && p.wm[0] == -1)  // the x columns are at least half zero padding
        p.ramp ? go(T_{}, T_{}) : go(T_{}, F_{});
      else
        p.ramp ? go(F_{}, T_{}) : go(F_{}, F_{});
    });
  });
  if (!ok) return false;
  RowInvOut o{y, x, s, nullptr, int(p.H), p.o[2], p.S[2], 0, 0, 0,
              1.f / (float(p.F[0]) * float(p.F[1]) * float(p.F[2] / 2)), gi};
  return inner_inv<DT, ND_OUT_Y, GM>(p, wsy, BH, p.S[0], p.o[1], p.S[1], o, tw, st);
}

// The wave-local adjoint of 128-point axis-0 columns (nd_col_bwd_w128_kernel);
// NSQ_ND_BWD_W128=0 selects the workgroup-tile kernel for every shape.
inline bool w128_bwd_on() {
  static const bool on = [] {
    const char* e = std::getenv("NSQ_ND_BWD_W128");
    return !(e && e[0] == '0');
  }();
  return on;
}

// GATED: the Hyena gates fused into the first and last passes, operands in
// *gate (x is then q, g the gradient of the gated output, gx receives dq;
// gated_nd_bwd).
template <int DT, bool GATED = false>
bool run_nd_bwd(const NdPlan& p, const void* g, const void* x, const float* k, const void* s, void* gx, float* gk,
                float* gs, float2* ws, bool fwd_state, const float2* tw, hipStream_t st, const GatedIO* gate = nullptr) {
  if (p.r3) {
    if constexpr (GATED) return false;
    else return run_r3_bwd<DT>(p, g, x, k, s, gx, gk, gs, ws, fwd_state, tw, st);
  }
  const int64_t BH = p.B * p.H, NK = p.kb * p.H;
  float2* wsg = ws;
  float2* wsx = wsg + BH * p.spec;
  float2* wsk = wsx + BH * p.spec;
  float2* wsq = wsk + NK * p.spec;
  const GatedIO gi = GATED ? *gate : GatedIO{};
  if (!fwd_state) {
    if (!filter_spectrum(p, k, wsk, tw, st)) return false;
    if (!inner_fwd<DT, GATED ? GATED_FWD : GATED_NONE>(p, x, BH, p.S[0], p.S[1], p.S[2], true, wsx, tw, st, gi))
      return false;
  }
  if (!inner_fwd<DT, GATED ? GATED_BWD : GATED_NONE>(p, g, BH, p.S[0], p.S[1], p.S[2], true, wsg, tw, st, gi))
    return false;
  const ColGeom cg = axis0_geom(p);
  const Ramp rp{p.c[0], p.c[1], p.c[2], p.lF[0], p.lF[1], p.lF[2], p.FH};
  const int nz = bwd_batch_split(p);  // partial Q blocks follow Q in the workspace
  bool ok = with_log<4, kNdMaxLogF>(p.lF[0], [&](auto L) {
    constexpr int LOGF = decltype(L)::value;
    col_blocks<LOGF, kNdBwdTile>(cg.inner_count, [&](auto tile, int gy, int jbase) {
      constexpr int TGT = decltype(tile)::value;
      const dim3 grid{unsigned(NK), unsigned(gy), unsigned(nz)};
      auto go = [&](auto half, auto pack) {
        if constexpr (LOGF == 7 && TGT == kNdBwdTile && !decltype(pack)::value) {
          static_assert(ColNdCfg<LOGF, TGT>::M == 16 && ColNdCfg<LOGF, TGT>::T == 128, "wave-local adjoint tile");
          if (w128_bwd_on()) {
            hipLaunchKernelGGL((nd_col_bwd_w128_kernel<decltype(half)::value>), grid, dim3(128), 0, st, wsg,
                               (const float2*)wsx, (const float2*)wsk, wsq, cg, int(p.B), int(p.H), int(p.kb != 1),
                               p.S[0], p.wm[0], p.K[0], rp, jbase, NK, tw);
            return;
          }
        }
        hipLaunchKernelGGL((nd_col_bwd_kernel<LOGF, TGT, decltype(half)::value, decltype(pack)::value>), grid,
                           dim3(ColNdCfg<LOGF, TGT>::T), 0, st, wsg, (const float2*)wsx, (const float2*)wsk, wsq,
                           cg, int(p.B), int(p.H), int(p.kb != 1), p.S[0], p.wm[0], p.K[0], rp, jbase, NK, tw);
      };
      using T_ = std::true_type;
      using F_ = std::false_type;
      if (2 * p.S[0] <= p.F[0] && p.wm[0] == -1)  // the g and x columns are at least half zero padding
        p.pack ? go(T_{}, T_{}) : go(T_{}, F_{});
      else
        p.pack ? go(F_{}, T_{}) : go(F_{}, F_{});
    });
  });
  if (!ok) return false;
  if (nz > 1) {
    const int64_t count = int64_t(p.K[0]) * p.F[1] * p.RS;  // rows [0, K0) of a block
    const int64_t blocks = (NK * count + 255) / 256;
    hipLaunchKernelGGL(nd_q_reduce_kernel, dim3(unsigned(blocks < 8192 ? blocks : 8192)), dim3(256), 0, st, wsq, NK,
                       p.spec, count, nz);
  }
  const float scale = 1.f / (float(p.F[0]) * float(p.F[1]) * float(p.F[2] / 2));
  RowInvOut og{gx, g, s, nullptr, int(p.H), 0, p.S[2], 0, 0, 0, scale, gi};
  if (!inner_inv<DT, ND_OUT_Y, GATED ? GATED_BWD : GATED_NONE>(p, wsg, BH, p.S[0], 0, p.S[1], og, tw, st))
    return false;
  RowInvOut ok_{gk, nullptr, nullptr, gs, int(p.H), 0, p.K[2], p.c[0], p.c[1], p.c[2], scale * p.gk_scale};
  return inner_inv<NSQ_DTYPE_F32, ND_OUT_GK>(p, wsq, NK, p.K[0], 0, p.K[1], ok_, tw, st);
}

inline int validate_nd(int nd, const void* a, const void* b, const float* k, int dtype, int64_t B, int64_t H,
                       const int64_t* S, const int64_t* K, int64_t kb, unsigned periodic, NdPlan& p) {
  NSQ_CHECK_ARG(a && b && k && S && K, "fftconv_nd: null pointer argument");
  NSQ_CHECK_ARG(nd == 2 || nd == 3, "fftconv_nd: nd must be 2 or 3 (got %d)", nd);
  NSQ_CHECK_ARG(valid_dtype(dtype), "fftconv_nd: unsupported dtype code %d", dtype);
  NSQ_CHECK_ARG(B >= 1 && H >= 1, "fftconv_nd: sizes must be positive");
  NSQ_CHECK_ARG(kb == 1 || kb == B, "fftconv_nd: kernel batch must be 1 or B (got %lld, B=%lld)", (long long)kb,
                (long long)B);
  NSQ_CHECK_ARG((periodic >> nd) == 0, "fftconv_nd: periodic mask 0x%x names an axis >= nd=%d", periodic, nd);
  for (int d = 0; d < nd; ++d) {
    if ((periodic >> d) & 1u) {
      NSQ_CHECK_ARG(S[d] >= 1 && K[d] >= 1 && K[d] <= S[d],
                    "fftconv_nd: periodic axis %d: kernel size %lld must be in [1, %lld]", d, (long long)K[d],
                    (long long)S[d]);
      if (S[d] > (1 << kNdMaxLogF) || (S[d] & (S[d] - 1))) {
        set_error("fftconv_nd: unsupported shape: periodic axis %d has length %lld; the HIP kernels take periodic "
                  "lengths that are powers of two up to %d",
                  d, (long long)S[d], 1 << kNdMaxLogF);
        return NSQ_ERR_UNSUPPORTED;
      }
    } else {
      NSQ_CHECK_ARG(S[d] >= 1 && K[d] >= 1 && K[d] <= 2 * S[d],
                    "fftconv_nd: axis %d: kernel size %lld must be in [1, 2*%lld]", d, (long long)K[d],
                    (long long)S[d]);
    }
  }
  if (!make_nd_plan(nd, B, H, S, K, kb, periodic, p)) {
    set_error("fftconv_nd: unsupported shape: every axis needs an FFT length <= %d", 1 << kNdMaxLogF);
    return NSQ_ERR_UNSUPPORTED;
  }
  if (B * H * int64_t(p.F[0]) * p.F[1] >= (int64_t(1) << 31)) {  // row passes index rows in 32 bits
    set_error("fftconv_nd: unsupported shape: B*H*F0*F1 = %lld rows exceeds 2^31 - 1",
              (long long)(B * H * int64_t(p.F[0]) * p.F[1]));
    return NSQ_ERR_UNSUPPORTED;
  }
  if (p.spec * int64_t(sizeof(float2)) >= (int64_t(1) << 31)) {  // column passes: 32-bit offsets in a block
    set_error("fftconv_nd: unsupported shape: one spectrum block of %lld complex values exceeds 2 GiB",
              (long long)p.spec);
    return NSQ_ERR_UNSUPPORTED;
  }
  return NSQ_OK;
}

inline size_t nd_workspace_bytes(int nd, int64_t B, int64_t H, const int64_t* S, const int64_t* K, int64_t kbatch,
                                 unsigned periodic, int direction) {
  NdPlan p;
  if (!S || !K || !make_nd_plan(nd, B, H, S, K, kbatch, periodic, p)) return 0;
  const int64_t blocks = direction == NSQ_DIR_BWD
                             ? (2 * B * H + (1 + bwd_batch_split(p)) * kbatch * H)
                             : (B * H + kbatch * H);
  return size_t(blocks * p.spec) * sizeof(float2);
}

// The run_nd_* instances are compiled once each, in fftconv_nd_{f32,bf16,f16}.hip
// (plain) and fftconv_nd_gated_{f32,bf16,f16}.hip (GATED), so that the long
// kernel instantiations build in parallel.
#define NSQ_ND_RUN_INSTANCES(EXT, DT, GATED)                                                                       \
  EXT template bool run_nd_fwd<DT, GATED>(const NdPlan&, const void*, const float*, const void*, void*, float2*,    \
                                          bool, const float2*, hipStream_t, const GatedIO*);                      \
  EXT template bool run_nd_bwd<DT, GATED>(const NdPlan&, const void*, const void*, const float*, const void*,      \
                                          void*, float*, float*, float2*, bool, const float2*, hipStream_t,        \
                                          const GatedIO*);
NSQ_ND_RUN_INSTANCES(extern, NSQ_DTYPE_F32, false)
NSQ_ND_RUN_INSTANCES(extern, NSQ_DTYPE_BF16, false)
NSQ_ND_RUN_INSTANCES(extern, NSQ_DTYPE_F16, false)
NSQ_ND_RUN_INSTANCES(extern, NSQ_DTYPE_F32, true)
NSQ_ND_RUN_INSTANCES(extern, NSQ_DTYPE_BF16, true)
NSQ_ND_RUN_INSTANCES(extern, NSQ_DTYPE_F16, true)

// Plain and mixed-boundary conv (fftconv_nd.hip).
int nd_fwd(int nd, const void* x, const float* k, const void* shortcut, void* y, int dtype, int64_t B, int64_t H,
           const int64_t* S, const int64_t* K, int64_t kbatch, unsigned periodic, void* workspace,
           size_t workspace_bytes, void* stream);
int nd_bwd(int nd, const void* g, const void* x, const float* k, const void* shortcut, void* gx, float* gk, float* gs,
           int dtype, int64_t B, int64_t H, const int64_t* S, const int64_t* K, int64_t kbatch, unsigned periodic,
           void* workspace, size_t workspace_bytes, int fwd_state, void* stream);

}  // namespace nsq
