// 2D / 3D non-causal "same" FFT convolution at the reference's own FFT sizes.
//
// nvsubquadratic/ops/fftconv.py:699-702 (2D) and :774-778 (3D) pad axis d to
// F_d = S_d + ceil(K_d / 2) points and transform with torch.fft, whose plans
// are mixed-radix.  The power-of-two plan of fftconv_nd_impl.h rounds F_d up
// to 2^m instead: the same results (no wrapped term reaches the cropped
// window either way), but at the Hyena shapes S_d = K_d = 2^a the reference's
// F_d = 3 * 2^(a-1) gives a spectrum 2.37x (3D) or 1.76x (2D) smaller than the
// power-of-two one.  This plan runs those sizes: every axis of length 48 or 96
// (192 on axis 0, and on both axes of a 2D plane), each the smallest such
// length >= S_d + ceil(K_d / 2), used when its spectrum is smaller than the
// power-of-two plan's.  Layout and passes are those of the power-of-two plan:
//   workspace block [F0][F1][FH], FH = F2/2 + 1 (2D: F1 = 1);
//   r3_plane_fwd : (3D) real transforms along axis 2 and complex ones along
//                  axis 1 of one (b, h, a0) plane in LDS;
//   r3_row_fwd   : (2D) real transforms along the last axis;
//   r3_col_fwd   : axis-0 forward transform (the filter);
//   r3_col_mul   : axis-0 forward, spectral product, inverse, crop;
//   r3_col_bwd   : axis-0 adjoint: P = G R conj(K), Q = R sum_b G conj(X),
//                  R the shift ramp that puts gx and gk at window 0;
//   r3_plane_inv : (3D) inverse along axis 1, crop, inverse real rows, epilogue;
//   r3_row_inv   : (2D) inverse real rows, crop, epilogue.
// The transforms are fft_mixed.h's radix-3-first Stockham passes.
#pragma once

#include "fft_mixed.h"
#include "fftconv_nd_impl.h"

namespace nsq {

// ---------------------------------------------------------------------------
// Plane passes (axes 1 and 2 of one plane in LDS).
// ---------------------------------------------------------------------------
template <int N2, int F1>
struct R3PlaneCfg {
  static constexpr int N = N2;             // packed row length F2 / 2
  static constexpr int FH = N2 + 1;        // spectrum bins per row
  static constexpr int RS = N2 + N2 / 16;  // LDS row stride (pad16 positions)
  static constexpr int T = 192;
  // rows per row tile: 64 for 48-point rows in a 96-row plane (a Hyena
  // volume's 64 valid rows in one tile), else a divisor of F1; the inverse
  // takes the rows past the last whole tile in one tile of MRB = F1 % MR rows,
  // so no tile reaches past the plane.
  static constexpr int MR = (N2 == 48 && F1 == 96) ? 64 : (F1 * N2 > 2304 ? 2304 / N2 : F1);
  static constexpr int MRB = F1 % MR;
  static constexpr int ROWR = 16;                 // largest power-of-two radix of the row passes
  static constexpr int COLR = F1 == 48 ? 16 : 8;  // ... of the column passes
  static constexpr int Q = F1 > 2 * N2 ? F1 : 2 * N2;  // roots staged in LDS: W_Q covers every pass and the real unpack
  static_assert(MR <= F1, "R3PlaneCfg: row tile");
};

// THIRD: len <= 2 F2 / 3 and n1 <= 2 F1 / 3, so the third input of every
// first-pass radix-3 butterfly (rows and columns) is zero padding.
template <int N2, int F1, int DT, bool AL, bool THIRD>
__global__ __launch_bounds__(192) void r3_plane_fwd_kernel(const typename Elem<DT>::T* __restrict__ src, int n0,
                                                           int n1, int len, float2* __restrict__ ws, int64_t spec,
                                                           const float2* __restrict__ tw) {
  using C = R3PlaneCfg<N2, F1>;
  constexpr int N = C::N, RS = C::RS, T = C::T, MR = C::MR;
  __shared__ float2 P[F1 * RS];
  __shared__ float2 twl[C::Q];
  const int64_t plane = blockIdx.x;  // bh * n0 + a0
  const int64_t xoff = plane * n1 * len;
  const auto tws = stage_roots<C::Q, T>(twl, tw);
  __syncthreads();
  // Axis 2: real transforms of the valid rows, unpacked in place to V (V[0]
  // = U[0] + i U[N], V[p] = U[p]); rows of a tile past n1 transform zeros.
  // A last tile that would pass the plane's end moves back and recomputes
  // rows already done (from the input, so with the same values).
  for (int rb = 0; rb < n1; rb += MR) {
    const int r0 = rb + MR <= F1 ? rb : F1 - MR;
    LdsTile<RS, true> rows{P + r0 * RS};
    auto ld = [&](int m, int n) -> float2 {
      const int a1 = r0 + m;
      const bool ok = a1 < n1;
      return load_pair_nb<DT, AL>(src + xoff + int64_t(ok ? a1 : 0) * len, 2 * int64_t(n), ok ? len : 0);
    };
    TailZeroLoad<3, 2, THIRD, decltype(ld)> ld1{ld};
    fft_mixed<N, false, MR, T, false, C::ROWR>(ld1, rows, rows, tws);
    const int ts = opaque_tid();
    constexpr int SLOTS = (MR * (N / 2) + T - 1) / T;
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int s = ts + i * T;
      if (s >= MR * (N / 2)) continue;
      const int m = s / (N / 2), p = s - m * (N / 2);
      const bool p0 = (p == 0);
      float2* z = P + (r0 + m) * RS;
      const int pb = pad16(p0 ? N / 2 : N - p);
      float2 A, Bc;
      real_unpack(p0, z[pad16(p)], z[pb], tws.template root<2 * N>(p), A, Bc);
      z[pad16(p)] = A;
      z[pb] = p0 ? Bc : cconj(Bc);
    }
    __syncthreads();
  }
  // Axis 1: complex transforms of the N packed columns; rows >= n1 are zero.
  LdsCols<RS> cols{P, 0};
  auto ldc = [&](int m, int n) -> float2 {
    const bool ok = n < n1;
    const float2 v = P[(ok ? n : 0) * RS + pad16(m)];
    return make_float2(ok ? v.x : 0.f, ok ? v.y : 0.f);
  };
  TailZeroLoad<3, 2, THIRD, decltype(ldc)> ldc1{ldc};
  fft_mixed<F1, false, N, T, true, C::COLR>(ldc1, cols, cols, tws);
  // Store [F1][FH]; column 0 separates into the DC (j = 0) and Nyquist (j = N) bins.
  float2* out = ws + (plane / n0) * spec + (plane % n0) * int64_t(F1) * C::FH;
  const int t = opaque_tid();
#pragma unroll 4
  for (int e = t; e < F1 * N; e += T) {
    const int k1 = e / N, j = e - k1 * N;
    const float2 v = P[k1 * RS + pad16(j)];
    if (j != 0) out[int64_t(k1) * C::FH + j] = v;
  }
  for (int k1 = t; k1 < F1; k1 += T) {
    const float2 v = P[k1 * RS];
    const float2 zc = cconj(P[(k1 ? F1 - k1 : 0) * RS]);
    out[int64_t(k1) * C::FH] = cscale(cadd(v, zc), 0.5f);
    out[int64_t(k1) * C::FH + N] = mul_neg_i(cscale(csub(v, zc), 0.5f));
  }
}

// The same forward pass with wave-local transforms: 256 threads, each wave
// owning MR / 4 rows of a row tile and N / 4 columns, so every pass
// synchronises on the wave's own in-order LDS operations (fft_mixed_wave) and
// a plane takes workgroup barriers only between its phases.
template <int N2, int F1, int DT, bool AL, bool THIRD>
__global__ __launch_bounds__(256) void r3_plane_fwd_w_kernel(const typename Elem<DT>::T* __restrict__ src, int n0,
                                                             int n1, int len, float2* __restrict__ ws, int64_t spec,
                                                             const float2* __restrict__ tw) {
  using C = R3PlaneCfg<N2, F1>;
  constexpr int N = C::N, RS = C::RS, T = 256, MR = C::MR, W = T / 64;
  constexpr int MRW = MR / W, NW = N / W;
  static_assert(MR % W == 0 && N % W == 0, "r3_plane_fwd_w_kernel: wave split");
  __shared__ float2 P[F1 * RS];
  __shared__ float2 twl[C::Q];
  const int64_t plane = blockIdx.x;  // bh * n0 + a0
  const int64_t xoff = plane * n1 * len;
  const auto tws = stage_roots<C::Q, T>(twl, tw);
  const int wv = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  __syncthreads();
  for (int rb = 0; rb < n1; rb += MR) {
    const int r0 = (rb + MR <= F1 ? rb : F1 - MR) + wv * MRW;  // the wave's rows of the tile
    LdsTile<RS, true> rows{P + r0 * RS};
    auto ld = [&](int m, int n) -> float2 {
      const int a1 = r0 + m;
      const bool ok = a1 < n1;
      return load_pair_nb<DT, AL>(src + xoff + int64_t(ok ? a1 : 0) * len, 2 * int64_t(n), ok ? len : 0);
    };
    TailZeroLoad<3, 2, THIRD, decltype(ld)> ld1{ld};
    fft_mixed_wave<N, false, MRW, false, C::ROWR>(ld1, rows, rows, tws);
    const int lane = opaque_tid() & 63;
    constexpr int SLOTS = (MRW * (N / 2) + 63) / 64;
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int s = lane + i * 64;
      if (s >= MRW * (N / 2)) continue;
      const int m = s / (N / 2), p = s - m * (N / 2);
      const bool p0 = (p == 0);
      float2* z = P + (r0 + m) * RS;
      const int pb = pad16(p0 ? N / 2 : N - p);
      float2 A, Bc;
      real_unpack(p0, z[pad16(p)], z[pb], tws.template root<2 * N>(p), A, Bc);
      z[pad16(p)] = A;
      z[pb] = p0 ? Bc : cconj(Bc);
    }
    __syncthreads();  // a last tile moved back overlaps rows of other waves
  }
  const int c0 = wv * NW;  // the wave's packed columns
  LdsCols<RS> cols{P, c0};
  auto ldc = [&](int m, int n) -> float2 {
    const bool ok = n < n1;
    const float2 v = P[(ok ? n : 0) * RS + pad16(c0 + m)];
    return make_float2(ok ? v.x : 0.f, ok ? v.y : 0.f);
  };
  TailZeroLoad<3, 2, THIRD, decltype(ldc)> ldc1{ldc};
  fft_mixed_wave<F1, false, NW, true, C::COLR>(ldc1, cols, cols, tws);
  __syncthreads();
  float2* out = ws + (plane / n0) * spec + (plane % n0) * int64_t(F1) * C::FH;
  const int t = opaque_tid();
#pragma unroll 4
  for (int e = t; e < F1 * N; e += T) {
    const int k1 = e / N, j = e - k1 * N;
    const float2 v = P[k1 * RS + pad16(j)];
    if (j != 0) out[int64_t(k1) * C::FH + j] = v;
  }
  for (int k1 = t; k1 < F1; k1 += T) {
    const float2 v = P[k1 * RS];
    const float2 zc = cconj(P[(k1 ? F1 - k1 : 0) * RS]);
    out[int64_t(k1) * C::FH] = cscale(cadd(v, zc), 0.5f);
    out[int64_t(k1) * C::FH + N] = mul_neg_i(cscale(csub(v, zc), 0.5f));
  }
}

// Inverse: plane [F1][FH] -> inverse along axis 1 keeping rows [off1, off1 +
// n1out) (moved to the front) -> inverse real rows, crop [off2, off2 + w2),
// epilogue (RowInvOut: ND_OUT_Y with shortcut, or ND_OUT_GK with the lag
// value gs).
template <int N2, int F1, int DT, int MODE, bool HAS_S>
__global__ __launch_bounds__(192) void r3_plane_inv_kernel(const float2* __restrict__ ws, int64_t spec, int n0,
                                                           int off1, int n1out, RowInvOut o,
                                                           const float2* __restrict__ tw) {
  using C = R3PlaneCfg<N2, F1>;
  using ET = typename Elem<DT>::T;
  constexpr int N = C::N, RS = C::RS, T = C::T, MR = C::MR;
  __shared__ float2 P[F1 * RS];
  const int64_t plane = blockIdx.x;  // bh * n0 + a0
  const int64_t bh = plane / n0;
  const int a0 = int(plane - bh * n0);
  const float2* in = ws + bh * spec + int64_t(a0) * F1 * C::FH;
  __shared__ float2 twl[C::Q];
  const auto tws = stage_roots<C::Q, T>(twl, tw);
  const int t = opaque_tid();
#pragma unroll 8
  for (int e = t; e < F1 * N; e += T) {
    const int k1 = e / N, j = e - k1 * N;
    P[k1 * RS + pad16(j)] = in[int64_t(k1) * C::FH + j];
  }
  __syncthreads();
  for (int k1 = t; k1 < F1; k1 += T) {  // pack DC + i Nyquist into column 0
    const float2 w = in[int64_t(k1) * C::FH + N];
    const float2 v = P[k1 * RS];
    P[k1 * RS] = make_float2(v.x - w.y, v.y + w.x);
  }
  __syncthreads();
  LdsCols<RS> cols{P, 0};
  auto stc = [&](int m, int k, float2 v) {
    const int r = k - off1;
    if (r >= 0 && r < n1out) P[r * RS + pad16(m)] = v;
  };
  fft_mixed<F1, true, N, T, true, C::COLR>(cols, cols, stc, tws);
  const ET* __restrict__ aux = (const ET*)o.aux;
  const int h = int(bh % o.H);
  const float sv = HAS_S ? Elem<DT>::round(Elem<DT>::load((const ET*)o.s, h)) : 0.f;
  const bool fast = MODE == ND_OUT_Y && (o.off2 & 1) == 0 && (o.w2 & 7) == 0 && o.w2 <= 2 * N &&
                    ((reinterpret_cast<uintptr_t>(o.out) | (HAS_S ? reinterpret_cast<uintptr_t>(o.aux) : 0)) & 15) == 0;
  // One tile of MRT rows from row r0: repack, inverse, epilogue.
  auto row_tile = [&](auto mrc, int r0) {
    constexpr int MRT = decltype(mrc)::value;
    constexpr int SLOTS = (MRT * (N / 2) + T - 1) / T;
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int s = t + i * T;
      if (s >= MRT * (N / 2)) continue;
      const int m = s / (N / 2), p = s - m * (N / 2);
      const bool p0 = (p == 0);
      float2* z = P + (r0 + m) * RS;
      const int pb = pad16(p0 ? N / 2 : N - p);
      const float2 b = z[pb];
      float2 zp, zq;
      real_repack(p0, z[pad16(p)], p0 ? b : cconj(b), tws.template root<2 * N>(p), zp, zq);
      z[pad16(p)] = zp;
      z[pb] = zq;
    }
    __syncthreads();
    LdsTile<RS, true> rows{P + r0 * RS};
    fft_mixed<N, true, MRT, T, false, C::ROWR>(rows, rows, rows, tws);
    const int nrows = (n1out - r0) < MRT ? (n1out - r0) : MRT;
    if constexpr (MODE == ND_OUT_Y) {
      if (fast) {
        // 8 consecutive kept samples per thread: four complex values from
        // LDS, one 16-byte shortcut load, one 16-byte store.
        const int cpr = o.w2 >> 3;
        const int64_t row0 = plane * n1out + r0;
        const RowBuf<DT, false> ab(aux + row0 * o.w2, HAS_S ? nrows * o.w2 : 0);
        const RowBuf<DT, true> ob((ET*)o.out + row0 * o.w2, nrows * o.w2);
        for (int ch = t; ch < nrows * cpr; ch += T) {
          const int m = ch / cpr, c8 = (ch - m * cpr) * 8;
          const int e0 = m * o.w2 + c8;
          Win8<DT, true> a{};
          if constexpr (HAS_S) a.load(ab, e0);
          const float2* zr = P + (r0 + m) * RS;
          const int nc = (c8 + o.off2) >> 1;
          float yv[8];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const float2 z = zr[pad16(nc + u)];
            yv[2 * u] = epilogue<DT>(z.x * o.scale, HAS_S, sv, a.at(2 * u));
            yv[2 * u + 1] = epilogue<DT>(z.y * o.scale, HAS_S, sv, a.at(2 * u + 1));
          }
          store8<DT, true>(ob, e0, yv);
        }
        __syncthreads();
        return;
      }
    }
    for (int e = t; e < nrows * o.w2; e += T) {
      const int m = e / o.w2, c = e - m * o.w2;
      const int sidx = c + o.off2;
      const float2 zz = P[(r0 + m) * RS + pad16(sidx >> 1)];
      const float v = ((sidx & 1) ? zz.y : zz.x) * o.scale;
      const int64_t idx = (plane * n1out + r0 + m) * o.w2 + c;
      if constexpr (MODE == ND_OUT_Y) {
        const float a = HAS_S ? Elem<DT>::load(aux, idx) : 0.f;
        Elem<DT>::store((ET*)o.out, idx, epilogue<DT>(v, HAS_S, sv, a));
      } else {
        ((float*)o.out)[idx] = v;
        if (o.gs && c == o.ga2 && a0 == o.ga0 && r0 + m == o.ga1) o.gs[bh] = v;
      }
    }
    __syncthreads();
  };
  for (int r0 = 0; r0 < n1out;) {  // in place, so tiles do not overlap: whole tiles, then MRB rows
    if (r0 + MR <= F1) {
      row_tile(std::integral_constant<int, MR>{}, r0);
      r0 += MR;
    } else {
      if constexpr (C::MRB > 0) row_tile(std::integral_constant<int, C::MRB>{}, r0);
      r0 += C::MRB > 0 ? C::MRB : F1;  // (MRB = 0: MR divides F1 and this branch is not reached)
    }
  }
}

// The same inverse with wave-local transforms (256 threads): each wave owns
// N / 4 packed columns, then a quarter of each row tile, so only the phase
// boundaries take workgroup barriers.
template <int N2, int F1, int DT, int MODE, bool HAS_S>
__global__ __launch_bounds__(256) void r3_plane_inv_w_kernel(const float2* __restrict__ ws, int64_t spec, int n0,
                                                             int off1, int n1out, RowInvOut o,
                                                             const float2* __restrict__ tw) {
  using C = R3PlaneCfg<N2, F1>;
  using ET = typename Elem<DT>::T;
  constexpr int N = C::N, RS = C::RS, T = 256, MR = C::MR, W = T / 64, NW = N / W;
  static_assert(MR % W == 0 && C::MRB % W == 0 && N % W == 0, "r3_plane_inv_w_kernel: wave split");
  __shared__ float2 P[F1 * RS];
  const int64_t plane = blockIdx.x;  // bh * n0 + a0
  const int64_t bh = plane / n0;
  const int a0 = int(plane - bh * n0);
  const float2* in = ws + bh * spec + int64_t(a0) * F1 * C::FH;
  __shared__ float2 twl[C::Q];
  const auto tws = stage_roots<C::Q, T>(twl, tw);
  const int t = opaque_tid();
  const int wv = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int lane = t & 63;
#pragma unroll 8
  for (int e = t; e < F1 * N; e += T) {
    const int k1 = e / N, j = e - k1 * N;
    P[k1 * RS + pad16(j)] = in[int64_t(k1) * C::FH + j];
  }
  __syncthreads();
  for (int k1 = t; k1 < F1; k1 += T) {  // pack DC + i Nyquist into column 0
    const float2 w = in[int64_t(k1) * C::FH + N];
    const float2 v = P[k1 * RS];
    P[k1 * RS] = make_float2(v.x - w.y, v.y + w.x);
  }
  __syncthreads();
  const int c0 = wv * NW;  // the wave's packed columns
  LdsCols<RS> cols{P, c0};
  auto stc = [&](int m, int k, float2 v) {
    const int r = k - off1;
    if (r >= 0 && r < n1out) P[r * RS + pad16(c0 + m)] = v;
  };
  fft_mixed_wave<F1, true, NW, true, C::COLR>(cols, cols, stc, tws);
  __syncthreads();
  const ET* __restrict__ aux = (const ET*)o.aux;
  const int h = int(bh % o.H);
  const float sv = HAS_S ? Elem<DT>::round(Elem<DT>::load((const ET*)o.s, h)) : 0.f;
  const bool fast = MODE == ND_OUT_Y && (o.off2 & 1) == 0 && (o.w2 & 7) == 0 && o.w2 <= 2 * N &&
                    ((reinterpret_cast<uintptr_t>(o.out) | (HAS_S ? reinterpret_cast<uintptr_t>(o.aux) : 0)) & 15) == 0;
  // The wave's MRT / W rows of a tile of MRT rows from row r0t: repack,
  // inverse, epilogue (tiles do not overlap: no barrier between them).
  auto row_tile = [&](auto mrc, int r0t) {
    constexpr int MRT = decltype(mrc)::value / W;
    const int r0 = r0t + wv * MRT;
    constexpr int SLOTS = (MRT * (N / 2) + 63) / 64;
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int s = lane + i * 64;
      if (s >= MRT * (N / 2)) continue;
      const int m = s / (N / 2), p = s - m * (N / 2);
      const bool p0 = (p == 0);
      float2* z = P + (r0 + m) * RS;
      const int pb = pad16(p0 ? N / 2 : N - p);
      const float2 b = z[pb];
      float2 zp, zq;
      real_repack(p0, z[pad16(p)], p0 ? b : cconj(b), tws.template root<2 * N>(p), zp, zq);
      z[pad16(p)] = zp;
      z[pb] = zq;
    }
    mixed_sync<true>();
    LdsTile<RS, true> rows{P + r0 * RS};
    fft_mixed_wave<N, true, MRT, false, C::ROWR>(rows, rows, rows, tws);
    const int nrows = (n1out - r0) < MRT ? ((n1out - r0) > 0 ? (n1out - r0) : 0) : MRT;
    if constexpr (MODE == ND_OUT_Y) {
      if (fast) {
        // 8 consecutive kept samples per thread: four complex values from
        // LDS, one 16-byte shortcut load, one 16-byte store.
        const int cpr = o.w2 >> 3;
        const int64_t row0 = plane * n1out + r0;
        const RowBuf<DT, false> ab(aux + row0 * o.w2, HAS_S ? nrows * o.w2 : 0);
        const RowBuf<DT, true> ob((ET*)o.out + row0 * o.w2, nrows * o.w2);
        for (int ch = lane; ch < nrows * cpr; ch += 64) {
          const int m = ch / cpr, c8 = (ch - m * cpr) * 8;
          const int e0 = m * o.w2 + c8;
          Win8<DT, true> a{};
          if constexpr (HAS_S) a.load(ab, e0);
          const float2* zr = P + (r0 + m) * RS;
          const int nc = (c8 + o.off2) >> 1;
          float yv[8];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const float2 z = zr[pad16(nc + u)];
            yv[2 * u] = epilogue<DT>(z.x * o.scale, HAS_S, sv, a.at(2 * u));
            yv[2 * u + 1] = epilogue<DT>(z.y * o.scale, HAS_S, sv, a.at(2 * u + 1));
          }
          store8<DT, true>(ob, e0, yv);
        }
        return;
      }
    }
    for (int e = lane; e < nrows * o.w2; e += 64) {
      const int m = e / o.w2, c = e - m * o.w2;
      const int sidx = c + o.off2;
      const float2 zz = P[(r0 + m) * RS + pad16(sidx >> 1)];
      const float v = ((sidx & 1) ? zz.y : zz.x) * o.scale;
      const int64_t idx = (plane * n1out + r0 + m) * o.w2 + c;
      if constexpr (MODE == ND_OUT_Y) {
        const float a = HAS_S ? Elem<DT>::load(aux, idx) : 0.f;
        Elem<DT>::store((ET*)o.out, idx, epilogue<DT>(v, HAS_S, sv, a));
      } else {
        ((float*)o.out)[idx] = v;
        if (o.gs && c == o.ga2 && a0 == o.ga0 && r0 + m == o.ga1) o.gs[bh] = v;
      }
    }
  };
  for (int r0 = 0; r0 < n1out;) {  // in place, so tiles do not overlap: whole tiles, then MRB rows
    if (r0 + MR <= F1) {
      row_tile(std::integral_constant<int, MR>{}, r0);
      r0 += MR;
    } else {
      if constexpr (C::MRB > 0) row_tile(std::integral_constant<int, C::MRB>{}, r0);
      r0 += C::MRB > 0 ? C::MRB : F1;  // (MRB = 0: MR divides F1 and this branch is not reached)
    }
  }
}

// ---------------------------------------------------------------------------
// Row passes of the 2D plan: real transforms along the last axis between the
// [rows][len] tensor (row r = (bh, a0), a0 < n0) and row a0 of spectrum block
// bh ([F0][FH], FH = F2/2 + 1).  M rows of N2 = F2/2 packed points per
// workgroup.
// ---------------------------------------------------------------------------
template <int N2>
struct R3RowCfg {
  static constexpr int N = N2;
  static constexpr int FH = N2 + 1;
  static constexpr int RS = N2 + N2 / 16;  // LDS row stride (pad16 positions)
  static constexpr int T = 192;
  static constexpr int M = 2304 / N2;      // 96, 48 or 24 rows
  static constexpr int MW = M / (T / 64);  // rows of each wave
  static constexpr int R = 16;             // largest power-of-two radix
  static constexpr int SLOTS = (M * (N2 / 2) + T - 1) / T;
};

// THIRD: len <= 2 F2 / 3 (the third input of each first-pass radix-3
// butterfly is zero padding).
template <int N2, int DT, bool AL, bool THIRD>
__global__ __launch_bounds__(192) void r3_row_fwd_kernel(const typename Elem<DT>::T* __restrict__ src, int nrows,
                                                         int n0, int len, float2* __restrict__ ws, int64_t spec,
                                                         const float2* __restrict__ tw) {
  using C = R3RowCfg<N2>;
  constexpr int N = C::N, RS = C::RS, T = C::T, M = C::M;
  __shared__ float2 P[M * RS];
  __shared__ float2 twl[2 * N];
  const auto tws = stage_roots<2 * N, T>(twl, tw);
  __syncthreads();
  const int r0 = int(blockIdx.x) * M;
  // each wave transforms its own M / 3 rows (fft_mixed_wave: no workgroup
  // barrier inside the transform)
  const int wv = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  LdsTile<RS, true> rows{P + wv * C::MW * RS};
  auto ld = [&](int m, int n) -> float2 {
    const int r = r0 + wv * C::MW + m;
    const bool ok = r < nrows;
    return load_pair_nb<DT, AL>(src + int64_t(ok ? r : 0) * len, 2 * int64_t(n), ok ? len : 0);
  };
  TailZeroLoad<3, 2, THIRD, decltype(ld)> ld1{ld};
  fft_mixed_wave<N, false, C::MW, false, C::R>(ld1, rows, rows, tws);
  __syncthreads();
  const int ts = opaque_tid();
#pragma unroll
  for (int i = 0; i < C::SLOTS; ++i) {
    const int s = ts + i * T;
    const int m = s / (N / 2), p = s - m * (N / 2);
    const int r = r0 + m;
    if (s >= M * (N / 2) || r >= nrows) continue;
    const bool p0 = (p == 0);
    const float2* z = P + m * RS;
    float2 A, Bc;
    real_unpack(p0, z[pad16(p)], z[pad16(p0 ? N / 2 : N - p)], tws.template root<2 * N>(p), A, Bc);
    const int bh = int(uint32_t(r) / uint32_t(n0)), a0 = r - bh * n0;
    float2* out = ws + int64_t(bh) * spec + int64_t(a0) * C::FH;
    if (p0) {
      out[0] = make_float2(A.x, 0.f);
      out[N] = make_float2(A.y, 0.f);
      out[N / 2] = Bc;
    } else {
      out[p] = A;
      out[N - p] = cconj(Bc);
    }
  }
}

// Inverse: rows r < nrows ((bh, a0), a0 < n0) of the spectrum -> inverse
// real transforms, window [off2, off2 + w2), epilogue (RowInvOut; output row
// r at r * w2; ND_OUT_GK: gs[bh] = the value at (ga0, ga2)).
template <int N2, int DT, int MODE, bool HAS_S>
__global__ __launch_bounds__(192) void r3_row_inv_kernel(const float2* __restrict__ ws, int nrows, int n0,
                                                         int64_t spec, RowInvOut o, const float2* __restrict__ tw) {
  using C = R3RowCfg<N2>;
  using ET = typename Elem<DT>::T;
  constexpr int N = C::N, RS = C::RS, T = C::T, M = C::M;
  __shared__ float2 P[M * RS];
  __shared__ float2 twl[2 * N];
  const auto tws = stage_roots<2 * N, T>(twl, tw);
  __syncthreads();
  const int r0 = int(blockIdx.x) * M;
  const int t = opaque_tid();
#pragma unroll
  for (int i = 0; i < C::SLOTS; ++i) {
    const int s = t + i * T;
    if (s >= M * (N / 2)) continue;
    const int m = s / (N / 2), p = s - m * (N / 2);
    const int r = r0 + m;
    const bool rok = r < nrows;
    const int rr = rok ? r : 0;
    const int bh = int(uint32_t(rr) / uint32_t(n0)), a0 = rr - bh * n0;
    const float2* in = ws + int64_t(bh) * spec + int64_t(a0) * C::FH;
    const bool p0 = (p == 0);
    const float2 u0 = in[p0 ? 0 : p];
    const float2 u1 = in[p0 ? N : N - p];
    const float2 u2 = p0 ? in[N / 2] : make_float2(0.f, 0.f);  // slot 0 only
    float2 A = p0 ? make_float2(u0.x, u1.x) : u0;
    float2 Bc = p0 ? u2 : cconj(u1);
    A = make_float2(rok ? A.x : 0.f, rok ? A.y : 0.f);
    Bc = make_float2(rok ? Bc.x : 0.f, rok ? Bc.y : 0.f);
    float2 zp, zq;
    real_repack(p0, A, Bc, tws.template root<2 * N>(p), zp, zq);
    float2* z = P + m * RS;
    z[pad16(p)] = zp;
    z[pad16(p0 ? N / 2 : N - p)] = zq;
  }
  __syncthreads();
  const int wv = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  LdsTile<RS, true> rows{P + wv * C::MW * RS};
  fft_mixed_wave<N, true, C::MW, false, C::R>(rows, rows, rows, tws);
  __syncthreads();
  const ET* __restrict__ aux = (const ET*)o.aux;
  const int nr = (nrows - r0) < M ? (nrows - r0) : M;
  const bool fast = MODE == ND_OUT_Y && (o.off2 & 1) == 0 && (o.w2 & 7) == 0 && o.w2 <= 2 * N &&
                    ((reinterpret_cast<uintptr_t>(o.out) | (HAS_S ? reinterpret_cast<uintptr_t>(o.aux) : 0)) & 15) == 0;
  if constexpr (MODE == ND_OUT_Y) {
    if (fast) {
      // 8 consecutive kept samples per thread: four complex values from LDS,
      // one 16-byte shortcut load, one 16-byte store.
      const int cpr = o.w2 >> 3;
      const int64_t tb = int64_t(r0) * o.w2;
      const RowBuf<DT, false> ab(aux + tb, HAS_S ? nr * o.w2 : 0);
      const RowBuf<DT, true> ob((ET*)o.out + tb, nr * o.w2);
      for (int ch = t; ch < nr * cpr; ch += T) {
        const int m = ch / cpr, c8 = (ch - m * cpr) * 8;
        const int e0 = m * o.w2 + c8;
        Win8<DT, true> a{};
        if constexpr (HAS_S) a.load(ab, e0);
        const int bh = int(uint32_t(r0 + m) / uint32_t(n0));
        const float sv = HAS_S ? Elem<DT>::round(Elem<DT>::load((const ET*)o.s, bh % o.H)) : 0.f;
        const float2* zr = P + m * RS;
        const int nc = (c8 + o.off2) >> 1;
        float yv[8];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float2 z = zr[pad16(nc + u)];
          yv[2 * u] = epilogue<DT>(z.x * o.scale, HAS_S, sv, a.at(2 * u));
          yv[2 * u + 1] = epilogue<DT>(z.y * o.scale, HAS_S, sv, a.at(2 * u + 1));
        }
        store8<DT, true>(ob, e0, yv);
      }
      return;
    }
  }
  for (int e = t; e < nr * o.w2; e += T) {
    const int m = e / o.w2, c = e - m * o.w2;
    const int sidx = c + o.off2;
    const float2 zz = P[m * RS + pad16(sidx >> 1)];
    const float v = ((sidx & 1) ? zz.y : zz.x) * o.scale;
    const int r = r0 + m;
    const int bh = int(uint32_t(r) / uint32_t(n0));
    const int64_t idx = int64_t(r) * o.w2 + c;
    if constexpr (MODE == ND_OUT_Y) {
      const float sv = HAS_S ? Elem<DT>::round(Elem<DT>::load((const ET*)o.s, bh % o.H)) : 0.f;
      const float a = HAS_S ? Elem<DT>::load(aux, idx) : 0.f;
      Elem<DT>::store((ET*)o.out, idx, epilogue<DT>(v, HAS_S, sv, a));
    } else {
      ((float*)o.out)[idx] = v;
      if (o.gs && c == o.ga2 && r - bh * n0 == o.ga0) o.gs[bh] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Axis-0 column passes: M columns of a block per workgroup (lanes on
// consecutive inner indices, so each row segment is one coalesced access),
// transposed tile (element n of column m at m * S + n, S odd).
// ---------------------------------------------------------------------------
template <int F0>
struct R3ColCfg {
  static constexpr int M = F0 == 48 ? 32 : 16;
  static constexpr int S = F0 + 1;
  static constexpr int T = F0 == 192 ? 256 : 128;  // 12 points per thread (24 for F0 = 192 at 128 threads: 256 VGPRs)
  static constexpr int RMAX = F0 == 48 ? 16 : 8;
  static constexpr int PT = M * F0 / T;  // spectrum elements per thread (one column, stride T / M)
  // Occupancy target of the adjoint: 3 waves/SIMD (<= 168 VGPRs), which costs
  // 13 spilled registers at F0 = 96 and runs 801 -> 749 us at config 5
  // (measured).
  static constexpr int BWD_WAVES = 3;
  static_assert(T % M == 0 && (M * F0) % T == 0, "R3ColCfg: tile");
};

// Forward transform of the first in_cnt rows (the rest zero), all F0 outputs
// written; grid = (blocks, ceil(inner / M)).  THIRD: in_cnt <= 2 F0 / 3.
template <int F0, bool THIRD>
__global__ __launch_bounds__(R3ColCfg<F0>::T) void r3_col_fwd_kernel(float2* __restrict__ ws, ColGeom cg, int in_cnt,
                                                         const float2* __restrict__ tw) {
  using C = R3ColCfg<F0>;
  __shared__ float2 lds[C::M * C::S];
  __shared__ float2 twl[F0];
  const auto tws = stage_roots<F0, C::T>(twl, tw);
  __syncthreads();
  const ColBuf cb(ws + int64_t(blockIdx.x) * cg.spec, cg);
  const int j0 = int(blockIdx.y) * C::M;
  auto ld = [&](int m, int n) -> float2 { return cb.load(n, j0 + m, j0 + m < cg.inner_count && n < in_cnt); };
  auto st = [&](int m, int k, float2 v) { cb.store(k, j0 + m, j0 + m < cg.inner_count, v); };
  TailZeroLoad<3, 2, THIRD, decltype(ld)> ld1{ld};
  LdsTile<C::S, false> tile{lds};
  fft_mixed<F0, false, C::M, C::T, true, C::RMAX>(ld1, tile, st, tws);
}

// The same transform written transposed, out[blk][j][k] (a column's F0
// frequencies contiguous), through the LDS tile so the stores are coalesced:
// the filter spectrum of the one-kernel image forward.
template <int F0, bool THIRD>
__global__ __launch_bounds__(R3ColCfg<F0>::T) void r3_col_fwd_t_kernel(const float2* __restrict__ ws, ColGeom cg,
                                                           int in_cnt, float2* __restrict__ out,
                                                           const float2* __restrict__ tw) {
  using C = R3ColCfg<F0>;
  __shared__ float2 lds[C::M * C::S];
  __shared__ float2 twl[F0];
  const auto tws = stage_roots<F0, C::T>(twl, tw);
  __syncthreads();
  const ColBuf cb(ws + int64_t(blockIdx.x) * cg.spec, cg);
  const int j0 = int(blockIdx.y) * C::M;
  auto ld = [&](int m, int n) -> float2 { return cb.load(n, j0 + m, j0 + m < cg.inner_count && n < in_cnt); };
  TailZeroLoad<3, 2, THIRD, decltype(ld)> ld1{ld};
  LdsTile<C::S, false> tile{lds};
  fft_mixed<F0, false, C::M, C::T, true, C::RMAX>(ld1, tile, tile, tws);
  float2* ob = out + (int64_t(blockIdx.x) * cg.inner_count + j0) * F0;
  const int nm = min(C::M, cg.inner_count - j0);
  for (int e = int(threadIdx.x); e < nm * F0; e += C::T) {
    const int m = e / F0, k = e - m * F0;
    ob[e] = *tile.at(m, k);
  }
}

// Forward conv along axis 0: FFT(x column) * Khat -> IFFT -> window [c0, c0 +
// S0) to rows [0, S0), from wsx to wsy (the same buffer for an in-place
// product).  Shared filter (kfilm = 0): grid.x = H * bsplit, a workgroup
// loops over its share of the batch (its filter columns are read once);
// FiLM: grid.x = B*H.  grid.y = column blocks.  THIRD: S0 <= 2 F0 / 3.
template <int F0, bool THIRD>
__global__ __launch_bounds__(R3ColCfg<F0>::T) void r3_col_mul_kernel(const float2* wsx, float2* wsy,
                                                         const float2* __restrict__ wsk, ColGeom cg, int B, int H,
                                                         int kfilm, int S0, int c0, int bsplit,
                                                         const float2* __restrict__ tw) {
  using C = R3ColCfg<F0>;
  __shared__ float2 lds[C::M * C::S];
  __shared__ float2 twl[F0];
  const auto tws = stage_roots<F0, C::T>(twl, tw);
  __syncthreads();
  const int64_t hk = blockIdx.x / bsplit;
  const int part = int(blockIdx.x % bsplit);
  const ColBuf kb(wsk + hk * cg.spec, cg);
  const int j0 = int(blockIdx.y) * C::M;
  const int tp = opaque_tid();
  const int m = tp % C::M, kfirst = tp / C::M;
  const bool jok = j0 + m < cg.inner_count;
  float2 kv[C::PT];
#pragma unroll
  for (int it = 0; it < C::PT; ++it) kv[it] = kb.load(kfirst + it * (C::T / C::M), j0 + m, jok);
  const int nb = kfilm ? 1 : B;
  const int b_begin = part * nb / bsplit, b_end = (part + 1) * nb / bsplit;
  LdsTile<C::S, false> tile{lds};
  for (int bi = b_begin; bi < b_end; ++bi) {
    const int64_t blk = (kfilm ? hk : int64_t(bi) * H + hk) * cg.spec;
    const ColBuf in(wsx + blk, cg);
    const ColBuf out(wsy + blk, cg);
    auto ld = [&](int mm, int n) -> float2 { return in.load(n, j0 + mm, j0 + mm < cg.inner_count && n < S0); };
    TailZeroLoad<3, 2, THIRD, decltype(ld)> ld1{ld};
    fft_mixed<F0, false, C::M, C::T, true, C::RMAX>(ld1, tile, tile, tws);
#pragma unroll
    for (int it = 0; it < C::PT; ++it) {
      float2& z = lds[m * C::S + kfirst + it * (C::T / C::M)];
      z = cmul(z, kv[it]);
    }
    __syncthreads();
    auto st = [&](int mm, int k, float2 v) {
      const int e = k - c0;
      out.store(e, j0 + mm, j0 + mm < cg.inner_count && uint32_t(e) < uint32_t(S0), v);
    };
    fft_mixed<F0, true, C::M, C::T, true, C::RMAX>(tile, tile, st, tws);
  }
}

// Shift ramp of the adjoint: R = W_F0^{c0 k0} W_F1^{c1 k1} W_F2^{c2 k2} at
// spectrum position (k0, j), (k1, k2) = (j / FH, j % FH).
struct R3Ramp {
  int c0, c1, c2;
  int F1, F2, FH;
};

__device__ __forceinline__ float2 r3_ramp_inner(const R3Ramp& rp, const TwAny& ta, int j) {
  const int k1 = j / rp.FH, k2 = j - k1 * rp.FH;
  return cmul(ta.root_rt(rp.F1, (rp.c1 * k1) % rp.F1), ta.root_rt(rp.F2, (rp.c2 * k2) % rp.F2));
}

// Adjoint along axis 0.  Shared kernel (kfilm = 0): grid.x = H, loops over
// the batch; FiLM: grid.x = B*H.  P = G R conj(K) (gx pre-image, window
// [0, S0)) is written over G in wsg; Q = R sum_b G conj(X) (gk pre-image,
// window [0, K0)) goes to block z * qsplit + hk of wsq.  grid.z > 1: the
// batch is split across workgroups and the partial Q blocks are summed by
// nd_q_reduce_kernel.  THIRD: S0 <= 2 F0 / 3.
template <int F0, bool THIRD>
__global__ __launch_bounds__(R3ColCfg<F0>::T)
__attribute__((amdgpu_waves_per_eu(R3ColCfg<F0>::BWD_WAVES))) void r3_col_bwd_kernel(float2* __restrict__ wsg, const float2* __restrict__ wsx,
                                                         const float2* __restrict__ wsk, float2* __restrict__ wsq,
                                                         ColGeom cg, int B, int H, int kfilm, int S0, int K0,
                                                         R3Ramp rp, int64_t qsplit, const float2* __restrict__ tw) {
  using C = R3ColCfg<F0>;
  __shared__ float2 ldsG[C::M * C::S];
  __shared__ float2 ldsX[C::M * C::S];  // X of the current image; at the end, Q
  __shared__ float2 twl[F0];
  const auto tws = stage_roots<F0, C::T>(twl, tw);
  __syncthreads();
  const int64_t hk = blockIdx.x;
  const int j0 = int(blockIdx.y) * C::M;
  const ColBuf kb(wsk + hk * cg.spec, cg);
  const int tp = opaque_tid();
  const int m = tp % C::M, kfirst = tp / C::M;
  const int j = j0 + m;
  const bool jok = j < cg.inner_count;
  const TwAny ta(tw);
  const float2 r12 = r3_ramp_inner(rp, ta, jok ? j : 0);
  // R conj(K) of this thread's spectrum elements, and the running sum of G conj(X)
  float2 kr[C::PT], q[C::PT];
#pragma unroll
  for (int it = 0; it < C::PT; ++it) {
    const int k = kfirst + it * (C::T / C::M);
    const float2 kv = kb.load(k, j, jok);
    kr[it] = cmulc(cmul(r12, tws.template root<F0>((rp.c0 * k) % F0)), kv);
    q[it] = make_float2(0.f, 0.f);
  }
  const int nb = kfilm ? 1 : B;
  const int nz = int(gridDim.z), z = int(blockIdx.z);
  LdsTile<C::S, false> tG{ldsG};
  LdsTile<C::S, false> tX{ldsX};
  for (int bi = z * nb / nz; bi < (z + 1) * nb / nz; ++bi) {
    const int64_t bh = kfilm ? hk : (int64_t(bi) * H + hk);
    const ColBuf gb(wsg + bh * cg.spec, cg);
    const ColBuf xb(wsx + bh * cg.spec, cg);
    auto ldg = [&](int mm, int n) -> float2 { return gb.load(n, j0 + mm, j0 + mm < cg.inner_count && n < S0); };
    auto ldx = [&](int mm, int n) -> float2 { return xb.load(n, j0 + mm, j0 + mm < cg.inner_count && n < S0); };
    TailZeroLoad<3, 2, THIRD, decltype(ldg)> ldg1{ldg};
    TailZeroLoad<3, 2, THIRD, decltype(ldx)> ldx1{ldx};
    fft_mixed<F0, false, C::M, C::T, true, C::RMAX>(ldg1, tG, tG, tws);
    fft_mixed<F0, false, C::M, C::T, true, C::RMAX>(ldx1, tX, tX, tws);
#pragma unroll
    for (int it = 0; it < C::PT; ++it) {
      const int a = m * C::S + kfirst + it * (C::T / C::M);
      const float2 g = ldsG[a];
      q[it] = cadd(q[it], cmulc(g, ldsX[a]));
      ldsG[a] = cmul(g, kr[it]);
    }
    __syncthreads();
    auto st = [&](int mm, int k, float2 v) { gb.store(k, j0 + mm, j0 + mm < cg.inner_count && k < S0, v); };
    fft_mixed<F0, true, C::M, C::T, true, C::RMAX>(tG, tG, st, tws);  // ends with a barrier: ldsX is free
  }
#pragma unroll
  for (int it = 0; it < C::PT; ++it) {
    const int k = kfirst + it * (C::T / C::M);
    ldsX[m * C::S + k] = cmul(q[it], cmul(r12, tws.template root<F0>((rp.c0 * k) % F0)));
  }
  __syncthreads();
  const ColBuf qb(wsq + (z * qsplit + hk) * cg.spec, cg);
  auto stq = [&](int mm, int k, float2 v) { qb.store(k, j0 + mm, j0 + mm < cg.inner_count && k < K0, v); };
  fft_mixed<F0, true, C::M, C::T, true, C::RMAX>(tX, tX, stq, tws);
}

}  // namespace nsq
