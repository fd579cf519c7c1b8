// Causal 1D FFT convolution (forward and backward) for gfx950.
//
// Semantics: nvsubquadratic/ops/fftconv.py:546-600 (causal_fftconv1d_fp32_bhl)
// with the wrapper epilogue of nvsubquadratic/ops/fftconv_custom.py:307-335.
//
// Two execution plans, chosen by the FFT length F (a power of two, real):
//
//  * fused  (F <= 16384): one workgroup owns M channels.  It transforms the
//    filter once (spectrum kept in registers, slot-owned by each thread), then
//    for each batch row: real FFT of x in LDS -> spectral product -> inverse
//    FFT -> crop/cast/shortcut epilogue straight to HBM.  HBM traffic is the
//    algorithmic minimum (x, k read once; y written once).
//  * 4-step (2^15 <= F <= 2^24): the packed complex length N = F/2 is split as
//    N = N1 x N2 (Cooley-Tukey).  Three kernels:
//      col_fwd  : length-N1 DFTs down the columns of each signal (x, k, g),
//                 times the twiddle W_N^{n2 k1}, to a workspace;
//      row      : length-N2 DFTs along rows k1 and N1-k1 (the rows that hold
//                 the Hermitian partners k and N-k), real-spectrum unpack,
//                 spectral product / correlation, repack, inverse row DFT,
//                 written back in place;
//      col_inv  : times W_N^{-n2 k1} as loaded, inverse length-N1 DFTs down
//                 the columns, crop and epilogue.
//
// Real signals of length F are packed as z[n] = u[2n] + i u[2n+1] (N = F/2
// complex points); see real_unpack/real_repack in fft_core.h.
#pragma once

#include <cstdlib>

#include "fft_core.h"
#include "gate.h"

namespace nsq {


// ===========================================================================
// Plan selection
// ===========================================================================
struct Plan1D {
  int logF;   // real FFT length 2^logF
  int logN;   // packed complex length, logF - 1
  bool fold;  // K > L+1: the reference's FFT length 2L wraps (fused plan: full[n + 2L] folded into y[n];
              // 4-step plan: a copy of x, or of g in the backward, at the wrap offset; see fold_rows_kernel)
  bool fused;
  int logN1, logN2;  // 4-step split (fused == false)
};

// 4-step split N = N1 x N2: columns of N1 <= 256 points (two LDS passes) and
// rows of N2 <= 4096 points; N1 grows beyond 256 only when N2 would exceed 4096,
// up to 2048 (a column tile of 8 x 2048 points is 131 KB of LDS and 1024
// threads): N <= 2048 x 4096 = 2^23.
__host__ __device__ constexpr int split_log_n1(int logN) {
  return (logN - 12 > ((logN / 2) < 8 ? (logN / 2) : 8)) ? (logN - 12) : ((logN / 2) < 8 ? (logN / 2) : 8);
}
constexpr int kMaxLogN = 23;

inline bool make_plan(int64_t L, int64_t K, Plan1D& p) {
  if (L < 1 || K < 1 || K > 2 * L) return false;
  p.fold = K > L + 1;
  int64_t need = p.fold ? 3 * L : L + K - 1;
  int logF = ilog2_ceil(need);
  if (logF < 4) logF = 4;
  p.logF = logF;
  p.logN = logF - 1;
  p.fused = p.logN <= 13;
  if (!p.fused) {
    if (p.logN > kMaxLogN) return false;
    p.logN1 = split_log_n1(p.logN);
    p.logN2 = p.logN - p.logN1;
  } else {
    p.logN1 = p.logN2 = 0;
  }
  return true;
}

// ===========================================================================
// Fused plan
// ===========================================================================
template <int LOGN>
struct FusedCfg {
  static constexpr int N = 1 << LOGN;
  static constexpr int M = LOGN >= 11 ? 1 : (2048 >> LOGN);  // channels per workgroup
  static constexpr int TILE = M * N;
  static constexpr int SP = Padded<N>::SIZE;                   // padded LDS stride per transform
  static constexpr int TILE_P = M * SP;                        // LDS elements of a tile
  static constexpr int T = TILE / 16;                          // threads
  static constexpr int E = 16;                                 // points per thread
  static constexpr int SLOTS = E / 2;                          // spectral slots per thread
};

// Slot s of the tile -> (transform m, slot p within the transform).
template <int LOGN>
__device__ __forceinline__ void slot_of(int s, int& m, int& p) {
  m = s >> (LOGN - 1);
  p = s & ((1 << (LOGN - 1)) - 1);
}

// Reads the packed real spectrum of transform m / slot p out of `z` (natural
// order, stride N per transform) in slot form.
template <int LOGN>
__device__ __forceinline__ void lds_unpack(const float2* z, int m, int p, const float2* __restrict__ tw,
                                           float2& A, float2& Bc) {
  constexpr int N = 1 << LOGN;
  const float2* zz = z + m * Padded<N>::SIZE;
  const bool s0 = (p == 0);
  float2 zp = zz[pad16(p)];
  float2 zq = zz[pad16(s0 ? N / 2 : N - p)];
  real_unpack(s0, zp, zq, root<LOGN + 1>(tw, p), A, Bc);  // W^0 = 1 for slot 0
}

template <int LOGN>
__device__ __forceinline__ void lds_repack(float2* z, int m, int p, const float2* __restrict__ tw, float2 A,
                                           float2 Bc) {
  constexpr int N = 1 << LOGN;
  float2* zz = z + m * Padded<N>::SIZE;
  const bool s0 = (p == 0);
  float2 zp, zq;
  real_repack(s0, A, Bc, root<LOGN + 1>(tw, p), zp, zq);
  zz[pad16(p)] = zp;
  zz[pad16(s0 ? N / 2 : N - p)] = zq;
}

// Shift ramp of the circular conv on one spectral slot (slot form: see
// real_unpack).  The real spectrum U[f], f in [0, N] (F = 2N), is multiplied by
// rho(f) = e^{+2 pi i c f / F} = conj(W_F^{c f}):
//   slot p > 0: A = U[p] -> A * conj(W^{cp});  Bc = conj(U[N-p]) -> Bc * W^{c(N-p)};
//   slot 0:     A = (U[0], U[N]) -> (U[0], (-1)^c U[N]);  Bc = U[N/2] -> Bc * conj(W^{cN/2}).
template <int LOGN>
__device__ __forceinline__ void circ_ramp(int p, int c, const float2* __restrict__ tw, float2& A, float2& Bc) {
  constexpr int N = 1 << LOGN, F = 2 * N;
  const TwTable tt(tw);
  const bool s0 = p == 0;
  const float2 wa = tt.load(F, (c * p) & (F - 1));
  const float2 wb = tt.load(F, (c * (s0 ? N / 2 : N - p)) & (F - 1));
  const float2 a = cmulc(A, wa);
  const float2 b = cmul(Bc, wb);
  const float2 b0 = cmulc(Bc, wb);
  A.x = s0 ? A.x : a.x;
  A.y = s0 ? ((c & 1) ? -A.y : A.y) : a.y;
  Bc.x = s0 ? b0.x : b.x;
  Bc.y = s0 ? b0.y : b.y;
}

// Filter spectrum of channels h0..h0+M-1 into per-thread slot registers.
// `lds` must hold a tile; leaves it free (ends with a barrier).  CIRC: the
// spectrum is multiplied by the ramp e^{+2 pi i c f / F} (F = 2N, the real
// FFT length), which rolls the circular conv's output by -c (see circ_ramp).
template <int LOGN, bool CIRC = false>
__device__ __forceinline__ void filter_spectrum(float2* lds, const float* __restrict__ k, int h0, int H, int K,
                                                const float2* __restrict__ tw, float2* hA, float2* hB, int c = 0) {
  using C = FusedCfg<LOGN>;
  auto ld = [&](int m, int n) -> float2 {
    const int h = h0 + m;
    if (h >= H) return make_float2(0.f, 0.f);
    return load_pair<NSQ_DTYPE_F32>(k + int64_t(h) * K, 2 * int64_t(n), K);
  };
  LdsTile<C::SP, true> st{lds};
  fft<LOGN, false, C::M, C::T, C::SP>(lds, ld, st, tw);
#pragma unroll
  for (int i = 0; i < C::SLOTS; ++i) {
    NSQ_SLOT_FENCE();
    int m, p;
    slot_of<LOGN>(opaque_tid() + i * C::T, m, p);
    lds_unpack<LOGN>(lds, m, p, tw, hA[i], hB[i]);
    if constexpr (CIRC) circ_ramp<LOGN>(p, c, tw, hA[i], hB[i]);
  }
  __syncthreads();
}

// Forward, fused plan.  grid = (ceil(H/M), nb_split); each workgroup handles
// batch rows [b0, b0 + b_per_wg).  CIRC: circular conv at FFT length 2N = L
// (no padding, no crop) rolled by -c through the filter ramp; a period L < 16
// runs at length 16 on the periodic extension of x (sample i read at i & wm,
// wm = L - 1; -1 otherwise).  kfilm: the filter is per image ([B, H, K]); the
// launch then gives one image per workgroup (b_per_wg = 1).  GATE (Hyena
// gates, gate.h): x is the query q; the transform reads z = q act1(k) and the
// epilogue writes y = y1 act2(v), y1 = conv(z) + s z (kept in ga.y1 if given).
template <int LOGN, int DT, bool FOLD, bool CIRC = false, bool GATE = false>
__global__ __launch_bounds__(FusedCfg<LOGN>::T) void fused_fwd_kernel(
    const typename Elem<DT>::T* __restrict__ x, const float* __restrict__ k,
    const typename Elem<DT>::T* __restrict__ s, typename Elem<DT>::T* __restrict__ y, int B, int H, int L,
    int K, int b_per_wg, const float2* __restrict__ tw, int c, int kfilm, int wm, GateArgs ga) {
  using ET = typename Elem<DT>::T;
  using C = FusedCfg<LOGN>;
  __shared__ float2 lds[C::TILE_P];
  const int h0 = blockIdx.x * C::M;
  const int b0 = blockIdx.y * b_per_wg;
  const int b1 = min(B, b0 + b_per_wg);

  float2 hA[C::SLOTS], hB[C::SLOTS];
  filter_spectrum<LOGN, CIRC>(lds, kfilm ? k + int64_t(b0) * H * K : k, h0, H, K, tw, hA, hB, c);

  const float scale = 1.f / float(C::N);
  for (int b = b0; b < b1; ++b) {
    auto ld = [&](int m, int n) -> float2 {
      const int h = h0 + m;
      if (h >= H) return make_float2(0.f, 0.f);
      const int64_t row = (int64_t(b) * H + h) * L, i = (2 * int64_t(n)) & wm;
      const float2 q = load_pair<DT>(x + row, i, L);
      if constexpr (GATE) {
        const float2 kk = load_pair<DT>((const ET*)ga.kg + row, i, L);
        return make_float2(gate1<DT>(ga.act1, q.x, kk.x), gate1<DT>(ga.act1, q.y, kk.y));
      }
      return q;
    };
    LdsTile<C::SP, true> st{lds};
    fft<LOGN, false, C::M, C::T, C::SP>(lds, ld, st, tw);
#pragma unroll
    for (int i = 0; i < C::SLOTS; ++i) {
    NSQ_SLOT_FENCE();
      int m, p;
      slot_of<LOGN>(opaque_tid() + i * C::T, m, p);
      float2 A, Bc;
      lds_unpack<LOGN>(lds, m, p, tw, A, Bc);
      A = slot_mul(p == 0, A, hA[i]);
      Bc = cmul(Bc, hB[i]);
      lds_repack<LOGN>(lds, m, p, tw, A, Bc);
    }
    __syncthreads();

    auto epi = [&](int m, int n, float2 v) {
      const int h = h0 + m;
      if (h >= H) return;
      const int64_t row = (int64_t(b) * H + h) * L;
      const float sv = s ? Elem<DT>::round(Elem<DT>::load(s, h)) : 0.f;
      const int64_t i0 = 2 * int64_t(n);
      auto out = [&](int64_t i, float conv) {
        if constexpr (GATE) {
          const float zi = s ? gate1<DT>(ga.act1, Elem<DT>::load(x, row + i), Elem<DT>::load((const ET*)ga.kg, row + i))
                             : 0.f;
          const float y1 = epilogue<DT>(conv, s != nullptr, sv, zi);
          if (ga.y1) Elem<DT>::store((ET*)ga.y1, row + i, y1);
          Elem<DT>::store(y, row + i, y1 * Elem<DT>::round(gate_act(ga.act2, Elem<DT>::load((const ET*)ga.v, row + i))));
        } else {
          Elem<DT>::store(y, row + i, epilogue<DT>(conv, s != nullptr, sv, s ? Elem<DT>::load(x, row + i) : 0.f));
        }
      };
      if (i0 < L) out(i0, v.x * scale);
      if (i0 + 1 < L) out(i0 + 1, v.y * scale);
    };
    if constexpr (!FOLD) {
      LdsTile<C::SP, true> ldl{lds};
      fft<LOGN, true, C::M, C::T, C::SP>(lds, ldl, epi, tw);
    } else {
      fft_lds<LOGN, true, C::M, C::T, C::SP>(lds, tw);
      // y[j] = full[j] + full[j + 2L]; in packed units index n and n + L.
      for (int e = threadIdx.x; e < C::TILE; e += C::T) {
        const int m = e >> LOGN, n = e & (C::N - 1);
        if (2 * n >= L) continue;
        float2 v = lds[m * C::SP + pad16(n)];
        if (n + L < C::N) v = cadd(v, lds[m * C::SP + pad16(n + L)]);
        epi(m, n, v);
      }
      __syncthreads();
    }
  }
}

// Forward, fused plan, for grids too small to fill the GPU (M == 1 lengths,
// few (channel, batch row) pairs): fused_fwd_kernel then runs one workgroup
// of N/16 threads per row, one wave per SIMD, and transforms the filter and
// the row one after the other.  Here a workgroup of 2 N/2^LOGRMAX threads
// owns one (channel h = blockIdx.x, batch row b = blockIdx.y) and holds a
// two-transform tile: transform 0 is the filter, transform 1 the row, both
// transformed at once (the first half of the threads load the filter, the
// rest the row).  The product reads both spectra from LDS slot by slot and
// leaves the result in transform 1; the inverse transform runs over the whole
// tile and the epilogue keeps transform 1.  With LOGRMAX = 4 the arithmetic
// per element is that of fused_fwd_kernel (bitwise equal outputs); LOGRMAX =
// 3 runs radix-8 passes at 8 points per thread (agreement to fp32 rounding).
// Plain causal conv (no fold, ramp or gates); kfilm: the filter row is image
// b's.
template <int LOGN, int DT, int LOGRMAX = 4>
__global__ __launch_bounds__(2 * (FusedCfg<LOGN>::N >> LOGRMAX)) void fused_fwd_pair_kernel(
    const typename Elem<DT>::T* __restrict__ x, const float* __restrict__ k,
    const typename Elem<DT>::T* __restrict__ s, typename Elem<DT>::T* __restrict__ y, int H, int L, int K,
    const float2* __restrict__ tw, int kfilm) {
  using C = FusedCfg<LOGN>;
  static_assert(C::M == 1, "fused_fwd_pair_kernel: one transform per channel");
  constexpr int T = 2 * (C::N >> LOGRMAX), SL = C::N / 2 / T;  // threads; product slots per thread
  static_assert(SL >= 1 && (C::N / 2) % T == 0, "fused_fwd_pair_kernel: slot split");
  __shared__ float2 lds[2 * C::SP];
  const int h = blockIdx.x, b = blockIdx.y;
  const int64_t row = (int64_t(b) * H + h) * L;
  const float* kr = k + (kfilm ? int64_t(b) * H + h : int64_t(h)) * K;

  auto ld = [&](int m, int n) -> float2 {
    if (m == 0) return load_pair<NSQ_DTYPE_F32>(kr, 2 * int64_t(n), K);
    return load_pair<DT>(x + row, 2 * int64_t(n), L);
  };
  LdsTile<C::SP, true> st{lds};
  fft_radix<LOGRMAX, LOGN, false, 2, T, C::SP>(lds, ld, st, tw);
#pragma unroll
  for (int i = 0; i < SL; ++i) {
    NSQ_SLOT_FENCE();
    const int p = opaque_tid() + i * T;
    float2 hA, hB, A, Bc;
    lds_unpack<LOGN>(lds, 0, p, tw, hA, hB);
    lds_unpack<LOGN>(lds, 1, p, tw, A, Bc);
    A = slot_mul(p == 0, A, hA);
    Bc = cmul(Bc, hB);
    lds_repack<LOGN>(lds, 1, p, tw, A, Bc);
  }
  __syncthreads();

  const float scale = 1.f / float(C::N);
  const float sv = s ? Elem<DT>::round(Elem<DT>::load(s, h)) : 0.f;
  auto epi = [&](int m, int n, float2 v) {
    if (m == 0) return;
    const int64_t i0 = 2 * int64_t(n);
    if (i0 < L)
      Elem<DT>::store(y, row + i0, epilogue<DT>(v.x * scale, s != nullptr, sv, s ? Elem<DT>::load(x, row + i0) : 0.f));
    if (i0 + 1 < L)
      Elem<DT>::store(y, row + i0 + 1,
                      epilogue<DT>(v.y * scale, s != nullptr, sv, s ? Elem<DT>::load(x, row + i0 + 1) : 0.f));
  };
  LdsTile<C::SP, true> ldl{lds};
  fft_radix<LOGRMAX, LOGN, true, 2, T, C::SP>(lds, ldl, epi, tw);
}

// Backward, fused plan.  grid = ceil(H/M); each workgroup loops over all
// batch rows (the filter gradient sums over the batch in a fixed order).
// kfilm: grid = (ceil(H/M), B), one image per workgroup, whose filter and
// filter-gradient rows are that image's.  CIRC: as the forward; the filter
// gradient gk[j] = sum_n g[n] x[(n + c - j) mod L] is the correlation read at
// lag (j - c) mod L; on a periodic extension (wm = L - 1) every lag repeats
// 2N / L times, so gk and gs are scaled by gks = L / 2N (1 otherwise).
template <int LOGN, int DT, bool FOLD, bool CIRC = false>
__global__ __launch_bounds__(FusedCfg<LOGN>::T) void fused_bwd_kernel(
    const typename Elem<DT>::T* __restrict__ g, const typename Elem<DT>::T* __restrict__ x,
    const float* __restrict__ k, const typename Elem<DT>::T* __restrict__ s, typename Elem<DT>::T* __restrict__ gx,
    float* __restrict__ gk, float* __restrict__ gs, int B, int H, int L, int K, const float2* __restrict__ tw, int c,
    int kfilm, int wm, float gks) {
  using C = FusedCfg<LOGN>;
  __shared__ float2 ldsG[C::TILE_P];
  __shared__ float2 ldsX[C::TILE_P];
  const int h0 = blockIdx.x * C::M;
  const int bb0 = kfilm ? int(blockIdx.y) : 0, bb1 = kfilm ? bb0 + 1 : B;
  const int64_t koff = kfilm ? int64_t(bb0) * H * K : 0;
  if (kfilm) {
    gk += koff;
    if (gs) gs += int64_t(bb0) * H;
  }

  float2 hA[C::SLOTS], hB[C::SLOTS];
  filter_spectrum<LOGN, CIRC>(ldsG, k + koff, h0, H, K, tw, hA, hB, c);
  float2 qA[C::SLOTS], qB[C::SLOTS];
#pragma unroll
  for (int i = 0; i < C::SLOTS; ++i) qA[i] = qB[i] = make_float2(0.f, 0.f);

  const float scale = 1.f / float(C::N);
  for (int b = bb0; b < bb1; ++b) {
    // g extended by its adjoint fold copy at offset 2L (FOLD only).
    auto ldg = [&](int m, int n) -> float2 {
      const int h = h0 + m;
      if (h >= H) return make_float2(0.f, 0.f);
      const int64_t ro = (int64_t(b) * H + h) * L;
      const typename Elem<DT>::T* row = g + ro;
      const int64_t i0 = 2 * int64_t(n);
      const bool fold = FOLD && i0 >= 2 * int64_t(L);
      const int64_t i = fold ? i0 - 2 * int64_t(L) : (i0 & wm);
      return load_pair<DT>(row, i, L);
    };
    auto ldx = [&](int m, int n) -> float2 {
      const int h = h0 + m;
      if (h >= H) return make_float2(0.f, 0.f);
      const int64_t ro = (int64_t(b) * H + h) * L, i = (2 * int64_t(n)) & wm;
      return load_pair<DT>(x + ro, i, L);
    };
    LdsTile<C::SP, true> stG{ldsG};
    LdsTile<C::SP, true> stX{ldsX};
    fft<LOGN, false, C::M, C::T, C::SP>(ldsG, ldg, stG, tw);
    fft<LOGN, false, C::M, C::T, C::SP>(ldsX, ldx, stX, tw);
#pragma unroll
    for (int i = 0; i < C::SLOTS; ++i) {
    NSQ_SLOT_FENCE();
      int m, p;
      slot_of<LOGN>(opaque_tid() + i * C::T, m, p);
      float2 GA, GB, XA, XB;
      lds_unpack<LOGN>(ldsG, m, p, tw, GA, GB);
      lds_unpack<LOGN>(ldsX, m, p, tw, XA, XB);
      const bool s0 = (p == 0);
      qA[i] = cadd(qA[i], slot_mulc(s0, GA, XA));
      qB[i] = cadd(qB[i], cmulc(GB, XB));
      lds_repack<LOGN>(ldsG, m, p, tw, slot_mulc(s0, GA, hA[i]), cmulc(GB, hB[i]));
    }
    __syncthreads();
    auto epi = [&](int m, int n, float2 v) {
      const int h = h0 + m;
      if (h >= H) return;
      const int64_t row = (int64_t(b) * H + h) * L;
      const float sv = s ? Elem<DT>::round(Elem<DT>::load(s, h)) : 0.f;
      const int64_t i0 = 2 * int64_t(n);
      auto out = [&](int64_t i, float conv) {
        Elem<DT>::store(gx, row + i, epilogue<DT>(conv, s != nullptr, sv, s ? Elem<DT>::load(g, row + i) : 0.f));
      };
      if (i0 < L) out(i0, v.x * scale);
      if (i0 + 1 < L) out(i0 + 1, v.y * scale);
    };
    LdsTile<C::SP, true> ldl{ldsG};
    fft<LOGN, true, C::M, C::T, C::SP>(ldsG, ldl, epi, tw);
  }

  // Filter gradient (and shortcut gradient = its lag-0 value).
#pragma unroll
  for (int i = 0; i < C::SLOTS; ++i) {
    NSQ_SLOT_FENCE();
    int m, p;
    slot_of<LOGN>(opaque_tid() + i * C::T, m, p);
    lds_repack<LOGN>(ldsX, m, p, tw, qA[i], qB[i]);
  }
  __syncthreads();
  auto epik = [&](int m, int n, float2 v) {
    const int h = h0 + m;
    if (h >= H) return;
    if constexpr (CIRC) {
      constexpr int F = 2 * C::N;
      const int j0 = (2 * n + c) & (F - 1), j1 = (2 * n + 1 + c) & (F - 1);
      if (j0 < K) gk[int64_t(h) * K + j0] = v.x * scale * gks;
      if (j1 < K) gk[int64_t(h) * K + j1] = v.y * scale * gks;
    } else {
      const int64_t i0 = 2 * int64_t(n);
      if (i0 < K) gk[int64_t(h) * K + i0] = v.x * scale;
      if (i0 + 1 < K) gk[int64_t(h) * K + i0 + 1] = v.y * scale;
    }
    if (n == 0 && gs) gs[h] = v.x * scale * gks;
  };
  LdsTile<C::SP, true> ldl{ldsX};
  fft<LOGN, true, C::M, C::T, C::SP>(ldsX, ldl, epik, tw);
}

// ===========================================================================
// 4-step plan
// ===========================================================================
// Column kernels: a workgroup owns C adjacent columns (n2) of one signal row
// and runs their length-N1 transforms.  Thread lanes map to consecutive columns
// (TMAJOR passes), so the first pass reads row segments of C consecutive packed
// samples straight from HBM and the last pass writes row segments of C complex
// values straight to the workspace: no separate staging copies.
template <int LOGN1>
struct ColCfg {
  static constexpr int N1 = 1 << LOGN1;
  static constexpr int M = (8192 >> LOGN1) < 8 ? 8 : ((8192 >> LOGN1) > 32 ? 32 : (8192 >> LOGN1));  // columns
  static constexpr int S = N1 + 1;  // odd transform stride: consecutive columns hit distinct LDS banks
  static constexpr int TILE = M * N1;
  static constexpr int T = TILE / 16;
};

// Description of a real input signal set: rows of `valid` samples with row
// stride `stride` (elements), zero-extended to length F.
template <int DT>
struct RealRows {
  const typename Elem<DT>::T* p;
  int64_t stride;
  int64_t valid;
};

// The 4-step plan's HBM streams are read or written once per kernel: the
// complex intermediates (each written once and read once by a later kernel)
// and the rows of x, k, g, y, gx and gk.  They go through the nontemporal
// (streaming) cache policy.  Measured at config 3, same box, alternating
// runs: 27.93 / 28.10 ms per step with the default policy, 27.62 / 27.62 with
// streaming intermediates, 27.44 / 27.46 with the row I/O streaming too.
constexpr int kStreamAux = 2;  // buffer-intrinsic cache policy: bit 1 = nt on gfx950
__device__ __forceinline__ void ws_store(float2* p, float2 v) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  __builtin_nontemporal_store(v2f{v.x, v.y}, reinterpret_cast<v2f*>(p));
}
__device__ __forceinline__ float2 ws_load(const float2* p) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  const v2f v = __builtin_nontemporal_load(reinterpret_cast<const v2f*>(p));
  return make_float2(v.x, v.y);
}

// Last-pass store of col_fwd: out[k1][n2] = v * W_N^{n2 k1}.  A butterfly's
// outputs k1 = base + r*NS share n2, so the twiddle starts at W_N^{n2 base}
// and steps by W_N^{n2 NS}: two hardware sin/cos pairs per butterfly instead
// of one per output (the recurrence adds at most R-1 roundings, ~1e-6).
template <int LOGN, int N2>
struct TwiddledColumnStore {
  static constexpr bool kRunStore = true;
  float2* out;
  int c0;
  const float2* tw;
  template <int R, int NS>
  __device__ __forceinline__ void run(int m, int base, const float2 (&v)[R]) const {
    const uint32_t n2 = uint32_t(c0 + m);
    float2 w = root<LOGN>(tw, n2 * uint32_t(base));
    const float2 step = root<LOGN>(tw, n2 * uint32_t(NS));
#pragma unroll
    for (int r = 0; r < R; ++r) {
      ws_store(out + int64_t(base + r * NS) * N2 + n2, cmul(v[r], w));
      if (r + 1 < R) w = cmul(w, step);
    }
  }
};

// Column tiles per workgroup.  Workgroup w runs tiles w, w + G, w + 2G, ...
// (G = grid size), so the workgroups resident together still cover adjacent
// column blocks of the same rows, and each prefetches its next tile's
// first-pass inputs while it transforms the current one.
constexpr int kColTilesPerWG = 8;

// col_fwd: A[row][k1][n2] = W_N^{n2 k1} * sum_{n1} z[N2 n1 + n2] W_{N1}^{n1 k1}.
// Tile t = row * (N2 / M) + column block: column block fastest.  The first
// pass is one radix-R butterfly per thread (T = M * N1 / R); its R input
// pairs for the next tile are loaded as raw bits before the current tile's
// passes run and converted when that tile starts.  HALF (valid <= N real
// samples, i.e. at least half the transform is zero padding, as in every
// causal conv with K > 1): the inputs n1 >= N1/2 of a column are zero, so only
// R/2 pairs are loaded and the first pass's butterflies fold the zeros away.
template <int LOGN1, int LOGN, int DT, bool AL, bool HALF>
__global__ __launch_bounds__(ColCfg<LOGN1>::T) __attribute__((amdgpu_waves_per_eu(4))) void col_fwd_kernel(
    RealRows<DT> src, float2* __restrict__ ws, const float2* __restrict__ tw, int64_t ntiles) {
  using C = ColCfg<LOGN1>;
  using RB = RowBuf<DT, AL, kStreamAux>;
  constexpr int N2 = 1 << (LOGN - LOGN1);
  constexpr int NCB = N2 / C::M;
  constexpr int R = 1 << (LOGN1 < 4 ? LOGN1 : 4);  // first-pass radix, as chosen by fft_rec
  constexpr int NR = C::N1 / R;
  constexpr int RL = HALF ? R / 2 : R;             // inputs that can be nonzero
  static_assert(C::M * NR == C::T, "col_fwd: one first-pass butterfly per thread");
  __shared__ float2 lds[C::M * C::S];
  const int tid = threadIdx.x;
  const int m = tid % C::M, j = tid / C::M;  // the first pass's (transform, butterfly) of this thread
  typename RB::PairBits raw[RL];
  auto issue = [&](int64_t t) {
    const int c0 = int(t % NCB) * C::M;
    const RB in(src.p + (t / NCB) * src.stride, src.valid);
#pragma unroll
    for (int r = 0; r < RL; ++r) raw[r] = in.load_pair_bits(2 * (int64_t(j + r * NR) * N2 + c0 + m));
  };
  int64_t t = blockIdx.x;  // grid <= ntiles
  issue(t);
  for (;;) {
    float2 v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = r < RL ? RB::pair_from_bits(raw[r < RL ? r : 0]) : make_float2(0.f, 0.f);
    const int64_t tn = t + gridDim.x;
    if (tn < ntiles) issue(tn);
    RegStream<R> ld{v};
    LdsTile<C::S, false> tile{lds};
    TwiddledColumnStore<LOGN, N2> st{ws + (t / NCB) * (int64_t(1) << LOGN), int(t % NCB) * C::M, tw};
    fft_rec<LOGN1, 0, false, C::M, C::T, true>(ld, tile, tile, st, tw);
    if (tn >= ntiles) break;
    t = tn;
  }
}

// First-pass loader of the inverse column pass: B[k1][n2] * W_N^{-n2 k1}, the
// 4-step twiddle of the inverse row outputs.  The pass calls it R times per
// butterfly with k1 = j + r*NR (r = 0..R-1, n2 fixed), so the twiddle starts at
// W_N^{-n2 j} and steps by W_N^{-n2 NR}: two hardware sin/cos pairs per
// butterfly (the recurrence adds at most R-1 roundings, ~1e-6).
template <int LOGN, int N2, int R, int NR>
struct TwiddledColumnLoad {
  const float2* ws_row;
  int c0;
  const float2* tw;
  int q = 0;
  float2 w, step;
  __device__ __forceinline__ float2 operator()(int m, int k1) {
    const uint32_t n2 = uint32_t(c0 + m);
    if (q % R == 0) {  // a butterfly's first input (q is a constant after unrolling)
      w = root<LOGN>(tw, n2 * uint32_t(k1));
      step = root<LOGN>(tw, n2 * uint32_t(NR));
    }
    const float2 v = cmulc(ws_load(ws_row + int64_t(k1) * N2 + c0 + m), w);
    if (q % R != R - 1) w = cmul(w, step);
    ++q;
    return v;
  }
};

// col_inv: z[N2 n1 + n2] = sum_{k1} (B[row][k1][n2] W_N^{-n2 k1}) W_{N1}^{-n1 k1};
// the epilogue functor consumes (packed output index m = N2 n1 + n2, value).
template <int LOGN1, int LOGN, class EPI>
__device__ __forceinline__ void col_inv_body(const float2* __restrict__ ws_row, int c0, EPI& epi,
                                             const float2* __restrict__ tw, float2* lds) {
  using C = ColCfg<LOGN1>;
  constexpr int N2 = 1 << (LOGN - LOGN1);
  constexpr int R = 1 << (LOGN1 < 4 ? LOGN1 : 4);  // first-pass radix, as chosen by fft_rec
  constexpr int NR = C::N1 / R;
  static_assert(C::M * NR == C::T, "col_inv: one first-pass butterfly per thread");
  TwiddledColumnLoad<LOGN, N2, R, NR> ld{ws_row, c0, tw};
  auto st = [&](int m, int n1, float2 v) { epi(int64_t(n1) * N2 + c0 + m, v); };
  fft<LOGN1, true, C::M, C::T, C::S, true>(lds, ld, st, tw);
}

// Output epilogue for y (forward) or gx (backward): out = epi(conv, s, aux)
// where aux is x (forward) or g (backward).  grid = B*H * (N2/M), column block
// fastest.  Without a shortcut the aux row is an empty buffer (reads 0, no
// traffic).
template <int LOGN1, int LOGN, int DT, bool AL>
__global__ __launch_bounds__(ColCfg<LOGN1>::T) void col_inv_out_kernel(
    const float2* __restrict__ ws, const typename Elem<DT>::T* __restrict__ aux,
    const typename Elem<DT>::T* __restrict__ s, typename Elem<DT>::T* __restrict__ out, int H, int L,
    const float2* __restrict__ tw) {
  using C = ColCfg<LOGN1>;
  constexpr int NCB = (1 << (LOGN - LOGN1)) / C::M;
  __shared__ float2 lds[C::M * C::S];
  const int64_t row = blockIdx.x / NCB;
  const int c0 = int(blockIdx.x % NCB) * C::M;
  const int h = int(row % H);
  const float scale = 1.f / float(int64_t(1) << LOGN);
  const bool has_s = s != nullptr;
  const float sv = has_s ? Elem<DT>::round(Elem<DT>::load(s, h)) : 0.f;
  const RowBuf<DT, AL, kStreamAux> orow(out + row * L, L);
  const RowBuf<DT, AL, kStreamAux> arow(aux + row * L, has_s ? L : 0);
  auto epi = [&](int64_t m, float2 v) {
    const int64_t i0 = 2 * m;
    const float2 a = arow.load_pair(i0);
    orow.store_pair(i0, make_float2(epilogue<DT>(v.x * scale, has_s, sv, a.x),
                                    epilogue<DT>(v.y * scale, has_s, sv, a.y)));
  };
  col_inv_body<LOGN1, LOGN>(ws + row * (int64_t(1) << LOGN), c0, epi, tw, lds);
}

// Filter-gradient epilogue: gk[h, 0:K] fp32, gs[h] = lag-0 value.
// grid = H * (N2/M), column block fastest.
template <int LOGN1, int LOGN, bool AL>
__global__ __launch_bounds__(ColCfg<LOGN1>::T) void col_inv_gk_kernel(const float2* __restrict__ ws,
                                                                       float* __restrict__ gk, float* __restrict__ gs,
                                                                       int K, const float2* __restrict__ tw) {
  using C = ColCfg<LOGN1>;
  constexpr int NCB = (1 << (LOGN - LOGN1)) / C::M;
  __shared__ float2 lds[C::M * C::S];
  const int64_t h = blockIdx.x / NCB;
  const int c0 = int(blockIdx.x % NCB) * C::M;
  const float scale = 1.f / float(int64_t(1) << LOGN);
  const RowBuf<NSQ_DTYPE_F32, AL, kStreamAux> grow(gk + h * K, K);
  bool has0 = false;  // this thread produced lag 0 (selects, not a branch per element)
  float g0 = 0.f;
  auto epi = [&](int64_t m, float2 v) {
    grow.store_pair(2 * m, make_float2(v.x * scale, v.y * scale));
    has0 = has0 || (m == 0);
    g0 = (m == 0) ? v.x * scale : g0;
  };
  col_inv_body<LOGN1, LOGN>(ws + h * (int64_t(1) << LOGN), c0, epi, tw, lds);
  if (gs && has0) gs[h] = g0;
}

// Row kernels.  Workgroup q handles the row pair {q, N1-q} (q >= 1) or the two
// self-paired rows {0, N1/2} (q == 0) of one channel; a tile is 2 rows of N2.
template <int LOGN2>
struct RowCfg {
  static constexpr int N2 = 1 << LOGN2;
  static constexpr int N2P = Padded<N2>::SIZE;  // padded LDS stride of a row
  static constexpr int TILE = 2 * N2;
  static constexpr int TILE_P = 2 * N2P;
  static constexpr int T = TILE / 16;
  static constexpr int SLOTS = 8;  // N2 slots per workgroup / T threads
};

// Spectral slots of the row-pair tile.  Slot s = t + i*T (thread t, i <
// SLOTS) pairs two bins of the real spectrum:
//  * q > 0: element s of tile row 0 (row q) with element N2-1-s of tile row 1
//    (row N1-q);
//  * q == 0, i < SLOTS/2: row 0 with itself, s <-> N2-s (slot 0 holds bins 0,
//    N and N/2);
//  * q == 0, i >= SLOTS/2: tile row 1 (k1 = N1/2) with itself, s2 <-> N2-1-s2,
//    s2 = s - N2/2.
// The unpack root of the slot is W_2N^{k1 + N1 s2}.  Since T is a multiple of
// 16, pad16(x + c) = pad16(x) + pad16(c) for c a multiple of 16 and
// pad16(c - x) = pad16(c) - pad16(x) for c = 15 mod 16, so each LDS position
// is a per-thread base plus a compile-time offset plus a per-workgroup
// constant; and the root factors as a per-workgroup root W_2N^{k1} (times i
// on the second q == 0 half) times the table root W_{2 N2}^s.  (All formulas
// were checked against the direct index arithmetic for every slot of N1 in
// [2^7, 2^10], N2 in [2^7, 2^12].)
template <int LOGN1, int LOGN2>
struct RowSlots {
  using C = RowCfg<LOGN2>;
  static constexpr int N1 = 1 << LOGN1, N2 = 1 << LOGN2, N2P = C::N2P, T = C::T;
  static_assert(T % 16 == 0 && 2 * N2 <= (1 << 14), "RowSlots: tile shape");
  TwTable tt;
  int t;
  bool qz;     // q == 0
  int base;    // pad16(t)
  int corr;    // q == 0 first half: pad16(N2 - s) = pad16(N2 - 1) - pad16(s) + 1 + (s % 16 == 0)
  float2 u0;   // W_2N^q (q > 0), 1 (q == 0)
  float2 u1;   // W_2N^{N1/2} * i (q == 0, second half)
  float2 wt;   // W_{2 N2}^t: slot i's table root W_{2 N2}^{t + i T} is wt * W_16^i (2 N2 = 16 T)
  __device__ __forceinline__ RowSlots(int q, const float2* __restrict__ tw) : RowSlots(q, tw, opaque_tid()) {}
  // tl: the thread's index among the T threads of its row pair (a workgroup
  // may run several row pairs side by side, each on its own 2-row sub-tile).
  __device__ __forceinline__ RowSlots(int q, const float2* __restrict__ tw, int tl) : tt(tw) {
    constexpr int LOGN = LOGN1 + LOGN2;
    t = tl;
    qz = (q == 0);
    base = pad16(t);
    corr = (t & 15) == 0 ? 1 : 0;
    u0 = qz ? make_float2(1.f, 0.f) : root<LOGN + 1>(tw, uint32_t(q));
    u1 = mul_i(root<LOGN + 1>(tw, uint32_t(N1 / 2)));
    wt = tt.load(2 * N2, t);
  }
  __device__ __forceinline__ bool s0(int i) const { return qz && i == 0 && t == 0; }
  __device__ __forceinline__ void at(int i, int& pa, int& pb, float2& w) const {
    const bool sec = qz && (i >= C::SLOTS / 2);
    const bool f0 = qz && (i < C::SLOTS / 2);
    const int oi = pad16(i * T);
    pa = base + oi + (sec ? N2P - pad16(N2 / 2) : 0);
    const int ub = !qz ? N2P + pad16(N2 - 1) : (sec ? N2P + pad16(3 * N2 / 2 - 1) : pad16(N2 - 1) + 1);
    pb = ub - base - oi + (f0 ? corr : 0);
    pb = s0(i) ? pad16(N2 / 2) : pb;
    static_assert(2 * N2 == 16 * T, "RowSlots: slot roots step by W_16");
    w = cmul_fixed(sec ? u1 : u0, rot16(wt, i));
  }
};

// Loads the two rows of the pair into a tile: tile row 0 = row q (or 0), tile
// row 1 = row N1-q (or N1/2), then forward row DFTs; spectrum in natural order.
template <int LOGN1, int LOGN2>
__device__ __forceinline__ void row_pair_fft(float2* lds, const float2* __restrict__ sig, int q,
                                             const float2* __restrict__ tw) {
  using C = RowCfg<LOGN2>;
  constexpr int N1 = 1 << LOGN1;
  const int ra = q, rb = (q == 0) ? N1 / 2 : N1 - q;
  auto ld = [&](int m, int n) -> float2 { return ws_load(sig + int64_t(m == 0 ? ra : rb) * C::N2 + n); };
  LdsTile<C::N2P, true> st{lds};
  fft<LOGN2, false, 2, C::T, C::N2P>(lds, ld, st, tw);
}

// Last-pass store of an inverse row pair: sig[k1][n] = v, k1 = ra (tile row
// 0) or rb (tile row 1).  The 4-step twiddle W_N^{-n k1} of these values is
// applied by the inverse column pass as it loads them (TwiddledColumnLoad):
// the row kernels are bound by their VALU issue, the column pass is not.
template <int N2>
struct RowStore {
  float2* sig;
  int ra, rb;
  __device__ __forceinline__ void operator()(int m, int n, float2 v) const {
    ws_store(sig + int64_t(m == 0 ? ra : rb) * N2 + n, v);
  }
};

// Inverse row DFT of the tile, stored to sig rows (untwiddled, see RowStore).
template <int LOGN1, int LOGN2>
__device__ __forceinline__ void row_pair_ifft_store(float2* lds, float2* __restrict__ sig, int q,
                                                    const float2* __restrict__ tw) {
  using C = RowCfg<LOGN2>;
  constexpr int N1 = 1 << LOGN1;
  const int ra = q, rb = (q == 0) ? N1 / 2 : N1 - q;
  LdsTile<C::N2P, true> ld{lds};
  RowStore<C::N2> st{sig, ra, rb};
  fft<LOGN2, true, 2, C::T, C::N2P>(lds, ld, st, tw);
}

template <int LOGN1, int LOGN2>
__device__ __forceinline__ void row_unpack(const float2* lds, const RowSlots<LOGN1, LOGN2>& rs, int i, float2& A,
                                           float2& Bc) {
  int pa, pb;
  float2 w;
  rs.at(i, pa, pb, w);
  real_unpack(rs.s0(i), lds[pa], lds[pb], w, A, Bc);
}

template <int LOGN1, int LOGN2>
__device__ __forceinline__ void row_repack(float2* lds, const RowSlots<LOGN1, LOGN2>& rs, int i, float2 A,
                                           float2 Bc) {
  int pa, pb;
  float2 w;
  rs.at(i, pa, pb, w);
  float2 zp, zq;
  real_repack(rs.s0(i), A, Bc, w, zp, zq);
  lds[pa] = zp;
  lds[pb] = zq;
}

// ---------------------------------------------------------------------------
// Row pairs with the spectral slots in registers (rows of N2 = 1024: forward
// passes of radix 16, 16, 4; inverse passes of radix 4, 16, 16).
//
// The last forward pass (radix 4, 256 butterflies per row) gives butterfly j
// the elements {j + 256 r}, r < 4, in and out.  Assigning the butterflies so
// that a thread owns both Hermitian partners of each output lets the real
// unpack, the spectral product and the repack run on registers, and the
// inverse transform starts with the matching radix-4 pass (first pass,
// butterfly j reads {j + 256 r}) on the same registers.  Against the tile
// round trip of row_unpack/row_repack this saves, per transform, one LDS
// write and read of the whole tile and two barriers.
//
// Thread t (of 128 per pair) owns four butterflies b = (tile row, j):
//   q > 0 : (0, t), (1, 255 - t), (0, 255 - t), (1, t).  Row-0 element
//           j + 256 r pairs with row-1 element (255 - j) + 256 (3 - r), so
//           group g = {b = 2g, 2g + 1} holds slots (b0 out r, b1 out 3 - r).
//   q == 0: rows 0 and N1/2 pair within themselves: (0, t), (0, 256 - t),
//           (1, t), (1, 255 - t); thread 0's row-0 butterflies are (0, 0) and
//           (0, 128), each paired with itself (out r with out (4 - r) mod 4,
//           slot 0 = elements 0 and 512; out r with out 3 - r).
// Slot (g, e), e < 4, is element s = j_{2g} + 256 e of row k1: frequency
// p = k1 + N1 s, unpack root W_2N^{k1} W_2048^{j} W_16^{2e}.
// ---------------------------------------------------------------------------
template <bool QZ>
struct RegPair {
  static constexpr int LOGN2 = 10, N2 = 1024, T = 128, NB = 4, R = 4, NRL = 256;
  bool sp;  // q == 0 and thread 0: row-0 butterflies self-paired
  int m[NB], j[NB];
  __device__ __forceinline__ explicit RegPair(int tl) {
    sp = QZ && (tl == 0);
    m[0] = 0;
    j[0] = tl;
    m[1] = QZ ? 0 : 1;
    j[1] = QZ ? (tl == 0 ? NRL / 2 : NRL - tl) : NRL - 1 - tl;
    m[2] = QZ ? 1 : 0;
    j[2] = QZ ? tl : NRL - 1 - tl;
    m[3] = 1;
    j[3] = QZ ? NRL - 1 - tl : tl;
  }
};
constexpr int kRegPairLogN2 = 10;

// Forward passes 1 and 2 of M rows of 1024 (first pass reads through ld).
template <int M, int T, class LD>
__device__ __forceinline__ void rows1024_fwd_head(float2* lds, LD& ld, const float2* __restrict__ tw) {
  LdsTile<RowCfg<10>::N2P, true> tile{lds};
  stockham_pass<10, 4, 0, false, M, T, false>(ld, tile, tw);
  stockham_pass<10, 4, 4, false, M, T, false>(tile, tile, tw);
}

// Inverse passes 2 and 3 of M rows of 1024 (radix 16 after the radix-4 first
// pass), the last one storing through st.
template <int M, int T, class ST>
__device__ __forceinline__ void rows1024_inv_tail(float2* lds, ST& st, const float2* __restrict__ tw) {
  LdsTile<RowCfg<10>::N2P, true> tile{lds};
  stockham_pass<10, 4, 2, true, M, T, false>(tile, tile, tw);
  stockham_pass<10, 4, 6, true, M, T, false>(tile, st, tw);
}

// Last forward pass of a row pair (its 2-row sub-tile `sub`) into registers.
// Reads only; the caller's next tile write must follow a barrier.
template <bool QZ>
__device__ __forceinline__ void regpair_last_fwd(const float2* sub, const RegPair<QZ>& rp,
                                                 const float2* __restrict__ tw, float2 (&v)[4][4]) {
  using TL = LdsTile<RowCfg<10>::N2P, true>;
  const TL tile{const_cast<float2*>(sub)};
  const TwTable tt(tw);
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    float2 w[4];
    pass_twiddles<4>(tt, 1 << 10, rp.j[b], w);
    const float2* p = tile.at(rp.m[b], rp.j[b]);
#pragma unroll
    for (int r = 0; r < 4; ++r) v[b][r] = p[TL::off(r * 256)];
#pragma unroll
    for (int r = 1; r < 4; ++r) v[b][r] = cmul(v[b][r], w[r]);
    dft<4, false>(v[b]);
  }
}

// First inverse pass (radix 4, no twiddles) of the pair's registers into its
// sub-tile: butterfly j's outputs go to elements 4 j + r.  The caller puts a
// barrier before (the tile may still be read) and after.
template <bool QZ>
__device__ __forceinline__ void regpair_first_inv(float2* sub, const RegPair<QZ>& rp, float2 (&v)[4][4]) {
  using TL = LdsTile<RowCfg<10>::N2P, true>;
  const TL tile{sub};
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    dft<4, true>(v[b]);
    float2* p = tile.at(rp.m[b], 4 * rp.j[b]);
#pragma unroll
    for (int r = 0; r < 4; ++r) p[TL::off(r)] = v[b][r];
  }
}

__device__ __forceinline__ float2 sel2(bool c, float2 a, float2 b) {
  return make_float2(c ? a.x : b.x, c ? a.y : b.y);
}

// Runs f(i, s0, A, Bc) on the pair's 8 spectral slots i = 4 g + e in order
// (slot form, see real_unpack; s0 marks slot 0 of the q == 0 pair).  With
// REPACK the slot values f leaves in (A, Bc) are repacked into the butterfly
// registers in place: each slot reads and writes its own two positions, which
// no other slot touches, so slot-at-a-time is exact and holds no slot arrays.
// Slot (g, e) is element j_{2g} + 256 e of its row: root W_2N^{k1}
// W_2048^{j_{2g}} W_16^{2e}; for thread 0 of q == 0, group 0 holds the
// self-paired elements 0/512 (slot 0), 256/768, 128/896 and 384/640.
// UNPACK = false: f sets the slot values itself (a spectrum formed from slots
// alone, such as a sum over batch rows) and nothing is read from v.
template <int LOGN1, bool QZ, bool REPACK, bool UNPACK = true, class F>
__device__ __forceinline__ void regpair_slots(const RegPair<QZ>& rp, int q, float2 (&v)[4][4],
                                              const float2* __restrict__ tw, F&& f) {
  constexpr int LOGN = LOGN1 + 10, N1 = 1 << LOGN1;
  const TwTable tt(tw);
  float2 u[2], wj[2];
  u[0] = QZ ? make_float2(1.f, 0.f) : root<LOGN + 1>(tw, uint32_t(q));
  u[1] = QZ ? root<LOGN + 1>(tw, uint32_t(N1 / 2)) : u[0];
  wj[0] = tt.load(2048, rp.j[0]);
  wj[1] = tt.load(2048, rp.j[2]);
#pragma unroll
  for (int g = 0; g < 2; ++g) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      NSQ_SLOT_FENCE();
      const int b0 = 2 * g, b1 = 2 * g + 1;
      float2 zp = v[b0][e], zq = v[b1][3 - e];
      float2 w = cmul_fixed(u[g], rot16(wj[g], 2 * e));
      const bool spg = QZ && g == 0;  // thread 0 of q == 0 may take the self-paired form
      if (spg) {
        const float2 spp = e < 2 ? v[0][e] : v[1][e - 2];
        const float2 spq = e < 2 ? v[0][e + 2] : v[1][5 - e];
        zp = sel2(rp.sp, spp, zp);
        zq = sel2(rp.sp, spq, zq);
        if (e >= 2) w = sel2(rp.sp, rot16(make_float2(1.f, 0.f), 2 * e - 3), w);  // W_16^1, W_16^3
      }
      const bool s0 = spg && e == 0 && rp.sp;
      float2 A = make_float2(0.f, 0.f), Bc = A;
      if constexpr (UNPACK) real_unpack(s0, zp, zq, w, A, Bc);
      f(4 * g + e, s0, A, Bc);
      if constexpr (REPACK) {
        real_repack(s0, A, Bc, w, zp, zq);
        if (spg) {  // both position sets, the unused one keeping its value (e < 2 share v[0][e])
          const bool S = rp.sp;
          if (e < 2) {
            v[0][e] = zp;
            v[1][3 - e] = sel2(S, v[1][3 - e], zq);
            v[0][e + 2] = sel2(S, zq, v[0][e + 2]);
          } else {
            v[0][e] = sel2(S, v[0][e], zp);
            v[1][3 - e] = sel2(S, v[1][3 - e], zq);
            v[1][e - 2] = sel2(S, zp, v[1][e - 2]);
            v[1][5 - e] = sel2(S, zq, v[1][5 - e]);
          }
        } else {
          v[b0][e] = zp;
          v[b1][3 - e] = zq;
        }
      }
    }
  }
}

// Last forward pass and slot loop of one row pair, for a pair index q known
// only at run time (the q == 0 pair pairs its rows within themselves).  No
// barriers inside, so the threads of one workgroup may take either branch.
template <int LOGN1, bool REPACK, class F>
__device__ __forceinline__ void regpair_fwd_slots(const float2* sub, int q, int tl, const float2* __restrict__ tw,
                                                  float2 (&v)[4][4], F&& f) {
  if (q == 0) {
    const RegPair<true> rp(tl);
    regpair_last_fwd(sub, rp, tw, v);
    regpair_slots<LOGN1, true, REPACK>(rp, q, v, tw, f);
  } else {
    const RegPair<false> rp(tl);
    regpair_last_fwd(sub, rp, tw, v);
    regpair_slots<LOGN1, false, REPACK>(rp, q, v, tw, f);
  }
}

// Repack of slot values that f supplies (no forward pass, nothing unpacked)
// into the butterfly registers, for a pair index q known only at run time.
template <int LOGN1, class F>
__device__ __forceinline__ void regpair_set_slots(int q, int tl, const float2* __restrict__ tw, float2 (&v)[4][4],
                                                  F&& f) {
  if (q == 0)
    regpair_slots<LOGN1, true, true, false>(RegPair<true>(tl), q, v, tw, f);
  else
    regpair_slots<LOGN1, false, true, false>(RegPair<false>(tl), q, v, tw, f);
}

// The inverse transform of a row pair held in registers: first pass into the
// pair's sub-tile, then passes 2 and 3 over the whole tile of M rows (T
// threads), the last one storing through st.
template <int M, int T, class ST>
__device__ __forceinline__ void regpair_inverse(float2* lds, float2* sub, int q, int tl, float2 (&v)[4][4], ST& st,
                                                const float2* __restrict__ tw) {
  __syncthreads();
  if (q == 0)
    regpair_first_inv(sub, RegPair<true>(tl), v);
  else
    regpair_first_inv(sub, RegPair<false>(tl), v);
  __syncthreads();
  rows1024_inv_tail<M, T>(lds, st, tw);
}

// Forward row kernel.  grid = H * N1/2 (block = h * N1/2 + q).  wsx rows are
// [B*H][N] (column-transformed x), wsk [H][N] (column-transformed k); the
// product's inverse rows go to wsy (== wsx for in-place, or a separate region
// so that wsx and wsk survive for the backward).  The slot geometry (RowSlots)
// is rebuilt per loop so that none of it stays live across the transforms.
template <int LOGN1, int LOGN2>
__global__ __launch_bounds__(RowCfg<LOGN2>::T) __attribute__((amdgpu_waves_per_eu(4))) void row_fwd_kernel(
    const float2* __restrict__ wsx, const float2* __restrict__ wsk, float2* __restrict__ wsy, int B, int H,
    const float2* __restrict__ tw) {
  using C = RowCfg<LOGN2>;
  using RS = RowSlots<LOGN1, LOGN2>;
  constexpr int64_t N = int64_t(1) << (LOGN1 + LOGN2);
  __shared__ float2 lds[C::TILE_P];
  const int q = blockIdx.x % ((1 << LOGN1) / 2);
  const int h = blockIdx.x / ((1 << LOGN1) / 2);
  float2 hA[C::SLOTS], hB[C::SLOTS];
  if constexpr (LOGN2 == kRegPairLogN2) {
    constexpr int N1 = 1 << LOGN1;
    const int ra = q, rb = (q == 0) ? N1 / 2 : N1 - q;
    const int tl = opaque_tid();
    float2 v[4][4];
    auto head = [&](const float2* sig) {
      auto ld = [&](int m, int n) -> float2 { return ws_load(sig + int64_t(m == 0 ? ra : rb) * C::N2 + n); };
      rows1024_fwd_head<2, C::T>(lds, ld, tw);
    };
    head(wsk + int64_t(h) * N);
    regpair_fwd_slots<LOGN1, false>(lds, q, tl, tw, v, [&](int i, bool, float2& A, float2& Bc) {
      hA[i] = A;
      hB[i] = Bc;
    });
    for (int b = 0; b < B; ++b) {
      head(wsx + (int64_t(b) * H + h) * N);
      regpair_fwd_slots<LOGN1, true>(lds, q, tl, tw, v, [&](int i, bool s0, float2& A, float2& Bc) {
        A = slot_mul(s0, A, hA[i]);
        Bc = cmul(Bc, hB[i]);
      });
      RowStore<C::N2> st{wsy + (int64_t(b) * H + h) * N, ra, rb};
      regpair_inverse<2, C::T>(lds, lds, q, tl, v, st, tw);
    }
    return;
  }
  row_pair_fft<LOGN1, LOGN2>(lds, wsk + int64_t(h) * N, q, tw);
  {
    const RS rs(q, tw);
#pragma unroll
    for (int i = 0; i < C::SLOTS; ++i) {
      NSQ_SLOT_FENCE();
      row_unpack(lds, rs, i, hA[i], hB[i]);
    }
  }
  __syncthreads();
  for (int b = 0; b < B; ++b) {
    row_pair_fft<LOGN1, LOGN2>(lds, wsx + (int64_t(b) * H + h) * N, q, tw);
    const RS rs(q, tw);
#pragma unroll
    for (int i = 0; i < C::SLOTS; ++i) {
      NSQ_SLOT_FENCE();
      float2 A, Bc;
      row_unpack(lds, rs, i, A, Bc);
      row_repack(lds, rs, i, slot_mul(rs.s0(i), A, hA[i]), cmul(Bc, hB[i]));
    }
    __syncthreads();
    row_pair_ifft_store<LOGN1, LOGN2>(lds, wsy + (int64_t(b) * H + h) * N, q, tw);
  }
}

// Backward row kernel, any batch.  wsg rows [B*H][N] (in: column-transformed
// g; out: gx pre-image), wsx rows [B*H][N] (column-transformed x), wsk [H][N]
// (in: column-transformed k; out: gk pre-image).  grid = H * N1/2.  Two LDS
// tiles: G and X of one batch row are transformed side by side and the gk
// correlation accumulates over the batch in registers.  The two tiles (2 x 17
// KB per 2-wave workgroup) allow 4 workgroups per CU, i.e. 2 waves per SIMD,
// whatever the register count: the occupancy hint says so.  Rows of 1024 take
// the register-pair path with one tile.
template <int LOGN1, int LOGN2>
__global__ __launch_bounds__(RowCfg<LOGN2>::T) __attribute__((amdgpu_waves_per_eu(2))) void row_bwd_kernel(
    float2* __restrict__ wsg, const float2* __restrict__ wsx, float2* __restrict__ wsk, int B, int H,
    const float2* __restrict__ tw) {
  using C = RowCfg<LOGN2>;
  using RS = RowSlots<LOGN1, LOGN2>;
  constexpr int64_t N = int64_t(1) << (LOGN1 + LOGN2);
  __shared__ float2 ldsG[C::TILE_P];
  __shared__ float2 ldsX[LOGN2 == kRegPairLogN2 ? 1 : C::TILE_P];  // the register-pair path needs one tile
  const int q = blockIdx.x % ((1 << LOGN1) / 2);
  const int h = blockIdx.x / ((1 << LOGN1) / 2);
  float2 hA[C::SLOTS], hB[C::SLOTS], qA[C::SLOTS], qB[C::SLOTS];
  if constexpr (LOGN2 == kRegPairLogN2) {
    // One tile, spectral slots in registers (RegPair): per batch row X's slots
    // are held while G is transformed; the gk correlation accumulates over the
    // batch in slot registers (fixed order b = 0, 1, ...) and is repacked and
    // inverted after the loop.  Its ~170 live VGPRs keep it at 2 waves per
    // SIMD (capped at 3 it spilled 88 bytes per lane and ran slower); it gains
    // from the fewer tile round trips.  Measured at B=4 D=1024 L=K=2^18 bf16:
    // backward 12.57 -> 12.10-12.15 ms.
    constexpr int N1 = 1 << LOGN1;
    const int ra = q, rb = (q == 0) ? N1 / 2 : N1 - q;
    const int tl = opaque_tid();
    float2 v[4][4], xA[C::SLOTS], xB[C::SLOTS];
    auto head = [&](const float2* sig) {
      auto ld = [&](int m, int n) -> float2 { return ws_load(sig + int64_t(m == 0 ? ra : rb) * C::N2 + n); };
      rows1024_fwd_head<2, C::T>(ldsG, ld, tw);
    };
    head(wsk + int64_t(h) * N);
    regpair_fwd_slots<LOGN1, false>(ldsG, q, tl, tw, v, [&](int i, bool, float2& A, float2& Bc) {
      hA[i] = A;
      hB[i] = Bc;
      qA[i] = qB[i] = make_float2(0.f, 0.f);
    });
    for (int b = 0; b < B; ++b) {
      float2* sigg = wsg + (int64_t(b) * H + h) * N;
      head(wsx + (int64_t(b) * H + h) * N);
      regpair_fwd_slots<LOGN1, false>(ldsG, q, tl, tw, v, [&](int i, bool, float2& A, float2& Bc) {
        xA[i] = A;
        xB[i] = Bc;
      });
      head(sigg);
      regpair_fwd_slots<LOGN1, true>(ldsG, q, tl, tw, v, [&](int i, bool s0, float2& A, float2& Bc) {
        qA[i] = cadd(qA[i], slot_mulc(s0, A, xA[i]));
        qB[i] = cadd(qB[i], cmulc(Bc, xB[i]));
        A = slot_mulc(s0, A, hA[i]);
        Bc = cmulc(Bc, hB[i]);
      });
      RowStore<C::N2> st{sigg, ra, rb};
      regpair_inverse<2, C::T>(ldsG, ldsG, q, tl, v, st, tw);
    }
    regpair_set_slots<LOGN1>(q, tl, tw, v, [&](int i, bool, float2& A, float2& Bc) {
      A = qA[i];
      Bc = qB[i];
    });
    RowStore<C::N2> st{wsk + int64_t(h) * N, ra, rb};
    regpair_inverse<2, C::T>(ldsG, ldsG, q, tl, v, st, tw);
    return;
  }
  row_pair_fft<LOGN1, LOGN2>(ldsG, wsk + int64_t(h) * N, q, tw);
  {
    const RS rs(q, tw);
#pragma unroll
    for (int i = 0; i < C::SLOTS; ++i) {
      NSQ_SLOT_FENCE();
      row_unpack(ldsG, rs, i, hA[i], hB[i]);
      qA[i] = qB[i] = make_float2(0.f, 0.f);
    }
  }
  __syncthreads();
  for (int b = 0; b < B; ++b) {
    float2* sigg = wsg + (int64_t(b) * H + h) * N;
    row_pair_fft<LOGN1, LOGN2>(ldsG, sigg, q, tw);
    row_pair_fft<LOGN1, LOGN2>(ldsX, wsx + (int64_t(b) * H + h) * N, q, tw);
    const RS rs(q, tw);
#pragma unroll
    for (int i = 0; i < C::SLOTS; ++i) {
      NSQ_SLOT_FENCE();
      const bool s0 = rs.s0(i);
      float2 GA, GB, XA, XB;
      row_unpack(ldsG, rs, i, GA, GB);
      row_unpack(ldsX, rs, i, XA, XB);
      qA[i] = cadd(qA[i], slot_mulc(s0, GA, XA));
      qB[i] = cadd(qB[i], cmulc(GB, XB));
      row_repack(ldsG, rs, i, slot_mulc(s0, GA, hA[i]), cmulc(GB, hB[i]));
    }
    __syncthreads();
    row_pair_ifft_store<LOGN1, LOGN2>(ldsG, sigg, q, tw);
  }
  {
    const RS rs(q, tw);
#pragma unroll
    for (int i = 0; i < C::SLOTS; ++i) {
      NSQ_SLOT_FENCE();
      row_repack(ldsX, rs, i, qA[i], qB[i]);
    }
  }
  __syncthreads();
  row_pair_ifft_store<LOGN1, LOGN2>(ldsX, wsk + int64_t(h) * N, q, tw);
}

// Backward row kernel for a single batch row (B == 1), one LDS tile.  Same
// buffers as row_bwd_kernel.  Order K -> G -> X: the K slots live in registers
// while G is transformed; unpacking G forms the gx product (repacked in place)
// and the G slots replace the K slots; unpacking X forms the gk correlation
// G*conj(X).  One spectrum's slots are live per transform, as in the forward.
template <int LOGN1, int LOGN2>
__global__ __launch_bounds__(RowCfg<LOGN2>::T) __attribute__((amdgpu_waves_per_eu(4))) void row_bwd1_kernel(
    float2* __restrict__ wsg, const float2* __restrict__ wsx, float2* __restrict__ wsk, int H,
    const float2* __restrict__ tw) {
  using C = RowCfg<LOGN2>;
  using RS = RowSlots<LOGN1, LOGN2>;
  constexpr int64_t N = int64_t(1) << (LOGN1 + LOGN2);
  __shared__ float2 lds[C::TILE_P];
  const int q = blockIdx.x % ((1 << LOGN1) / 2);
  const int h = blockIdx.x / ((1 << LOGN1) / 2);
  float2 sA[C::SLOTS], sB[C::SLOTS];  // K slots, then G slots
  if constexpr (LOGN2 == kRegPairLogN2) {
    constexpr int N1 = 1 << LOGN1;
    const int ra = q, rb = (q == 0) ? N1 / 2 : N1 - q;
    const int tl = opaque_tid();
    float2 v[4][4];
    auto head = [&](const float2* sig) {
      auto ld = [&](int m, int n) -> float2 { return ws_load(sig + int64_t(m == 0 ? ra : rb) * C::N2 + n); };
      rows1024_fwd_head<2, C::T>(lds, ld, tw);
    };
    head(wsk + int64_t(h) * N);
    regpair_fwd_slots<LOGN1, false>(lds, q, tl, tw, v, [&](int i, bool, float2& A, float2& Bc) {
      sA[i] = A;
      sB[i] = Bc;
    });
    float2* sigg = wsg + int64_t(h) * N;
    head(sigg);
    // gx slots G conj K; the G slots replace the K slots
    regpair_fwd_slots<LOGN1, true>(lds, q, tl, tw, v, [&](int i, bool s0, float2& A, float2& Bc) {
      const float2 ga = A, gb = Bc;
      A = slot_mulc(s0, ga, sA[i]);
      Bc = cmulc(gb, sB[i]);
      sA[i] = ga;
      sB[i] = gb;
    });
    {
      RowStore<C::N2> st{sigg, ra, rb};
      regpair_inverse<2, C::T>(lds, lds, q, tl, v, st, tw);
    }
    head(wsx + int64_t(h) * N);
    // gk slots G conj X
    regpair_fwd_slots<LOGN1, true>(lds, q, tl, tw, v, [&](int i, bool s0, float2& A, float2& Bc) {
      A = slot_mulc(s0, sA[i], A);
      Bc = cmulc(sB[i], Bc);
    });
    RowStore<C::N2> st{wsk + int64_t(h) * N, ra, rb};
    regpair_inverse<2, C::T>(lds, lds, q, tl, v, st, tw);
    return;
  }
  row_pair_fft<LOGN1, LOGN2>(lds, wsk + int64_t(h) * N, q, tw);
  {
    const RS rs(q, tw);
#pragma unroll
    for (int i = 0; i < C::SLOTS; ++i) {
      NSQ_SLOT_FENCE();
      row_unpack(lds, rs, i, sA[i], sB[i]);
    }
  }
  __syncthreads();
  float2* sigg = wsg + int64_t(h) * N;
  row_pair_fft<LOGN1, LOGN2>(lds, sigg, q, tw);
  {
    const RS rs(q, tw);
#pragma unroll
    for (int i = 0; i < C::SLOTS; ++i) {
      NSQ_SLOT_FENCE();
      float2 GA, GB;
      row_unpack(lds, rs, i, GA, GB);
      row_repack(lds, rs, i, slot_mulc(rs.s0(i), GA, sA[i]), cmulc(GB, sB[i]));
      sA[i] = GA;
      sB[i] = GB;
    }
  }
  __syncthreads();
  row_pair_ifft_store<LOGN1, LOGN2>(lds, sigg, q, tw);
  row_pair_fft<LOGN1, LOGN2>(lds, wsx + int64_t(h) * N, q, tw);
  {
    const RS rs(q, tw);
#pragma unroll
    for (int i = 0; i < C::SLOTS; ++i) {
      NSQ_SLOT_FENCE();
      float2 XA, XB;
      row_unpack(lds, rs, i, XA, XB);
      row_repack(lds, rs, i, slot_mulc(rs.s0(i), sA[i], XA), cmulc(sB[i], XB));
    }
  }
  __syncthreads();
  row_pair_ifft_store<LOGN1, LOGN2>(lds, wsk + int64_t(h) * N, q, tw);
}

// ===========================================================================
// Host launchers
// ===========================================================================
// Largest B*H that the forward runs on fused_fwd_pair_kernel (M == 1 lengths,
// no fold).  FFT length 16384 (radix-16 pair kernel): as many rows as one
// round of pair workgroups covers, 256 CUs times the pair tiles that fit a
// CU's 160 KB of LDS (256 rows; measured, one-transform -> pair kernel: H=256
// 29.4 -> 23.2 us, H=512 39.4 -> 43.1 us).  FFT lengths 4096 and 8192
// (radix-8 pair kernel): 1536 rows.  Measured at B=2 (kernel time, one-
// transform -> pair kernel): length 8192, 256 rows 19.5 -> 13.5 us, 512 22.1
// -> 20.0, 768 25.8 -> 26.3, 1024 38.4 -> 33.6, 1536 50.1 -> 48.5; length
// 4096, 256 rows 16.2 -> 9.0 us, 1024 20.5 -> 17.8, 1536 25.7 -> 23.7, 2048
// 28.7 -> 29.7.  NSQ_1D_PAIR_MAX_ROWS overrides the bound for every length (0
// turns the pair kernel off).
template <int LOGN>
inline int64_t fused_pair_max_rows() {
  static const int64_t env = [] {
    const char* e = std::getenv("NSQ_1D_PAIR_MAX_ROWS");
    return e ? int64_t(std::atoll(e)) : int64_t(-1);
  }();
  if (env >= 0) return env;
  if constexpr (LOGN <= 12) return 1536;
  constexpr int lds = 2 * FusedCfg<LOGN>::SP * int(sizeof(float2));
  constexpr int per_cu = (160 * 1024) / lds;
  return int64_t(256) * (per_cu < 1 ? 1 : per_cu);
}

// kfilm: per-sample filters [B*H, K]; one image per workgroup.
template <int LOGN, int DT>
static void launch_fused_fwd(const Plan1D& p, const void* x, const float* k, const void* s, void* y, int B, int H,
                             int L, int K, int kfilm, const float2* tw, hipStream_t st) {
  using C = FusedCfg<LOGN>;
  using ET = typename Elem<DT>::T;
  if constexpr (C::M == 1) {
    if (!p.fold && int64_t(H) * B <= fused_pair_max_rows<LOGN>()) {
      // radix-8 passes up to N = 4096 (2 N / 8 <= 1024 threads): twice the waves of the radix-16 form to cover
      // the pass latencies of a grid of one round (FFT length 8192 at B=2 H=128: 17.6 -> 15.7 us per step)
      constexpr int LOGR = LOGN <= 12 ? 3 : 4;
      hipLaunchKernelGGL((fused_fwd_pair_kernel<LOGN, DT, LOGR>), dim3(H, B), dim3(2 * (C::N >> LOGR)), 0, st,
                         (const ET*)x, k, (const ET*)s, (ET*)y, H, L, K, tw, kfilm);
      return;
    }
  }
  const int gh = int(ceil_div(H, C::M));
  int nb = int(ceil_div(2048, gh));
  nb = nb < 1 ? 1 : (nb > B ? B : nb);
  const int bpw = kfilm ? 1 : int(ceil_div(B, nb));
  nb = int(ceil_div(B, bpw));
  dim3 grid(gh, nb);
  if (p.fold)
    hipLaunchKernelGGL((fused_fwd_kernel<LOGN, DT, true>), grid, dim3(C::T), 0, st, (const ET*)x, k, (const ET*)s,
                       (ET*)y, B, H, L, K, bpw, tw, 0, kfilm, -1, GateArgs{});
  else
    hipLaunchKernelGGL((fused_fwd_kernel<LOGN, DT, false>), grid, dim3(C::T), 0, st, (const ET*)x, k, (const ET*)s,
                       (ET*)y, B, H, L, K, bpw, tw, 0, kfilm, -1, GateArgs{});
}

template <int LOGN, int DT>
static void launch_fused_bwd(const Plan1D& p, const void* g, const void* x, const float* k, const void* s, void* gx,
                             float* gk, float* gs, int B, int H, int L, int K, int kfilm, const float2* tw,
                             hipStream_t st) {
  using C = FusedCfg<LOGN>;
  using ET = typename Elem<DT>::T;
  dim3 grid(unsigned(ceil_div(H, C::M)), unsigned(kfilm ? B : 1));
  if (p.fold)
    hipLaunchKernelGGL((fused_bwd_kernel<LOGN, DT, true>), grid, dim3(C::T), 0, st, (const ET*)g, (const ET*)x, k,
                       (const ET*)s, (ET*)gx, gk, gs, B, H, L, K, tw, 0, kfilm, -1, 1.f);
  else
    hipLaunchKernelGGL((fused_bwd_kernel<LOGN, DT, false>), grid, dim3(C::T), 0, st, (const ET*)g, (const ET*)x, k,
                       (const ET*)s, (ET*)gx, gk, gs, B, H, L, K, tw, 0, kfilm, -1, 1.f);
}

// Gated (Hyena) fused plan: the GATE variant of the fused forward kernel.
template <int LOGN, int DT>
static void launch_gated_fused_fwd(const Plan1D& p, const void* q, const float* k, const void* s, void* y, int B,
                                   int H, int L, int K, int kfilm, const GateArgs& ga, const float2* tw,
                                   hipStream_t st) {
  using C = FusedCfg<LOGN>;
  using ET = typename Elem<DT>::T;
  const int gh = int(ceil_div(H, C::M));
  int nb = int(ceil_div(2048, gh));
  nb = nb < 1 ? 1 : (nb > B ? B : nb);
  const int bpw = kfilm ? 1 : int(ceil_div(B, nb));
  nb = int(ceil_div(B, bpw));
  const dim3 grid(gh, nb);
  if (p.fold)
    hipLaunchKernelGGL((fused_fwd_kernel<LOGN, DT, true, false, true>), grid, dim3(C::T), 0, st, (const ET*)q, k,
                       (const ET*)s, (ET*)y, B, H, L, K, bpw, tw, 0, kfilm, -1, ga);
  else
    hipLaunchKernelGGL((fused_fwd_kernel<LOGN, DT, false, false, true>), grid, dim3(C::T), 0, st, (const ET*)q, k,
                       (const ET*)s, (ET*)y, B, H, L, K, bpw, tw, 0, kfilm, -1, ga);
}

// Shifted 1D convs on the fused plan, output rolled by -c through the filter
// ramp (circ_ramp); kfilm = per-image filters [B, H, K] (one image per
// workgroup).  zpad = false: circular conv at FFT length L = 2N (or its
// periodic extension), c = (K-1)/2.  zpad = true: the zero-padded "same" conv,
// x zero-extended from L to 2N >= L + ceil(K/2), c = K/2 (no sample wraps
// into the output window [0, L), see nsq_mixed_fftconv1d_fwd).
template <int LOGN, int DT>
static void launch_circ_fwd(const void* x, const float* k, const void* s, void* y, int B, int H, int L, int K,
                            int kfilm, int c, bool zpad, const float2* tw, hipStream_t st) {
  using C = FusedCfg<LOGN>;
  using ET = typename Elem<DT>::T;
  const int gh = int(ceil_div(H, C::M));
  int bpw = 1;
  if (!kfilm) {
    int nb = int(ceil_div(2048, gh));
    nb = nb < 1 ? 1 : (nb > B ? B : nb);
    bpw = int(ceil_div(B, nb));
  }
  const dim3 grid(gh, unsigned(ceil_div(B, bpw)));
  // a period shorter than the transform: periodic extension (L = 1, K = 1: plain zero padding is exact)
  const int wm = (!zpad && L > 1 && L < 2 * C::N) ? L - 1 : -1;
  hipLaunchKernelGGL((fused_fwd_kernel<LOGN, DT, false, true>), grid, dim3(C::T), 0, st, (const ET*)x, k,
                     (const ET*)s, (ET*)y, B, H, L, K, bpw, tw, c, kfilm, wm, GateArgs{});
}

template <int LOGN, int DT>
static void launch_circ_bwd(const void* g, const void* x, const float* k, const void* s, void* gx, float* gk,
                            float* gs, int B, int H, int L, int K, int kfilm, int c, bool zpad, const float2* tw,
                            hipStream_t st) {
  using C = FusedCfg<LOGN>;
  using ET = typename Elem<DT>::T;
  const dim3 grid(unsigned(ceil_div(H, C::M)), unsigned(kfilm ? B : 1));
  const int wm = (!zpad && L > 1 && L < 2 * C::N) ? L - 1 : -1;
  hipLaunchKernelGGL((fused_bwd_kernel<LOGN, DT, false, true>), grid, dim3(C::T), 0, st, (const ET*)g,
                     (const ET*)x, k, (const ET*)s, (ET*)gx, gk, gs, B, H, L, K, tw, c, kfilm, wm,
                     wm == -1 ? 1.f : float(L) / float(2 * C::N));
}

// Workspace layout of the 4-step plan (rows of N complex64; NK = H, or B*H for
// per-sample filters):
//   [0, BH)            column-transformed x  (X')
//   [BH, BH+NK)        column-transformed k  (K')
//   [BH+NK, 2BH+NK)    forward: inverse-row product (Y') when `save`; backward: G'
// With `save`, X' and K' survive the forward so the backward can reuse them.
// Per-sample filters run the row passes as one image of B*H channels (every
// row then has its own filter row); the epilogues still index the shortcut by
// row % H.
// Column-pass launches; `al` selects the aligned-pair row access.
template <int LOGN1, int LOGN, int DT>
static void launch_col_fwd(RealRows<DT> src, int64_t rows, float2* out, const float2* tw, hipStream_t st) {
  const int64_t nb = rows * ((int64_t(1) << (LOGN - LOGN1)) / ColCfg<LOGN1>::M);
  const unsigned grid = unsigned(ceil_div(nb, kColTilesPerWG));
  auto go = [&](auto al, auto half) {
    hipLaunchKernelGGL((col_fwd_kernel<LOGN1, LOGN, DT, decltype(al)::value, decltype(half)::value>), dim3(grid),
                       dim3(ColCfg<LOGN1>::T), 0, st, src, out, tw, nb);
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  const bool al = pairs_aligned<DT>(src.p, src.stride, src.valid);
  if (src.valid <= (int64_t(1) << LOGN))  // packed samples [N/2, N) all zero
    al ? go(T_{}, T_{}) : go(F_{}, T_{});
  else
    al ? go(T_{}, F_{}) : go(F_{}, F_{});
}

template <int LOGN1, int LOGN, int DT>
static void launch_col_inv_out(const float2* ws, const void* aux, const void* s, void* out, int64_t rows, int H,
                               int L, const float2* tw, hipStream_t st) {
  using ET = typename Elem<DT>::T;
  const int64_t nb = rows * ((int64_t(1) << (LOGN - LOGN1)) / ColCfg<LOGN1>::M);
  if (pairs_aligned<DT>(out, L, L) && pairs_aligned<DT>(aux, L, L))
    hipLaunchKernelGGL((col_inv_out_kernel<LOGN1, LOGN, DT, true>), dim3(unsigned(nb)), dim3(ColCfg<LOGN1>::T), 0,
                       st, ws, (const ET*)aux, (const ET*)s, (ET*)out, H, L, tw);
  else
    hipLaunchKernelGGL((col_inv_out_kernel<LOGN1, LOGN, DT, false>), dim3(unsigned(nb)), dim3(ColCfg<LOGN1>::T), 0,
                       st, ws, (const ET*)aux, (const ET*)s, (ET*)out, H, L, tw);
}

template <int LOGN1, int LOGN>
static void launch_col_inv_gk(const float2* ws, float* gk, float* gs, int H, int K, const float2* tw,
                              hipStream_t st) {
  const int64_t nb = int64_t(H) * ((int64_t(1) << (LOGN - LOGN1)) / ColCfg<LOGN1>::M);
  if (pairs_aligned<NSQ_DTYPE_F32>(gk, K, K))
    hipLaunchKernelGGL((col_inv_gk_kernel<LOGN1, LOGN, true>), dim3(unsigned(nb)), dim3(ColCfg<LOGN1>::T), 0, st, ws,
                       gk, gs, K, tw);
  else
    hipLaunchKernelGGL((col_inv_gk_kernel<LOGN1, LOGN, false>), dim3(unsigned(nb)), dim3(ColCfg<LOGN1>::T), 0, st,
                       ws, gk, gs, K, tw);
}

// K > L+1 on the 4-step plan.  The reference's circular conv at length 2L
// wraps: y[n] = sum_j k[j] x[(n - j) mod 2L], n < L, K <= 2L.  At the plan's
// FFT length F >= 3L the same sums come out of the plain circular products
// when one operand carries a copy of itself at the wrap offset:
//  * forward: x_ext = x on [0, L) and x[t - (F - 2L)] on [F - 2L, F - L):
//    for j > n, (n - j) mod F = F + n - j lands in the copy exactly when
//    n - j + 2L is in [0, L), i.e. the wrapped term x[n - j + 2L];
//  * backward: g_ext = g on [0, L) and g[t - 2L] on [2L, 3L) (the adjoint
//    fold of the fused plan): gx[m] = sum_t g_ext[t] k[t - m] and gk[j] =
//    sum_t g_ext[t] x[t - j] gain the wrapped terms g[n] k[n + 2L - m] and
//    g[n] x[n + 2L - j].
// The windows are disjoint (offset >= L) and every other index of [0, F) is
// beyond both supports, so nothing aliases.  The copy goes to one workspace
// block of B*H rows of F values (it fits: a block is B*H*N complex values).
template <int DT>
__global__ __launch_bounds__(256) void fold_rows_kernel(const typename Elem<DT>::T* __restrict__ src,
                                                        typename Elem<DT>::T* __restrict__ dst, int64_t rows, int L,
                                                        int F, int off) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows * F) return;
  const int64_t r = i / F;
  const int t = int(i - r * F);
  const int u = t < L ? t : t - off;
  Elem<DT>::store(dst, i, (u >= 0 && u < L) ? Elem<DT>::load(src, r * L + u) : 0.f);
}

template <int DT>
static const void* launch_fold_rows(const void* src, float2* block, int64_t rows, int L, int F, int off,
                                    hipStream_t st) {
  using ET = typename Elem<DT>::T;
  const int64_t n = rows * F;
  hipLaunchKernelGGL((fold_rows_kernel<DT>), dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, (const ET*)src,
                     (ET*)block, rows, L, F, off);
  return block;
}

// k == nullptr: the filter's column transforms are already in the k block (the SIREN path forms them from the
// transformed activation rows).
template <int LOGN1, int LOGN2, int DT>
static void launch_4step_fwd(const void* x, const float* k, const void* s, void* y, int B, int H, int L, int K,
                             int kfilm, float2* ws, bool save, const float2* tw, hipStream_t st, bool fold) {
  constexpr int LOGN = LOGN1 + LOGN2;
  constexpr int64_t N = int64_t(1) << LOGN;
  constexpr int F = int(2 * N);
  using ET = typename Elem<DT>::T;
  const int64_t BH = int64_t(B) * H, NK = kfilm ? BH : H;
  const int rb = kfilm ? 1 : B, rh = kfilm ? int(BH) : H;  // row-pass images and channels
  float2* wsx = ws;
  float2* wsk = ws + BH * N;
  float2* wsy = save ? ws + (BH + NK) * N : wsx;
  if (fold) {  // x with its wrap copy at F - 2L, in the block after x and k (save is off with a fold)
    const void* xe = launch_fold_rows<DT>(x, ws + (BH + NK) * N, BH, L, F, F - 2 * L, st);
    launch_col_fwd<LOGN1, LOGN, DT>(RealRows<DT>{(const ET*)xe, F, F}, BH, wsx, tw, st);
  } else {
    launch_col_fwd<LOGN1, LOGN, DT>(RealRows<DT>{(const ET*)x, L, L}, BH, wsx, tw, st);
  }
  if (k) launch_col_fwd<LOGN1, LOGN, NSQ_DTYPE_F32>(RealRows<NSQ_DTYPE_F32>{k, K, K}, NK, wsk, tw, st);
  hipLaunchKernelGGL((row_fwd_kernel<LOGN1, LOGN2>), dim3(unsigned(rh) * ((1 << LOGN1) / 2)), dim3(RowCfg<LOGN2>::T),
                     0, st, (const float2*)wsx, (const float2*)wsk, wsy, rb, rh, tw);
  launch_col_inv_out<LOGN1, LOGN, DT>(wsy, x, s, y, BH, H, L, tw, st);
}

// k == nullptr: the k block already holds the filter's column transforms (recomputing x's only, when there is
// no forward state).  gk == nullptr: the filter gradient's spectrum is left in the k block (the SIREN path reads
// it there) and gs is not formed.
template <int LOGN1, int LOGN2, int DT>
static void launch_4step_bwd(const void* g, const void* x, const float* k, const void* s, void* gx, float* gk,
                             float* gs, int B, int H, int L, int K, int kfilm, float2* ws, bool fwd_state,
                             const float2* tw, hipStream_t st, bool fold) {
  constexpr int LOGN = LOGN1 + LOGN2;
  constexpr int64_t N = int64_t(1) << LOGN;
  constexpr int F = int(2 * N);
  using ET = typename Elem<DT>::T;
  const int64_t BH = int64_t(B) * H, NK = kfilm ? BH : H;
  const int rb = kfilm ? 1 : B, rh = kfilm ? int(BH) : H;  // row-pass images and channels
  float2* wsx = ws;
  float2* wsk = ws + BH * N;
  float2* wsg = ws + (BH + NK) * N;
  if (fold) {  // g with its adjoint copy at 2L, in the block after g; the forward's x block held x's copy: redo x
    const void* ge = launch_fold_rows<DT>(g, ws + (2 * BH + NK) * N, BH, L, F, 2 * L, st);
    launch_col_fwd<LOGN1, LOGN, DT>(RealRows<DT>{(const ET*)ge, F, F}, BH, wsg, tw, st);
    fwd_state = false;
  } else {
    launch_col_fwd<LOGN1, LOGN, DT>(RealRows<DT>{(const ET*)g, L, L}, BH, wsg, tw, st);
  }
  if (!fwd_state) {
    launch_col_fwd<LOGN1, LOGN, DT>(RealRows<DT>{(const ET*)x, L, L}, BH, wsx, tw, st);
    if (k) launch_col_fwd<LOGN1, LOGN, NSQ_DTYPE_F32>(RealRows<NSQ_DTYPE_F32>{k, K, K}, NK, wsk, tw, st);
  }
  if (rb == 1)
    hipLaunchKernelGGL((row_bwd1_kernel<LOGN1, LOGN2>), dim3(unsigned(rh) * ((1 << LOGN1) / 2)),
                       dim3(RowCfg<LOGN2>::T), 0, st, wsg, (const float2*)wsx, wsk, rh, tw);
  else
    hipLaunchKernelGGL((row_bwd_kernel<LOGN1, LOGN2>), dim3(unsigned(rh) * ((1 << LOGN1) / 2)),
                       dim3(RowCfg<LOGN2>::T), 0, st, wsg, (const float2*)wsx, wsk, rb, rh, tw);
  launch_col_inv_out<LOGN1, LOGN, DT>(wsg, g, s, gx, BH, H, L, tw, st);
  if (gk) launch_col_inv_gk<LOGN1, LOGN>(wsk, gk, gs, int(NK), K, tw, st);
}

// Shifted convs (circular, or zero-padded "same") beyond the fused plan, on
// the 4-step plan at FFT length F = 2N.  The shift is moved into a rolled copy
// of one operand (shift_rows_kernel): the forward transforms xr[t] = x[(t + c)
// mod P] and the backward gr[t] = g[(t - c) mod P] (P = L circular, F zero-
// padded; indices >= L read zero), so the plain 4-step circular products give
//   y[i]  = sum_j k[j] xr[(i - j) mod F] = sum_j k[j] x[i + c - j],
//   gx[i] = sum_t gr[t] k[(t - i) mod F],  gk[j] = sum_t gr[t] x[(t - j) mod F],
// and the shortcut terms read the unshifted x and g; the shortcut gradient
// sum_n g[n] x[n] = sum_t gr[t] x[t - c] is the filter gradient's lag c.
// Zero-padded: F >= L + ceil(K/2) keeps every wrapped index out of the window
// (no aliasing).
template <int DT>
__global__ __launch_bounds__(256) void shift_rows_kernel(const typename Elem<DT>::T* __restrict__ src,
                                                         typename Elem<DT>::T* __restrict__ dst, int64_t rows, int L,
                                                         int F, int off, int period) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows * F) return;
  const int64_t r = i / F;
  const int t = int(i - r * F);
  int idx = (t + off) % period;
  if (idx < 0) idx += period;
  Elem<DT>::store(dst, i, idx < L ? Elem<DT>::load(src, r * L + idx) : 0.f);
}

template <int UNUSED = 0>  // a template: one definition across the per-dtype translation units
__global__ __launch_bounds__(256) void lag_gather_kernel(const float* __restrict__ gk, float* __restrict__ gs,
                                                         int64_t rows, int K, int c) {
  const int64_t r = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (r < rows) gs[r] = gk[r * K + c];
}

template <int LOGN1, int LOGN2, int DT>
static void launch_4step_shift_fwd(const void* xr, const void* x, const float* k, const void* s, void* y, int B,
                                   int H, int L, int K, int kfilm, float2* ws, const float2* tw, hipStream_t st) {
  constexpr int LOGN = LOGN1 + LOGN2;
  constexpr int64_t N = int64_t(1) << LOGN;
  using ET = typename Elem<DT>::T;
  const int64_t BH = int64_t(B) * H, NK = kfilm ? BH : H;
  const int rb = kfilm ? 1 : B, rh = kfilm ? int(BH) : H;
  float2* wsx = ws;
  float2* wsk = ws + BH * N;
  launch_col_fwd<LOGN1, LOGN, DT>(RealRows<DT>{(const ET*)xr, 2 * N, 2 * N}, BH, wsx, tw, st);
  launch_col_fwd<LOGN1, LOGN, NSQ_DTYPE_F32>(RealRows<NSQ_DTYPE_F32>{k, K, K}, NK, wsk, tw, st);
  hipLaunchKernelGGL((row_fwd_kernel<LOGN1, LOGN2>), dim3(unsigned(rh) * ((1 << LOGN1) / 2)), dim3(RowCfg<LOGN2>::T),
                     0, st, (const float2*)wsx, (const float2*)wsk, wsx, rb, rh, tw);
  launch_col_inv_out<LOGN1, LOGN, DT>(wsx, x, s, y, BH, H, L, tw, st);
}

template <int LOGN1, int LOGN2, int DT>
static void launch_4step_shift_bwd(const void* gr, const void* g, const void* x, const float* k, const void* s,
                                   void* gx, float* gk, float* gs, int B, int H, int L, int K, int kfilm, int c,
                                   float2* ws, const float2* tw, hipStream_t st) {
  constexpr int LOGN = LOGN1 + LOGN2;
  constexpr int64_t N = int64_t(1) << LOGN;
  using ET = typename Elem<DT>::T;
  const int64_t BH = int64_t(B) * H, NK = kfilm ? BH : H;
  const int rb = kfilm ? 1 : B, rh = kfilm ? int(BH) : H;
  float2* wsx = ws;
  float2* wsk = ws + BH * N;
  float2* wsg = ws + (BH + NK) * N;
  launch_col_fwd<LOGN1, LOGN, DT>(RealRows<DT>{(const ET*)gr, 2 * N, 2 * N}, BH, wsg, tw, st);
  launch_col_fwd<LOGN1, LOGN, DT>(RealRows<DT>{(const ET*)x, L, L}, BH, wsx, tw, st);
  launch_col_fwd<LOGN1, LOGN, NSQ_DTYPE_F32>(RealRows<NSQ_DTYPE_F32>{k, K, K}, NK, wsk, tw, st);
  if (rb == 1)
    hipLaunchKernelGGL((row_bwd1_kernel<LOGN1, LOGN2>), dim3(unsigned(rh) * ((1 << LOGN1) / 2)),
                       dim3(RowCfg<LOGN2>::T), 0, st, wsg, (const float2*)wsx, wsk, rh, tw);
  else
    hipLaunchKernelGGL((row_bwd_kernel<LOGN1, LOGN2>), dim3(unsigned(rh) * ((1 << LOGN1) / 2)),
                       dim3(RowCfg<LOGN2>::T), 0, st, wsg, (const float2*)wsx, wsk, rb, rh, tw);
  launch_col_inv_out<LOGN1, LOGN, DT>(wsg, g, s, gx, BH, H, L, tw, st);
  launch_col_inv_gk<LOGN1, LOGN>(wsk, gk, nullptr, int(NK), K, tw, st);
  if (gs)
    hipLaunchKernelGGL(lag_gather_kernel<0>, dim3(unsigned(ceil_div(NK, 256))), dim3(256), 0, st, (const float*)gk, gs, NK,
                       K, c);
}

template <int DT>
static void launch_shift_rows(const void* src, void* dst, int64_t rows, int L, int F, int off, int period,
                              hipStream_t st) {
  using ET = typename Elem<DT>::T;
  const int64_t n = rows * F;
  hipLaunchKernelGGL((shift_rows_kernel<DT>), dim3(unsigned(ceil_div(n, 256))), dim3(256), 0, st, (const ET*)src,
                     (ET*)dst, rows, L, F, off, period);
}

// Runtime -> compile-time dispatch helpers.
template <template <int> class F, int LO, int HI, class... A>
static bool dispatch_int(int v, A&&... a) {
  if constexpr (LO > HI) {
    return false;
  } else {
    if (v == LO) {
      F<LO>::run(static_cast<A&&>(a)...);
      return true;
    }
    return dispatch_int<F, LO + 1, HI>(v, static_cast<A&&>(a)...);
  }
}

template <int DT>
struct FusedFwd {
  template <int LOGN>
  struct At {
    template <class... A>
    static void run(A&&... a) {
      launch_fused_fwd<LOGN, DT>(static_cast<A&&>(a)...);
    }
  };
};

template <int DT>
struct FusedBwd {
  template <int LOGN>
  struct At {
    template <class... A>
    static void run(A&&... a) {
      launch_fused_bwd<LOGN, DT>(static_cast<A&&>(a)...);
    }
  };
};

template <int DT>
struct GatedFused {
  template <int LOGN>
  struct At {
    template <class... A>
    static void run(A&&... a) {
      launch_gated_fused_fwd<LOGN, DT>(static_cast<A&&>(a)...);
    }
  };
};

template <int DT, bool BWD>
struct CircFused {
  template <int LOGN>
  struct At {
    template <class... A>
    static void run(A&&... a) {
      if constexpr (BWD)
        launch_circ_bwd<LOGN, DT>(static_cast<A&&>(a)...);
      else
        launch_circ_fwd<LOGN, DT>(static_cast<A&&>(a)...);
    }
  };
};

template <int DT, bool BWD>
struct FourStepShift {
  template <int LOGN>
  struct At {
    static constexpr int L1 = split_log_n1(LOGN);
    static constexpr int L2 = LOGN - L1;
    template <class... A>
    static void run(A&&... a) {
      if constexpr (BWD)
        launch_4step_shift_bwd<L1, L2, DT>(static_cast<A&&>(a)...);
      else
        launch_4step_shift_fwd<L1, L2, DT>(static_cast<A&&>(a)...);
    }
  };
};

// 4-step instantiations: logN in [14, kMaxLogN] split by split_log_n1.
template <int DT, bool BWD>
struct FourStep {
  template <int LOGN>
  struct At {
    static constexpr int L1 = split_log_n1(LOGN);
    static constexpr int L2 = LOGN - L1;
    template <class... A>
    static void run(A&&... a) {
      if constexpr (BWD)
        launch_4step_bwd<L1, L2, DT>(static_cast<A&&>(a)...);
      else
        launch_4step_fwd<L1, L2, DT>(static_cast<A&&>(a)...);
    }
  };
};

// Per-dtype entry used by the C ABI; explicitly instantiated once per dtype in
// fftconv1d_<dtype>.hip so the three instantiation sets compile in parallel.
// kfilm: per-sample filters (k, gk: [B*H, K]; gs: [B*H] partials).
template <int DT>
bool run_fwd(const Plan1D& p, const void* x, const float* k, const void* s, void* y, int B, int H, int L, int K,
             int kfilm, float2* ws, bool save, const float2* tw, hipStream_t st) {
  if (p.fused)
    return dispatch_int<FusedFwd<DT>::template At, 3, 13>(p.logN, p, x, k, s, y, B, H, L, K, kfilm, tw, st);
  return dispatch_int<FourStep<DT, false>::template At, 14, kMaxLogN>(p.logN, x, k, s, y, B, H, L, K, kfilm, ws,
                                                                 save && !p.fold, tw, st, p.fold);
}

template <int DT>
bool run_bwd(const Plan1D& p, const void* g, const void* x, const float* k, const void* s, void* gx, float* gk,
             float* gs, int B, int H, int L, int K, int kfilm, float2* ws, bool fwd_state, const float2* tw,
             hipStream_t st) {
  if (p.fused)
    return dispatch_int<FusedBwd<DT>::template At, 3, 13>(p.logN, p, g, x, k, s, gx, gk, gs, B, H, L, K, kfilm, tw,
                                                          st);
  return dispatch_int<FourStep<DT, true>::template At, 14, kMaxLogN>(p.logN, g, x, k, s, gx, gk, gs, B, H, L, K, kfilm, ws,
                                                                fwd_state && !p.fold, tw, st, p.fold);
}

// Column passes of float rows on their own, at the 4-step plan of FFT length 2^(logN + 1) (logN in
// [14, kMaxLogN]): rows of `valid` samples (row stride `stride`) into the plan's column transforms (N complex
// values per row), and back: the inverse column pass of `rows` blocks into float rows of K samples (row stride
// K; out[r][0] also to gs[r] when gs != nullptr), scaled by 1/N like the filter gradient.
template <bool INV>
struct ColRows {
  template <int LOGN>
  struct At {
    static constexpr int L1 = split_log_n1(LOGN);
    static void run(const float* src, int64_t stride, int64_t valid, const float2* spec, float* out, float* gs,
                    int64_t rows, int K, float2* dst, const float2* tw, hipStream_t st) {
      if constexpr (INV)
        launch_col_inv_gk<L1, LOGN>(spec, out, gs, int(rows), K, tw, st);
      else
        launch_col_fwd<L1, LOGN, NSQ_DTYPE_F32>(RealRows<NSQ_DTYPE_F32>{src, stride, valid}, rows, dst, tw, st);
    }
  };
};

template <int UNUSED>  // a template: one definition (fftconv1d_f32.hip) across the translation units
bool run_col_fwd_rows(int logN, const float* src, int64_t stride, int64_t valid, int64_t rows, float2* out,
                      const float2* tw, hipStream_t st) {
  return dispatch_int<ColRows<false>::template At, 14, kMaxLogN>(logN, src, stride, valid, nullptr, nullptr,
                                                                 nullptr, rows, 0, out, tw, st);
}

template <int UNUSED>
bool run_col_inv_rows(int logN, const float2* spec, float* out, float* gs, int64_t rows, int K, const float2* tw,
                      hipStream_t st) {
  return dispatch_int<ColRows<true>::template At, 14, kMaxLogN>(logN, nullptr, int64_t(0), int64_t(0), spec, out,
                                                                gs, rows, K, nullptr, tw, st);
}

// Whether the fused plan's forward runs the gated kernel (gates in its first pass and epilogue) rather than the
// gate kernels around the plain fused kernel.  Both round the same way (same bits).  The gated kernel adds four
// operand streams (q and k in place of z, then q, k and v again in its epilogue, y1 beside y) to a kernel that
// holds one or two workgroups per CU, so it only pays where launches dominate: measured on MI355X (bf16 fwd),
// B=4 H=1024 L=8192 0.436 ms against 0.351 ms for the three kernels, B=1 H=1024 L=8192 0.110 / 0.100 ms,
// B=2 H=256 L=4096 0.037 / 0.038 ms, B=1 H=64 L=2048 0.031 / 0.038 ms.  Below 2^22 elements the gated kernel;
// NSQ_1D_GATES_FUSED=0 / 1 forces either.
inline bool gates_fused_1d(const Plan1D& p, int64_t elems) {
  static const int force = [] {
    const char* e = std::getenv("NSQ_1D_GATES_FUSED");
    return e ? (e[0] == '0' ? 0 : 1) : -1;
  }();
  if (!p.fused || force == 0) return false;
  return force == 1 || elems < (int64_t(1) << 22);
}

// Gated (Hyena) causal conv.  Forward, fused plan: one gated kernel for small calls (gates_fused_1d), else, and
// on the 4-step plan, the elementwise gate kernels around the plain conv, with the
// intermediates in `gws` (forward: z [, y1 when the caller keeps none];
// backward: z, dy1, dz), the conv's own workspace in `ws`.
// Forward: y = (conv(z) + s z) act2(v), z = q act1(k_gate); ga.y1 (optional)
// receives conv(z) + s z.  Backward: needs ga.y1.
template <int DT>
bool run_gated_fwd(const Plan1D& p, const void* q, const float* k, const void* s, void* y, int B, int H, int L,
                   int K, int kfilm, const GateArgs& ga, void* gws, float2* ws, const float2* tw, hipStream_t st) {
  if (gates_fused_1d(p, int64_t(B) * H * L))
    return dispatch_int<GatedFused<DT>::template At, 3, 13>(p.logN, p, q, k, s, y, B, H, L, K, kfilm, ga, tw,
                                                                   st);
  using ET = typename Elem<DT>::T;
  const int64_t n = int64_t(B) * H * L;
  const int64_t stride = int64_t(round256(size_t(n) * sizeof(ET)) / sizeof(ET));  // 256-byte aligned sub-buffers
  ET* z = (ET*)gws;
  ET* y1 = ga.y1 ? (ET*)ga.y1 : z + stride;
  launch_gate_ew<DT, GATE_OP_FWD1>(GateEw{q, ga.kg, nullptr, z, nullptr, ga.act1}, n, st);
  if (!run_fwd<DT>(p, z, k, s, y1, B, H, L, K, kfilm, ws, false, tw, st)) return false;
  launch_gate_ew<DT, GATE_OP_FWD2>(GateEw{y1, ga.v, nullptr, y, nullptr, ga.act2}, n, st);
  return true;
}

// The backward runs the elementwise gate kernels around the plain conv adjoint
// for every plan.  A gated fused adjoint (gates in the fused backward kernel's
// loads and epilogue) measured slower on MI355X: with one 139 KB-LDS workgroup
// per CU at FFT length 16384, its five extra operand streams add latency that
// occupancy cannot hide (B=4 D=1024 L=8192 bf16: 0.96 ms against 0.58 ms for
// the plain adjoint plus 0.15 ms of gate kernels), so it is not built.
template <int DT>
bool run_gated_bwd(const Plan1D& p, const void* g, const void* q, const float* k, const void* s, void* dq, float* gk,
                   float* gs, int B, int H, int L, int K, int kfilm, const GateArgs& ga, void* gws, float2* ws,
                   const float2* tw, hipStream_t st) {
  using ET = typename Elem<DT>::T;
  const int64_t n = int64_t(B) * H * L;
  const int64_t stride = int64_t(round256(size_t(n) * sizeof(ET)) / sizeof(ET));  // 256-byte aligned sub-buffers
  ET* z = (ET*)gws;
  ET* dy1 = z + stride;
  ET* dz = dy1 + stride;
  launch_gate_ew<DT, GATE_OP_BWD2>(GateEw{g, ga.v, ga.y1, dy1, ga.dv, ga.act2}, n, st);
  launch_gate_ew<DT, GATE_OP_FWD1>(GateEw{q, ga.kg, nullptr, z, nullptr, ga.act1}, n, st);
  if (!run_bwd<DT>(p, dy1, z, k, s, dz, gk, gs, B, H, L, K, kfilm, ws, false, tw, st)) return false;
  launch_gate_ew<DT, GATE_OP_BWD1>(GateEw{dz, q, ga.kg, dq, ga.dk, ga.act1}, n, st);
  return true;
}

// Circular 1D: logN = max(log2(L), 4) - 1 in [3, 13] (L a power of two <= 16384;
// L < 16 runs at transform length 16 on the periodic extension).
template <int DT>
bool run_circ_fwd(int logN, const void* x, const float* k, const void* s, void* y, int B, int H, int L, int K,
                  int kfilm, int c, bool zpad, const float2* tw, hipStream_t st) {
  return dispatch_int<CircFused<DT, false>::template At, 3, 13>(logN, x, k, s, y, B, H, L, K, kfilm, c, zpad, tw,
                                                                st);
}

template <int DT>
bool run_circ_bwd(int logN, const void* g, const void* x, const float* k, const void* s, void* gx, float* gk,
                  float* gs, int B, int H, int L, int K, int kfilm, int c, bool zpad, const float2* tw,
                  hipStream_t st) {
  return dispatch_int<CircFused<DT, true>::template At, 3, 13>(logN, g, x, k, s, gx, gk, gs, B, H, L, K, kfilm, c,
                                                               zpad, tw, st);
}

// Shifted convs on the 4-step plan (logN in [14, kMaxLogN]); `roll` holds B*H rows of
// F = 2^(logN+1) I/O-dtype values, `ws` the 4-step workspace without `save`.
template <int DT>
bool run_shift4_fwd(int logN, const void* x, const float* k, const void* s, void* y, int B, int H, int L, int K,
                    int kfilm, int c, bool zpad, void* roll, float2* ws, const float2* tw, hipStream_t st) {
  if (logN < 14 || logN > kMaxLogN) return false;
  const int F = 2 << logN;
  launch_shift_rows<DT>(x, roll, int64_t(B) * H, L, F, c, zpad ? F : L, st);
  return dispatch_int<FourStepShift<DT, false>::template At, 14, kMaxLogN>(logN, (const void*)roll, x, k, s, y, B, H, L, K,
                                                                     kfilm, ws, tw, st);
}

template <int DT>
bool run_shift4_bwd(int logN, const void* g, const void* x, const float* k, const void* s, void* gx, float* gk,
                    float* gs, int B, int H, int L, int K, int kfilm, int c, bool zpad, void* roll, float2* ws,
                    const float2* tw, hipStream_t st) {
  if (logN < 14 || logN > kMaxLogN) return false;
  const int F = 2 << logN;
  launch_shift_rows<DT>(g, roll, int64_t(B) * H, L, F, -c, zpad ? F : L, st);
  return dispatch_int<FourStepShift<DT, true>::template At, 14, kMaxLogN>(logN, (const void*)roll, g, x, k, s, gx, gk, gs,
                                                                    B, H, L, K, kfilm, c, ws, tw, st);
}

#define NSQ_DECLARE_FFTCONV1D(DT)                                                                               \
  extern template bool run_fwd<DT>(const Plan1D&, const void*, const float*, const void*, void*, int, int, int, \
                                   int, int, float2*, bool, const float2*, hipStream_t);                        \
  extern template bool run_bwd<DT>(const Plan1D&, const void*, const void*, const float*, const void*, void*,   \
                                   float*, float*, int, int, int, int, int, float2*, bool, const float2*,       \
                                   hipStream_t);                                                                \
  extern template bool run_circ_fwd<DT>(int, const void*, const float*, const void*, void*, int, int, int, int, \
                                        int, int, bool, const float2*, hipStream_t);                            \
  extern template bool run_circ_bwd<DT>(int, const void*, const void*, const float*, const void*, void*, float*, \
                                        float*, int, int, int, int, int, int, bool, const float2*, hipStream_t); \
  extern template bool run_shift4_fwd<DT>(int, const void*, const float*, const void*, void*, int, int, int, int, \
                                          int, int, bool, void*, float2*, const float2*, hipStream_t);          \
  extern template bool run_shift4_bwd<DT>(int, const void*, const void*, const float*, const void*, void*,      \
                                          float*, float*, int, int, int, int, int, int, bool, void*, float2*,   \
                                          const float2*, hipStream_t);                                          \
  extern template bool run_gated_fwd<DT>(const Plan1D&, const void*, const float*, const void*, void*, int, int, \
                                         int, int, int, const GateArgs&, void*, float2*, const float2*,         \
                                         hipStream_t);                                                          \
  extern template bool run_gated_bwd<DT>(const Plan1D&, const void*, const void*, const float*, const void*,     \
                                         void*, float*, float*, int, int, int, int, int, const GateArgs&, void*, \
                                         float2*, const float2*, hipStream_t);

#define NSQ_INSTANTIATE_FFTCONV1D(DT)                                                                    \
  template bool run_fwd<DT>(const Plan1D&, const void*, const float*, const void*, void*, int, int, int, \
                            int, int, float2*, bool, const float2*, hipStream_t);                        \
  template bool run_bwd<DT>(const Plan1D&, const void*, const void*, const float*, const void*, void*,   \
                            float*, float*, int, int, int, int, int, float2*, bool, const float2*,       \
                            hipStream_t);                                                                \
  template bool run_circ_fwd<DT>(int, const void*, const float*, const void*, void*, int, int, int, int, int, \
                                 int, bool, const float2*, hipStream_t);                                    \
  template bool run_circ_bwd<DT>(int, const void*, const void*, const float*, const void*, void*, float*, float*, \
                                 int, int, int, int, int, int, bool, const float2*, hipStream_t);              \
  template bool run_shift4_fwd<DT>(int, const void*, const float*, const void*, void*, int, int, int, int, int, \
                                   int, bool, void*, float2*, const float2*, hipStream_t);                     \
  template bool run_shift4_bwd<DT>(int, const void*, const void*, const float*, const void*, void*, float*,    \
                                   float*, int, int, int, int, int, int, bool, void*, float2*, const float2*,  \
                                   hipStream_t);                                                               \
  template bool run_gated_fwd<DT>(const Plan1D&, const void*, const float*, const void*, void*, int, int, int, int, \
                                  int, const GateArgs&, void*, float2*, const float2*, hipStream_t);             \
  template bool run_gated_bwd<DT>(const Plan1D&, const void*, const void*, const float*, const void*, void*,      \
                                  float*, float*, int, int, int, int, int, const GateArgs&, void*, float2*,       \
                                  const float2*, hipStream_t);

NSQ_DECLARE_FFTCONV1D(NSQ_DTYPE_F32)
NSQ_DECLARE_FFTCONV1D(NSQ_DTYPE_BF16)
NSQ_DECLARE_FFTCONV1D(NSQ_DTYPE_F16)
extern template bool run_col_fwd_rows<0>(int, const float*, int64_t, int64_t, int64_t, float2*, const float2*,
                                         hipStream_t);
extern template bool run_col_inv_rows<0>(int, const float2*, float*, float*, int64_t, int, const float2*,
                                         hipStream_t);

}  // namespace nsq
