// Mixed-radix LDS transforms of length N = 3 * 2^m (or 2^m), gfx950.
//
// The reference pads each 2D/3D axis to F_d = S_d + ceil(K_d / 2) points and
// lets torch.fft choose a mixed-radix plan (nvsubquadratic/ops/fftconv.py:
// 699-702, 774-778); lengths 3 * 2^m (48, 96, 192) are the ones its shapes
// reach.  These transforms are Stockham passes as in fft_core.h, generalised:
//  * the first pass of a 3 * 2^m transform is radix 3 and needs no twiddles;
//    the later passes are radix 2^a with twiddles W_L, L = 3 * 2^b, read from
//    the twiddle table's mixed-radix segments (TwAny);
//  * a pass whose butterfly count is not a multiple of the thread count runs
//    its last round predicated (every index is clamped in range, the stores
//    of the idle lanes are skipped);
//  * LDS tiles are addressed element by element (LdsTile::at), since the
//    compile-time offset trick of fft_core.h relies on power-of-two strides.
// With x zero past two thirds of the axis (S_d <= 2 F_d / 3, i.e. K_d >= S_d,
// the usual Hyena filter), the radix-3 first pass reads only its first two
// inputs (TailZeroLoad): the third is zero padding.
#pragma once

#include "fft_core.h"

namespace nsq {

constexpr bool pow2_len(int n) { return n > 0 && (n & (n - 1)) == 0; }
constexpr bool mixed_len(int n) { return pow2_len(n) || (n % 3 == 0 && pow2_len(n / 3)); }
// Table entry of W_L^0 (layout in nsq_common.h).
constexpr int tw_segment(int L) { return pow2_len(L) ? L : kTwPow2Entries + L; }

// Roots of unity of every length the table holds, through one raw buffer.
struct TwAny {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ explicit TwAny(const float2* tw)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<float2*>(tw), 0, int(kTwEntries * sizeof(float2)),
                                            0x00020000)) {}
  // W_L^m, 0 <= m < L, L a compile-time length.
  template <int L>
  __device__ __forceinline__ float2 root(int m) const {
    static_assert(mixed_len(L) && (pow2_len(L) ? L <= (1 << 14) : L <= (3 << kTw3MaxLog)), "TwAny: length");
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, m * int(sizeof(float2)),
                                                                          tw_segment(L) * int(sizeof(float2)), 0));
  }
  // W_L^m for a run-time length L (2^b or 3 * 2^b within the table), 0 <= m < L.
  __device__ __forceinline__ float2 root_rt(int L, int m) const {
    const int seg = (L & (L - 1)) == 0 ? L : kTwPow2Entries + L;
    return __builtin_bit_cast(float2,
                              __builtin_amdgcn_raw_buffer_load_b64(r, (seg + m) * int(sizeof(float2)), 0, 0));
  }
};

// The roots W_Q^m (m < Q) of one length Q staged in LDS by the workgroup: a
// pass of period L (Q a multiple of L) reads W_L^x = W_Q^{x Q / L} there,
// an LDS read instead of a global one in every pass of every transform.
template <int Q>
struct TwLds {
  const float2* s;
  template <int L>
  __device__ __forceinline__ float2 root(int x) const {
    static_assert(Q % L == 0, "TwLds: the staged length must be a multiple of the pass period");
    return s[x * (Q / L)];
  }
};

// Stages W_Q^m for m < Q into s (all T threads; the caller synchronises).
template <int Q, int T>
__device__ __forceinline__ TwLds<Q> stage_roots(float2* s, const float2* __restrict__ tw) {
  const TwAny ta(tw);
  for (int m = int(threadIdx.x); m < Q; m += T) s[m] = ta.root<Q>(m);
  return TwLds<Q>{s};
}

// In-register DFT of 3 points (natural order in and out), INV with conjugate
// roots (unscaled): X0 = a + s, X1,2 = a - s/2 -/+ i sin(2 pi / 3) d, with
// s = b + c, d = b - c.
template <bool INV>
__device__ __forceinline__ void dft3(float2* v) {
  constexpr float h = 0.86602540378443864676f;  // sin(2 pi / 3)
  const float2 s = cadd(v[1], v[2]), d = csub(v[1], v[2]);
  const float2 m = make_float2(v[0].x - 0.5f * s.x, v[0].y - 0.5f * s.y);
  const float2 ihd = make_float2(-h * d.y, h * d.x);  // i h d
  v[0] = cadd(v[0], s);
  v[1] = INV ? cadd(m, ihd) : csub(m, ihd);
  v[2] = INV ? csub(m, ihd) : cadd(m, ihd);
}

template <int R, bool INV>
__device__ __forceinline__ void dft_mixed(float2* v) {
  if constexpr (R == 3)
    dft3<INV>(v);
  else
    dft<R, INV>(v);
}

// Radix of the pass after sub-transforms of length NS: 3 first for a 3 * 2^m
// length, then powers of two of at most RMAX.
// R2 (nonzero): the radix of the pass right after the radix-3 one.
constexpr int mixed_radix(int N, int NS, int RMAX, int R2 = 0) {
  return (NS == 1 && N % 3 == 0) ? 3 : (R2 && NS == 3) ? R2 : ((N / NS) < RMAX ? (N / NS) : RMAX);
}

// First-pass loader that returns zero for inputs r >= RZ of each radix-R
// butterfly when ON (the pass calls its loader in a fixed unrolled order,
// butterfly by butterfly, so r is a constant after unrolling).
template <int R, int RZ, bool ON, class LD>
struct TailZeroLoad {
  LD& ld;
  int q = 0;
  __device__ __forceinline__ float2 operator()(int m, int n) {
    const int r = q % R;
    ++q;
    if (ON && r >= RZ) return make_float2(0.f, 0.f);
    return ld(m, n);
  }
};

template <class LD>
__device__ __forceinline__ float2 mixed_load(LD& ld, int m, int n) {
  if constexpr (IsLdsTile<LD>::value)
    return *ld.at(m, n);
  else
    return ld(m, n);
}
template <class ST>
__device__ __forceinline__ void mixed_store(ST& st, int m, int n, float2 v) {
  if constexpr (IsLdsTile<ST>::value)
    *st.at(m, n) = v;
  else
    st(m, n, v);
}

// Pass synchronisation: a workgroup barrier, or (WAVE) the wave's own
// in-order LDS operations when one wave owns every transform of the pass.
template <bool WAVE>
__device__ __forceinline__ void mixed_sync() {
  if constexpr (WAVE) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  } else {
    __syncthreads();
  }
}

// One radix-R Stockham pass over M transforms of length N by T threads,
// after sub-transforms of length NS (WAVE: T = 64, the lanes of one wave,
// which owns the M transforms; no workgroup barrier): butterfly (m, j), j < N/R, reads
// elements j + r N/R, multiplies by W_{NS R}^{r (j mod NS)}, transforms, and
// writes elements (j - j mod NS) R + j mod NS + r NS.  TMAJOR as in
// stockham_pass.  Barriers bracket the writes, so LD and ST may alias.
// TW: the roots' source (TwAny: the global table; TwLds: roots staged in LDS).
template <int N, int R, int NS, bool INV, int M, int T, bool TMAJOR, bool WAVE = false, class LD, class ST,
          class TW>
__device__ __forceinline__ void mixed_pass(LD& ld, ST& st, const TW& tws) {
  static_assert(!WAVE || T == 64, "mixed_pass: a wave-local pass runs on the 64 lanes of one wave");
  constexpr int NR = N / R;
  constexpr int NB = M * NR;
  constexpr int PER = (NB + T - 1) / T;
  constexpr bool EXACT = NB % T == 0;
  constexpr int L = NS * R;
  static_assert(N % R == 0 && NR % NS == 0, "mixed_pass: radix does not divide the transform");
  const int tid = WAVE ? (opaque_tid() & 63) : opaque_tid();
  float2 w[PER][R];
  if constexpr (NS > 1) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int bf = EXACT ? tid + i * T : ((tid + i * T) < NB ? tid + i * T : 0);
      const int j = TMAJOR ? (bf / M) : (bf % NR);
      const int k = j % NS;
#pragma unroll
      for (int r = 1; r < R; ++r) w[i][r] = tws.template root<L>(r * k);
    }
  }
  float2 v[PER][R];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int bf = EXACT ? tid + i * T : ((tid + i * T) < NB ? tid + i * T : 0);
    const int m = TMAJOR ? (bf % M) : (bf / NR);
    const int j = TMAJOR ? (bf / M) : (bf % NR);
#pragma unroll
    for (int r = 0; r < R; ++r) v[i][r] = mixed_load(ld, m, j + r * NR);
  }
  mixed_sync<WAVE>();
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int bf = tid + i * T;
    if (!EXACT && bf >= NB) continue;
    const int m = TMAJOR ? (bf % M) : (bf / NR);
    const int j = TMAJOR ? (bf / M) : (bf % NR);
    const int k = j % NS;
    if constexpr (NS > 1) {
#pragma unroll
      for (int r = 1; r < R; ++r) v[i][r] = INV ? cmulc(v[i][r], w[i][r]) : cmul(v[i][r], w[i][r]);
    }
    dft_mixed<R, INV>(v[i]);
    const int base = (j - k) * R + k;
#pragma unroll
    for (int r = 0; r < R; ++r) mixed_store(st, m, base + r * NS, v[i][r]);
  }
  mixed_sync<WAVE>();
}

// Full transform of M length-N sequences (first pass through ld_first, last
// through st_last, the passes between in the LDS tile st_lds / ld_lds), radix
// at most RMAX after the radix-3 pass.  Ends with a barrier (WAVE: a wave
// sync).
template <int N, int NS, bool INV, int M, int T, bool TMAJOR, int RMAX, bool WAVE, int R2, class LDF, class STL,
          class LDL, class STF, class TW>
__device__ __forceinline__ void fft_mixed_rec(LDF& ld_first, STL& st_lds, LDL& ld_lds, STF& st_last, const TW& tws) {
  constexpr int R = mixed_radix(N, NS, RMAX, R2);
  constexpr bool FIRST = NS == 1;
  constexpr bool LAST = NS * R == N;
  if constexpr (FIRST && LAST) {
    mixed_pass<N, R, NS, INV, M, T, TMAJOR, WAVE>(ld_first, st_last, tws);
  } else if constexpr (FIRST) {
    mixed_pass<N, R, NS, INV, M, T, TMAJOR, WAVE>(ld_first, st_lds, tws);
    fft_mixed_rec<N, NS * R, INV, M, T, TMAJOR, RMAX, WAVE, R2>(ld_first, st_lds, ld_lds, st_last, tws);
  } else if constexpr (LAST) {
    mixed_pass<N, R, NS, INV, M, T, TMAJOR, WAVE>(ld_lds, st_last, tws);
  } else {
    mixed_pass<N, R, NS, INV, M, T, TMAJOR, WAVE>(ld_lds, st_lds, tws);
    fft_mixed_rec<N, NS * R, INV, M, T, TMAJOR, RMAX, WAVE, R2>(ld_first, st_lds, ld_lds, st_last, tws);
  }
}

template <int N, bool INV, int M, int T, bool TMAJOR, int RMAX, class LDF, class TILE, class STF, class TW>
__device__ __forceinline__ void fft_mixed(LDF& ld_first, TILE& tile, STF& st_last, const TW& tws) {
  static_assert(mixed_len(N), "fft_mixed: length must be 2^m or 3 * 2^m");
  fft_mixed_rec<N, 1, INV, M, T, TMAJOR, RMAX, false, 0>(ld_first, tile, tile, st_last, tws);
}

// fft_mixed by one wave on transforms that it alone reads and writes; R2 as
// in mixed_radix.
template <int N, bool INV, int M, bool TMAJOR, int RMAX, int R2 = 0, class LDF, class TILE, class STF, class TW>
__device__ __forceinline__ void fft_mixed_wave(LDF& ld_first, TILE& tile, STF& st_last, const TW& tws) {
  static_assert(mixed_len(N), "fft_mixed_wave: length must be 2^m or 3 * 2^m");
  fft_mixed_rec<N, 1, INV, M, 64, TMAJOR, RMAX, true, R2>(ld_first, tile, tile, st_last, tws);
}

}  // namespace nsq
