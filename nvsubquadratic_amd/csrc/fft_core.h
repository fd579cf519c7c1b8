// Device building blocks for LDS-resident Stockham FFTs on gfx950.
//
// Design (CDNA4, wave64):
//  * A workgroup holds a tile of M independent power-of-two transforms in LDS
//    and each thread owns E = M*N/T complex points per pass (E = 16 in every
//    kernel of this library, i.e. 32 VGPRs of data).
//  * Each Stockham pass reads R points per butterfly, multiplies by the pass
//    twiddles, runs an in-register radix-R DFT (R <= 16, unrolled radix-2
//    DIT with trivial roots special-cased) and writes the autosorted result.
//    The output of the last pass is in natural order, so no bit reversal.
//  * The first pass may read from global memory and the last pass may write
//    to global memory through functors, so a transform that starts and ends
//    in HBM costs only (passes - 1) LDS round trips.
//  * Twiddles of transforms up to 2^14 come from the table built in
//    twiddle.hip (double-precision roots rounded once), a pass loading the
//    roots at r = 1, 2, 4, 8 and forming the others as products of two
//    (pass_twiddles); longer-period roots use the hardware sin/cos (see root<>
//    below).  No running recurrences on device.
#pragma once

#include <type_traits>

#include "nsq_common.h"

namespace nsq {

// ---------------------------------------------------------------------------
// Complex helpers (float2 = re, im)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
  return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
// a * conj(b)
__device__ __forceinline__ float2 cmulc(float2 a, float2 b) {
  return make_float2(a.x * b.x + a.y * b.y, a.y * b.x - a.x * b.y);
}
__device__ __forceinline__ float2 cconj(float2 a) { return make_float2(a.x, -a.y); }
__device__ __forceinline__ float2 cscale(float2 a, float s) { return make_float2(a.x * s, a.y * s); }
__device__ __forceinline__ float2 mul_i(float2 a) { return make_float2(-a.y, a.x); }
__device__ __forceinline__ float2 mul_neg_i(float2 a) { return make_float2(a.y, -a.x); }

// ---------------------------------------------------------------------------
// Roots of unity W_{2^LOGB}^m (forward sign).
//  * LOGB <= 14: one load from the table segment of size 2^LOGB (correctly
//    rounded roots; segment b starts at entry 2^b).
//  * LOGB > 14 (the long-transform twiddles of the 4-step plan and the real
//    unpack): the hardware sin/cos of gfx950, whose argument is in revolutions,
//    on the exact fraction m / 2^LOGB.  Measured on MI355X against double
//    precision over 2^20 arguments: max abs error 1.25e-7, rms 3.5e-8 (a
//    correctly rounded float table: 3.0e-8), i.e. ~2 ulp, far inside the 1e-4
//    rel-L2 budget of the fp32 path, and with no scattered table loads.
// ---------------------------------------------------------------------------
template <int LOGB>
__device__ __forceinline__ float2 root(const float2* __restrict__ tw, uint32_t m) {
  static_assert(LOGB >= 0 && LOGB <= 24, "root: size out of range");
  if constexpr (LOGB <= 14) {
    return tw[(1u << LOGB) + (m & ((1u << LOGB) - 1u))];
  } else {
    const float a = float(m & ((1u << LOGB) - 1u)) * (1.0f / float(1u << LOGB));
    return make_float2(__builtin_amdgcn_cosf(a), -__builtin_amdgcn_sinf(a));
  }
}


// Keeps the scheduler from hoisting the loads of every unrolled spectral slot
// (or twiddle, or filter value) ahead of the first one, which otherwise
// multiplies the live registers.
#define NSQ_SLOT_FENCE() __builtin_amdgcn_sched_barrier(0)

// Thread index hidden from loop-invariant code motion.  Pass twiddles and
// addresses depend only on the thread index; inside a batch loop the compiler
// would otherwise hoist all of them out of the loop and keep them live across
// it, tripling the register footprint (and halving occupancy).  Recomputing
// them per use is cheaper than the lost occupancy.
__device__ __forceinline__ int opaque_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// ---------------------------------------------------------------------------
// Compile-time loop
// ---------------------------------------------------------------------------
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Multiply by the constant root W_R^K (forward) or its conjugate (INV).
template <int R, int K, bool INV>
__device__ __forceinline__ float2 const_twiddle(float2 a) {
  constexpr int K16 = K * (16 / R);  // angle in units of 2*pi/16, K16 in [0, 8)
  static_assert(K16 >= 0 && K16 < 8, "const_twiddle: K out of range");
  constexpr float r2 = 0.70710678118654752440f;  // cos(pi/4)
  if constexpr (K16 == 0) {
    return a;
  } else if constexpr (K16 == 4) {
    return INV ? mul_i(a) : mul_neg_i(a);
  } else if constexpr (K16 == 2) {
    // forward (1 - i)/sqrt2, inverse (1 + i)/sqrt2
    return INV ? make_float2(r2 * (a.x - a.y), r2 * (a.y + a.x))
               : make_float2(r2 * (a.x + a.y), r2 * (a.y - a.x));
  } else if constexpr (K16 == 6) {
    // forward (-1 - i)/sqrt2, inverse (-1 + i)/sqrt2
    return INV ? make_float2(-r2 * (a.x + a.y), r2 * (a.x - a.y))
               : make_float2(r2 * (a.y - a.x), -r2 * (a.x + a.y));
  } else {
    // cos/sin of k*pi/8 for k = 1, 3, 5, 7
    constexpr float c = (K16 == 1) ? 0.92387953251128675613f
                      : (K16 == 3) ? 0.38268343236508977173f
                      : (K16 == 5) ? -0.38268343236508977173f
                                   : -0.92387953251128675613f;
    constexpr float s = (K16 == 1 || K16 == 7) ? 0.38268343236508977173f : 0.92387953251128675613f;
    // forward multiplies by (c - i s), inverse by (c + i s)
    return INV ? make_float2(a.x * c - a.y * s, a.y * c + a.x * s)
               : make_float2(a.x * c + a.y * s, a.y * c - a.x * s);
  }
}

// Complex product with its two fused multiply-adds written out, so every
// kernel that inlines it rounds identically (with contraction left to the
// compiler, a*b - c*d may become fma(a, b, -c*d) in one kernel and
// fma(-c, d, a*b) in another).  Used for the roots this file derives from
// table roots, which kernels of different plans must reproduce bit for bit.
__device__ __forceinline__ float2 cmul_fixed(float2 a, float2 b) {
  return make_float2(__builtin_fmaf(a.x, b.x, -(a.y * b.y)), __builtin_fmaf(a.x, b.y, a.y * b.x));
}

// a * W_16^i for i in [0, 8); i is a constant after unrolling, so one case
// remains.  The roots are the correctly rounded float constants.
__device__ __forceinline__ float2 rot16(float2 a, int i) {
  constexpr float c1 = 0.92387953251128675613f, s1 = 0.38268343236508977173f, r2 = 0.70710678118654752440f;
  switch (i) {
    case 1: return cmul_fixed(a, make_float2(c1, -s1));
    case 2: return cmul_fixed(a, make_float2(r2, -r2));
    case 3: return cmul_fixed(a, make_float2(s1, -c1));
    case 4: return mul_neg_i(a);
    case 5: return cmul_fixed(a, make_float2(-s1, -c1));
    case 6: return cmul_fixed(a, make_float2(-r2, -r2));
    case 7: return cmul_fixed(a, make_float2(-c1, -s1));
    default: return a;
  }
}

// In-register DFT of R = 2, 4, 8 or 16 points, natural order in and out.
// Forward: X[k] = sum_n v[n] W_R^{nk}; INV uses conjugate roots (unscaled).
template <int R, bool INV>
__device__ __forceinline__ void dft(float2* v) {
  if constexpr (R == 1) {
    return;
  } else if constexpr (R == 2) {
    float2 a = v[0], b = v[1];
    v[0] = cadd(a, b);
    v[1] = csub(a, b);
  } else if constexpr (R == 4) {
    float2 t0 = cadd(v[0], v[2]);
    float2 t1 = csub(v[0], v[2]);
    float2 t2 = cadd(v[1], v[3]);
    float2 d = csub(v[1], v[3]);
    float2 t3 = INV ? mul_i(d) : mul_neg_i(d);
    v[0] = cadd(t0, t2);
    v[2] = csub(t0, t2);
    v[1] = cadd(t1, t3);
    v[3] = csub(t1, t3);
  } else {
    float2 e[R / 2], o[R / 2];
#pragma unroll
    for (int i = 0; i < R / 2; ++i) {
      e[i] = v[2 * i];
      o[i] = v[2 * i + 1];
    }
    dft<R / 2, INV>(e);
    dft<R / 2, INV>(o);
    static_for<0, R / 2>([&](auto kk) {
      constexpr int k = decltype(kk)::value;
      float2 t = const_twiddle<R, k, INV>(o[k]);
      v[k] = cadd(e[k], t);
      v[k + R / 2] = csub(e[k], t);
    });
  }
}

// LDS position of element n in an element-major tile: one pad slot per 16
// elements, so the stride-R writes of a Stockham pass (lanes j -> j*R + r)
// spread over the 64 banks instead of hitting two of them.
__device__ __forceinline__ constexpr int pad16(int n) { return n + (n >> 4); }
template <int N>
struct Padded {
  static constexpr int SIZE = N + N / 16;  // padded length of one transform
};

// A tile of transforms in LDS: transform m at p[m*S ...], element n at
// pad16(n) (PAD, element-major tiles) or at n (TMAJOR tiles, whose odd stride
// S already spreads the banks).  For every access pattern of a power-of-two
// Stockham pass -- element j + r*NR read, element base + r*NS written --
// pad16(x + r*D) == pad16(x) + pad16(r*D) (checked exhaustively for all
// transform lengths <= 2^14), so a pass computes one address per butterfly
// and reaches its R elements through compile-time offsets.
template <int S, bool PAD>
struct LdsTile {
  float2* p;
  __device__ __forceinline__ float2* at(int m, int n) const { return p + m * S + (PAD ? pad16(n) : n); }
  static constexpr int off(int d) { return PAD ? pad16(d) : d; }
};
// Columns of a row-major LDS matrix with padded rows of stride RS (complex):
// transform m is column j0 + m, its element n at p[pad16(j0 + m) + n*RS].
template <int RS>
struct LdsCols {
  float2* p;
  int j0;
  __device__ __forceinline__ float2* at(int m, int n) const { return p + pad16(j0 + m) + n * RS; }
  static constexpr int off(int d) { return d * RS; }
};

// Store functors of a last pass may take a butterfly's R outputs at once,
// run<R, NS>(m, base, v) for outputs base + r*NS (r < R) of transform m,
// e.g. to step a twiddle from one output to the next instead of computing
// each.  Marked by a member `static constexpr bool kRunStore = true`.
template <class X, class = void>
struct HasRunStore : std::false_type {};
template <class X>
struct HasRunStore<X, std::void_t<decltype(X::kRunStore)>> : std::true_type {};

template <class X>
struct IsLdsTile : std::false_type {};
template <int S, bool PAD>
struct IsLdsTile<LdsTile<S, PAD>> : std::true_type {};
template <int RS>
struct IsLdsTile<LdsCols<RS>> : std::true_type {};

// Twiddle-table loads through a raw buffer resource: 32-bit offsets from one
// scalar base, so a butterfly's R-1 twiddle addresses are a multiply each.
struct TwTable {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ explicit TwTable(const float2* tw)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<float2*>(tw), 0, int((2 << 14) * sizeof(float2)), 0x00020000)) {}
  // entry seg + idx of the table (seg = 2^b selects the W_{2^b} segment)
  __device__ __forceinline__ float2 load(int seg, int idx) const {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, idx * int(sizeof(float2)),
                                                                          seg * int(sizeof(float2)), 0));
  }
};

// The R-1 twiddles W_S^{r k} (r = 1..R-1) of one butterfly, S = the segment
// of this pass.  Only the roots at r = 1, 2, 4, 8 are table loads; the others
// are products of two of them (r = 3 = 2+1, 5..7 = 4 + 1..3, 9..15 = 8 +
// 1..7), at most three products deep (W^{15k} = W^{8k} (W^{4k} (W^{2k}
// W^k))): a few ulp (measured 2.3e-7 rel-L2 over a 2^19-point transform
// against all-table twiddles).  Measured on MI355X: each vector-memory load
// of a pass waits, in issue order, behind the tile's HBM loads and stores, so
// 4 loads and 11 complex products per radix-16 butterfly instead of 15 loads
// take ~10% off the 4-step row kernels, whose VALU is far from busy.
template <int R>
__device__ __forceinline__ void pass_twiddles(const TwTable& tt, int seg, int k, float2* w) {
  w[1] = tt.load(seg, k);
  if constexpr (R >= 4) {
    w[2] = tt.load(seg, 2 * k);
    w[3] = cmul_fixed(w[2], w[1]);
  }
  if constexpr (R >= 8) {
    w[4] = tt.load(seg, 4 * k);
#pragma unroll
    for (int r = 5; r < 8; ++r) w[r] = cmul_fixed(w[4], w[r - 4]);
  }
  if constexpr (R >= 16) {
    w[8] = tt.load(seg, 8 * k);
#pragma unroll
    for (int r = 9; r < 16; ++r) w[r] = cmul_fixed(w[8], w[r - 8]);
  }
  static_assert(R <= 16, "pass_twiddles: radix up to 16");
}

// ---------------------------------------------------------------------------
// One radix-2^LOGR Stockham pass over M transforms of length 2^LOGN executed by
// T threads.  LD(m, n) -> float2 reads input element n of transform m; ST(m, n,
// v) writes output element n.  LOGNS = log2 of the sub-transform length already
// done (0 for the first pass).  Barriers bracket the write phase so LD and ST
// may alias the same LDS buffer.  Butterfly b of the tile is owned by thread
// b % T; TMAJOR selects whether consecutive butterflies step through the
// transforms first (m = b % M: consecutive lanes touch consecutive transforms,
// i.e. consecutive columns of a row-major matrix in global memory) or through
// the elements of one transform first (m = b / (N/R)).
// ---------------------------------------------------------------------------
template <int LOGN, int LOGR, int LOGNS, bool INV, int M, int T, bool TMAJOR, class LD, class ST>
__device__ __forceinline__ void stockham_pass(LD& ld, ST& st, const float2* __restrict__ tw) {
  constexpr int R = 1 << LOGR;
  constexpr int NR = 1 << (LOGN - LOGR);
  constexpr int NS = 1 << LOGNS;
  constexpr int PER = (M * NR) / T;
  static_assert((M * NR) % T == 0, "stockham_pass: tile not divisible by threads");
  static_assert(LOGNS + LOGR <= 14, "stockham_pass: transform too long for the twiddle table");
  const int tid = opaque_tid();
  // Twiddles first: their loads depend only on the thread index, so they are
  // in flight while the pass reads its inputs and waits at the barrier.
  float2 w[PER][R];
  if constexpr (LOGNS > 0) {
    const TwTable tt(tw);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int bf = tid + i * T;
      const int j = TMAJOR ? (bf / M) : (bf & (NR - 1));
      const int k = j & (NS - 1);
      pass_twiddles<R>(tt, 1 << (LOGNS + LOGR), k, w[i]);
    }
  }
  float2 v[PER][R];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int bf = tid + i * T;
    const int m = TMAJOR ? (bf % M) : (bf >> (LOGN - LOGR));
    const int j = TMAJOR ? (bf / M) : (bf & (NR - 1));
    if constexpr (IsLdsTile<LD>::value) {
      const float2* q = ld.at(m, j);
#pragma unroll
      for (int r = 0; r < R; ++r) v[i][r] = q[LD::off(r * NR)];
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) v[i][r] = ld(m, j + r * NR);
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int bf = tid + i * T;
    const int m = TMAJOR ? (bf % M) : (bf >> (LOGN - LOGR));
    const int j = TMAJOR ? (bf / M) : (bf & (NR - 1));
    const int k = j & (NS - 1);
    if constexpr (LOGNS > 0) {
#pragma unroll
      for (int r = 1; r < R; ++r) v[i][r] = INV ? cmulc(v[i][r], w[i][r]) : cmul(v[i][r], w[i][r]);
    }
    dft<R, INV>(v[i]);
    const int base = ((j - k) << LOGR) + k;
    if constexpr (IsLdsTile<ST>::value) {
      float2* q = st.at(m, base);
#pragma unroll
      for (int r = 0; r < R; ++r) q[ST::off(r * NS)] = v[i][r];
    } else if constexpr (HasRunStore<ST>::value) {
      st.template run<R, NS>(m, base, v[i]);
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) st(m, base + r * NS, v[i][r]);
    }
  }
  __syncthreads();
}

// First-pass loader over values already in registers: the pass calls its
// loader in a fixed, fully unrolled order (butterfly i, then point r), so the
// values are handed out in that order and every index is a constant after
// unrolling.
template <int NV>
struct RegStream {
  const float2 (&v)[NV];
  int k = 0;
  __device__ __forceinline__ float2 operator()(int, int) { return v[k++]; }
};

// First-pass loader wrapper for zero-padded transforms: with HALF, the inputs
// r >= R/2 of each radix-R first-pass butterfly (elements j + r*N/R >= N/2)
// are zero, returned as constants (the call order is fixed and unrolled, so r
// is a constant) and the butterflies fold them away; the rest go to LD.
template <int R, bool HALF, class LD>
struct HalfZeroLoad {
  LD& ld;
  int q = 0;
  __device__ __forceinline__ float2 operator()(int m, int n) {
    const int r = q % R;
    ++q;
    if (HALF && r >= R / 2) return make_float2(0.f, 0.f);
    return ld(m, n);
  }
};

// LOGRMAX: the largest pass radix (log2; 4 = radix 16, E = 16 points per
// thread; 3 = radix 8 for E = 8).
template <int LOGN, int LOGNS, bool INV, int M, int T, bool TMAJOR, int LOGRMAX = 4, class LDF, class STL, class LDL,
          class STF>
__device__ __forceinline__ void fft_rec(LDF& ld_first, STL& st_lds, LDL& ld_lds, STF& st_last,
                                        const float2* __restrict__ tw) {
  constexpr int REM = LOGN - LOGNS;
  constexpr int LOGR = REM < LOGRMAX ? REM : LOGRMAX;
  constexpr bool FIRST = (LOGNS == 0);
  constexpr bool LAST = (LOGNS + LOGR == LOGN);
  if constexpr (FIRST && LAST) {
    stockham_pass<LOGN, LOGR, LOGNS, INV, M, T, TMAJOR>(ld_first, st_last, tw);
  } else if constexpr (FIRST) {
    stockham_pass<LOGN, LOGR, LOGNS, INV, M, T, TMAJOR>(ld_first, st_lds, tw);
    fft_rec<LOGN, LOGNS + LOGR, INV, M, T, TMAJOR, LOGRMAX>(ld_first, st_lds, ld_lds, st_last, tw);
  } else if constexpr (LAST) {
    stockham_pass<LOGN, LOGR, LOGNS, INV, M, T, TMAJOR>(ld_lds, st_last, tw);
  } else {
    stockham_pass<LOGN, LOGR, LOGNS, INV, M, T, TMAJOR>(ld_lds, st_lds, tw);
    fft_rec<LOGN, LOGNS + LOGR, INV, M, T, TMAJOR, LOGRMAX>(ld_first, st_lds, ld_lds, st_last, tw);
  }
}

// Full transform of M length-2^LOGN sequences.  Passes 2..n-1 run in `lds`
// (an LdsTile: transform m at lds[m*S ...], padded element-major unless
// TMAJOR); the first pass reads through ld_first and the last pass writes
// through st_last, each either a functor (m, n[, v]) or an LdsTile of the
// same layout.  Ends with a barrier.
template <int LOGN, bool INV, int M, int T, int S, bool TMAJOR = false, class LDF, class STF>
__device__ __forceinline__ void fft(float2* lds, LDF& ld_first, STF& st_last, const float2* __restrict__ tw) {
  LdsTile<S, !TMAJOR> tile{lds};
  fft_rec<LOGN, 0, INV, M, T, TMAJOR>(ld_first, tile, tile, st_last, tw);
}
// The same with passes of radix at most 2^LOGRMAX (element-major tile).
template <int LOGRMAX, int LOGN, bool INV, int M, int T, int S, class LDF, class STF>
__device__ __forceinline__ void fft_radix(float2* lds, LDF& ld_first, STF& st_last, const float2* __restrict__ tw) {
  LdsTile<S, true> tile{lds};
  fft_rec<LOGN, 0, INV, M, T, false, LOGRMAX>(ld_first, tile, tile, st_last, tw);
}

// Transform that starts and ends in LDS.
template <int LOGN, bool INV, int M, int T, int S, bool TMAJOR = false>
__device__ __forceinline__ void fft_lds(float2* lds, const float2* __restrict__ tw) {
  LdsTile<S, !TMAJOR> tile{lds};
  fft_rec<LOGN, 0, INV, M, T, TMAJOR>(tile, tile, tile, tile, tw);
}

// ---------------------------------------------------------------------------
// Real-FFT packing.  A real sequence u[0, 2N) is packed as z[n] = u[2n] +
// i*u[2n+1]; Z = FFT_N(z).  The real spectrum U[0..N] is handled in "slots":
//   slot p in [1, N/2): (A, Bc) = (U[p], conj(U[N-p]))
//   slot 0:             A = (U[0], U[N]) (two reals), Bc = U[N/2]
// With this representation forward products are slot-wise A1*A2, Bc1*Bc2 and
// correlations A1*conj(A2), Bc1*conj(Bc2), except slot 0's A whose two reals
// multiply separately.
// ---------------------------------------------------------------------------
// zp = Z[p], zq = Z[N-p] (for p = 0: zp = Z[0], zq = Z[N/2]); w = W_{2N}^p.
// Branch-free: both the regular and the slot-0 forms are computed and one is
// selected, so a slot loop has no divergent control flow.
__device__ __forceinline__ void real_unpack(bool slot0, float2 zp, float2 zq, float2 w, float2& A, float2& Bc) {
  const float2 bc = cconj(zq);
  const float2 fe = cscale(cadd(zp, bc), 0.5f);
  const float2 fo = mul_neg_i(cscale(csub(zp, bc), 0.5f));
  const float2 wfo = cmul(w, fo);
  const float2 a_reg = cadd(fe, wfo);
  const float2 b_reg = csub(fe, wfo);
  A.x = slot0 ? zp.x + zp.y : a_reg.x;
  A.y = slot0 ? zp.x - zp.y : a_reg.y;
  Bc.x = slot0 ? bc.x : b_reg.x;
  Bc.y = slot0 ? bc.y : b_reg.y;
}

// Inverse of real_unpack for a Hermitian spectrum given in slot form; returns
// the values to place at Z[p] and Z[N-p] (slot 0: Z[0] and Z[N/2]) so that the
// unscaled inverse FFT_N gives N * (u[2n] + i u[2n+1]).  Branch-free.
__device__ __forceinline__ void real_repack(bool slot0, float2 A, float2 Bc, float2 w, float2& zp, float2& zq) {
  const float2 fe = cscale(cadd(A, Bc), 0.5f);
  const float2 fo = cmulc(cscale(csub(A, Bc), 0.5f), w);  // * conj(w)
  const float2 p_reg = cadd(fe, mul_i(fo));
  const float2 q_reg = cadd(cconj(fe), mul_i(cconj(fo)));
  zp.x = slot0 ? 0.5f * (A.x + A.y) : p_reg.x;
  zp.y = slot0 ? 0.5f * (A.x - A.y) : p_reg.y;
  zq.x = slot0 ? Bc.x : q_reg.x;
  zq.y = slot0 ? -Bc.y : q_reg.y;
}

__device__ __forceinline__ float2 slot_mul(bool slot0_a, float2 a, float2 b) {
  const float2 c = cmul(a, b);
  return make_float2(slot0_a ? a.x * b.x : c.x, slot0_a ? a.y * b.y : c.y);
}
__device__ __forceinline__ float2 slot_mulc(bool slot0_a, float2 a, float2 b) {
  const float2 c = cmulc(a, b);
  return make_float2(slot0_a ? a.x * b.x : c.x, slot0_a ? a.y * b.y : c.y);
}

// ---------------------------------------------------------------------------
// Pair load/store of a real row: (u[i], u[i+1]) with zeros outside [0, valid).
// Uses one 2-element vector access when the pair is in range and aligned
// (always the case for even row strides), else two scalar accesses.
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ float2 load_pair(const typename Elem<DT>::T* __restrict__ row, int64_t i, int64_t valid) {
  using ET = typename Elem<DT>::T;
  const ET* p = row + i;
  if (i + 1 < valid && (reinterpret_cast<uintptr_t>(p) & (2 * sizeof(ET) - 1)) == 0) {
    if constexpr (DT == NSQ_DTYPE_F32) {
      return *reinterpret_cast<const float2*>(p);
    } else if constexpr (DT == NSQ_DTYPE_BF16) {
      const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
      return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
    } else {
      return __half22float2(*reinterpret_cast<const __half2*>(p));
    }
  }
  float a = (i < valid) ? Elem<DT>::load(row, i) : 0.f;
  float b = (i + 1 < valid) ? Elem<DT>::load(row, i + 1) : 0.f;
  return make_float2(a, b);
}

// Branch-free pair access for streaming kernels.  The load is always issued,
// from a clamped in-bounds address (row[0] for out-of-range pairs, so `valid`
// must be >= 1 for generic rows and >= 2 when ALIGNED), and out-of-range lanes
// select zero afterwards: a run of these loads stays in flight together
// instead of each waiting behind a branch.  ALIGNED means `valid` is even and
// the row base is 2-element aligned (even row stride, aligned pointer; the
// host checks), so a pair at an even index is one vector access that lies
// wholly inside or wholly outside the row.
template <int DT>
__device__ __forceinline__ float2 load2(const typename Elem<DT>::T* __restrict__ p) {
  if constexpr (DT == NSQ_DTYPE_F32) {
    return *reinterpret_cast<const float2*>(p);
  } else if constexpr (DT == NSQ_DTYPE_BF16) {
    const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
    return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
  } else {
    return __half22float2(*reinterpret_cast<const __half2*>(p));
  }
}

template <int DT>
__device__ __forceinline__ void store2(typename Elem<DT>::T* __restrict__ p, float2 v) {
  if constexpr (DT == NSQ_DTYPE_F32) {
    *reinterpret_cast<float2*>(p) = v;
  } else if constexpr (DT == NSQ_DTYPE_BF16) {
    *reinterpret_cast<uint32_t*>(p) = f32x2_to_bf16x2_bits(v.x, v.y);
  } else {
    *reinterpret_cast<__half2*>(p) = __floats2half2_rn(v.x, v.y);
  }
}

template <int DT, bool ALIGNED>
__device__ __forceinline__ float2 load_pair_nb(const typename Elem<DT>::T* __restrict__ row, int64_t i,
                                               int64_t valid) {
  if constexpr (ALIGNED) {
    const bool in = i < valid;
    const float2 v = load2<DT>(row + (in ? i : 0));
    return make_float2(in ? v.x : 0.f, in ? v.y : 0.f);
  } else {
    const bool ina = i < valid, inb = i + 1 < valid;
    const float a = Elem<DT>::load(row, ina ? i : 0);
    const float b = Elem<DT>::load(row, inb ? i + 1 : 0);
    return make_float2(ina ? a : 0.f, inb ? b : 0.f);
  }
}

template <int DT, bool ALIGNED>
__device__ __forceinline__ void store_pair_nb(typename Elem<DT>::T* __restrict__ row, int64_t i, int64_t valid,
                                              float2 v) {
  if constexpr (ALIGNED) {
    if (i < valid) store2<DT>(row + i, v);
  } else {
    if (i < valid) Elem<DT>::store(row, i, v.x);
    if (i + 1 < valid) Elem<DT>::store(row, i + 1, v.y);
  }
}

// A real row of `valid` elements as a raw buffer resource.  The hardware range
// check returns 0 for loads past the end and drops stores past it, so row
// accesses need no branches, a run of loads stays in flight together, and the
// zero padding of a transform costs no memory traffic.  Offsets are 32-bit
// byte offsets from the row start (rows here are below 2^28 elements); every
// offset is non-negative (see elem_halo for positions before the row).
// ALIGNED: see load_pair_nb; a pair at an even index is then one access.
template <int DT, bool ALIGNED, int AUX = 0>
struct RowBuf {
  using ET = typename Elem<DT>::T;
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ RowBuf(const ET* row, int64_t valid)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<ET*>(row), 0, int(valid * int64_t(sizeof(ET))),
                                            0x00020000)) {}
  __device__ __forceinline__ float elem(int64_t i) const {
    const int off = int(i) * int(sizeof(ET));
    if constexpr (DT == NSQ_DTYPE_F32) {
      return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX));
    } else if constexpr (DT == NSQ_DTYPE_BF16) {
      return bf16_bits_to_f32(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, AUX));
    } else {
      return __half2float(__builtin_bit_cast(__half, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, AUX)));
    }
  }
  // Element at a position that may be negative (a halo before the row start),
  // zero there.  A negative byte offset is not safe on its own: the compiler
  // may fold a constant of the index into the instruction's immediate offset,
  // and the 32-bit sum can wrap back into range.  Positions before 0 therefore
  // use offset 2^31, which no immediate brings into range, and the offset is
  // hidden from further folding.
  __device__ __forceinline__ float elem_halo(int n) const { return bits_to_f32(elem_halo_bits(n)); }
  // The element's raw bits (zero-extended), for loaders that convert later:
  // converting each value right after its load would hold the next load
  // behind the previous one's completion.
  __device__ __forceinline__ uint32_t elem_halo_bits(int n) const {
    int off = n < 0 ? int(0x80000000u) : n * int(sizeof(ET));
    asm volatile("" : "+v"(off));
    if constexpr (DT == NSQ_DTYPE_F32) {
      return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX);
    } else {
      return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, AUX);
    }
  }
  __device__ __forceinline__ static float bits_to_f32(uint32_t b) {
    if constexpr (DT == NSQ_DTYPE_F32) {
      return __builtin_bit_cast(float, b);
    } else if constexpr (DT == NSQ_DTYPE_BF16) {
      return __uint_as_float(b << 16);
    } else {
      return __half2float(__builtin_bit_cast(__half, uint16_t(b)));
    }
  }
  __device__ __forceinline__ void store_elem(int64_t i, float v) const {
    const int off = int(i) * int(sizeof(ET));
    if constexpr (DT == NSQ_DTYPE_F32) {
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, AUX);
    } else if constexpr (DT == NSQ_DTYPE_BF16) {
      __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(v), r, off, 0, AUX);
    } else {
      __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, __float2half_rn(v)), r, off, 0, AUX);
    }
  }
  // (u[i], u[i+1]); i even when ALIGNED.
  __device__ __forceinline__ float2 load_pair(int64_t i) const {
    if constexpr (ALIGNED) {
      const int off = int(i) * int(sizeof(ET));
      if constexpr (DT == NSQ_DTYPE_F32) {
        return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, AUX));
      } else if constexpr (DT == NSQ_DTYPE_BF16) {
        const uint32_t u = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX);
        return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
      } else {
        return __half22float2(__builtin_bit_cast(__half2, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX)));
      }
    } else {
      return make_float2(elem(i), elem(i + 1));
    }
  }
  // load_pair split into the access and the conversion, so that a loader can
  // keep a pair's raw bits in flight across other work (a prefetch).
  struct PairBits {
    uint32_t a, b;
  };
  __device__ __forceinline__ PairBits load_pair_bits(int64_t i) const {
    const int off = int(i) * int(sizeof(ET));
    if constexpr (ALIGNED && DT == NSQ_DTYPE_F32) {
      const auto u = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, AUX);
      return PairBits{u[0], u[1]};
    } else if constexpr (ALIGNED) {
      return PairBits{__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX), 0u};
    } else if constexpr (DT == NSQ_DTYPE_F32) {
      return PairBits{__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX),
                      __builtin_amdgcn_raw_buffer_load_b32(r, off + 4, 0, AUX)};
    } else {
      return PairBits{__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, AUX),
                      __builtin_amdgcn_raw_buffer_load_b16(r, off + 2, 0, AUX)};
    }
  }
  __device__ __forceinline__ static float2 pair_from_bits(PairBits p) {
    if constexpr (ALIGNED && DT == NSQ_DTYPE_BF16) {
      return make_float2(__uint_as_float(p.a << 16), __uint_as_float(p.a & 0xffff0000u));
    } else if constexpr (ALIGNED && DT == NSQ_DTYPE_F16) {
      return __half22float2(__builtin_bit_cast(__half2, p.a));
    } else {
      return make_float2(bits_to_f32(p.a), bits_to_f32(p.b));
    }
  }
  __device__ __forceinline__ void store_pair(int64_t i, float2 v) const {
    if constexpr (ALIGNED) {
      const int off = int(i) * int(sizeof(ET));
      if constexpr (DT == NSQ_DTYPE_F32) {
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(uint32_t __attribute__((ext_vector_type(2))), v), r,
                                              off, 0, 0);
      } else if constexpr (DT == NSQ_DTYPE_BF16) {
        __builtin_amdgcn_raw_buffer_store_b32(f32x2_to_bf16x2_bits(v.x, v.y), r, off, 0, AUX);
      } else {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, __floats2half2_rn(v.x, v.y)), r, off, 0,
                                              0);
      }
    } else {
      store_elem(i, v.x);
      store_elem(i + 1, v.y);
    }
  }
};

// Samples x[n + i], i < 8, of one row as raw bits.  AL (16-bit types: len %
// 8 == 0; fp32: len % 4 == 0; 16-byte aligned rows): n is a multiple of 8 and
// the chunk is one (16-bit types) or two (fp32) aligned 16-byte loads lying
// wholly inside or wholly outside [0, len); otherwise eight element loads.  A
// chunk before the row (n < 0) reads as zero.
template <int DT, bool AL>
struct Win8 {
  static constexpr bool HALF = DT != NSQ_DTYPE_F32;
  static constexpr int W = (HALF && AL) ? 4 : 8;
  uint32_t w[W];
  __device__ __forceinline__ void load(const RowBuf<DT, false>& rb, int n) {
    if constexpr (AL) {
      constexpr int ES = HALF ? 2 : 4;
      int off = n < 0 ? int(0x80000000u) : n * ES;
      asm volatile("" : "+v"(off));
      if constexpr (HALF) {
        const auto m = __builtin_amdgcn_raw_buffer_load_b128(rb.r, off, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = m[i];
      } else {
        const auto m0 = __builtin_amdgcn_raw_buffer_load_b128(rb.r, off, 0, 0);
        const auto m1 = __builtin_amdgcn_raw_buffer_load_b128(rb.r, off + 16, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) { w[i] = m0[i]; w[4 + i] = m1[i]; }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = rb.elem_halo_bits(n + i);
    }
  }
  __device__ __forceinline__ float at(int i) const {  // i is a compile-time constant after unrolling
    if constexpr (HALF && AL) {
      const uint32_t v = (i & 1) ? (w[i >> 1] >> 16) : (w[i >> 1] & 0xffffu);
      return RowBuf<DT, false>::bits_to_f32(v);
    } else {
      return RowBuf<DT, false>::bits_to_f32(w[i]);
    }
  }
};

// Stores v[i] at positions n + i, i < 8, of one row.  AL as for Win8: n is a
// multiple of 8 and the chunk goes out as one (16-bit types) or two (fp32)
// 16-byte stores, dropped as a whole past the row end; otherwise pair stores.
template <int DT, bool AL>
__device__ __forceinline__ void store8(const RowBuf<DT, AL>& rb, int n, const float (&v)[8]) {
  if constexpr (AL) {
    using U4 = uint32_t __attribute__((ext_vector_type(4)));
    const int off = n * int(sizeof(typename Elem<DT>::T));
    if constexpr (DT == NSQ_DTYPE_F32) {
      __builtin_amdgcn_raw_buffer_store_b128(U4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                                __float_as_uint(v[3])},
                                             rb.r, off, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(U4{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                                                __float_as_uint(v[7])},
                                             rb.r, off + 16, 0, 0);
    } else {
      uint32_t u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (DT == NSQ_DTYPE_BF16)
          u[i] = f32x2_to_bf16x2_bits(v[2 * i], v[2 * i + 1]);
        else
          u[i] = __builtin_bit_cast(uint32_t, __floats2half2_rn(v[2 * i], v[2 * i + 1]));
      }
      __builtin_amdgcn_raw_buffer_store_b128(U4{u[0], u[1], u[2], u[3]}, rb.r, off, 0, 0);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; i += 2) rb.store_pair(n + i, make_float2(v[i], v[i + 1]));
  }
}

// True when a row set with this base pointer and row stride (elements) can use
// the ALIGNED pair accesses for rows of `valid` elements.
template <int DT>
inline bool pairs_aligned(const void* base, int64_t stride, int64_t valid) {
  using ET = typename Elem<DT>::T;
  return base != nullptr && (reinterpret_cast<uintptr_t>(base) % (2 * sizeof(ET))) == 0 && stride % 2 == 0 &&
         valid % 2 == 0 && valid >= 2;
}

// Stores (v.x, v.y) at row[i], row[i+1] for the indices below `valid`.
template <int DT>
__device__ __forceinline__ void store_pair(typename Elem<DT>::T* __restrict__ row, int64_t i, int64_t valid, float2 v) {
  using ET = typename Elem<DT>::T;
  ET* p = row + i;
  if (i + 1 < valid && (reinterpret_cast<uintptr_t>(p) & (2 * sizeof(ET) - 1)) == 0) {
    if constexpr (DT == NSQ_DTYPE_F32) {
      *reinterpret_cast<float2*>(p) = v;
    } else if constexpr (DT == NSQ_DTYPE_BF16) {
      *reinterpret_cast<uint32_t*>(p) = f32x2_to_bf16x2_bits(v.x, v.y);
    } else {
      *reinterpret_cast<__half2*>(p) = __floats2half2_rn(v.x, v.y);
    }
    return;
  }
  if (i < valid) Elem<DT>::store(row, i, v.x);
  if (i + 1 < valid) Elem<DT>::store(row, i + 1, v.y);
}

}  // namespace nsq
