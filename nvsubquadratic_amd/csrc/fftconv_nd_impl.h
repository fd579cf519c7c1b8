// Non-causal "same" 2D / 3D FFT convolution (forward and backward), gfx950.
//
// Semantics: nvsubquadratic/ops/fftconv.py:662-733 (fftconv2d_fp32_bhl) and
// :736-812 (fftconv3d_fp32_bhl): zero-padded linear convolution, crop
// [K_d//2, K_d//2 + S_d) per axis, cast to x.dtype, + shortcut * x.  Any FFT
// length F_d >= S_d + ceil(K_d/2) gives the reference's result exactly (no
// aliasing reaches the cropped window), so each axis uses the next power of two.
//
// Periodic axes (circular / mixed boundaries, nvsubquadratic/ops/
// circular_fftconv.py, mixed_fftconv.py) use F_d = S_d, no crop, and a shift
// ramp on the filter spectrum (nd_col_mul RAMP); see the plan in
// fftconv_nd.hip.
//
// Plan: the spectrum of one (b, h) image / volume is laid out in a workspace
// block as [F0][F1][F2/2 + 1] (3D) or [F0][F2/2] (2D, F1 = 1: the rows' real DC
// and Nyquist bins packed in bin 0, see pack_split) for the last (contiguous,
// real) axis.  Passes:
//   nd_row_fwd : real FFT along the last axis of the valid rows;
//   nd_col     : complex FFT along axis 0 or 1 (strided), reading only the valid
//                input rows (the rest is implicit zero padding) and writing
//                either all F_d outputs (forward) or a cropped window moved to
//                the front of the column (inverse);
//   nd_col_mul : forward FFT along axis 0, spectral product, inverse FFT along
//                axis 0 and crop, in one kernel (forward conv);
//   nd_col_bwd : the same for the adjoint: P = G conj(K) R, Q = sum_b G conj(X) R,
//                R = exp(-2 pi i sum_d c_d k_d / F_d) places g at the crop
//                offset c_d (shift theorem), so gx and gk come out at window 0;
//   nd_row_inv : inverse real FFT along the last axis, crop and epilogue.
// Column passes map lanes to consecutive inner indices (coalesced row segments).
#pragma once

#include "fft_core.h"
#include "fft_wave128.h"
#include "gate.h"

namespace nsq {

// ---------------------------------------------------------------------------
// Hyena gates inside the first and last passes (GATED_* of gate.h; the gated
// ops of fftconv_nd_gated.hip): z = q act1(kg), or dy1 = g act2(v), formed as
// the first pass loads its sample pairs; gate 2, or dq, dkg, dv, in the last
// pass's epilogue (16-byte operand windows there: dv's scattered stores from
// the loader cost more than its extra y1 window).
// ---------------------------------------------------------------------------
// Sample pair (i, i + 1) of the row at element offset roff of the first pass's
// source (src, then q or g; the second operand kg or v from gi).  Samples at
// or past `valid` read zero, and every gate maps zero to zero.
template <int DT, bool AL, int GL>
__device__ __forceinline__ float2 gated_pair(const typename Elem<DT>::T* __restrict__ src, const GatedIO& gi,
                                             int64_t roff, int64_t i, int64_t valid) {
  using ET = typename Elem<DT>::T;
  const float2 a = load_pair_nb<DT, AL>(src + roff, i, valid);
  if constexpr (GL == GATED_NONE) {
    return a;
  } else {
    const float2 b = load_pair_nb<DT, AL>((const ET*)(GL == GATED_FWD ? gi.kg : gi.v) + roff, i, valid);
    return make_float2(gated_input<DT, GL>(gi.act1, gi.act2, a.x, b.x),
                       gated_input<DT, GL>(gi.act1, gi.act2, a.y, b.y));
  }
}

// ---------------------------------------------------------------------------
// Real row passes along the last axis (element-major tiles, M rows per WG).
// ---------------------------------------------------------------------------
template <int LOGN>
struct RowNdCfg {
  static constexpr int N = 1 << LOGN;  // packed complex length = F2 / 2
  static constexpr int M = LOGN >= 11 ? 1 : (2048 >> LOGN);
  static constexpr int SP = Padded<N>::SIZE;
  static constexpr int T = (M * N) / 16;
  static constexpr int SLOTS = 8;
};

// Rows are flattened over (bh, a0 < n0, a1 < n1).  The host keeps the row
// count of a pass below 2^31, so the decomposition is 32-bit arithmetic (a
// 64-bit division is a long instruction sequence, and it runs per slot).
struct RowIdx {
  int bh;
  int a0, a1;
};
__device__ __forceinline__ RowIdx row_index(int64_t r64, int n0, int n1) {
  const uint32_t r = uint32_t(r64);
  const uint32_t t = r / uint32_t(n1);
  RowIdx o;
  o.a1 = int(r - t * uint32_t(n1));
  o.bh = int(t / uint32_t(n0));
  o.a0 = int(t - uint32_t(o.bh) * uint32_t(n0));
  return o;
}

// Row block geometry shared by the row passes.
struct RowGeom {
  int64_t rows;  // bh * n0 * n1
  int n0, n1;    // valid counts of axes 0 and 1 for these rows
  int64_t spec;  // spectrum block size (complex elements)
  int F1, RS;    // rows per axis-0 index; spectrum row stride (complex elements)
};

// Forward real FFT of rows of a contiguous [BH][n0][n1][len] real tensor,
// zero-padded to F2 = 2N, into workspace bins [0, FH) of row (a0, a1).
// AL: aligned pair access (even len, aligned base; see load_pair_nb).
// HALF: len <= N (at least half of each row is zero padding): the first pass
// folds the zero half (HalfZeroLoad).  PACK (2D spectra): N bins per row, the
// real DC and Nyquist values packed in bin 0 as U[0] + i U[N] (see
// pack_split); otherwise N + 1 bins.  wm: sample index mask, -1, or len - 1
// for a periodic row of a power-of-two length len < F2 read as its periodic
// extension (sample i of the transform is row[i & wm]).
// GL: gate formed as the pairs are loaded (gated_pair; src is then q or g).
template <int LOGN, int DT, bool AL, bool HALF = false, bool PACK = false, int GL = GATED_NONE>
__global__ __launch_bounds__(RowNdCfg<LOGN>::T) void nd_row_fwd_kernel(const typename Elem<DT>::T* __restrict__ src,
                                                                        int len, int wm, RowGeom rg,
                                                                        float2* __restrict__ ws,
                                                                        const float2* __restrict__ tw, GatedIO gi) {
  using C = RowNdCfg<LOGN>;
  __shared__ float2 lds[C::M * C::SP];
  __shared__ int64_t rowoff[C::M];  // spectrum row of each tile row (one index decomposition per row)
  const int64_t r0 = int64_t(blockIdx.x) * C::M;
  const int tslot = opaque_tid();  // once: the asm statement would order the unrolled loads
  for (int m = tslot; m < C::M; m += C::T) {  // ordered before its use by the transform's barriers
    const int64_t r = r0 + m;
    const RowIdx q = row_index(r < rg.rows ? r : 0, rg.n0, rg.n1);
    rowoff[m] = int64_t(q.bh) * rg.spec + (int64_t(q.a0) * rg.F1 + q.a1) * rg.RS;
  }
  auto ld = [&](int m, int n) -> float2 {
    const int64_t r = r0 + m;
    const bool rok = r < rg.rows;  // tail rows read row 0 and select zero
    return gated_pair<DT, AL, GL>(src, gi, (rok ? r : 0) * len, (2 * int64_t(n)) & wm, rok ? len : 0);
  };
  HalfZeroLoad<(LOGN < 4 ? (1 << LOGN) : 16), HALF, decltype(ld)> ld1{ld};
  LdsTile<C::SP, true> st{lds};
  fft<LOGN, false, C::M, C::T, C::SP>(lds, ld1, st, tw);
#pragma unroll
  for (int i = 0; i < C::SLOTS; ++i) {
    const int s = tslot + i * C::T;
    const int m = s >> (LOGN - 1), p = s & (C::N / 2 - 1);
    const int64_t r = r0 + m;
    if (r >= rg.rows) continue;
    const float2* zz = lds + m * C::SP;
    const bool slot0 = (p == 0);
    float2 A, Bc;
    real_unpack(slot0, zz[pad16(p)], zz[pad16(slot0 ? C::N / 2 : C::N - p)],
                root<LOGN + 1>(tw, p), A, Bc);
    float2* out = ws + rowoff[m];
    if (slot0) {
      if constexpr (PACK) {
        out[0] = A;
      } else {
        out[0] = make_float2(A.x, 0.f);
        out[C::N] = make_float2(A.y, 0.f);
      }
      out[C::N / 2] = Bc;
    } else {
      out[p] = A;
      out[C::N - p] = cconj(Bc);
    }
  }
}

// Output epilogues of the inverse row pass.
enum { ND_OUT_Y = 0, ND_OUT_GK = 1 };

struct RowInvOut {
  void* out;           // [rows][w2] (dtype for ND_OUT_Y, float for ND_OUT_GK)
  const void* aux;     // x (forward) or g (backward) with the layout of `out` (ND_OUT_Y)
  const void* s;       // shortcut [H] (ND_OUT_Y, may be null)
  float* gs;           // [rows / (n0*n1)] lag-c value (ND_OUT_GK, may be null)
  int H;               // channels (shortcut index = bh % H)
  int off2, w2;        // last-axis window [off2, off2 + w2)
  int ga0, ga1, ga2;   // lag whose value is the shortcut gradient (ND_OUT_GK)
  float scale;         // 1 / (F0 * F1 * F2/2)
  GatedIO gio;        // gated epilogues (GE != GATED_NONE; aux is then q or g)
};

// HAS_S: a shortcut is given (ND_OUT_Y); its term reads aux.  Loads are
// branch-free (clamped indices, zero selected) so they overlap; only stores
// are predicated.  FAST (ND_OUT_Y; even off2, w2 a multiple of 8, out and aux
// 16-byte aligned): the epilogue moves 8 consecutive kept samples per thread,
// four complex values from LDS, one 16-byte aux load and one 16-byte store.
// GE (FAST only): gated epilogue (gated_output; o.aux is q or g, the other
// operands and the second output in o.gio, all with the layout of `out`).
template <int LOGN, int DT, int MODE, bool HAS_S, bool FAST = false, bool PACK = false, int GE = GATED_NONE>
__global__ __launch_bounds__(RowNdCfg<LOGN>::T) void nd_row_inv_kernel(const float2* __restrict__ ws, RowGeom rg,
                                                                        RowInvOut o, const float2* __restrict__ tw) {
  using C = RowNdCfg<LOGN>;
  using ET = typename Elem<DT>::T;
  __shared__ float2 lds[C::M * C::SP];
  __shared__ int64_t rowoff[C::M];  // spectrum row of each tile row (one index decomposition per row)
  const int64_t r0 = int64_t(blockIdx.x) * C::M;
  const int tslot = opaque_tid();  // once: the asm statement would order the unrolled loads
  // every tile row (short rows give tiles of more rows than threads)
  for (int m = tslot; m < C::M; m += C::T) {
    const int64_t r = r0 + m;
    const RowIdx q = row_index(r < rg.rows ? r : 0, rg.n0, rg.n1);
    rowoff[m] = int64_t(q.bh) * rg.spec + (int64_t(q.a0) * rg.F1 + q.a1) * rg.RS;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < C::SLOTS; ++i) {
    const int s = tslot + i * C::T;
    const int m = s >> (LOGN - 1), p = s & (C::N / 2 - 1);
    const int64_t r = r0 + m;
    const bool rok = r < rg.rows;
    const bool slot0 = (p == 0);
    const float2* in = ws + rowoff[m];
    const float2 u0 = in[slot0 ? 0 : p];
    const float2 u1 = in[slot0 ? (PACK ? 0 : C::N) : C::N - p];  // PACK: no bin N (row stride may be N)
    const float2 u2 = in[C::N / 2];
    float2 A = slot0 ? (PACK ? u0 : make_float2(u0.x, u1.x)) : u0;
    float2 Bc = slot0 ? u2 : cconj(u1);
    A = make_float2(rok ? A.x : 0.f, rok ? A.y : 0.f);
    Bc = make_float2(rok ? Bc.x : 0.f, rok ? Bc.y : 0.f);
    float2 zp, zq;
    real_repack(slot0, A, Bc, root<LOGN + 1>(tw, p), zp, zq);
    float2* zz = lds + m * C::SP;
    zz[pad16(p)] = zp;
    zz[pad16(slot0 ? C::N / 2 : C::N - p)] = zq;
  }
  __syncthreads();
  // Inverse in place, then a batched epilogue: the real samples of row m are
  // (u[2n], u[2n+1]) = (z[n].x, z[n].y); a thread issues the shortcut loads of
  // 8 outputs before their stores (in a store functor of the last pass each
  // load would wait behind the previous stores).
  LdsTile<C::SP, true> tile{lds};
  fft_rec<LOGN, 0, true, C::M, C::T, false>(tile, tile, tile, tile, tw);
  __shared__ float svs[C::M];  // shortcut value of each tile row
  const ET* __restrict__ aux = (const ET*)o.aux;
  if constexpr (MODE == ND_OUT_Y && HAS_S) {
    for (int m = tslot; m < C::M; m += C::T) {
      const int64_t r = r0 + m;
      const RowIdx q = row_index(r < rg.rows ? r : 0, rg.n0, rg.n1);
      svs[m] = Elem<DT>::round(Elem<DT>::load((const ET*)o.s, q.bh % o.H));
    }
    __syncthreads();
  }
  const int nrows = (rg.rows - r0) < C::M ? int(rg.rows - r0) : C::M;
  const int nvalid = nrows * o.w2;  // the tile's outputs are e in [0, nvalid), row-major
  const int64_t tbase = r0 * o.w2;   // 32-bit offsets from here (M * w2 is small)
  const ET* aux_t = aux + (HAS_S ? tbase : 0);
  static_assert(GE == GATED_NONE || (FAST && MODE == ND_OUT_Y), "nd_row_inv_kernel: gates need the FAST epilogue");
  if constexpr (FAST) {
    static_assert(MODE == ND_OUT_Y, "nd_row_inv_kernel: FAST epilogue writes y");
    const int cpr = o.w2 >> 3;  // 8-sample chunks per row
    // operands of the gate formed here (a: aux, q or g; b: kg or v), the others (c: v or q; d: kg; e: y1); the
    // forward reads a and b only for the shortcut term, the backward always (dv)
    constexpr bool BWD = GE == GATED_BWD;
    const bool need_ab = HAS_S || BWD;
    const ET* a_t = aux + tbase;
    const ET* gb = (const ET*)(GE == GATED_FWD ? o.gio.kg : o.gio.v);
    const ET* gc = (const ET*)(GE == GATED_FWD ? o.gio.v : o.gio.q);
    const RowBuf<DT, false> ab(need_ab ? a_t : aux_t, need_ab ? nvalid : 0);
    const RowBuf<DT, false> bb(GE != GATED_NONE && need_ab ? gb + tbase : aux_t,
                               GE != GATED_NONE && need_ab ? nvalid : 0);
    const RowBuf<DT, false> cb(GE != GATED_NONE ? gc + tbase : aux_t, GE != GATED_NONE ? nvalid : 0);
    const RowBuf<DT, false> db(BWD ? (const ET*)o.gio.kg + tbase : aux_t, BWD ? nvalid : 0);
    const RowBuf<DT, false> eb(BWD ? (const ET*)o.gio.y1 + tbase : aux_t, BWD ? nvalid : 0);
    void* out2 = GE == GATED_FWD ? o.gio.y1out : o.gio.dkg;
    const RowBuf<DT, true> ob((ET*)o.out + tbase, nvalid);
    const RowBuf<DT, true> ob2(out2 ? (ET*)out2 + tbase : (ET*)o.out + tbase, out2 ? nvalid : 0);
    const RowBuf<DT, true> ob3(BWD ? (ET*)o.gio.dv + tbase : (ET*)o.out + tbase, BWD ? nvalid : 0);
    for (int ch = tslot; ch < C::M * cpr; ch += C::T) {
      const int m = ch / cpr, c8 = (ch - m * cpr) * 8;
      const bool ok = m < nrows;
      const int e0 = ok ? m * o.w2 + c8 : nvalid;  // past the range: the aux load reads 0, the store is dropped
      Win8<DT, true> a, b, c, d, ew;
      a.load(ab, e0);
      if constexpr (GE != GATED_NONE) {
        b.load(bb, e0);
        c.load(cb, e0);
      }
      if constexpr (BWD) {
        d.load(db, e0);
        ew.load(eb, e0);
      }
      const float2* zr = lds + (ok ? m : 0) * C::SP;
      const int n0 = (c8 + o.off2) >> 1;
      float y[8], y2[8], y3[8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float2 z = zr[pad16(n0 + u)];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int i = 2 * u + h;
          const float cv = (h ? z.y : z.x) * o.scale;
          if constexpr (GE == GATED_NONE) {
            y[i] = epilogue<DT>(cv, HAS_S, HAS_S ? svs[m] : 0.f, a.at(i));
          } else {
            y[i] = gated_output<DT, GE>(cv, HAS_S, HAS_S ? svs[m] : 0.f, a.at(i), b.at(i), c.at(i),
                                        BWD ? d.at(i) : 0.f, BWD ? ew.at(i) : 0.f, o.gio.act1, o.gio.act2, y2[i],
                                        y3[i]);
          }
        }
      }
      store8<DT, true>(ob, e0, y);
      if constexpr (GE != GATED_NONE) {
        if (out2) store8<DT, true>(ob2, e0, y2);
      }
      if constexpr (BWD) store8<DT, true>(ob3, e0, y3);
    }
    return;
  }
  // (row, column) of output e = eb + tslot + u*T for the LDS read, stepped without division
  int m_next = tslot / o.w2, c_next = tslot - m_next * o.w2;
  for (int eb = 0; eb < C::M * o.w2; eb += 8 * C::T) {
    float a[8], v[8];
    int mm[8], cc[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      mm[u] = m_next;
      cc[u] = c_next;
      c_next += C::T;
      while (c_next >= o.w2) {
        c_next -= o.w2;
        ++m_next;
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = eb + tslot + u * C::T;
      const bool ok = e < nvalid;
      const int sidx = cc[u] + o.off2;  // sample index in the row
      const float2 zz = lds[(ok ? mm[u] : 0) * C::SP + pad16(sidx >> 1)];
      v[u] = ((sidx & 1) ? zz.y : zz.x) * o.scale;
      a[u] = 0.f;
      if constexpr (MODE == ND_OUT_Y && HAS_S) a[u] = Elem<DT>::load(aux_t, ok ? e : 0);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = eb + tslot + u * C::T;
      if (e >= nvalid) continue;
      if constexpr (MODE == ND_OUT_Y) {
        Elem<DT>::store((ET*)o.out + tbase, e, epilogue<DT>(v[u], HAS_S, HAS_S ? svs[mm[u]] : 0.f, a[u]));
      } else {
        ((float*)o.out + tbase)[e] = v[u];
        if (o.gs && cc[u] == o.ga2) {
          const RowIdx q = row_index(r0 + mm[u], rg.n0, rg.n1);
          if (q.a0 == o.ga0 && q.a1 == o.ga1) o.gs[q.bh] = v[u];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Plane passes (3D): the two inner axes of one (b, h, a0) plane in LDS, used
// when a plane fits (PlaneCfg::OK).  A plane is F1 rows of a packed real-row
// spectrum: row a1 holds V[0..N), V[p] = U[p] for 1 <= p < N and V[0] =
// U[0] + i U[N] (the row's real DC and Nyquist bins packed in one complex).
// Along axis 1 the packed column transforms to Z = A + i B (A, B the
// transforms of the real columns U[0], U[N]), separated with the Hermitian
// pairing A[k] = (Z[k] + conj Z[-k]) / 2, B[k] = (Z[k] - conj Z[-k]) / 2i.
// The forward pass replaces nd_row_fwd + the axis-1 nd_col pass, the inverse
// the axis-1 inverse nd_col pass + nd_row_inv: one spectrum round trip each
// instead of two.
// ---------------------------------------------------------------------------
template <int LOGN, int LOGF1>
struct PlaneCfg {
  static constexpr int N = 1 << LOGN;          // packed row length F2 / 2
  static constexpr int F1 = 1 << LOGF1;
  static constexpr int FH = N + 1;
  static constexpr int RS = Padded<N>::SIZE;   // LDS row stride
  static constexpr int T = 256;
  static constexpr int MR = (16 * T) >> LOGN;  // rows per row-transform tile
  static constexpr int MC = (16 * T) >> LOGF1; // columns per column-transform tile
  static constexpr int SLOTS = 8;              // MR * N / 2 slots per tile / T
  static constexpr bool OK = LOGN >= 4 && LOGF1 >= 4 && MR >= 1 && MR <= F1 && MC >= 1 && MC <= N &&
                             F1 * RS * 8 <= 80 * 1024;
};

// HALF: len <= N and n1 <= F1/2 (each row and each column at least half zero
// padding): both first passes fold the zero half (HalfZeroLoad).  GL: gate
// formed as the pairs are loaded (gated_pair; src is then q or g).
template <int LOGN, int LOGF1, int DT, bool AL, bool HALF = false, int GL = GATED_NONE>
__global__ __launch_bounds__(256) void nd_plane_fwd_kernel(const typename Elem<DT>::T* __restrict__ src, int n0,
                                                           int n1, int len, int wm1, int wm2, float2* __restrict__ ws,
                                                           int64_t spec, const float2* __restrict__ tw, GatedIO gi) {
  using C = PlaneCfg<LOGN, LOGF1>;
  static_assert(C::OK, "nd_plane_fwd_kernel: plane does not fit");
  constexpr int N = C::N, RS = C::RS;
  __shared__ float2 P[C::F1 * RS];
  const int64_t plane = blockIdx.x;  // bh * n0 + a0
  const int64_t xoff = plane * n1 * len;
  // Axis 2: real transforms of the valid rows, unpacked in place to V.
  for (int r0 = 0; r0 < n1; r0 += C::MR) {
    LdsTile<RS, true> rows{P + r0 * RS};
    auto ld = [&](int m, int n) -> float2 {
      const int a1 = r0 + m;
      const bool ok = a1 < n1;
      return gated_pair<DT, AL, GL>(src, gi, xoff + int64_t(ok ? a1 : 0) * len, (2 * int64_t(n)) & wm2,
                                    ok ? len : 0);
    };
    HalfZeroLoad<16, HALF, decltype(ld)> ld1{ld};  // LOGN >= 4: radix-16 first pass
    fft_rec<LOGN, 0, false, C::MR, C::T, false>(ld1, rows, rows, rows, tw);
    const int tslot = opaque_tid();  // once: the asm statement would order the unrolled loads
#pragma unroll
    for (int i = 0; i < C::SLOTS; ++i) {
      const int s = tslot + i * C::T;
      const int m = s >> (LOGN - 1), p = s & (N / 2 - 1);
      const bool p0 = (p == 0);
      float2* z = P + (r0 + m) * RS;
      const int pb = pad16(p0 ? N / 2 : N - p);
      float2 A, Bc;
      real_unpack(p0, z[pad16(p)], z[pb], root<LOGN + 1>(tw, uint32_t(p)), A, Bc);
      z[pad16(p)] = A;                          // p = 0: U[0] + i U[N]
      z[pb] = p0 ? Bc : cconj(Bc);              // U[N/2] or U[N-p]
    }
    __syncthreads();
  }
  // Axis 1: complex transforms of the N packed columns; rows >= n1 are zero.
  for (int j0 = 0; j0 < N; j0 += C::MC) {
    LdsCols<RS> cols{P, j0};
    auto ld = [&](int m, int n) -> float2 {
      n &= wm1;  // periodic extension of a short axis 1
      const bool ok = n < n1;
      const float2 v = P[(ok ? n : 0) * RS + pad16(j0 + m)];
      return make_float2(ok ? v.x : 0.f, ok ? v.y : 0.f);
    };
    HalfZeroLoad<16, HALF, decltype(ld)> ld1{ld};  // LOGF1 >= 4: radix-16 first pass
    fft_rec<LOGF1, 0, false, C::MC, C::T, true>(ld1, cols, cols, cols, tw);
  }
  // Store [F1][FH]; column 0 separates into the DC (j = 0) and Nyquist (j = N) bins.
  float2* out = ws + (plane / n0) * spec + (plane % n0) * int64_t(C::F1) * C::FH;
  const int tst = opaque_tid();
  static_assert((C::F1 * N) % C::T == 0, "nd_plane_fwd_kernel: store batches");
#pragma unroll 4
  for (int e = tst; e < C::F1 * N; e += C::T) {  // bins 1 .. N-1 of each row as they are
    const int k1 = e >> LOGN, j = e & (N - 1);
    const float2 v = P[k1 * RS + pad16(j)];
    if (j != 0) out[int64_t(k1) * C::FH + j] = v;
  }
  for (int k1 = tst; k1 < C::F1; k1 += C::T) {  // packed column 0 -> DC (j = 0) and Nyquist (j = N)
    const float2 v = P[k1 * RS];
    const float2 zc = cconj(P[((C::F1 - k1) & (C::F1 - 1)) * RS]);
    out[int64_t(k1) * C::FH] = cscale(cadd(v, zc), 0.5f);
    out[int64_t(k1) * C::FH + N] = mul_neg_i(cscale(csub(v, zc), 0.5f));
  }
}

// Inverse: plane [F1][FH] of the spectrum (after the axis-0 pass) -> inverse
// along axis 1, rows [off1, off1 + n1out) -> inverse real transforms along
// axis 2, crop and epilogue (RowInvOut; output rows [plane][n1out][w2]).
// GE: gated epilogue (gated_output; o.aux is q or g, the other operands and
// the second output in o.gio).
template <int LOGN, int LOGF1, int DT, int MODE, bool HAS_S, int GE = GATED_NONE>
__global__ __launch_bounds__(256) void nd_plane_inv_kernel(const float2* __restrict__ ws, int64_t spec, int n0,
                                                           int off1, int n1out, RowInvOut o,
                                                           const float2* __restrict__ tw) {
  using C = PlaneCfg<LOGN, LOGF1>;
  static_assert(C::OK, "nd_plane_inv_kernel: plane does not fit");
  using ET = typename Elem<DT>::T;
  constexpr int N = C::N, RS = C::RS;
  __shared__ float2 P[C::F1 * RS];
  const int64_t plane = blockIdx.x;  // bh * n0 + a0
  const int64_t bh = plane / n0;
  const int a0 = int(plane % n0);
  const float2* in = ws + bh * spec + int64_t(a0) * C::F1 * C::FH;
  // Load the plane (unrolled so that the loads of a batch are in flight
  // together), then pack DC + i * Nyquist into column 0.
  static_assert((C::F1 * N) % (8 * C::T) == 0, "nd_plane_inv_kernel: load batches");
  // One read of the thread index for the batched loops: opaque_tid is an asm
  // statement, which the scheduler does not move loads across.
  const int t = opaque_tid();
#pragma unroll 8
  for (int it = 0; it < C::F1 * N / C::T; ++it) {
    const int e = t + it * C::T;
    const int k1 = e >> LOGN, j = e & (N - 1);
    P[k1 * RS + pad16(j)] = in[int64_t(k1) * C::FH + j];
  }
  __syncthreads();
  for (int k1 = t; k1 < C::F1; k1 += C::T) {
    const float2 w = in[int64_t(k1) * C::FH + N];
    const float2 v = P[k1 * RS];
    P[k1 * RS] = make_float2(v.x - w.y, v.y + w.x);
  }
  __syncthreads();
  // Axis 1 inverse; the last pass keeps rows [off1, off1 + n1out), moved to the front.
  for (int j0 = 0; j0 < N; j0 += C::MC) {
    LdsCols<RS> cols{P, j0};
    auto st = [&](int m, int k, float2 v) {
      const int r = k - off1;
      if (r >= 0 && r < n1out) P[r * RS + pad16(j0 + m)] = v;
    };
    fft_rec<LOGF1, 0, true, C::MC, C::T, true>(cols, cols, cols, st, tw);
  }
  // Axis 2: repack each kept row, invert it in LDS, then the epilogue reads the
  // real samples back (u[2n], u[2n+1]) = (z[n].x, z[n].y), crops, and stores;
  // all of a thread's shortcut loads are issued before its stores.
  const ET* __restrict__ aux = (const ET*)o.aux;
  const ET* __restrict__ sh = (const ET*)o.s;
  const int h = int(bh % o.H);
  const float sv = HAS_S ? Elem<DT>::round(Elem<DT>::load(sh, h)) : 0.f;
  // FAST epilogue: even window start, w2 a multiple of 8, 16-byte aligned rows.
  const bool fast = (o.off2 & 1) == 0 && (o.w2 & 7) == 0 && o.w2 <= 2 * N &&
                    ((reinterpret_cast<uintptr_t>(o.out) | (HAS_S ? reinterpret_cast<uintptr_t>(o.aux) : 0)) & 15) == 0;
  for (int r0 = 0; r0 < n1out; r0 += C::MR) {
#pragma unroll
    for (int i = 0; i < C::SLOTS; ++i) {
      const int s = t + i * C::T;
      const int m = s >> (LOGN - 1), p = s & (N / 2 - 1);
      const bool p0 = (p == 0);
      float2* z = P + (r0 + m) * RS;
      const int pb = pad16(p0 ? N / 2 : N - p);
      const float2 b = z[pb];
      float2 zp, zq;
      real_repack(p0, z[pad16(p)], p0 ? b : cconj(b), root<LOGN + 1>(tw, uint32_t(p)), zp, zq);
      z[pad16(p)] = zp;
      z[pb] = zq;
    }
    __syncthreads();
    LdsTile<RS, true> rows{P + r0 * RS};
    fft_rec<LOGN, 0, true, C::MR, C::T, false>(rows, rows, rows, rows, tw);
    // Epilogue over the tile's real samples: MR rows x w2 kept samples.
    const int nrows = (n1out - r0) < C::MR ? (n1out - r0) : C::MR;
    static_assert(GE == GATED_NONE || MODE == ND_OUT_Y, "nd_plane_inv_kernel: gates on y only");
    if constexpr (MODE == ND_OUT_Y && GE == GATED_NONE) {
      if (fast) {
        // 8 consecutive kept samples per thread: four complex values from LDS,
        // one 16-byte shortcut load, one 16-byte store.  Chunk ch of the tile
        // is row ch / cpr (a float reciprocal: ch < 2^14, so the quotient's
        // rounding error stays far below the 1 / (2 cpr) margin of ch + 1/2).
        const int cpr = o.w2 >> 3;
        const float rcpr = 1.f / float(cpr);
        const int64_t row0 = plane * n1out + r0;
        const RowBuf<DT, false> ab(aux + row0 * o.w2, HAS_S ? nrows * o.w2 : 0);
        const RowBuf<DT, true> ob((ET*)o.out + row0 * o.w2, nrows * o.w2);
        for (int ch = t; ch < nrows * cpr; ch += C::T) {
          const int m = int((float(ch) + 0.5f) * rcpr), c8 = (ch - m * cpr) * 8;
          const int e0 = m * o.w2 + c8;
          Win8<DT, true> a{};
          if constexpr (HAS_S) a.load(ab, e0);
          const float2* zr = P + (r0 + m) * RS;
          const int nc = (c8 + o.off2) >> 1;  // first complex value of the chunk
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
        continue;
      }
    }
    constexpr bool BWD = GE == GATED_BWD;
    const ET* __restrict__ gb = (const ET*)(GE == GATED_FWD ? o.gio.kg : o.gio.v);
    const ET* __restrict__ gc = (const ET*)(GE == GATED_FWD ? o.gio.v : o.gio.q);
    const ET* __restrict__ gd = (const ET*)o.gio.kg;
    const ET* __restrict__ ge = (const ET*)o.gio.y1;
    ET* out2 = (ET*)(GE == GATED_FWD ? o.gio.y1out : o.gio.dkg);
    for (int eb = 0; eb < C::MR * o.w2; eb += 8 * C::T) {
      float a[8], v[8], b[8], c2[8], d[8], e2[8];
      int64_t idx[8];
      bool ok[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = eb + t + u * C::T;
        const int m = e / o.w2, c = e - m * o.w2;
        ok[u] = m < nrows;
        const int sidx = c + o.off2;  // sample index in the row
        const float2 zz = P[(r0 + (ok[u] ? m : 0)) * RS + pad16(sidx >> 1)];
        v[u] = ((sidx & 1) ? zz.y : zz.x) * o.scale;
        idx[u] = (plane * n1out + r0 + (ok[u] ? m : 0)) * o.w2 + c;
        const int64_t li = ok[u] ? idx[u] : 0;
        a[u] = b[u] = c2[u] = d[u] = e2[u] = 0.f;
        if constexpr (HAS_S || BWD) a[u] = Elem<DT>::load(aux, li);
        if constexpr (GE != GATED_NONE) {
          if constexpr (HAS_S || BWD) b[u] = Elem<DT>::load(gb, li);
          c2[u] = Elem<DT>::load(gc, li);
        }
        if constexpr (BWD) {
          d[u] = Elem<DT>::load(gd, li);
          e2[u] = Elem<DT>::load(ge, li);
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (!ok[u]) continue;
        if constexpr (MODE == ND_OUT_Y) {
          if constexpr (GE == GATED_NONE) {
            Elem<DT>::store((ET*)o.out, idx[u], epilogue<DT>(v[u], HAS_S, sv, a[u]));
          } else {
            float y2, y3;
            Elem<DT>::store((ET*)o.out, idx[u],
                            gated_output<DT, GE>(v[u], HAS_S, sv, a[u], b[u], c2[u], d[u], e2[u], o.gio.act1,
                                                 o.gio.act2, y2, y3));
            if (out2) Elem<DT>::store(out2, idx[u], y2);
            if constexpr (BWD) Elem<DT>::store((ET*)o.gio.dv, idx[u], y3);
          }
        } else {
          ((float*)o.out)[idx[u]] = v[u];
          const int e = eb + t + u * C::T;
          const int m = e / o.w2, c = e - m * o.w2;
          if (o.gs && c == o.ga2 && a0 == o.ga0 && r0 + m == o.ga1) o.gs[bh] = v[u];
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Column passes along axis 0 or 1 (strided; TMAJOR tiles of M columns).
// ---------------------------------------------------------------------------
// M columns per workgroup (tile of about TARGET points), 16 points per thread.
template <int LOGF, int TARGET = 8192>
struct ColNdCfg {
  static constexpr int F = 1 << LOGF;
  static constexpr int M = (TARGET >> LOGF) < 4 ? 4 : ((TARGET >> LOGF) > 16 ? 16 : (TARGET >> LOGF));
  static constexpr int S = F + 1;
  static constexpr int TILE = M * F;
  static constexpr int T = TILE / 16;
};
constexpr int kNdBwdTile = 4096;  // three tiles in LDS for the adjoint pass
template <int LOGF>
using ColNdBwdCfg = ColNdCfg<LOGF, kNdBwdTile>;
constexpr int kNdMaxLogF = 10;    // 2D/3D axes: FFT length <= 1024

// Column block geometry: column (o, j) with o = bh * n_mid + mid and inner
// index j < inner_count starts at ws + bh*spec + mid*mid_stride + j; element
// n of the column is at stride axis_stride.
struct ColGeom {
  int n_mid;
  int64_t mid_stride;
  int64_t spec;
  int64_t axis_stride;
  int inner_count;
};

__device__ __forceinline__ int64_t col_base(const ColGeom& cg, int64_t o) {
  return (o / cg.n_mid) * cg.spec + (o % cg.n_mid) * cg.mid_stride;
}

// A column group of one workspace block as a raw buffer resource: element n
// of inner column j is at byte n * 8 * axis_stride + 8 j from the block base.
// Offsets are 32-bit (a block spans < 2^31 bytes) and the n * stride product
// is a 24-bit multiply (axis lengths <= 2^10, strides < 2^21 elements), so a
// pass's address math is one multiply-add and one select per element.  An
// access the caller marks invalid (column past inner_count, element outside
// the read or write window) uses offset 2^31, past the range: loads read zero
// and stores are dropped, with no branch, so a pass's loads stay in flight
// together.
struct ColBuf {
  __amdgpu_buffer_rsrc_t r;
  uint32_t stride8;
  __device__ __forceinline__ ColBuf(const float2* base, const ColGeom& cg)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<float2*>(base), 0, 0x7fffffff, 0x00020000)),
        stride8(uint32_t(cg.axis_stride) * 8u) {}
  __device__ __forceinline__ int off(int n, int j, bool ok) const {
    int o = ok ? int(__umul24(uint32_t(n), stride8) + 8u * uint32_t(j)) : int(0x80000000u);
    asm volatile("" : "+v"(o));  // keep the offset whole (no constant folded into the immediate)
    return o;
  }
  __device__ __forceinline__ float2 load(int n, int j, bool ok) const {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, off(n, j, ok), 0, 0));
  }
  __device__ __forceinline__ void store(int n, int j, bool ok, float2 v) const {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(uint32_t __attribute__((ext_vector_type(2))), v), r,
                                          off(n, j, ok), 0, 0);
  }
};

// Generic pass: reads elements [0, in_cnt) (rest zero; element n is read at
// n & wm, wm = -1 or the mask of a short periodic axis), transforms, writes
// outputs [out_off, out_off + out_cnt) to positions [0, out_cnt).
// grid = (n_outer, ceil(inner_count / M)).
template <int LOGF, bool INV, int TARGET = 8192>
__global__ __launch_bounds__((ColNdCfg<LOGF, TARGET>::T)) void nd_col_kernel(float2* __restrict__ ws, ColGeom cg,
                                                                            int in_cnt, int wm, int out_off,
                                                                            int out_cnt, int jbase,
                                                                            const float2* __restrict__ tw) {
  using C = ColNdCfg<LOGF, TARGET>;
  __shared__ float2 lds[C::M * C::S];
  const ColBuf cb(ws + col_base(cg, blockIdx.x), cg);
  const int j0 = jbase + blockIdx.y * C::M;
  auto ld = [&](int m, int n) -> float2 {
    n &= wm;
    return cb.load(n, j0 + m, j0 + m < cg.inner_count && n < in_cnt);
  };
  auto st = [&](int m, int k, float2 v) {
    const int e = k - out_off;
    cb.store(e, j0 + m, j0 + m < cg.inner_count && uint32_t(e) < uint32_t(out_cnt), v);
  };
  fft<LOGF, INV, C::M, C::T, C::S, true>(lds, ld, st, tw);
}

// Shift ramp parameters (3 axes; unused axes have c = 0).
struct Ramp {
  int c0, c1, c2;
  int lF0, lF1, lF2;  // log2 sizes (lF1 = 0 for 2D)
  int FH;             // inner index j -> (k1, k2) = (j / FH, j % FH) on axis-0 passes
};

// Factor of the shift ramp at axis-0 frequency k of inner index j, without
// the axis-0 term:  W_F1^{c1 k1} * W_F2^{c2 k2}  (table roots, W = e^{-2 pi i / F}).
__device__ __forceinline__ float2 ramp_inner(const Ramp& rp, const TwTable& tt, int j) {
  const int k1 = j / rp.FH, k2 = j - k1 * rp.FH;
  const int f1 = 1 << rp.lF1, f2 = 1 << rp.lF2;
  return cmul(tt.load(f1, (rp.c1 * k1) & (f1 - 1)), tt.load(f2, (rp.c2 * k2) & (f2 - 1)));
}

// Packed DC / Nyquist column of a 2D spectrum (PACK): bin 0 of every row holds
// d + i n with d, n the rows' real DC and Nyquist values, so along axis 0 it
// transforms to Cc = D + i Nq with D, Nq Hermitian (transforms of real
// columns).  Separation by the pairing of k and F-k:
//   D[k] = (Cc[k] + conj Cc[-k]) / 2,  Nq[k] = (Cc[k] - conj Cc[-k]) / 2i.
// A product Y = X H per column becomes Yc = Xd Hd + i Xn Hn on this column
// (H = filter times ramp; the Nyquist ramp is the DC one times (-1)^{c2}).
__device__ __forceinline__ void pack_split(float2 c, float2 cm, float2& d, float2& n) {
  const float2 cc = cconj(cm);
  d = cscale(cadd(c, cc), 0.5f);
  n = mul_neg_i(cscale(csub(c, cc), 0.5f));
}

// Column-0 filter factors of a PACK workgroup (j0 = 0) for the threads whose
// elements are column 0 (pc0; their frequencies k = kf + it * step): kv[it]
// holds the packed filter value Kc[k] on entry and fd * Kd[k] on exit, and
// kcol[k] = fn * Kn[k], fd / fn the DC / Nyquist factors given by `fac`
// (fac(it, k, fd, fn)).  Uses kcol for the exchange; all threads of the
// workgroup must call it (it has barriers).
template <int F, int PT, class FAC>
__device__ __forceinline__ void pack_filter(bool pc0, int kf, int step, float2* kv, float2* kcol, FAC&& fac) {
  if (pc0) {
#pragma unroll
    for (int it = 0; it < PT; ++it) kcol[kf + it * step] = kv[it];
  }
  __syncthreads();
  float2 kn[PT];
  if (pc0) {
#pragma unroll
    for (int it = 0; it < PT; ++it) {
      const int k = kf + it * step;
      float2 d, n, fd, fn;
      pack_split(kv[it], kcol[(F - k) & (F - 1)], d, n);
      fac(it, k, fd, fn);
      kv[it] = cmul(d, fd);
      kn[it] = cmul(n, fn);
    }
  }
  __syncthreads();
  if (pc0) {
#pragma unroll
    for (int it = 0; it < PT; ++it) kcol[kf + it * step] = kn[it];
  }
}

// Occupancy target of nd_col_mul: 4 waves per SIMD (<= 128 VGPRs) where the
// compiler reaches it without spilling (the HALF variants' first pass holds
// half the inputs; with a ramp but no packed column the ramp factors push it
// over), else no bound (150 VGPRs, 3 waves).  Checked with the compiler's
// resource report for every instantiation.
template <int LOGF, bool HALF, bool RAMP, bool PACK>
struct ColMulOcc {
  static constexpr int WAVES = (HALF && (PACK || !RAMP) && LOGF >= 6 && LOGF <= 8) ? 4 : 1;
};

// Forward conv, axis 0: FFT(x col) * Khat -> IFFT -> window [c0, c0 + S0),
// read from wsx and written to wsy (the same buffer for an in-place product).
// Shared filter (kfilm = 0): grid.x = H * bsplit and a workgroup loops over
// its share of the batch, so its slice of Khat is read once per channel (per
// bsplit share), not once per image; FiLM: grid.x = B*H, one image each.
// grid.y = column blocks.  The first pass is one radix-R butterfly per thread
// over elements j + r*NR of column m; the next image's inputs are loaded
// before the current image's transforms.  HALF (S0 <= F/2, the zero padding
// of a conv is at least half the axis): inputs r >= R/2 are zero, so only R/2
// are loaded and the first pass's butterflies fold the zeros away.  RAMP
// (periodic axes): the filter values are multiplied by conj(R), R the shift
// ramp of `rf`, as they are loaded, which rolls the output by -c_d along
// every axis (the circular "same" alignment; c0 is then 0).  wm0: row index
// mask of the x columns (-1, or S0 - 1 for a short periodic axis 0 read as
// its periodic extension).  PACK (2D): the
// inner index j = 0 is the packed DC / Nyquist column (pack_split).
template <int LOGF, int TARGET = 8192, bool HALF = false, bool RAMP = false, bool PACK = false>
__global__ __launch_bounds__((ColNdCfg<LOGF, TARGET>::T))
__attribute__((amdgpu_waves_per_eu(ColMulOcc<LOGF, HALF, RAMP, PACK>::WAVES))) void nd_col_mul_kernel(const float2* wsx, float2* wsy,
                                                                                const float2* __restrict__ wsk,
                                                                                ColGeom cg, int B, int H, int kfilm,
                                                                                int S0, int wm0, int c0, Ramp rf,
                                                                                int jbase, int bsplit,
                                                                                const float2* __restrict__ tw) {
  using C = ColNdCfg<LOGF, TARGET>;
  constexpr int R = 1 << (LOGF < 4 ? LOGF : 4);  // first-pass radix, as chosen by fft_rec
  constexpr int NR = C::F / R;
  constexpr int RL = HALF ? R / 2 : R;           // first-pass inputs that can be nonzero
  static_assert(C::M * NR == C::T, "nd_col_mul_kernel: one first-pass butterfly per thread");
  __shared__ float2 lds[C::M * C::S];
  const int64_t hk = blockIdx.x / bsplit;  // filter (channel, or FiLM image)
  const int part = int(blockIdx.x % bsplit);
  const ColBuf kb(wsk + hk * cg.spec, cg);
  const int j0 = jbase + blockIdx.y * C::M;
  // Filter spectrum of this column block (element e -> column e % M,
  // frequency e / M), loaded before the first transform so its latency hides.
  constexpr int PT = C::TILE / C::T;
  static_assert(C::T % C::M == 0, "nd_col_mul_kernel: a thread's elements share one column");
  float2 kv[PT];
  const int tk = opaque_tid();
  // PACK: this thread's elements are the packed column (k = tk / M + it * T / M)
  const bool pc0 = PACK && j0 == 0 && tk % C::M == 0;
  __shared__ float2 kcol[PACK ? C::F : 1];
  __shared__ float2 ycol[PACK ? C::F : 1];  // column-0 products (registers would cost occupancy)
#pragma unroll
  for (int it = 0; it < PT; ++it) {
    const int e = tk + it * C::T;
    const int jj = j0 + e % C::M, k = e / C::M;
    kv[it] = kb.load(k, jj, jj < cg.inner_count);
    if constexpr (RAMP) {
      if (!pc0) {
        const TwTable tt(tw);
        const float2 r =
            cmul(ramp_inner(rf, tt, jj < cg.inner_count ? jj : 0), tt.load(C::F, (rf.c0 * k) & (C::F - 1)));
        kv[it] = cmulc(kv[it], r);
      }
    }
  }
  if constexpr (PACK) {
    if (j0 == 0) {  // (uniform) kv of pc0 threads -> conj(Rd) Kd, kcol -> conj(Rn) Kn
      pack_filter<C::F, PT>(pc0, tk / C::M, C::T / C::M, kv, kcol, [&](int, int k, float2& fd, float2& fn) {
        fd = make_float2(1.f, 0.f);
        if constexpr (RAMP) fd = cconj(TwTable(tw).load(C::F, (rf.c0 * k) & (C::F - 1)));
        fn = (RAMP && (rf.c2 & 1)) ? make_float2(-fd.x, -fd.y) : fd;
      });
    }
  }
  const int nb = kfilm ? 1 : B;
  // bsplit > 1: this workgroup takes batches [part * nb / bsplit, (part + 1) * nb / bsplit)
  const int b_begin = part * nb / bsplit, b_end = (part + 1) * nb / bsplit;
  const int m1 = int(threadIdx.x) % C::M, j1 = int(threadIdx.x) / C::M;  // first-pass butterfly of this thread
  const bool colok = j0 + m1 < cg.inner_count;
  auto block = [&](int bi) { return (kfilm ? hk : int64_t(bi) * H + hk) * cg.spec; };
  float2 raw[RL];
  auto issue = [&](int bi) {
    const ColBuf in(wsx + block(bi), cg);
#pragma unroll
    for (int r = 0; r < RL; ++r) {
      const int n = (j1 + r * NR) & wm0;
      raw[r] = in.load(n, j0 + m1, colok && n < S0);
    }
  };
  if (b_begin < b_end) issue(b_begin);
  for (int bi = b_begin; bi < b_end; ++bi) {
    float2 v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = r < RL ? raw[r] : make_float2(0.f, 0.f);
    if (bi + 1 < b_end) issue(bi + 1);  // the block is read before the (in-place) output is written
    const ColBuf out(wsy + block(bi), cg);
    RegStream<R> ld{v};
    LdsTile<C::S, false> tile{lds};
    fft<LOGF, false, C::M, C::T, C::S, true>(lds, ld, tile, tw);
    const int tp = opaque_tid();
#pragma unroll
    for (int it = 0; it < PT; ++it) {
      const int e = tp + it * C::T;
      float2& z = lds[(e % C::M) * C::S + e / C::M];
      if (PACK && pc0) {  // column 0: Yc = Xd Hd + i Xn Hn, staged until every pair is read
        const int k = e / C::M;
        float2 xd, xn;
        pack_split(z, lds[(C::F - k) & (C::F - 1)], xd, xn);
        ycol[PACK ? k : 0] = cadd(cmul(xd, kv[it]), mul_i(cmul(xn, kcol[PACK ? k : 0])));
      } else {
        z = cmul(z, kv[it]);
      }
    }
    if constexpr (PACK) {
      if (j0 == 0) {
        __syncthreads();
        if (pc0) {
#pragma unroll
          for (int it = 0; it < PT; ++it) {
            const int k = (tp + it * C::T) / C::M;
            lds[k] = ycol[k];
          }
        }
      }
    }
    __syncthreads();
    auto st = [&](int m, int k, float2 val) {
      const int e = k - c0;
      out.store(e, j0 + m, j0 + m < cg.inner_count && uint32_t(e) < uint32_t(S0), val);
    };
    fft<LOGF, true, C::M, C::T, C::S, true>(lds, tile, st, tw);
  }
}


// Adjoint, axis 0.  Shared kernel (kfilm = 0): grid.x = H, loops b; FiLM:
// grid.x = B*H, one b.  Writes P (gx pre-image, window [0, S0)) into wsg and
// Q (gk pre-image, window [0, K0)) into wsq.  grid.z > 1 (shared kernel, few
// channels and column blocks for the CUs): workgroup z takes images
// [z*B/nz, (z+1)*B/nz) and writes its partial Q to block z*qsplit + hk; the
// partials are then summed into block hk by nd_q_reduce_kernel.
template <int LOGF, int TARGET = kNdBwdTile, bool HALF = false, bool PACK = false>
__global__ __launch_bounds__((ColNdCfg<LOGF, TARGET>::T)) void nd_col_bwd_kernel(float2* __restrict__ wsg,
                                                                                const float2* __restrict__ wsx,
                                                                                const float2* __restrict__ wsk,
                                                                                float2* __restrict__ wsq, ColGeom cg,
                                                                                int B, int H, int kfilm, int S0,
                                                                                int wm0, int K0, Ramp rp, int jbase,
                                                                                int64_t qsplit,
                                                                                const float2* __restrict__ tw) {
  using C = ColNdCfg<LOGF, TARGET>;
  static_assert(C::T % C::M == 0, "nd_col_bwd_kernel: a thread's elements share one column");
  constexpr int PT = C::TILE / C::T;
  __shared__ float2 ldsG[C::M * C::S];
  __shared__ float2 ldsX[C::M * C::S];  // X of the current image; at the end, Q
  const int64_t hk = blockIdx.x;
  const int j0 = jbase + blockIdx.y * C::M;
  const ColBuf kb(wsk + hk * cg.spec, cg);
  // Element it of a thread is column m = tp % M (fixed), frequency k = tp / M
  // + it * T / M.  Its filter value and shift ramp
  //   R = W_F0^{c0 k} * W_F1^{c1 k1} * W_F2^{c2 k2},  (k1, k2) = (j / FH, j % FH),
  // do not depend on the image: built once, the column factor once per thread
  // (table roots; every axis length here is <= 2^10).
  const int tp = opaque_tid();
  const int m = tp % C::M, kfirst = tp / C::M;
  const int j = j0 + m;
  const TwTable tt(tw);
  const float2 r12 = ramp_inner(rp, tt, j < cg.inner_count ? j : 0);
  float2 kv[PT], rr[PT], q[PT];
#pragma unroll
  for (int it = 0; it < PT; ++it) {
    const int k = kfirst + it * (C::T / C::M);
    kv[it] = kb.load(k, j, j < cg.inner_count);
    rr[it] = cmul(r12, tt.load(C::F, (rp.c0 * k) & (C::F - 1)));
    q[it] = make_float2(0.f, 0.f);
  }
  // PACK: column 0 is the packed DC / Nyquist column (pack_split): kv -> Kd,
  // kcol -> Kn; the Nyquist ramp is the DC one (rr) times (-1)^{c2}.
  const bool pc0 = PACK && j0 == 0 && m == 0;
  __shared__ float2 kcol[PACK ? C::F : 1];
  __shared__ float2 pcol[PACK ? C::F : 1];  // column-0 P values, staged until every pair is read
  const float nys = (rp.c2 & 1) ? -1.f : 1.f;
  if constexpr (PACK) {
    if (j0 == 0)
      pack_filter<C::F, PT>(pc0, kfirst, C::T / C::M, kv, kcol, [](int, int, float2& fd, float2& fn) {
        fd = fn = make_float2(1.f, 0.f);
      });
  }
  const int nb = kfilm ? 1 : B;
  const int nz = int(gridDim.z), z = int(blockIdx.z);
  for (int bi = z * nb / nz; bi < (z + 1) * nb / nz; ++bi) {
    const int64_t bh = kfilm ? hk : (int64_t(bi) * H + hk);
    const ColBuf gb(wsg + bh * cg.spec, cg);
    const ColBuf xb(wsx + bh * cg.spec, cg);
    auto ldg = [&](int mm, int n) -> float2 {
      n &= wm0;
      return gb.load(n, j0 + mm, j0 + mm < cg.inner_count && n < S0);
    };
    auto ldx = [&](int mm, int n) -> float2 {
      n &= wm0;
      return xb.load(n, j0 + mm, j0 + mm < cg.inner_count && n < S0);
    };
    LdsTile<C::S, false> stG{ldsG};
    LdsTile<C::S, false> stX{ldsX};
    constexpr int R1 = 1 << (LOGF < 4 ? LOGF : 4);  // first-pass radix
    HalfZeroLoad<R1, HALF, decltype(ldg)> ldg1{ldg};  // HALF: S0 <= F/2
    HalfZeroLoad<R1, HALF, decltype(ldx)> ldx1{ldx};
    fft<LOGF, false, C::M, C::T, C::S, true>(ldsG, ldg1, stG, tw);
    fft<LOGF, false, C::M, C::T, C::S, true>(ldsX, ldx1, stX, tw);
#pragma unroll
    for (int it = 0; it < PT; ++it) {
      const int a = m * C::S + kfirst + it * (C::T / C::M);
      if (PACK && pc0) {
        // column 0: P = Gd Rd conj(Kd) + i Gn Rn conj(Kn),  Q += Gd Rd conj(Xd) + i Gn Rn conj(Xn)
        const int k = kfirst + it * (C::T / C::M), km = (C::F - k) & (C::F - 1);
        float2 gd, gn, xd, xn;
        pack_split(ldsG[k], ldsG[km], gd, gn);
        pack_split(ldsX[k], ldsX[km], xd, xn);
        const float2 gdr = cmul(gd, rr[it]), gnr = cscale(cmul(gn, rr[it]), nys);
        q[it] = cadd(q[it], cadd(cmulc(gdr, xd), mul_i(cmulc(gnr, xn))));
        pcol[PACK ? k : 0] = cadd(cmulc(gdr, kv[it]), mul_i(cmulc(gnr, kcol[PACK ? k : 0])));
      } else {
        const float2 gsh = cmul(ldsG[a], rr[it]);
        q[it] = cadd(q[it], cmulc(gsh, ldsX[a]));
        ldsG[a] = cmulc(gsh, kv[it]);
      }
    }
    if constexpr (PACK) {
      if (j0 == 0) {
        __syncthreads();  // every column-0 pair read before it is overwritten
        if (pc0) {
#pragma unroll
          for (int it = 0; it < PT; ++it) {
            const int k = kfirst + it * (C::T / C::M);
            ldsG[k] = pcol[k];
          }
        }
      }
    }
    __syncthreads();
    LdsTile<C::S, false> ldl{ldsG};
    auto st = [&](int mm, int k, float2 v) { gb.store(k, j0 + mm, j0 + mm < cg.inner_count && k < S0, v); };
    fft<LOGF, true, C::M, C::T, C::S, true>(ldsG, ldl, st, tw);  // ends with a barrier: ldsX is free
  }
#pragma unroll
  for (int it = 0; it < PT; ++it) ldsX[m * C::S + kfirst + it * (C::T / C::M)] = q[it];
  __syncthreads();
  const ColBuf qb(wsq + (z * qsplit + hk) * cg.spec, cg);
  LdsTile<C::S, false> ldq{ldsX};
  auto stq = [&](int mm, int k, float2 v) { qb.store(k, j0 + mm, j0 + mm < cg.inner_count && k < K0, v); };
  fft<LOGF, true, C::M, C::T, C::S, true>(ldsX, ldq, stq, tw);
}

// The adjoint above for 128-point axis-0 columns without a packed column
// (nd_col_bwd_kernel<7, kNdBwdTile, HALF, false>: same grid, arguments and
// results): each wave owns 8 of the workgroup's 16 columns, 8 lanes per
// column (fft_wave128.h), in an LDS block of 128 rows x 8 columns of its own,
// so no step waits for the other wave.  A lane holds its column's spectral
// values at k = 2 jb + q + 16 r (q < 2, r < 8), with their filter values,
// shift ramps and Q accumulators; G's and X's columns of an image are loaded
// together before either transform.
template <bool HALF>
__global__ __launch_bounds__(128) void nd_col_bwd_w128_kernel(float2* __restrict__ wsg, const float2* __restrict__ wsx,
                                                              const float2* __restrict__ wsk, float2* __restrict__ wsq,
                                                              ColGeom cg, int B, int H, int kfilm, int S0, int wm0,
                                                              int K0, Ramp rp, int jbase, int64_t qsplit,
                                                              const float2* __restrict__ tw) {
  constexpr int F = 128, RSX = 8, NV = HALF ? 8 : 16;  // HALF: S0 <= F/2, inputs n >= 64 are zero
  __shared__ float2 blk[2][F * RSX];
  const int64_t hk = blockIdx.x;
  const int t = opaque_tid();
  const int wv = t >> 6, lane = t & 63;
  const W128Col ic{lane & 7, lane >> 3};
  const int jb = ic.jb;
  const int j = jbase + int(blockIdx.y) * 16 + 8 * wv + ic.col;
  const bool jok = j < cg.inner_count;
  const W128ColX<RSX> cx{blk[wv], ic, jb};
  const ColBuf kb(wsk + hk * cg.spec, cg);
  const TwTable tt(tw);
  const float2 r12 = ramp_inner(rp, tt, jok ? j : 0);
  float2 kv[2][8], rr[2][8], q[2][8];
#pragma unroll
  for (int q2 = 0; q2 < 2; ++q2)
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int k = 2 * jb + q2 + 16 * r;
      kv[q2][r] = kb.load(k, j, jok);
      rr[q2][r] = cmul(r12, tt.load(F, (rp.c0 * k) & (F - 1)));
      q[q2][r] = make_float2(0.f, 0.f);
    }
  const int nb = kfilm ? 1 : B;
  const int nz = int(gridDim.z), z = int(blockIdx.z);
  for (int bi = z * nb / nz; bi < (z + 1) * nb / nz; ++bi) {
    const int64_t bh = kfilm ? hk : (int64_t(bi) * H + hk);
    const ColBuf gb(wsg + bh * cg.spec, cg);
    const ColBuf xb(wsx + bh * cg.spec, cg);
    float2 vg[16], vx[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {  // column values n = jb + 8 r
      const int n = (jb + 8 * r) & wm0;
      const bool ok = r < NV && jok && n < S0;
      vg[r] = r < NV ? gb.load(n, j, ok) : make_float2(0.f, 0.f);
      vx[r] = r < NV ? xb.load(n, j, ok) : make_float2(0.f, 0.f);
    }
    float2 gs[2][8], xs[2][8];
    w128_dft_fwd(cx, vg, gs, tw);
    w128_dft_fwd(cx, vx, xs, tw);
#pragma unroll
    for (int q2 = 0; q2 < 2; ++q2)
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const float2 gsh = cmul(gs[q2][r], rr[q2][r]);
        q[q2][r] = cadd(q[q2][r], cmulc(gsh, xs[q2][r]));
        gs[q2][r] = cmulc(gsh, kv[q2][r]);
      }
    w128_dft_inv(cx, gs, vg, tw);  // P at n = jb + 8 r
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int n = jb + 8 * r;
      gb.store(n, j, jok && n < S0, vg[r]);
    }
  }
  float2 u[16];
  w128_dft_inv(cx, q, u, tw);
  const ColBuf qb(wsq + (z * qsplit + hk) * cg.spec, cg);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int n = jb + 8 * r;
    qb.store(n, j, jok && n < K0, u[r]);
  }
}

// Sum of the batch-split partial Q blocks: for h < nk, block h += blocks
// z*nk + h, z = 1..nz-1, over the first `count` complex values of each block
// (the rows [0, K0) the adjoint wrote; padding columns are summed too and
// never read).  One thread per complex value, fixed summation order.
static __global__ __launch_bounds__(256) void nd_q_reduce_kernel(float2* __restrict__ wsq, int64_t nk,
                                                                 int64_t spec, int64_t count, int nz) {
  const int64_t total = nk * count;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += int64_t(gridDim.x) * 256) {
    const int64_t h = i / count, e = i - h * count;
    float2* q = wsq + h * spec + e;
    float2 acc = *q;
    for (int z = 1; z < nz; ++z) acc = cadd(acc, q[int64_t(z) * nk * spec]);
    *q = acc;
  }
}

}  // namespace nsq
