// 128-point DFTs of lines (columns or rows of an LDS tile) held by 8 lanes of
// one wave, 16 values per lane: radix 16 in registers, one exchange through
// the line's own 128 slots, radix 8.  A line's lanes sit in one wave, so the
// exchanges need only the wave's in-order LDS operations (w128_wave_sync),
// never a workgroup barrier.  Used by the one-kernel 2D image forward
// (fftconv2d_image.h) and the axis-0 adjoint pass of 128-point columns
// (fftconv_nd_impl.h).
#pragma once

#include "fft_core.h"

namespace nsq {

// A column of a tile whose rows are RSX complex apart: lane jb (0..7) of the
// column's 8 lanes.
struct W128Col {
  int col, jb;
};

// LDS operations of one wave take effect in program order; this keeps the
// compiler from moving a lane's slot reads above its neighbours' slot writes.
__device__ __forceinline__ void w128_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Exchange slot n (0..127) of a column lives in tile row
//   e(n) = (n & ~3) | ((gray(n & 3) ^ h(n >> 2)) & 3),  h(m) = (m >> 2) + 2 (m & 1),
// a permutation inside each aligned quad of rows.  A row stride of 8 mod 32
// complex (136 for the padded 128-bin rows, 8 for an 8-column block) moves a
// row 16 banks, so only e(n) mod 4 picks a lane group's banks; e(n) gives the
// 8 lanes of a column distinct values mod 4 (and alternating parity) in every
// exchange pattern of the DFTs below (n = 16 jb + K, 2 jb + q + 16 r,
// jb + 8 r), so a wave's 8 adjacent columns x 8 lanes cover all banks once per
// 8-byte access (checked exhaustively for 64- and 32-bank layouts).  The three
// patterns reduce to four per-lane row pointers and a constant offset per slot.
__device__ __forceinline__ constexpr int w128_gray2(int x) { return (x ^ (x >> 1)) & 3; }
__device__ __forceinline__ int w128_swz(int n) {
  const int h = (n >> 4) + 2 * ((n >> 2) & 1);
  return (n & ~3) | ((w128_gray2(n & 3) ^ h) & 3);
}
template <int RSX>
struct W128Slots {
  static_assert(RSX % 32 == 8, "W128Slots: a row must move 16 banks");
  float2* p[4];
  __device__ __forceinline__ W128Slots(float2* tile, int col, int base, int l) {
#pragma unroll
    for (int c = 0; c < 4; ++c) p[c] = tile + (base + (c ^ l)) * RSX + pad16(col);
  }
};
// n = 16 jb + K (K < 16): row 16 jb + (K & 12) + (cK ^ (jb & 3))
template <int RSX>
__device__ __forceinline__ W128Slots<RSX> w128_slots_w(float2* tile, const W128Col& ic) {
  return W128Slots<RSX>(tile, ic.col, 16 * ic.jb, ic.jb & 3);
}
template <int RSX>
__device__ __forceinline__ float2& w128_w(const W128Slots<RSX>& s, int K) {
  return s.p[w128_gray2(K & 3) ^ (2 * ((K >> 2) & 1))][(K & 12) * RSX];
}
// n = 2 jb + q + 16 r: row 16 r + 4 (jb >> 1) + (((q ^ r) & 3) ^ L)
template <int RSX>
__device__ __forceinline__ W128Slots<RSX> w128_slots_r1(float2* tile, const W128Col& ic) {
  return W128Slots<RSX>(tile, ic.col, 4 * (ic.jb >> 1), (3 * (ic.jb & 1)) ^ (2 * ((ic.jb >> 1) & 1)));
}
template <int RSX>
__device__ __forceinline__ float2& w128_r1(const W128Slots<RSX>& s, int q, int r) {
  return s.p[(q ^ r) & 3][16 * r * RSX];
}
// n = jb + 8 r: row 8 r + 4 (jb >> 2) + (((r >> 1) & 3) ^ L)
template <int RSX>
__device__ __forceinline__ W128Slots<RSX> w128_slots_r2(float2* tile, const W128Col& ic) {
  return W128Slots<RSX>(tile, ic.col, 4 * (ic.jb >> 2), w128_gray2(ic.jb & 3) ^ (2 * (ic.jb >> 2)));
}
template <int RSX>
__device__ __forceinline__ float2& w128_r2(const W128Slots<RSX>& s, int r) {
  return s.p[(r >> 1) & 3][8 * r * RSX];
}

// Slot access policies of the DFTs below: slots_w() gives slot 16 jb + K,
// slots_r1() slot 2 jb + q + 16 r, slots_r2() slot jb + 8 r.
// W128ColX: a tile column (rows permuted by w128_swz).
template <int RSX>
struct W128ColX {
  float2* tile;
  W128Col ic;
  int jb;
  struct W {
    W128Slots<RSX> s;
    __device__ __forceinline__ float2& operator()(int K) const { return w128_w(s, K); }
  };
  struct R1 {
    W128Slots<RSX> s;
    __device__ __forceinline__ float2& operator()(int q, int r) const { return w128_r1(s, q, r); }
  };
  struct R2 {
    W128Slots<RSX> s;
    __device__ __forceinline__ float2& operator()(int r) const { return w128_r2(s, r); }
  };
  __device__ __forceinline__ W slots_w() const { return {w128_slots_w<RSX>(tile, ic)}; }
  __device__ __forceinline__ R1 slots_r1() const { return {w128_slots_r1<RSX>(tile, ic)}; }
  __device__ __forceinline__ R2 slots_r2() const { return {w128_slots_r2<RSX>(tile, ic)}; }
};

// Forward 128-point DFT of the thread's inputs v[r] = c[jb + 8 r] (r < 16):
// radix 16 in registers, exchange through the line's slots (SX: W128ColX or
// a row policy with the same three slot patterns), radix 8; leaves X[jj + 16 r] (r < 8) of the butterflies
// jj = 2 jb + q (q < 2) in xo[q][r].  The line's earlier slot reads precede
// it in the wave's program order.
template <class SX>
__device__ __forceinline__ void w128_dft_fwd(const SX& sx, float2 (&v)[16], float2 (&xo)[2][8],
                                               const float2* __restrict__ tw) {
  dft<16, false>(v);  // first pass: outputs at 16 jb + r
  {
    const auto sw = sx.slots_w();
    w128_wave_sync();
#pragma unroll
    for (int r = 0; r < 16; ++r) sw(r) = v[r];
  }
  w128_wave_sync();
  const TwTable tt(tw);
  const auto s1 = sx.slots_r1();
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int jj = 2 * sx.jb + q;  // second pass (NS = 16): butterfly jj reads jj + 16 r, k = jj
    float2 w[8];
    pass_twiddles<8>(tt, 128, jj, w);
#pragma unroll
    for (int r = 0; r < 8; ++r) xo[q][r] = s1(q, r);
#pragma unroll
    for (int r = 1; r < 8; ++r) xo[q][r] = cmul(xo[q][r], w[r]);
    dft<8, false>(xo[q]);  // outputs at jj + 16 r: natural order
  }
  w128_wave_sync();
}

// u[r] *= conj(W_128^{r k}), r = 1..15: the roots at r = 1, 2, 4, 8 are table
// loads and each other root the product of two (as pass_twiddles), formed
// and applied one output at a time so that no 16-root array is live.
__device__ __forceinline__ void w128_twiddle16_inv(float2 (&u)[16], const float2* __restrict__ tw, int k) {
  const TwTable tt(tw);
  const float2 w1 = tt.load(128, k), w2 = tt.load(128, 2 * k), w4 = tt.load(128, 4 * k), w8 = tt.load(128, 8 * k);
  float2 lo[8];
  lo[1] = w1;
  lo[2] = w2;
  lo[3] = cmul_fixed(w2, w1);
  lo[4] = w4;
#pragma unroll
  for (int r = 1; r < 8; ++r) {
    NSQ_SLOT_FENCE();
    if (r >= 5) lo[r] = cmul_fixed(w4, lo[r - 4]);
    u[r] = cmulc(u[r], lo[r]);
  }
  u[8] = cmulc(u[8], w8);
#pragma unroll
  for (int r = 9; r < 16; ++r) {
    NSQ_SLOT_FENCE();
    u[r] = cmulc(u[r], cmul_fixed(w8, lo[r - 8]));
  }
}

// Inverse 128-point DFT (unnormalised) of Y[jj + 16 r] in yv[q][r] (the
// layout w128_dft_fwd leaves): radix 8 in registers (first pass, butterfly
// jj reads jj + 16 r), exchange, radix 16 (butterfly jb reads jb + 8 r,
// k = jb); leaves y[jb + 8 r] in u[r].
template <class SX>
__device__ __forceinline__ void w128_dft_inv(const SX& sx, float2 (&yv)[2][8], float2 (&u)[16],
                                               const float2* __restrict__ tw) {
  {
    const auto sw = sx.slots_w();
    w128_wave_sync();
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      dft<8, true>(yv[q]);  // outputs at 8 jj + r = 16 jb + 8 q + r
#pragma unroll
      for (int r = 0; r < 8; ++r) sw(8 * q + r) = yv[q][r];
    }
  }
  w128_wave_sync();
  {
    const auto s2 = sx.slots_r2();
#pragma unroll
    for (int r = 0; r < 16; ++r) u[r] = s2(r);
  }
  w128_twiddle16_inv(u, tw, sx.jb);
  dft<16, true>(u);  // outputs at jb + 8 r
  w128_wave_sync();
}

}  // namespace nsq
