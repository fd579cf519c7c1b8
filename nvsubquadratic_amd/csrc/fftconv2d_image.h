// One-kernel 2D forward FFT convolution of whole images on 256 x 256 FFT
// planes (zero-padded axes, S0 and S2 <= 128, shared filter): the spectrum of
// an image never leaves the CU.
//
// Semantics: nvsubquadratic/ops/fftconv.py:662-733 (fftconv2d_fp32_bhl), as
// the three-pass plan of fftconv_nd_impl.h computes it: zero-padded linear
// conv, window [K_d//2, K_d//2 + S_d) per axis, cast, + shortcut * x.
//
// The three-pass plan moves each image's packed spectrum (128 rows x 128
// complex bins, 128 KB) through HBM twice.  Here one workgroup of 512 threads
// holds it in LDS, one image per workgroup and one workgroup per CU:
//   A  real FFTs of the S0 rows of x (256 points, half zero padding) into the
//      tile, packed as in the three-pass plan (bin 0 = U[0] + i U[128]);
//   B  each of the 128 bin columns: its 256-point zero-padded DFT as two
//      128-point DFTs of the 128 nonzero values c[n] (pad at n >= 128):
//        X[2m] = DFT128(c)[m],   X[2m+1] = DFT128(c[n] W256^n)[m],
//      times the filter spectrum (Khat rows 2m and 2m+1), two 128-point
//      inverse DFTs, and the unnormalised 256-point inverse at the kept rows
//        y[n] = ye[n mod 128] + W256^-n yo[n mod 128],  n in [o0, o0 + S0),
//      so each half's exchanges fit the column's own 128 tile slots.  The
//      packed column 0 separates its DC and Nyquist columns with the pairing
//      of k and -k (k = 2m <-> 2(-m mod 128), k = 2m+1 <-> 2(127-m)+1);
//   C  inverse real FFTs of the kept rows, window [o2, o2 + S2), epilogue.
// A column's two halves run one after the other on the same lanes, which
// keep the column's values for the second half, the first half's result and
// the next half's filter values (issued ahead, so their L2 latency overlaps a
// DFT): ~250 VGPRs.  With 1024 threads (128 VGPRs each) that spilled 320 bytes
// per lane, so the workgroup has 512 threads (2 waves per SIMD) and phase B
// takes the columns in two rounds of 64.
// Every wave owns whole lines: 8 columns in each round of phase B (8 lanes per
// column), 16 rows in phases A and C (8 lanes per row), so the DFT exchanges
// rely on the wave's in-order LDS operations and an image takes two
// workgroup barriers (after A and after B).
// Measured on MI355X, config 4 (B=16 C=384 128^2, bf16): 0.864 ms for the
// kernel, 0.865-0.873 ms per call with the filter spectrum, against 1.145 ms
// for the three passes; VALU 44% busy, LDS 33% busy: the latency of 2 waves
// per SIMD bounds it.
// HBM traffic per image is x in, y out and the channel's filter spectrum,
// which the images of a channel read from their XCD's L2: workgroup w runs on
// XCD w % 8 and the images of a channel take consecutive slots there.
#pragma once

#include "fft_wave128.h"
#include "fftconv_nd_impl.h"

namespace nsq {

constexpr int kImgThreads = 512;               // 8 waves: 2 per SIMD, up to 256 VGPRs
constexpr int kImgRS = Padded<128>::SIZE;      // tile row stride (complex): 136
constexpr int kImgTile = 128 * kImgRS;         // 128 rows x 136 = 139,264 bytes

// Image (b, h) of workgroup w: channel-major within each XCD (w % 8), so the
// B images of a channel run side by side on one XCD and share its filter
// spectrum in that XCD's L2.  Needs H % 8 == 0 (else plain row-major order).
__device__ __forceinline__ void img_of(int w, int B, int H, int& b, int& h) {
  if ((H & 7) == 0) {
    const int x = w & 7, i = w >> 3;
    h = x + 8 * (i / B);
    b = i - (i / B) * B;
  } else {
    h = w % H;
    b = w / H;
  }
}

// The per-column state of phase B (W128Col): in round q (q < 2) wave w owns
// the 8 columns col = 64 q + 8 w + (lane & 7), and lane l runs butterfly
// jb = l >> 3 of its column's 128-point DFTs (w128_dft_fwd / w128_dft_inv).

// Element n of column col in the tile (rows of kImgRS, pad16 inside a row).
__device__ __forceinline__ float2& img_at(float2* tile, int n, int col) { return tile[n * kImgRS + pad16(col)]; }

// ImgRowX: a tile row in its natural layout (element n at pad16(n)); the
// slots of a pattern are constant offsets from one per-lane pointer.  With 8
// rows per wave (lane = 8 row + jb) the 16 jb + K and jb + 8 r patterns are
// free of bank conflicts and 2 jb + q + 16 r has 2-way conflicts.
struct ImgRowX {
  float2* row;
  int jb;
  struct W {
    float2* b;
    __device__ __forceinline__ float2& operator()(int K) const { return b[K]; }  // pad16(16 jb + K) = 17 jb + K
  };
  struct R1 {
    float2* b;
    __device__ __forceinline__ float2& operator()(int q, int r) const { return b[q + 17 * r]; }
  };
  struct R2 {
    float2* b;
    __device__ __forceinline__ float2& operator()(int r) const { return b[8 * r + (r >> 1)]; }
  };
  __device__ __forceinline__ W slots_w() const { return {row + 17 * jb}; }
  __device__ __forceinline__ R1 slots_r1() const { return {row + 2 * jb}; }
  __device__ __forceinline__ R2 slots_r2() const { return {row + jb}; }
};

// Filter values of one half (ODD: frequencies k = 2m + 1, else 2m) for the
// thread's outputs m = 2 jb + q + 16 r of w128_dft_fwd: Khat[k][col], and
// for the packed column 0 also Khat[-k][0].  Issued before the half's DFT so
// their L2 latency overlaps it.
template <bool ODD>
__device__ __forceinline__ void img_filter_load(const W128Col& ic, const float2* __restrict__ kc, int rsk,
                                                float2 (&kv)[2][8], float2 (&km)[2][8]) {
  const bool c0 = ic.col == 0;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int k = 2 * (2 * ic.jb + q + 16 * r) + (ODD ? 1 : 0);
      kv[q][r] = kc[k * rsk + ic.col];
      float2 t = make_float2(0.f, 0.f);
      if (c0) t = kc[((256 - k) & 255) * rsk];  // -k, column 0 only
      km[q][r] = t;
    }
  }
}

// Spectral product of one half with the values img_filter_load fetched.
// Column 0 is the packed DC / Nyquist column: Y = Xd Kd + i Xn Kn with the
// pairs of k and -k (pack_split); its partner values go through the column's
// slots (lanes of one wave).
template <bool ODD>
__device__ __forceinline__ void img_col_product(float2* tile, const W128Col& ic, float2 (&xo)[2][8],
                                                const float2 (&kv)[2][8], const float2 (&km)[2][8]) {
  const bool c0 = ic.col == 0;
  if (c0) {
    const auto s1 = w128_slots_r1<kImgRS>(tile, ic);
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int r = 0; r < 8; ++r) w128_r1(s1, q, r) = xo[q][r];  // slot m = 2 jb + q + 16 r
  }
  w128_wave_sync();
#pragma unroll
  for (int q = 0; q < 2; ++q) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if (c0) {
        const int m = 2 * ic.jb + q + 16 * r;
        const int mp = ODD ? 127 - m : (128 - m) & 127;  // -k
        float2 xd, xn, kd, kn;
        pack_split(xo[q][r], img_at(tile, w128_swz(mp), 0), xd, xn);
        pack_split(kv[q][r], km[q][r], kd, kn);
        xo[q][r] = cadd(cmul(xd, kd), mul_i(cmul(xn, kn)));
      } else {
        xo[q][r] = cmul(xo[q][r], kv[q][r]);
      }
    }
  }
  w128_wave_sync();
}

// The image kernel.  kc: filter spectra [H][256][rsk] (the three-pass plan's
// Khat layout, packed bin 0).  x, y: [B*H][S0][S2].  o0, o2: crop offsets.
// scale = 1 / (F0 * F2/2).  AL: x and y 16-byte aligned, S2 % 8 == 0 (the
// epilogue moves 8 samples per access).
template <int DT, bool HAS_S, int kImgT>
__global__ __launch_bounds__(kImgT) void nd2_image_fwd_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                              const float2* __restrict__ khat, int rsk,
                                                              const typename Elem<DT>::T* __restrict__ s,
                                                              typename Elem<DT>::T* __restrict__ y, int B, int H,
                                                              int S0, int S2, int o0, int o2, float scale,
                                                              const float2* __restrict__ tw) {
  using ET = typename Elem<DT>::T;
  static_assert(kImgT == 512, "phases A and C give each of the 8 waves 16 of the 128 rows");
  __shared__ float2 tile[kImgTile];
  int b, h;
  img_of(int(blockIdx.x), B, H, b, h);
  const int64_t img = (int64_t(b) * H + h) * S0 * S2;
  const ET* __restrict__ xi = x + img;
  const float2* __restrict__ kc = khat + int64_t(h) * 256 * rsk;
  // Each phase takes its own opaque thread index: phases A and C address the
  // same slots, and values shared between them would stay live (spilled)
  // across phase B.

  // ---- A: real row FFTs (128 complex = 256 real points, samples >= S2 zero) ----
  // Wave w owns rows 16 w .. 16 w + 15, 8 at a time (lane = 8 row + jb): the
  // row DFTs and the unpack exchange only through the wave's own rows.
  {
    const int tid = opaque_tid();
    const int wv = tid >> 6, lane = tid & 63, jb = lane & 7;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int m = 16 * wv + 8 * g + (lane >> 3);
      const ImgRowX rx{tile + m * kImgRS, jb};
      float2 xo[2][8];
      if (16 * wv + 8 * g >= S0) {  // zero-padding rows only (wave-uniform)
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int r = 0; r < 8; ++r) xo[q][r] = make_float2(0.f, 0.f);
      } else {
        float2 v[16];
#pragma unroll
        for (int r = 0; r < 8; ++r) {  // complex sample n = jb + 8 r: x[m][2n], x[m][2n + 1]
          const int n = jb + 8 * r;
          const bool ok = m < S0 && 2 * n < S2;
          v[r] = load_pair_nb<DT, true>(xi + int64_t(ok ? m : 0) * S2, ok ? 2 * n : 0, ok ? S2 : 0);
        }
#pragma unroll
        for (int r = 8; r < 16; ++r) v[r] = make_float2(0.f, 0.f);  // n >= 64: the zero half
        w128_dft_fwd(rx, v, xo, tw);
      }
      const auto s1 = rx.slots_r1();
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int r = 0; r < 8; ++r) s1(q, r) = xo[q][r];  // X[jj + 16 r], natural order
    }
    w128_wave_sync();
#pragma unroll
    for (int i = 0; i < 16; ++i) {  // unpack in place: slot (row m, p < 64) owns elements p and 128 - p (0: 0, 64)
      const int m = 16 * wv + i, p = lane;
      float2* z = tile + m * kImgRS;
      const bool p0 = p == 0;
      const int pb = p0 ? 64 : 128 - p;
      float2 A, Bc;
      real_unpack(p0, z[pad16(p)], z[pad16(pb)], root<8>(tw, uint32_t(p)), A, Bc);
      z[pad16(p)] = A;
      z[pad16(pb)] = p0 ? Bc : cconj(Bc);
    }
    __syncthreads();
  }

  // ---- B: columns: two 128-point halves, product, inverse, combine, crop ----
  constexpr int CPR = kImgT / 8;  // columns per round: 8 lanes per column, 8 columns per wave
  for (int round = 0; round < 128 / CPR; ++round) {
    const int tid = opaque_tid();
    const W128Col ic{CPR * round + 8 * (tid >> 6) + (tid & 7), (tid >> 3) & 7};
    const W128ColX<kImgRS> cx{tile, ic, ic.jb};
    const TwTable tt(tw);
    float2 c[16], v[16], ye[16];
    float2 xo[2][8], kv[2][8], km[2][8];
    img_filter_load<false>(ic, kc, rsk, kv, km);
#pragma unroll
    for (int r = 0; r < 16; ++r) c[r] = img_at(tile, ic.jb + 8 * r, ic.col);  // rows >= S0 are zero
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = c[r];
    w128_dft_fwd(cx, v, xo, tw);
    img_col_product<false>(tile, ic, xo, kv, km);
    img_filter_load<true>(ic, kc, rsk, kv, km);
    w128_dft_inv(cx, xo, ye, tw);
    float2 wt[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) wt[r] = tt.load(256, ic.jb + 8 * r);
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = cmul(c[r], wt[r]);  // c[n] W256^n
    w128_dft_fwd(cx, v, xo, tw);
    img_col_product<true>(tile, ic, xo, kv, km);
    w128_dft_inv(cx, xo, v, tw);
    // y[n] = ye[p] + W256^-n yo[p] for the kept n = p or p + 128 in [o0, o0 + S0)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int p = ic.jb + 8 * r;
      const int n = (p >= o0 && p < o0 + S0) ? p : p + 128;
      wt[r] = tt.load(256, n & 255);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int p = ic.jb + 8 * r;
      const int n = (p >= o0 && p < o0 + S0) ? p : p + 128;
      const bool keep = n >= o0 && n < o0 + S0;
      if (keep) img_at(tile, n - o0, ic.col) = cadd(ye[r], cmulc(v[r], wt[r]));
    }
    w128_wave_sync();
  }
  __syncthreads();

  // ---- C: inverse real row FFTs of the kept rows, window [o2, o2 + S2), epilogue ----
  // Wave w again owns rows 16 w .. 16 w + 15 (as in A).
  {
    const int tid = opaque_tid();
    const int wv = tid >> 6, lane = tid & 63, jb = lane & 7;
#pragma unroll
    for (int i = 0; i < 16; ++i) {  // repack in place (three-pass plan's nd_row_inv, PACK)
      const int m = 16 * wv + i, p = lane;
      float2* z = tile + m * kImgRS;
      const bool p0 = p == 0;
      const int pb = p0 ? 64 : 128 - p;
      const float2 u0 = z[pad16(p)], u1 = z[pad16(pb)];
      float2 A = u0, Bc = p0 ? u1 : cconj(u1);
      if (m >= S0) A = Bc = make_float2(0.f, 0.f);
      float2 zp, zq;
      real_repack(p0, A, Bc, root<8>(tw, uint32_t(p)), zp, zq);
      z[pad16(p)] = zp;
      z[pad16(pb)] = zq;
    }
    w128_wave_sync();
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      if (16 * wv + 8 * g >= S0) continue;  // no output rows (wave-uniform)
      const int m = 16 * wv + 8 * g + (lane >> 3);
      const ImgRowX rx{tile + m * kImgRS, jb};
      float2 yv[2][8], u[16];
      const auto s1 = rx.slots_r1();
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int r = 0; r < 8; ++r) yv[q][r] = s1(q, r);
      w128_dft_inv(rx, yv, u, tw);
      const auto s2 = rx.slots_r2();
#pragma unroll
      for (int r = 0; r < 16; ++r) s2(r) = u[r];  // y[jb + 8 r], natural order
    }
    w128_wave_sync();
    const float sv = HAS_S ? Elem<DT>::round(Elem<DT>::load(s, h)) : 0.f;
    const int cpr = S2 >> 3;  // 8-sample chunks per output row
    const int nr = min(16, S0 - 16 * wv);  // the wave's output rows
    const RowBuf<DT, false> ab(xi, HAS_S ? S0 * S2 : 0);
    const RowBuf<DT, true> ob(y + img, S0 * S2);
    for (int ch = lane; ch < nr * cpr; ch += 64) {
      const int mi = ch / cpr, m = 16 * wv + mi, c8 = (ch - mi * cpr) * 8;
      const int e0 = m * S2 + c8;
      Win8<DT, true> a;
      a.load(ab, e0);
      const float2* zr = tile + m * kImgRS;
      const int n0 = (c8 + o2) >> 1;
      float yo[8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float2 z = zr[pad16(n0 + u)];
        yo[2 * u] = epilogue<DT>(z.x * scale, HAS_S, sv, a.at(2 * u));
        yo[2 * u + 1] = epilogue<DT>(z.y * scale, HAS_S, sv, a.at(2 * u + 1));
      }
      store8<DT, true>(ob, e0, yo);
    }
  }
}

}  // namespace nsq
