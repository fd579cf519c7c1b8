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
// A column's two halves run one after the other on the same threads, which
// keep the column's values for the second half, the first half's result and
// the next half's filter values (issued ahead, so their L2 latency overlaps a
// DFT): ~250 VGPRs.  With 1024 threads (128 VGPRs each) that spilled 320 bytes
// per lane, so the workgroup has 512 threads (2 waves per SIMD) and phase B
// takes the columns in two rounds of 64.
// Measured on MI355X, config 4 (B=16 C=384 128^2, bf16): 0.99 ms for the
// kernel, 1.037 ms with the filter spectrum, against 1.153 ms for the three
// passes.  One workgroup per CU with barrier-separated phases keeps the VALU
// ~27% busy (about 41 us per image against ~11 us of VALU issue).
// HBM traffic per image is x in, y out and the channel's filter spectrum,
// which the images of a channel read from their XCD's L2: workgroup w runs on
// XCD w % 8 and the images of a channel take consecutive slots there.
#pragma once

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

// The per-column state of phase B: in round q (q < 2) thread t owns column
// col = 64 q + t % 64 and first-pass butterfly jb = t / 64 of its 128-point
// DFTs (TMAJOR passes: the 64 lanes of a wave read 64 consecutive columns of
// one tile row).
struct ImgCol {
  int col, jb;
};

// Element n of column col in the tile (rows of kImgRS, pad16 inside a row).
__device__ __forceinline__ float2& img_at(float2* tile, int n, int col) { return tile[n * kImgRS + pad16(col)]; }

// Forward 128-point DFT of the thread's column inputs v[r] = c[jb + 8 r]
// (r < 16): radix 16 in registers, exchange through the column's slots,
// radix 8; leaves X[jj + 16 r] (r < 8) of the butterflies jj = 2 jb + q
// (q < 2) in xo[q][r].  Starts and ends with a barrier.
__device__ __forceinline__ void img_col_dft_fwd(float2* tile, const ImgCol& ic, float2 (&v)[16], float2 (&xo)[2][8],
                                                const float2* __restrict__ tw) {
  dft<16, false>(v);  // first pass: outputs at 16 jb + r
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 16; ++r) img_at(tile, 16 * ic.jb + r, ic.col) = v[r];
  __syncthreads();
  const TwTable tt(tw);
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int jj = 2 * ic.jb + q;  // second pass (NS = 16): butterfly jj reads jj + 16 r, k = jj
    float2 w[8];
    pass_twiddles<8>(tt, 128, jj, w);
#pragma unroll
    for (int r = 0; r < 8; ++r) xo[q][r] = img_at(tile, jj + 16 * r, ic.col);
#pragma unroll
    for (int r = 1; r < 8; ++r) xo[q][r] = cmul(xo[q][r], w[r]);
    dft<8, false>(xo[q]);  // outputs at jj + 16 r: natural order
  }
  __syncthreads();
}

// u[r] *= conj(W_128^{r k}), r = 1..15: the roots at r = 1, 2, 4, 8 are table
// loads and each other root the product of two (as pass_twiddles), formed
// and applied one output at a time so that no 16-root array is live.
__device__ __forceinline__ void img_twiddle16_inv(float2 (&u)[16], const float2* __restrict__ tw, int k) {
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
// layout img_col_dft_fwd leaves): radix 8 in registers (first pass, butterfly
// jj reads jj + 16 r), exchange, radix 16 (butterfly jb reads jb + 8 r,
// k = jb); leaves y[jb + 8 r] in u[r].  The caller's barrier precedes it;
// ends with a barrier.
__device__ __forceinline__ void img_col_dft_inv(float2* tile, const ImgCol& ic, float2 (&yv)[2][8], float2 (&u)[16],
                                                const float2* __restrict__ tw) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int jj = 2 * ic.jb + q;
    dft<8, true>(yv[q]);  // outputs at 8 jj + r
#pragma unroll
    for (int r = 0; r < 8; ++r) img_at(tile, 8 * jj + r, ic.col) = yv[q][r];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 16; ++r) u[r] = img_at(tile, ic.jb + 8 * r, ic.col);
  img_twiddle16_inv(u, tw, ic.jb);
  dft<16, true>(u);  // outputs at jb + 8 r
  __syncthreads();
}

// Filter values of one half (ODD: frequencies k = 2m + 1, else 2m) for the
// thread's outputs m = 2 jb + q + 16 r of img_col_dft_fwd: Khat[k][col], and
// for the packed column 0 also Khat[-k][0].  Issued before the half's DFT so
// their L2 latency overlaps it.
template <bool ODD>
__device__ __forceinline__ void img_filter_load(const ImgCol& ic, const float2* __restrict__ kc, int rsk,
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
// slots, so every thread takes the two barriers.
template <bool ODD>
__device__ __forceinline__ void img_col_product(float2* tile, const ImgCol& ic, float2 (&xo)[2][8],
                                                const float2 (&kv)[2][8], const float2 (&km)[2][8]) {
  const bool c0 = ic.col == 0;
  if (c0) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int r = 0; r < 8; ++r) img_at(tile, 2 * ic.jb + q + 16 * r, 0) = xo[q][r];
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 2; ++q) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      if (c0) {
        const int m = 2 * ic.jb + q + 16 * r;
        const int mp = ODD ? 127 - m : (128 - m) & 127;  // -k
        float2 xd, xn, kd, kn;
        pack_split(xo[q][r], img_at(tile, mp, 0), xd, xn);
        pack_split(kv[q][r], km[q][r], kd, kn);
        xo[q][r] = cadd(cmul(xd, kd), mul_i(cmul(xn, kn)));
      } else {
        xo[q][r] = cmul(xo[q][r], kv[q][r]);
      }
    }
  }
  __syncthreads();
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
  {
    const int tid = opaque_tid();
    auto ld = [&](int m, int n) -> float2 {
      const bool ok = m < S0 && 2 * n < S2;
      return load_pair_nb<DT, true>(xi + int64_t(ok ? m : 0) * S2, ok ? 2 * n : 0, ok ? S2 : 0);
    };
    HalfZeroLoad<16, true, decltype(ld)> ld1{ld};
    LdsTile<kImgRS, true> st{tile};
    fft<7, false, 128, kImgT, kImgRS>(tile, ld1, st, tw);
#pragma unroll
    for (int i = 0; i < 8192 / kImgT; ++i) {  // unpack in place: slot (row m, p < 64) owns elements p and 128 - p (0: 0, 64)
      const int sl = tid + i * kImgT;
      const int m = sl >> 6, p = sl & 63;
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
  constexpr int CPR = kImgT / 8;  // columns per round: 8 threads per column
  for (int round = 0; round < 128 / CPR; ++round) {
    const int tid = opaque_tid();
    const ImgCol ic{CPR * round + tid % CPR, tid / CPR};
    const TwTable tt(tw);
    float2 c[16], v[16], ye[16];
    float2 xo[2][8], kv[2][8], km[2][8];
    img_filter_load<false>(ic, kc, rsk, kv, km);
#pragma unroll
    for (int r = 0; r < 16; ++r) c[r] = img_at(tile, ic.jb + 8 * r, ic.col);  // rows >= S0 are zero
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = c[r];
    img_col_dft_fwd(tile, ic, v, xo, tw);
    img_col_product<false>(tile, ic, xo, kv, km);
    img_filter_load<true>(ic, kc, rsk, kv, km);
    img_col_dft_inv(tile, ic, xo, ye, tw);
    float2 wt[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) wt[r] = tt.load(256, ic.jb + 8 * r);
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = cmul(c[r], wt[r]);  // c[n] W256^n
    img_col_dft_fwd(tile, ic, v, xo, tw);
    img_col_product<true>(tile, ic, xo, kv, km);
    img_col_dft_inv(tile, ic, xo, v, tw);
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
    __syncthreads();
  }

  // ---- C: inverse real row FFTs of the kept rows, window [o2, o2 + S2), epilogue ----
  {
    const int tid = opaque_tid();
#pragma unroll
    for (int i = 0; i < 8192 / kImgT; ++i) {  // repack in place (three-pass plan's nd_row_inv, PACK)
      const int sl = tid + i * kImgT;
      const int m = sl >> 6, p = sl & 63;
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
    __syncthreads();
    LdsTile<kImgRS, true> t{tile};
    fft_rec<7, 0, true, 128, kImgT, false>(t, t, t, t, tw);
    const float sv = HAS_S ? Elem<DT>::round(Elem<DT>::load(s, h)) : 0.f;
    const int cpr = S2 >> 3;  // 8-sample chunks per output row
    const RowBuf<DT, false> ab(xi, HAS_S ? S0 * S2 : 0);
    const RowBuf<DT, true> ob(y + img, S0 * S2);
    for (int ch = tid; ch < S0 * cpr; ch += kImgT) {
      const int m = ch / cpr, c8 = (ch - m * cpr) * 8;
      const int e0 = m * S2 + c8;
      Win8<DT, true> a;
      a.load(ab, e0);
      const float2* zr = tile + m * kImgRS;
      const int n0 = (c8 + o2) >> 1;
      float yv[8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float2 z = zr[pad16(n0 + u)];
        yv[2 * u] = epilogue<DT>(z.x * scale, HAS_S, sv, a.at(2 * u));
        yv[2 * u + 1] = epilogue<DT>(z.y * scale, HAS_S, sv, a.at(2 * u + 1));
      }
      store8<DT, true>(ob, e0, yv);
    }
  }
}

}  // namespace nsq
