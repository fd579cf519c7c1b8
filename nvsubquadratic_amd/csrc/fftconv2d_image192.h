// One-kernel 2D forward FFT convolution of whole images on the reference's
// own 192 x 192 FFT plane (zero-padded axes, S0 and S2 <= 128, F_d = 192 =
// S_d + ceil(K_d / 2) at S = K = 128, nvsubquadratic/ops/fftconv.py:699-702):
// the spectrum of an image never leaves the CU.
//
// Semantics: nvsubquadratic/ops/fftconv.py:662-733 (fftconv2d_fp32_bhl), as
// the mixed-radix plan computes it (fftconv_nd_r3.h): zero-padded linear conv,
// window [K_d//2, K_d//2 + S_d) per axis, cast, + shortcut * x.
//
// The mixed-radix plan's three passes move each image's spectrum (S0 rows x 97
// bins) through HBM twice.  Here one workgroup holds it in LDS, one image per
// workgroup and one workgroup per CU.  Every phase gives each wave whole
// lines, so its transforms synchronise on the wave's in-order LDS operations
// (fft_mixed_wave) and an image takes two workgroup barriers:
//   A  real FFTs of the S0 rows of x (192 points as 96 complex, samples >= S2
//      zero: the radix-3 first pass reads two of its three inputs), unpacked
//      in place into 96 slots per row, slot 0 holding the DC and Nyquist bins
//      as X[0] + i X[96] (both real);
//   B  each of the 96 slot columns: its 192-point DFT over the rows (rows >=
//      S0 zero), times the filter spectrum, the inverse DFT, rows [o0, o0 +
//      S0) kept; the packed column 0 separates its DC and Nyquist columns
//      with the pairing of k and -k, takes each its own filter column and
//      packs the products again;
//   C  inverse real FFTs of the kept rows, window [o2, o2 + S2), epilogue.
// The filter spectrum comes in transposed ([H][97][192], a column's 192
// frequencies contiguous), so the product's loads are coalesced; the images
// of a channel run side by side on one XCD (img_of) and read it from L2.
#pragma once

#include "fft_mixed.h"
#include "fftconv2d_image.h"

namespace nsq {

constexpr int kI3F = 192;               // FFT length of both axes
constexpr int kI3N2 = kI3F / 2;         // complex length of a packed real row
constexpr int kI3Bins = kI3N2 + 1;      // bins of a real row (the filter spectrum's columns)
constexpr int kI3Rows = 128;            // S0 <= 128
constexpr int kI3RS = kI3N2 + 1;        // tile row stride (complex): 96 slots, odd stride
constexpr int kI3CS = kI3F + 4;         // column scratch line stride

template <int T>
struct Img192Cfg {
  static constexpr int WAVES = T / 64;
  static constexpr int ROWS = kI3Rows / WAVES;  // rows per wave in phases A and C
  static constexpr int COLS = kI3N2 / WAVES;    // slot columns per wave in phase B
  static constexpr int CM = T == 512 ? 4 : 2;   // columns per transform batch
  static constexpr int CHUNKS = COLS / CM;
  // Column passes (measured at config 4): 3, 4, 16 for 4 columns per wave;
  // 3, 8, 8 for 2, where 3, 4, 16 leaves 40 lanes idle in the radix-16 pass
  // (0.73 -> 0.85 ms) and 3, 4, 4, 4 adds a pass (0.80 ms).  The rows run
  // 3, 4, 8: a radix-4 pass after the radix-3 one stores without bank
  // conflicts (its butterfly groups of 3 land 12 slots apart), a radix-8 one
  // 2-way (24 apart).
  static constexpr int CRMAX = CM == 4 ? 16 : 8;
  static constexpr int CR2 = CM == 4 ? 4 : 0;
  static constexpr int LDS = (kI3Rows * kI3RS + WAVES * CM * kI3CS + kI3F) * 8;
  static_assert(kI3Rows % WAVES == 0 && kI3N2 % WAVES == 0 && COLS % CM == 0, "Img192Cfg: wave split");
  static_assert(LDS <= 160 * 1024, "Img192Cfg: LDS");
};

// Lines of `stride` complex values in LDS, as loader and as store.
struct I3Lines {
  float2* p;
  int stride;
  __device__ __forceinline__ float2 operator()(int m, int n) const { return p[m * stride + n]; }
  __device__ __forceinline__ void operator()(int m, int n, float2 v) const { p[m * stride + n] = v; }
};

// The image kernel.  kt: transposed filter spectra [H][97][192].  x, y:
// [B*H][S0][S2].  o0, o2: crop offsets (o2 even).  scale = 1 / (192 * 96).
// x and y 16-byte aligned, S2 % 8 == 0 (16-byte epilogue).
template <int DT, bool HAS_S, int T>
__global__ __launch_bounds__(T) void nd2_image192_fwd_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                             const float2* __restrict__ kt,
                                                             const typename Elem<DT>::T* __restrict__ s,
                                                             typename Elem<DT>::T* __restrict__ y, int B, int H,
                                                             int S0, int S2, int o0, int o2, float scale,
                                                             const float2* __restrict__ tw) {
  using ET = typename Elem<DT>::T;
  using C = Img192Cfg<T>;
  __shared__ float2 tile[kI3Rows * kI3RS];
  __shared__ float2 cscr[C::WAVES * C::CM * kI3CS];
  __shared__ float2 twl[kI3F];
  const auto tws = stage_roots<kI3F, T>(twl, tw);
  int b, h;
  img_of(int(blockIdx.x), B, H, b, h);
  const int64_t img = (int64_t(b) * H + h) * S0 * S2;
  const ET* __restrict__ xi = x + img;
  const float2* __restrict__ kc = kt + int64_t(h) * kI3Bins * kI3F;
  const int wv = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int rw0 = C::ROWS * wv;  // the wave's rows in phases A and C
  __syncthreads();

  // ---- A: real row FFTs (96 complex = 192 real points, samples >= S2 zero), unpack ----
  if (rw0 < S0) {
    const int lane = opaque_tid() & 63;
    float2* rows = tile + rw0 * kI3RS;
    auto ld = [&](int m, int n) -> float2 {  // complex sample n of row rw0 + m: x[2n], x[2n + 1]
      const int r = rw0 + m;
      const bool ok = r < S0 && 2 * n < S2;
      return load_pair_nb<DT, true>(xi + int64_t(ok ? r : 0) * S2, ok ? 2 * n : 0, ok ? S2 : 0);
    };
    TailZeroLoad<3, 2, true, decltype(ld)> ld1{ld};
    I3Lines tl{rows, kI3RS};
    fft_mixed_wave<kI3N2, false, C::ROWS, false, 8, 4>(ld1, tl, tl, tws);
#pragma unroll
    for (int i = 0; i < C::ROWS * (kI3N2 / 2) / 64; ++i) {  // slot pair (p, 96 - p) of row m; p = 0: (0, 48)
      const int jj = lane + 64 * i, m = jj / (kI3N2 / 2), p = jj - m * (kI3N2 / 2);
      float2* z = rows + m * kI3RS;
      const bool p0 = p == 0;
      const int pb = p0 ? kI3N2 / 2 : kI3N2 - p;
      float2 A, Bc;
      real_unpack(p0, z[p], z[pb], tws.template root<kI3F>(p), A, Bc);
      z[p] = A;
      z[pb] = p0 ? Bc : cconj(Bc);
    }
  }
  __syncthreads();

  // ---- B: slot columns: 192-point DFT over the rows, product, inverse, crop ----
  {
    float2* sc = cscr + wv * C::CM * kI3CS;
    I3Lines sl{sc, kI3CS};
    const int lane = opaque_tid() & 63;
    for (int q = 0; q < C::CHUNKS; ++q) {
      const int c0 = C::COLS * wv + C::CM * q;  // first slot column of the batch
      auto ldc = [&](int m, int n) -> float2 {  // row n of column c0 + m (rows >= S0 zero)
        return n < S0 ? tile[n * kI3RS + c0 + m] : make_float2(0.f, 0.f);
      };
      TailZeroLoad<3, 2, true, decltype(ldc)> ldc1{ldc};
      auto stc = [&](int m, int n, float2 v) {  // keep rows [o0, o0 + S0)
        const int r = n - o0;
        if (r >= 0 && r < S0) tile[r * kI3RS + c0 + m] = v;
      };
      if constexpr (C::CM == 2) {
        // Forward passes 3, 8, then one pass in registers: the forward's last
        // radix-8 pass (butterfly j < 24 of column m = lane / 24 reads and
        // writes elements j + 24 r), the filter product, and the inverse's
        // first pass, the inverse running radix 8, 8, 3 (its first pass reads
        // the same elements j + 24 r).  One LDS round trip fewer.
        const bool act = lane < 2 * 24;
        const int m = act ? lane / 24 : 0, j = lane - 24 * (lane / 24);
        const int c = c0 + m;
        float2 kf[8], kn[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) kf[r] = act ? kc[c * kI3F + j + 24 * r] : make_float2(0.f, 0.f);
        if (c0 == 0) {  // the packed column's Nyquist filter column (wave-uniform)
#pragma unroll
          for (int r = 0; r < 8; ++r) kn[r] = act ? kc[kI3N2 * kI3F + j + 24 * r] : make_float2(0.f, 0.f);
        }
        mixed_pass<kI3F, 3, 1, false, 2, 64, false, true>(ldc1, sl, tws);
        mixed_pass<kI3F, 8, 3, false, 2, 64, false, true>(sl, sl, tws);
        float2 v[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) v[r] = sc[m * kI3CS + j + 24 * r];
        mixed_sync<true>();
#pragma unroll
        for (int r = 1; r < 8; ++r) v[r] = cmul(v[r], tws.template root<kI3F>(r * j));
        dft<8, false>(v);  // X[j + 24 r]
        if (c0 == 0) {
          // -k of k = j + 24 r: (24 - j) + 24 (7 - r) in lane 24 - j for j > 0,
          // 24 ((8 - r) mod 8) in this lane for j = 0
          const int src = j == 0 ? lane : 24 - j;
          float2 pm[8];
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            const float2 o = v[7 - r];
            pm[r] = make_float2(__shfl(o.x, src), __shfl(o.y, src));
            if (j == 0) pm[r] = v[(8 - r) & 7];
          }
          if (c == 0) {  // packed DC / Nyquist column: Y = Xd Kdc + i Xn Knyq
#pragma unroll
            for (int r = 0; r < 8; ++r) {
              float2 xd, xn;
              pack_split(v[r], pm[r], xd, xn);
              v[r] = cadd(cmul(xd, kf[r]), mul_i(cmul(xn, kn[r])));
            }
          } else {
#pragma unroll
            for (int r = 0; r < 8; ++r) v[r] = cmul(v[r], kf[r]);
          }
        } else {
#pragma unroll
          for (int r = 0; r < 8; ++r) v[r] = cmul(v[r], kf[r]);
        }
        dft<8, true>(v);  // the inverse's first pass (no twiddles): elements 8 j + r
        if (act) {
#pragma unroll
          for (int r = 0; r < 8; ++r) sc[m * kI3CS + 8 * j + r] = v[r];
        }
        mixed_sync<true>();
        mixed_pass<kI3F, 8, 8, true, 2, 64, false, true>(sl, sl, tws);
        mixed_pass<kI3F, 3, 64, true, 2, 64, false, true>(sl, stc, tws);
      } else {
        // The inverse's first pass (radix 3, butterfly (m, j = lane)) reads
        // elements lane + 64 r of each column m: their filter values are issued
        // here, so their L2 latency overlaps the forward transform.
        float2 kf[C::CM][3], kn[C::CM][3];
#pragma unroll
        for (int m = 0; m < C::CM; ++m)
#pragma unroll
          for (int r = 0; r < 3; ++r) kf[m][r] = kc[(c0 + m) * kI3F + lane + 64 * r];
        if (c0 == 0) {  // the packed column's Nyquist filter column (wave-uniform)
#pragma unroll
          for (int r = 0; r < 3; ++r) kn[0][r] = kc[kI3N2 * kI3F + lane + 64 * r];
        }
        fft_mixed_wave<kI3F, false, C::CM, false, C::CRMAX, C::CR2>(ldc1, sl, sl, tws);
        // the spectral product, read by the inverse's first pass (which reads
        // every value of the batch before it writes), in its call order
        struct Prod {
          const float2* sc;
          const float2 (&kf)[C::CM][3];
          const float2 (&kn)[C::CM][3];
          int c0;
          int q = 0;
          __device__ __forceinline__ float2 operator()(int m, int n) {
            const int r = q % 3;
            ++q;
            const float2 X = sc[m * kI3CS + n];
            if (c0 + m == 0) {  // packed DC / Nyquist column: Y = Xd Kdc + i Xn Knyq
              const float2 Xm = sc[m * kI3CS + (n == 0 ? 0 : kI3F - n)];
              float2 xd, xn;
              pack_split(X, Xm, xd, xn);
              return cadd(cmul(xd, kf[0][r]), mul_i(cmul(xn, kn[0][r])));
            }
            return cmul(X, kf[m][r]);
          }
        } ldp{sc, kf, kn, c0};
        fft_mixed_wave<kI3F, true, C::CM, false, C::CRMAX, C::CR2>(ldp, sl, stc, tws);
      }
    }
  }
  __syncthreads();

  // ---- C: inverse real row FFTs of the kept rows, window [o2, o2 + S2), epilogue ----
  if (rw0 < S0) {
    const int lane = opaque_tid() & 63;
    float2* rows = tile + rw0 * kI3RS;
#pragma unroll
    for (int i = 0; i < C::ROWS * (kI3N2 / 2) / 64; ++i) {  // repack in place
      const int jj = lane + 64 * i, m = jj / (kI3N2 / 2), p = jj - m * (kI3N2 / 2);
      float2* z = rows + m * kI3RS;
      const bool p0 = p == 0;
      const int pb = p0 ? kI3N2 / 2 : kI3N2 - p;
      const float2 u0 = z[p], u1 = z[pb];
      float2 zp, zq;
      real_repack(p0, u0, p0 ? u1 : cconj(u1), tws.template root<kI3F>(p), zp, zq);
      z[p] = zp;
      z[pb] = zq;
    }
    mixed_sync<true>();
    I3Lines tl{rows, kI3RS};
    fft_mixed_wave<kI3N2, true, C::ROWS, false, 8, 4>(tl, tl, tl, tws);
    const float sv = HAS_S ? Elem<DT>::round(Elem<DT>::load(s, h)) : 0.f;
    const int cpr = S2 >> 3;  // 8-sample chunks per output row
    const int nr = min(C::ROWS, S0 - rw0);
    const RowBuf<DT, false> ab(xi, HAS_S ? S0 * S2 : 0);
    const RowBuf<DT, true> ob(y + img, S0 * S2);
    for (int ch = lane; ch < nr * cpr; ch += 64) {
      const int mi = ch / cpr, m = rw0 + mi, c8 = (ch - mi * cpr) * 8;
      const int e0 = m * S2 + c8;
      Win8<DT, true> a;
      a.load(ab, e0);
      const float2* zr = tile + m * kI3RS;
      const int n0 = (c8 + o2) >> 1;
      float yo[8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float2 z = zr[n0 + u];
        yo[2 * u] = epilogue<DT>(z.x * scale, HAS_S, sv, a.at(2 * u));
        yo[2 * u + 1] = epilogue<DT>(z.y * scale, HAS_S, sv, a.at(2 * u + 1));
      }
      store8<DT, true>(ob, e0, yo);
    }
  }
}

}  // namespace nsq
