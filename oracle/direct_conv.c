/*
 * oracle/direct_conv.c - TEST INFRASTRUCTURE ONLY (the checker, never the product).
 *
 * Brute-force direct (non-FFT) convolutions in double precision, used to pin
 * the FFT restatement in oracle/fftconv_ref.py and to write the golden
 * fixtures under tests/golden/.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library.
 *
 * Each function states the closed form it evaluates and the reference code it
 * stands for.  All arrays are row-major and contiguous.
 */
#include <stdint.h>

/*
 * Causal 1D convolution with the reference's FFT length F = min(L+K, 2L)
 * (nvsubquadratic/ops/fftconv.py:546-600):
 *   full[j] = sum_m k[h,m] x[b,h,j-m]            (linear convolution)
 *   y[b,h,n] = sum_{j == n (mod F)} full[j]      (circular fold at length F)
 * For K <= L+1 the fold is empty and y is the plain causal convolution of the
 * reference test helper tests/ops/test_fftconv.py:76-83.
 * x: [B,H,L], k: [H,K], y: [B,H,L].
 */
void oracle_causal_conv1d(const double* x, const double* k, double* y, int64_t B, int64_t H, int64_t L,
                          int64_t K) {
  const int64_t F = (L + K < 2 * L) ? L + K : 2 * L;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h) {
      const double* xr = x + (b * H + h) * L;
      const double* kr = k + h * K;
      double* yr = y + (b * H + h) * L;
      for (int64_t n = 0; n < L; ++n) {
        double acc = 0.0;
        /* contributions j = n + t*F, t >= 0, j <= L+K-2 */
        for (int64_t j = n; j <= L + K - 2; j += F)
          for (int64_t m = 0; m < K; ++m) {
            int64_t i = j - m;
            if (i >= 0 && i < L) acc += kr[m] * xr[i];
          }
        yr[n] = acc;
      }
    }
}

/*
 * Adjoint of oracle_causal_conv1d (what autograd derives for the reference
 * path): with the same fold,
 *   gx[b,h,i] = sum_n g[b,h,n] * dy[n]/dx[i],  gk[h,m] = sum_{b,n} g * dy[n]/dk[m].
 * Evaluated by brute force over the (n, m) pairs of the forward.
 */
void oracle_causal_conv1d_bwd(const double* g, const double* x, const double* k, double* gx, double* gk,
                              int64_t B, int64_t H, int64_t L, int64_t K) {
  const int64_t F = (L + K < 2 * L) ? L + K : 2 * L;
  for (int64_t i = 0; i < B * H * L; ++i) gx[i] = 0.0;
  for (int64_t i = 0; i < H * K; ++i) gk[i] = 0.0;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h) {
      const double* xr = x + (b * H + h) * L;
      const double* gr = g + (b * H + h) * L;
      const double* kr = k + h * K;
      double* gxr = gx + (b * H + h) * L;
      double* gkr = gk + h * K;
      for (int64_t n = 0; n < L; ++n)
        for (int64_t j = n; j <= L + K - 2; j += F)
          for (int64_t m = 0; m < K; ++m) {
            int64_t i = j - m;
            if (i >= 0 && i < L) {
              gxr[i] += gr[n] * kr[m];
              gkr[m] += gr[n] * xr[i];
            }
          }
    }
}

/*
 * Depthwise causal conv with nn.Conv1d tap order (cross-correlation, left pad
 * K-1), tests/ops/test_causal_conv1d_custom.py:65-72:
 *   y[b,c,n] = sum_{j<K} w[c,j] x[b,c,n-K+1+j] + bias[c]   (bias may be NULL)
 */
void oracle_direct_causal_conv1d(const double* x, const double* w, const double* bias, double* y, int64_t B,
                                 int64_t C, int64_t L, int64_t K) {
  for (int64_t b = 0; b < B; ++b)
    for (int64_t c = 0; c < C; ++c) {
      const double* xr = x + (b * C + c) * L;
      const double* wr = w + c * K;
      double* yr = y + (b * C + c) * L;
      for (int64_t n = 0; n < L; ++n) {
        double acc = bias ? bias[c] : 0.0;
        for (int64_t j = 0; j < K; ++j) {
          int64_t i = n - K + 1 + j;
          if (i >= 0) acc += wr[j] * xr[i];
        }
        yr[n] = acc;
      }
    }
}

/*
 * Non-causal "same" N-d depthwise convolution (N = 1, 2, 3; unused trailing
 * dims of size 1), the closed form the reference tests use for the 2D/3D FFT
 * ops (tests/ops/test_fftconv.py:68-101):
 *   y[b,h,p] = sum_q k[h,q] x[b,h,p + c - q],  c = K//2 per axis,
 * taps outside x are zero.  x: [B,H,X,Y,Z], k: [H,KX,KY,KZ].
 */
void oracle_conv3d_same(const double* x, const double* k, double* y, int64_t B, int64_t H, int64_t X, int64_t Y,
                        int64_t Z, int64_t KX, int64_t KY, int64_t KZ) {
  const int64_t cx = KX / 2, cy = KY / 2, cz = KZ / 2;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h) {
      const double* xr = x + (b * H + h) * X * Y * Z;
      const double* kr = k + h * KX * KY * KZ;
      double* yr = y + (b * H + h) * X * Y * Z;
      for (int64_t px = 0; px < X; ++px)
        for (int64_t py = 0; py < Y; ++py)
          for (int64_t pz = 0; pz < Z; ++pz) {
            double acc = 0.0;
            for (int64_t qx = 0; qx < KX; ++qx) {
              int64_t ix = px + cx - qx;
              if (ix < 0 || ix >= X) continue;
              for (int64_t qy = 0; qy < KY; ++qy) {
                int64_t iy = py + cy - qy;
                if (iy < 0 || iy >= Y) continue;
                for (int64_t qz = 0; qz < KZ; ++qz) {
                  int64_t iz = pz + cz - qz;
                  if (iz < 0 || iz >= Z) continue;
                  acc += kr[(qx * KY + qy) * KZ + qz] * xr[(ix * Y + iy) * Z + iz];
                }
              }
            }
            yr[(px * Y + py) * Z + pz] = acc;
          }
    }
}
