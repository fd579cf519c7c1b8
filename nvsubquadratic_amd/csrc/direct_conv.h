// Depthwise causal direct convolution building blocks (gfx950).
//
// Tap convention of nn.Conv1d with left padding K-1
// (nvsubquadratic/modules/causal_conv1d.py:113-139, and the reference test
// helper tests/ops/test_causal_conv1d_custom.py:65-72):
//   y[b,c,n] = act( sum_{j<K} w[c,j] * x[b,c,n-K+1+j] + bias[c] )
//
// Work decomposition: a workgroup owns a tile of kTile outputs of one (b, c)
// row.  The input tile plus its K-1 halo is staged once in LDS as fp32; each
// thread produces kPer consecutive outputs from a register sliding window
// (kPer new values per kPer taps), so LDS traffic is 2 reads per kPer^2 FMAs.
// Weights are wave-uniform and are read through the scalar cache.
#pragma once

#include "fft_core.h"

namespace nsq {

constexpr int kConvThreads = 256;
constexpr int kConvPer = 8;                            // outputs per thread
constexpr int kConvTile = kConvThreads * kConvPer;    // outputs per workgroup
constexpr int kConvMaxK = 256;

// Activation codes NSQ_ACT_IDENTITY / NSQ_ACT_SILU come from include/nsq_hip.h.

__device__ __forceinline__ float sigmoidf_(float v) { return 1.f / (1.f + __expf(-v)); }

template <int ACT>
__device__ __forceinline__ float act_fwd(float v) {
  if constexpr (ACT == NSQ_ACT_SILU) return v * sigmoidf_(v);
  return v;
}

// d silu(p) / dp = s(p) * (1 + p * (1 - s(p)))
__device__ __forceinline__ float dsilu(float p) {
  const float s = sigmoidf_(p);
  return s * (1.f + p * (1.f - s));
}

// LDS floats needed for a tile with halo K-1 plus the window's read-ahead.
constexpr int conv_tile_floats(int kmax) { return kConvTile + kmax - 1 + 2 * kConvPer; }

// Staging of row[first + i], i in [0, count <= MAXC), as fp32 with zeros
// outside [0, len).  load() issues every element load of the thread at once
// (fixed trip count), so they are in flight together; store() writes them to
// LDS.  Several rows can be loaded before any is stored.  The row is a raw
// buffer of len elements (its pointer is uniform: one (b, c) row per
// workgroup): positions at or beyond len read as zero through the hardware
// range check, positions before 0 through RowBuf::elem_halo.
template <int DT, int MAXC>
struct RowStage {
  static constexpr int IT = (MAXC + kConvThreads - 1) / kConvThreads;
  float v[IT];
  __device__ __forceinline__ void load(const typename Elem<DT>::T* __restrict__ row, int64_t first, int count,
                                       int64_t len) {
    (void)count;
    const RowBuf<DT, false> rb(row, len);
    const int f = int(first);  // first >= -(2 * kConvMaxK); rows are < 2^31 elements
#pragma unroll
    for (int it = 0; it < IT; ++it) v[it] = rb.elem_halo(f + int(threadIdx.x) + it * kConvThreads);
  }
  __device__ __forceinline__ void store(float* dst, int count) const {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int i = int(threadIdx.x) + it * kConvThreads;
      if (i < count) dst[i] = v[it];
    }
  }
};

// One row staged into LDS; ends with a barrier.
template <int DT, int MAXC>
__device__ __forceinline__ void stage_row(float* dst, const typename Elem<DT>::T* __restrict__ row, int64_t first,
                                          int count, int64_t len) {
  RowStage<DT, MAXC> rs;
  rs.load(row, first, count, len);
  rs.store(dst, count);
  __syncthreads();
}

// LDS floats of a staged weight row (K <= kConvMaxK, zero-padded to a
// multiple of kConvPer).
constexpr int kConvWeightFloats = kConvMaxK;
static_assert(kConvMaxK == kConvThreads && kConvMaxK % kConvPer == 0, "stage_weights: one tap per thread");

// One channel's depthwise weights staged in LDS for slide_fma: wl[j] = w[j]
// (w[K-1-j] when REV, the correlation of the adjoints) for j < K, zero up to
// the next multiple of kConvPer.  The caller's staging barrier must follow.
template <bool REV>
__device__ __forceinline__ void stage_weights(float* wl, const float* __restrict__ w, int K) {
  const int j = int(threadIdx.x);
  const int kp = (K + kConvPer - 1) / kConvPer * kConvPer;
  const bool ok = j < K;
  const float v = w[ok ? (REV ? K - 1 - j : j) : 0];
  if (j < kp) wl[j] = ok ? v : 0.f;
}

// acc[e] += sum_{j<K} wl[j] * xs[base + e + j], e < kConvPer, using a
// register window.  wl: weights staged by stage_weights (all lanes read the
// same LDS words: broadcast, and no per-tap branch or scalar-load wait).  xs
// must hold base + K + 7 valid entries (the caller's tile has kConvPer slack).
// xs, wl and base are 16-byte aligned (base a multiple of kConvPer), and the
// window / weight refills are explicit 16-byte LDS reads: as pairs of 4-byte
// reads at the 32-byte lane stride of `base` they conflicted on the banks.
__device__ __forceinline__ void slide_fma(float (&acc)[kConvPer], const float* xs, int base, int K,
                                          const float* wl) {
  static_assert(kConvPer == 8, "slide_fma: two 16-byte refills per step");
  float win[2 * kConvPer];
  {
    const float4 a = *reinterpret_cast<const float4*>(xs + base);
    const float4 b = *reinterpret_cast<const float4*>(xs + base + 4);
    win[0] = a.x; win[1] = a.y; win[2] = a.z; win[3] = a.w;
    win[4] = b.x; win[5] = b.y; win[6] = b.z; win[7] = b.w;
  }
  for (int jb = 0; jb < K; jb += kConvPer) {
    const float4 a = *reinterpret_cast<const float4*>(xs + base + jb + kConvPer);
    const float4 b = *reinterpret_cast<const float4*>(xs + base + jb + kConvPer + 4);
    const float4 wa = *reinterpret_cast<const float4*>(wl + jb);
    const float4 wb = *reinterpret_cast<const float4*>(wl + jb + 4);
    win[8] = a.x; win[9] = a.y; win[10] = a.z; win[11] = a.w;
    win[12] = b.x; win[13] = b.y; win[14] = b.z; win[15] = b.w;
    const float w[kConvPer] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
    for (int jj = 0; jj < kConvPer; ++jj) {
#pragma unroll
      for (int e = 0; e < kConvPer; ++e) acc[e] = fmaf(w[jj], win[e + jj], acc[e]);
    }
#pragma unroll
    for (int e = 0; e < kConvPer; ++e) win[e] = win[kConvPer + e];
  }
}

// Per-channel reduction for depthwise weight / bias gradients:
//   gw[c, j] += sum_n gp[n] * x[n - K + 1 + j],  gb[c] += sum_n gp[n]
// over one staged tile: gps[i] = gp[n0 + i] (i < kConvTile), xs[i] = x[n0 - K + 1 + i].
// Thread t owns lag block lb = t % LB (lags 8*lb .. 8*lb+7) and the output
// chunk nc = t / LB; acc and bacc persist across tiles.
__device__ __forceinline__ void wgrad_tile(float (&acc)[kConvPer], float& bacc, const float* gps, const float* xs,
                                           int K, int count) {
  const int LB = (K + kConvPer - 1) / kConvPer;
  const int NC = kConvThreads / LB;
  const int t = threadIdx.x;
  const int lb = t % LB, nc = t / LB;
  if (nc >= NC) return;
  const int chunk = (kConvTile + NC - 1) / NC;
  const int nb = nc * chunk;
  const int ne = min(count, nb + chunk);
  if (nb >= ne) return;
  float win[kConvPer];
#pragma unroll
  for (int jj = 0; jj < kConvPer; ++jj) win[jj] = xs[nb + lb * kConvPer + jj];
  for (int n = nb; n < ne; ++n) {
    const float g = gps[n];
#pragma unroll
    for (int jj = 0; jj < kConvPer; ++jj) acc[jj] = fmaf(g, win[jj], acc[jj]);
    if (lb == 0) bacc += g;
#pragma unroll
    for (int jj = 0; jj < kConvPer - 1; ++jj) win[jj] = win[jj + 1];
    win[kConvPer - 1] = xs[n + 1 + lb * kConvPer + kConvPer - 1];
  }
}

// Fixed-order reduction of the wgrad_tile accumulators over the output
// chunks (deterministic), then the store of gw[c, 0:K] and gb[c].
__device__ __forceinline__ void wgrad_finish(float (&acc)[kConvPer], float bacc, float* red, float* gw_row, float* gb,
                                             int K) {
  const int LB = (K + kConvPer - 1) / kConvPer;
  const int NC = kConvThreads / LB;
  const int t = threadIdx.x;
  const int lb = t % LB, nc = t / LB;
  __syncthreads();
  // red layout: [NC][LB*8] then [NC] for the bias partials
  if (nc < NC) {
#pragma unroll
    for (int jj = 0; jj < kConvPer; ++jj) red[nc * LB * kConvPer + lb * kConvPer + jj] = acc[jj];
    if (lb == 0) red[NC * LB * kConvPer + nc] = bacc;
  }
  __syncthreads();
  for (int j = t; j < K; j += kConvThreads) {
    float s = 0.f;
    for (int c = 0; c < NC; ++c) s += red[c * LB * kConvPer + j];
    gw_row[j] = s;
  }
  if (t == 0 && gb) {
    float s = 0.f;
    for (int c = 0; c < NC; ++c) s += red[NC * LB * kConvPer + c];
    *gb = s;
  }
}

// Kernels shared by the causal conv and B2B backward passes.
// gx[i] = sum_j w[j] gp[i + K - 1 - j]  (gp = gpre in GT precision).  grid as forward.
template <int DT, int GT>
__global__ __launch_bounds__(kConvThreads) void cconv_gx_kernel(const typename Elem<GT>::T* __restrict__ gp,
                                                                 const float* __restrict__ w,
                                                                 typename Elem<DT>::T* __restrict__ gx, int C, int L,
                                                                 int K) {
  __shared__ __align__(16) float gs[conv_tile_floats(kConvMaxK)];
  __shared__ __align__(16) float wl[kConvWeightFloats];
  const int64_t row = blockIdx.x;
  const int c = int(row % C);
  const int64_t n0 = int64_t(blockIdx.y) * kConvTile;
  stage_weights<true>(wl, w + int64_t(c) * K, K);
  stage_row<GT, conv_tile_floats(kConvMaxK)>(gs, gp + row * L, n0, kConvTile + K - 1 + 2 * kConvPer, L);
  float acc[kConvPer];
#pragma unroll
  for (int e = 0; e < kConvPer; ++e) acc[e] = 0.f;
  const int base = threadIdx.x * kConvPer;
  // acc[e] = sum_m w[K-1-m] gs[base + e + m]
  slide_fma(acc, gs, base, K, wl);
  typename Elem<DT>::T* gr = gx + row * L;
#pragma unroll
  for (int e = 0; e < kConvPer; e += 2) {
    const int64_t n = n0 + base + e;
    if (n < L) store_pair<DT>(gr, n, L, make_float2(acc[e], acc[e + 1]));
  }
}

// Weight / bias gradients, one workgroup per channel (fixed-order sums over
// batch and length).  grid = C.
template <int DT, int GT>
__global__ __launch_bounds__(kConvThreads) void cconv_wgrad_kernel(const typename Elem<GT>::T* __restrict__ gp,
                                                                    const typename Elem<DT>::T* __restrict__ x,
                                                                    float* __restrict__ gw, float* __restrict__ gb,
                                                                    int B, int C, int L, int K) {
  __shared__ float xs[conv_tile_floats(kConvMaxK)];
  __shared__ float gps[kConvTile + 2 * kConvPer];
  __shared__ float red[kConvThreads * kConvPer + kConvThreads];
  const int c = blockIdx.x;
  float acc[kConvPer];
#pragma unroll
  for (int e = 0; e < kConvPer; ++e) acc[e] = 0.f;
  float bacc = 0.f;
  for (int b = 0; b < B; ++b) {
    const int64_t row = int64_t(b) * C + c;
    for (int64_t n0 = 0; n0 < L; n0 += kConvTile) {
      const int count = int((L - n0) < kConvTile ? (L - n0) : kConvTile);
      stage_row<DT, conv_tile_floats(kConvMaxK)>(xs, x + row * L, n0 - (K - 1), kConvTile + K - 1 + 2 * kConvPer, L);
      stage_row<GT, conv_tile_floats(1)>(gps, gp + row * L, n0, kConvTile + 2 * kConvPer, L);
      wgrad_tile(acc, bacc, gps, xs, K, count);
      __syncthreads();
    }
  }
  wgrad_finish(acc, bacc, red, gw + int64_t(c) * K, gb ? gb + c : nullptr, K);
}

}  // namespace nsq
