// Depthwise causal direct convolution (k = 1..256), forward and backward.
//
// Replaces the native kernel the reference binds at
// nvsubquadratic/ops/causal_conv1d_custom.py:81-98 (subquadratic_ops_torch
// .causal_conv1d(x, w, bias, activation)), used by the Hyena short-conv slot
// through nvsubquadratic/modules/subq_ops_causal_conv1d.py:77-83.
#include <mutex>

#include "direct_conv.h"

namespace nsq {

// Scratch of nsq_causal_conv1d_bwd_noalloc: one copy per GPU, resident from
// module load to process exit.  In host code `scratch` names a host-side
// stand-in, not device memory: the device address of each GPU's copy comes
// from hipGetSymbolAddress (noalloc_scratch below) and only that address is
// ever handed to kernels.
constexpr size_t kNoAllocScratchBytes = NSQ_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

// Forward for K <= 16 taps from registers: thread t of a tile owns outputs
// n = n0 + 8t + e, e < 8; with the taps left-padded to KP = 4, 8 or 16,
// y[n] = act(bias + sum_j wk[j] x[n - KP + 1 + j]).  Its x window
// [n0 + 8t - 8 XB, n0 + 8t + 8) comes straight from HBM in aligned chunks of 8
// (Win8; the chunks before the thread's own are its neighbours', read again
// from L2), so no LDS staging or barrier.  grid = (B*C, ceil(L / kConvTile)).
template <int DT, bool AL, int ACT, int KP>
__global__ __launch_bounds__(kConvThreads) void cconv_fwd_short_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                                        const float* __restrict__ w,
                                                                        const float* __restrict__ bias,
                                                                        typename Elem<DT>::T* __restrict__ y, int C,
                                                                        int L, int K) {
  static_assert(KP == 4 || KP == 8 || KP == 16, "cconv_fwd_short: taps padded to 4, 8 or 16");
  static_assert(kConvPer == 8, "cconv_fwd_short: 8 outputs per thread");
  constexpr int XB = (KP - 1 + 7) / 8;  // chunks before the outputs: positions >= 1 - KP
  const int64_t row = blockIdx.x;
  const int c = int(row % C);
  const int base = int(blockIdx.y) * kConvTile + kConvPer * int(threadIdx.x);
  float wk[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    const int sl = j - (KP - K);
    wk[j] = sl >= 0 ? w[int64_t(c) * K + (sl >= 0 ? sl : 0)] : 0.f;
  }
  const float b0 = bias ? bias[c] : 0.f;
  const RowBuf<DT, false> xb(x + row * L, L);
  Win8<DT, AL> xc[XB + 1];
#pragma unroll
  for (int i = 0; i <= XB; ++i) xc[i].load(xb, base + 8 * (i - XB));
  auto xat = [&](int p) { return xc[(p + 8 * XB) >> 3].at((p + 8 * XB) & 7); };
  float out[kConvPer];
#pragma unroll
  for (int e = 0; e < kConvPer; ++e) {
    float a = b0;
#pragma unroll
    for (int j = 0; j < KP; ++j) a = fmaf(wk[j], xat(e - KP + 1 + j), a);
    out[e] = act_fwd<ACT>(a);
  }
  store8<DT, AL>(RowBuf<DT, AL>(y + row * L, L), base, out);
}

// ---------------------------------------------------------------------------
// Matrix-core path (K >= 16; used above 16 taps): a workgroup walks a segment of
// kConvSegTiles tiles of one (b, c) row; per tile the source window (fp32,
// in the split layout ToeplitzMfma reads) is staged from registers loaded during the
// previous tile, the MFMA band gives acc[p] for the tile's 2048 outputs, and
// the epilogue stores from the accumulator layout through a range-checked row
// buffer.  Modes:
//   FWD (ACT identity / silu): src = x from n0 - K + 1, y = act(acc + bias);
//   GPRE: the same conv, out (fp32) = gy * silu'(acc + bias);
//   CORR: src = gp from n0 on the reversed band, gx = acc
//         (gx[n] = sum_j w[j] gp[n + K - 1 - j]).
// ---------------------------------------------------------------------------
enum { CC_FWD_ID = 0, CC_FWD_SILU = 1, CC_GPRE = 2, CC_CORR = 3 };
constexpr int kConvSegTiles = 4;

template <int DS, int DO, int NS, int MODE>
__global__ __launch_bounds__(kConvThreads) __attribute__((amdgpu_waves_per_eu(3))) void cconv_mfma_kernel(
    const typename Elem<DS>::T* __restrict__ src, const float* __restrict__ w, const float* __restrict__ bias,
    const typename Elem<DO>::T* __restrict__ gy, void* __restrict__ out, int C, int L, int K) {
  constexpr int ZW = mfma_src_count<NS>();
  constexpr int ZR = win_half(ZW);
  __shared__ __align__(16) float zp[win_words(ZW)];
  __shared__ __align__(16) float wl[kConvWeightFloats];
  const int64_t row = blockIdx.x;
  const int c = int(row % C);
  const int ntiles = (L + kConvTile - 1) / kConvTile;
  const int t_begin = int(blockIdx.y) * kConvSegTiles;
  const int t_end = min(ntiles, t_begin + kConvSegTiles);
  const int t = int(threadIdx.x);
  constexpr bool CORR = MODE == CC_CORR;
  if (CORR)
    stage_weights<true>(wl, w + int64_t(c) * K, K);
  else
    stage_weights<false>(wl, w + int64_t(c) * K, K);
  const int shift = CORR ? 0 : K - 1;  // window word m is src[n0 - shift + m]
  RowStage<DS, ZW> sw;
  sw.load(src + row * L, int64_t(t_begin) * kConvTile - shift, 0, L);
  __syncthreads();  // weights staged
  ToeplitzMfma<NS> tm;
  tm.load_weights(wl, K);
  const float b0 = (!CORR && bias) ? bias[c] : 0.f;
  const RowBuf<DO, false> ob((typename Elem<DO>::T*)out + row * L, L);
  const RowBuf<NSQ_DTYPE_F32, false> ofb((float*)out + row * L, L);
  const RowBuf<DO, false> gyb(gy + row * L, L);
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
  for (int ti = t_begin; ti < t_end; ++ti) {
    const int64_t n0 = int64_t(ti) * kConvTile;
#pragma unroll
    for (int it = 0; it < RowStage<DS, ZW>::IT; ++it) {
      const int m = t + it * kConvThreads;
      if (m < ZW) zp[win_at(m, ZR)] = RowBuf<DS, false>::bits_to_f32(sw.v[it]);
    }
    __syncthreads();
    if (ti + 1 < t_end) sw.load(src + row * L, n0 + kConvTile - shift, 0, L);
    nsq_f32x4_t acc0, acc1;
    tm.run2(zp, ZR, 16 * wave, 16 * (wave + kConvWaves), acc0, acc1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int p = 16 * (16 * (wave + h * kConvWaves) + 4 * (l >> 4) + r) + (l & 15);
        const float a = (h ? acc1[r] : acc0[r]) + b0;
        if constexpr (MODE == CC_FWD_ID) {
          ob.store_elem(n0 + p, a);
        } else if constexpr (MODE == CC_FWD_SILU) {
          ob.store_elem(n0 + p, act_fwd<NSQ_ACT_SILU>(a));
        } else if constexpr (MODE == CC_GPRE) {
          ofb.store_elem(n0 + p, gyb.elem(n0 + p) * dsilu(a));
        } else {
          ob.store_elem(n0 + p, a);
        }
      }
    }
    __syncthreads();
  }
}

// Weight / bias gradients on the matrix cores (K >= 16; used above 16 taps): per tile,
//   D[i][t] += sum_a gp[16a + i] * xwin[16a + t],  xwin[m] = x[n0 - K + 1 + m],
// gw[j] = sum_i D[i][i + j] over the workgroup's tiles (one channel, a segment
// of its (b, tile) sequence), gb = sum gp; fixed-order reduction into a
// per-workgroup partial [K + 1], summed by cconv_wgrad_reduce_kernel.
template <int DG, int DX, int NS>
__global__ __launch_bounds__(kConvThreads) __attribute__((amdgpu_waves_per_eu(2))) void cconv_wgrad_mfma_kernel(
    const typename Elem<DG>::T* __restrict__ gp, const typename Elem<DX>::T* __restrict__ x, float* __restrict__ part,
    int B, int C, int L, int K) {
  constexpr int ZW = mfma_src_count<NS>();
  constexpr int ZR = win_half(ZW);
  constexpr int ZWORDS = win_words(ZW);
  constexpr int TG = NS / 4;
  constexpr int RW = 4 * NS;
  static_assert(16 * RW <= ZWORDS + kConvTile, "cconv_wgrad_mfma_kernel: reduction area");
  __shared__ __align__(16) float sm[ZWORDS + kConvTile];
  float* zp = sm;
  float* gs = sm + ZWORDS;  // gp of the tile, plain
  const int c = int(blockIdx.x);
  const int ntiles = (L + kConvTile - 1) / kConvTile;
  const int g_begin = int(blockIdx.y) * kConvSegTiles;
  const int g_end = min(B * ntiles, g_begin + kConvSegTiles);
  const int t = int(threadIdx.x);
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
  const int kk = l >> 4, li = l & 15;
  nsq_f32x4_t D[TG];
#pragma unroll
  for (int tg = 0; tg < TG; ++tg) D[tg] = nsq_f32x4_t{0.f, 0.f, 0.f, 0.f};
  float bacc = 0.f;
  for (int g = g_begin; g < g_end; ++g) {
    const int b = g / ntiles, ti = g - b * ntiles;
    const int64_t row = int64_t(b) * C + c;
    const int64_t n0 = int64_t(ti) * kConvTile;
    {
      RowStage<DX, ZW> sx;
      RowStage<DG, kConvTile> sg;
      sx.load(x + row * L, n0 - (K - 1), 0, L);
      sg.load(gp + row * L, n0, 0, L);
#pragma unroll
      for (int it = 0; it < RowStage<DX, ZW>::IT; ++it) {
        const int m = t + it * kConvThreads;
        if (m < ZW) zp[win_at(m, ZR)] = RowBuf<DX, false>::bits_to_f32(sx.v[it]);
      }
      sg.store(gs, kConvTile);
#pragma unroll
      for (int it = 0; it < RowStage<DG, kConvTile>::IT; ++it) bacc += RowBuf<DG, false>::bits_to_f32(sg.v[it]);
    }
    __syncthreads();
    // win_at(16 (a0 + kk + tg) + li) = win_at(16 kk + li) + 8 (a0 + tg)
    const float* zl = zp + win_at(16 * kk + li, ZR);
#pragma unroll 2
    for (int a0 = 32 * wave; a0 < 32 * wave + 32; a0 += 4) {
      const float av = gs[16 * (a0 + kk) + li];
#pragma unroll
      for (int tg = 0; tg < TG; ++tg) {
        const float bv = zl[8 * (a0 + tg)];
        D[tg] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, D[tg], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  float* red = sm;
  for (int w = 0; w < kConvWaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int tg = 0; tg < TG; ++tg)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float& dst = red[(4 * kk + r) * RW + 16 * tg + li];
          dst = (w == 0 ? 0.f : dst) + D[tg][r];
        }
    }
    __syncthreads();
  }
  const int nparts = int(gridDim.y);
  float* pw = part + (int64_t(c) * nparts + blockIdx.y) * (K + 1);
  if (t < K) {
    float sacc = 0.f;
    for (int i = 0; i < 16; ++i) sacc += red[i * RW + i + t];
    pw[t] = sacc;
  }
  __syncthreads();
  red[t] = bacc;  // bias partial: fixed-order sum over the threads
  __syncthreads();
  if (t == 0) {
    float sacc = 0.f;
    for (int i = 0; i < kConvThreads; ++i) sacc += red[i];
    pw[K] = sacc;
  }
}

__global__ void cconv_wgrad_reduce_kernel(const float* __restrict__ part, int nparts, int K, float* __restrict__ gw,
                                          float* __restrict__ gb) {
  const int c = blockIdx.x, j = threadIdx.x;
  if (j > K) return;
  const float* pc = part + int64_t(c) * nparts * (K + 1) + j;
  float sacc = 0.f;
  for (int p = 0; p < nparts; ++p) sacc += pc[int64_t(p) * (K + 1)];
  if (j < K)
    gw[int64_t(c) * K + j] = sacc;
  else if (gb)
    gb[c] = sacc;
}

static int64_t cconv_wgrad_parts(int64_t B, int64_t L) {
  return ceil_div(B * ceil_div(L, kConvTile), kConvSegTiles);
}

template <int DT, int NS>
static void launch_fwd_mfma(const void* x, const float* w, const float* bias, void* y, int act, int B, int C, int L,
                            int K, hipStream_t st) {
  using ET = typename Elem<DT>::T;
  dim3 grid(B * C, unsigned(ceil_div(ceil_div(L, kConvTile), kConvSegTiles)));
  if (act == NSQ_ACT_SILU)
    hipLaunchKernelGGL((cconv_mfma_kernel<DT, DT, NS, CC_FWD_SILU>), grid, dim3(kConvThreads), 0, st, (const ET*)x, w,
                       bias, (const ET*)nullptr, y, C, L, K);
  else
    hipLaunchKernelGGL((cconv_mfma_kernel<DT, DT, NS, CC_FWD_ID>), grid, dim3(kConvThreads), 0, st, (const ET*)x, w,
                       bias, (const ET*)nullptr, y, C, L, K);
}

template <int DT, int NS>
static void launch_bwd_mfma(const void* gy, const void* x, const float* w, const float* bias, void* gx, float* gw,
                            float* gb, int act, int B, int C, int L, int K, float* ws, hipStream_t st) {
  using ET = typename Elem<DT>::T;
  dim3 grid(B * C, unsigned(ceil_div(ceil_div(L, kConvTile), kConvSegTiles)));
  const int64_t nparts = cconv_wgrad_parts(B, L);
  dim3 wgrid(C, unsigned(nparts));
  if (act == NSQ_ACT_SILU) {
    float* gpre = ws;
    float* part = ws + int64_t(B) * C * L;
    hipLaunchKernelGGL((cconv_mfma_kernel<DT, DT, NS, CC_GPRE>), grid, dim3(kConvThreads), 0, st, (const ET*)x, w,
                       bias, (const ET*)gy, (void*)gpre, C, L, K);
    hipLaunchKernelGGL((cconv_mfma_kernel<NSQ_DTYPE_F32, DT, NS, CC_CORR>), grid, dim3(kConvThreads), 0, st,
                       (const float*)gpre, w, (const float*)nullptr, (const ET*)nullptr, gx, C, L, K);
    hipLaunchKernelGGL((cconv_wgrad_mfma_kernel<NSQ_DTYPE_F32, DT, NS>), wgrid, dim3(kConvThreads), 0, st,
                       (const float*)gpre, (const ET*)x, part, B, C, L, K);
    hipLaunchKernelGGL(cconv_wgrad_reduce_kernel, dim3(C), dim3(kConvThreads + 64), 0, st, (const float*)part,
                       int(nparts), K, gw, gb);
  } else {
    float* part = ws;
    hipLaunchKernelGGL((cconv_mfma_kernel<DT, DT, NS, CC_CORR>), grid, dim3(kConvThreads), 0, st, (const ET*)gy, w,
                       (const float*)nullptr, (const ET*)nullptr, gx, C, L, K);
    hipLaunchKernelGGL((cconv_wgrad_mfma_kernel<DT, DT, NS>), wgrid, dim3(kConvThreads), 0, st, (const ET*)gy,
                       (const ET*)x, part, B, C, L, K);
    hipLaunchKernelGGL(cconv_wgrad_reduce_kernel, dim3(C), dim3(kConvThreads + 64), 0, st, (const float*)part,
                       int(nparts), K, gw, gb);
  }
}

// ---------------------------------------------------------------------------
// Backward for K <= 16 taps in one register-resident pass (the Hyena
// short-conv case).  Thread t of a tile owns outputs n = n0 + 8t + e, e < 8.
// With the taps left-padded to KP = 4, 8 or 16 (wk[j] = w[j - (KP - K)]):
//   pre[n]  = bias + sum_j wk[j] x[n - KP + 1 + j],  gpre = gy * silu'(pre) (or gy)
//   gx[n]   = sum_s wr[s] gpre[n + s],                wr[s] = w[K - 1 - s] (s < K)
//   gwk[j] += gpre[n] x[n - KP + 1 + j],              gb += gpre[n]
// gpre is recomputed at the KP - 1 positions past the thread's 8 (its
// neighbour owns them).  x over [n0 + 8t - 8 XB, n0 + 8t + 8 XA) and gy over
// [n0 + 8t, n0 + 8t + 8 XA) come straight from HBM in aligned chunks of 8
// (Win8).  The weight / bias sums stay in registers over the workgroup's tiles
// (one channel, a segment of its (b, tile) sequence) and are reduced in a fixed
// order into a per-workgroup partial [K + 1].
// ---------------------------------------------------------------------------
template <int DT, bool AL, int ACT, int KP>
__global__ __launch_bounds__(kConvThreads) void cconv_bwd_short_kernel(
    const typename Elem<DT>::T* __restrict__ gy, const typename Elem<DT>::T* __restrict__ x,
    const float* __restrict__ w, const float* __restrict__ bias, typename Elem<DT>::T* __restrict__ gx,
    float* __restrict__ part, int B, int C, int L, int K) {
  static_assert(KP == 4 || KP == 8 || KP == 16, "cconv_bwd_short: taps padded to 4, 8 or 16");
  static_assert(kConvPer == 8, "cconv_bwd_short: 8 outputs per thread");
  constexpr int NG = kConvPer + KP - 1;  // gpre positions per thread: [0, NG)
  constexpr int XB = (KP - 1 + 7) / 8;   // x chunks before the outputs: positions >= 1 - KP
  constexpr int XA = (NG + 7) / 8;       // x and gy chunks from the outputs on: positions < NG
  __shared__ float red[(KP + 1) * kConvThreads];
  const int c = int(blockIdx.x);
  const int ntiles = (L + kConvTile - 1) / kConvTile;
  const int g_begin = int(blockIdx.y) * kConvSegTiles;
  const int g_end = min(B * ntiles, g_begin + kConvSegTiles);
  const int t = int(threadIdx.x);
  float wk[KP], wr[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    const int sl = j - (KP - K);
    wk[j] = sl >= 0 ? w[int64_t(c) * K + (sl >= 0 ? sl : 0)] : 0.f;
    wr[j] = j < K ? w[int64_t(c) * K + (j < K ? K - 1 - j : 0)] : 0.f;
  }
  const float b0 = bias ? bias[c] : 0.f;
  float gwk[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) gwk[j] = 0.f;
  float gbs = 0.f;
  for (int g = g_begin; g < g_end; ++g) {
    const int b = g / ntiles, ti = g - b * ntiles;
    const int64_t row = int64_t(b) * C + c;
    const int base = ti * kConvTile + kConvPer * t;
    const RowBuf<DT, false> xb(x + row * L, L), gb(gy + row * L, L);
    Win8<DT, AL> xc[XB + XA], gc[XA];
#pragma unroll
    for (int i = 0; i < XB + XA; ++i) xc[i].load(xb, base + 8 * (i - XB));
#pragma unroll
    for (int i = 0; i < XA; ++i) gc[i].load(gb, base + 8 * i);
    // x at position base + p for p in [-8 XB, 8 XA), gy at base + p for p in [0, 8 XA)
    auto xat = [&](int p) { return xc[(p + 8 * XB) >> 3].at((p + 8 * XB) & 7); };
    auto gat = [&](int p) { return gc[p >> 3].at(p & 7); };
    float gp[NG];  // gpre at base + e
#pragma unroll
    for (int e = 0; e < NG; ++e) {
      float pre = b0;
#pragma unroll
      for (int j = 0; j < KP; ++j) pre = fmaf(wk[j], xat(e - KP + 1 + j), pre);
      gp[e] = (ACT == NSQ_ACT_SILU) ? gat(e) * dsilu(pre) : gat(e);
    }
    float out[kConvPer];
#pragma unroll
    for (int e = 0; e < kConvPer; ++e) {
      float a = 0.f;
#pragma unroll
      for (int sidx = 0; sidx < KP; ++sidx) a = fmaf(wr[sidx], gp[e + sidx], a);
      out[e] = a;
      gbs += gp[e];  // positions >= L have gy = 0, so gpre = 0
#pragma unroll
      for (int j = 0; j < KP; ++j) gwk[j] = fmaf(gp[e], xat(e - KP + 1 + j), gwk[j]);
    }
    const RowBuf<DT, AL> ob(gx + row * L, L);
#pragma unroll
    for (int e = 0; e < kConvPer; e += 2) ob.store_pair(base + e, make_float2(out[e], out[e + 1]));
  }
#pragma unroll
  for (int j = 0; j < KP; ++j) red[j * kConvThreads + t] = gwk[j];
  red[KP * kConvThreads + t] = gbs;
  __syncthreads();
  if (t <= KP) {
    float sacc = 0.f;
    for (int i = 0; i < kConvThreads; ++i) sacc += red[t * kConvThreads + i];
    // left-padded tap t -> weight index t - (KP - K); slot KP -> the bias
    const int nparts = int(gridDim.y);
    float* pw = part + (int64_t(c) * nparts + blockIdx.y) * (K + 1);
    if (t == KP)
      pw[K] = sacc;
    else if (t >= KP - K)
      pw[t - (KP - K)] = sacc;
  }
}

template <int DT>
static void launch_bwd_short(const void* gy, const void* x, const float* w, const float* bias, void* gx, float* gw,
                             float* gb, int act, int B, int C, int L, int K, float* ws, hipStream_t st) {
  using ET = typename Elem<DT>::T;
  const int64_t nparts = cconv_wgrad_parts(B, L);
  dim3 grid(C, unsigned(nparts));
  const bool al = L % (DT == NSQ_DTYPE_F32 ? 4 : 8) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(gy) & 15) == 0 && (reinterpret_cast<uintptr_t>(gx) & 15) == 0;
  auto go = [&](auto al_c, auto act_c) {
    constexpr bool A = decltype(al_c)::value;
    constexpr int F = decltype(act_c)::value;
    if (K <= 4)
      hipLaunchKernelGGL((cconv_bwd_short_kernel<DT, A, F, 4>), grid, dim3(kConvThreads), 0, st, (const ET*)gy,
                         (const ET*)x, w, bias, (ET*)gx, ws, B, C, L, K);
    else if (K <= 8)
      hipLaunchKernelGGL((cconv_bwd_short_kernel<DT, A, F, 8>), grid, dim3(kConvThreads), 0, st, (const ET*)gy,
                         (const ET*)x, w, bias, (ET*)gx, ws, B, C, L, K);
    else
      hipLaunchKernelGGL((cconv_bwd_short_kernel<DT, A, F, 16>), grid, dim3(kConvThreads), 0, st, (const ET*)gy,
                         (const ET*)x, w, bias, (ET*)gx, ws, B, C, L, K);
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  using SILU = std::integral_constant<int, NSQ_ACT_SILU>;
  using IDN = std::integral_constant<int, NSQ_ACT_IDENTITY>;
  if (al)
    act == NSQ_ACT_SILU ? go(T_{}, SILU{}) : go(T_{}, IDN{});
  else
    act == NSQ_ACT_SILU ? go(F_{}, SILU{}) : go(F_{}, IDN{});
  hipLaunchKernelGGL(cconv_wgrad_reduce_kernel, dim3(C), dim3(kConvThreads + 64), 0, st, (const float*)ws,
                     int(nparts), K, gw, gb);
}

template <int DT>
static void launch_fwd(const void* x, const float* w, const float* bias, void* y, int act, int B, int C, int L, int K,
                       hipStream_t st) {
  using ET = typename Elem<DT>::T;
  if (K > 16) {  // matrix cores; up to 16 taps the register kernel below is faster
    switch (mfma_steps_for(K)) {  // 17 <= K <= 256 (validated)
      case 12: return launch_fwd_mfma<DT, 12>(x, w, bias, y, act, B, C, L, K, st);
      case 20: return launch_fwd_mfma<DT, 20>(x, w, bias, y, act, B, C, L, K, st);
      case 36: return launch_fwd_mfma<DT, 36>(x, w, bias, y, act, B, C, L, K, st);
      default: return launch_fwd_mfma<DT, 68>(x, w, bias, y, act, B, C, L, K, st);
    }
  }
  dim3 grid(B * C, unsigned(ceil_div(L, kConvTile)));
  const bool al = L % (DT == NSQ_DTYPE_F32 ? 4 : 8) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(y) & 15) == 0;
  auto go = [&](auto al_c, auto act_c) {
    constexpr bool A = decltype(al_c)::value;
    constexpr int F = decltype(act_c)::value;
    if (K <= 4)
      hipLaunchKernelGGL((cconv_fwd_short_kernel<DT, A, F, 4>), grid, dim3(kConvThreads), 0, st, (const ET*)x, w,
                         bias, (ET*)y, C, L, K);
    else if (K <= 8)
      hipLaunchKernelGGL((cconv_fwd_short_kernel<DT, A, F, 8>), grid, dim3(kConvThreads), 0, st, (const ET*)x, w,
                         bias, (ET*)y, C, L, K);
    else
      hipLaunchKernelGGL((cconv_fwd_short_kernel<DT, A, F, 16>), grid, dim3(kConvThreads), 0, st, (const ET*)x, w,
                         bias, (ET*)y, C, L, K);
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  using SILU = std::integral_constant<int, NSQ_ACT_SILU>;
  using IDN = std::integral_constant<int, NSQ_ACT_IDENTITY>;
  if (al)
    act == NSQ_ACT_SILU ? go(T_{}, SILU{}) : go(T_{}, IDN{});
  else
    act == NSQ_ACT_SILU ? go(F_{}, SILU{}) : go(F_{}, IDN{});
}

template <int DT>
static void launch_bwd(const void* gy, const void* x, const float* w, const float* bias, void* gx, float* gw,
                       float* gb, int act, int B, int C, int L, int K, float* ws, hipStream_t st) {
  if (K <= 16) return launch_bwd_short<DT>(gy, x, w, bias, gx, gw, gb, act, B, C, L, K, ws, st);
  switch (mfma_steps_for(K)) {  // 17 <= K <= 256 (validated)
    case 12: return launch_bwd_mfma<DT, 12>(gy, x, w, bias, gx, gw, gb, act, B, C, L, K, ws, st);
    case 20: return launch_bwd_mfma<DT, 20>(gy, x, w, bias, gx, gw, gb, act, B, C, L, K, ws, st);
    case 36: return launch_bwd_mfma<DT, 36>(gy, x, w, bias, gx, gw, gb, act, B, C, L, K, ws, st);
    default: return launch_bwd_mfma<DT, 68>(gy, x, w, bias, gx, gw, gb, act, B, C, L, K, ws, st);
  }
}

static int validate_cconv(const void* a, const void* b, const float* w, int dtype, int act, int64_t B, int64_t C,
                          int64_t L, int64_t K) {
  NSQ_CHECK_ARG(a && b && w, "causal_conv1d: null tensor pointer");
  NSQ_CHECK_ARG(valid_dtype(dtype), "causal_conv1d: unsupported dtype code %d", dtype);
  NSQ_CHECK_ARG(act == NSQ_ACT_IDENTITY || act == NSQ_ACT_SILU, "causal_conv1d: activation code %d not in {0, 1}", act);
  NSQ_CHECK_ARG(B >= 1 && C >= 1 && L >= 1, "causal_conv1d: sizes must be positive");
  NSQ_CHECK_ARG(K >= 1 && K <= kConvMaxK, "causal_conv1d: kernel size %lld outside [1, %d]", (long long)K, kConvMaxK);
  NSQ_CHECK_ARG(B * C <= 0x7fffffff && L < (int64_t(1) << 28), "causal_conv1d: tensor too large (rows are staged through 32-bit byte offsets: L < 2^28)");
  return NSQ_OK;
}

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch[kMaxScratchDevices] = {nullptr};
}  // namespace

// Device address of the current GPU's scratch, looked up on the first call
// made with that device current and kept for later calls.  nullptr on failure
// (error recorded).
static float* noalloc_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) {
    set_error("causal_conv1d_bwd_noalloc: no current HIP device (or device index >= %d)", kMaxScratchDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("causal_conv1d_bwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch[dev] = static_cast<float*>(p);
  }
  return g_scratch[dev];
}

template <class... A>
static void launch_bwd_dtype(int dtype, A... a) {
  switch (dtype) {
    case NSQ_DTYPE_F32: launch_bwd<NSQ_DTYPE_F32>(a...); break;
    case NSQ_DTYPE_BF16: launch_bwd<NSQ_DTYPE_BF16>(a...); break;
    default: launch_bwd<NSQ_DTYPE_F16>(a...); break;
  }
}

}  // namespace nsq

using namespace nsq;

extern "C" {

size_t nsq_causal_conv1d_bwd_workspace_bytes(int64_t B, int64_t C, int64_t L, int64_t K, int activation) {
  // K <= 16 (one fused pass): the weight / bias gradient partials
  // [C][parts][K + 1] only; otherwise (matrix cores) silu: gy * silu'(pre)
  // [B, C, L], then the partials
  if (K >= 1 && K <= 16) return size_t(C * cconv_wgrad_parts(B, L) * (K + 1)) * sizeof(float);
  const int64_t pre = activation == NSQ_ACT_SILU ? B * C * L : 0;
  const int64_t parts = K <= kConvMaxK ? C * cconv_wgrad_parts(B, L) * (K + 1) : 0;
  return size_t(pre + parts) * sizeof(float);
}

int nsq_causal_conv1d_fwd(const void* x, const float* weight, const float* bias, void* y, int dtype, int activation,
                          int64_t B, int64_t C, int64_t L, int64_t K, void* stream) {
  clear_error();
  int rc = validate_cconv(x, y, weight, dtype, activation, B, C, L, K);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case NSQ_DTYPE_F32: launch_fwd<NSQ_DTYPE_F32>(x, weight, bias, y, activation, int(B), int(C), int(L), int(K), st); break;
    case NSQ_DTYPE_BF16: launch_fwd<NSQ_DTYPE_BF16>(x, weight, bias, y, activation, int(B), int(C), int(L), int(K), st); break;
    default: launch_fwd<NSQ_DTYPE_F16>(x, weight, bias, y, activation, int(B), int(C), int(L), int(K), st); break;
  }
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

int nsq_causal_conv1d_bwd(const void* gy, const void* x, const float* weight, const float* bias, void* gx,
                          float* gweight, float* gbias, int dtype, int activation, int64_t B, int64_t C, int64_t L,
                          int64_t K, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = validate_cconv(gy, x, weight, dtype, activation, B, C, L, K);
  if (rc) return rc;
  NSQ_CHECK_ARG(gx && gweight, "causal_conv1d_bwd: null gradient output pointer");
  const size_t need = nsq_causal_conv1d_bwd_workspace_bytes(B, C, L, K, activation);
  NSQ_CHECK_ARG(need == 0 || (workspace && workspace_bytes >= need),
                "causal_conv1d_bwd: workspace of %zu bytes required, got %zu", need, workspace_bytes);
  launch_bwd_dtype(dtype, gy, x, weight, bias, gx, gweight, gbias, activation, int(B), int(C), int(L), int(K),
                   (float*)workspace, (hipStream_t)stream);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

// The scratch regions the backward uses (partials, the silu pre-activation
// gradient) are written in full by one kernel before the next reads them, so
// the buffer needs no clearing between calls.
int nsq_causal_conv1d_bwd_noalloc(const void* gy, const void* x, const float* weight, const float* bias, void* gx,
                                  float* gweight, float* gbias, int dtype, int activation, int64_t B, int64_t C,
                                  int64_t L, int64_t K, void* stream) {
  clear_error();
  int rc = validate_cconv(gy, x, weight, dtype, activation, B, C, L, K);
  if (rc) return rc;
  NSQ_CHECK_ARG(gx && gweight, "causal_conv1d_bwd_noalloc: null gradient output pointer");
  const size_t need = nsq_causal_conv1d_bwd_workspace_bytes(B, C, L, K, activation);
  if (need > kNoAllocScratchBytes) {
    set_error("causal_conv1d_bwd_noalloc: B=%lld C=%lld L=%lld K=%lld needs %zu bytes of scratch, more than the "
              "fixed %zu-byte device buffer; call nsq_causal_conv1d_bwd with a workspace instead",
              (long long)B, (long long)C, (long long)L, (long long)K, need, kNoAllocScratchBytes);
    return NSQ_ERR_UNSUPPORTED;
  }
  float* ws = nullptr;
  if (need) {
    ws = noalloc_scratch();
    if (!ws) return NSQ_ERR_HIP;
  }
  launch_bwd_dtype(dtype, gy, x, weight, bias, gx, gweight, gbias, activation, int(B), int(C), int(L), int(K), ws,
                   (hipStream_t)stream);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

}  // extern "C"
