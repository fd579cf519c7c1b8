// Back-to-back striped-Hyena short-conv block, forward and backward (gfx950).
//
// Replaces subquadratic_ops_torch.b2b_causal_conv1d bound at
// nvsubquadratic/ops/causal_conv1d_custom.py:101-121 ("projection conv,
// pre-gate, mixer conv with skip, post-gate").  The reference does not state
// the exact algorithm (its only test checks shape and finiteness,
// tests/ops/test_causal_conv1d_custom.py:112-133), so this build fixes it as
// follows, in fp32 throughout with one rounding of the output:
//   p   = causal_conv(x; w_proj)   on all 3C channels (nn.Conv1d tap order)
//   q, k, v = p[:, 0:C], p[:, C:2C], p[:, 2C:3C]
//   z   = k * v                                   (pre-gate)
//   h   = causal_conv(z; w_mixer) + skip * z      (mixer conv with skip)
//   out = q * h                                   (post-gate)
// The forward is one pass over HBM: 3 input rows read, 1 output row written.
#include <cstdlib>
#include <type_traits>

#include "direct_conv.h"

namespace nsq {

// Dynamic LDS layout of b2b_fwd_kernel / b2b_bwd1_kernel, sized by the actual
// tap counts (a static layout for 256 taps would cost a workgroup per CU).
// Float offsets, each a multiple of 8 so the sliding-window reads stay aligned.
struct B2BLds {
  int q, k, v, z, wq, wk, wv, wm, total;
  __host__ __device__ static int up8(int n) { return (n + 7) & ~7; }
  __host__ __device__ B2BLds(int Kp, int Km) {
    const int hp = Kp - 1, hz = Km - 1;
    q = 0;
    k = q + up8(kConvTile + hp + 2 * kConvPer);
    v = k + up8(kConvTile + hz + hp + 2 * kConvPer);
    z = v + up8(kConvTile + hz + hp + 2 * kConvPer);
    wq = z + up8(kConvTile + hz + 2 * kConvPer);
    wk = wq + up8(Kp);
    wv = wk + up8(Kp);
    wm = wv + up8(Kp);
    total = wm + up8(Km);
  }
};

// grid = (B*C, ceil(L / kConvTile)).  xs_*: staged input rows; zs: z with the
// mixer halo.
template <int DT>
__global__ __launch_bounds__(kConvThreads) void b2b_fwd_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                                const float* __restrict__ wp,
                                                                const float* __restrict__ wm,
                                                                const float* __restrict__ skip,
                                                                typename Elem<DT>::T* __restrict__ y, int C, int L,
                                                                int Kp, int Km) {
  constexpr int TF = conv_tile_floats(2 * kConvMaxK);
  extern __shared__ __align__(16) float smem[];
  const B2BLds lay(Kp, Km);
  float* xs_q = smem + lay.q;
  float* xs_k = smem + lay.k;
  float* xs_v = smem + lay.v;
  float* zs = smem + lay.z;
  float* wlq = smem + lay.wq;
  float* wlk = smem + lay.wk;
  float* wlv = smem + lay.wv;
  float* wlm = smem + lay.wm;
  const int64_t row = blockIdx.x;  // b*C + c
  const int b = int(row / C), c = int(row % C);
  const int64_t n0 = int64_t(blockIdx.y) * kConvTile;
  const int64_t xq = (int64_t(b) * 3 * C + c) * L;
  const int64_t xk = xq + int64_t(C) * L;
  const int64_t xv = xk + int64_t(C) * L;
  const int hz = Km - 1, hp = Kp - 1;
  // q needs [n0 - hp, n0 + tile); k, v need [n0 - hz - hp, n0 + tile).
  stage_weights<false>(wlq, wp + int64_t(c) * Kp, Kp);
  stage_weights<false>(wlk, wp + int64_t(C + c) * Kp, Kp);
  stage_weights<false>(wlv, wp + int64_t(2 * C + c) * Kp, Kp);
  stage_weights<false>(wlm, wm + int64_t(c) * Km, Km);
  {
    // all three rows' loads in flight together, then the LDS stores
    RowStage<DT, conv_tile_floats(kConvMaxK)> sq;
    RowStage<DT, TF> sk, sv;
    sq.load(x + xq, n0 - hp, kConvTile + hp + 2 * kConvPer, L);
    sk.load(x + xk, n0 - hz - hp, kConvTile + hz + hp + 2 * kConvPer, L);
    sv.load(x + xv, n0 - hz - hp, kConvTile + hz + hp + 2 * kConvPer, L);
    sq.store(xs_q, kConvTile + hp + 2 * kConvPer);
    sk.store(xs_k, kConvTile + hz + hp + 2 * kConvPer);
    sv.store(xs_v, kConvTile + hz + hp + 2 * kConvPer);
    __syncthreads();
  }
  // z[n] for n in [n0 - hz, n0 + tile): zs[i] = z[n0 - hz + i]; z of positions
  // before the sequence start is 0 (the mixer conv's causal padding).
  const int zcount = kConvTile + hz + 2 * kConvPer;
  for (int i = threadIdx.x; i < zcount; i += kConvThreads) {
    const int64_t n = n0 - hz + i;
    float kk = 0.f, vv = 0.f;
    if (n >= 0 && n < L) {
      for (int j = 0; j < Kp; ++j) {
        kk = fmaf(wlk[j], xs_k[i + j], kk);
        vv = fmaf(wlv[j], xs_v[i + j], vv);
      }
    }
    zs[i] = kk * vv;
  }
  __syncthreads();
  const int base = threadIdx.x * kConvPer;
  float qa[kConvPer], ha[kConvPer];
#pragma unroll
  for (int e = 0; e < kConvPer; ++e) qa[e] = ha[e] = 0.f;
  slide_fma(qa, xs_q, base, Kp, wlq);
  slide_fma(ha, zs, base, Km, wlm);
  const float sk = skip ? skip[c] : 0.f;
  typename Elem<DT>::T* yr = y + row * L;
#pragma unroll
  for (int e = 0; e < kConvPer; e += 2) {
    const int64_t n = n0 + base + e;
    if (n < L) {
      const float h0 = fmaf(sk, zs[base + e + hz], ha[e]);
      const float h1 = fmaf(sk, zs[base + e + 1 + hz], ha[e + 1]);
      store_pair<DT>(yr, n, L, make_float2(qa[e] * h0, qa[e + 1] * h1));
    }
  }
}

// The same forward with the mixer conv on the matrix cores (ToeplitzMfma, NS
// steps, Km <= 4*NS - 15).  A workgroup walks a segment of up to kB2BSegTiles
// consecutive tiles of one (b, c) row, so the mixer's weight band is built
// once per segment and z is computed once per position: the Km - 1 values of
// z before a tile are the last ones of the previous tile (the first tile of a
// segment computes them from its staged halo).  Per tile, with a barrier
// after each phase:
//   1. the staged rows (registers, loaded during the previous tile) go to LDS,
//      and the next tile's loads are issued;
//   2. z = k*v for the tile's 2048 positions into the window buffer (split
//      layout; zero at positions >= L), q into qs;
//   3. MFMA: two interleaved 16-block M-tiles per wave; out = q*(y + skip*z)
//      into qs;
//   4. row stores; the last Km - 1 z values move to the window's front.
constexpr int kB2BSegTiles = 4;

template <int NS>
struct B2BMfmaLds {
  int q, k, v, qs, z, wq, wk, wv, wm, total, hk;
  __host__ __device__ static int up8(int n) { return (n + 7) & ~7; }
  __host__ __device__ B2BMfmaLds(int Kp, int Km) {
    const int hp = Kp - 1, hz = Km - 1;
    hk = hp + up8(hz);  // k, v rows are staged from n0 - hk (aligned window bases)
    q = 0;
    qs = 0;  // q values (qs_pad layout) replace the staged q row once it is consumed
    const int qwords = kConvTile + kConvTile / 4 > kConvTile + hp + 2 * kConvPer ? kConvTile + kConvTile / 4
                                                                                   : kConvTile + hp + 2 * kConvPer;
    k = up8(qwords);
    v = k + up8(kConvTile + hk + 2 * kConvPer);
    z = v + up8(kConvTile + hk + 2 * kConvPer);
    wq = z + win_words(mfma_src_count<NS>());
    wk = wq + up8(Kp);
    wv = wk + up8(Kp);
    wm = wv + up8(Kp);
    total = wm + up8(Km);
  }
};

// Output-tile slot of position p (kConvTile + kConvTile / 4 words per tile):
// runs of 8 from a multiple of 8 stay contiguous; 4 words of pad per 32 put
// the 16-byte writes of 8 consecutive lanes (stride 8) on distinct banks, and
// a further 8 per 64 puts the 4-byte epilogue reads of two lane groups 64
// positions apart on opposite 16-bank halves.
__device__ __forceinline__ int qs_pad(int p) { return p + 4 * (p >> 5) + 8 * (p >> 6); }
// qs_pad(p0 + 16 r) - qs_pad(p0) for p0 % 64 < 16, r < 4 (an MFMA lane's epilogue
// positions: the lane's base slot plus a constant).
__device__ __forceinline__ constexpr int qs_step(int r) { return 16 * r + 4 * (r >> 1); }

// acc[e] += sum_{j<4} wl[j] xs[base + e + j] (taps >= K are zero in wl).
__device__ __forceinline__ void slide_fma4(float (&acc)[kConvPer], const float* xs, int base, const float* wl) {
  const float4 a = *reinterpret_cast<const float4*>(xs + base);
  const float4 b = *reinterpret_cast<const float4*>(xs + base + 4);
  const float4 c = *reinterpret_cast<const float4*>(xs + base + 8);
  const float4 w = *reinterpret_cast<const float4*>(wl);
  const float win[12] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w};
  const float ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
    for (int e = 0; e < kConvPer; ++e) acc[e] = fmaf(ww[jj], win[e + jj], acc[e]);
  }
}

template <bool SHORT>
__device__ __forceinline__ void slide_proj(float (&acc)[kConvPer], const float* xs, int base, int K, const float* wl) {
  if constexpr (SHORT) {
    slide_fma4(acc, xs, base, wl);
  } else {
    slide_fma(acc, xs, base, K, wl);
  }
}

// SHORT: projection taps Kp <= 4.
// Staged words of the k, v rows: the tile, the mixer halo (aligned) and the
// projection halo, plus the window read-ahead.
template <int NS, bool SHORT>
constexpr int b2b_kv_stage_words() {
  return kConvTile + (SHORT ? 3 : kConvMaxK - 1) + ((4 * NS - 16 + 7) & ~7) + 2 * kConvPer;
}

// PF: the next tile's rows are loaded into registers during the current tile
// (fewer waves fit); without it each tile loads at its start and the other
// resident workgroups cover the latency.
template <int DT, int NS, bool SHORT, bool PF>
__global__ __launch_bounds__(kConvThreads) __attribute__((amdgpu_waves_per_eu(PF ? 3 : 4))) void b2b_fwd_mfma_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                                     const float* __restrict__ wp,
                                                                     const float* __restrict__ wm,
                                                                     const float* __restrict__ skip,
                                                                     typename Elem<DT>::T* __restrict__ y, int C, int L,
                                                                     int Kp, int Km) {
  constexpr int TF = b2b_kv_stage_words<NS, SHORT>();
  extern __shared__ __align__(16) float smem[];
  const B2BMfmaLds<NS> lay(Kp, Km);
  float* xs_q = smem + lay.q;
  float* xs_k = smem + lay.k;
  float* xs_v = smem + lay.v;
  float* qs = smem + lay.qs;
  float* zp = smem + lay.z;
  float* wlq = smem + lay.wq;
  float* wlk = smem + lay.wk;
  float* wlv = smem + lay.wv;
  float* wlm = smem + lay.wm;
  const int64_t row = blockIdx.x;  // b*C + c
  const int b = int(row / C), c = int(row % C);
  const int ntiles = (L + kConvTile - 1) / kConvTile;
  const int t_begin = int(blockIdx.y) * kB2BSegTiles;
  const int t_end = min(ntiles, t_begin + kB2BSegTiles);
  const typename Elem<DT>::T* xq = x + (int64_t(b) * 3 * C + c) * L;
  const typename Elem<DT>::T* xk = xq + int64_t(C) * L;
  const typename Elem<DT>::T* xv = xk + int64_t(C) * L;
  // the band gets d leading zero taps so that the z halo hz = Km - 1 + d is a
  // multiple of 4: a thread's 8 z values are two aligned 16-byte writes
  const int d = ((Km - 1 + 3) & ~3) + 1 - Km;
  const int hz = Km - 1 + d, hp = Kp - 1, hk = lay.hk;
  const int t = int(threadIdx.x);
  stage_weights<false>(wlq, wp + int64_t(c) * Kp, Kp);
  stage_weights<false>(wlk, wp + int64_t(C + c) * Kp, Kp);
  stage_weights<false>(wlv, wp + int64_t(2 * C + c) * Kp, Kp);
  stage_weights<false>(wlm, wm + int64_t(c) * Km, Km);
  // the window's tail beyond the tile's last use meets zero taps: keep it finite
  constexpr int ZW = mfma_src_count<NS>();
  constexpr int ZR = win_half(ZW);
  for (int m = kConvTile + t; m < ZW; m += kConvThreads) zp[win_at(m, ZR)] = 0.f;
  RowStage<DT, kConvTile + (SHORT ? 3 : kConvMaxK - 1) + 2 * kConvPer> sq;
  RowStage<DT, TF> sk, sv;
  if constexpr (PF) {
    const int64_t n0 = int64_t(t_begin) * kConvTile;
    sq.load(xq, n0 - hp, 0, L);
    sk.load(xk, n0 - hk, 0, L);
    sv.load(xv, n0 - hk, 0, L);
  }
  __syncthreads();  // weights staged
  ToeplitzMfma<NS> tm;
  tm.load_weights(wlm, Km, skip ? skip[c] : 0.f, d);  // h = conv(z) + skip*z: skip joins the last tap
  const RowBuf<DT, false> yb(y + row * L, L);
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
  const int base = t * kConvPer;
  for (int ti = t_begin; ti < t_end; ++ti) {
    const int64_t n0 = int64_t(ti) * kConvTile;
    // 1. staged rows to LDS, next tile's loads in flight
    if constexpr (!PF) {
      sq.load(xq, n0 - hp, 0, L);
      sk.load(xk, n0 - hk, 0, L);
      sv.load(xv, n0 - hk, 0, L);
    }
    sq.store(xs_q, kConvTile + hp + 2 * kConvPer);
    sk.store(xs_k, kConvTile + hk + 2 * kConvPer);
    sv.store(xs_v, kConvTile + hk + 2 * kConvPer);
    __syncthreads();
    if (PF && ti + 1 < t_end) {
      sq.load(xq, n0 + kConvTile - hp, 0, L);
      sk.load(xk, n0 + kConvTile - hk, 0, L);
      sv.load(xv, n0 + kConvTile - hk, 0, L);
    }
    // 2. z at n0 + base + e -> window word hz + base + e; q -> qs
    {
      float ka[kConvPer], va[kConvPer], qa[kConvPer];
#pragma unroll
      for (int e = 0; e < kConvPer; ++e) ka[e] = va[e] = qa[e] = 0.f;
      const int bz = hk - hp + base;  // xs_k[bz + e + j] = x_k[n0 + base + e - hp + j]
      slide_proj<SHORT>(ka, xs_k, bz, Kp, wlk);
      slide_proj<SHORT>(va, xs_v, bz, Kp, wlv);
      slide_proj<SHORT>(qa, xs_q, base, Kp, wlq);
#pragma unroll
      for (int e = 0; e < kConvPer; ++e) ka[e] = (n0 + base + e < L) ? ka[e] * va[e] : 0.f;
      win_store8(zp, ZR, hz + base, ka);
      if (ti == t_begin) {
        // z at n0 - hz + m (m < hz): the causal zero padding before the row
        // start, else recomputed from the staged halo
        for (int m = t; m < hz; m += kConvThreads) {
          const int64_t n = n0 - hz + m;
          float kv = 0.f, vv = 0.f;
          if (n >= 0) {
            const int i0 = hk - hp - hz + m;  // xs_k[i0 + j] = x_k[n - hp + j]
            for (int j = 0; j < Kp; ++j) {
              kv = fmaf(wlk[j], xs_k[i0 + j], kv);
              vv = fmaf(wlv[j], xs_v[i0 + j], vv);
            }
          }
          zp[win_at(m, ZR)] = kv * vv;
        }
      }
      __syncthreads();  // the q stage is consumed: q takes its place
      float* qd = qs + qs_pad(base);
      *reinterpret_cast<float4*>(qd) = make_float4(qa[0], qa[1], qa[2], qa[3]);
      *reinterpret_cast<float4*>(qd + 4) = make_float4(qa[4], qa[5], qa[6], qa[7]);
    }
    __syncthreads();
    // 3. MFMA tiles (wave w: M-tiles w and w + 4); out = q * h stored from the
    //    accumulator layout (16 consecutive outputs per lane group; the row
    //    buffer's range check drops positions >= L)
    {
      static_assert(kMfmaTiles == 2 * kConvWaves, "b2b MFMA: two M-tiles per wave");
      nsq_f32x4_t acc0, acc1;
      tm.run2(zp, ZR, 16 * wave, 16 * (wave + kConvWaves), acc0, acc1);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int mt = wave + h * kConvWaves;
        const float* ql = qs + qs_pad(16 * (16 * mt + 4 * (l >> 4)) + (l & 15));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int p = 16 * (16 * mt + 4 * (l >> 4) + r) + (l & 15);
          const float hv = h ? acc1[r] : acc0[r];
          yb.store_elem(n0 + p, ql[qs_step(r)] * hv);
        }
      }
    }
    __syncthreads();
    // 4. z of the next tile's halo to the window front (ordered before the
    //    next tile's reads by its first barrier)
    for (int m = t; m < hz; m += kConvThreads) zp[win_at(m, ZR)] = zp[win_at(kConvTile + m, ZR)];
  }
}

// Projection taps left-padded to 4: w4[j] = w[j - (4 - Kp)].
__device__ __forceinline__ void load_taps4(float (&w4)[4], const float* __restrict__ w, int Kp) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int s = j - (4 - Kp);
    w4[j] = s >= 0 ? w[s >= 0 ? s : 0] : 0.f;
  }
}

// ---------------------------------------------------------------------------
// Backward with the mixer on the matrix cores (Km >= 16), three kernels:
//  bwd1 (row walker like the forward): z into the window, q; h = conv(z) +
//       skip*z on the MFMA band; gq = g*h -> gp (q rows), gh = g*q -> gh
//       workspace; and the mixer weight gradient of each tile as an MFMA
//       product over the same windows,
//         D[i][t] += sum_a gh[16a + i] * zwin[16a + t],  gw[j] = sum_i D[i][i + j]
//       (zwin[m] = z[n0 - hz + m]; t = i + j + d < 4 NS, d the band's leading
//       zero taps), kept in registers over
//       the workgroup's tiles and reduced in a fixed order (waves, then the
//       diagonal) into a per-workgroup partial;
//  bwd2: gz = corr(gh; w_mixer) + skip*gh on the reversed band over a forward
//       window of gh; k, v recomputed; gk = gz*v, gv = gz*k -> gp (k, v rows);
//  reduce: the partials of a channel summed in a fixed order -> gw_mixer, and
//       its lag Km-1 -> gskip.
// ---------------------------------------------------------------------------
template <int NS>
struct B2BBwd1Lds {
  B2BMfmaLds<NS> f;
  int gh, total;
  __host__ __device__ B2BBwd1Lds(int Kp, int Km) : f(Kp, Km) {
    gh = f.total;  // gh of the tile, qs_pad layout
    total = gh + kConvTile + kConvTile / 4;
    const int red = 16 * 4 * NS;  // end-of-segment reduction (aliases the start)
    if (total < red) total = red;
  }
};

template <int DT, int NS, bool SHORT>
__global__ __launch_bounds__(kConvThreads) __attribute__((amdgpu_waves_per_eu(2))) void b2b_bwd1_mfma_kernel(
    const typename Elem<DT>::T* __restrict__ g, const typename Elem<DT>::T* __restrict__ x, const float* __restrict__ wp,
    const float* __restrict__ wm, const float* __restrict__ skip, float* __restrict__ gp, float* __restrict__ ghw,
    float* __restrict__ gw_part, int B, int C, int L, int Kp, int Km) {
  constexpr int TF = b2b_kv_stage_words<NS, SHORT>();
  constexpr int TG = NS / 4;  // 16-column groups of the window
  extern __shared__ __align__(16) float smem[];
  const B2BBwd1Lds<NS> lay(Kp, Km);
  float* xs_q = smem + lay.f.q;
  float* xs_k = smem + lay.f.k;
  float* xs_v = smem + lay.f.v;
  float* qs = smem + lay.f.qs;
  float* zp = smem + lay.f.z;
  float* wlq = smem + lay.f.wq;
  float* wlk = smem + lay.f.wk;
  float* wlv = smem + lay.f.wv;
  float* wlm = smem + lay.f.wm;
  float* ghs = smem + lay.gh;
  const int64_t row = blockIdx.x;  // b*C + c
  const int b = int(row / C), c = int(row % C);
  const int ntiles = (L + kConvTile - 1) / kConvTile;
  const int t_begin = int(blockIdx.y) * kB2BSegTiles;
  const int t_end = min(ntiles, t_begin + kB2BSegTiles);
  const typename Elem<DT>::T* xq = x + (int64_t(b) * 3 * C + c) * L;
  const typename Elem<DT>::T* xk = xq + int64_t(C) * L;
  const typename Elem<DT>::T* xv = xk + int64_t(C) * L;
  // d leading zero taps: the z halo hz = Km - 1 + d is a multiple of 4 (as in the forward)
  const int d = ((Km - 1 + 3) & ~3) + 1 - Km;
  const int hz = Km - 1 + d, hp = Kp - 1, hk = lay.f.hk;
  const int t = int(threadIdx.x);
  stage_weights<false>(wlq, wp + int64_t(c) * Kp, Kp);
  stage_weights<false>(wlk, wp + int64_t(C + c) * Kp, Kp);
  stage_weights<false>(wlv, wp + int64_t(2 * C + c) * Kp, Kp);
  stage_weights<false>(wlm, wm + int64_t(c) * Km, Km);
  constexpr int ZW = mfma_src_count<NS>();
  constexpr int ZR = win_half(ZW);
  for (int m = kConvTile + t; m < ZW; m += kConvThreads) zp[win_at(m, ZR)] = 0.f;
  RowStage<DT, kConvTile + (SHORT ? 3 : kConvMaxK - 1) + 2 * kConvPer> sq;
  RowStage<DT, TF> sk, sv;
  {
    const int64_t n0 = int64_t(t_begin) * kConvTile;
    sq.load(xq, n0 - hp, 0, L);
    sk.load(xk, n0 - hk, 0, L);
    sv.load(xv, n0 - hk, 0, L);
  }
  __syncthreads();  // weights staged
  ToeplitzMfma<NS> tm;
  tm.load_weights(wlm, Km, skip ? skip[c] : 0.f, d);  // h = conv(z) + skip*z
  const RowBuf<DT, false> gb(g + row * L, L);
  const RowBuf<NSQ_DTYPE_F32, false> gqb(gp + (int64_t(b) * 3 * C + c) * L, L);
  const RowBuf<NSQ_DTYPE_F32, false> ghb(ghw + row * L, L);
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
  const int kk = l >> 4, li = l & 15;
  const int base = t * kConvPer;
  nsq_f32x4_t D[TG];
#pragma unroll
  for (int tg = 0; tg < TG; ++tg) D[tg] = nsq_f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int ti = t_begin; ti < t_end; ++ti) {
    const int64_t n0 = int64_t(ti) * kConvTile;
    // 1. staged rows to LDS, next tile's loads in flight
    sq.store(xs_q, kConvTile + hp + 2 * kConvPer);
    sk.store(xs_k, kConvTile + hk + 2 * kConvPer);
    sv.store(xs_v, kConvTile + hk + 2 * kConvPer);
    __syncthreads();
    if (ti + 1 < t_end) {
      sq.load(xq, n0 + kConvTile - hp, 0, L);
      sk.load(xk, n0 + kConvTile - hk, 0, L);
      sv.load(xv, n0 + kConvTile - hk, 0, L);
    }
    // 2. z and q as in the forward
    {
      float ka[kConvPer], va[kConvPer], qa[kConvPer];
#pragma unroll
      for (int e = 0; e < kConvPer; ++e) ka[e] = va[e] = qa[e] = 0.f;
      const int bz = hk - hp + base;
      slide_proj<SHORT>(ka, xs_k, bz, Kp, wlk);
      slide_proj<SHORT>(va, xs_v, bz, Kp, wlv);
      slide_proj<SHORT>(qa, xs_q, base, Kp, wlq);
#pragma unroll
      for (int e = 0; e < kConvPer; ++e) ka[e] = (n0 + base + e < L) ? ka[e] * va[e] : 0.f;
      win_store8(zp, ZR, hz + base, ka);
      if (ti == t_begin) {
        for (int m = t; m < hz; m += kConvThreads) {
          const int64_t n = n0 - hz + m;
          float kv = 0.f, vv = 0.f;
          if (n >= 0) {
            const int i0 = hk - hp - hz + m;
            for (int j = 0; j < Kp; ++j) {
              kv = fmaf(wlk[j], xs_k[i0 + j], kv);
              vv = fmaf(wlv[j], xs_v[i0 + j], vv);
            }
          }
          zp[win_at(m, ZR)] = kv * vv;
        }
      }
      __syncthreads();  // the q stage is consumed: q takes its place
      float* qd = qs + qs_pad(base);
      *reinterpret_cast<float4*>(qd) = make_float4(qa[0], qa[1], qa[2], qa[3]);
      *reinterpret_cast<float4*>(qd + 4) = make_float4(qa[4], qa[5], qa[6], qa[7]);
    }
    __syncthreads();
    // 3. h on the MFMA band; gq = g*h, gh = g*q (positions >= L: g reads 0)
    {
      nsq_f32x4_t acc0, acc1;
      tm.run2(zp, ZR, 16 * wave, 16 * (wave + kConvWaves), acc0, acc1);
      float gv[8];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int p = 16 * (16 * (wave + h * kConvWaves) + 4 * kk + r) + li;
          gv[4 * h + r] = gb.elem(n0 + p);
        }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int ql = qs_pad(16 * (16 * (wave + h * kConvWaves) + 4 * kk) + li);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int p = 16 * (16 * (wave + h * kConvWaves) + 4 * kk + r) + li;
          const float hv = h ? acc1[r] : acc0[r];
          const float ghv = gv[4 * h + r] * qs[ql + qs_step(r)];
          gqb.store_elem(n0 + p, gv[4 * h + r] * hv);
          ghb.store_elem(n0 + p, ghv);
          ghs[ql + qs_step(r)] = ghv;
        }
      }
    }
    __syncthreads();
    // 4. mixer weight gradient of the tile: wave w takes blocks [32w, 32w + 32)
    //    (qs_pad(16 (a0 + kk) + li) = 20 a0 + 16 kk + 4 (kk / 2) + li for a0 % 4 == 0)
    //    (win_at(16 (a0 + kk + tg) + li) = win_at(16 kk + li) + 8 (a0 + tg))
    const float* ghl = ghs + 16 * kk + 4 * (kk >> 1) + li;
    const float* zl = zp + win_at(16 * kk + li, ZR);
#pragma unroll 2
    for (int a0 = 32 * wave; a0 < 32 * wave + 32; a0 += 4) {
      const float av = ghl[20 * a0];
#pragma unroll
      for (int tg = 0; tg < TG; ++tg) {
        const float bv = zl[8 * (a0 + tg)];
        D[tg] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, D[tg], 0, 0, 0);
      }
    }
    __syncthreads();
    // 5. z of the next tile's halo to the window front
    for (int m = t; m < hz; m += kConvThreads) zp[win_at(m, ZR)] = zp[win_at(kConvTile + m, ZR)];
  }
  // Fixed-order reduction: D of waves 0..3 summed into red[i][t], then
  // gw[j] = sum_i red[i][i + j].
  __syncthreads();
  float* red = smem;
  constexpr int RW = 4 * NS;
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
  if (t < Km) {
    float sacc = 0.f;
    for (int i = 0; i < 16; ++i) sacc += red[i * RW + i + t + d];
    const int nparts = B * int(gridDim.y);
    const int part = b * int(gridDim.y) + int(blockIdx.y);
    gw_part[(int64_t(c) * nparts + part) * Km + t] = sacc;
  }
}

template <int DT, int NS, bool SHORT>
struct B2BBwd2Lds {
  static constexpr int GR = win_half(mfma_src_count<NS>());
  static constexpr int GWORDS = win_words(mfma_src_count<NS>());
  int gw, k, v, ks, vs, wk, wv, wr, total;
  __host__ __device__ static int up8(int n) { return (n + 7) & ~7; }
  __host__ __device__ B2BBwd2Lds(int Kp, int Km) {
    const int hp = Kp - 1;
    gw = 0;
    k = GWORDS;
    v = k + up8(kConvTile + hp + 2 * kConvPer);
    ks = v + up8(kConvTile + hp + 2 * kConvPer);
    vs = ks + kConvTile + kConvTile / 4;
    wk = vs + kConvTile + kConvTile / 4;
    wv = wk + up8(Kp);
    wr = wv + up8(Kp);
    total = wr + up8(Km);
  }
};

template <int DT, int NS, bool SHORT>
__global__ __launch_bounds__(kConvThreads) __attribute__((amdgpu_waves_per_eu(3))) void b2b_bwd2_mfma_kernel(
    const typename Elem<DT>::T* __restrict__ x, const float* __restrict__ wp, const float* __restrict__ wm,
    const float* __restrict__ skip, const float* __restrict__ ghw, float* __restrict__ gp, int C, int L, int Kp,
    int Km) {
  constexpr int ZW = mfma_src_count<NS>();
  constexpr int GR = B2BBwd2Lds<DT, NS, SHORT>::GR;
  constexpr int GIT = (ZW + kConvThreads - 1) / kConvThreads;
  extern __shared__ __align__(16) float smem[];
  const B2BBwd2Lds<DT, NS, SHORT> lay(Kp, Km);
  float* gwin = smem + lay.gw;
  float* xs_k = smem + lay.k;
  float* xs_v = smem + lay.v;
  float* ks = smem + lay.ks;
  float* vs = smem + lay.vs;
  float* wlk = smem + lay.wk;
  float* wlv = smem + lay.wv;
  float* wlr = smem + lay.wr;
  const int64_t row = blockIdx.x;  // b*C + c
  const int b = int(row / C), c = int(row % C);
  const int ntiles = (L + kConvTile - 1) / kConvTile;
  const int t_begin = int(blockIdx.y) * kB2BSegTiles;
  const int t_end = min(ntiles, t_begin + kB2BSegTiles);
  const typename Elem<DT>::T* xk = x + (int64_t(b) * 3 * C + C + c) * L;
  const typename Elem<DT>::T* xv = xk + int64_t(C) * L;
  const float* ghr = ghw + row * L;
  const int hp = Kp - 1;
  const int t = int(threadIdx.x);
  stage_weights<false>(wlk, wp + int64_t(C + c) * Kp, Kp);
  stage_weights<false>(wlv, wp + int64_t(2 * C + c) * Kp, Kp);
  stage_weights<true>(wlr, wm + int64_t(c) * Km, Km);  // wlr[j] = w[Km-1-j]: gz[n] = sum_j wlr[j] gh[n + j]
  RowStage<DT, kConvTile + (SHORT ? 3 : kConvMaxK - 1) + 2 * kConvPer> sk, sv;
  float gstage[GIT];
  auto load_tile = [&](int64_t n0) {
    sk.load(xk, n0 - hp, 0, L);
    sv.load(xv, n0 - hp, 0, L);
    const RowBuf<NSQ_DTYPE_F32, false> rb(ghr, L);
#pragma unroll
    for (int it = 0; it < GIT; ++it) gstage[it] = rb.elem(n0 + t + it * kConvThreads);  // n0 >= 0
  };
  load_tile(int64_t(t_begin) * kConvTile);
  __syncthreads();  // weights staged
  ToeplitzMfma<NS> tm;
  tm.load_weights(wlr, Km, 0.f, 0, skip ? skip[c] : 0.f);  // + skip*gh[n]: tap 0
  const RowBuf<NSQ_DTYPE_F32, false> gkb(gp + (int64_t(b) * 3 * C + C + c) * L, L);
  const RowBuf<NSQ_DTYPE_F32, false> gvb(gp + (int64_t(b) * 3 * C + 2 * C + c) * L, L);
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
  const int kk = l >> 4, li = l & 15;
  const int base = t * kConvPer;
  for (int ti = t_begin; ti < t_end; ++ti) {
    const int64_t n0 = int64_t(ti) * kConvTile;
    // 1. staged rows to LDS (gh window: word m = gh[n0 + m], m < ZW)
    sk.store(xs_k, kConvTile + hp + 2 * kConvPer);
    sv.store(xs_v, kConvTile + hp + 2 * kConvPer);
#pragma unroll
    for (int it = 0; it < GIT; ++it) {
      const int m = t + it * kConvThreads;
      if (m < ZW) gwin[win_at(m, GR)] = gstage[it];
    }
    __syncthreads();
    if (ti + 1 < t_end) load_tile(n0 + kConvTile);
    // 2. k, v of the tile
    {
      float ka[kConvPer], va[kConvPer];
#pragma unroll
      for (int e = 0; e < kConvPer; ++e) ka[e] = va[e] = 0.f;
      slide_proj<SHORT>(ka, xs_k, base, Kp, wlk);
      slide_proj<SHORT>(va, xs_v, base, Kp, wlv);
      float* kd = ks + qs_pad(base);
      float* vd = vs + qs_pad(base);
      *reinterpret_cast<float4*>(kd) = make_float4(ka[0], ka[1], ka[2], ka[3]);
      *reinterpret_cast<float4*>(kd + 4) = make_float4(ka[4], ka[5], ka[6], ka[7]);
      *reinterpret_cast<float4*>(vd) = make_float4(va[0], va[1], va[2], va[3]);
      *reinterpret_cast<float4*>(vd + 4) = make_float4(va[4], va[5], va[6], va[7]);
    }
    __syncthreads();
    // 3. gz on the reversed band; gk = gz*v, gv = gz*k
    {
      nsq_f32x4_t acc0, acc1;
      tm.run2(gwin, GR, 16 * wave, 16 * (wave + kConvWaves), acc0, acc1);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int ql = qs_pad(16 * (16 * (wave + h * kConvWaves) + 4 * kk) + li);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int p = 16 * (16 * (wave + h * kConvWaves) + 4 * kk + r) + li;
          const float gz = h ? acc1[r] : acc0[r];
          gkb.store_elem(n0 + p, gz * vs[ql + qs_step(r)]);
          gvb.store_elem(n0 + p, gz * ks[ql + qs_step(r)]);
        }
      }
    }
    __syncthreads();
  }
}

// bwd2 for projection taps Kp <= 4, fused with the input gradient and the
// projection weight gradient: per tile, gz on the reversed band (and by a
// short dot product at the Kp - 1 positions past the tile), gk = gz*v and
// gv = gz*k into LDS, gq from the workspace; then
//   gx_c[n] = sum_j w_c[j] gc[n + Kp - 1 - j]   (c = q, k, v)
// stored directly, and gw_c[j] += sum_n gc[n] x_c[n - Kp + 1 + j] kept per
// thread over the workgroup's tiles, reduced in a fixed order into a
// per-workgroup partial [3][4].  (Neither gk, gv nor gx need a workspace pass.)
constexpr int kB2BBwdExtra = 4;  // positions past the tile with gk, gv (>= Kp - 1, keeps 16-byte alignment)

// A 16-byte LDS read kept whole.  Of a window read as four float4 only some
// values may be used; the compiler then narrows the reads to those values as
// misaligned 4- and 8-byte reads, which at a lane stride of 8 words fall 8 to
// a bank (4-byte accesses are served 32 lanes at a time over 32 banks).
__device__ __forceinline__ float4 lds_read16(const float* p) {
  float4 v = *reinterpret_cast<const float4*>(p);
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
  return v;
}

template <int NS>
struct B2BBwd2fLds {
  static constexpr int GR = win_half(mfma_src_count<NS>() + kB2BBwdExtra);
  static constexpr int GWORDS = win_words(mfma_src_count<NS>() + kB2BBwdExtra);
  static constexpr int XW = kConvTile + 3 + kB2BBwdExtra + 2 * kConvPer;  // staged x / g words per row
  static constexpr int XS = (XW + 7) & ~7;
  int gw, xq, xk, xv, gq, gk, gv, ks, vs, wq, wk, wv, wr, total;
  __host__ __device__ B2BBwd2fLds(int Km) {
    gw = 0;
    xq = GWORDS;
    xk = xq + XS;
    xv = xk + XS;
    gq = xv + XS;
    gk = gq + XS;
    gv = gk + XS;
    ks = gv + XS;  // k, v at tile positions p (+ the extra ones), index p
    vs = ks + XS;
    wq = vs + XS;  // three reversed 4-tap sets (padded to 8), then the reversed mixer
    wk = wq + 8;
    wv = wk + 8;
    wr = wv + 8;
    total = wr + ((Km + 7) & ~7);
    if (total < 12 * kConvThreads) total = 12 * kConvThreads;  // end-of-segment reduction
  }
};

template <int DT, int NS>
__global__ __launch_bounds__(kConvThreads) __attribute__((amdgpu_waves_per_eu(2))) void b2b_bwd2f_mfma_kernel(
    const typename Elem<DT>::T* __restrict__ x, const float* __restrict__ wp, const float* __restrict__ wm,
    const float* __restrict__ skip, const float* __restrict__ ghw, const float* __restrict__ gpw,
    typename Elem<DT>::T* __restrict__ gx, float* __restrict__ gwp_part, int B, int C, int L, int Kp, int Km) {
  using ET = typename Elem<DT>::T;
  constexpr int ZW = mfma_src_count<NS>() + kB2BBwdExtra;
  constexpr int GIT = (ZW + kConvThreads - 1) / kConvThreads;
  using LY = B2BBwd2fLds<NS>;
  constexpr int GR = LY::GR;
  extern __shared__ __align__(16) float smem[];
  const LY lay(Km);
  float* gwin = smem + lay.gw;
  float* xs[3] = {smem + lay.xq, smem + lay.xk, smem + lay.xv};
  float* gs_q = smem + lay.gq;
  float* gs_k = smem + lay.gk;
  float* gs_v = smem + lay.gv;
  float* ks = smem + lay.ks;
  float* vs = smem + lay.vs;
  float* wl[3] = {smem + lay.wq, smem + lay.wk, smem + lay.wv};
  float* wlr = smem + lay.wr;
  const int64_t row = blockIdx.x;  // b*C + c
  const int b = int(row / C), c = int(row % C);
  const int ntiles = (L + kConvTile - 1) / kConvTile;
  const int t_begin = int(blockIdx.y) * kB2BSegTiles;
  const int t_end = min(ntiles, t_begin + kB2BSegTiles);
  const ET* xrow[3];
  xrow[0] = x + (int64_t(b) * 3 * C + c) * L;
  xrow[1] = xrow[0] + int64_t(C) * L;
  xrow[2] = xrow[1] + int64_t(C) * L;
  const float* ghr = ghw + row * L;
  const float* gqr = gpw + (int64_t(b) * 3 * C + c) * L;
  const int hp = Kp - 1;
  const int t = int(threadIdx.x);
  // 4-tap sets, left-padded as in the forward (w4[j] = w[j - (4 - Kp)]) for
  // the projection convs, and reversed (wr4[j] = w[Kp - 1 - j], zero for j >=
  // Kp) for the input-gradient correlations
  if (t < 24) {
    const int set = t / 8, j = t % 8;
    const int ch = set * C + c;
    wl[set][j] = (j < Kp) ? wp[int64_t(ch) * Kp + (Kp - 1 - j)] : 0.f;
  }
  float w4[3][4];
#pragma unroll
  for (int set = 0; set < 3; ++set) load_taps4(w4[set], wp + int64_t(set * C + c) * Kp, Kp);
  stage_weights<true>(wlr, wm + int64_t(c) * Km, Km);
  // staged words: x rows and gq from n0 - 3 (xs index i <-> position n0 - 3 + i)
  constexpr int XW = LY::XW;
  RowStage<DT, XW> sx0, sx1, sx2;
  RowStage<NSQ_DTYPE_F32, XW> sgq;
  float gstage[GIT];
  auto load_tile = [&](int64_t n0) {
    sx0.load(xrow[0], n0 - 3, 0, L);
    sx1.load(xrow[1], n0 - 3, 0, L);
    sx2.load(xrow[2], n0 - 3, 0, L);
    sgq.load(gqr, n0 - 3, 0, L);
    const RowBuf<NSQ_DTYPE_F32, false> rb(ghr, L);
#pragma unroll
    for (int it = 0; it < GIT; ++it) gstage[it] = rb.elem(n0 + t + it * kConvThreads);
  };
  __syncthreads();  // weights staged
  ToeplitzMfma<NS> tm;
  const float skv = skip ? skip[c] : 0.f;
  tm.load_weights(wlr, Km, 0.f, 0, skv);
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
  const int kk = l >> 4, li = l & 15;
  const int base = t * kConvPer;
  float wacc[3][4];  // projection weight-gradient partials of this thread
#pragma unroll
  for (int cc = 0; cc < 3; ++cc)
#pragma unroll
    for (int j = 0; j < 4; ++j) wacc[cc][j] = 0.f;
  for (int ti = t_begin; ti < t_end; ++ti) {
    const int64_t n0 = int64_t(ti) * kConvTile;
    // 1. stage (loaded here: holding the next tile in registers would spill)
    load_tile(n0);
    sx0.store(xs[0], XW);
    sx1.store(xs[1], XW);
    sx2.store(xs[2], XW);
    sgq.store(gs_q, XW);
#pragma unroll
    for (int it = 0; it < GIT; ++it) {
      const int m = t + it * kConvThreads;
      if (m < ZW) gwin[win_at(m, GR)] = gstage[it];
    }
    // The k / v windows below read x words that other waves staged: the
    // stores above must be complete in every wave first.
    __syncthreads();
    // k, v at the tile positions p = base + e (4-tap convs over xs index p + j, x at n0 + p - 3 + j)
    {
      float ka[kConvPer], va[kConvPer];
#pragma unroll
      for (int e = 0; e < kConvPer; ++e) ka[e] = va[e] = 0.f;
      slide_fma4(ka, xs[1], base, w4[1]);
      slide_fma4(va, xs[2], base, w4[2]);
      *reinterpret_cast<float4*>(ks + base) = make_float4(ka[0], ka[1], ka[2], ka[3]);
      *reinterpret_cast<float4*>(ks + base + 4) = make_float4(ka[4], ka[5], ka[6], ka[7]);
      *reinterpret_cast<float4*>(vs + base) = make_float4(va[0], va[1], va[2], va[3]);
      *reinterpret_cast<float4*>(vs + base + 4) = make_float4(va[4], va[5], va[6], va[7]);
      if (t < kB2BBwdExtra) {  // the positions past the tile
        const int p = kConvTile + t;
        float kv = 0.f, vv = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          kv = fmaf(w4[1][j], xs[1][p + j], kv);
          vv = fmaf(w4[2][j], xs[2][p + j], vv);
        }
        ks[p] = kv;
        vs[p] = vv;
      }
    }
    __syncthreads();
    // 2. gz on the band; gk = gz*v, gv = gz*k at tile positions p (LDS index p + 3)
    {
      nsq_f32x4_t acc0, acc1;
      tm.run2(gwin, GR, 16 * wave, 16 * (wave + kConvWaves), acc0, acc1);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int p = 16 * (16 * (wave + h * kConvWaves) + 4 * kk + r) + li;
          const float gz = h ? acc1[r] : acc0[r];
          gs_k[p + 3] = gz * vs[p];
          gs_v[p + 3] = gz * ks[p];
        }
      }
      // the kB2BBwdExtra positions past the tile: wave w takes position 2048 + w,
      // its lanes split the taps, and a fixed shuffle tree sums them
      static_assert(kB2BBwdExtra == kConvWaves, "b2b bwd2: one wave per extra position");
      {
        const int p = kConvTile + wave;
        float part = 0.f;
        for (int j = l; j < Km; j += 64) part = fmaf(wlr[j], gwin[win_at(p + j, GR)], part);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off, 64);
        if (l == 0) {
          const float gz = fmaf(skv, gwin[win_at(p, GR)], part);
          gs_k[p + 3] = gz * vs[p];
          gs_v[p + 3] = gz * ks[p];
        }
      }
    }
    __syncthreads();
    // 3. input gradients and weight-gradient partials at n0 + base + e
    {
      const float* gsrc[3] = {gs_q, gs_k, gs_v};
#pragma unroll
      for (int cc = 0; cc < 3; ++cc) {
        // window gc[n0 + base - 3 + i], i < 16 (LDS index base + i); x at the same offsets
        float gw_[16], xw_[12];
        {
          const float4 a = lds_read16(gsrc[cc] + base);
          const float4 b4 = lds_read16(gsrc[cc] + base + 4);
          const float4 c4 = lds_read16(gsrc[cc] + base + 8);
          const float4 d4 = lds_read16(gsrc[cc] + base + 12);
          const float tmp[16] = {a.x, a.y, a.z, a.w, b4.x, b4.y, b4.z, b4.w,
                                 c4.x, c4.y, c4.z, c4.w, d4.x, d4.y, d4.z, d4.w};
#pragma unroll
          for (int i = 0; i < 16; ++i) gw_[i] = tmp[i];
          const float4 xa = *reinterpret_cast<const float4*>(xs[cc] + base);
          const float4 xb = *reinterpret_cast<const float4*>(xs[cc] + base + 4);
          const float4 xc = *reinterpret_cast<const float4*>(xs[cc] + base + 8);
          const float xt[12] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w, xc.x, xc.y, xc.z, xc.w};
#pragma unroll
          for (int i = 0; i < 12; ++i) xw_[i] = xt[i];
        }
        const float4 wr4 = *reinterpret_cast<const float4*>(wl[cc]);
        const float wr[4] = {wr4.x, wr4.y, wr4.z, wr4.w};
        float out[kConvPer];
#pragma unroll
        for (int e = 0; e < kConvPer; ++e) {
          // gx[n] = sum_j w[Kp-1-j] gc[n + j], n = n0 + base + e -> window index e + 3 + j
          float a = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) a = fmaf(wr[j], gw_[e + 3 + j], a);
          out[e] = a;
          // gw[j] += gc[n] x[n - Kp + 1 + j], x window index e + 3 - hp + j
          const float gcv = (n0 + base + e < L) ? gw_[e + 3] : 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int xi = e + 3 - hp + j;  // 0 <= xi < 12 for hp <= 3, j <= 3
            wacc[cc][j] = fmaf(gcv, (j < Kp) ? xw_[xi < 0 ? 0 : (xi > 11 ? 11 : xi)] : 0.f, wacc[cc][j]);
          }
        }
        ET* gr = gx + (int64_t(b) * 3 * C + cc * C + c) * L;
#pragma unroll
        for (int e = 0; e < kConvPer; e += 2) {
          const int64_t n = n0 + base + e;
          if (n < L) store_pair<DT>(gr, n, L, make_float2(out[e], out[e + 1]));
        }
      }
    }
    __syncthreads();
  }
  // Fixed-order reduction of the weight-gradient partials: red[v][t], v < 12.
  float* red = smem;
#pragma unroll
  for (int cc = 0; cc < 3; ++cc)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[(cc * 4 + j) * kConvThreads + t] = wacc[cc][j];
  __syncthreads();
  if (t < 12) {
    float sacc = 0.f;
    for (int i = 0; i < kConvThreads; ++i) sacc += red[t * kConvThreads + i];
    const int nparts = B * int(gridDim.y);
    const int part = b * int(gridDim.y) + int(blockIdx.y);
    gwp_part[(int64_t(c) * nparts + part) * 12 + t] = sacc;
  }
}

// gw_proj[set*C + c, j] = sum of the channel's partials (fixed order), j < Kp.
__global__ void b2b_pwgrad_reduce_kernel(const float* __restrict__ part, int nparts, int C, int Kp,
                                         float* __restrict__ gw) {
  const int c = blockIdx.x, v = threadIdx.x;  // v = set * 4 + j
  if (v >= 12 || (v % 4) >= Kp) return;
  const float* pc = part + int64_t(c) * nparts * 12 + v;
  float sacc = 0.f;
  for (int p = 0; p < nparts; ++p) sacc += pc[int64_t(p) * 12];
  gw[int64_t((v / 4) * C + c) * Kp + (v % 4)] = sacc;
}

// gw_mixer[c, j] = sum over the channel's partials (fixed order); gskip[c] = its lag Km-1.
__global__ void b2b_wgrad_reduce_kernel(const float* __restrict__ part, int nparts, int Km, float* __restrict__ gw,
                                        float* __restrict__ gskip) {
  const int c = blockIdx.x, j = threadIdx.x;
  if (j >= Km) return;
  const float* pc = part + int64_t(c) * nparts * Km + j;
  float sacc = 0.f;
  for (int p = 0; p < nparts; ++p) sacc += pc[int64_t(p) * Km];
  gw[int64_t(c) * Km + j] = sacc;
  if (gskip && j == Km - 1) gskip[c] = sacc;
}

// ---------------------------------------------------------------------------
// Wave-specialized matrix-core forward for projection taps Kp <= 4 (the
// striped-Hyena short conv).  A workgroup of 8 waves owns one channel c and
// walks kB2BWsSegTiles consecutive tiles of the channel's (batch, tile)
// sequence, g = b * ntiles + tile (one weight set for all of them):
//   * waves 4..7 (producers) build tile u+1: each thread reads its 12-sample
//     windows of the q, k, v rows straight from HBM (vector loads, issued a
//     tile ahead), runs the 4-tap projection convs in registers and writes
//     z = k*v and q to the LDS buffers of tile u+1;
//   * waves 0..3 (consumers) run the mixer conv of tile u on the matrix cores
//     (ToeplitzMfma, two M-tiles per wave) and store out = q * h.
// One barrier per tile hands the double-buffered z/q over; on each SIMD a
// producer wave's VALU work overlaps a consumer wave's MFMA chain.
// The mixer band gets `d` leading zero taps so that its halo hz = Km - 1 + d
// is a multiple of 4 (fp32) or 8 (bf16 halves): z of a tile then starts at a
// 16-byte boundary of the window buffer.
constexpr int kB2BWsThreads = 512;
constexpr int kB2BWsSegTiles = 16;  // 4, 6, 8, 12, 16, 32 measured at config 2: 16 and 32 fastest

// BF (16-bit I/O): z is stored as two plain bf16 arrays (hi, lo;
// ToeplitzMfmaBf16), ZE elements each, in the words of one z buffer; fp32: one
// window in the split layout (region stride ZR).
template <int NS, bool BF = false>
struct B2BWsLds {
  static constexpr int ZCOUNT = BF ? kConvTile + 32 * bf16_steps<NS>() - 16 : mfma_src_count<NS>();
  static constexpr int ZE = (ZCOUNT + 15) & ~15;
  static constexpr int ZR = win_half(mfma_src_count<NS>());
  static constexpr int ZWORDS = BF ? ZE : win_words(mfma_src_count<NS>());
  static constexpr int QWORDS = kConvTile + kConvTile / 4;  // qs_pad layout
  static constexpr int z0 = 0, q0 = 2 * ZWORDS, wm = 2 * ZWORDS + 2 * QWORDS;
  static constexpr int total = wm + kConvMaxK;
};

// out[e] = sum_{j<4} w4[j] x[n + e - 3 + j], e < 8, from a window at n.
template <int DT, bool AL>
__device__ __forceinline__ void conv4_from_window(float (&out)[kConvPer], const Win12<DT, AL>& win, const float (&w4)[4]) {
  float xv[12];
#pragma unroll
  for (int i = 0; i < 12; ++i) xv[i] = win.at(i);
#pragma unroll
  for (int e = 0; e < kConvPer; ++e) {
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) a = fmaf(w4[j], xv[e + 1 + j], a);
    out[e] = a;
  }
}

template <int DT, int NS, bool AL, bool BF = false>
__global__ __launch_bounds__(kB2BWsThreads) void b2b_fwd_ws_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                                    const float* __restrict__ wp,
                                                                    const float* __restrict__ wm,
                                                                    const float* __restrict__ skip,
                                                                    typename Elem<DT>::T* __restrict__ y, int B, int C,
                                                                    int L, int Kp, int Km) {
  using LY = B2BWsLds<NS, BF>;
  using ET = typename Elem<DT>::T;
  extern __shared__ __align__(16) float smem[];
  float* const zbuf = smem + LY::z0;  // buffer u: zbuf + u * ZWORDS
  float* const qbuf = smem + LY::q0;  // buffer u: qbuf + u * QWORDS
  float* const wlm = smem + LY::wm;
  const int c = int(blockIdx.x);
  const int ntiles = (L + kConvTile - 1) / kConvTile;
  const int g_begin = int(blockIdx.y) * kB2BWsSegTiles;
  const int g_end = min(B * ntiles, g_begin + kB2BWsSegTiles);
  // leading zero taps of the band: the halo hz = Km - 1 + d is a multiple of 4
  // (fp32 words) or 8 (bf16 halves), so a tile's z starts on a 16-byte boundary
  const int d = BF ? ((Km - 1 + 7) & ~7) + 1 - Km : ((Km - 1 + 3) & ~3) + 1 - Km;
  const int hz = Km - 1 + d;
  const int t = int(threadIdx.x);
  const bool producer = t >= kB2BWsThreads / 2;
  // z of position m of buffer zb (float words of that buffer)
  auto zput = [&](float* zb, int m, float v) {
    if constexpr (BF) {
      __bf16* zh = reinterpret_cast<__bf16*>(zb);
      __bf16 hi, lo;
      split_bf16(v, hi, lo);
      zh[m] = hi;
      zh[LY::ZE + m] = lo;
    } else {
      zb[win_at(m, LY::ZR)] = v;
    }
  };
  auto zcopy = [&](float* zb, int m, const float* zo, int mo) {
    if constexpr (BF) {
      __bf16* zh = reinterpret_cast<__bf16*>(zb);
      const __bf16* oh = reinterpret_cast<const __bf16*>(zo);
      zh[m] = oh[mo];
      zh[LY::ZE + m] = oh[LY::ZE + mo];
    } else {
      zb[win_at(m, LY::ZR)] = zo[win_at(mo, LY::ZR)];
    }
  };
  if (t < kConvThreads) stage_weights<false>(wlm, wm + int64_t(c) * Km, Km);
  for (int m = kConvTile + hz + t; m < LY::ZCOUNT; m += kB2BWsThreads) {
    zput(zbuf, m, 0.f);
    zput(zbuf + LY::ZWORDS, m, 0.f);
  }
  // q row of batch b; k and v rows follow at C*L and 2*C*L
  auto qrow = [&](int b) -> const ET* { return x + (int64_t(b) * 3 * C + c) * L; };
  if (producer) {
    const int pt = t - kB2BWsThreads / 2;
    float wq4[4], wk4[4], wv4[4];
    load_taps4(wq4, wp + int64_t(c) * Kp, Kp);
    load_taps4(wk4, wp + int64_t(C + c) * Kp, Kp);
    load_taps4(wv4, wp + int64_t(2 * C + c) * Kp, Kp);
    Win12<DT, AL> cq, ck, cv;
    auto load_tile = [&](int g, Win12<DT, AL>& wq_, Win12<DT, AL>& wk_, Win12<DT, AL>& wv_) {
      const int b = g / ntiles, ti = g - b * ntiles;
      const ET* xq = qrow(b);
      const int n = ti * kConvTile + 8 * pt;
      wq_.load(RowBuf<DT, false>(xq, L), n);
      wk_.load(RowBuf<DT, false>(xq + int64_t(C) * L, L), n);
      wv_.load(RowBuf<DT, false>(xq + 2 * int64_t(C) * L, L), n);
    };
    load_tile(g_begin, cq, ck, cv);
    // builds tile g into buffer nb from the windows in cq/ck/cv; the z halo is
    // zero at a row start, recomputed from the row at the segment start, else
    // carried over from buffer ob
    auto produce = [&](int g, int nb, int ob) {
      const int b = g / ntiles, ti = g - b * ntiles;
      const int n0 = ti * kConvTile;
      Win12<DT, AL> nq, nk, nv;
      const bool more = g + 1 < g_end;
      if (more) load_tile(g + 1, nq, nk, nv);
      float* zb = zbuf + nb * LY::ZWORDS;
      float* qb = qbuf + nb * LY::QWORDS;
      float ka[kConvPer], va[kConvPer], qa[kConvPer];
      conv4_from_window(ka, ck, wk4);
      conv4_from_window(va, cv, wv4);
      conv4_from_window(qa, cq, wq4);
      const int n = n0 + 8 * pt;
      float zv[kConvPer];
#pragma unroll
      for (int e = 0; e < kConvPer; ++e) zv[e] = (n + e < L) ? ka[e] * va[e] : 0.f;
      if constexpr (BF) {
        nsq_bf16x8_t h8, l8;
#pragma unroll
        for (int e = 0; e < kConvPer; ++e) {
          __bf16 hi, lo;
          split_bf16(zv[e], hi, lo);
          h8[e] = hi;
          l8[e] = lo;
        }
        __bf16* zh = reinterpret_cast<__bf16*>(zb);
        *reinterpret_cast<nsq_bf16x8_t*>(zh + hz + 8 * pt) = h8;
        *reinterpret_cast<nsq_bf16x8_t*>(zh + LY::ZE + hz + 8 * pt) = l8;
      } else {
        win_store8(zb, LY::ZR, hz + 8 * pt, zv);
      }
      float* qd = qb + qs_pad(8 * pt);
      *reinterpret_cast<float4*>(qd) = make_float4(qa[0], qa[1], qa[2], qa[3]);
      *reinterpret_cast<float4*>(qd + 4) = make_float4(qa[4], qa[5], qa[6], qa[7]);
      if (ti == 0) {
        if (pt < hz) zput(zb, pt, 0.f);  // causal padding before the row start
      } else if (g == g_begin) {
        if (8 * pt < hz) {  // z at n0 - hz + m, m < hz
          const ET* xq = qrow(b);
          Win12<DT, false> hk, hv;
          const int nh = n0 - hz + 8 * pt;
          hk.load(RowBuf<DT, false>(xq + int64_t(C) * L, L), nh);
          hv.load(RowBuf<DT, false>(xq + 2 * int64_t(C) * L, L), nh);
          float kh[kConvPer], vh[kConvPer];
          conv4_from_window(kh, hk, wk4);
          conv4_from_window(vh, hv, wv4);
#pragma unroll
          for (int e = 0; e < kConvPer; ++e)
            if (8 * pt + e < hz) zput(zb, 8 * pt + e, kh[e] * vh[e]);
        }
      } else {
        const float* zo = zbuf + ob * LY::ZWORDS;
        if (pt < hz) zcopy(zb, pt, zo, kConvTile + pt);
      }
      if (more) {
        cq = nq; ck = nk; cv = nv;
      }
    };
    produce(g_begin, 0, 1);
    __syncthreads();
    for (int g = g_begin; g < g_end; ++g) {
      const int cb = (g - g_begin) & 1;
      if (g + 1 < g_end) produce(g + 1, cb ^ 1, cb);
      __syncthreads();
    }
  } else {
    __syncthreads();  // weights staged, first tile produced
    using TM = std::conditional_t<BF, ToeplitzMfmaBf16<bf16_steps<NS>()>, ToeplitzMfma<NS>>;
    TM tm;
    tm.load_weights(wlm, Km, skip ? skip[c] : 0.f, d);
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
    for (int g = g_begin; g < g_end; ++g) {
      const int cb = (g - g_begin) & 1;
      const int b = g / ntiles, ti = g - b * ntiles;
      const RowBuf<DT, false> yb(y + (int64_t(b) * C + c) * L, L);
      const float* zb = zbuf + cb * LY::ZWORDS;
      const float* qb = qbuf + cb * LY::QWORDS;
      nsq_f32x4_t acc0, acc1;
      if constexpr (BF) {
        const __bf16* zh = reinterpret_cast<const __bf16*>(zb);
        tm.run2(zh, zh + LY::ZE, 16 * wave, 16 * (wave + kConvWaves), acc0, acc1);
      } else {
        tm.run2(zb, LY::ZR, 16 * wave, 16 * (wave + kConvWaves), acc0, acc1);
      }
      const int n0 = ti * kConvTile;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int mt = wave + h * kConvWaves;
        const float* ql = qb + qs_pad(16 * (16 * mt + 4 * (l >> 4)) + (l & 15));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int p = 16 * (16 * mt + 4 * (l >> 4) + r) + (l & 15);
          yb.store_elem(n0 + p, ql[qs_step(r)] * (h ? acc1[r] : acc0[r]));
        }
      }
      __syncthreads();
    }
  }
}

// Backward step 1: recompute q, z, h; write gq = g*h into gp (q rows),
// gh = g*q and z (fp32 workspaces).  grid as forward.
template <int DT>
__global__ __launch_bounds__(kConvThreads) void b2b_bwd1_kernel(const typename Elem<DT>::T* __restrict__ g,
                                                                 const typename Elem<DT>::T* __restrict__ x,
                                                                 const float* __restrict__ wp,
                                                                 const float* __restrict__ wm,
                                                                 const float* __restrict__ skip,
                                                                 float* __restrict__ gp, float* __restrict__ gh,
                                                                 float* __restrict__ zw, int C, int L, int Kp, int Km) {
  constexpr int TF = conv_tile_floats(2 * kConvMaxK);
  extern __shared__ __align__(16) float smem[];
  const B2BLds lay(Kp, Km);
  float* xs_q = smem + lay.q;
  float* xs_k = smem + lay.k;
  float* xs_v = smem + lay.v;
  float* zs = smem + lay.z;
  float* wlq = smem + lay.wq;
  float* wlk = smem + lay.wk;
  float* wlv = smem + lay.wv;
  float* wlm = smem + lay.wm;
  const int64_t row = blockIdx.x;
  const int b = int(row / C), c = int(row % C);
  const int64_t n0 = int64_t(blockIdx.y) * kConvTile;
  const int64_t xq = (int64_t(b) * 3 * C + c) * L;
  const int64_t xk = xq + int64_t(C) * L;
  const int64_t xv = xk + int64_t(C) * L;
  const int hz = Km - 1, hp = Kp - 1;
  stage_weights<false>(wlq, wp + int64_t(c) * Kp, Kp);
  stage_weights<false>(wlk, wp + int64_t(C + c) * Kp, Kp);
  stage_weights<false>(wlv, wp + int64_t(2 * C + c) * Kp, Kp);
  stage_weights<false>(wlm, wm + int64_t(c) * Km, Km);
  {
    // all three rows' loads in flight together, then the LDS stores
    RowStage<DT, conv_tile_floats(kConvMaxK)> sq;
    RowStage<DT, TF> sk, sv;
    sq.load(x + xq, n0 - hp, kConvTile + hp + 2 * kConvPer, L);
    sk.load(x + xk, n0 - hz - hp, kConvTile + hz + hp + 2 * kConvPer, L);
    sv.load(x + xv, n0 - hz - hp, kConvTile + hz + hp + 2 * kConvPer, L);
    sq.store(xs_q, kConvTile + hp + 2 * kConvPer);
    sk.store(xs_k, kConvTile + hz + hp + 2 * kConvPer);
    sv.store(xs_v, kConvTile + hz + hp + 2 * kConvPer);
    __syncthreads();
  }
  const int zcount = kConvTile + hz + 2 * kConvPer;
  for (int i = threadIdx.x; i < zcount; i += kConvThreads) {
    const int64_t n = n0 - hz + i;
    float kk = 0.f, vv = 0.f;
    if (n >= 0 && n < L) {
      for (int j = 0; j < Kp; ++j) {
        kk = fmaf(wlk[j], xs_k[i + j], kk);
        vv = fmaf(wlv[j], xs_v[i + j], vv);
      }
    }
    zs[i] = kk * vv;
  }
  __syncthreads();
  const int base = threadIdx.x * kConvPer;
  float qa[kConvPer], ha[kConvPer];
#pragma unroll
  for (int e = 0; e < kConvPer; ++e) qa[e] = ha[e] = 0.f;
  slide_fma(qa, xs_q, base, Kp, wlq);
  slide_fma(ha, zs, base, Km, wlm);
  const float sk = skip ? skip[c] : 0.f;
  const int64_t orow = row * L;                           // [B, C, L] rows
  const int64_t prow = (int64_t(b) * 3 * C + c) * L;      // q rows of gp [B, 3C, L]
  float gva[kConvPer];
#pragma unroll
  for (int e = 0; e < kConvPer; ++e) {  // all loads first (clamped), then predicated stores
    const int64_t n = n0 + base + e;
    gva[e] = Elem<DT>::load(g, orow + (n < L ? n : 0));
  }
#pragma unroll
  for (int e = 0; e < kConvPer; ++e) {
    const int64_t n = n0 + base + e;
    if (n < L) {
      const float zv = zs[base + e + hz];
      const float hv = fmaf(sk, zv, ha[e]);
      gp[prow + n] = gva[e] * hv;
      gh[orow + n] = gva[e] * qa[e];
      zw[orow + n] = zv;
    }
  }
}

// Backward step 2: gz = corr(gh, w_mixer) + skip*gh; recompute k, v;
// gk = gz*v, gv = gz*k into gp (k and v rows).  grid as forward.
template <int DT>
__global__ __launch_bounds__(kConvThreads) void b2b_bwd2_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                                 const float* __restrict__ wp,
                                                                 const float* __restrict__ wm,
                                                                 const float* __restrict__ skip,
                                                                 const float* __restrict__ gh, float* __restrict__ gp,
                                                                 int C, int L, int Kp, int Km) {
  __shared__ __align__(16) float ghs[conv_tile_floats(kConvMaxK)];
  __shared__ __align__(16) float xs_k[conv_tile_floats(kConvMaxK)];
  __shared__ __align__(16) float xs_v[conv_tile_floats(kConvMaxK)];
  __shared__ __align__(16) float wlm[kConvWeightFloats];
  __shared__ __align__(16) float wlk[kConvWeightFloats];
  __shared__ __align__(16) float wlv[kConvWeightFloats];
  const int64_t row = blockIdx.x;
  const int b = int(row / C), c = int(row % C);
  const int64_t n0 = int64_t(blockIdx.y) * kConvTile;
  stage_weights<true>(wlm, wm + int64_t(c) * Km, Km);
  stage_weights<false>(wlk, wp + int64_t(C + c) * Kp, Kp);
  stage_weights<false>(wlv, wp + int64_t(2 * C + c) * Kp, Kp);
  const int64_t xk = (int64_t(b) * 3 * C + C + c) * L;
  const int64_t xv = xk + int64_t(C) * L;
  const int hp = Kp - 1;
  {
    RowStage<NSQ_DTYPE_F32, conv_tile_floats(kConvMaxK)> sh;
    RowStage<DT, conv_tile_floats(kConvMaxK)> sk, sv;
    sh.load(gh + row * L, n0, kConvTile + Km - 1 + 2 * kConvPer, L);
    sk.load(x + xk, n0 - hp, kConvTile + hp + 2 * kConvPer, L);
    sv.load(x + xv, n0 - hp, kConvTile + hp + 2 * kConvPer, L);
    sh.store(ghs, kConvTile + Km - 1 + 2 * kConvPer);
    sk.store(xs_k, kConvTile + hp + 2 * kConvPer);
    sv.store(xs_v, kConvTile + hp + 2 * kConvPer);
    __syncthreads();
  }
  const int base = threadIdx.x * kConvPer;
  float gz[kConvPer], ka[kConvPer], va[kConvPer];
#pragma unroll
  for (int e = 0; e < kConvPer; ++e) gz[e] = ka[e] = va[e] = 0.f;
  slide_fma(gz, ghs, base, Km, wlm);
  slide_fma(ka, xs_k, base, Kp, wlk);
  slide_fma(va, xs_v, base, Kp, wlv);
  const float sk = skip ? skip[c] : 0.f;
#pragma unroll
  for (int e = 0; e < kConvPer; ++e) {
    const int64_t n = n0 + base + e;
    if (n < L) {
      const float gzv = fmaf(sk, ghs[base + e], gz[e]);
      gp[xk + n] = gzv * va[e];
      gp[xv + n] = gzv * ka[e];
    }
  }
}

__global__ void copy_column_kernel(const float* __restrict__ src, int ld, int col, float* __restrict__ dst, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[int64_t(i) * ld + col];
}

template <int DT, int NS>
static void launch_b2b_fwd_mfma(const void* x, const float* wp, const float* wm, const float* skip, void* y, int B,
                                int C, int L, int Kp, int Km, hipStream_t st) {
  using ET = typename Elem<DT>::T;
  dim3 grid(B * C, unsigned(ceil_div(ceil_div(L, kConvTile), kB2BSegTiles)));
  const size_t lds = size_t(B2BMfmaLds<NS>(Kp, Km).total) * sizeof(float);
  if (Kp <= 4) {
    // wave-specialized kernel; vector window loads when every row starts 16-byte aligned
    const bool al = L % (DT == NSQ_DTYPE_F32 ? 4 : 8) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    dim3 gws(C, unsigned(ceil_div(int64_t(B) * ceil_div(L, kConvTile), kB2BWsSegTiles)));
    // 16-bit I/O: the mixer's products as three bf16 products (ToeplitzMfmaBf16);
    // NSQ_B2B_BF16_SPLIT=0 keeps the fp32 matrix-core band for every dtype
    static const bool split_env = [] {
      const char* e = std::getenv("NSQ_B2B_BF16_SPLIT");
      return !(e && e[0] == '0');
    }();
    auto go = [&](auto bf) {
      constexpr bool BF = decltype(bf)::value;
      const size_t lws = size_t(B2BWsLds<NS, BF>::total) * sizeof(float);
      if (al)
        hipLaunchKernelGGL((b2b_fwd_ws_kernel<DT, NS, true, BF>), gws, dim3(kB2BWsThreads), lws, st, (const ET*)x,
                           wp, wm, skip, (ET*)y, B, C, L, Kp, Km);
      else
        hipLaunchKernelGGL((b2b_fwd_ws_kernel<DT, NS, false, BF>), gws, dim3(kB2BWsThreads), lws, st, (const ET*)x,
                           wp, wm, skip, (ET*)y, B, C, L, Kp, Km);
    };
    if (DT != NSQ_DTYPE_F32 && split_env)
      go(std::true_type{});
    else
      go(std::false_type{});
  } else {
    hipLaunchKernelGGL((b2b_fwd_mfma_kernel<DT, NS, false, true>), grid, dim3(kConvThreads), lds, st, (const ET*)x,
                       wp, wm, skip, (ET*)y, C, L, Kp, Km);
  }
}

template <int DT>
static void launch_b2b_fwd(const void* x, const float* wp, const float* wm, const float* skip, void* y, int B, int C,
                           int L, int Kp, int Km, hipStream_t st) {
  using ET = typename Elem<DT>::T;
  switch (mfma_steps_for(Km)) {  // mixer conv on the matrix cores from 16 taps up
    case 12: return launch_b2b_fwd_mfma<DT, 12>(x, wp, wm, skip, y, B, C, L, Kp, Km, st);
    case 20: return launch_b2b_fwd_mfma<DT, 20>(x, wp, wm, skip, y, B, C, L, Kp, Km, st);
    case 36: return launch_b2b_fwd_mfma<DT, 36>(x, wp, wm, skip, y, B, C, L, Kp, Km, st);
    case 68: return launch_b2b_fwd_mfma<DT, 68>(x, wp, wm, skip, y, B, C, L, Kp, Km, st);
    default: break;
  }
  dim3 grid(B * C, unsigned(ceil_div(L, kConvTile)));
  hipLaunchKernelGGL((b2b_fwd_kernel<DT>), grid, dim3(kConvThreads), size_t(B2BLds(Kp, Km).total) * sizeof(float), st, (const ET*)x, wp, wm, skip, (ET*)y, C, L,
                     Kp, Km);
}

// Partials of the matrix-core mixer weight gradient: [C][B * segments][Km].
static int64_t b2b_wgrad_parts(int64_t B, int64_t L) { return B * ceil_div(ceil_div(L, kConvTile), kB2BSegTiles); }

template <int DT, int NS>
static void launch_b2b_bwd_mfma(const void* g, const void* x, const float* wp, const float* wm, const float* skip,
                                void* gx, float* gwp, float* gwm, float* gskip, int B, int C, int L, int Kp, int Km,
                                float* gp, float* gh, float* part, hipStream_t st) {
  using ET = typename Elem<DT>::T;
  dim3 grid(B * C, unsigned(ceil_div(ceil_div(L, kConvTile), kB2BSegTiles)));
  const size_t l1 = size_t(B2BBwd1Lds<NS>(Kp, Km).total) * sizeof(float);
  if (Kp <= 4) {
    hipLaunchKernelGGL((b2b_bwd1_mfma_kernel<DT, NS, true>), grid, dim3(kConvThreads), l1, st, (const ET*)g,
                       (const ET*)x, wp, wm, skip, gp, gh, part, B, C, L, Kp, Km);
    // fused: gz, gk, gv, the input gradient and the projection weight-gradient partials
    float* ppart = part + int64_t(C) * b2b_wgrad_parts(B, L) * Km;
    const size_t l2 = size_t(B2BBwd2fLds<NS>(Km).total) * sizeof(float);
    hipLaunchKernelGGL((b2b_bwd2f_mfma_kernel<DT, NS>), grid, dim3(kConvThreads), l2, st, (const ET*)x, wp, wm, skip,
                       (const float*)gh, (const float*)gp, (ET*)gx, ppart, B, C, L, Kp, Km);
    hipLaunchKernelGGL(b2b_pwgrad_reduce_kernel, dim3(C), dim3(64), 0, st, (const float*)ppart,
                       int(b2b_wgrad_parts(B, L)), C, Kp, gwp);
  } else {
    const size_t l2 = size_t(B2BBwd2Lds<DT, NS, false>(Kp, Km).total) * sizeof(float);
    hipLaunchKernelGGL((b2b_bwd1_mfma_kernel<DT, NS, false>), grid, dim3(kConvThreads), l1, st, (const ET*)g,
                       (const ET*)x, wp, wm, skip, gp, gh, part, B, C, L, Kp, Km);
    hipLaunchKernelGGL((b2b_bwd2_mfma_kernel<DT, NS, false>), grid, dim3(kConvThreads), l2, st, (const ET*)x, wp, wm,
                       skip, (const float*)gh, gp, C, L, Kp, Km);
  }
  hipLaunchKernelGGL(b2b_wgrad_reduce_kernel, dim3(C), dim3(kConvThreads), 0, st, (const float*)part,
                     int(b2b_wgrad_parts(B, L)), Km, gwm, gskip);
}

template <int DT>
static void launch_b2b_bwd(const void* g, const void* x, const float* wp, const float* wm, const float* skip, void* gx,
                           float* gwp, float* gwm, float* gskip, int B, int C, int L, int Kp, int Km, float* ws,
                           hipStream_t st) {
  using ET = typename Elem<DT>::T;
  const int64_t E = int64_t(B) * C * L;
  float* gp = ws;            // [B, 3C, L]
  float* gh = ws + 3 * E;    // [B, C, L]
  float* zw = ws + 4 * E;    // [B, C, L] (FMA path), or the weight-gradient partials (MFMA path)
  const int ns = mfma_steps_for(Km);
  if (ns) {
    switch (ns) {
      case 12: launch_b2b_bwd_mfma<DT, 12>(g, x, wp, wm, skip, gx, gwp, gwm, gskip, B, C, L, Kp, Km, gp, gh, zw, st); break;
      case 20: launch_b2b_bwd_mfma<DT, 20>(g, x, wp, wm, skip, gx, gwp, gwm, gskip, B, C, L, Kp, Km, gp, gh, zw, st); break;
      case 36: launch_b2b_bwd_mfma<DT, 36>(g, x, wp, wm, skip, gx, gwp, gwm, gskip, B, C, L, Kp, Km, gp, gh, zw, st); break;
      default: launch_b2b_bwd_mfma<DT, 68>(g, x, wp, wm, skip, gx, gwp, gwm, gskip, B, C, L, Kp, Km, gp, gh, zw, st); break;
    }
    if (Kp <= 4) return;  // input and projection gradients came with bwd2
    dim3 grid3(B * 3 * C, unsigned(ceil_div(L, kConvTile)));
    hipLaunchKernelGGL((cconv_gx_kernel<DT, NSQ_DTYPE_F32>), grid3, dim3(kConvThreads), 0, st, (const float*)gp, wp,
                       (ET*)gx, 3 * C, L, Kp);
    hipLaunchKernelGGL((cconv_wgrad_kernel<DT, NSQ_DTYPE_F32>), dim3(3 * C), dim3(kConvThreads), 0, st,
                       (const float*)gp, (const ET*)x, gwp, (float*)nullptr, B, 3 * C, L, Kp);
    return;
  }
  dim3 grid(B * C, unsigned(ceil_div(L, kConvTile)));
  hipLaunchKernelGGL((b2b_bwd1_kernel<DT>), grid, dim3(kConvThreads), size_t(B2BLds(Kp, Km).total) * sizeof(float), st, (const ET*)g, (const ET*)x, wp, wm, skip,
                     gp, gh, zw, C, L, Kp, Km);
  hipLaunchKernelGGL((b2b_bwd2_kernel<DT>), grid, dim3(kConvThreads), 0, st, (const ET*)x, wp, wm, skip,
                     (const float*)gh, gp, C, L, Kp, Km);
  // input gradient and projection-weight gradient over all 3C channels
  dim3 grid3(B * 3 * C, unsigned(ceil_div(L, kConvTile)));
  hipLaunchKernelGGL((cconv_gx_kernel<DT, NSQ_DTYPE_F32>), grid3, dim3(kConvThreads), 0, st, (const float*)gp, wp, (ET*)gx,
                     3 * C, L, Kp);
  hipLaunchKernelGGL((cconv_wgrad_kernel<DT, NSQ_DTYPE_F32>), dim3(3 * C), dim3(kConvThreads), 0, st,
                     (const float*)gp, (const ET*)x, gwp, (float*)nullptr, B, 3 * C, L, Kp);
  // mixer-weight gradient: sum_n gh[n] z[n-Km+1+j]; its lag Km-1 is the skip gradient
  hipLaunchKernelGGL((cconv_wgrad_kernel<NSQ_DTYPE_F32, NSQ_DTYPE_F32>), dim3(C), dim3(kConvThreads), 0, st,
                     (const float*)gh, (const float*)zw, gwm, (float*)nullptr, B, C, L, Km);
  if (gskip)
    hipLaunchKernelGGL(copy_column_kernel, dim3(unsigned(ceil_div(C, 256))), dim3(256), 0, st, (const float*)gwm, Km,
                       Km - 1, gskip, C);
}

static int validate_b2b(const void* a, const void* b, const float* wp, const float* wm, int dtype, int64_t B, int64_t C,
                        int64_t L, int64_t Kp, int64_t Km) {
  NSQ_CHECK_ARG(a && b && wp && wm, "b2b_causal_conv1d: null tensor pointer");
  NSQ_CHECK_ARG(valid_dtype(dtype), "b2b_causal_conv1d: unsupported dtype code %d", dtype);
  NSQ_CHECK_ARG(B >= 1 && C >= 1 && L >= 1, "b2b_causal_conv1d: sizes must be positive");
  NSQ_CHECK_ARG(Kp >= 1 && Kp <= kConvMaxK && Km >= 1 && Km <= kConvMaxK,
                "b2b_causal_conv1d: kernel sizes (%lld, %lld) outside [1, %d]", (long long)Kp, (long long)Km, kConvMaxK);
  NSQ_CHECK_ARG(B * 3 * C <= 0x7fffffff && L < (int64_t(1) << 28), "b2b_causal_conv1d: tensor too large (rows are staged through 32-bit byte offsets: L < 2^28)");
  return NSQ_OK;
}

}  // namespace nsq

using namespace nsq;

extern "C" {

int nsq_b2b_causal_conv1d_fwd(const void* x, const float* weight_proj, const float* weight_mixer,
                              const float* skip_bias, void* y, int dtype, int64_t B, int64_t C, int64_t L, int64_t Kp,
                              int64_t Km, void* stream) {
  clear_error();
  int rc = validate_b2b(x, y, weight_proj, weight_mixer, dtype, B, C, L, Kp, Km);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case NSQ_DTYPE_F32: launch_b2b_fwd<NSQ_DTYPE_F32>(x, weight_proj, weight_mixer, skip_bias, y, int(B), int(C), int(L), int(Kp), int(Km), st); break;
    case NSQ_DTYPE_BF16: launch_b2b_fwd<NSQ_DTYPE_BF16>(x, weight_proj, weight_mixer, skip_bias, y, int(B), int(C), int(L), int(Kp), int(Km), st); break;
    default: launch_b2b_fwd<NSQ_DTYPE_F16>(x, weight_proj, weight_mixer, skip_bias, y, int(B), int(C), int(L), int(Kp), int(Km), st); break;
  }
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

size_t nsq_b2b_causal_conv1d_bwd_workspace_bytes(int64_t B, int64_t C, int64_t L, int64_t Kp, int64_t Km) {
  (void)Kp;
  // gp [B,3C,L], gh [B,C,L], then z [B,C,L] (FMA path) or the weight-gradient
  // partials [C][B * segments][Km] and [C][B * segments][12] (matrix-core
  // path, Km >= 16)
  const int64_t E = B * C * L;
  const int64_t tail = Km >= 16 ? C * b2b_wgrad_parts(B, L) * (Km + 12) : E;
  return size_t(4 * E + (tail > E ? tail : E)) * sizeof(float);
}

int nsq_b2b_causal_conv1d_bwd(const void* gy, const void* x, const float* weight_proj, const float* weight_mixer,
                              const float* skip_bias, void* gx, float* gweight_proj, float* gweight_mixer,
                              float* gskip, int dtype, int64_t B, int64_t C, int64_t L, int64_t Kp, int64_t Km,
                              void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = validate_b2b(gy, x, weight_proj, weight_mixer, dtype, B, C, L, Kp, Km);
  if (rc) return rc;
  NSQ_CHECK_ARG(gx && gweight_proj && gweight_mixer, "b2b_causal_conv1d_bwd: null gradient output pointer");
  const size_t need = nsq_b2b_causal_conv1d_bwd_workspace_bytes(B, C, L, Kp, Km);
  NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "b2b_causal_conv1d_bwd: workspace of %zu bytes required, got %zu",
                need, workspace_bytes);
  hipStream_t st = (hipStream_t)stream;
  float* ws = (float*)workspace;
  switch (dtype) {
    case NSQ_DTYPE_F32:
      launch_b2b_bwd<NSQ_DTYPE_F32>(gy, x, weight_proj, weight_mixer, skip_bias, gx, gweight_proj, gweight_mixer, gskip, int(B), int(C), int(L), int(Kp), int(Km), ws, st);
      break;
    case NSQ_DTYPE_BF16:
      launch_b2b_bwd<NSQ_DTYPE_BF16>(gy, x, weight_proj, weight_mixer, skip_bias, gx, gweight_proj, gweight_mixer, gskip, int(B), int(C), int(L), int(Kp), int(Km), ws, st);
      break;
    default:
      launch_b2b_bwd<NSQ_DTYPE_F16>(gy, x, weight_proj, weight_mixer, skip_bias, gx, gweight_proj, gweight_mixer, gskip, int(B), int(C), int(L), int(Kp), int(Km), ws, st);
      break;
  }
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

}  // extern "C"
