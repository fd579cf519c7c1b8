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
  uint32_t v[IT];  // raw element bits; converted to fp32 by store()
  __device__ __forceinline__ void load(const typename Elem<DT>::T* __restrict__ row, int64_t first, int count,
                                       int64_t len) {
    (void)count;
    const RowBuf<DT, false> rb(row, len);
    const int f = int(first);  // first >= -(2 * kConvMaxK); rows are < 2^31 elements
#pragma unroll
    for (int it = 0; it < IT; ++it) v[it] = rb.elem_halo_bits(f + int(threadIdx.x) + it * kConvThreads);
  }
  __device__ __forceinline__ void store(float* dst, int count) const {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int i = int(threadIdx.x) + it * kConvThreads;
      if (i < count) dst[i] = RowBuf<DT, false>::bits_to_f32(v[it]);
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

// ---------------------------------------------------------------------------
// Depthwise conv on the matrix cores: v_mfma_f32_16x16x4_f32 (fp32 products,
// fp32 accumulation; the same arithmetic as the FMA loop up to summation
// order).  Over a staged tile, output block a (tile outputs 16a .. 16a+15) is
// row a of
//     Y = Xw T,   Xw[a][t] = src[16a + t],   T[t][i] = w[t - i] (0 outside [0, K)),
// t < 4*NS, i.e. y[16a + i] = sum_j w[j] src[16a + i + j]: a banded Toeplitz
// GEMM whose window is 16 + K - 1 wide, so the MFMA does (4*NS) / K <= 1.125x
// the multiply-adds of the tap loop (K = 128), at twice the VALU FMA rate.
//
// MFMA lane layout (wave64, 16x16x4): lane l supplies A[l % 16][l / 16] and
// B[l / 16][l % 16] and receives D[4 (l / 16) + r][l % 16] in accumulator r.
// The window column of step s and k-slot kk = l / 16 is
//     t = 16 (s / 4) + 4 kk + (s % 4),
// so a lane's A values of four consecutive steps are four consecutive src
// words: one 16-byte LDS read.  T follows the same column order and lives in
// NS registers per lane for the whole tile.
//
// src lives in LDS in a split layout: each 16-word block is stored as two
// 8-word halves, the first halves of all blocks in one region and the second
// halves in another R words further on,
//     win_at(m, R) = 8 (m / 16) + m % 8 + R ((m / 8) % 2),   R % 32 == 16.
// The banks of gfx950 (measured with the LDS bank-conflict counters): a
// 16-byte read is served 32 lanes at a time over 128 four-byte banks, a
// 16-byte write 8 lanes at a time over 32 banks, a 4-byte access 32 lanes at a
// time over 32 banks.  The A reads of a step (lanes kk = 0, 1 over 16
// consecutive blocks, and kk = 2, 3) are then one contiguous 512-byte run of a
// region each, the B-operand style 4-byte reads of two consecutive blocks
// (lanes 0-15 and 16-31) fall on opposite 16-bank halves (R % 32 == 16), and
// a step's address is the lane's base plus a constant (an immediate offset).
// ---------------------------------------------------------------------------
typedef float nsq_f32x4_t __attribute__((ext_vector_type(4)));

__host__ __device__ __forceinline__ constexpr int win_at(int m, int R) {
  return 8 * (m >> 4) + (m & 7) + R * ((m >> 3) & 1);
}
// Region stride for a window of count elements: the smallest R >= 8 ceil(count / 16) with R % 32 == 16.
__host__ __device__ constexpr int win_half(int count) { return ((8 * ((count + 15) / 16) + 15) / 32) * 32 + 16; }
// LDS words of such a window.
__host__ __device__ constexpr int win_words(int count) { return 2 * win_half(count); }
// Elements P .. P+7 of a split-layout window (P % 4 == 0) as two 16-byte
// writes.  Odd lanes write their upper four first, so that the 8 lanes of a
// write phase (lane stride 8 elements) cover the 32 banks once.
// (Per-value selects: a select of whole float4s is lowered through scratch
// memory.)
__device__ __forceinline__ void win_store8(float* win, int R, int P, const float (&v)[8]) {
  const bool sw = (threadIdx.x & 1) != 0;
  const float4 first = make_float4(sw ? v[4] : v[0], sw ? v[5] : v[1], sw ? v[6] : v[2], sw ? v[7] : v[3]);
  const float4 second = make_float4(sw ? v[0] : v[4], sw ? v[1] : v[5], sw ? v[2] : v[6], sw ? v[3] : v[7]);
  *reinterpret_cast<float4*>(win + win_at(P + (sw ? 4 : 0), R)) = first;
  *reinterpret_cast<float4*>(win + win_at(P + (sw ? 0 : 4), R)) = second;
}

// Steps for K taps: 4*NS >= K + 15 window columns, NS a multiple of 4.
template <int NS>
struct ToeplitzMfma {
  static_assert(NS % 4 == 0 && NS >= 4, "ToeplitzMfma: NS must be a multiple of 4");
  static constexpr int KMAX = 4 * NS - 15;  // largest tap count this NS covers
  float b[NS];
  // wl: the K taps in LDS (conv orientation: y[n] = sum_j wl[j] src[n + j]).
  // last_add is added to tap K-1 (a skip term c * src[n + K - 1] folded into
  // the band).
  // shift: zero taps prepended to the band (tap j of the band is wl[j - shift]);
  // first_add joins tap 0 (a skip term c * src[n] of a correlation).
  __device__ __forceinline__ void load_weights(const float* wl, int K, float last_add = 0.f, int shift = 0,
                                               float first_add = 0.f) {
    const int l = int(threadIdx.x) & 63, kk = l >> 4, i = l & 15;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int j = 16 * (s >> 2) + 4 * kk + (s & 3) - i - shift;
      const bool ok = j >= 0 && j < K;
      const float v = wl[ok ? j : 0] + (j == K - 1 ? last_add : 0.f) + (j == 0 ? first_add : 0.f);
      b[s] = ok ? v : 0.f;
    }
  }
  // Lane base of the A reads: element 16 (a0 + a) + 4 kk of the window (step
  // group q adds 8 q words).
  __device__ __forceinline__ static const float* a_base(const float* srcp, int R, int a0) {
    const int l = int(threadIdx.x) & 63, kk = l >> 4, a = l & 15;
    return srcp + 8 * (a0 + a) + 4 * (kk & 1) + R * (kk >> 1);
  }
  // The lane's four outputs of the 16 blocks starting at block a0:
  // out[r] = y of block a0 + 4 (l / 16) + r, position l % 16 in the block.
  // srcp: src in the split layout with region stride R; reads src[16 a0,
  // 16 (a0 + 16) + 4 NS - 16).
  __device__ __forceinline__ nsq_f32x4_t run(const float* srcp, int R, int a0) const {
    const float* p = a_base(srcp, R, a0);
    nsq_f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < NS / 4; ++q) {
      const float4 v = *reinterpret_cast<const float4*>(p + 8 * q);
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(v.x, b[4 * q + 0], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(v.y, b[4 * q + 1], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(v.z, b[4 * q + 2], c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(v.w, b[4 * q + 3], c, 0, 0, 0);
    }
    return c;
  }
  // Two M-tiles (blocks a0.. and a1..) with their steps interleaved: two
  // independent accumulation chains keep the matrix pipeline busy.
  __device__ __forceinline__ void run2(const float* srcp, int R, int a0, int a1, nsq_f32x4_t& c0,
                                       nsq_f32x4_t& c1) const {
    const float* p0 = a_base(srcp, R, a0);
    const float* p1 = a_base(srcp, R, a1);
    c0 = nsq_f32x4_t{0.f, 0.f, 0.f, 0.f};
    c1 = nsq_f32x4_t{0.f, 0.f, 0.f, 0.f};
    // operands of step group q+1 are read before the MFMAs of group q issue
    float4 un = *reinterpret_cast<const float4*>(p0);
    float4 vn = *reinterpret_cast<const float4*>(p1);
#pragma unroll
    for (int q = 0; q < NS / 4; ++q) {
      const float4 u = un, v = vn;
      if (q + 1 < NS / 4) {
        un = *reinterpret_cast<const float4*>(p0 + 8 * (q + 1));
        vn = *reinterpret_cast<const float4*>(p1 + 8 * (q + 1));
      }
      c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(u.x, b[4 * q + 0], c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(v.x, b[4 * q + 0], c1, 0, 0, 0);
      c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(u.y, b[4 * q + 1], c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(v.y, b[4 * q + 1], c1, 0, 0, 0);
      c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(u.z, b[4 * q + 2], c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(v.z, b[4 * q + 2], c1, 0, 0, 0);
      c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(u.w, b[4 * q + 3], c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(v.w, b[4 * q + 3], c1, 0, 0, 0);
    }
  }
};

// ---------------------------------------------------------------------------
// The same banded Toeplitz product on v_mfma_f32_16x16x32_bf16, for 16-bit
// I/O: src and the taps are split into bf16 halves, v = hi + lo with hi =
// bf16(v) and lo = bf16(v - hi) (16 mantissa bits together), and each 32-column
// step runs three products hi*hi + hi*lo + lo*hi with fp32 accumulation: a
// product's relative error is ~2^-17 (the dropped lo*lo term and lo's rounding),
// far below the 2^-9 of the 16-bit output it feeds, at 16x the fp32 MFMA rate
// per product.  Lane layout (checked on MI355X with integer operands): lane l
// supplies A[l % 16][8 (l / 16) + e] and B[8 (l / 16) + e][l % 16], e < 8, and
// receives D[4 (l / 16) + r][l % 16] -- the accumulator of the fp32 form.
// src halves are plain bf16 arrays: a lane's 8 values of one step are one
// 16-byte read, and the 32 lanes of a read phase (kk = 0, 1 over 16
// consecutive blocks) read one contiguous 512-byte run: no bank conflicts.
// ---------------------------------------------------------------------------
typedef __bf16 nsq_bf16x8_t __attribute__((ext_vector_type(8)));

// v = hi + lo (bf16 halves, round to nearest even each).
__device__ __forceinline__ void split_bf16(float v, __bf16& hi, __bf16& lo) {
  hi = static_cast<__bf16>(v);
  lo = static_cast<__bf16>(v - static_cast<float>(hi));
}

// S32 steps of 32 window columns: 32 * S32 >= K + 15.
template <int S32>
struct ToeplitzMfmaBf16 {
  nsq_bf16x8_t bh[S32], bl[S32];
  // As ToeplitzMfma::load_weights: tap j of the band is wl[j - shift], tap K-1
  // of wl gets last_add; T[t][i] = band[t - i], t = 32 s + 8 (l / 16) + e.
  __device__ __forceinline__ void load_weights(const float* wl, int K, float last_add = 0.f, int shift = 0) {
    const int l = int(threadIdx.x) & 63, kk = l >> 4, i = l & 15;
#pragma unroll
    for (int s = 0; s < S32; ++s) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = 32 * s + 8 * kk + e - i - shift;
        const bool ok = j >= 0 && j < K;
        const float v = ok ? wl[ok ? j : 0] + (j == K - 1 ? last_add : 0.f) : 0.f;
        __bf16 h, lo;
        split_bf16(v, h, lo);
        bh[s][e] = h;
        bl[s][e] = lo;
      }
    }
  }
  // Two M-tiles (blocks a0.. and a1..) of the bf16 src halves zh, zl:
  // c = the lane's four outputs of each (as ToeplitzMfma::run2).
  __device__ __forceinline__ void run2(const __bf16* zh, const __bf16* zl, int a0, int a1, nsq_f32x4_t& c0,
                                       nsq_f32x4_t& c1) const {
    const int l = int(threadIdx.x) & 63, kk = l >> 4, a = l & 15;
    const int o0 = 16 * (a0 + a) + 8 * kk, o1 = 16 * (a1 + a) + 8 * kk;
    c0 = nsq_f32x4_t{0.f, 0.f, 0.f, 0.f};
    c1 = nsq_f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < S32; ++s) {
      const nsq_bf16x8_t h0 = *reinterpret_cast<const nsq_bf16x8_t*>(zh + o0 + 32 * s);
      const nsq_bf16x8_t h1 = *reinterpret_cast<const nsq_bf16x8_t*>(zh + o1 + 32 * s);
      const nsq_bf16x8_t g0 = *reinterpret_cast<const nsq_bf16x8_t*>(zl + o0 + 32 * s);
      const nsq_bf16x8_t g1 = *reinterpret_cast<const nsq_bf16x8_t*>(zl + o1 + 32 * s);
      c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h0, bh[s], c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h1, bh[s], c1, 0, 0, 0);
      c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h0, bl[s], c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(h1, bl[s], c1, 0, 0, 0);
      c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(g0, bh[s], c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(g1, bh[s], c1, 0, 0, 0);
    }
  }
};
// bf16 steps for the fp32 form's NS (12, 20, 36, 68 -> 2, 3, 5, 9): covers
// K <= 4 NS - 15 taps plus up to 7 leading zero taps.
template <int NS>
constexpr int bf16_steps() { return (NS + 4) / 8; }

// Tile geometry of the MFMA path: kConvTile outputs = kConvTile / 16 blocks,
// in M-tiles of 16 blocks spread over the workgroup's waves.
constexpr int kMfmaBlocks = kConvTile / 16;
constexpr int kMfmaTiles = kMfmaBlocks / 16;
constexpr int kConvWaves = kConvThreads / 64;
static_assert(kMfmaTiles % kConvWaves == 0, "MFMA conv: M-tiles per wave");
// src words read by a tile with NS steps (window of the last block).
template <int NS>
constexpr int mfma_src_count() { return kConvTile + 4 * NS - 16; }

// Smallest supported step count for K taps (0: use the FMA path).
inline int mfma_steps_for(int K) {
  if (K < 16) return 0;
  if (K <= ToeplitzMfma<12>::KMAX) return 12;
  if (K <= ToeplitzMfma<20>::KMAX) return 20;
  if (K <= ToeplitzMfma<36>::KMAX) return 36;
  return 68;  // K <= 257
}

// Samples x[n - 4 + i], i < 12, of one row as raw bits.  AL (16-bit types:
// len % 8 == 0; fp32: len % 4 == 0; 16-byte aligned rows): n is a multiple of
// 8 and the window is three aligned vector loads that lie wholly inside or
// wholly outside [0, len); otherwise twelve element loads.  Positions before
// the row read as zero (offset 2^31, see RowBuf::elem_halo).
template <int DT, bool AL>
struct Win12 {
  static constexpr bool HALF = DT != NSQ_DTYPE_F32;
  static constexpr int W = (HALF && AL) ? 6 : 12;
  uint32_t w[W];
  __device__ __forceinline__ void load(const RowBuf<DT, false>& rb, int n) {
    if constexpr (AL) {
      constexpr int ES = HALF ? 2 : 4;
      int off_h = n < 4 ? int(0x80000000u) : (n - 4) * ES;
      asm volatile("" : "+v"(off_h));
      const int off_m = n * ES;
      if constexpr (HALF) {
        const auto h = __builtin_amdgcn_raw_buffer_load_b64(rb.r, off_h, 0, 0);
        const auto m = __builtin_amdgcn_raw_buffer_load_b128(rb.r, off_m, 0, 0);
        w[0] = h[0]; w[1] = h[1];
        w[2] = m[0]; w[3] = m[1]; w[4] = m[2]; w[5] = m[3];
      } else {
        const auto h = __builtin_amdgcn_raw_buffer_load_b128(rb.r, off_h, 0, 0);
        const auto m0 = __builtin_amdgcn_raw_buffer_load_b128(rb.r, off_m, 0, 0);
        const auto m1 = __builtin_amdgcn_raw_buffer_load_b128(rb.r, off_m + 16, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) { w[i] = h[i]; w[4 + i] = m0[i]; w[8 + i] = m1[i]; }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 12; ++i) w[i] = rb.elem_halo_bits(n - 4 + i);
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
