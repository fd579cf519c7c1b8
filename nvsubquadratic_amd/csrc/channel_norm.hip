// Hyena's output epilogue as one pass over HBM: the second gate, the RMSNorm
// over channels and the channels-first -> channels-last rearrange
// (nvsubquadratic/modules/hyena_nd.py:570 y * act2(v), :573-580 output_norm on
// y.movedim(1, -1), :583 rearrange "b c ... -> b ... c"; the norm is
// nvsubquadratic/modules/rms_norm.py:71-77 _rmsnorm_pytorch, or its
// channels-first twin rms_norm_channel_first.py:71-80, which is the same
// arithmetic along dim 1).  The same pass with the first gate and a
// channels-first output is the pixelhyena_norm site (hyena_nd.py:546-556,
// z = q * act1(k) normalised over channels).
//
//   u[b,c,s]   = round(y * round(act(v)))           (y alone without a gate)
//   r[b,s]     = rsqrt(mean_c u[b,c,s]^2 + eps)     (fp32)
//   out[b,s,c] = round(w[c] * (u[b,c,s] * r[b,s]))  (or out[b,c,s])
//
// Data: y, v, dy, dv are [B, C, S] (S the flattened spatial axes), out and
// dout [B, S, C] or [B, C, S]; w and dw fp32 [C].  A workgroup owns a tile of
// TS consecutive positions of one batch row and all C channels, staged in LDS
// as fp32 with an odd row stride (TS + 1): the channels-first sides are read
// and written as runs of TS positions per channel (lanes along s), the
// channels-last side as runs of C channels per position (lanes along c), and
// the sum over channels is a tree over the TS-wide lane groups.  Tiles that
// share 128-byte lines of the channels-first rows sit on one XCD (the
// workgroup index is remapped so that XCD x = blockIdx % 8 takes a contiguous
// range of tiles), so a line is fetched from HBM once per XCD's L2.
//
// Backward, per tile: recompute u and r, stage dout, m[s] = mean_c(w dout
// xhat), du = r (w dout - xhat m) rounded to the I/O dtype (the reference's
// fp32 upcast hands its gradient back in that dtype), then the gate's
// adjoint: dy = round(du * round(act(v))), dv = round(round(du * y) act'(v)).
// dw = sum over positions of dout * xhat: each workgroup walks every nwg-th
// tile, sums its share per channel in LDS (each channel owned by one
// thread), writes one partial row, and a second kernel adds the rows in a
// fixed order (deterministic).
//
// LayerNorm mode (torch.nn.LayerNorm(C) at the pixelhyena_norm site, the
// reference's configs' other choice there; applied to z.movedim(1, -1) as
// hyena_nd.py:551-556 does): mu[b,s] = mean_c u, r[b,s] = rsqrt(mean_c (u -
// mu)^2 + eps) (the mean first, then the squared deviations from the tile
// kept in LDS), out = round(w[c] ((u - mu) r) + bias[c]); backward with xhat =
// (u - mu) r and g = w dout: du = r (g - mean_c g - xhat mean_c(g xhat)),
// dw = sum dout xhat, dbias = sum dout (two rows of partials per workgroup).
//
// L2 mode (the QK-norm, nvsubquadratic/utils/qk_norm.py L2Norm: F.normalize(x,
// p=2, dim=channels, eps)): n[b,s] = max(round(sqrt(sum_c u^2)), eps) (torch's
// norm of a 16-bit tensor returns that dtype), out = round(u / n), no weight;
// backward du = (dout - xhat sum_c(dout xhat)) / n, or dout / n where n was
// clamped to eps (the clamp passes no gradient to the norm).
#include "gate.h"
#include "nsq_common.h"

#include <initializer_list>

namespace nsq {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxWG = 512;  // backward workgroups (partial dw rows): two per CU

// workgroup index -> logical index, consecutive logical indices on one XCD
__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t n) {
  if (n % 8 != 0) return bid;
  return (bid % 8) * (n / 8) + bid / 8;
}

// VW consecutive elements as floats (VW * sizeof(T) == 16: one 16-byte access; VW == 1: one element)
template <int DT, int VW>
__device__ __forceinline__ void ld_vec(const typename Elem<DT>::T* p, int64_t i, float (&o)[VW]) {
  using T = typename Elem<DT>::T;
  if constexpr (VW == 1) {
    o[0] = Elem<DT>::load(p, i);
  } else {
    static_assert(VW * sizeof(T) == 16, "16-byte vectors");
    const uint4 u = *reinterpret_cast<const uint4*>(p + i);
    const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
    for (int k = 0; k < VW; ++k) o[k] = Elem<DT>::load(e, k);
  }
}

template <int DT, int VW>
__device__ __forceinline__ void st_vec(typename Elem<DT>::T* p, int64_t i, const float (&o)[VW]) {
  using T = typename Elem<DT>::T;
  if constexpr (VW == 1) {
    Elem<DT>::store(p, i, o[0]);
  } else {
    uint4 u;
    T* e = reinterpret_cast<T*>(&u);
#pragma unroll
    for (int k = 0; k < VW; ++k) Elem<DT>::store(e, k, o[k]);
    *reinterpret_cast<uint4*>(p + i) = u;
  }
}

// Channels-first side: lane (lr, g) covers positions lr*VW .. lr*VW+VW-1 of the
// tile and channels g, g + G, ...; a thread issues the loads of kNB channels
// before it uses any of them.
template <int VW>
struct CfMap {
  static constexpr int kNB = VW == 1 ? 8 : 4;
  int LPR, G, lr, g;
  __device__ __forceinline__ CfMap(int TS) {
    LPR = TS / VW;
    G = kThreads / LPR;
    lr = threadIdx.x % LPR;
    g = threadIdx.x / LPR;
  }
};

// Norms over channels (the `mode` argument of the kernels).
enum { CHN_RMS = 0, CHN_L2 = 1, CHN_LN = 2 };

// Phase shared by both directions: u into U[c][s] (zero past S), per-position
// r = rsqrt(mean u^2 + eps) (RMS), 1 / max(round(||u||), eps) (L2) or
// rsqrt(mean (u - mu)^2 + eps) (LN, with U then holding u - mu) into rs[];
// L2 with cl: cl[s] = 0 where the norm was clamped to eps, else 1.  red holds
// G x TS partial sums.
template <int DT, int VW>
__device__ __forceinline__ void load_tile_u(const typename Elem<DT>::T* __restrict__ y,
                                            const typename Elem<DT>::T* __restrict__ v, bool gated, int act,
                                            int64_t rowbase, int C, int64_t S, int64_t s0, int TS, float eps,
                                            float* U, float* red, float* rs, int mode = CHN_RMS,
                                            float* cl = nullptr) {
#pragma clang fp contract(off)
  const CfMap<VW> m(TS);
  constexpr int NB = CfMap<VW>::kNB;
  const int ld = TS + 1, p0 = m.lr * VW;
  const int64_t pos = s0 + p0;
  const bool ok = pos < S;  // S is a multiple of VW: the whole vector is in or out
  float ss[VW];
#pragma unroll
  for (int k = 0; k < VW; ++k) ss[k] = 0.f;
  for (int c0 = m.g; c0 < C; c0 += m.G * NB) {
    float yv[NB][VW], vv[NB][VW];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int c = c0 + j * m.G;
      const int64_t i = rowbase + int64_t(c) * S + pos;
      if (ok && c < C) {
        ld_vec<DT, VW>(y, i, yv[j]);
        if (gated) ld_vec<DT, VW>(v, i, vv[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int c = c0 + j * m.G;
      if (c < C) {
#pragma unroll
        for (int k = 0; k < VW; ++k) {
          float u = 0.f;
          if (ok) u = gated ? Elem<DT>::round(yv[j][k] * Elem<DT>::round(gate_act(act, vv[j][k]))) : yv[j][k];
          U[c * ld + p0 + k] = u;
          ss[k] = mode == CHN_LN ? ss[k] + u : fmaf(u, u, ss[k]);
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < VW; ++k) red[m.g * TS + p0 + k] = ss[k];
  __syncthreads();
  if (threadIdx.x < TS) {
    float sum = 0.f;
    for (int k = 0; k < m.G; ++k) sum += red[k * TS + threadIdx.x];
    if (mode == CHN_L2) {
      const float n = Elem<DT>::round(sqrtf(sum));
      rs[threadIdx.x] = 1.f / fmaxf(n, eps);
      if (cl) cl[threadIdx.x] = n < eps ? 0.f : 1.f;
    } else if (mode == CHN_LN) {
      rs[threadIdx.x] = sum / float(C);  // the mean, until the second sweep
    } else {
      rs[threadIdx.x] = rsqrtf(sum * (1.f / float(C)) + eps);
    }
  }
  __syncthreads();
  if (mode == CHN_LN) {  // second sweep over the tile: U -= mu, sum of squared deviations
    float dd[VW];
#pragma unroll
    for (int k = 0; k < VW; ++k) dd[k] = 0.f;
    for (int c = m.g; c < C; c += m.G) {
#pragma unroll
      for (int k = 0; k < VW; ++k) {
        const float d = U[c * ld + p0 + k] - rs[p0 + k];
        U[c * ld + p0 + k] = d;
        dd[k] = fmaf(d, d, dd[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < VW; ++k) red[m.g * TS + p0 + k] = dd[k];
    __syncthreads();
    if (threadIdx.x < TS) {
      float sum = 0.f;
      for (int k = 0; k < m.G; ++k) sum += red[k * TS + threadIdx.x];
      rs[threadIdx.x] = rsqrtf(sum * (1.f / float(C)) + eps);
    }
    __syncthreads();
  }
}

// Channels-last side: item q = (s, cv), s = q mod TS fastest (consecutive lanes
// read consecutive LDS words), cv a run of VW channels (one 16-byte access).
template <int DT, int VW, int MODE>
__global__ __launch_bounds__(kThreads) void chnorm_fwd_kernel(const typename Elem<DT>::T* __restrict__ y,
                                                              const typename Elem<DT>::T* __restrict__ v,
                                                              const float* __restrict__ w,
                                                              const float* __restrict__ bias,
                                                              typename Elem<DT>::T* __restrict__ out, int C,
                                                              int64_t S, int TS, int64_t tiles_per_b, int64_t ntiles,
                                                              float eps, int gated, int act, int out_blh) {
#pragma clang fp contract(off)
  constexpr int mode = MODE;  // a compile-time norm: RMS / L2 kernels carry no LayerNorm code
  extern __shared__ float smem[];
  const int ld = TS + 1;
  float* U = smem;
  float* red = U + C * ld;
  float* rs = red + kThreads * VW;
  const int64_t tile = xcd_remap(blockIdx.x, ntiles);
  const int64_t b = tile / tiles_per_b, s0 = (tile % tiles_per_b) * TS;
  const int64_t rowbase = b * C * S;
  load_tile_u<DT, VW>(y, v, gated != 0, act, rowbase, C, S, s0, TS, eps, U, red, rs, mode);
  const int t = threadIdx.x;
  const int nval = int(S - s0 < TS ? S - s0 : TS);
  // LN: U holds u - mu; the bias is added after the scale (torch's layer_norm order)
  auto norm_out = [&](int c, int s) {
    const float o = (w ? w[c] : 1.f) * (U[c * ld + s] * rs[s]);
    return (mode == CHN_LN && bias) ? o + bias[c] : o;
  };
  if (out_blh) {
    const int nitems = TS * (C / VW);
    for (int q = t; q < nitems; q += kThreads) {
      const int s = q % TS, c = (q / TS) * VW;
      if (s < nval) {
        float o[VW];
#pragma unroll
        for (int k = 0; k < VW; ++k) o[k] = norm_out(c + k, s);
        st_vec<DT, VW>(out, (b * S + s0 + s) * int64_t(C) + c, o);
      }
    }
  } else {
    const CfMap<VW> m(TS);
    const int p0 = m.lr * VW;
    if (p0 < nval)
      for (int c = m.g; c < C; c += m.G) {
        float o[VW];
#pragma unroll
        for (int k = 0; k < VW; ++k) o[k] = norm_out(c, p0 + k);
        st_vec<DT, VW>(out, rowbase + int64_t(c) * S + s0 + p0, o);
      }
  }
}

template <int DT, int VW, int MODE>
__global__ __launch_bounds__(kThreads) void chnorm_bwd_kernel(
    const typename Elem<DT>::T* __restrict__ dout, const typename Elem<DT>::T* __restrict__ y,
    const typename Elem<DT>::T* __restrict__ v, const float* __restrict__ w, typename Elem<DT>::T* __restrict__ dy,
    typename Elem<DT>::T* __restrict__ dv, float* __restrict__ dw_part, float* __restrict__ db_part, int C, int64_t S,
    int TS, int64_t tiles_per_b, int64_t ntiles, float eps, int gated, int act, int in_blh) {
#pragma clang fp contract(off)
  constexpr int mode = MODE;
  extern __shared__ float smem[];
  const int ld = TS + 1;
  float* U = smem;                  // u, then xhat
  float* D = U + C * ld;            // dout (fp32)
  float* gacc = D + C * ld;         // dw share of this workgroup
  float* red = gacc + C;            // G x TS partial sums
  float* rs = red + kThreads * VW;  // r per position
  float* ms = rs + TS;              // mean_c(w dout xhat) (RMS, LN) or sum_c(dout xhat) unless clamped (L2)
  float* cl = ms + TS;              // L2: 0 where the norm was clamped; LN: mean_c(w dout)
  float* gaccb = cl + TS;           // LN: dbias share of this workgroup
  const int t = threadIdx.x;
  const CfMap<VW> m(TS);
  constexpr int NB = CfMap<VW>::kNB;
  const int p0 = m.lr * VW;
  const int64_t wg = xcd_remap(blockIdx.x, gridDim.x);
  for (int c = t; c < C; c += kThreads) gacc[c] = 0.f;
  if (mode == CHN_LN)
    for (int c = t; c < C; c += kThreads) gaccb[c] = 0.f;
  // tiles wg, wg + nwg, ...: the workgroups of one XCD (consecutive wg) work on
  // neighbouring tiles at the same time, so the 128-byte lines they share are
  // read from HBM once into that XCD's L2
  for (int64_t tile = wg; tile < ntiles; tile += gridDim.x) {
    const int64_t b = tile / tiles_per_b, s0 = (tile % tiles_per_b) * TS;
    const int64_t rowbase = b * C * S;
    const int nval = int(S - s0 < TS ? S - s0 : TS);
    load_tile_u<DT, VW>(y, v, gated != 0, act, rowbase, C, S, s0, TS, eps, U, red, rs, mode, cl);
    // dout into D[c][s] (zero past S)
    if (in_blh) {
      const int nitems = TS * (C / VW);
      for (int q0 = t; q0 < nitems; q0 += kThreads * NB) {
        float d[NB][VW];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int q = q0 + j * kThreads, s = q % TS, c = (q / TS) * VW;
          if (q < nitems && s < nval) {
            ld_vec<DT, VW>(dout, (b * S + s0 + s) * int64_t(C) + c, d[j]);
          } else {
#pragma unroll
            for (int k = 0; k < VW; ++k) d[j][k] = 0.f;
          }
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int q = q0 + j * kThreads, s = q % TS, c = (q / TS) * VW;
          if (q < nitems)
#pragma unroll
            for (int k = 0; k < VW; ++k) D[(c + k) * ld + s] = d[j][k];
        }
      }
    } else {
      for (int c0 = m.g; c0 < C; c0 += m.G * NB) {
        float d[NB][VW];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int c = c0 + j * m.G;
          if (p0 < nval && c < C) {
            ld_vec<DT, VW>(dout, rowbase + int64_t(c) * S + s0 + p0, d[j]);
          } else {
#pragma unroll
            for (int k = 0; k < VW; ++k) d[j][k] = 0.f;
          }
        }
#pragma unroll
        for (int j = 0; j < NB; ++j)
          if (c0 + j * m.G < C)
#pragma unroll
            for (int k = 0; k < VW; ++k) D[(c0 + j * m.G) * ld + p0 + k] = d[j][k];
      }
    }
    __syncthreads();
    // xhat in place of u (LN: of u - mu); per-position sums of (w dout) xhat and (LN) of w dout
    float sg[VW];
    {
      float dot[VW];
#pragma unroll
      for (int k = 0; k < VW; ++k) dot[k] = sg[k] = 0.f;
      for (int c = m.g; c < C; c += m.G) {
        const float wc = w ? w[c] : 1.f;
#pragma unroll
        for (int k = 0; k < VW; ++k) {
          const float xh = U[c * ld + p0 + k] * rs[p0 + k];
          U[c * ld + p0 + k] = xh;
          const float g = wc * D[c * ld + p0 + k];
          dot[k] = fmaf(g, xh, dot[k]);
          sg[k] += g;
        }
      }
#pragma unroll
      for (int k = 0; k < VW; ++k) red[m.g * TS + p0 + k] = dot[k];
    }
    __syncthreads();
    if (t < TS) {
      float sum = 0.f;
      for (int k = 0; k < m.G; ++k) sum += red[k * TS + t];
      ms[t] = mode == CHN_L2 ? sum * cl[t] : sum * (1.f / float(C));
    }
    if (mode == CHN_LN) {  // second reduction, through the same buffer
      __syncthreads();
#pragma unroll
      for (int k = 0; k < VW; ++k) red[m.g * TS + p0 + k] = sg[k];
      __syncthreads();
      if (t < TS) {
        float sum = 0.f;
        for (int k = 0; k < m.G; ++k) sum += red[k * TS + t];
        cl[t] = sum * (1.f / float(C));
      }
    }
    // dw (and LN's dbias) share: each channel summed over the tile's positions by its owner thread
    for (int c = t; c < C && w; c += kThreads) {
      float a = gacc[c];
      for (int s = 0; s < TS; ++s) a = fmaf(D[c * ld + s], U[c * ld + s], a);
      gacc[c] = a;
    }
    if (mode == CHN_LN && db_part)
      for (int c = t; c < C; c += kThreads) {
        float a = gaccb[c];
        for (int s = 0; s < TS; ++s) a += D[c * ld + s];
        gaccb[c] = a;
      }
    __syncthreads();
    if (p0 < nval) {
      for (int c0 = m.g; c0 < C; c0 += m.G * NB) {
        float yv[NB][VW], vv[NB][VW];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int c = c0 + j * m.G;
          const int64_t i = rowbase + int64_t(c) * S + s0 + p0;
          if (gated && c < C) {
            ld_vec<DT, VW>(y, i, yv[j]);
            ld_vec<DT, VW>(v, i, vv[j]);
          }
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const int c = c0 + j * m.G;
          if (c < C) {
            const float wc = w ? w[c] : 1.f;
            float o0[VW], o1[VW];
#pragma unroll
            for (int k = 0; k < VW; ++k) {
              const float xh = U[c * ld + p0 + k];
              const float g = wc * D[c * ld + p0 + k];
              const float du = Elem<DT>::round(rs[p0 + k] * ((mode == CHN_LN ? g - cl[p0 + k] : g) - xh * ms[p0 + k]));
              if (gated) {
                o0[k] = du * Elem<DT>::round(gate_act(act, vv[j][k]));
                o1[k] = Elem<DT>::round(du * yv[j][k]) * gate_dact(act, vv[j][k]);
              } else {
                o0[k] = du;
                o1[k] = 0.f;
              }
            }
            const int64_t i = rowbase + int64_t(c) * S + s0 + p0;
            st_vec<DT, VW>(dy, i, o0);
            if (gated) st_vec<DT, VW>(dv, i, o1);
          }
        }
      }
    }
    __syncthreads();  // U and D are reused by the next tile
  }
  if (dw_part)
    for (int c = t; c < C; c += kThreads) dw_part[wg * C + c] = gacc[c];
  if (mode == CHN_LN && db_part)
    for (int c = t; c < C; c += kThreads) db_part[wg * C + c] = gaccb[c];
}

// dw[c] = sum over the partial rows: a workgroup takes 64 channels, its four
// lane groups rows r = 4k + q (q = 0..3, four running sums each over r mod 16),
// combined in a fixed order (deterministic).
__global__ __launch_bounds__(kThreads) void chnorm_dw_reduce_kernel(const float* __restrict__ part,
                                                                    float* __restrict__ dw, int C, int64_t rows) {
  __shared__ float acc[4][64];
  const int t = threadIdx.x, q = t / 64;
  const int64_t c = int64_t(blockIdx.x) * 64 + (t % 64);
  float a[4] = {0.f, 0.f, 0.f, 0.f};
  if (c < C) {
    int64_t r = q;
    for (; r + 12 < rows; r += 16) {
#pragma unroll
      for (int j = 0; j < 4; ++j) a[j] += part[(r + 4 * j) * C + c];
    }
    for (; r < rows; r += 4) a[0] += part[r * C + c];
  }
  acc[q][t % 64] = (a[0] + a[1]) + (a[2] + a[3]);
  __syncthreads();
  if (q == 0 && c < C) dw[c] = (acc[0][t] + acc[1][t]) + (acc[2][t] + acc[3][t]);
}

size_t fwd_lds(int C, int TS, int VW) { return (size_t(C) * (TS + 1) + size_t(kThreads) * VW + TS) * 4; }
// LN adds the dbias share (C floats).
size_t bwd_lds(int C, int TS, int VW, bool ln = false) {
  return (size_t(C) * (TS + 1) * 2 + C + size_t(kThreads) * VW + 3 * TS + (ln ? C : 0)) * 4;
}
constexpr size_t kLdsPreferred = 64 * 1024;  // leaves room for two or more workgroups per CU
constexpr size_t kLdsMax = 160 * 1024;       // gfx950's LDS per workgroup
// Tile width: the widest of 64, 32, ..., 4 positions whose LDS fits 64 KB, else
// 4 positions up to the whole LDS (wide C), else 0 (unsupported C).  Sized for
// the widest vector (VW = 8), so the tile does not depend on the vector path.
int pick_ts(int C, bool bwd, bool ln = false) {
  for (int ts = 64; ts >= 4; ts /= 2)
    if ((bwd ? bwd_lds(C, ts, 8, ln) : fwd_lds(C, ts, 8)) <= kLdsPreferred) return ts;
  return (bwd ? bwd_lds(C, 4, 8, ln) : fwd_lds(C, 4, 8)) <= kLdsMax ? 4 : 0;
}
struct BwdPlan {
  int TS;
  int64_t tiles_per_b, ntiles, nwg;
};
BwdPlan bwd_plan(int64_t B, int C, int64_t S, bool ln = false) {
  BwdPlan p{};
  p.TS = pick_ts(C, true, ln);
  if (!p.TS) return p;
  p.tiles_per_b = ceil_div(S, int64_t(p.TS));
  p.ntiles = B * p.tiles_per_b;
  // a multiple of 8 workgroups (when there are 8 tiles or more), so the XCD remap applies
  int64_t nwg = p.ntiles < kMaxWG ? p.ntiles : kMaxWG;
  if (nwg >= 8) nwg -= nwg % 8;
  p.nwg = nwg;
  return p;
}
// 16-byte vectors when every run of VW elements the kernel moves is whole and aligned
bool use_vec(int vw, int C, int64_t S, int TS, std::initializer_list<const void*> ptrs) {
  if (S % vw || C % vw || TS % vw) return false;
  for (const void* q : ptrs)
    if (q && (reinterpret_cast<uintptr_t>(q) & 15)) return false;
  return true;
}
template <class K>
void allow_lds(K* kernel, size_t lds) {
  if (lds > kLdsPreferred)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                              int(lds));
}
// The kernels take the norm as a template argument.
template <class F>
void with_mode(int mode, F&& f) {
  if (mode == CHN_LN)
    f(std::integral_constant<int, CHN_LN>{});
  else if (mode == CHN_L2)
    f(std::integral_constant<int, CHN_L2>{});
  else
    f(std::integral_constant<int, CHN_RMS>{});
}
template <int DT, int VW>
void launch_fwd_vw(const void* y, const void* v, const float* w, const float* bias, void* out, int64_t B, int C,
                   int64_t S, int TS, float eps, int gated, int act, int out_blh, int mode, hipStream_t st) {
  using T = typename Elem<DT>::T;
  const int64_t tpb = ceil_div(S, int64_t(TS)), nt = B * tpb;
  const size_t lds = fwd_lds(C, TS, VW);
  with_mode(mode, [&](auto mc) {
    constexpr int M = decltype(mc)::value;
    allow_lds(&chnorm_fwd_kernel<DT, VW, M>, lds);
    hipLaunchKernelGGL((chnorm_fwd_kernel<DT, VW, M>), dim3(unsigned(nt)), dim3(kThreads), lds, st, (const T*)y,
                       (const T*)v, w, bias, (T*)out, C, S, TS, tpb, nt, eps, gated, act, out_blh);
  });
}
template <int DT>
void launch_fwd(const void* y, const void* v, const float* w, void* out, int64_t B, int C, int64_t S, float eps,
                int gated, int act, int out_blh, hipStream_t st, int mode = CHN_RMS, const float* bias = nullptr) {
  constexpr int VW = 16 / int(sizeof(typename Elem<DT>::T));
  const int TS = pick_ts(C, false);
  if (use_vec(VW, C, S, TS, {y, v, out}))
    launch_fwd_vw<DT, VW>(y, v, w, bias, out, B, C, S, TS, eps, gated, act, out_blh, mode, st);
  else
    launch_fwd_vw<DT, 1>(y, v, w, bias, out, B, C, S, TS, eps, gated, act, out_blh, mode, st);
}
template <int DT, int VW>
void launch_bwd_vw(const void* dout, const void* y, const void* v, const float* w, void* dy, void* dv, float* part,
                   float* partb, const BwdPlan& p, int C, int64_t S, float eps, int gated, int act, int out_blh,
                   int mode, hipStream_t st) {
  using T = typename Elem<DT>::T;
  const size_t lds = bwd_lds(C, p.TS, VW, mode == CHN_LN);
  with_mode(mode, [&](auto mc) {
    constexpr int M = decltype(mc)::value;
    allow_lds(&chnorm_bwd_kernel<DT, VW, M>, lds);
    hipLaunchKernelGGL((chnorm_bwd_kernel<DT, VW, M>), dim3(unsigned(p.nwg)), dim3(kThreads), lds, st,
                       (const T*)dout, (const T*)y, (const T*)v, w, (T*)dy, (T*)dv, part, partb, C, S, p.TS,
                       p.tiles_per_b, p.ntiles, eps, gated, act, out_blh);
  });
}
// part: nwg rows of C dw partials (LN: then nwg rows of dbias partials, partb).
template <int DT>
void launch_bwd(const void* dout, const void* y, const void* v, const float* w, void* dy, void* dv, float* dw,
                float* part, const BwdPlan& p, int64_t B, int C, int64_t S, float eps, int gated, int act,
                int out_blh, hipStream_t st, int mode = CHN_RMS, float* db = nullptr) {
  (void)B;
  constexpr int VW = 16 / int(sizeof(typename Elem<DT>::T));
  float* partb = (mode == CHN_LN && db) ? part + p.nwg * int64_t(C) : nullptr;
  if (use_vec(VW, C, S, p.TS, {dout, y, v, dy, dv}))
    launch_bwd_vw<DT, VW>(dout, y, v, w, dy, dv, part, partb, p, C, S, eps, gated, act, out_blh, mode, st);
  else
    launch_bwd_vw<DT, 1>(dout, y, v, w, dy, dv, part, partb, p, C, S, eps, gated, act, out_blh, mode, st);
  const dim3 rgrid(unsigned(ceil_div(int64_t(C), int64_t(64))));
  if (dw) hipLaunchKernelGGL(chnorm_dw_reduce_kernel, rgrid, dim3(kThreads), 0, st, (const float*)part, dw, C, p.nwg);
  if (partb)
    hipLaunchKernelGGL(chnorm_dw_reduce_kernel, rgrid, dim3(kThreads), 0, st, (const float*)partb, db, C, p.nwg);
}
int check_common(const char* who, int dtype, int64_t B, int C, int64_t S, float eps, int gated, int act) {
  NSQ_CHECK_ARG(dtype == NSQ_DTYPE_F32 || dtype == NSQ_DTYPE_BF16 || dtype == NSQ_DTYPE_F16, "%s: bad dtype %d", who,
                dtype);
  NSQ_CHECK_ARG(B >= 1 && C >= 1 && S >= 1, "%s: sizes must be positive (B=%lld C=%d S=%lld)", who, (long long)B, C,
                (long long)S);
  NSQ_CHECK_ARG(eps >= 0.f, "%s: eps must be >= 0", who);
  NSQ_CHECK_ARG(act == NSQ_GATE_IDENTITY || act == NSQ_GATE_SIGMOID || act == NSQ_GATE_SILU, "%s: bad act %d", who,
                act);
  (void)gated;
  return NSQ_OK;
}

}  // namespace
}  // namespace nsq

extern "C" size_t nsq_channel_rmsnorm_bwd_workspace_bytes(int64_t B, int64_t C, int64_t S) {
  using namespace nsq;
  if (B < 1 || C < 1 || C > 0x7fffffff || S < 1) return 0;
  const BwdPlan p = bwd_plan(B, int(C), S);
  if (!p.TS) return 0;
  return size_t(p.nwg) * size_t(C) * sizeof(float);
}

extern "C" int nsq_channel_rmsnorm_fwd(const void* y, const void* v, const float* w, void* out, int dtype, int64_t B,
                                       int64_t C, int64_t S, float eps, int act, int out_channels_last,
                                       void* stream) {
  using namespace nsq;
  clear_error();
  NSQ_CHECK_ARG(y && w && out, "channel_rmsnorm_fwd: null pointer argument");
  NSQ_CHECK_ARG(C >= 1 && C <= 0x7fffffff, "channel_rmsnorm_fwd: C=%lld out of range", (long long)C);
  const int gated = v != nullptr;
  if (int e = check_common("channel_rmsnorm_fwd", dtype, B, int(C), S, eps, gated, act)) return e;
  const int TS = pick_ts(int(C), false);
  if (TS == 0) {
    set_error("channel_rmsnorm_fwd: C=%lld exceeds the LDS tile (C <= 7781)", (long long)C);
    return NSQ_ERR_UNSUPPORTED;
  }
  NSQ_CHECK_ARG(B * ceil_div(S, int64_t(TS)) <= 0x7fffffff, "channel_rmsnorm_fwd: B*S too large for the grid");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == NSQ_DTYPE_F32)
    launch_fwd<NSQ_DTYPE_F32>(y, v, w, out, B, int(C), S, eps, gated, act, out_channels_last, st);
  else if (dtype == NSQ_DTYPE_BF16)
    launch_fwd<NSQ_DTYPE_BF16>(y, v, w, out, B, int(C), S, eps, gated, act, out_channels_last, st);
  else
    launch_fwd<NSQ_DTYPE_F16>(y, v, w, out, B, int(C), S, eps, gated, act, out_channels_last, st);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

extern "C" int nsq_channel_rmsnorm_bwd(const void* dout, const void* y, const void* v, const float* w, void* dy,
                                       void* dv, float* dw, int dtype, int64_t B, int64_t C, int64_t S, float eps,
                                       int act, int out_channels_last, void* workspace, size_t workspace_bytes,
                                       void* stream) {
  using namespace nsq;
  clear_error();
  NSQ_CHECK_ARG(dout && y && w && dy && dw, "channel_rmsnorm_bwd: null pointer argument");
  NSQ_CHECK_ARG((v == nullptr) == (dv == nullptr), "channel_rmsnorm_bwd: v and dv must be given together");
  NSQ_CHECK_ARG(C >= 1 && C <= 0x7fffffff, "channel_rmsnorm_bwd: C=%lld out of range", (long long)C);
  const int gated = v != nullptr;
  if (int e = check_common("channel_rmsnorm_bwd", dtype, B, int(C), S, eps, gated, act)) return e;
  const BwdPlan p = bwd_plan(B, int(C), S);
  if (p.TS == 0) {
    set_error("channel_rmsnorm_bwd: C=%lld exceeds the LDS tiles (C <= 3536)", (long long)C);
    return NSQ_ERR_UNSUPPORTED;
  }
  const size_t need = size_t(p.nwg) * size_t(C) * sizeof(float);
  NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "channel_rmsnorm_bwd: workspace of %zu bytes needed", need);
  hipStream_t st = (hipStream_t)stream;
  float* part = (float*)workspace;
  if (dtype == NSQ_DTYPE_F32)
    launch_bwd<NSQ_DTYPE_F32>(dout, y, v, w, dy, dv, dw, part, p, B, int(C), S, eps, gated, act, out_channels_last,
                              st);
  else if (dtype == NSQ_DTYPE_BF16)
    launch_bwd<NSQ_DTYPE_BF16>(dout, y, v, w, dy, dv, dw, part, p, B, int(C), S, eps, gated, act, out_channels_last,
                               st);
  else
    launch_bwd<NSQ_DTYPE_F16>(dout, y, v, w, dy, dv, dw, part, p, B, int(C), S, eps, gated, act, out_channels_last,
                              st);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

extern "C" int nsq_channel_l2norm_fwd(const void* x, void* out, int dtype, int64_t B, int64_t C, int64_t S, float eps,
                                      int out_channels_last, void* stream) {
  using namespace nsq;
  clear_error();
  NSQ_CHECK_ARG(x && out, "channel_l2norm_fwd: null pointer argument");
  NSQ_CHECK_ARG(C >= 1 && C <= 0x7fffffff, "channel_l2norm_fwd: C=%lld out of range", (long long)C);
  if (int e = check_common("channel_l2norm_fwd", dtype, B, int(C), S, eps, 0, NSQ_GATE_IDENTITY)) return e;
  const int TS = pick_ts(int(C), false);
  if (TS == 0) {
    set_error("channel_l2norm_fwd: C=%lld exceeds the LDS tile (C <= 7781)", (long long)C);
    return NSQ_ERR_UNSUPPORTED;
  }
  NSQ_CHECK_ARG(B * ceil_div(S, int64_t(TS)) <= 0x7fffffff, "channel_l2norm_fwd: B*S too large for the grid");
  hipStream_t st = (hipStream_t)stream;
  const int oc = out_channels_last;
  if (dtype == NSQ_DTYPE_F32)
    launch_fwd<NSQ_DTYPE_F32>(x, nullptr, nullptr, out, B, int(C), S, eps, 0, NSQ_GATE_IDENTITY, oc, st, 1);
  else if (dtype == NSQ_DTYPE_BF16)
    launch_fwd<NSQ_DTYPE_BF16>(x, nullptr, nullptr, out, B, int(C), S, eps, 0, NSQ_GATE_IDENTITY, oc, st, 1);
  else
    launch_fwd<NSQ_DTYPE_F16>(x, nullptr, nullptr, out, B, int(C), S, eps, 0, NSQ_GATE_IDENTITY, oc, st, 1);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

extern "C" int nsq_channel_l2norm_bwd(const void* dout, const void* x, void* dx, int dtype, int64_t B, int64_t C,
                                      int64_t S, float eps, int out_channels_last, void* stream) {
  using namespace nsq;
  clear_error();
  NSQ_CHECK_ARG(dout && x && dx, "channel_l2norm_bwd: null pointer argument");
  NSQ_CHECK_ARG(C >= 1 && C <= 0x7fffffff, "channel_l2norm_bwd: C=%lld out of range", (long long)C);
  if (int e = check_common("channel_l2norm_bwd", dtype, B, int(C), S, eps, 0, NSQ_GATE_IDENTITY)) return e;
  const BwdPlan p = bwd_plan(B, int(C), S);
  if (p.TS == 0) {
    set_error("channel_l2norm_bwd: C=%lld exceeds the LDS tiles (C <= 3536)", (long long)C);
    return NSQ_ERR_UNSUPPORTED;
  }
  hipStream_t st = (hipStream_t)stream;
  const int oc = out_channels_last;
  if (dtype == NSQ_DTYPE_F32)
    launch_bwd<NSQ_DTYPE_F32>(dout, x, nullptr, nullptr, dx, nullptr, nullptr, nullptr, p, B, int(C), S, eps, 0,
                              NSQ_GATE_IDENTITY, oc, st, 1);
  else if (dtype == NSQ_DTYPE_BF16)
    launch_bwd<NSQ_DTYPE_BF16>(dout, x, nullptr, nullptr, dx, nullptr, nullptr, nullptr, p, B, int(C), S, eps, 0,
                               NSQ_GATE_IDENTITY, oc, st, 1);
  else
    launch_bwd<NSQ_DTYPE_F16>(dout, x, nullptr, nullptr, dx, nullptr, nullptr, nullptr, p, B, int(C), S, eps, 0,
                              NSQ_GATE_IDENTITY, oc, st, 1);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

// LayerNorm over channels (LN mode of the kernels above).
extern "C" size_t nsq_channel_layernorm_bwd_workspace_bytes(int64_t B, int64_t C, int64_t S) {
  using namespace nsq;
  if (B < 1 || C < 1 || C > 0x7fffffff || S < 1) return 0;
  const BwdPlan p = bwd_plan(B, int(C), S, true);
  if (!p.TS) return 0;
  return 2 * size_t(p.nwg) * size_t(C) * sizeof(float);  // dw rows, then dbias rows
}

extern "C" int nsq_channel_layernorm_fwd(const void* y, const void* v, const float* w, const float* b, void* out,
                                         int dtype, int64_t B, int64_t C, int64_t S, float eps, int act,
                                         int out_channels_last, void* stream) {
  using namespace nsq;
  clear_error();
  NSQ_CHECK_ARG(y && out, "channel_layernorm_fwd: null pointer argument");
  NSQ_CHECK_ARG(C >= 1 && C <= 0x7fffffff, "channel_layernorm_fwd: C=%lld out of range", (long long)C);
  const int gated = v != nullptr;
  if (int e = check_common("channel_layernorm_fwd", dtype, B, int(C), S, eps, gated, act)) return e;
  const int TS = pick_ts(int(C), false);
  if (TS == 0) {
    set_error("channel_layernorm_fwd: C=%lld exceeds the LDS tile (C <= 7781)", (long long)C);
    return NSQ_ERR_UNSUPPORTED;
  }
  NSQ_CHECK_ARG(B * ceil_div(S, int64_t(TS)) <= 0x7fffffff, "channel_layernorm_fwd: B*S too large for the grid");
  hipStream_t st = (hipStream_t)stream;
  const int oc = out_channels_last;
  if (dtype == NSQ_DTYPE_F32)
    launch_fwd<NSQ_DTYPE_F32>(y, v, w, out, B, int(C), S, eps, gated, act, oc, st, CHN_LN, b);
  else if (dtype == NSQ_DTYPE_BF16)
    launch_fwd<NSQ_DTYPE_BF16>(y, v, w, out, B, int(C), S, eps, gated, act, oc, st, CHN_LN, b);
  else
    launch_fwd<NSQ_DTYPE_F16>(y, v, w, out, B, int(C), S, eps, gated, act, oc, st, CHN_LN, b);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

extern "C" int nsq_channel_layernorm_bwd(const void* dout, const void* y, const void* v, const float* w, void* dy,
                                         void* dv, float* dw, float* db, int dtype, int64_t B, int64_t C, int64_t S,
                                         float eps, int act, int out_channels_last, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  using namespace nsq;
  clear_error();
  NSQ_CHECK_ARG(dout && y && dy, "channel_layernorm_bwd: null pointer argument");
  NSQ_CHECK_ARG((v == nullptr) == (dv == nullptr), "channel_layernorm_bwd: v and dv must be given together");
  NSQ_CHECK_ARG(w || !dw, "channel_layernorm_bwd: dw needs the weight w");
  NSQ_CHECK_ARG(C >= 1 && C <= 0x7fffffff, "channel_layernorm_bwd: C=%lld out of range", (long long)C);
  const int gated = v != nullptr;
  if (int e = check_common("channel_layernorm_bwd", dtype, B, int(C), S, eps, gated, act)) return e;
  const BwdPlan p = bwd_plan(B, int(C), S, true);
  if (p.TS == 0) {
    set_error("channel_layernorm_bwd: C=%lld exceeds the LDS tiles (C <= 3241)", (long long)C);
    return NSQ_ERR_UNSUPPORTED;
  }
  const size_t need = 2 * size_t(p.nwg) * size_t(C) * sizeof(float);
  float* part = nullptr;
  if (dw || db) {
    NSQ_CHECK_ARG(workspace && workspace_bytes >= need, "channel_layernorm_bwd: workspace of %zu bytes needed", need);
    part = (float*)workspace;
  }
  hipStream_t st = (hipStream_t)stream;
  const int oc = out_channels_last;
  if (dtype == NSQ_DTYPE_F32)
    launch_bwd<NSQ_DTYPE_F32>(dout, y, v, w, dy, dv, dw, part, p, B, int(C), S, eps, gated, act, oc, st, CHN_LN, db);
  else if (dtype == NSQ_DTYPE_BF16)
    launch_bwd<NSQ_DTYPE_BF16>(dout, y, v, w, dy, dv, dw, part, p, B, int(C), S, eps, gated, act, oc, st, CHN_LN,
                               db);
  else
    launch_bwd<NSQ_DTYPE_F16>(dout, y, v, w, dy, dv, dw, part, p, B, int(C), S, eps, gated, act, oc, st, CHN_LN, db);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}
