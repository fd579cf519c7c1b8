// Implicit filter generation (SIREN MLP) for gfx950: the hidden stack.
//
// Semantics: nvsubquadratic/modules/kernels_nd.py:1149-1190 (SIRENKernelND
// without FiLM):
//   a_0[g] = sin(W0 x_g + b0),  a_i[g] = sin(W_i a_{i-1}[g] + b_i) (i = 1..nh),
//   k[h][g] = W_out[h] . a_nh[g] + b_out[h].
// These kernels produce the last activation transposed, A_ext = [a_nh^T; 1]
// ([HD + 1][G]), the filter k = W_out a_nh + b_out straight in the [H][G]
// layout the FFT convs read (siren_readout_fwd_kernel), and the hidden weights'
// gradients from dA = W_out^T gk.  The readout's two gradient products are
// plain library GEMMs (hipBLASLt; the ones row of A_ext gives b_out's), which
// run this shape (K = H, and K = G split in 16 slices) at ~70% of the fp32
// matrix rate.
//
// Design (MI355X):
//  * A wave owns 16 grid points.  Every product is a v_mfma_f32_16x16x4_f32
//    (fp32 in, fp32 accumulate: the reference's fp32 linear layers up to
//    summation order).  Lane l supplies A[l % 16][s] and B[s][l % 16] for
//    k-slot s = l / 16 and receives D[4 (l / 16) + r][l % 16].  The k index
//    of slot s at step kb is K/4 * s + kb, so a lane's operands of one product
//    are K/4 consecutive words of one row (vector loads) and the 16 points'
//    activations (B) stay in registers across every output tile.
//  * The hidden layers run out of a per-wave LDS tile; the forward writes
//    only A_ext (HD + 1 floats per point) to HBM.
//  * Backward: siren_bwd_delta_kernel reads dA for its 16 points, recomputes
//    the layers and back-propagates, writing every layer's activations and
//    deltas transposed ([rows][Gp]); siren_gram_kernel then forms each weight
//    gradient X Y^T and bias row sums over the points as per-chunk partials,
//    reduced in a fixed order (bitwise repeatable).
#include <type_traits>

#include "nsq_common.h"
#include "siren_readout.h"

namespace nsq {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kSirenWaves = 4;  // waves per workgroup, 16 grid points each
constexpr int kSirenThreads = 64 * kSirenWaves;

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Keeps the compiler from moving LDS accesses of one wave across each other;
// the LDS executes a wave's instructions in order, so no barrier is needed
// between lanes of the same wave.
__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Row stride (words) of a per-wave activation tile [16 points][D]: D + 4
// spreads the 16 rows of a B-operand read over the 64 banks.
template <int D>
struct Tile {
  static constexpr int S = D + 4;
  static constexpr int WORDS = 16 * S;
};

// Layer geometry: layer i (i = 1..nh) maps IN -> HD, IN = E for i = 1.
// FiLM (kernels_nd.py:1165-1187, film.py:75): per sample s, film[s][f] holds
// (gamma[HD], beta[HD]) for FiLM slot f; slot f modulates the output of layer
// f + 1 - film_first (layer 0 = the positional embedding, modulated only when
// film_first, which needs E == HD): h = gamma * sin(z) + beta.  film == null:
// no modulation.
struct SirenNet {
  const float* w0;  // [E][d]
  const float* b0;  // [E] or null
  const float* wh;  // packed W_1 [HD][E], W_2.. [HD][HD]
  const float* bh;  // packed [nh][HD] or null
  int d, nh;
  const float* film = nullptr;  // [nb][nfilm][2][HD]
  int film_first = 0;
  __device__ __forceinline__ int nfilm() const { return nh + film_first; }
  // (gamma, beta) of layer L (0 = embedding) for sample s, or nulls
  __device__ __forceinline__ const float* film_of(int s, int L, int HD) const {
    const int f = L - 1 + film_first;
    return (film && f >= 0) ? film + (int64_t(s) * nfilm() + f) * 2 * HD : nullptr;
  }
};

__device__ __forceinline__ const float* layer_w(const SirenNet& n, int i, int E, int HD) {
  return n.wh + (i == 1 ? 0 : int64_t(HD) * E + int64_t(i - 2) * HD * HD);
}

// Coordinates of point g (zeros past G), unrolled over the at most 3 axes.
__device__ __forceinline__ void load_coords(const float* __restrict__ grid, int64_t G, int d, int64_t g, float* x) {
#pragma unroll
  for (int c = 0; c < 3; ++c) x[c] = (g < G && c < d) ? grid[g * d + c] : 0.f;
}

// Pre-activation of embedding feature e: W0[e] . x + b0[e].
__device__ __forceinline__ float embed_pre(const SirenNet& n, int e, const float* x) {
  float z = n.b0 ? n.b0[e] : 0.f;
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    if (c < n.d) z = __builtin_fmaf(n.w0[e * n.d + c], x[c], z);
  }
  return z;
}

// Positional embedding of the wave's 16 points into tile a0 [16][E] (and the
// pre-activation into z0 if given): lane l, point l % 16, features l / 16 + 4t.
template <int E>
__device__ __forceinline__ void pos_embed(const SirenNet& n, const float* __restrict__ grid, int64_t G, int64_t g0,
                                          float* a0, float* z0, const float* fm = nullptr) {
  const int l = int(threadIdx.x) & 63, p = l & 15;
  const int64_t g = g0 + p;
  float x[3];
  load_coords(grid, G, n.d, g, x);
#pragma unroll
  for (int t = 0; t < E / 4; ++t) {
    const int e = (l >> 4) + 4 * t;
    const float z = embed_pre(n, e, x);
    const float sv = sinf(z);
    a0[p * Tile<E>::S + e] = fm ? __builtin_fmaf(fm[e], sv, fm[E + e]) : sv;
    if (z0) z0[p * Tile<E>::S + e] = z;
  }
}

// One hidden layer on the matrix cores: out[p][o] = sin(W[o] . in[p] + b[o])
// for the wave's 16 points; z (optional) keeps the pre-activation.
// SIN / SOUT: row strides of the input and output tiles.
template <int IN, int HD, int SIN = Tile<IN>::S, int SOUT = Tile<HD>::S>
__device__ __forceinline__ void hidden_layer(const float* __restrict__ w, const float* __restrict__ b, const float* in,
                                             float* out, float* z, const float* fm = nullptr) {
  constexpr int KB = IN / 4;
  const int l = int(threadIdx.x) & 63, s = l >> 4, p = l & 15;
  float bv[KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) bv[kb] = in[p * SIN + KB * s + kb];
#pragma unroll
  for (int o0 = 0; o0 < HD; o0 += 16) {
    const float* wr = w + (o0 + p) * IN + KB * s;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) acc = mfma4(wr[kb], bv[kb], acc);
    // D[m = o0 + 4 s + r][n = point p]
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int o = o0 + 4 * s + r;
      const float zz = acc[r] + (b ? b[o] : 0.f);
      const float sv = sinf(zz);
      out[p * SOUT + o] = fm ? __builtin_fmaf(fm[o], sv, fm[HD + o]) : sv;  // FiLM: gamma sin + beta
      if (z) z[p * SOUT + o] = zz;
    }
  }
}

// Layers 1..nh for the wave's tile; returns the tile holding a_nh.  fwd keeps
// only two tiles (ping-pong); the backward passes per-layer tiles (act[i],
// zt[i]) so every layer's activation and pre-activation survive.
template <int E, int HD>
__device__ __forceinline__ const float* run_layers(const SirenNet& n, float* const* act, float* const* zt, int smp) {
  for (int i = 1; i <= n.nh; ++i) {
    const float* w = layer_w(n, i, E, HD);
    const float* b = n.bh ? n.bh + (i - 1) * HD : nullptr;
    const float* fm = n.film_of(smp, i, HD);
    wave_lds_order();
    if (i == 1)
      hidden_layer<E, HD>(w, b, act[0], act[1], zt ? zt[1] : nullptr, fm);
    else
      hidden_layer<HD, HD>(w, b, act[i - 1], act[i], zt ? zt[i] : nullptr, fm);
  }
  wave_lds_order();
  return act[n.nh];
}

// ---------------------------------------------------------------------------
// Forward.  grid = ceil(G / 64) workgroups of 4 waves (16 points each);
// dynamic LDS per wave: a0 [16][E] and two ping-pong tiles [16][HD].  Writes
// the last layer transposed, act[j][g] = a_nh[g][j] (j < HD), and the ones
// row act[HD][g] = 1 that carries the readout bias through the readout GEMM.
// ---------------------------------------------------------------------------
template <int E, int HD>
__global__ __launch_bounds__(kSirenThreads) void siren_mlp_fwd_kernel(const float* __restrict__ grid, int64_t G,
                                                                      SirenNet n, float* __restrict__ act,
                                                                      int64_t lda) {
  extern __shared__ float lds[];
  const int wv = int(threadIdx.x) >> 6, l = int(threadIdx.x) & 63, s = l >> 4, p = l & 15;
  float* base = lds + wv * (Tile<E>::WORDS + 2 * Tile<HD>::WORDS);
  float* t0 = base;
  float* t1 = base + Tile<E>::WORDS;
  float* t2 = t1 + Tile<HD>::WORDS;
  const int64_t g0 = (int64_t(blockIdx.x) * kSirenWaves + wv) * 16;
  const int smp = int(blockIdx.y);  // sample (FiLM); act rows of sample smp follow those of smp - 1
  act += int64_t(smp) * (HD + 1) * lda;
  pos_embed<E>(n, grid, G, g0, t0, nullptr, n.film_of(smp, 0, HD));
  // ping-pong: a_i in t1 for odd i, t2 for even i >= 2
  float* tiles[9] = {t0, t1, t2, t1, t2, t1, t2, t1, t2};
  const float* last = run_layers<E, HD>(n, tiles, nullptr, smp);
  const int64_t g = g0 + p;
  if (g < G) {
    for (int j = s; j < HD; j += 4) act[int64_t(j) * lda + g] = last[p * Tile<HD>::S + j];
    if (s == 0) act[int64_t(HD) * lda + g] = 1.f;
  }
}

// Backward pass 1.  grid = (ceil(G / (16 waves)), nb): sample smp = blockIdx.y.
// Rows are written for all samples side by side, column smp * Gp + g (GT = nb
// Gp columns; points g >= G written as zeros), so the Gram reductions over the
// GT columns sum every weight gradient over the samples.  FiLM slot f's
// gradients are row sums over one sample's columns of fdh = dL/dh (beta) and
// fds = dL/dh * sin(z) (gamma), rows f * HD + o.
template <int E, int HD>
__global__ __launch_bounds__(kSirenThreads) void siren_bwd_delta_kernel(
    const float* __restrict__ gact, int64_t sj, int64_t sg, int64_t ss, const float* __restrict__ grid, int64_t G,
    int64_t Gp, SirenNet n, float* __restrict__ act, float* __restrict__ del, float* __restrict__ gridT,
    float* __restrict__ fdh, float* __restrict__ fds, int nwaves_wg) {
  extern __shared__ float lds[];
  constexpr int D = E > HD ? E : HD;
  constexpr int TS = Tile<D>::S, TW = Tile<D>::WORDS;
  const int wv = int(threadIdx.x) >> 6, l = int(threadIdx.x) & 63, s = l >> 4, p = l & 15;
  const int per_wave = (2 * (n.nh + 1) + 2) * TW;
  float* base = lds + wv * per_wave;
  float* at[9];
  float* zt[9];
  for (int i = 0; i <= n.nh; ++i) {
    at[i] = base + i * TW;
    zt[i] = base + (n.nh + 1 + i) * TW;
  }
  float* dA = base + 2 * (n.nh + 1) * TW;
  float* dB = dA + TW;
  const int64_t g0 = (int64_t(blockIdx.x) * nwaves_wg + wv) * 16;
  const int64_t g = g0 + p;
  const bool gok = g < G;
  const int smp = int(blockIdx.y);
  const int64_t GT = int64_t(gridDim.y) * Gp;
  const int64_t col = int64_t(smp) * Gp + g;  // this point's column in the rows of all samples
  const bool colok = g < Gp;

  // dA[p][j] = gact[smp ss + j sj + (g0 + p) sg], the gradient of the last layer's output (W_out^T gk)
  for (int j = s; j < HD; j += 4) dA[p * TS + j] = gok ? gact[smp * ss + int64_t(j) * sj + g * sg] : 0.f;

  // forward recompute with pre-activations; every tile has the D-wide stride TS
  {
    float x[3];
    load_coords(grid, G, n.d, g, x);
    const float xs = s == 0 ? x[0] : (s == 1 ? x[1] : x[2]);
    if (s < n.d && colok) gridT[int64_t(s) * GT + col] = gok ? xs : 0.f;
    const float* fm0 = n.film_of(smp, 0, HD);
#pragma unroll
    for (int t = 0; t < E / 4; ++t) {
      const int e = s + 4 * t;
      const float z = embed_pre(n, e, x);
      const float sv = sinf(z);
      at[0][p * TS + e] = fm0 ? __builtin_fmaf(fm0[e], sv, fm0[E + e]) : sv;
      zt[0][p * TS + e] = z;
    }
    for (int i = 1; i <= n.nh; ++i) {
      const float* w = layer_w(n, i, E, HD);
      const float* b = n.bh ? n.bh + (i - 1) * HD : nullptr;
      const float* fm = n.film_of(smp, i, HD);
      wave_lds_order();
      if (i == 1)
        hidden_layer<E, HD, TS, TS>(w, b, at[0], at[1], zt[1], fm);
      else
        hidden_layer<HD, HD, TS, TS>(w, b, at[i - 1], at[i], zt[i], fm);
    }
    wave_lds_order();
  }

  // Through layer L's output h = gamma sin(z) + beta (FiLM) or sin(z): from dh, delta = dh gamma cos(z); FiLM rows
  // fdh = dh, fds = dh sin(z) at row f * HD + o, column col.
  auto through = [&](int L, int pp, int j, float dh, float z) -> float {
    const float* fm = n.film_of(smp, L, HD);
    if (fm) {
      const int64_t row = int64_t(L - 1 + n.film_first) * HD + j;
      const int64_t c = int64_t(smp) * Gp + g0 + pp;
      if (g0 + pp < Gp) {
        const bool ok = g0 + pp < G;
        fdh[row * GT + c] = ok ? dh : 0.f;
        fds[row * GT + c] = ok ? dh * sinf(z) : 0.f;
      }
      dh *= fm[j];
    }
    return dh * cosf(z);
  };
  // delta_nh = through(dA); for i = nh..1: delta_{i-1}[p][j] = through(sum_o delta_i[p][o] W_i[o][j])
  // (D[m = j][n = p] = sum_o W_i^T[j][o] delta_i^T[o][p]: A[m = j][k = o] = W_i[o][j], B[k = o][n = p]).
  float* cur = dA;
  float* nxt = dB;
  for (int e = l; e < 16 * HD; e += 64) {
    const int pp = e / HD, j = e - pp * HD;
    cur[pp * TS + j] = through(n.nh, pp, j, cur[pp * TS + j], zt[n.nh][pp * TS + j]);
  }
  wave_lds_order();
  for (int i = n.nh; i >= 0; --i) {
    const int rows = i == 0 ? E : HD;
    // write a_i^T and delta_i^T rows for these 16 points
    const int64_t roff = i == 0 ? 0 : E + int64_t(i - 1) * HD;
    for (int e = s; e < rows; e += 4) {
      if (colok) {
        act[(roff + e) * GT + col] = gok ? at[i][p * TS + e] : 0.f;
        del[(roff + e) * GT + col] = gok ? cur[p * TS + e] : 0.f;
      }
    }
    if (i == 0) break;
    const int IN = i == 1 ? E : HD;
    const float* w = layer_w(n, i, E, HD);
    // B operand: delta_i^T[o][p] for o = (HD/4) s + kb
    constexpr int KBO = HD / 4;
    float bv[KBO];
#pragma unroll
    for (int kb = 0; kb < KBO; ++kb) bv[kb] = cur[p * TS + KBO * s + kb];
    for (int j0 = 0; j0 < IN; j0 += 16) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < KBO; ++kb) acc = mfma4(w[(KBO * s + kb) * IN + j0 + p], bv[kb], acc);
      // D[m = j = j0 + 4 s + r][n = point p]
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = j0 + 4 * s + r;
        nxt[p * TS + j] = through(i - 1, p, j, acc[r], zt[i - 1][p * TS + j]);
      }
    }
    wave_lds_order();
    float* t = cur;
    cur = nxt;
    nxt = t;
  }
}

// ---------------------------------------------------------------------------
// Gram reduction over points: part[c][m][n] = sum_{g in chunk c} X[m][g] Y[n][g]
// (n < N; rows n >= NY of Y read as zero) and rsum[c][m] = sum_g X[m][g].
// X rows have stride ldx, Y rows stride ldy.  grid = (M / 16, chunks); the 4
// waves split a chunk (chunk a multiple of 64) and are reduced through LDS.
// Each wave loads the next 16 points' operands before the current products.
// VEC: 16-byte loads (ldx, ldy multiples of 4 and 16-byte aligned bases).
// ---------------------------------------------------------------------------
template <int NT, bool VEC>
__global__ __launch_bounds__(kSirenThreads) void siren_gram_kernel(const float* __restrict__ X, int64_t ldx,
                                                                   const float* __restrict__ Y, int64_t ldy, int NY,
                                                                   int64_t G, int M, int64_t chunk,
                                                                   float* __restrict__ part, float* __restrict__ rsum) {
  __shared__ float red[kSirenWaves][NT * 16 * 16 + 16];
  const int wv = int(threadIdx.x) >> 6, l = int(threadIdx.x) & 63, s = l >> 4, p = l & 15;
  const int m0 = int(blockIdx.x) * 16;
  const int64_t gbeg = int64_t(blockIdx.y) * chunk + int64_t(wv) * (chunk / kSirenWaves);
  const int64_t gend0 = gbeg + chunk / kSirenWaves;
  const int64_t gend = gend0 < G ? gend0 : G;
  const float* xr = X + int64_t(m0 + p) * ldx;
  // slot s takes points gb + 4 s + i, i = 0..3 (one 16-byte segment per row)
  auto ld4 = [&](const float* row, int64_t gs, float* v) {
    if (VEC && gs + 3 < G) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(row + gs);
      v[0] = t[0]; v[1] = t[1]; v[2] = t[2]; v[3] = t[3];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = gs + i < G ? row[gs + i] : 0.f;
    }
  };
  float xv[4], yv[NT][4], xn[4], yn[NT][4];
  auto load = [&](int64_t gb, float* x, float (*y)[4]) {
    const int64_t gs = gb + 4 * s;
    ld4(xr, gs, x);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int nrow = 16 * t + p;
      if (nrow < NY) {
        ld4(Y + int64_t(nrow) * ldy, gs, y[t]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) y[t][i] = 0.f;
      }
    }
  };
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float rs = 0.f;
  if (gbeg < gend) load(gbeg, xv, yv);
  for (int64_t gb = gbeg; gb < gend; gb += 16) {
    if (gb + 16 < gend) load(gb + 16, xn, yn);
    rs += (xv[0] + xv[1]) + (xv[2] + xv[3]);
    // A[m = p][k slot s] = X[m0 + p][gs + i], B[k][n = p] = Y[16 t + p][gs + i]
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t] = mfma4(xv[i], yv[t][i], acc[t]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xv[i] = xn[i];
#pragma unroll
      for (int t = 0; t < NT; ++t) yv[t][i] = yn[t][i];
    }
  }
  // D[m = 4 s + r][n = p] of tile t; row sums: lanes of slot s hold row p partials
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wv][t * 256 + (4 * s + r) * 16 + p] = acc[t][r];
  }
  rs += __shfl_xor(rs, 16);
  rs += __shfl_xor(rs, 32);
  if (s == 0) red[wv][NT * 256 + p] = rs;
  __syncthreads();
  const int64_t cidx = blockIdx.y;
  for (int e = int(threadIdx.x); e < NT * 256; e += kSirenThreads) {
    const float v = (red[0][e] + red[1][e]) + (red[2][e] + red[3][e]);
    const int t = e / 256, mm = (e % 256) / 16, nn = e % 16;
    part[(cidx * M + m0 + mm) * (NT * 16) + 16 * t + nn] = v;
  }
  if (threadIdx.x < 16) {
    const int e = NT * 256 + int(threadIdx.x);
    rsum[cidx * M + m0 + int(threadIdx.x)] = (red[0][e] + red[1][e]) + (red[2][e] + red[3][e]);
  }
}

// out[m][n] (n < N) = sum_c part[c][m][n] (row stride NP) and rout[m] = sum_c
// rpart[c][m] (if given): one wave per output, lanes take chunks c = lane,
// lane + 64, ... and a fixed butterfly adds the lanes (deterministic).
__global__ __launch_bounds__(256) void siren_reduce_kernel(const float* __restrict__ part, int64_t chunks, int M,
                                                           int NP, int N, float* __restrict__ out,
                                                           const float* __restrict__ rpart,
                                                           float* __restrict__ rout) {
  const int64_t e = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = int(threadIdx.x) & 63;
  const int64_t nout = int64_t(M) * N;
  const bool is_out = e < nout;
  const bool is_row = !is_out && rout && e < nout + M;
  if (!is_out && !is_row) return;  // a whole wave leaves together
  float acc = 0.f;
  if (is_out) {
    const int m = int(e / N), nn = int(e % N);
    for (int64_t c = lane; c < chunks; c += 64) acc += part[(c * M + m) * NP + nn];
  } else {
    const int64_t m = e - nout;
    for (int64_t c = lane; c < chunks; c += 64) acc += rpart[c * M + m];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
  if (lane == 0) {
    if (is_out)
      out[e] = acc;
    else
      rout[e - nout] = acc;
  }
}

bool siren_dims_ok(int E, int HD) {
  auto ok = [](int v) { return v == 16 || v == 32 || v == 64 || v == 128; };
  return ok(E) && ok(HD);
}

template <template <int, int> class F, class... A>
bool siren_dispatch(int E, int HD, A&&... a) {
#define NSQ_SIREN_CASE(e, h) \
  if (E == e && HD == h) return F<e, h>::run(static_cast<A&&>(a)...), true;
  NSQ_SIREN_CASE(16, 16) NSQ_SIREN_CASE(16, 32) NSQ_SIREN_CASE(16, 64) NSQ_SIREN_CASE(16, 128)
  NSQ_SIREN_CASE(32, 16) NSQ_SIREN_CASE(32, 32) NSQ_SIREN_CASE(32, 64) NSQ_SIREN_CASE(32, 128)
  NSQ_SIREN_CASE(64, 16) NSQ_SIREN_CASE(64, 32) NSQ_SIREN_CASE(64, 64) NSQ_SIREN_CASE(64, 128)
  NSQ_SIREN_CASE(128, 16) NSQ_SIREN_CASE(128, 32) NSQ_SIREN_CASE(128, 64) NSQ_SIREN_CASE(128, 128)
#undef NSQ_SIREN_CASE
  return false;
}

template <int E, int HD>
struct SirenFwd {
  static void run(const float* grid, int64_t G, const SirenNet& n, float* act, int64_t lda, int64_t nb,
                  hipStream_t st) {
    const size_t lds = size_t(kSirenWaves) * (Tile<E>::WORDS + 2 * Tile<HD>::WORDS) * sizeof(float);
    const dim3 grd(unsigned(ceil_div(G, 16 * kSirenWaves)), unsigned(nb));
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&siren_mlp_fwd_kernel<E, HD>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    hipLaunchKernelGGL((siren_mlp_fwd_kernel<E, HD>), grd, dim3(kSirenThreads), lds, st, grid, G, n, act, lda);
  }
};

// Readout k[h][g] = b_out[h] + sum_j W_out[h][j] a[j][g] (j < HD, in order):
// a lane owns V consecutive points and keeps their HD activations in
// registers; a workgroup takes a block of ReadoutCfg::ROWS channels whose W_out
// rows it stages in LDS (wave-uniform broadcast reads) and produces CH of them
// at a time (CH x V independent FMA chains).  Each store is V consecutive
// floats per lane, so a wave writes 64 V contiguous floats of one filter row.
// The pass is bound by writing k (4 bytes per output: 0.63 ms for 4.3 GB on
// MI355X) against HD fused multiply-adds per output on the VALU.
template <int HD>
struct ReadoutCfg {
  static constexpr int V = HD <= 32 ? 4 : (HD == 64 ? 2 : 1);  // points per lane: V * HD activations in registers
  static constexpr int CH = V == 4 ? 4 : 8;                      // channels per step
  static constexpr int ROWS = (8192 / HD) < 256 ? (8192 / HD) : 256;  // channels per workgroup (32 KB of W_out)
};

// VEC: V-wide accesses (G a multiple of V, k and act 16-byte aligned, lda a
// multiple of V); otherwise one point per lane.
template <int HD, bool VEC>
__global__ __launch_bounds__(256) void siren_readout_fwd_kernel(const float* __restrict__ wout,
                                                                const float* __restrict__ bout,
                                                                const float* __restrict__ act, int64_t lda,
                                                                int64_t G, int64_t H, float* __restrict__ k) {
  using C = ReadoutCfg<HD>;
  constexpr int V = VEC ? C::V : 1;
  constexpr int CH = C::CH, ROWS = C::ROWS;
  __shared__ float ws[ROWS * HD];
  __shared__ float bs[ROWS];
  const int64_t g = (int64_t(blockIdx.x) * 256 + threadIdx.x) * V;
  const bool gok = g < G;  // VEC: the V points are whole (G % V == 0)
  const int64_t h0 = int64_t(blockIdx.y) * ROWS;
  act += int64_t(blockIdx.z) * (HD + 1) * lda;  // sample blockIdx.z (per-sample FiLM filters)
  k += int64_t(blockIdx.z) * H * G;
  const int nrows = H - h0 < ROWS ? int(H - h0) : ROWS;
  for (int i = threadIdx.x; i < ROWS * HD; i += 256) ws[i] = i < nrows * HD ? wout[h0 * HD + i] : 0.f;
  for (int i = threadIdx.x; i < ROWS; i += 256) bs[i] = (bout && i < nrows) ? bout[h0 + i] : 0.f;
  float a[HD][V];
  const float* ap = act + (gok ? g : 0);
#pragma unroll
  for (int j = 0; j < HD; ++j) {
    if constexpr (V == 4) {
      const float4 t = *reinterpret_cast<const float4*>(ap + int64_t(j) * lda);
      a[j][0] = t.x; a[j][1] = t.y; a[j][2] = t.z; a[j][3] = t.w;
    } else if constexpr (V == 2) {
      const float2 t = *reinterpret_cast<const float2*>(ap + int64_t(j) * lda);
      a[j][0] = t.x; a[j][1] = t.y;
    } else {
      a[j][0] = ap[int64_t(j) * lda];
    }
  }
  __syncthreads();
  for (int hh = 0; hh < nrows; hh += CH) {
    float acc[CH][V];
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int v = 0; v < V; ++v) acc[c][v] = bs[hh + c < ROWS ? hh + c : 0];
#pragma unroll
    for (int j = 0; j < HD; ++j)
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const float wv = ws[(hh + c < ROWS ? hh + c : 0) * HD + j];
#pragma unroll
        for (int v = 0; v < V; ++v) acc[c][v] = __builtin_fmaf(wv, a[j][v], acc[c][v]);
      }
    if (gok) {
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        if (hh + c >= nrows) break;
        float* o = k + (h0 + hh + c) * G + g;
        if constexpr (V == 4)
          *reinterpret_cast<float4*>(o) = make_float4(acc[c][0], acc[c][1], acc[c][2], acc[c][3]);
        else if constexpr (V == 2)
          *reinterpret_cast<float2*>(o) = make_float2(acc[c][0], acc[c][1]);
        else
          *o = acc[c][0];
      }
    }
  }
}

template <int HD>
static void launch_readout(const float* wout, const float* bout, const float* act, int64_t lda, int64_t G, int64_t H,
                           float* k, int64_t nb, hipStream_t st) {
  using C = ReadoutCfg<HD>;
  const bool vec = G % C::V == 0 && lda % C::V == 0 && (reinterpret_cast<uintptr_t>(k) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(act) & 15) == 0;
  const int v = vec ? C::V : 1;
  const dim3 grd(unsigned(ceil_div(G, int64_t(256) * v)), unsigned(ceil_div(H, int64_t(C::ROWS))), unsigned(nb));
  if (vec)
    hipLaunchKernelGGL((siren_readout_fwd_kernel<HD, true>), grd, dim3(256), 0, st, wout, bout, act, lda, G, H, k);
  else
    hipLaunchKernelGGL((siren_readout_fwd_kernel<HD, false>), grd, dim3(256), 0, st, wout, bout, act, lda, G, H, k);
}

// ---------------------------------------------------------------------------
// Readout backward in one pass over the filter gradient gk (read once):
//   gact[nb][j][g] = sum_h W_out[h][j] gk[nb][h][g]            (K = h)
//   gW[h][j]       = sum_nb sum_g gk[nb][h][g] a[nb][j][g]      (K = g)
//   gb[h]          = sum_nb sum_g gk[nb][h][g]
// (a = rows 0..HD-1 of act).  Both products run on v_mfma_f32_16x16x32_bf16
// with every operand split v = hi + lo into bf16 halves (hi = bf16(v), lo =
// bf16(v - hi)) and three products per step, hi.hi + hi.lo + lo.hi, fp32
// accumulation: ~2^-17 relative error per product (the dropped lo.lo term and
// lo's rounding), against ~5x the time on the fp32 matrix path (whose rate is
// the VALU's, so a one-pass fp32 kernel would be bound by its multiply-adds,
// not by reading gk).  Lane layout of the product (checked on MI355X):
// A[l % 16][8 (l / 16) + e], B[8 (l / 16) + e][l % 16], D[4 (l / 16) + r][l % 16].
//
// Work split.  A workgroup of 8 waves owns kRbGpw * 8 consecutive points of
// one sample nb and a slice of the channels; wave w owns kRbGpw of the points
// and sweeps the slice in chunks of 32 channels:
//  * gact: the wave's [HD][kRbGpw] accumulator stays in registers across the
//    sweep (B operand: gk loaded as 8 channels x 1 point per lane);
//  * gW, gb: each chunk's [32][HD] product over the wave's points (A operand:
//    gk loaded as 1 channel x 8 points per lane; the second load of the same
//    lines is an L2 hit) is summed over the 8 waves through LDS in a fixed
//    order and written as the workgroup's partial; siren_sum_parts_kernel adds
//    the partials of all workgroups in a fixed order.
// With several channel slices (small G), gact is written per slice and
// siren_sum_parts_kernel adds the slices in order.  Deterministic throughout.
// ---------------------------------------------------------------------------
typedef float nsq_f32x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 nsq_bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kRbWaves = 8;
constexpr int kRbThreads = 64 * kRbWaves;
constexpr int kRbGpw = 64;   // points per wave
constexpr int kRbHc = 32;    // channels per chunk

__device__ __forceinline__ void split8(const nsq_f32x8_t& v, nsq_bf16x8_t& hi, nsq_bf16x8_t& lo) {
  hi = __builtin_convertvector(v, nsq_bf16x8_t);
  const nsq_f32x8_t r = v - __builtin_convertvector(hi, nsq_f32x8_t);
  lo = __builtin_convertvector(r, nsq_bf16x8_t);
}

__device__ __forceinline__ f32x4 mfma_split(const nsq_bf16x8_t& ah, const nsq_bf16x8_t& al, const nsq_bf16x8_t& bh,
                                            const nsq_bf16x8_t& bl, f32x4 c) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, c, 0, 0, 0);
  return c;
}

// 8 consecutive floats p[0..7] of a row whose valid length from p is n (zeros
// past it).  VEC: p 16-byte aligned.
template <bool VEC>
__device__ __forceinline__ nsq_f32x8_t load8(const float* __restrict__ p, int64_t n) {
  nsq_f32x8_t v;
  if (VEC && n >= 8) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
    v = nsq_f32x8_t{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = e < n ? p[e] : 0.f;
  }
  return v;
}

// Raw buffer resource over bytes [p, p + bytes): loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rb_rsrc(const float* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, bytes, 0x00020000);
}

// bw (optional, G floats): gb weighted by it, gb[h] = sum_g gk[h][g] bw[g], instead of the row sum.
template <int HD, bool VEC>
__global__ __launch_bounds__(kRbThreads) void siren_readout_bwd_kernel(
    const float* __restrict__ gk, int64_t ldk, const float* __restrict__ act, int64_t lda,
    const float* __restrict__ bw, const float* __restrict__ wout, int64_t G, int H, int hslice,
    float* __restrict__ gact, int64_t gact_slice, float* __restrict__ gw_part, float* __restrict__ gb_part) {
  constexpr int NJ = HD / 16, NGB = kRbGpw / 16, NKS = kRbGpw / 32, RS = HD + 1;
  // TS: row stride (words) of a wave's transposition tile [32 channels][kRbGpw points]: 66 puts the 4 channel
  // groups of a gact operand read (rows 8q + e) 16 banks apart, so a read covers the 64 banks once
  constexpr int TS = kRbGpw + 2;
  // chunk partials double-buffered where LDS allows (HD <= 32), else one buffer and a second barrier
  constexpr int NBUF = (2 * kRbWaves * kRbHc * RS + kRbWaves * kRbHc * TS) * 4 <= 160 * 1024 ? 2 : 1;
  __shared__ float red[NBUF][kRbWaves][kRbHc * RS];
  __shared__ float tile[kRbWaves][kRbHc * TS];
  const int wv = int(threadIdx.x) >> 6, l = int(threadIdx.x) & 63, q = l >> 4, p = l & 15;
  const int64_t ngb = gridDim.x;
  const int nb = int(blockIdx.z), hs = int(blockIdx.y);
  const int64_t gw0 = (int64_t(blockIdx.x) * kRbWaves + wv) * kRbGpw;
  const int hb = hs * hslice, he = hb + hslice < H ? hb + hslice : H;
  const float* gkb = gk + int64_t(nb) * H * ldk;
  const float* ab = act + int64_t(nb) * (HD + 1) * lda;
  // every point of this wave's block is < G (wave-uniform): the gW operand loads need no per-point guard
  const bool full = VEC && gw0 + kRbGpw <= G;
  const int rowb = int(ldk) * 4;  // bytes per gk row (ldk <= 2^23, checked by the entry point)
  // byte offsets of this lane inside a chunk's rows (chunk base = row h0, column 0; gw0 < G + 512 <= 2^23 + 512)
  // (the whole offset goes in the lane's offset register, which the buffer range check covers; only compile-time
  // steps ride in the instruction's immediate)
  int off_w[2];  // gW operand: row 16 hbk + p, points gw0 + 32 ks + 8q + e
#pragma unroll
  for (int hbk = 0; hbk < 2; ++hbk) off_w[hbk] = ((16 * hbk + p) * int(ldk) + int(gw0) + 8 * q) * 4;
  const int off_o = (8 * q * HD + p) * 4;  // W_out operand: row 8q + e, column 16 jt + p

  // act as the gW product's B operand, B[k = g][n = j] = a[j][g]: held for the whole sweep
  nsq_bf16x8_t bah[NJ][NKS], bal[NJ][NKS];
#pragma unroll
  for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int64_t g = gw0 + 32 * ks + 8 * q;
      const nsq_f32x8_t v = load8<VEC>(ab + int64_t(16 * jt + p) * lda + g, G - g);
      split8(v, bah[jt][ks], bal[jt][ks]);
    }
  nsq_f32x8_t bwv[NKS];  // gb weights at this lane's points
  if (bw) {
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int64_t g = gw0 + 32 * ks + 8 * q;
      bwv[ks] = load8<VEC>(bw + g, G - g);
    }
  }
  f32x4 acc_a[NJ][NGB];  // gact^T tiles D[j][g]
#pragma unroll
  for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) acc_a[jt][gb] = f32x4{0.f, 0.f, 0.f, 0.f};

  // gW operand of a chunk (rows h0 + 16 hbk + p, 8 points per k-step), loaded one chunk ahead
  auto load_gw_operand = [&](int h0, int hn, nsq_f32x8_t (&v)[2][NKS]) {
    if (full) {
      const __amdgpu_buffer_rsrc_t r = rb_rsrc(gkb + int64_t(h0) * ldk, hn * rowb);
#pragma unroll
      for (int hbk = 0; hbk < 2; ++hbk)
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const auto x = __builtin_amdgcn_raw_buffer_load_b128(r, off_w[hbk] + 128 * ks, 0, 0);
          const auto y = __builtin_amdgcn_raw_buffer_load_b128(r, off_w[hbk] + 128 * ks + 16, 0, 0);
          v[hbk][ks] = nsq_f32x8_t{__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]),
                                   __uint_as_float(x[3]), __uint_as_float(y[0]), __uint_as_float(y[1]),
                                   __uint_as_float(y[2]), __uint_as_float(y[3])};
        }
    } else {
#pragma unroll
      for (int hbk = 0; hbk < 2; ++hbk) {
        const int hh = 16 * hbk + p;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const int64_t g = gw0 + 32 * ks + 8 * q;
          v[hbk][ks] = hh < hn ? load8<false>(gkb + int64_t(h0 + hh) * ldk + g, G - g) : nsq_f32x8_t{};
        }
      }
    }
  };

  nsq_f32x8_t cur[2][NKS], nxt[2][NKS];
  if (hb < he) load_gw_operand(hb, he - hb < kRbHc ? he - hb : kRbHc, cur);
  int buf = 0;
  for (int h0 = hb; h0 < he; h0 += kRbHc, buf = NBUF == 2 ? buf ^ 1 : 0) {
    const int hn = he - h0 < kRbHc ? he - h0 : kRbHc;  // valid channels of this chunk
    const __amdgpu_buffer_rsrc_t ro = rb_rsrc(wout + int64_t(h0) * HD, hn * HD * 4);
    // gact's A operand, A[m = j][k = h] = W_out[h][j] (rows >= hn read as 0)
    nsq_f32x8_t wv8[NJ];
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        wv8[jt][e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ro, off_o + 64 * jt + e * HD * 4, 0, 0));
    // the next chunk's gW operand, in flight while this chunk's products run
    const int h1 = h0 + kRbHc;
    if (h1 < he) load_gw_operand(h1, he - h1 < kRbHc ? he - h1 : kRbHc, nxt);
    // the chunk's gk values (arrived during the previous chunk) into the wave's transposition tile, row 16 hbk +
    // p, points 32 ks + 8 q + e: the gact operand reads them back as 8 channels x 1 point per lane
    float* tw_ = tile[wv];
#pragma unroll
    for (int hbk = 0; hbk < 2; ++hbk)
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        float* d = tw_ + (16 * hbk + p) * TS + 32 * ks + 8 * q;
#pragma unroll
        for (int e = 0; e < 8; e += 2) *reinterpret_cast<float2*>(d + e) = make_float2(cur[hbk][ks][e], cur[hbk][ks][e + 1]);
      }
    // --- gW: A[m = h][k = g] = gk[h][g], B[k = g][n = j] = a[j][g]; gb from the same values
    f32x4 acc_w[2][NJ];
    float bsum[2] = {0.f, 0.f};
#pragma unroll
    for (int hbk = 0; hbk < 2; ++hbk) {
#pragma unroll
      for (int jt = 0; jt < NJ; ++jt) acc_w[hbk][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const nsq_f32x8_t v = cur[hbk][ks];
        if (bw) {
          const nsq_f32x8_t u = v * bwv[ks];
          bsum[hbk] += ((u[0] + u[1]) + (u[2] + u[3])) + ((u[4] + u[5]) + (u[6] + u[7]));
        } else {
          bsum[hbk] += ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
        }
        nsq_bf16x8_t ah, al;
        split8(v, ah, al);
#pragma unroll
        for (int jt = 0; jt < NJ; ++jt)
          acc_w[hbk][jt] = mfma_split(ah, al, bah[jt][ks], bal[jt][ks], acc_w[hbk][jt]);
      }
    }
    // the wave's chunk partials to LDS: D[m = h = 16 hbk + 4 q + r][n = j = 16 jt + p]; gb per channel
    float* rw = red[buf][wv];
#pragma unroll
    for (int hbk = 0; hbk < 2; ++hbk) {
#pragma unroll
      for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) rw[(16 * hbk + 4 * q + r) * RS + 16 * jt + p] = acc_w[hbk][jt][r];
      float b = bsum[hbk];
      b += __shfl_xor(b, 16);
      b += __shfl_xor(b, 32);
      if (q == 0) rw[(16 * hbk + p) * RS + HD] = b;
    }
    // --- gact: B[k = h][n = g] = gk[h][g] from the tile (the wave's own LDS writes above, in order); rows >= hn
    // are zero, points >= G only reach output columns that are not stored
    wave_lds_order();
    nsq_bf16x8_t wah[NJ], wal[NJ];
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt) split8(wv8[jt], wah[jt], wal[jt]);
#pragma unroll
    for (int gb = 0; gb < NGB; ++gb) {
      nsq_f32x8_t gv;
#pragma unroll
      for (int e = 0; e < 8; ++e) gv[e] = tw_[(8 * q + e) * TS + 16 * gb + p];
      nsq_bf16x8_t bh, bl;
      split8(gv, bh, bl);
#pragma unroll
      for (int jt = 0; jt < NJ; ++jt) acc_a[jt][gb] = mfma_split(wah[jt], wal[jt], bh, bl, acc_a[jt][gb]);
    }
    __syncthreads();
    // fixed-order sum over the 8 waves; one partial row block per workgroup and chunk
    const int64_t prow = (int64_t(nb) * ngb + blockIdx.x) * H;
    for (int e = int(threadIdx.x); e < kRbHc * RS; e += kRbThreads) {
      const int hh = e / RS, j = e - hh * RS;
      if (hh >= hn) continue;
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < kRbWaves; ++w) sum += red[buf][w][e];
      if (j < HD)
        gw_part[(prow + h0 + hh) * HD + j] = sum;
      else if (gb_part)
        gb_part[prow + h0 + hh] = sum;
    }
    // double-buffered, no second barrier: the next chunk writes the other buffer, and the chunk after it follows
    // this chunk's successor's barrier, which every reader of this buffer has passed
    if constexpr (NBUF == 1) __syncthreads();
#pragma unroll
    for (int hbk = 0; hbk < 2; ++hbk)
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) cur[hbk][ks] = nxt[hbk][ks];
  }
  // gact^T tiles: D[m = j = 16 jt + 4 q + r][n = g = 16 gb + p]
  float* ga = gact + int64_t(hs) * gact_slice + int64_t(nb) * HD * G;
#pragma unroll
  for (int gb = 0; gb < NGB; ++gb) {
    const int64_t g = gw0 + 16 * gb + p;
    if (g < G) {
#pragma unroll
      for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
        for (int r = 0; r < 4; ++r) ga[int64_t(16 * jt + 4 * q + r) * G + g] = acc_a[jt][gb][r];
    }
  }
}

// out[i] = scale * sum_{s < ns} part[s * n + i] for i < n: thread i walks the parts in order with 16 interleaved
// running sums (s = 0, 16, 32, ... / 1, 17, ...; 16 loads in flight per thread) added in a fixed tree at the end,
// so the result is bitwise repeatable.
__global__ __launch_bounds__(256) void siren_sum_parts_kernel(const float* __restrict__ part, int64_t ns, int64_t n,
                                                              float* __restrict__ out, float scale) {
  constexpr int U = 16;
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  float s[U];
#pragma unroll
  for (int u = 0; u < U; ++u) s[u] = 0.f;
  int64_t k = 0;
  for (; k + U <= ns; k += U) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = part[(k + u) * n + i];
#pragma unroll
    for (int u = 0; u < U; ++u) s[u] += v[u];
  }
  for (int u = 0; k < ns; ++k, ++u) s[u] += part[k * n + i];
#pragma unroll
  for (int w = U / 2; w >= 1; w /= 2)
#pragma unroll
    for (int u = 0; u < w; ++u) s[u] += s[u + w];
  out[i] = s[0] * scale;
}

// Readout-backward launch geometry: point blocks of 8 waves x kRbGpw, channel
// slices of whole 32-channel chunks chosen so that the grid reaches ~512
// workgroups (two per CU) when the points alone do not.
struct RbPlan {
  int64_t ngb;
  int hs, hslice;
  size_t gw_part, gb_part, gact_part, total;  // float offsets / count
};

RbPlan rb_plan(int64_t H, int HD, int64_t G, int64_t nb) {
  RbPlan p{};
  p.ngb = ceil_div(G, int64_t(kRbWaves) * kRbGpw);
  const int64_t chunks = ceil_div(H, int64_t(kRbHc));
  int64_t hs = ceil_div(512, p.ngb * nb);
  hs = hs < 1 ? 1 : (hs > chunks ? chunks : hs);
  p.hslice = int(ceil_div(chunks, hs) * kRbHc);
  p.hs = int(ceil_div(H, int64_t(p.hslice)));
  auto al = [](size_t v) { return (v + 63) / 64 * 64; };
  p.gw_part = 0;
  p.gb_part = al(size_t(nb * p.ngb) * size_t(H) * HD);
  p.gact_part = al(p.gb_part + size_t(nb * p.ngb) * size_t(H));
  p.total = al(p.gact_part + (p.hs > 1 ? size_t(p.hs) * size_t(nb) * HD * size_t(G) : 0));
  return p;
}

template <int HD>
void launch_readout_bwd(const float* gk, int64_t ldk, const float* act, int64_t lda, const float* bw,
                        const float* wout, int64_t H, int64_t G, int64_t nb, float* gact, float* gwout, float* gbout,
                        float scale, float* ws, hipStream_t st) {
  const RbPlan p = rb_plan(H, HD, G, nb);
  const bool vec = ldk % 4 == 0 && lda % 4 == 0 && (reinterpret_cast<uintptr_t>(gk) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(act) & 15) == 0 && (reinterpret_cast<uintptr_t>(bw) & 15) == 0;
  float* ga = p.hs > 1 ? ws + p.gact_part : gact;
  const int64_t gslice = int64_t(nb) * HD * G;
  const dim3 grd(unsigned(p.ngb), unsigned(p.hs), unsigned(nb));
  float* gbp = gbout ? ws + p.gb_part : nullptr;
  if (vec)
    hipLaunchKernelGGL((siren_readout_bwd_kernel<HD, true>), grd, dim3(kRbThreads), 0, st, gk, ldk, act, lda, bw,
                       wout, G, int(H), p.hslice, ga, gslice, ws + p.gw_part, gbp);
  else
    hipLaunchKernelGGL((siren_readout_bwd_kernel<HD, false>), grd, dim3(kRbThreads), 0, st, gk, ldk, act, lda, bw,
                       wout, G, int(H), p.hslice, ga, gslice, ws + p.gw_part, gbp);
  if (p.hs > 1)
    hipLaunchKernelGGL(siren_sum_parts_kernel, dim3(unsigned(ceil_div(gslice, 256))), dim3(256), 0, st, ga,
                       int64_t(p.hs), gslice, gact, 1.f);
  const int64_t nparts = nb * p.ngb, nw = H * HD;
  hipLaunchKernelGGL(siren_sum_parts_kernel, dim3(unsigned(ceil_div(nw, 256))), dim3(256), 0, st, ws + p.gw_part,
                     nparts, nw, gwout, scale);
  if (gbout)
    hipLaunchKernelGGL(siren_sum_parts_kernel, dim3(unsigned(ceil_div(H, 256))), dim3(256), 0, st, gbp, nparts, H,
                       gbout, scale);
}

constexpr int kSirenMaxLds = 160 * 1024;

// LDS bytes per wave of the backward pass 1.
inline int delta_lds_per_wave(int E, int HD, int nh) {
  const int D = E > HD ? E : HD;
  return (2 * (nh + 1) + 2) * 16 * (D + 4) * int(sizeof(float));
}

template <int E, int HD>
struct SirenDelta {
  static void run(const float* gact, int64_t sj, int64_t sg, int64_t ss, const float* grid, int64_t G, int64_t Gp,
                  int64_t nb, const SirenNet& n, float* act, float* del, float* gridT, float* fdh, float* fds,
                  hipStream_t st) {
    const int per = delta_lds_per_wave(E, HD, n.nh);
    int waves = kSirenMaxLds / per;
    waves = waves > kSirenWaves ? kSirenWaves : waves;
    const dim3 grd(unsigned(ceil_div(G, 16 * waves)), unsigned(nb));
    const size_t lds = size_t(per) * waves;
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&siren_bwd_delta_kernel<E, HD>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    hipLaunchKernelGGL((siren_bwd_delta_kernel<E, HD>), grd, dim3(64 * waves), lds, st, gact, sj, sg, ss, grid, G,
                       Gp, n, act, del, gridT, fdh, fds, waves);
  }
};

// FiLM gradients gfilm[s][f][c][o] (c = 0: gamma, 1: beta) = sum_{g < G} of row f * HD + o of fds (gamma) or fdh
// (beta) over sample s's columns [s Gp, s Gp + G): one wave per output, lanes over the points, a fixed butterfly
// adds the lanes (deterministic).
__global__ __launch_bounds__(256) void siren_film_grad_kernel(const float* __restrict__ fdh,
                                                              const float* __restrict__ fds, int64_t GT, int64_t Gp,
                                                              int64_t G, int64_t nb, int nfilm, int HD,
                                                              float* __restrict__ gfilm) {
  const int64_t e = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = int(threadIdx.x) & 63;
  if (e >= nb * nfilm * 2 * HD) return;  // a whole wave leaves together
  const int o = int(e % HD);
  const int c = int((e / HD) % 2);
  const int f = int((e / (2 * HD)) % nfilm);
  const int64_t smp = e / (int64_t(2) * HD * nfilm);
  const float* row = (c == 0 ? fds : fdh) + (int64_t(f) * HD + o) * GT + smp * Gp;
  float acc = 0.f;
  for (int64_t g = lane; g < G; g += 64) acc += row[g];
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) acc += __shfl_xor(acc, w);
  if (lane == 0) gfilm[e] = acc;
}

// Points per Gram workgroup: enough chunks that M/16 x chunks reaches ~2048
// workgroups (8 per CU), at least 64 points (16 per wave) and a multiple of 64.
int64_t gram_chunk(int64_t G, int M) {
  const int64_t tiles = M / 16;
  int64_t chunks = ceil_div(2048, tiles);
  const int64_t cmax = ceil_div(G, 64);
  chunks = chunks < 1 ? 1 : (chunks > cmax ? cmax : chunks);
  return ceil_div(ceil_div(G, chunks), 64) * 64;
}
int64_t gram_chunks(int64_t G, int M) { return ceil_div(G, gram_chunk(G, M)); }

template <int NT>
void launch_gram(const float* X, int64_t ldx, const float* Y, int64_t ldy, int NY, int64_t G, int M, float* part,
                 float* rpart, hipStream_t st) {
  const bool vec = ldx % 4 == 0 && ldy % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(Y) & 15) == 0;
  const int64_t chunk = gram_chunk(G, M);
  const dim3 grd(unsigned(M / 16), unsigned(gram_chunks(G, M)));
  if (vec)
    hipLaunchKernelGGL((siren_gram_kernel<NT, true>), grd, dim3(kSirenThreads), 0, st, X, ldx, Y, ldy, NY, G, M,
                       chunk, part, rpart);
  else
    hipLaunchKernelGGL((siren_gram_kernel<NT, false>), grd, dim3(kSirenThreads), 0, st, X, ldx, Y, ldy, NY, G, M,
                       chunk, part, rpart);
}

// Output tiles of 16 columns a Gram launch covers for NY columns: 1, 2, 4 or 8.
int gram_nt(int NY) { return NY <= 16 ? 1 : (NY <= 32 ? 2 : (NY <= 64 ? 4 : 8)); }

void gram(const float* X, int64_t ldx, const float* Y, int64_t ldy, int NY, int64_t G, int M, float* out, float* rout,
          float* part, float* rpart, hipStream_t st) {
  const int NT = gram_nt(NY);
  switch (NT) {
    case 1: launch_gram<1>(X, ldx, Y, ldy, NY, G, M, part, rpart, st); break;
    case 2: launch_gram<2>(X, ldx, Y, ldy, NY, G, M, part, rpart, st); break;
    case 4: launch_gram<4>(X, ldx, Y, ldy, NY, G, M, part, rpart, st); break;
    default: launch_gram<8>(X, ldx, Y, ldy, NY, G, M, part, rpart, st); break;
  }
  const int NP = 16 * NT;
  const int64_t nwaves = int64_t(M) * NY + M;
  hipLaunchKernelGGL(siren_reduce_kernel, dim3(unsigned(ceil_div(nwaves, 4))), dim3(256), 0, st, part,
                     gram_chunks(G, M), M, NP, NY, out, rpart, rout);
}

// Workspace layout (floats): act [E + nh HD][GT], del [same], gridT [d][GT],
// part [chunks][max(E, HD)][max NT*16], rpart [chunks][max(E, HD)], and the
// FiLM rows fdh, fds [nfilm HD][GT].  GT = nb Gp: every row holds the nb
// samples side by side (one sample: Gp columns, its Gram launches over G).
struct SirenWs {
  int64_t Gp, GT, GG, rows;
  size_t act, del, gridT, part, rpart, fdh, fds, total;  // float offsets / count
};

SirenWs siren_ws(int64_t G, int d, int E, int nh, int HD, int64_t nb = 1, int nfilm = 0) {
  SirenWs w;
  w.Gp = (G + 15) / 16 * 16;
  w.GT = nb * w.Gp;
  w.GG = nb == 1 ? G : w.GT;  // points of the Gram launches (zeros at each sample's padding)
  w.rows = E + int64_t(nh) * HD;
  // partial sums of the largest Gram launch: hidden (M = HD, N = E or HD), embedding (M = E, N = d)
  auto psz = [&](int64_t M, int NY) { return size_t(gram_chunks(w.GG, int(M))) * M * 16 * gram_nt(NY); };
  auto rsz = [&](int64_t M) { return size_t(gram_chunks(w.GG, int(M))) * M; };
  size_t pmax = psz(HD, E > HD ? E : HD);
  pmax = psz(E, d) > pmax ? psz(E, d) : pmax;
  size_t rmax = rsz(HD) > rsz(E) ? rsz(HD) : rsz(E);
  auto al = [](size_t v) { return (v + 63) / 64 * 64; };  // 256-byte sub-buffers
  w.act = 0;
  w.del = al(w.act + size_t(w.rows) * w.GT);
  w.gridT = al(w.del + size_t(w.rows) * w.GT);
  w.part = al(w.gridT + size_t(d) * w.GT);
  w.rpart = al(w.part + pmax);
  w.fdh = al(w.rpart + rmax);
  w.fds = al(w.fdh + size_t(nfilm) * HD * w.GT);
  w.total = al(w.fds + size_t(nfilm) * HD * w.GT);
  return w;
}

int siren_validate(const float* grid, int64_t G, int d, const float* w0, int E, const float* wh, int nh, int HD) {
  NSQ_CHECK_ARG(grid && w0 && wh, "siren_mlp: null weight or grid pointer");
  NSQ_CHECK_ARG(G >= 1 && G <= (int64_t(1) << 30), "siren_mlp: G=%lld out of range", (long long)G);
  NSQ_CHECK_ARG(d >= 1 && d <= 3, "siren_mlp: data_dim %d must be 1..3", d);
  NSQ_CHECK_ARG(nh >= 1 && nh <= 8, "siren_mlp: hidden layer count %d must be 1..8", nh);
  if (!siren_dims_ok(E, HD)) {
    set_error("siren_mlp: embedding_dim %d and mlp_hidden_dim %d must each be 16, 32, 64 or 128", E, HD);
    return NSQ_ERR_UNSUPPORTED;
  }
  return NSQ_OK;
}

}  // namespace

size_t siren_readout_bwd_ws_floats(int64_t H, int HD, int64_t G, int64_t nb) { return rb_plan(H, HD, G, nb).total; }

bool siren_readout_bwd_run(const float* gk, int64_t ldk, const float* act, int64_t lda, const float* bw,
                           const float* wout, int64_t H, int HD, int64_t G, int64_t nb, float* gact, float* gwout,
                           float* gbout, float scale, float* ws, hipStream_t st) {
  switch (HD) {
    case 16: launch_readout_bwd<16>(gk, ldk, act, lda, bw, wout, H, G, nb, gact, gwout, gbout, scale, ws, st); return true;
    case 32: launch_readout_bwd<32>(gk, ldk, act, lda, bw, wout, H, G, nb, gact, gwout, gbout, scale, ws, st); return true;
    case 64: launch_readout_bwd<64>(gk, ldk, act, lda, bw, wout, H, G, nb, gact, gwout, gbout, scale, ws, st); return true;
    default: return false;
  }
}
}  // namespace nsq

extern "C" {

int nsq_siren_mlp_film_fwd(const float* grid, int64_t G, int d, const float* w0, const float* b0, int E,
                           const float* wh, const float* bh, int nh, int HD, const float* film, int64_t nb,
                           int film_first, float* act, int64_t lda, void* stream) {
  using namespace nsq;
  clear_error();
  int rc = siren_validate(grid, G, d, w0, E, wh, nh, HD);
  if (rc) return rc;
  NSQ_CHECK_ARG(act && lda >= G, "siren_mlp_fwd: null output or row stride %lld < G", (long long)lda);
  NSQ_CHECK_ARG(nb >= 1 && nb <= 65535, "siren_mlp_fwd: %lld samples out of range", (long long)nb);
  NSQ_CHECK_ARG(film || (nb == 1 && !film_first), "siren_mlp_fwd: several samples or film_first need FiLM parameters");
  NSQ_CHECK_ARG(!film_first || E == HD, "siren_mlp_fwd: FiLM after the embedding needs embedding_dim %d == "
                "mlp_hidden_dim %d", E, HD);
  SirenNet n{w0, b0, wh, bh, d, nh};
  n.film = film;
  n.film_first = film_first ? 1 : 0;
  siren_dispatch<SirenFwd>(E, HD, grid, G, n, act, lda, nb, (hipStream_t)stream);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

int nsq_siren_mlp_fwd(const float* grid, int64_t G, int d, const float* w0, const float* b0, int E, const float* wh,
                      const float* bh, int nh, int HD, float* act, int64_t lda, void* stream) {
  return nsq_siren_mlp_film_fwd(grid, G, d, w0, b0, E, wh, bh, nh, HD, nullptr, 1, 0, act, lda, stream);
}

int nsq_siren_film_readout_fwd(const float* wout, const float* bout, int64_t H, int HD, const float* act,
                               int64_t lda, int64_t G, int64_t nb, float* k, void* stream) {
  using namespace nsq;
  clear_error();
  NSQ_CHECK_ARG(nb >= 1 && nb <= 65535, "siren_readout_fwd: %lld samples out of range", (long long)nb);
  NSQ_CHECK_ARG(wout && act && k, "siren_readout_fwd: null pointer argument");
  NSQ_CHECK_ARG(G >= 1 && G <= (int64_t(1) << 30) && lda >= G, "siren_readout_fwd: G=%lld, lda=%lld", (long long)G,
                (long long)lda);
  NSQ_CHECK_ARG(H >= 1 && H <= (int64_t(1) << 20), "siren_readout_fwd: H=%lld out of range", (long long)H);
  NSQ_CHECK_ARG(ceil_div(H, int64_t(64)) <= 65535, "siren_readout_fwd: H=%lld too large", (long long)H);
  hipStream_t st = (hipStream_t)stream;
  switch (HD) {
    case 16: launch_readout<16>(wout, bout, act, lda, G, H, k, nb, st); break;
    case 32: launch_readout<32>(wout, bout, act, lda, G, H, k, nb, st); break;
    case 64: launch_readout<64>(wout, bout, act, lda, G, H, k, nb, st); break;
    case 128: launch_readout<128>(wout, bout, act, lda, G, H, k, nb, st); break;
    default:
      set_error("siren_readout_fwd: mlp_hidden_dim %d must be 16, 32, 64 or 128", HD);
      return NSQ_ERR_UNSUPPORTED;
  }
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

int nsq_siren_readout_fwd(const float* wout, const float* bout, int64_t H, int HD, const float* act, int64_t lda,
                          int64_t G, float* k, void* stream) {
  return nsq_siren_film_readout_fwd(wout, bout, H, HD, act, lda, G, 1, k, stream);
}

size_t nsq_siren_readout_bwd_workspace_bytes(int64_t H, int HD, int64_t G, int64_t nb) {
  if (H < 1 || G < 1 || G > (int64_t(1) << 23) || nb < 1 || !(HD == 16 || HD == 32 || HD == 64)) return 0;
  return nsq::rb_plan(H, HD, G, nb).total * sizeof(float);
}

int nsq_siren_readout_bwd(const float* gk, int64_t ldk, const float* act, int64_t lda, const float* wout, int64_t H,
                          int HD, int64_t G, int64_t nb, float* gact, float* gwout, float* gbout, void* workspace,
                          size_t workspace_bytes, void* stream) {
  using namespace nsq;
  clear_error();
  NSQ_CHECK_ARG(gk && act && wout && gact && gwout, "siren_readout_bwd: null pointer argument");
  NSQ_CHECK_ARG(G >= 1 && ldk >= G && lda >= G && ldk <= (int64_t(1) << 23),
                "siren_readout_bwd: G=%lld, ldk=%lld, lda=%lld (rows of at most 2^23 points)", (long long)G,
                (long long)ldk, (long long)lda);
  NSQ_CHECK_ARG(H >= 1 && H <= (int64_t(1) << 20), "siren_readout_bwd: H=%lld out of range", (long long)H);
  NSQ_CHECK_ARG(nb >= 1 && nb <= 65535, "siren_readout_bwd: %lld samples out of range", (long long)nb);
  if (!(HD == 16 || HD == 32 || HD == 64)) {
    set_error("siren_readout_bwd: mlp_hidden_dim %d must be 16, 32 or 64", HD);
    return NSQ_ERR_UNSUPPORTED;
  }
  const RbPlan p = rb_plan(H, HD, G, nb);
  NSQ_CHECK_ARG(p.ngb <= 0x7fffffff && p.hs <= 65535, "siren_readout_bwd: launch grid too large");
  NSQ_CHECK_ARG(workspace && workspace_bytes >= p.total * sizeof(float),
                "siren_readout_bwd: workspace of %zu bytes required, got %zu", p.total * sizeof(float),
                workspace_bytes);
  hipStream_t st = (hipStream_t)stream;
  float* ws = static_cast<float*>(workspace);
  switch (HD) {
    case 16: launch_readout_bwd<16>(gk, ldk, act, lda, nullptr, wout, H, G, nb, gact, gwout, gbout, 1.f, ws, st); break;
    case 32: launch_readout_bwd<32>(gk, ldk, act, lda, nullptr, wout, H, G, nb, gact, gwout, gbout, 1.f, ws, st); break;
    default: launch_readout_bwd<64>(gk, ldk, act, lda, nullptr, wout, H, G, nb, gact, gwout, gbout, 1.f, ws, st); break;
  }
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

size_t nsq_siren_mlp_film_bwd_workspace_bytes(int64_t G, int d, int E, int nh, int HD, int64_t nb, int film_first) {
  if (G < 1 || d < 1 || d > 3 || nh < 1 || nh > 8 || !nsq::siren_dims_ok(E, HD) || nb < 1 || nb > 65535) return 0;
  if (film_first && E != HD) return 0;
  return nsq::siren_ws(G, d, E, nh, HD, nb, nh + (film_first ? 1 : 0)).total * sizeof(float);
}

size_t nsq_siren_mlp_bwd_workspace_bytes(int64_t G, int d, int E, int nh, int HD) {
  if (G < 1 || d < 1 || d > 3 || nh < 1 || nh > 8 || !nsq::siren_dims_ok(E, HD)) return 0;
  return nsq::siren_ws(G, d, E, nh, HD).total * sizeof(float);
}

int nsq_siren_mlp_film_bwd(const float* gact, int64_t gact_stride_j, int64_t gact_stride_g, int64_t gact_stride_s,
                           const float* grid, int64_t G, int d, const float* w0, const float* b0, int E,
                           const float* wh, const float* bh, int nh, int HD, const float* film, int64_t nb,
                           int film_first, float* gw0, float* gb0, float* gwh, float* gbh, float* gfilm,
                           void* workspace, size_t workspace_bytes, void* stream) {
  using namespace nsq;
  clear_error();
  int rc = siren_validate(grid, G, d, w0, E, wh, nh, HD);
  if (rc) return rc;
  NSQ_CHECK_ARG(gact && gw0 && gwh, "siren_mlp_bwd: null gradient pointer");
  NSQ_CHECK_ARG(gact_stride_j >= 0 && gact_stride_g >= 0 && gact_stride_s >= 0, "siren_mlp_bwd: negative gact stride");
  NSQ_CHECK_ARG(!b0 || gb0, "siren_mlp_bwd: gb0 required with b0");
  NSQ_CHECK_ARG(!bh || gbh, "siren_mlp_bwd: gbh required with bh");
  NSQ_CHECK_ARG(nb >= 1 && nb <= 65535, "siren_mlp_bwd: %lld samples out of range", (long long)nb);
  NSQ_CHECK_ARG(film || (nb == 1 && !film_first), "siren_mlp_bwd: several samples or film_first need FiLM parameters");
  NSQ_CHECK_ARG(!film || gfilm, "siren_mlp_bwd: gfilm required with FiLM parameters");
  NSQ_CHECK_ARG(!film_first || E == HD, "siren_mlp_bwd: FiLM after the embedding needs embedding_dim %d == "
                "mlp_hidden_dim %d", E, HD);
  const int nfilm = film ? nh + (film_first ? 1 : 0) : 0;
  const SirenWs w = siren_ws(G, d, E, nh, HD, nb, nfilm);
  NSQ_CHECK_ARG(workspace && workspace_bytes >= w.total * sizeof(float),
                "siren_mlp_bwd: workspace of %zu bytes required, got %zu", w.total * sizeof(float), workspace_bytes);
  NSQ_CHECK_ARG(delta_lds_per_wave(E, HD, nh) <= kSirenMaxLds, "siren_mlp_bwd: %d hidden layers of %d too large", nh,
                HD);
  hipStream_t st = (hipStream_t)stream;
  float* ws = static_cast<float*>(workspace);
  float* act = ws + w.act;
  float* del = ws + w.del;
  float* gridT = ws + w.gridT;
  float* part = ws + w.part;
  float* rpart = ws + w.rpart;
  SirenNet n{w0, b0, wh, bh, d, nh};
  n.film = film;
  n.film_first = film_first ? 1 : 0;
  siren_dispatch<SirenDelta>(E, HD, gact, gact_stride_j, gact_stride_g, gact_stride_s, grid, G, w.Gp, nb, n, act, del,
                             gridT, ws + w.fdh, ws + w.fds, st);
  // hidden layers i = nh..1: X = delta_i^T [HD], Y = a_{i-1}^T [IN] (summed over the samples' columns)
  for (int i = nh; i >= 1; --i) {
    const int IN = i == 1 ? E : HD;
    const int64_t xo = E + int64_t(i - 1) * HD, yo = i == 1 ? 0 : E + int64_t(i - 2) * HD;
    float* gw = gwh + (i == 1 ? 0 : int64_t(HD) * E + int64_t(i - 2) * HD * HD);
    gram(del + xo * w.GT, w.GT, act + yo * w.GT, w.GT, IN, w.GG, HD, gw, gbh ? gbh + (i - 1) * HD : nullptr, part,
         rpart, st);
  }
  // positional embedding: X = delta_0^T [E], Y = grid^T [d] (rows >= d read as zero)
  gram(del, w.GT, gridT, w.GT, d, w.GG, E, gw0, gb0, part, rpart, st);
  if (film) {
    const int64_t nout = nb * nfilm * 2 * HD;
    hipLaunchKernelGGL(siren_film_grad_kernel, dim3(unsigned(ceil_div(nout, 4))), dim3(256), 0, st, ws + w.fdh,
                       ws + w.fds, w.GT, w.Gp, G, nb, nfilm, HD, gfilm);
  }
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}

int nsq_siren_mlp_bwd(const float* gact, int64_t gact_stride_j, int64_t gact_stride_g, const float* grid, int64_t G,
                      int d, const float* w0, const float* b0, int E, const float* wh, const float* bh, int nh, int HD,
                      float* gw0, float* gb0, float* gwh, float* gbh, void* workspace, size_t workspace_bytes,
                      void* stream) {
  return nsq_siren_mlp_film_bwd(gact, gact_stride_j, gact_stride_g, 0, grid, G, d, w0, b0, E, wh, bh, nh, HD, nullptr,
                                1, 0, gw0, gb0, gwh, gbh, nullptr, workspace, workspace_bytes, stream);
}

}  // extern "C"
