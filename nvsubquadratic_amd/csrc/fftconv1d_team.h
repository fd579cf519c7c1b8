// Causal 1D FFT convolution, "team" plan: the 4-step transform of each
// channel with its column/row exchange kept on chip.
//
// The multi-kernel 4-step plan (fftconv1d_impl.h) moves every channel's
// complex intermediates through HBM between its column and row halves: six
// 2 MB round trips per channel at config 3, 6x the compulsory bytes.  Here
// one cooperative kernel runs the whole transform:
//
//  * 512-thread workgroups, two per CU; the workgroups of one XCD (read from
//    the hardware XCC_ID register, not assumed from blockIdx) form two teams,
//    and a team owns whole channels (h = t, t + nteams, ...);
//  * per channel three phases, each split over the team's workgroups:
//      A  column DFTs of x and k (HBM in) -> X', K' into the team's exchange
//         region (ordinary stores: they land in the XCD's L2),
//      B  row DFTs of X', K' row pairs, spectral product, inverse row DFTs ->
//         Y' in place of X',
//      C  inverse column DFTs of Y' -> crop / cast / shortcut -> y (HBM out);
//  * between phases a team barrier: each workgroup drains its stores
//    (s_waitcnt vmcnt(0)) and bumps the phase counter; waiters poll it and then
//    read the region with sc1 loads, which miss the CU's L1 and hit the shared
//    L2.  No agent-scope fence is used: its release writes back the L2 and its
//    acquire invalidates it, which is the traffic this plan exists to avoid;
//  * software pipeline over the team's channels: iteration s runs A(s),
//    C(s-1), B(s), so every wait is one phase of work after the arrivals it
//    needs, and the regions are double-buffered by channel parity;
//  * every wait is bounded: a timeout sets a status word and an abort flag in
//    the workspace, and every workgroup leaves at its next wait, so the grid
//    always drains.
//
// Workspace: a TeamCtl block, then 2 regions per team of NSIG complex signals
// of N = F/2 values (forward: X', K'; backward: G', X', K'), sized for up to
// kTeamMaxTeams teams whatever the device has.  Its size does not depend on D.
//
// Measured on MI355X at config 3 (per workgroup, two per CU): barrier waits
// take 18% of the forward; each phase runs at the rate of the same FFT code in
// the multi-kernel plan (a row tile of 4 pairs, L2-resident, alone: 12 us per
// CU, as row_fwd_kernel).  The exchange staying on chip does not pay while the
// row FFTs, not HBM, bound both plans.
#pragma once

#include "fftconv1d_impl.h"

namespace nsq {

constexpr int kTeamThreads = 512;
constexpr int kTeamMaxX = 16;           // XCC_ID is 4 bits
constexpr int kTeamSub = 2;             // teams per XCD: two workgroups per CU, one of each, interleave
constexpr int kTeamMaxTeams = kTeamMaxX * kTeamSub;
constexpr size_t kTeamCtlBytes = 16384;  // TeamCtl, padded
constexpr int kTeamMaxSpin = 1 << 21;    // ~1 s of polling at ~0.5 us per poll

struct TeamCtl {
  int reg[kTeamMaxX];  // workgroups registered per XCC
  int arrived;         // registration barrier
  int status;          // 0: ok; 1: a wait timed out (results invalid)
  int abort;           // set with status: every workgroup leaves at its next wait
  int pad[45];
  int bar[kTeamMaxTeams][64];  // per team: phase counters at [0], [16], [32], [48] (separate 64-byte sectors)
};
static_assert(sizeof(TeamCtl) <= kTeamCtlBytes, "TeamCtl: block size");

__device__ __forceinline__ int team_ld(const int* p) {
  return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void team_fail(TeamCtl* ctl) {
  __hip_atomic_store(&ctl->status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&ctl->abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Thread 0 polls `*cnt >= target` (bounded); the verdict reaches every thread
// through LDS.  Returns false on timeout or abort: the caller returns.
__device__ __forceinline__ bool team_wait(int* cnt, int target, TeamCtl* ctl, int max_spin) {
  __shared__ int ok;
  if (threadIdx.x == 0) {
    int good = 0;
    for (int i = 0; i < max_spin; ++i) {
      if (team_ld(cnt) >= target) {
        good = 1;
        break;
      }
      if (team_ld(&ctl->abort)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    if (!good && !team_ld(&ctl->abort)) team_fail(ctl);
    ok = good;
  }
  __syncthreads();
  const int r = ok;
  __syncthreads();  // `ok` is rewritten by the next wait
  return r;
}

// Every store of this workgroup is acknowledged by the L2 before the counter
// moves, so a waiter that sees the count also sees the data (in the L2 of this
// XCD, where every member of the team reads).
__device__ __forceinline__ void team_arrive(int* cnt) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct Team {
  int rank, P, t, n;  // rank in the team, team size, team index, number of teams
};

// Registration: each workgroup joins its XCD's group, in which the k-th
// arrival joins team k % kTeamSub; after every workgroup has registered, team
// sizes and dense team indices follow.  Both teams of an XCD share its L2, and
// with two workgroups resident per CU one team computes while the other waits
// on memory.
__device__ __forceinline__ bool team_join(TeamCtl* ctl, Team& tm, int max_spin) {
  __shared__ int sh[5];
  if (threadIdx.x == 0) {
    const int x = __builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11)) & (kTeamMaxX - 1);  // HW_REG_XCC_ID
    const int rank = __hip_atomic_fetch_add(&ctl->reg[x], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_fetch_add(&ctl->arrived, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int good = 0;
    for (int i = 0; i < max_spin; ++i) {
      if (team_ld(&ctl->arrived) >= int(gridDim.x)) {
        good = 1;
        break;
      }
      if (team_ld(&ctl->abort)) break;
      __builtin_amdgcn_s_sleep(2);
    }
    if (!good && !team_ld(&ctl->abort)) team_fail(ctl);
    int t = 0, n = 0;
    for (int j = 0; j < kTeamMaxX; ++j) {
      const int c = team_ld(&ctl->reg[j]);
      if (c > 0) {
        t += j < x ? 1 : 0;
        ++n;
      }
    }
    const int cnt = team_ld(&ctl->reg[x]);
    const int sub = rank % kTeamSub;
    sh[0] = rank / kTeamSub;
    sh[1] = (cnt - sub + kTeamSub - 1) / kTeamSub;  // members of team `sub` of this XCD
    sh[2] = t * kTeamSub + sub;
    sh[3] = n * kTeamSub;
    sh[4] = good;
  }
  __syncthreads();
  tm = Team{sh[0], sh[1], sh[2], sh[3]};
  const bool ok = sh[4] != 0;
  __syncthreads();
  return ok;
}

// Complex values of the exchange region read through the L2 (sc1: the load
// misses this CU's L1, whose lines may hold an earlier channel's values).
struct L2Signal {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ explicit L2Signal(const float2* base, int64_t n)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<float2*>(base), 0, int(n * int64_t(sizeof(float2))),
                                            0x00020000)) {}
  __device__ __forceinline__ float2 operator[](int i) const {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, i * int(sizeof(float2)), 0, 16));
  }
};

// ---------------------------------------------------------------------------
// Phase A: one column tile (M columns c0..c0+M-1 of the N1 x N2 matrix) of a
// real row, transformed and twiddled into `out` (col_fwd_kernel's tile body).
// ---------------------------------------------------------------------------
template <int LOGN1, int LOGN, int DT, bool AL, bool HALF>
__device__ __forceinline__ void team_col_fwd(const typename Elem<DT>::T* __restrict__ row, int64_t valid, int c0,
                                             float2* __restrict__ out, const float2* __restrict__ tw, float2* lds) {
  using C = ColCfg<LOGN1>;
  static_assert(C::T == kTeamThreads, "team_col_fwd: one tile per workgroup");
  constexpr int N2 = 1 << (LOGN - LOGN1);
  constexpr int R = 1 << (LOGN1 < 4 ? LOGN1 : 4);
  const RowBuf<DT, AL> in(row, valid);
  auto ld0 = [&](int m, int n) -> float2 { return in.load_pair(2 * (int64_t(n) * N2 + c0 + m)); };
  HalfZeroLoad<R, HALF, decltype(ld0)> ld{ld0};
  LdsTile<C::S, false> tile{lds};
  TwiddledColumnStore<LOGN, N2> st{out, c0, tw};
  fft_rec<LOGN1, 0, false, C::M, C::T, true>(ld, tile, tile, st, tw);
}

// First-pass loader of an inverse column tile from the exchange region:
// B[k1][n2] W_N^{-n2 k1} (as TwiddledColumnLoad, through the L2).
template <int LOGN, int N2, int R, int NR>
struct TeamColumnLoad {
  L2Signal src;
  int c0;
  const float2* tw;
  int q = 0;
  float2 w, step;
  __device__ __forceinline__ float2 operator()(int m, int k1) {
    const uint32_t n2 = uint32_t(c0 + m);
    if (q % R == 0) {
      w = root<LOGN>(tw, n2 * uint32_t(k1));
      step = root<LOGN>(tw, n2 * uint32_t(NR));
    }
    const float2 v = cmulc(src[k1 * N2 + c0 + m], w);
    if (q % R != R - 1) w = cmul(w, step);
    ++q;
    return v;
  }
};

// Phase C: inverse column tile; epi(m, v) receives packed output index m.
template <int LOGN1, int LOGN, class EPI>
__device__ __forceinline__ void team_col_inv(const float2* sig, int c0, EPI& epi, const float2* __restrict__ tw,
                                             float2* lds) {
  using C = ColCfg<LOGN1>;
  static_assert(C::T == kTeamThreads, "team_col_inv: one tile per workgroup");
  constexpr int N2 = 1 << (LOGN - LOGN1);
  constexpr int R = 1 << (LOGN1 < 4 ? LOGN1 : 4);
  constexpr int NR = C::N1 / R;
  TeamColumnLoad<LOGN, N2, R, NR> ld{L2Signal(sig, int64_t(1) << LOGN), c0, tw};
  auto st = [&](int m, int n1, float2 v) { epi(int64_t(n1) * N2 + c0 + m, v); };
  fft<LOGN1, true, C::M, C::T, C::S, true>(lds, ld, st, tw);
}

// Row pairs per workgroup tile in phase B.
template <int LOGN2>
struct TeamRowCfg {
  static constexpr int TP = RowCfg<LOGN2>::T;    // threads of one row pair
  static constexpr int NP = kTeamThreads / TP;   // row pairs per tile
  static constexpr int M = 2 * NP;               // rows per tile
  static constexpr int N2P = RowCfg<LOGN2>::N2P;
  static_assert(NP >= 1 && NP * TP == kTeamThreads, "TeamRowCfg: row pairs must fill the workgroup");
};

// Tile row m of row-pair tile q0: pair q = q0 + m/2 holds rows q and N1-q
// (q = 0: rows 0 and N1/2).
template <int LOGN1>
__device__ __forceinline__ int team_row_of(int q0, int m) {
  constexpr int N1 = 1 << LOGN1;
  const int q = q0 + (m >> 1);
  return (m & 1) ? (q == 0 ? N1 / 2 : N1 - q) : q;
}

// Phase B (forward): rows of NP pairs: K row spectra to registers (slot form),
// X row spectra times them, inverse rows written over X'.
template <int LOGN1, int LOGN2>
__device__ __forceinline__ void team_rows_fwd(float2* xsig, const float2* ksig, int q0, const float2* __restrict__ tw,
                                              float2* lds) {
  using TC = TeamRowCfg<LOGN2>;
  using RS = RowSlots<LOGN1, LOGN2>;
  constexpr int N2 = 1 << LOGN2, N = 1 << (LOGN1 + LOGN2);
  constexpr int SLOTS = RowCfg<LOGN2>::SLOTS;
  const int tid = opaque_tid();
  const int sp = tid / TC::TP, tl = tid % TC::TP;
  float2* sub = lds + sp * 2 * TC::N2P;
  LdsTile<TC::N2P, true> tile{lds};
  const L2Signal kin(ksig, N), xin(xsig, N);
  auto ldk = [&](int m, int n) -> float2 { return kin[team_row_of<LOGN1>(q0, m) * N2 + n]; };
  auto ldx = [&](int m, int n) -> float2 { return xin[team_row_of<LOGN1>(q0, m) * N2 + n]; };
  auto sty = [&](int m, int n, float2 v) { xsig[int64_t(team_row_of<LOGN1>(q0, m)) * N2 + n] = v; };
  if constexpr (LOGN2 == kRegPairLogN2) {  // the multi-kernel row_fwd_kernel's transforms, pair by pair
    const int q = q0 + sp;
    float2 v[4][4], hA[SLOTS], hB[SLOTS];
    rows1024_fwd_head<TC::M, kTeamThreads>(lds, ldk, tw);
    regpair_fwd_slots<LOGN1, false>(sub, q, tl, tw, v, [&](int i, bool, float2& A, float2& Bc) {
      hA[i] = A;
      hB[i] = Bc;
    });
    rows1024_fwd_head<TC::M, kTeamThreads>(lds, ldx, tw);
    regpair_fwd_slots<LOGN1, true>(sub, q, tl, tw, v, [&](int i, bool s0, float2& A, float2& Bc) {
      A = slot_mul(s0, A, hA[i]);
      Bc = cmul(Bc, hB[i]);
    });
    regpair_inverse<TC::M, kTeamThreads>(lds, sub, q, tl, v, sty, tw);
    return;
  }
  fft<LOGN2, false, TC::M, kTeamThreads, TC::N2P>(lds, ldk, tile, tw);
  float2 hA[SLOTS], hB[SLOTS];
  {
    const RS rs(q0 + sp, tw, tl);
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      NSQ_SLOT_FENCE();
      row_unpack(sub, rs, i, hA[i], hB[i]);
    }
  }
  __syncthreads();
  fft<LOGN2, false, TC::M, kTeamThreads, TC::N2P>(lds, ldx, tile, tw);
  {
    const RS rs(q0 + sp, tw, tl);
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      NSQ_SLOT_FENCE();
      float2 A, Bc;
      row_unpack(sub, rs, i, A, Bc);
      row_repack(sub, rs, i, slot_mul(rs.s0(i), A, hA[i]), cmul(Bc, hB[i]));
    }
  }
  __syncthreads();
  fft<LOGN2, true, TC::M, kTeamThreads, TC::N2P>(lds, tile, sty, tw);
}

// Phase B (backward, one batch row): order K -> G -> X as row_bwd1_kernel.
// gx pre-image (G conj K, inverse rows) written over K', gk pre-image
// (G conj X, inverse rows) over X'.
template <int LOGN1, int LOGN2>
__device__ __forceinline__ void team_rows_bwd(const float2* gsig, float2* xsig, float2* ksig, int q0,
                                              const float2* __restrict__ tw, float2* lds) {
  using TC = TeamRowCfg<LOGN2>;
  using RS = RowSlots<LOGN1, LOGN2>;
  constexpr int N2 = 1 << LOGN2, N = 1 << (LOGN1 + LOGN2);
  constexpr int SLOTS = RowCfg<LOGN2>::SLOTS;
  const int tid = opaque_tid();
  const int sp = tid / TC::TP, tl = tid % TC::TP;
  float2* sub = lds + sp * 2 * TC::N2P;
  LdsTile<TC::N2P, true> tile{lds};
  const L2Signal kin(ksig, N), gin(gsig, N), xin(xsig, N);
  if constexpr (LOGN2 == kRegPairLogN2) {  // the multi-kernel row_bwd1_kernel's transforms, pair by pair
    auto ldk = [&](int m, int n) -> float2 { return kin[team_row_of<LOGN1>(q0, m) * N2 + n]; };
    auto ldg = [&](int m, int n) -> float2 { return gin[team_row_of<LOGN1>(q0, m) * N2 + n]; };
    auto ldx = [&](int m, int n) -> float2 { return xin[team_row_of<LOGN1>(q0, m) * N2 + n]; };
    auto stk = [&](int m, int n, float2 v) { ksig[int64_t(team_row_of<LOGN1>(q0, m)) * N2 + n] = v; };
    auto stx = [&](int m, int n, float2 v) { xsig[int64_t(team_row_of<LOGN1>(q0, m)) * N2 + n] = v; };
    const int q = q0 + sp;
    float2 v[4][4], sA[SLOTS], sB[SLOTS];
    rows1024_fwd_head<TC::M, kTeamThreads>(lds, ldk, tw);
    regpair_fwd_slots<LOGN1, false>(sub, q, tl, tw, v, [&](int i, bool, float2& A, float2& Bc) {
      sA[i] = A;
      sB[i] = Bc;
    });
    rows1024_fwd_head<TC::M, kTeamThreads>(lds, ldg, tw);
    regpair_fwd_slots<LOGN1, true>(sub, q, tl, tw, v, [&](int i, bool s0, float2& A, float2& Bc) {
      const float2 ga = A, gb = Bc;
      A = slot_mulc(s0, ga, sA[i]);
      Bc = cmulc(gb, sB[i]);
      sA[i] = ga;
      sB[i] = gb;
    });
    regpair_inverse<TC::M, kTeamThreads>(lds, sub, q, tl, v, stk, tw);
    rows1024_fwd_head<TC::M, kTeamThreads>(lds, ldx, tw);
    regpair_fwd_slots<LOGN1, true>(sub, q, tl, tw, v, [&](int i, bool s0, float2& A, float2& Bc) {
      A = slot_mulc(s0, sA[i], A);
      Bc = cmulc(sB[i], Bc);
    });
    regpair_inverse<TC::M, kTeamThreads>(lds, sub, q, tl, v, stx, tw);
    return;
  }
  float2 sA[SLOTS], sB[SLOTS];  // K slots, then G slots
  auto ldk = [&](int m, int n) -> float2 { return kin[team_row_of<LOGN1>(q0, m) * N2 + n]; };
  fft<LOGN2, false, TC::M, kTeamThreads, TC::N2P>(lds, ldk, tile, tw);
  {
    const RS rs(q0 + sp, tw, tl);
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      NSQ_SLOT_FENCE();
      row_unpack(sub, rs, i, sA[i], sB[i]);
    }
  }
  __syncthreads();
  auto ldg = [&](int m, int n) -> float2 { return gin[team_row_of<LOGN1>(q0, m) * N2 + n]; };
  fft<LOGN2, false, TC::M, kTeamThreads, TC::N2P>(lds, ldg, tile, tw);
  {
    const RS rs(q0 + sp, tw, tl);
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      NSQ_SLOT_FENCE();
      float2 GA, GB;
      row_unpack(sub, rs, i, GA, GB);
      row_repack(sub, rs, i, slot_mulc(rs.s0(i), GA, sA[i]), cmulc(GB, sB[i]));
      sA[i] = GA;
      sB[i] = GB;
    }
  }
  __syncthreads();
  auto stk = [&](int m, int n, float2 v) { ksig[int64_t(team_row_of<LOGN1>(q0, m)) * N2 + n] = v; };
  fft<LOGN2, true, TC::M, kTeamThreads, TC::N2P>(lds, tile, stk, tw);
  auto ldx = [&](int m, int n) -> float2 { return xin[team_row_of<LOGN1>(q0, m) * N2 + n]; };
  fft<LOGN2, false, TC::M, kTeamThreads, TC::N2P>(lds, ldx, tile, tw);
  {
    const RS rs(q0 + sp, tw, tl);
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      NSQ_SLOT_FENCE();
      float2 XA, XB;
      row_unpack(sub, rs, i, XA, XB);
      row_repack(sub, rs, i, slot_mulc(rs.s0(i), sA[i], XA), cmulc(sB[i], XB));
    }
  }
  __syncthreads();
  auto stx = [&](int m, int n, float2 v) { xsig[int64_t(team_row_of<LOGN1>(q0, m)) * N2 + n] = v; };
  fft<LOGN2, true, TC::M, kTeamThreads, TC::N2P>(lds, tile, stx, tw);
}

// Plans the team kernels are built for: logN in [kTeamMinLogN, kTeamMaxLogN]
// (N1 = 256 columns of 512-thread tiles; N2 = 2^(logN-8) row length).
constexpr int kTeamMinLogN = 16;
constexpr int kTeamMaxLogN = 20;

// Host side (fftconv1d_team.hip).
bool team_plan_ok(const Plan1D& p, int64_t B, int64_t kbatch);
size_t team_workspace_bytes(const Plan1D& p, int direction);
int team_fwd(const Plan1D& p, int dtype, const void* x, const float* k, const void* s, void* y, int H, int L, int K,
             void* ws, const float2* tw, hipStream_t st);
int team_bwd(const Plan1D& p, int dtype, const void* g, const void* x, const float* k, const void* s, void* gx,
             float* gk, float* gs, int H, int L, int K, void* ws, const float2* tw, hipStream_t st);

}  // namespace nsq
