// Hyena gates around the long convolution (nvsubquadratic/modules/hyena_nd.py:546
// and :570): z = q * act1(k) before it, out = y1 * act2(v) after it, with y1 the
// conv output including its shortcut term.  Values are rounded to the I/O dtype
// where the reference's elementwise ops on I/O-dtype tensors round: act(k),
// the product, and each gradient product.
//
// The gates run either inside the fused 1D kernels (loaders and epilogues, see
// fftconv1d_impl.h) or, where the conv is a multi-kernel plan, as the
// elementwise kernels below around it.
#pragma once

#include "fft_core.h"

namespace nsq {

// The gate arithmetic is not contracted into FMAs (`fp contract(off)`): each
// product and sum rounds on its own, as the reference's separate elementwise ops
// do, and identically in every kernel that inlines it (the fused loaders and
// epilogues and the gate kernels give the same bits).
__device__ __forceinline__ float gate_sigmoid(float x) {
#pragma clang fp contract(off)
  return 1.f / (1.f + __expf(-x));
}

// act(x) for act in {identity, sigmoid, silu}
__device__ __forceinline__ float gate_act(int act, float x) {
#pragma clang fp contract(off)
  const float s = gate_sigmoid(x);
  return act == NSQ_GATE_SIGMOID ? s : (act == NSQ_GATE_SILU ? x * s : x);
}

// d act / dx
__device__ __forceinline__ float gate_dact(int act, float x) {
#pragma clang fp contract(off)
  const float s = gate_sigmoid(x);
  return act == NSQ_GATE_SIGMOID ? s * (1.f - s) : (act == NSQ_GATE_SILU ? s * (1.f + x * (1.f - s)) : 1.f);
}

// Pointers of a gated call beyond the conv's own (q is the conv's x, dq its
// gx, dout its g).  y1: the conv output before the second gate (written by a
// forward that keeps it for the backward, read by the backward).
struct GateArgs {
  const void* kg;  // key, gate-1 input
  const void* v;   // value, gate-2 input
  void* y1;
  void* dk;
  void* dv;
  int act1, act2;
};

template <int DT>
__device__ __forceinline__ float gate1(int act, float q, float k) {
#pragma clang fp contract(off)
  return Elem<DT>::round(q * Elem<DT>::round(gate_act(act, k)));
}

// Gates formed inside a conv pass (the N-d passes of fftconv_nd_impl.h, the
// 4-step column passes of fftconv1d_impl.h): GATED_FWD forms z = q act1(kg)
// as the first pass loads and applies gate 2 in the last epilogue; GATED_BWD
// forms dy1 = g act2(v) as the g-side first pass loads and dq, dkg, dv in the
// gx epilogue.  Roundings as gate_ew_kernel's, so the results equal the gate
// kernels composed around the plain conv.
enum { GATED_NONE = 0, GATED_FWD = 1, GATED_BWD = 2 };

// Operands of a gated pass beyond the conv's own (every tensor with the I/O
// layout of the conv's x).
struct GatedIO {
  const void* q;   // gate-1 operand (the forward's x; the backward's x-side and dq, dkg)
  const void* kg;  // gate-1 input
  const void* v;   // gate-2 input
  const void* y1;  // backward: the conv output before gate 2 (for dv)
  void* y1out;     // forward: y1 kept for the backward (may be null)
  void* dv;        // backward: written by the gx epilogue
  void* dkg;       // backward: written by the gx epilogue
  int act1, act2;
};

// The first pass's input from its two loaded operands (FWD: q, kg; BWD: g, v).
template <int DT, int GL>
__device__ __forceinline__ float gated_input(int act1, int act2, float a, float b) {
#pragma clang fp contract(off)
  if constexpr (GL == GATED_FWD)
    return gate1<DT>(act1, a, b);
  else if constexpr (GL == GATED_BWD)
    return Elem<DT>::round(a * Elem<DT>::round(gate_act(act2, b)));
  else
    return a;
}

// One output sample of a gated last pass.  `conv` is the scaled transform
// value, `a` / `b` the operands of the gate formed here (FWD: q, kg -> z, the
// shortcut term's input; BWD: g, v -> dy1 and dv), `c` / `d` / `e` the others
// (FWD: v; BWD: q, kg, y1).  Returns the stored output (FWD: out; BWD: dq) and
// sets o2 (FWD: y1; BWD: dkg) and o3 (BWD: dv).
template <int DT, int GE>
__device__ __forceinline__ float gated_output(float conv, bool has_s, float sv, float a, float b, float c, float d,
                                              float e, int act1, int act2, float& o2, float& o3) {
#pragma clang fp contract(off)
  o3 = 0.f;
  if constexpr (GE == GATED_FWD) {
    const float y1 = epilogue<DT>(conv, has_s, sv, gate1<DT>(act1, a, b));
    o2 = y1;
    return y1 * Elem<DT>::round(gate_act(act2, c));
  } else if constexpr (GE == GATED_BWD) {
    const float dy1 = Elem<DT>::round(a * Elem<DT>::round(gate_act(act2, b)));
    o3 = Elem<DT>::round(a * e) * gate_dact(act2, b);
    const float dz = epilogue<DT>(conv, has_s, sv, dy1);
    o2 = Elem<DT>::round(dz * c) * gate_dact(act1, d);
    return dz * Elem<DT>::round(gate_act(act1, d));
  } else {
    o2 = 0.f;
    return epilogue<DT>(conv, has_s, sv, a);
  }
}

// ---------------------------------------------------------------------------
// Elementwise gate kernels (flat over B*H*L; 8 elements per thread, one 16- or
// 32-byte vector access per operand when the run of 8 is whole, else scalar).
// ---------------------------------------------------------------------------
enum { GATE_OP_FWD1 = 0, GATE_OP_FWD2 = 1, GATE_OP_BWD2 = 2, GATE_OP_BWD1 = 3 };

struct GateEw {
  const void* a;  // FWD1: q    FWD2: y1   BWD2: dout   BWD1: dz
  const void* b;  // FWD1: k    FWD2: v    BWD2: v      BWD1: q
  const void* c;  //                       BWD2: y1     BWD1: k
  void* o0;       // FWD1: z    FWD2: out  BWD2: dy1    BWD1: dq
  void* o1;       //                       BWD2: dv     BWD1: dk
  int act;
};

template <int DT>
__device__ __forceinline__ void ew_load8(const void* p, int64_t i, bool whole, int64_t n, float (&v)[8]) {
  using T = typename Elem<DT>::T;
  const T* t = (const T*)p + i;
  if (whole) {
    if constexpr (DT == NSQ_DTYPE_F32) {
      const float4 a = ((const float4*)t)[0], b = ((const float4*)t)[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      const uint4 u = *(const uint4*)t;
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = RowBuf<DT, false>::bits_to_f32(w[j] & 0xffffu);
        v[2 * j + 1] = RowBuf<DT, false>::bits_to_f32(w[j] >> 16);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (i + j < n) ? Elem<DT>::load((const T*)p, i + j) : 0.f;
  }
}

template <int DT>
__device__ __forceinline__ void ew_store8(void* p, int64_t i, bool whole, int64_t n, const float (&v)[8]) {
  using T = typename Elem<DT>::T;
  T* t = (T*)p + i;
  if (whole) {
    if constexpr (DT == NSQ_DTYPE_F32) {
      ((float4*)t)[0] = make_float4(v[0], v[1], v[2], v[3]);
      ((float4*)t)[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (DT == NSQ_DTYPE_BF16)
          w[j] = f32x2_to_bf16x2_bits(v[2 * j], v[2 * j + 1]);
        else
          w[j] = __builtin_bit_cast(uint32_t, __floats2half2_rn(v[2 * j], v[2 * j + 1]));
      }
      *(uint4*)t = make_uint4(w[0], w[1], w[2], w[3]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (i + j < n) Elem<DT>::store((T*)p, i + j, v[j]);
  }
}

template <int DT, int OP>
__global__ __launch_bounds__(256) void gate_ew_kernel(GateEw g, int64_t n) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (i >= n) return;
  const bool whole = i + 8 <= n;  // base pointers are 16-byte aligned (checked by the host)
  float a[8], b[8], c[8], r0[8], r1[8];
  ew_load8<DT>(g.a, i, whole, n, a);
  ew_load8<DT>(g.b, i, whole, n, b);
  if constexpr (OP == GATE_OP_BWD2 || OP == GATE_OP_BWD1) ew_load8<DT>(g.c, i, whole, n, c);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (OP == GATE_OP_FWD1) {  // z = q act1(k)
      r0[j] = gate1<DT>(g.act, a[j], b[j]);
    } else if constexpr (OP == GATE_OP_FWD2) {  // out = y1 act2(v)
      r0[j] = a[j] * Elem<DT>::round(gate_act(g.act, b[j]));
    } else if constexpr (OP == GATE_OP_BWD2) {  // dy1 = dout act2(v), dv = (dout y1) act2'(v)
      r0[j] = a[j] * Elem<DT>::round(gate_act(g.act, b[j]));
      r1[j] = Elem<DT>::round(a[j] * c[j]) * gate_dact(g.act, b[j]);
    } else {  // dq = dz act1(k), dk = (dz q) act1'(k)
      r0[j] = a[j] * Elem<DT>::round(gate_act(g.act, c[j]));
      r1[j] = Elem<DT>::round(a[j] * b[j]) * gate_dact(g.act, c[j]);
    }
  }
  ew_store8<DT>(g.o0, i, whole, n, r0);
  if constexpr (OP == GATE_OP_BWD2 || OP == GATE_OP_BWD1) ew_store8<DT>(g.o1, i, whole, n, r1);
}

template <int DT, int OP>
static void launch_gate_ew(const GateEw& g, int64_t n, hipStream_t st) {
  if (n <= 0) return;
  const int64_t blocks = (n + 2047) / 2048;
  hipLaunchKernelGGL((gate_ew_kernel<DT, OP>), dim3(unsigned(blocks)), dim3(256), 0, st, g, n);
}

}  // namespace nsq
