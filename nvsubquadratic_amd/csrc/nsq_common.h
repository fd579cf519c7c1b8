// Shared host/device helpers for the nvsubquadratic_amd HIP library (gfx950).
//
// Error convention of the C ABI: every entry point returns an int status
// (NSQ_OK == 0) and records a human-readable message in a thread-local buffer
// readable through nsq_last_error().  Nothing here allocates device memory on
// the hot path; the only library-owned device memory is the immutable twiddle
// table built once per device (see twiddle.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/nsq_hip.h"

namespace nsq {

// ---------------------------------------------------------------------------
// Host-side error helpers
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
void clear_error();

#define NSQ_CHECK_ARG(cond, ...)                 \
  do {                                           \
    if (!(cond)) {                               \
      ::nsq::set_error(__VA_ARGS__);             \
      return NSQ_ERR_INVALID_ARGUMENT;           \
    }                                            \
  } while (0)

#define NSQ_CHECK_HIP(expr)                                                   \
  do {                                                                        \
    hipError_t _e = (expr);                                                   \
    if (_e != hipSuccess) {                                                   \
      ::nsq::set_error("HIP error '%s' at %s:%d (%s)", hipGetErrorString(_e), \
                       __FILE__, __LINE__, #expr);                            \
      return NSQ_ERR_HIP;                                                     \
    }                                                                         \
  } while (0)

#define NSQ_CHECK_LAUNCH()                                                    \
  do {                                                                        \
    hipError_t _e = hipGetLastError();                                        \
    if (_e != hipSuccess) {                                                   \
      ::nsq::set_error("kernel launch failed: '%s' at %s:%d",                 \
                       hipGetErrorString(_e), __FILE__, __LINE__);            \
      return NSQ_ERR_HIP;                                                     \
    }                                                                         \
  } while (0)

// Returns the per-device twiddle table (see twiddle.hip), building it on the
// first call for the current device.  nullptr on failure (error recorded).
const float2* twiddle_table();

// Twiddle table layout (float2 entries, forward roots W_L^j = e^{-2 pi i j / L}):
//   W_{2^b},   b <= 14:          entries 2^b + j;
//   W_{3*2^b}, b <= kTw3MaxLog:  entries kTwPow2Entries + 3*2^b + j.
constexpr int kTwPow2Entries = 2 << 14;
constexpr int kTw3MaxLog = 10;
constexpr int kTwEntries = kTwPow2Entries + (6 << kTw3MaxLog);

inline bool valid_dtype(int dt) {
  return dt == NSQ_DTYPE_F32 || dt == NSQ_DTYPE_BF16 || dt == NSQ_DTYPE_F16;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Sub-buffers carved out of one workspace start on 256-byte boundaries, so
// every kernel that takes one may use 16-byte vector accesses whatever the
// element counts before it.
inline size_t round256(size_t bytes) { return (bytes + 255) / 256 * 256; }

inline int ilog2_ceil(int64_t v) {
  int l = 0;
  while ((int64_t(1) << l) < v) ++l;
  return l;
}

// ---------------------------------------------------------------------------
// Device-side element conversion.  Rounding is round-to-nearest-even, the
// rounding torch applies in Tensor.to(bfloat16 / float16).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(uint32_t(b) << 16);
}

// gfx950 converts in hardware (v_cvt_pk_bf16_f32): round to nearest even,
// NaN stays NaN.  Branch-free, and a pair packs in one instruction.
typedef __bf16 nsq_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float nsq_f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// (bf16(a) | bf16(b) << 16)
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float a, float b) {
  const nsq_f32x2_t f = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, nsq_bf16x2_t));
}

template <int DT>
struct Elem;

template <>
struct Elem<NSQ_DTYPE_F32> {
  using T = float;
  __device__ __forceinline__ static float load(const T* p, int64_t i) { return p[i]; }
  __device__ __forceinline__ static void store(T* p, int64_t i, float v) { p[i] = v; }
  __device__ __forceinline__ static float round(float v) { return v; }
};

template <>
struct Elem<NSQ_DTYPE_BF16> {
  using T = uint16_t;
  __device__ __forceinline__ static float load(const T* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
  __device__ __forceinline__ static void store(T* p, int64_t i, float v) { p[i] = f32_to_bf16_bits(v); }
  __device__ __forceinline__ static float round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }
};

template <>
struct Elem<NSQ_DTYPE_F16> {
  using T = __half;
  __device__ __forceinline__ static float load(const T* p, int64_t i) { return __half2float(p[i]); }
  __device__ __forceinline__ static void store(T* p, int64_t i, float v) { p[i] = __float2half_rn(v); }
  __device__ __forceinline__ static float round(float v) { return __half2float(__float2half_rn(v)); }
};

// Output epilogue shared by every FFT-conv kernel, mirroring the wrapper
// semantics of the reference (nvsubquadratic/ops/fftconv_custom.py:327-335):
//   y = conv.to(x.dtype);  y = y + shortcut.to(x.dtype) * x
// Each torch op on a low-precision tensor rounds its result to that dtype, so
// the product s*x and the sum are rounded separately here as well.
template <int DT>
__device__ __forceinline__ float epilogue(float conv, bool has_s, float s_rounded, float xv) {
#pragma clang fp contract(off)  // s*x and the sum rounded apart in every kernel (fp32 rounding is the identity)
  const float y = Elem<DT>::round(conv);
  const float sx = Elem<DT>::round(s_rounded * xv);
  const float ys = Elem<DT>::round(y + sx);
  return has_s ? ys : y;  // select, not a branch: keeps streaming epilogues branch-free
}

}  // namespace nsq
