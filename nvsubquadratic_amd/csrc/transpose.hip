// Batched transpose of the two inner axes: dst[b][c][r] = src[b][r][c], for
// the channels-last (BLH) wrappers of the FFT convs (nvsubquadratic/ops/
// fftconv.py:163-232 and fftconv_custom.py:338-359 rearrange "b l h -> b h l"
// and back; torch materialises that permute-copy at ~1 TB/s for 16-bit
// elements on MI355X, a fifth of a plain copy).
//
// A workgroup moves a 64 x 64 tile through LDS: the source rows are read as
// 16-byte vectors (8 bf16/fp16 or 4 fp32 elements per lane, whole 128- or
// 256-byte row segments per 8 or 16 lanes), the destination rows written the
// same way; the LDS tile has a 2-element row pad so the column reads of the
// write phase spread over the banks.  Tiles on the matrix edge, and matrices
// whose rows are not 16-byte multiples, move element by element (still one
// coalesced row segment per lane group).
#include "nsq_common.h"

namespace nsq {
namespace {

constexpr int kTile = 64;
constexpr int kPad = 2;

template <class T, bool VEC>
__global__ __launch_bounds__(256) void batched_transpose_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                                int64_t R, int64_t C) {
  constexpr int E = 16 / int(sizeof(T));  // elements per 16-byte vector
  __shared__ T tile[kTile][kTile + kPad];
  // row tiles on grid.x (up to 2^31 - 1 of them: R is the long axis, L or L times the spatial volume),
  // column (channel) tiles on grid.y, the batch on grid.z
  const int64_t r0 = int64_t(blockIdx.x) * kTile, c0 = int64_t(blockIdx.y) * kTile;
  const int64_t boff = int64_t(blockIdx.z) * R * C;
  const T* s = src + boff;
  T* d = dst + boff;
  const int t = threadIdx.x;
  const bool full = VEC && r0 + kTile <= R && c0 + kTile <= C;
  if (full) {
    constexpr int LPR = kTile / E;        // lanes per 64-element row segment
    constexpr int RPI = 256 / LPR;        // rows per iteration
    const int lr = t / LPR, lc = (t % LPR) * E;
#pragma unroll
    for (int it = 0; it < kTile / RPI; ++it) {
      const int r = it * RPI + lr;
      const uint4 v = *reinterpret_cast<const uint4*>(s + (r0 + r) * C + c0 + lc);
      const T* e = reinterpret_cast<const T*>(&v);
#pragma unroll
      for (int i = 0; i < E; ++i) tile[r][lc + i] = e[i];
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < kTile / RPI; ++it) {
      const int c = it * RPI + lr;  // destination row (source column)
      uint4 v;
      T* e = reinterpret_cast<T*>(&v);
#pragma unroll
      for (int i = 0; i < E; ++i) e[i] = tile[lc + i][c];
      *reinterpret_cast<uint4*>(d + (c0 + c) * R + r0 + lc) = v;
    }
  } else {
    // element path: lane (t % 64) walks one column of the tile per row read
    const int lc = t % kTile, lr = t / kTile;  // 4 rows per iteration
    for (int r = lr; r < kTile; r += 4) {
      const int64_t gr = r0 + r, gc = c0 + lc;
      if (gr < R && gc < C) tile[r][lc] = s[gr * C + gc];
    }
    __syncthreads();
    for (int c = lr; c < kTile; c += 4) {
      const int64_t gc = c0 + c, gr = r0 + lc;
      if (gr < R && gc < C) d[gc * R + gr] = tile[lc][c];
    }
  }
}

template <class T>
void launch_transpose(const void* src, void* dst, int64_t B, int64_t R, int64_t C, hipStream_t st) {
  constexpr int E = 16 / int(sizeof(T));
  const bool vec = R % E == 0 && C % E == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(dst) & 15) == 0;
  const dim3 grid(unsigned(ceil_div(R, int64_t(kTile))), unsigned(ceil_div(C, int64_t(kTile))), unsigned(B));
  if (vec)
    hipLaunchKernelGGL((batched_transpose_kernel<T, true>), grid, dim3(256), 0, st, (const T*)src, (T*)dst, R, C);
  else
    hipLaunchKernelGGL((batched_transpose_kernel<T, false>), grid, dim3(256), 0, st, (const T*)src, (T*)dst, R, C);
}

}  // namespace
}  // namespace nsq

extern "C" int nsq_batched_transpose(const void* src, void* dst, int elem_bytes, int64_t B, int64_t R, int64_t C,
                                     void* stream) {
  using namespace nsq;
  clear_error();
  NSQ_CHECK_ARG(src && dst, "batched_transpose: null pointer argument");
  NSQ_CHECK_ARG(src != dst, "batched_transpose: src and dst must not alias");
  NSQ_CHECK_ARG(elem_bytes == 2 || elem_bytes == 4, "batched_transpose: element size %d must be 2 or 4", elem_bytes);
  NSQ_CHECK_ARG(B >= 1 && R >= 1 && C >= 1, "batched_transpose: sizes must be positive");
  NSQ_CHECK_ARG(B <= 65535 && ceil_div(C, int64_t(kTile)) <= 65535 && ceil_div(R, int64_t(kTile)) <= 0x7fffffff,
                "batched_transpose: B=%lld R=%lld C=%lld exceed the launch grid", (long long)B, (long long)R,
                (long long)C);
  hipStream_t st = (hipStream_t)stream;
  if (elem_bytes == 2)
    launch_transpose<uint16_t>(src, dst, B, R, C, st);
  else
    launch_transpose<uint32_t>(src, dst, B, R, C, st);
  NSQ_CHECK_LAUNCH();
  return NSQ_OK;
}
