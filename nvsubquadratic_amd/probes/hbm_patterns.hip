// HBM access-pattern probes for the config-3 multi-kernel plan (B=1, D=4096,
// packed FFT length N = 2^18 = 256 x 1024).  Each probe kernel issues the
// global loads and stores of one pass of the plan with no FFT arithmetic, so
// its rate is the ceiling that pass's memory traffic can reach on this GPU:
//   col    : col_fwd's pattern -- a workgroup of 512 threads per tile of 32
//            columns, bf16 pairs of the 128 nonzero rows in (4-byte lanes,
//            128-byte row segments), 256 x 32 complex values out (8-byte
//            lanes, 256-byte row segments); one tile per workgroup;
//   row    : the row kernels' pattern -- 128 threads per row pair {q, N1-q},
//            2 x 1024 complex values in and out;
//   copy16 : a plain 16-byte-lane copy of 8 GiB (grid-stride).
// Not part of the product library: built into libnsq_probes.so and run by
// bench.py --workload hbm-patterns.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int N1 = 256, N2 = 1024, M = 32, NCB = N2 / M, TC = 512;
constexpr int64_t N = int64_t(N1) * N2;

__global__ __launch_bounds__(TC) void col_pattern(const uint32_t* __restrict__ x, float2* __restrict__ ws) {
  const int tid = threadIdx.x, m = tid % M, j = tid / M;
  const int64_t t = blockIdx.x;
  const int64_t h = t / NCB;
  const int c0 = int(t % NCB) * M;
  const uint32_t* xr = x + h * (N / 2);  // one channel: N/2 bf16 pairs (the nonzero half of the packed row)
  uint32_t v[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) v[r] = xr[int64_t(j + r * 16) * N2 + c0 + m];
  float a = 0.f, b = 0.f;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    a += __uint_as_float(v[r] << 16);
    b += __uint_as_float(v[r] & 0xffff0000u);
  }
  float2* o = ws + h * N;
#pragma unroll
  for (int r = 0; r < 16; ++r) o[int64_t(j + r * 16) * N2 + c0 + m] = make_float2(a + float(r), b);
}

__global__ __launch_bounds__(128) void row_pattern(const float2* __restrict__ ws, float2* __restrict__ out) {
  const int q = blockIdx.x % (N1 / 2);
  const int64_t h = blockIdx.x / (N1 / 2);
  const int ra = q, rb = q == 0 ? N1 / 2 : N1 - q;
  float2 v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int e = threadIdx.x + 128 * i;
    v[i] = ws[h * N + int64_t(e < N2 ? ra : rb) * N2 + (e & (N2 - 1))];
  }
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) a += v[i].x + v[i].y;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int e = threadIdx.x + 128 * i;
    out[h * N + int64_t(e < N2 ? ra : rb) * N2 + (e & (N2 - 1))] = make_float2(a, float(i));
  }
}

__global__ void copy16(const uint4* __restrict__ a, uint4* __restrict__ b, int64_t n) {
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    b[i] = a[i];
}

}  // namespace

// Runs each probe over `channels` channels (best of 5 after one warm-up) and
// writes {col_ms, col_bytes, row_ms, row_bytes, copy_ms, copy_bytes} to out.
// Allocates its own buffers (3 x channels x 2 MB); returns 0 or a HIP error code.
extern "C" int nsq_probe_hbm_patterns(int channels, double* out) {
  const int64_t H = channels;
  uint32_t* x = nullptr;
  float2 *ws = nullptr, *ws2 = nullptr;
  hipError_t e = hipSuccess;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  auto timed = [&](auto launch, double* ms) {
    launch();
    if ((e = hipDeviceSynchronize()) != hipSuccess) return;
    float best = 1e30f;
    for (int rep = 0; rep < 5; ++rep) {
      (void)hipEventRecord(e0);
      launch();
      (void)hipEventRecord(e1);
      if ((e = hipEventSynchronize(e1)) != hipSuccess) return;
      float t = 0.f;
      (void)hipEventElapsedTime(&t, e0, e1);
      best = t < best ? t : best;
    }
    *ms = best;
  };
  if ((e = hipMalloc(&x, size_t(H) * (N / 2) * 4)) != hipSuccess) goto done;
  if ((e = hipMalloc(&ws, size_t(H) * N * 8)) != hipSuccess) goto done;
  if ((e = hipMalloc(&ws2, size_t(H) * N * 8)) != hipSuccess) goto done;
  if ((e = hipMemset(x, 0, size_t(H) * (N / 2) * 4)) != hipSuccess) goto done;
  if ((e = hipMemset(ws, 0, size_t(H) * N * 8)) != hipSuccess) goto done;
  if ((e = hipEventCreate(&e0)) != hipSuccess) goto done;
  if ((e = hipEventCreate(&e1)) != hipSuccess) goto done;
  timed([&] { hipLaunchKernelGGL(col_pattern, dim3(unsigned(H * NCB)), dim3(TC), 0, 0, x, ws); }, &out[0]);
  if (e != hipSuccess) goto done;
  out[1] = double(H) * (N / 2) * 4 + double(H) * N * 8;
  timed([&] { hipLaunchKernelGGL(row_pattern, dim3(unsigned(H * (N1 / 2))), dim3(128), 0, 0, ws, ws2); }, &out[2]);
  if (e != hipSuccess) goto done;
  out[3] = double(H) * N * 16;
  {
    const int64_t n16 = int64_t(H) * N * 8 / 16;
    timed([&] { hipLaunchKernelGGL(copy16, dim3(65536), dim3(256), 0, 0, (const uint4*)ws, (uint4*)ws2, n16); },
          &out[4]);
    out[5] = double(n16) * 32;
  }
done:
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipFree(x);
  (void)hipFree(ws);
  (void)hipFree(ws2);
  return int(e);
}
