// Twiddle table and error plumbing for the nvsubquadratic_amd C ABI.
//
// One immutable table per device, built on first use and kept for the life of
// the process: the library's only device allocation outside caller-provided
// buffers.  Layout (float2 = (cos, -sin), i.e. forward-transform roots):
//   segment b (b = 0..14) at entries [2^b, 2^(b+1)): W_{2^b}^j = exp(-2*pi*i*j/2^b)
// so a root of unity W_{2^b}^m with b <= 14 is one load, table[2^b + m], and a
// pass of a length-2^b transform reads one contiguous 2^b-entry segment;
//   then the roots of the mixed-radix lengths 3*2^b (b = 0..kTw3MaxLog) at
//   entries kTwPow2Entries + [3*2^b, 3*2^(b+1)).
// Values are computed on the host in double precision and rounded once to
// float (within 0.5 ulp of the exact root).
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <vector>

#include "nsq_common.h"

namespace nsq {

namespace {
thread_local char g_err[1024] = {0};
std::mutex g_tw_mutex;
constexpr int kMaxDevices = 64;
float2* g_tw[kMaxDevices] = {nullptr};
}  // namespace

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = 0; }

const float2* twiddle_table() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("twiddle_table: no current HIP device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_tw_mutex);
  if (g_tw[dev]) return g_tw[dev];
  constexpr int kLogMax = 14;
  static_assert(kTwPow2Entries == (2 << kLogMax), "twiddle table: power-of-two region size");
  std::vector<float2> host(size_t(kTwEntries), make_float2(1.f, 0.f));
  const double two_pi = 6.283185307179586476925286766559;
  auto segment = [&](size_t start, int n) {
    for (int j = 0; j < n; ++j) {
      const double a = two_pi * double(j) / double(n);
      host[start + j] = make_float2(float(std::cos(a)), float(-std::sin(a)));
    }
  };
  for (int b = 0; b <= kLogMax; ++b) segment(size_t(1) << b, 1 << b);
  for (int b = 0; b <= kTw3MaxLog; ++b) segment(size_t(kTwPow2Entries) + (size_t(3) << b), 3 << b);
  float2* d = nullptr;
  hipError_t e = hipMalloc(&d, host.size() * sizeof(float2));
  if (e != hipSuccess) {
    set_error("twiddle_table: hipMalloc failed: %s", hipGetErrorString(e));
    return nullptr;
  }
  e = hipMemcpy(d, host.data(), host.size() * sizeof(float2), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(d);
    set_error("twiddle_table: hipMemcpy failed: %s", hipGetErrorString(e));
    return nullptr;
  }
  g_tw[dev] = d;
  return d;
}

}  // namespace nsq

extern "C" {

const char* nsq_last_error(void) { return nsq::g_err; }

int nsq_abi_version(void) { return NSQ_ABI_VERSION; }

int nsq_init(void) {
  nsq::clear_error();
  return nsq::twiddle_table() ? NSQ_OK : NSQ_ERR_HIP;
}

}  // extern "C"
