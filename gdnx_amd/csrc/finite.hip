// Non-finite detection for the C ABI (gfx950).
//
// The reference trainer drops a step whose loss or gradient norm is not
// finite rather than let it reach the optimizer (its NaN/inf guard,
// train/train_gdn3_distill.py:329-354).  The ABI's entry points are
// asynchronous, so detecting a NaN or an infinity in their outputs needs a
// device-side scan and a host read.  That is opt-in: with
// gdnx_set_check_finite(1) the recurrence entry points scan what they wrote,
// synchronise their stream and return GDNX_ERR_NONFINITE when any value is
// NaN or infinite; gdnx_check_finite scans one buffer on demand.  Off (the
// default), nothing is added to the launch sequence.
//
// The flags the scans set are words of a per-device array in static device
// memory, reached through the address hipGetSymbolAddress returns for the
// current device.  Each checked call holds a word of its own from clear to
// read-back (taken from a free list, returned after its stream has
// synchronised), so calls on different streams or threads do not share one;
// at most kFlagWords checked calls may be in flight per device.  A lane that
// finds a non-finite value stores 1 in the call's word (a vector store from a
// divergent branch: concurrent writers all store the same value).  The check
// reads the flag back and synchronises the stream, which a stream under HIP
// graph capture cannot do: a checked call on a capturing stream is refused.
#include <atomic>
#include <mutex>

#include "gdnx_common.hpp"
#include "gdnx_internal.hpp"

namespace gdnx {

constexpr int kFlagWords = 64;
static __device__ __align__(256) unsigned nonfinite_flag[kFlagWords];

namespace {
std::atomic<int> g_check_on{0};
std::mutex g_flag_mu;
constexpr int kMaxDevices = 64;
unsigned* g_flag_ptr[kMaxDevices] = {};
unsigned long long g_flag_busy[kMaxDevices] = {};   // bit w: word w held by a call in flight

__global__ void flag_clear_kernel(unsigned* flag) {
  if (threadIdx.x == 0) flag[0] = 0u;   // lane 0 only: a vector store
}

template <typename T>
__device__ __forceinline__ bool finite_of(T x) {
  return isfinite((float)x);
}
template <>
__device__ __forceinline__ bool finite_of<double>(double x) {
  return isfinite(x);
}

// any non-finite element of x[0, n) sets *flag
template <typename T>
__global__ void __launch_bounds__(256) finite_scan_kernel(const T* __restrict__ x, long long n, unsigned* flag) {
  bool bad = false;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    bad |= !finite_of(x[i]);
  if (bad) flag[0] = 1u;
}

// a free flag word of the current device for one call: *out its address,
// *dev_out / *word_out to hand back with flag_release
int flag_acquire(unsigned** out, int* dev_out, int* word_out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(GDNX_ERR_HIP, "no current HIP device (or device index >= %d)", kMaxDevices);
  std::lock_guard<std::mutex> lock(g_flag_mu);
  if (!g_flag_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(nonfinite_flag));
    if (e != hipSuccess || !p) return set_error(GDNX_ERR_HIP, "non-finite flag address: %s", hipGetErrorString(e));
    g_flag_ptr[dev] = (unsigned*)p;
  }
  for (int w = 0; w < kFlagWords; ++w) {
    if (!(g_flag_busy[dev] >> w & 1ull)) {
      g_flag_busy[dev] |= 1ull << w;
      *out = g_flag_ptr[dev] + w;
      *dev_out = dev;
      *word_out = w;
      return GDNX_OK;
    }
  }
  return set_error(GDNX_ERR_HIP, "non-finite check: more than %d checked calls in flight on device %d",
                   kFlagWords, dev);
}

void flag_release(int dev, int word) {
  std::lock_guard<std::mutex> lock(g_flag_mu);
  g_flag_busy[dev] &= ~(1ull << word);
}
}  // namespace

bool check_finite_on() { return g_check_on.load(std::memory_order_relaxed) != 0; }

static int finite_check_word(const FiniteBuf* bufs, int nbuf, hipStream_t stream, unsigned* flag);

int finite_check(const FiniteBuf* bufs, int nbuf, hipStream_t stream) {
  unsigned* flag = nullptr;
  int dev = 0, word = 0;
  int rc = flag_acquire(&flag, &dev, &word);
  if (rc) return rc;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess)
    rc = set_error(GDNX_ERR_HIP, "non-finite check: cannot query the stream's capture status on device %d", dev);
  else if (cap != hipStreamCaptureStatusNone)
    rc = set_error(GDNX_ERR_ARG, "non-finite checking synchronises the stream and cannot run under graph "
                   "capture: turn it off (gdnx_set_check_finite(0)) while capturing");
  else
    rc = finite_check_word(bufs, nbuf, stream, flag);
  flag_release(dev, word);
  return rc;
}

static int finite_check_word(const FiniteBuf* bufs, int nbuf, hipStream_t stream, unsigned* flag) {
  int rc;
  hipLaunchKernelGGL(flag_clear_kernel, dim3(1), dim3(64), 0, stream, flag);
  if ((rc = check_launch("flag_clear_kernel"))) return rc;
  for (int i = 0; i < nbuf; ++i) {
    const FiniteBuf& b = bufs[i];
    if (!b.p || b.n == 0) continue;
    const long long nb = ((long long)b.n + 255) / 256;
    const dim3 grid((unsigned)(nb < 4096 ? nb : 4096));
    if (b.dtype == GDNX_DTYPE_BF16)
      hipLaunchKernelGGL(finite_scan_kernel<bf16>, grid, dim3(256), 0, stream, (const bf16*)b.p, (long long)b.n, flag);
    else if (b.dtype == GDNX_DTYPE_F64)
      hipLaunchKernelGGL(finite_scan_kernel<double>, grid, dim3(256), 0, stream, (const double*)b.p, (long long)b.n,
                         flag);
    else
      hipLaunchKernelGGL(finite_scan_kernel<float>, grid, dim3(256), 0, stream, (const float*)b.p, (long long)b.n, flag);
    if ((rc = check_launch("finite_scan_kernel"))) return rc;
  }
  unsigned host = 0;
  if (hipMemcpyAsync(&host, flag, sizeof(unsigned), hipMemcpyDeviceToHost, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return set_error(GDNX_ERR_HIP, "non-finite check: reading the flag failed");
  if (host) return set_error(GDNX_ERR_NONFINITE, "non-finite values (NaN or infinity) in the outputs");
  return GDNX_OK;
}

int finite_outputs(const FiniteBuf* bufs, int nbuf, hipStream_t stream) {
  return check_finite_on() ? finite_check(bufs, nbuf, stream) : GDNX_OK;
}

}  // namespace gdnx

using namespace gdnx;

extern "C" int gdnx_set_check_finite(int on) { return g_check_on.exchange(on ? 1 : 0); }

extern "C" int gdnx_check_finite(const void* x, long long n, int dtype, void* stream) {
  if (dtype != GDNX_DTYPE_F32 && dtype != GDNX_DTYPE_BF16 && dtype != GDNX_DTYPE_F64)
    return set_error(GDNX_ERR_ARG, "dtype %d is not GDNX_DTYPE_F32/BF16/F64", dtype);
  if (n < 0 || (n > 0 && !x)) return set_error(GDNX_ERR_ARG, "x must be non-null for n > 0");
  const FiniteBuf b{x, (size_t)n, dtype};
  return finite_check(&b, 1, (hipStream_t)stream);
}
