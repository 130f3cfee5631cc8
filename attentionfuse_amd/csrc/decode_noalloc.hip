// af_decode_noalloc: flash decoding whose split partials live in a
// fixed-size device array of the library instead of a caller workspace, for
// callers that cannot allocate device memory (code under HIP graph capture,
// serving loops that forbid allocation).  The kernels are the ones af_decode
// launches; only the partial-sum storage differs.
//
// Each GPU holds its own copy of `scratch` (AF_DECODE_NOALLOC_SCRATCH_BYTES) from the
// library's first use on that device until the process ends.  Calls on one
// GPU share it, so two calls that overlap in time on one GPU (different
// streams, or different host threads) race on the partials; calls on one
// stream are ordered and safe.  Nothing in it has to start at zero: the split
// kernel writes every (m, l, acc) row the combine kernel reads.
#include <stdio.h>

#include <mutex>

#include "attnfuse_hip.h"
#include "launch_decode.hpp"
#include "validate.hpp"

// The split partials of every af_decode_noalloc call on a GPU.  In host
// code this name is only a stand-in: kernels and copies get the address
// hipGetSymbolAddress returns for the device (scratch_on below).
static __device__ __align__(256) unsigned char scratch[AF_DECODE_NOALLOC_SCRATCH_BYTES];

namespace af {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on device `dev`, looked up once per device
// with that device current.
int scratch_on(int dev, void** out) {
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("device %d: af_decode_noalloc supports device ordinals below %d", dev, kMaxDevices);
    return AF_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) {
      set_error("hipGetDevice failed: %s", hipGetErrorString(e));
      return AF_ERR_LAUNCH;
    }
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) {
      set_error("hipSetDevice(%d) failed: %s", dev, hipGetErrorString(e));
      return AF_ERR_LAUNCH;
    }
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    const hipError_t e2 = cur != dev ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess || ptr == nullptr) {
      set_error("hipGetSymbolAddress(scratch) on device %d failed: %s", dev, hipGetErrorString(e));
      return AF_ERR_LAUNCH;
    }
    if (e2 != hipSuccess) {
      set_error("hipSetDevice(%d) failed: %s", cur, hipGetErrorString(e2));
      return AF_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return AF_OK;
}

}  // namespace
}  // namespace af

using namespace af;

extern "C" int af_decode_noalloc(const af_decode_args* a, void* stream) {
  DecodeParams p;
  size_t need = 0;
  int rc = plan_decode(a, AF_DECODE_NOALLOC_SCRATCH_BYTES, &p, &need);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int dev = -1;
  hipError_t e = s != nullptr ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("cannot find the stream's device: %s", hipGetErrorString(e));
    return AF_ERR_BAD_ARG;
  }
  void* ws = nullptr;
  if ((rc = scratch_on(dev, &ws))) return rc;
  return enqueue_decode(p, a, ws, s);
}
