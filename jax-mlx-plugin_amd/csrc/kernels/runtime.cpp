// Host-side support of libmfx_kernels.so: error strings, device scratch and
// version queries.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"

namespace mfx {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  g_last_error = std::string(what) + ": " + hipGetErrorString(e);
  return MFX_E_HIP;
}

namespace {
// Scratch of one (device, stream).  A buffer that grows is replaced, never
// freed: work queued earlier may still read it, and freeing it would need a
// synchronisation.  The retired buffers add up to less than the current one
// (each replacement at least doubles) and live until the process ends.
struct Scratch {
  void* ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_scratch_mu;
std::map<std::pair<int, hipStream_t>, Scratch> g_scratch;
std::vector<void*> g_retired;
}  // namespace

void* device_scratch(size_t bytes, hipStream_t stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    hip_fail(e, "hipGetDevice");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  Scratch& s = g_scratch[{dev, stream}];
  if (s.bytes >= bytes && s.ptr) return s.ptr;
  size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
  if (want < 2 * s.bytes) want = 2 * s.bytes;
  void* p = nullptr;
  e = hipMalloc(&p, want);
  if (e != hipSuccess) {
    hip_fail(e, "hipMalloc(scratch)");
    return nullptr;
  }
  if (s.ptr) g_retired.push_back(s.ptr);
  s.ptr = p;
  s.bytes = want;
  return s.ptr;
}

int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> counts;  // indexed by device ordinal, 0 = not queried
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 256;
  }
  std::lock_guard<std::mutex> lock(mu);
  if ((size_t)dev >= counts.size()) counts.resize(dev + 1, 0);
  if (counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      n = 256;
    }
    counts[dev] = n;
  }
  return counts[dev];
}

}  // namespace mfx

extern "C" {

const char* mfx_last_error(void) { return mfx::g_last_error.c_str(); }

int mfx_version(void) { return 1; }

int mfx_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

}  // extern "C"
