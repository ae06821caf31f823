// Shared device/host helpers for the gfx950 kernels of libmfx_kernels.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "mfx_kernels.h"

namespace mfx {

// ---- error reporting (host) -------------------------------------------------

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

#define MFX_HIP_CHECK(expr)                       \
  do {                                            \
    hipError_t _e = (expr);                       \
    if (_e != hipSuccess) return ::mfx::hip_fail(_e, #expr); \
  } while (0)

// Checks for a launch error after <<<>>>.
inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, what);
  return MFX_OK;
}

inline int dtype_size(int dt) {
  switch (dt) {
    case MFX_F32: return 4;
    case MFX_BF16: return 2;
    case MFX_F16: return 2;
    default: return 0;
  }
}

// Scratch buffer owned by the library for the current device and `stream`
// (so calls on different streams never share one): grown on demand by
// replacing it, the old buffer kept until the process ends, so work queued
// earlier stays valid and nothing waits.  Calls on one stream share it in
// stream order.  Growing allocates (hipMalloc): a caller that cannot, such as
// one capturing a graph, passes a workspace or uses mfx_sdpa_fwd_noalloc.
// Returns nullptr and sets the error on failure.
void* device_scratch(size_t bytes, hipStream_t stream);

// Compute units of the current device (cached per device; 256 if the query
// fails).
int device_cu_count();

// ---- device helpers ---------------------------------------------------------

typedef __bf16 bf16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f32(_Float16 v) { return static_cast<float>(v); }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float v) { return static_cast<bf16>(v); }
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float v) {
  return static_cast<_Float16>(v);
}

// Butterfly sum / max over groups of `width` consecutive lanes (width a power
// of two, at most 64); every lane of the group receives the result.
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int width>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int off = width / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace mfx
