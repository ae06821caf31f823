// Row-vector helpers shared by the forward and backward row kernels: 16-byte
// vectors of f32 / bf16 / f16 unpacked to fp32, parameter loads of any of
// those storage types, and sums / maxima over the lanes that own a row.
#pragma once

#include <type_traits>

#include "common.h"

namespace mfx {
namespace rowvec {

constexpr int kBlock = 256;

template <typename T>
struct Vec16;
template <>
struct Vec16<float> {
  static constexpr int N = 4;
  typedef float4 type;
};
template <>
struct Vec16<bf16> {
  static constexpr int N = 8;
  typedef uint4 type;
};
template <>
struct Vec16<_Float16> {
  static constexpr int N = 8;
  typedef uint4 type;
};

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// f16 halves of a dword taken with integer shifts.  (A bit_cast of a vector
// element to 2 x f16 has compiled to code that reads the wrong dword once
// the conversions fold into v_fma_mix.)
__device__ __forceinline__ float f16_lo(uint32_t x) {
  return static_cast<float>(__builtin_bit_cast(_Float16, (uint16_t)(x & 0xffffu)));
}
__device__ __forceinline__ float f16_hi(uint32_t x) {
  return static_cast<float>(__builtin_bit_cast(_Float16, (uint16_t)(x >> 16)));
}

template <typename T>
__device__ __forceinline__ void unpack16(const typename Vec16<T>::type& v, float* out);
template <>
__device__ __forceinline__ void unpack16<float>(const float4& v, float* out) {
  out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
}
template <>
__device__ __forceinline__ void unpack16<bf16>(const uint4& v, float* out) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

template <>
__device__ __forceinline__ void unpack16<_Float16>(const uint4& v, float* out) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = f16_lo(w[i]);
    out[2 * i + 1] = f16_hi(w[i]);
  }
}

template <typename T>
__device__ __forceinline__ typename Vec16<T>::type pack16(const float* in);
template <>
__device__ __forceinline__ float4 pack16<float>(const float* in) {
  return make_float4(in[0], in[1], in[2], in[3]);
}
template <>
__device__ __forceinline__ uint4 pack16<bf16>(const float* in) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bf16 lo = static_cast<bf16>(in[2 * i]);
    bf16 hi = static_cast<bf16>(in[2 * i + 1]);
    w[i] = (uint32_t)__builtin_bit_cast(uint16_t, lo) |
           ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}
template <>
__device__ __forceinline__ uint4 pack16<_Float16>(const float* in) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const half2_t h = {static_cast<_Float16>(in[2 * i]), static_cast<_Float16>(in[2 * i + 1])};
    w[i] = __builtin_bit_cast(uint32_t, h);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ float load_param(const void* p, int dt, int i) {
  if (dt == MFX_F32) return static_cast<const float*>(p)[i];
  if (dt == MFX_F16) return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  return static_cast<float>(static_cast<const bf16*>(p)[i]);
}

// VEC consecutive parameters of storage type PT starting at element e, as
// fp32, in 16-byte (f32) or 8/16-byte (bf16, f16) vector loads.
template <typename PT, int VEC>
__device__ __forceinline__ void load_params(const void* p, int e, float* out) {
  if constexpr (std::is_same<PT, float>::value) {
    const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + e);
#pragma unroll
    for (int j = 0; j < VEC / 4; ++j) {
      const float4 v = q[j];
      out[4 * j] = v.x; out[4 * j + 1] = v.y; out[4 * j + 2] = v.z; out[4 * j + 3] = v.w;
    }
  } else if constexpr (std::is_same<PT, _Float16>::value) {
    const _Float16* h = static_cast<const _Float16*>(p) + e;
    if constexpr (VEC == 8) {
      unpack16<_Float16>(*reinterpret_cast<const uint4*>(h), out);
    } else {
      const uint2 v = *reinterpret_cast<const uint2*>(h);
      out[0] = f16_lo(v.x); out[1] = f16_hi(v.x);
      out[2] = f16_lo(v.y); out[3] = f16_hi(v.y);
    }
  } else if constexpr (VEC == 8) {
    unpack16<bf16>(*reinterpret_cast<const uint4*>(static_cast<const bf16*>(p) + e), out);
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const bf16*>(p) + e);
    out[0] = __uint_as_float(v.x << 16); out[1] = __uint_as_float(v.x & 0xffff0000u);
    out[2] = __uint_as_float(v.y << 16); out[3] = __uint_as_float(v.y & 0xffff0000u);
  }
}

// Sum / max over the LANES threads that own a row.  For LANES > 64 the
// partials of the wavefronts meet in LDS.
template <int LANES, bool kMax>
__device__ __forceinline__ float row_reduce(float v, float* lds) {
  if constexpr (LANES <= 64) {
    return kMax ? group_max<LANES>(v) : group_sum<LANES>(v);
  } else {
    v = kMax ? group_max<64>(v) : group_sum<64>(v);
    const int wid = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) lds[wid] = v;
    __syncthreads();
    float r = lds[0];
#pragma unroll
    for (int i = 1; i < LANES / 64; ++i) r = kMax ? fmaxf(r, lds[i]) : r + lds[i];
    __syncthreads();
    return r;
  }
}

// Two independent row sums in one pass: for 256-lane rows one LDS exchange
// (two barriers) instead of two.  Each value is summed in row_reduce's order,
// so the results are the same bits.  lds holds 2 * (LANES / 64) floats.
template <int LANES>
__device__ __forceinline__ void row_reduce_sum2(float& a, float& b, float* lds) {
  if constexpr (LANES <= 64) {
    a = group_sum<LANES>(a);
    b = group_sum<LANES>(b);
  } else {
    a = group_sum<64>(a);
    b = group_sum<64>(b);
    const int wid = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
      lds[2 * wid] = a;
      lds[2 * wid + 1] = b;
    }
    __syncthreads();
    float ra = lds[0], rb = lds[1];
#pragma unroll
    for (int i = 1; i < LANES / 64; ++i) {
      ra += lds[2 * i];
      rb += lds[2 * i + 1];
    }
    __syncthreads();
    a = ra;
    b = rb;
  }
}

}  // namespace rowvec
}  // namespace mfx
