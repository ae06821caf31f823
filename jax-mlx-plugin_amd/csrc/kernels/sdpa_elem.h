// 16-bit element types of the MFMA attention kernels.
//
// The kernels move bf16 and f16 data through the same registers and LDS
// tiles as raw 16-bit patterns (operand reads, transposing V reads, Q rows
// are typed bf16x8 / s16x4 as bit containers).  Only four operations depend
// on the type, and E selects them: E = 0 bf16, E = 1 f16.
//   mfma16   32x32x16 product with fp32 accumulation
//   pack2    two fp32 probabilities rounded to the element type, one dword
//   dot2     fp32 sum of the two packed values (the row sums P was formed of)
//   store_e  an output value rounded to the element type, as 16 bits
// and one limit: kMaxP, the largest probability a tile may hold before the
// row's exp2 base is raised (f16 overflows past 65504).
#pragma once

#include "sdpa_common.h"

namespace mfx {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

template <int E>
__device__ __forceinline__ f32x16 mfma16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  if constexpr (E == 0) return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                   0, 0, 0);
}

template <int E>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (E == 0) {
    const bf16x2 w = {static_cast<bf16>(a), static_cast<bf16>(b)};
    return __builtin_bit_cast(uint32_t, w);
  } else {
    const f16x2 w = {static_cast<f16>(a), static_cast<f16>(b)};
    return __builtin_bit_cast(uint32_t, w);
  }
}

template <int E>
__device__ __forceinline__ float dot2(uint32_t w, float acc) {
  if constexpr (E == 0) {
    const bf16x2 one2 = {static_cast<bf16>(1.f), static_cast<bf16>(1.f)};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one2, acc, false);
  } else {
    const f16x2 one2 = {static_cast<f16>(1.f), static_cast<f16>(1.f)};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), one2, acc, false);
  }
}

// dot2 of elements i, i+1 of an eight-element bf16 fragment.  bf16 only:
// for f16 the same shape (pairs taken from elements of a 16-bit vector whose
// elements were inserted one at a time) compiles to wrong sums (operand
// pairs built from one value twice), so f16 code packs pairs with pack2 and
// sums the dwords with dot2.
template <int E>
__device__ __forceinline__ float dot2_at(const bf16x8& w, int i, float acc) {
  static_assert(E == 0, "f16: use pack2 + dot2");
  const bf16x2 one2 = {static_cast<bf16>(1.f), static_cast<bf16>(1.f)};
  return __builtin_amdgcn_fdot2_f32_bf16(bf16x2{w[i], w[i + 1]}, one2, acc, false);
}

template <int E>
__device__ __forceinline__ uint16_t store_e(float x) {
  if constexpr (E == 0) return __builtin_bit_cast(uint16_t, static_cast<bf16>(x));
  else return __builtin_bit_cast(uint16_t, static_cast<f16>(x));
}

// One element of a bf16 fragment to fp32 and back.  bf16 only: f16 code
// converts whole fragments (frag_f32 / f32_frag below), since per-element
// bit casts between 16-bit vector elements and f16 have compiled to wrong
// element selections once the conversions fold into other instructions.
template <int E>
__device__ __forceinline__ float elem_f32(bf16 x) {
  static_assert(E == 0, "f16: use frag_f32");
  return static_cast<float>(x);
}
template <int E>
__device__ __forceinline__ bf16 f32_elem(float x) {
  static_assert(E == 0, "f16: use f32_frag");
  return static_cast<bf16>(x);
}

// f16 halves of a dword, taken with integer shifts.
__device__ __forceinline__ float f16_lo(uint32_t x) {
  return static_cast<float>(__builtin_bit_cast(f16, (uint16_t)(x & 0xffffu)));
}
__device__ __forceinline__ float f16_hi(uint32_t x) {
  return static_cast<float>(__builtin_bit_cast(f16, (uint16_t)(x >> 16)));
}

// The eight f16 values of a fragment (held as bf16x8 bits) to fp32.
__device__ __forceinline__ void frag_f32_f16(const bf16x8& w, float (&out)[8]) {
  const u32x4 u = __builtin_bit_cast(u32x4, w);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = f16_lo(u[i]);
    out[2 * i + 1] = f16_hi(u[i]);
  }
}

// Eight fp32 values rounded to f16, as a fragment (bf16x8 bits).
__device__ __forceinline__ bf16x8 f32_frag_f16(const float (&in)[8]) {
  u32x4 u;
#pragma unroll
  for (int i = 0; i < 4; ++i) u[i] = pack2<1>(in[2 * i], in[2 * i + 1]);
  return __builtin_bit_cast(bf16x8, u);
}

// A tile's lane row sum (32 probabilities) above kMaxP sends the row to the
// rebase path, so no probability reaches it: 2^16 for bf16 (its range is
// fp32's), 2^15 for f16 (largest finite 65504).
template <int E>
constexpr float kMaxP = E == 0 ? 65536.f : 32768.f;

// Stores a wavefront's 32 output rows (lane column l32 = row, features
// dt*32 + g*8 + half*4 + e of a transposed 32x32 MFMA accumulator set,
// times `mul`; D = 64, 128 or 256) as whole rows: written into the wavefront's 32 x D region of free LDS
// (16-byte chunk c of row r at slot c ^ (r % (D/8)), so neither the 8-byte
// writes nor the 16-byte reads meet more than two lanes on a bank), read
// back row-contiguous, 16 bytes per lane, so each store instruction writes
// 64 / (D/8) whole rows, streamed past the L2 (whole lines, written once).
// Row r goes to dst + r * stride when r < nvalid (rows 16-byte aligned,
// checked on the host).
template <int D, int E>
__device__ __forceinline__ void store_rows_lds(bf16* lds, bf16* dst, int64_t stride, int nvalid, const f32x16* acc,
                                               int l32, int half, int lane, float mul) {
  constexpr int CPR = D / 8;    // 16-byte chunks per row
  constexpr int RPS = 64 / CPR;  // rows per store instruction
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u16x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = store_e<E>(acc[dt][g * 4 + e] * mul);
      const int c = dt * 4 + g;
      *reinterpret_cast<u16x4*>(lds + l32 * D + (c ^ (l32 & (CPR - 1))) * 8 + half * 4) = w;
    }
#pragma unroll
  for (int k = 0; k < 32 / RPS; ++k) {
    const int r = k * RPS + lane / CPR, c = lane % CPR;
    const u32x4 v = *reinterpret_cast<const u32x4*>(lds + r * D + (c ^ (r & (CPR - 1))) * 8);
    if (r < nvalid) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst + r * stride + c * 8));
  }
}

// Element code of an MFX dtype (MFX_BF16 -> 0, MFX_F16 -> 1).
inline int elem_code(int dt) { return dt == MFX_F16 ? 1 : 0; }

}  // namespace mfx
