// LDS tile staging shared by the MFMA attention kernels (flash prefill and
// split-KV decode): swizzled K/V tiles filled by asynchronous LDS-DMA loads.
#pragma once

#include <type_traits>

#include "sdpa_common.h"

namespace mfx {
namespace tiles {

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;

// Exponent slack of the lazy rescale: the running base of a row's exp2 is
// only raised when a new score exceeds it by more than this (log2 units), so
// un-normalised probabilities stay below 2^8 and the O / l rescale runs a
// handful of times per row instead of once per tile.  The result is exact:
// O and l always share the same base.
constexpr float kSlack = 8.0f;

// 16-byte chunk c of tile row r is stored at chunk slot c ^ tile_swz<D>(r).
// The K operand reads (lanes on consecutive rows, one chunk each) and the
// transposing V reads (4 rows x 2 chunks per 16 lanes) must spread over all
// banks whether the LDS serves 128 or 256 bytes per clock: for d = 128 the
// map is a bijection on each aligned run of 16 rows that is also one-to-one
// on bits 0-2 for 8 rows and on bits 1-2 and 2-3 for 4 rows; d = 64 rows
// have only 8 chunks and use a period-8 map.  d = 256 rows (512 bytes, two
// passes over the banks) take the d = 128 map: it stays within each
// 16-chunk half, so each half is spread as a d = 128 row is.
template <int D>
__host__ __device__ constexpr int tile_swz(int r) {
  if constexpr (D >= 128) return (r & 3) | (((r ^ (r >> 2)) & 3) << 2);
  return ((r & 3) << 1) | ((r >> 2) & 1);
}
template <int D>
constexpr int kSwzPeriod = D >= 128 ? 16 : 8;

// LDS operand reads as inline asm at an immediate byte offset from a
// per-lane LDS address, so the compiler neither batches them nor adds waits
// of its own; callers wait with lgkm_tie.
template <int IMM>
__device__ __forceinline__ void ds_b128(bf16x8& r, uint32_t a) {
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(IMM));
}
template <int IMM>
__device__ __forceinline__ void ds_tr(s16x4& r, uint32_t a) {
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(IMM));
}
// s_waitcnt lgkmcnt(N) that the named registers depend on, so their uses are
// not scheduled (or copied) before it.  LDS reads complete in order, so N is
// the number of reads issued after the one the registers came from.
template <int N>
__device__ __forceinline__ void lgkm_tie(bf16x8& r) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(r) : "i"(N));
}
template <int N>
__device__ __forceinline__ void lgkm_tie(s16x4& a, s16x4& b) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}
__device__ __forceinline__ void fence() { __builtin_amdgcn_sched_barrier(0); }

// f(integral_constant<int, J>) for J = B .. E-1, in order.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// s_waitcnt vmcnt(0), other counters left alone: this wave's LDS-DMA
// loads have landed.
__device__ __forceinline__ void wait_dma() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Copies rows [t*BN, t*BN + BN) x D (bf16) of one (batch, head) into a
// swizzled LDS tile with buffer loads to LDS, shared by the NW waves of a
// workgroup.  Instruction i of wave w fills tile chunks (NW*i + w)*64 .. +63,
// one 16-byte chunk per lane, i.e. rows (NW*i + w)*RPI .. +RPI-1 with
// RPI = 64 / (D/8).  Instructions NOFF apart start a swizzle period apart, so
// they share a per-lane source offset and differ by a scalar offset: NOFF
// VGPRs per operand, and the tile start and the step are scalar offsets.
// The resources span this (batch, head)'s elements, from its first row's
// first feature to its last row's `row_elems`-th (the head size, below D
// when rows load tile-wide): rows past Tk and the last row's features past
// the head are out of range and read as zeros (callers also mask their
// scores, so they contribute exactly 0), and no address leaves the tensor,
// also when heads are interleaved within a row.
template <int D, int BN, int NW>
struct TileLoader {
  static constexpr int DCH = D / 8;
  static constexpr int RPI = 64 / DCH;  // rows per load instruction
  static constexpr int LOADS = BN * DCH / (64 * NW);
  static constexpr int STEP = NW * RPI;  // rows between instructions of one wave
  static constexpr int NOFF = STEP >= kSwzPeriod<D> ? 1 : kSwzPeriod<D> / STEP;
  static_assert(LOADS >= 1 && LOADS % NOFF == 0, "tile must cover whole swizzle periods per wave");
  static constexpr bool swz_period_divides(int step) {
    for (int r = 0; r < BN; ++r)
      if (tile_swz<D>(r) != tile_swz<D>(r + step)) return false;
    return true;
  }
  bf16* base;
  int nbytes;             // extent of the resource: to the last row's last element
  uint32_t voff[NOFF];    // per-lane source offsets of instructions 0 .. NOFF-1
  uint32_t period_bytes;  // scalar offset step per NOFF instructions
  uint32_t tile_bytes;    // scalar offset step per tile

  __device__ __forceinline__ TileLoader(const bf16* b, int64_t row_stride, int Tk, int row_elems, int wave,
                                        int lane) {
    static_assert(swz_period_divides(NOFF * STEP), "the swizzle must repeat every NOFF instructions");
    base = const_cast<bf16*>(b);
    nbytes = Tk > 0 ? (int)(((int64_t)(Tk - 1) * row_stride + row_elems) * 2) : 0;
    tile_bytes = (uint32_t)(BN * row_stride * 2);
    period_bytes = (uint32_t)(NOFF * STEP * row_stride * 2);
#pragma unroll
    for (int j = 0; j < NOFF; ++j) {
      const int row = (NW * j + wave) * RPI + lane / DCH, slot = lane % DCH;
      voff[j] = (uint32_t)(((int64_t)row * row_stride + (slot ^ tile_swz<D>(row)) * 8) * 2);
    }
  }
  // The buffer-resource type exists only for the device target; the host
  // pass of a translation unit sees an empty body.
  //
  // The hardware range check covers the per-lane (VGPR) offset only, not the
  // scalar offset, so one resource spans the `nbytes` from `base` and every
  // offset -- the tile's `soff`, the instruction's row step and the lane's
  // row and chunk -- goes into the per-lane offset: rows past the end read
  // as zeros instead of touching memory beyond the span.  (soff + the lane
  // offsets stay below 2^32: soff is at most a tile past an extent below
  // 2^31.)  The resource is loop-invariant, so a caller's loop builds it
  // once; each instruction costs one vector add.
  __device__ __forceinline__ void load_at(uint32_t soff, bf16* lds, int wave) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(base, (short)0, nbytes > 0 ? nbytes : 0, 0x00020000);
#pragma unroll
    for (int i = 0; i < LOADS; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(lds + (NW * i + wave) * 64 * 8), 16,
                                               voff[i % NOFF] + soff + (uint32_t)(i / NOFF) * period_bytes, 0,
                                               0, 0);
#endif
  }
  __device__ __forceinline__ void load(int t, bf16* lds, int wave) const {
    load_at((uint32_t)t * tile_bytes, lds, wave);
  }
};

// 64 consecutive fp32 values (base + soff bytes onward) into LDS with one
// 4-byte LDS-DMA load per lane; values at or past `nbytes` read as zero.
__device__ __forceinline__ void load_row64_f32(const float* base, int nbytes, uint32_t soff, float* lds, int lane) {
#if defined(__HIP_DEVICE_COMPILE__)
  const int64_t rem = (int64_t)nbytes - (int64_t)soff;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<char*>(const_cast<float*>(base)) + soff, (short)0, rem > 0 ? (int)rem : 0, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)lds, 4, (uint32_t)lane * 4, 0, 0, 0);
#endif
}

}  // namespace tiles
}  // namespace mfx
