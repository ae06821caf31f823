// bf16 / f16 GEMM tile kernel on v_mfma_f32_32x32x16_{bf16,f16}:
//
//   C[b][m][n] = sum_k op(A)[b][m][k] * op(B)[b][k][n]   (fp32 accumulation)
//
// with A stored [m][k] or, transposed, [k][m], and B stored [k][n] or, transposed,
// [n][k]: the dense forward x W, and the backward products x^T dy (A
// transposed) and dy W^T (B transposed) of a training step.
//
// The kernel computes C^T = B^T A^T: the MFMA's A operand is indexed by n
// (taken from B), its B operand by m (taken from A), so an accumulator lane
// holds one row m of C and 16 columns n in runs of 4 -- 8- or 16-byte stores
// along the row.  Both operands have the same fragment shape (32 indices x
// 16 k, a lane holding 8 k values of one index), and each comes from one of
// two LDS tile forms:
//   k-contiguous operand (A not transposed, B transposed): [128 rows][64 k]
//     tiles, 128 bytes a row, 16-byte chunk c of row r at slot
//     c ^ tile_swz<64>(r); read directly as two ds_read_b64 (k slots = 8
//     consecutive k);
//   index-contiguous operand (B not transposed, A transposed): [64 k][128
//     indices] tiles, 256 bytes a row, swizzled by tile_swz<128>; read with
//     the transposing ds_read_b64_tr_b16, whose k slots are k 4h .. 4h+3 and
//     8+4h .. 8+4h+3 of the 16-k step (h = lane / 32), as the flash kernels
//     read V.
// The two operands of an MFMA must hold the same k in the same slot: when
// one side is read transposed and the other directly, the direct side reads
// its fragment as two 8-byte halves in the transposed order.
//
// Workgroup: 4 wavefronts, a 128 (m) x 128 (n) tile, each wavefront a 64 x
// 64 block as 2 x 2 MFMA accumulators (64 registers).  K advances in 64-wide
// k-tiles through two LDS stages (32 KB each, two workgroups per CU), loaded
// by LDS-DMA (buffer_load ... lds, 16 bytes a lane): one vmcnt wait and one
// barrier per k-tile; the next k-tile's loads are issued right after the
// barrier and land while this one is computed.  Within a k-tile the
// fragments of step s+1 are read (inline asm, one tied lgkmcnt wait) while
// the MFMAs of step s run.
//
// Range checks: the hardware checks only a raw buffer load's per-lane
// (VGPR) offset against the resource's extent, so every row and k offset is
// per-lane, the resource base is the operand's first element of this batch
// and row / column block, and the extent ends at the operand's last element.
// k-contiguous tiles point chunks at or past K (and rows past the operand's
// row count) out of range explicitly: they read as zeros, since a k column
// feeds every output of the tile.  Index-contiguous tiles read rows (k) at
// or past K as zeros the same way; their columns past the last index read
// the next row's elements (or zeros past the end) and only reach outputs
// that are never stored.
#include "gemm16.h"

#include "sdpa_elem.h"
#include "sdpa_tiles.h"

namespace mfx {
namespace {

constexpr int kBM = 128;  // tile rows (m)
constexpr int kBN = 128;  // tile columns (n)
constexpr int kBK = 64;   // k-tile
constexpr int kNT = 256;  // 4 wavefronts
constexpr int kTileElems = 128 * 64;              // elements of one operand tile (either form)
constexpr int kStageElems = 2 * kTileElems;       // A tile + B tile
constexpr uint32_t kOOR = 0x80000000u;            // an offset past every extent

using tiles::s16x4;
using tiles::tile_swz;
using tiles::lds_void_t;
using tiles::fence;

struct Params {
  const bf16* a;
  const bf16* b;
  void* c;
  float* part;         // split-K: fp32 partials [batch][splits][M][N] (null: no split)
  int64_t sa, sb, sc;  // batch strides (elements)
  int M, N, K;
  int lda, ldb, ldc;
  int tiles_m, tiles_n;
  int splits;          // k-ranges per output tile (grid.y = batch * splits)
  int kt_per_split;    // k-tiles per range
};

// Loads of one operand tile: 4 LDS-DMA instructions per wavefront, each
// filling 64 chunks (1 KB) of the tile: chunks (4*i + wave)*64 .. +63.
//   KC (k-contiguous, [128 rows][64 k]): instruction i covers rows
//     (4i + wave)*8 + lane/8, slot lane % 8, source chunk slot ^ swz(row);
//   IC (index-contiguous, [64 k][128 cols]): rows (4i + wave)*4 + lane/16,
//     slot lane % 16.
// The swizzle depends on the row modulo 8 (KC) or 16 (IC), which the
// instruction index does not change, so a lane's source chunk is fixed.
template <bool KC>
struct OperandLoader {
#if defined(__HIP_DEVICE_COMPILE__)
  __amdgpu_buffer_rsrc_t rsrc;
#endif
  uint32_t row_off[4];  // byte offset of this lane's row per instruction (KC: kOOR past the rows)
  uint32_t col_off;     // IC: byte offset of its chunk within the row (KC: in lane_k)
  int lane_k;           // KC: k of its chunk within a k-tile; IC: its row within a k-tile
  int ld_bytes;
  int K;

  // base: the operand's element (row0, 0) (KC) or (0, col0) (IC) of this
  // batch; rows: KC rows left from row0; extent_bytes: bytes from base to
  // the operand's last element (inclusive).
  __device__ __forceinline__ OperandLoader(const bf16* base, int ld, int rows, int k_total, int64_t extent_bytes,
                                           int wave, int lane) {
    ld_bytes = ld * 2;
    K = k_total;
    if constexpr (KC) {
      const int slot = lane & 7;
      const int r8 = lane >> 3;  // row modulo 8
      col_off = 0;
      lane_k = (slot ^ tile_swz<64>(r8)) * 8;  // the chunk's k (its byte offset is 2 lane_k)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = (4 * i + wave) * 8 + r8;
        row_off[i] = row < rows ? (uint32_t)(row * ld * 2) : kOOR;
      }
    } else {
      const int slot = lane & 15;
      const int rl = lane >> 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = (4 * i + wave) * 4 + rl;
        row_off[i] = (uint32_t)row;  // the row within a k-tile; scaled per load
      }
      const int r16 = (wave * 4 + rl) & 15;  // row modulo 16, the same for every instruction
      col_off = (uint32_t)((slot ^ tile_swz<128>(r16)) * 16);
      lane_k = 0;
    }
#if defined(__HIP_DEVICE_COMPILE__)
    const int64_t ext = extent_bytes < 0 ? 0 : (extent_bytes > 0x7fffffff ? 0x7fffffff : extent_bytes);
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(base), (short)0, (int)ext, 0x00020000);
#endif
  }

  // k-tile kt into the tile at `lds`.
  __device__ __forceinline__ void load(int kt, bf16* lds, int wave) const {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t off;
      if constexpr (KC) {
        const int k = kt * kBK + lane_k;
        off = (k < K && row_off[i] != kOOR) ? row_off[i] + (uint32_t)(k * 2) : kOOR;
      } else {
        const int k = kt * kBK + (int)row_off[i];
        off = k < K ? (uint32_t)k * (uint32_t)ld_bytes + col_off : kOOR;
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(lds + (4 * i + wave) * 64 * 8), 16, off, 0, 0,
                                               0);
    }
#endif
  }
};

// Fragment reads (LDS byte addresses), every fragment as two 8-byte halves
// so the tied wait below names the registers the reads wrote:
//   direct, natural order: chunk (2 ks + h) ^ swz, bytes 0-7 and 8-15;
//   direct, transposed order: chunks (2 ks) ^ swz and (2 ks + 1) ^ swz,
//     bytes 8h .. 8h+7 of each;
//   transposing: the two ds_read_b64_tr_b16 reads of the flash kernels' V^T
//     pattern for a 32-column block of the tile.
__device__ __forceinline__ void rd_b64(s16x4& r, uint32_t a) {
  asm volatile("ds_read_b64 %0, %1" : "=v"(r) : "v"(a));
}
__device__ __forceinline__ void rd_tr(s16x4& r, uint32_t a) {
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(a));
}

struct Frag {
  s16x4 lo, hi;
};
__device__ __forceinline__ bf16x8 frag_bits(const Frag& f) {
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(f.lo, f.hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// s_waitcnt lgkmcnt(0) tied to the four fragments of a k-step: their uses
// (and any copy of their registers) come after it.
__device__ __forceinline__ void wait_frags(Frag (&n)[2], Frag (&m)[2]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(n[0].lo), "+v"(n[0].hi), "+v"(n[1].lo), "+v"(n[1].hi), "+v"(m[0].lo), "+v"(m[0].hi),
                 "+v"(m[1].lo), "+v"(m[1].hi)
               :
               : "memory");
}

// Per-lane LDS byte offsets (within an operand tile) of the two halves of
// the fragments of 32-index block `blk`, for k-steps 0..3.
template <bool KC, bool PERM>
struct FragAddr {
  uint32_t a0[4], a1[4];
  __device__ __forceinline__ FragAddr(int blk, int lane) {
    const int half = lane >> 5, l32 = lane & 31;
    if constexpr (KC) {
      const int row = blk * 32 + l32;
      const int sw = tile_swz<64>(l32);  // row modulo 8 = l32 modulo 8
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if constexpr (!PERM) {
          a0[ks] = (uint32_t)((row * 64 + ((2 * ks + half) ^ sw) * 8) * 2);
          a1[ks] = a0[ks] + 8;
        } else {
          a0[ks] = (uint32_t)((row * 64 + ((2 * ks) ^ sw) * 8 + 4 * half) * 2);
          a1[ks] = (uint32_t)((row * 64 + ((2 * ks + 1) ^ sw) * 8 + 4 * half) * 2);
        }
      }
    } else {
      const int tj = lane & 15, tg = (lane >> 4) & 1;
      const int v_row = 4 * half + (tj >> 2);
      const int v_sw = tile_swz<128>(v_row), v_sw8 = tile_swz<128>(v_row + 8);
      const int v_chunk = tg * 2 + ((tj & 3) >> 1);
      const int v_sub = (tj & 1) * 4;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        a0[ks] = (uint32_t)(((ks * 16 + v_row) * 128 + v_sub + ((blk * 4 + v_chunk) ^ v_sw) * 8) * 2);
        a1[ks] = (uint32_t)(((ks * 16 + v_row + 8) * 128 + v_sub + ((blk * 4 + v_chunk) ^ v_sw8) * 8) * 2);
      }
    }
  }
  __device__ __forceinline__ void read(Frag& f, uint32_t tile, int ks) const {
    if constexpr (KC) {
      rd_b64(f.lo, tile + a0[ks]);
      rd_b64(f.hi, tile + a1[ks]);
    } else {
      rd_tr(f.lo, tile + a0[ks]);
      rd_tr(f.hi, tile + a1[ks]);
    }
  }
};

// TA: A stored [k][m]; TB: B stored [n][k].  E: 0 bf16, 1 f16 operands.
// OT: output type 0 f32, 1 bf16, 2 f16.
template <bool TA, bool TB, int E, int OT>
__global__ __launch_bounds__(kNT, 2) void gemm16_kernel(Params p) {
  constexpr bool A_KC = !TA;  // A read directly (k-contiguous rows)
  constexpr bool B_KC = TB;
  constexpr bool PERM = A_KC != B_KC;  // mixed: direct side in the transposed order
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * kStageElems];  // [stage][A tile | B tile]

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = lane >> 5, l32 = lane & 31;
  const int wm = wave & 1, wn = wave >> 1;
  const int tile = blockIdx.x, bz = blockIdx.y / p.splits, sp = blockIdx.y % p.splits;
  const int tm = tile / p.tiles_n, tn = tile % p.tiles_n;
  const int m0 = tm * kBM, n0 = tn * kBN;
  const int M = p.M, N = p.N, K = p.K;

  // Operand bases of this batch and tile, and their extents.
  const bf16* abase;
  int64_t aext;
  if constexpr (A_KC) {  // A [m][k]: rows m0 .. (last row M-1, ends at K)
    abase = p.a + bz * p.sa + (int64_t)m0 * p.lda;
    aext = ((int64_t)(M - 1 - m0) * p.lda + K) * 2;
  } else {  // A [k][m]: columns from m0, through row K-1's element M-1
    abase = p.a + bz * p.sa + m0;
    aext = ((int64_t)(K - 1) * p.lda + (M - m0)) * 2;
  }
  const bf16* bbase;
  int64_t bext;
  if constexpr (B_KC) {  // B [n][k]
    bbase = p.b + bz * p.sb + (int64_t)n0 * p.ldb;
    bext = ((int64_t)(N - 1 - n0) * p.ldb + K) * 2;
  } else {  // B [k][n]
    bbase = p.b + bz * p.sb + n0;
    bext = ((int64_t)(K - 1) * p.ldb + (N - n0)) * 2;
  }
  const OperandLoader<A_KC> aload(abase, p.lda, M - m0, K, aext, wave, lane);
  const OperandLoader<B_KC> bload(bbase, p.ldb, N - n0, K, bext, wave, lane);
  // This workgroup's k-tiles [kt0, kt1) (all of them without a split).
  const int nkt_all = (K + kBK - 1) / kBK;
  const int kt0 = sp * p.kt_per_split;
  const int kt1 = min(nkt_all, kt0 + p.kt_per_split);

  const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)smem;
  // MFMA A operand: n blocks wn*2 + j of the B tile; B operand: m blocks
  // wm*2 + i of the A tile.
  const FragAddr<B_KC, PERM && B_KC> fn0(wn * 2, lane), fn1(wn * 2 + 1, lane);
  const FragAddr<A_KC, PERM && A_KC> fm0(wm * 2, lane), fm1(wm * 2 + 1, lane);

  f32x16 acc[2][2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[j][i][e] = 0.f;

  if (kt0 < kt1) {
    aload.load(kt0, smem, wave);
    bload.load(kt0, smem + kTileElems, wave);
  }
  for (int kt = kt0; kt < kt1; ++kt) {
    tiles::wait_dma();
    __syncthreads();
    const int st = (kt - kt0) & 1;
    if (kt + 1 < kt1) {
      bf16* nxt = smem + (st ^ 1) * kStageElems;
      aload.load(kt + 1, nxt, wave);
      bload.load(kt + 1, nxt + kTileElems, wave);
    }
    const uint32_t at = lds0 + (uint32_t)(st * kStageElems * 2);
    const uint32_t bt = at + (uint32_t)(kTileElems * 2);
    Frag fn[2][2], fm[2][2];  // [set][block]
    fn0.read(fn[0][0], bt, 0);
    fn1.read(fn[0][1], bt, 0);
    fm0.read(fm[0][0], at, 0);
    fm1.read(fm[0][1], at, 0);
    wait_frags(fn[0], fm[0]);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int cs = ks & 1, ns = cs ^ 1;
      if (ks + 1 < 4) {
        fn0.read(fn[ns][0], bt, ks + 1);
        fn1.read(fn[ns][1], bt, ks + 1);
        fm0.read(fm[ns][0], at, ks + 1);
        fm1.read(fm[ns][1], at, ks + 1);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[j][i] = mfma16<E>(frag_bits(fn[cs][j]), frag_bits(fm[cs][i]), acc[j][i]);
      if (ks + 1 < 4) wait_frags(fn[ns], fm[ns]);
      fence();
    }
  }

  // Lane: row m = m0 + wm*64 + i*32 + l32; accumulator element g*4 + e:
  // column n = n0 + wn*64 + j*32 + g*8 + half*4 + e (N % 4 == 0: a run of
  // 4 is all in range or all out).
  if constexpr (OT != 0) {
    // 16-bit outputs through LDS, so each store instruction writes 8 rows x
    // 128 bytes of the wavefront's 64 x 64 block instead of 32 rows x 16:
    // after a barrier the stages are free (every wavefront's last fragments
    // are read and no load is in flight), 8 KB per wavefront; 16-byte chunk
    // c of row r at slot c ^ (r % 8).  Needs whole 16-byte chunks in range
    // and aligned: N, ldc and the batch stride multiples of 8, C 16-byte
    // aligned (uniform over the grid).  The rows are streamed past the L2
    // (whole lines, written once).
    if (!p.part && ((N | p.ldc) & 7) == 0 && (p.sc & 7) == 0 && ((uintptr_t)p.c & 15) == 0) {
      __syncthreads();
      bf16* const st = smem + wave * 64 * 64;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            u16x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = store_e<OT - 1>(acc[j][i][g * 4 + e]);
            const int r = i * 32 + l32, c = j * 4 + g;
            *reinterpret_cast<u16x4*>(st + r * 64 + (c ^ (r & 7)) * 8 + half * 4) = w;
          }
      // (The block's first row comes from an opaque copy, so no address is
      // hoisted into the k loop.)
      int mb = m0 + wm * 64;
      asm volatile("" : "+v"(mb));
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int r = k * 8 + (lane >> 3), c = lane & 7;
        const u32x4 v = *reinterpret_cast<const u32x4*>(st + r * 64 + (c ^ (r & 7)) * 8);
        const int m = mb + r, n = n0 + wn * 64 + c * 8;
        if (m < M && n < N)
          __builtin_nontemporal_store(
              v, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p.c) + bz * p.sc + (int64_t)m * p.ldc + n));
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = m0 + wm * 64 + i * 32 + l32;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * 64 + j * 32 + g * 8 + half * 4;
        if (n >= N) continue;
        if (p.part) {
          // Split-K partial of this k-range, fp32, [M][N] per (batch, range).
          const f32x4 w = {acc[j][i][g * 4], acc[j][i][g * 4 + 1], acc[j][i][g * 4 + 2], acc[j][i][g * 4 + 3]};
          float* dst = p.part + ((int64_t)blockIdx.y * M + m) * N + n;
          *reinterpret_cast<f32x4*>(dst) = w;
          continue;
        }
        const int64_t off = bz * p.sc + (int64_t)m * p.ldc + n;
        if constexpr (OT == 0) {
          const f32x4 w = {acc[j][i][g * 4], acc[j][i][g * 4 + 1], acc[j][i][g * 4 + 2], acc[j][i][g * 4 + 3]};
          *reinterpret_cast<f32x4*>(static_cast<float*>(p.c) + off) = w;
        } else {
          u16x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = store_e<OT - 1>(acc[j][i][g * 4 + e]);
          *reinterpret_cast<u16x4*>(static_cast<uint16_t*>(p.c) + off) = w;
        }
      }
  }
}

// C = sum over the k-ranges of the partials, rounded to the output type:
// one thread per 4 consecutive outputs of a row (N % 4 == 0), the ranges
// summed in order (deterministic).
template <int OT>
__global__ __launch_bounds__(256) void gemm16_sum_kernel(Params p, int64_t quads_per_batch) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int bz = blockIdx.y;
  if (q >= quads_per_batch) return;
  const int64_t e = q * 4;  // element of [M][N]
  const int m = (int)(e / p.N), n = (int)(e % p.N);
  const float* src = p.part + (int64_t)bz * p.splits * p.M * p.N + e;
  f32x4 acc = *reinterpret_cast<const f32x4*>(src);
  for (int s = 1; s < p.splits; ++s) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(src + (int64_t)s * p.M * p.N);
    acc += v;
  }
  const int64_t off = bz * p.sc + (int64_t)m * p.ldc + n;
  if constexpr (OT == 0) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(p.c) + off) = acc;
  } else {
    u16x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = store_e<OT - 1>(acc[i]);
    *reinterpret_cast<u16x4*>(static_cast<uint16_t*>(p.c) + off) = w;
  }
}

template <bool TA, bool TB, int E>
int launch_o(const Params& p, int c_dtype, int64_t batch, hipStream_t s) {
  const dim3 grid((unsigned)(p.tiles_m * p.tiles_n), (unsigned)(batch * p.splits));
  if (c_dtype == MFX_F32) hipLaunchKernelGGL((gemm16_kernel<TA, TB, E, 0>), grid, dim3(kNT), 0, s, p);
  else if (c_dtype == MFX_BF16) hipLaunchKernelGGL((gemm16_kernel<TA, TB, E, 1>), grid, dim3(kNT), 0, s, p);
  else hipLaunchKernelGGL((gemm16_kernel<TA, TB, E, 2>), grid, dim3(kNT), 0, s, p);
  int rc = launch_status("gemm16_kernel");
  if (rc != MFX_OK || !p.part) return rc;
  const int64_t quads = (int64_t)p.M * p.N / 4;
  const dim3 sgrid((unsigned)((quads + 255) / 256), (unsigned)batch);
  if (c_dtype == MFX_F32) hipLaunchKernelGGL((gemm16_sum_kernel<0>), sgrid, dim3(256), 0, s, p, quads);
  else if (c_dtype == MFX_BF16) hipLaunchKernelGGL((gemm16_sum_kernel<1>), sgrid, dim3(256), 0, s, p, quads);
  else hipLaunchKernelGGL((gemm16_sum_kernel<2>), sgrid, dim3(256), 0, s, p, quads);
  return launch_status("gemm16_sum_kernel");
}

template <int E>
int launch_e(const Params& p, const mfx_gemm_args& a, hipStream_t s) {
  if (a.trans_a) {
    return a.trans_b ? launch_o<true, true, E>(p, a.c_dtype, a.batch, s)
                     : launch_o<true, false, E>(p, a.c_dtype, a.batch, s);
  }
  return a.trans_b ? launch_o<false, true, E>(p, a.c_dtype, a.batch, s)
                   : launch_o<false, false, E>(p, a.c_dtype, a.batch, s);
}

bool aligned(const void* ptr, uintptr_t n) { return ((uintptr_t)ptr % n) == 0; }

}  // namespace

bool gemm16_supported(const mfx_gemm_args& a) {
  if (a.dtype != MFX_BF16 && a.dtype != MFX_F16) return false;
  if (a.c_dtype != MFX_F32 && a.c_dtype != MFX_BF16 && a.c_dtype != MFX_F16) return false;
  if (a.k <= 0 || a.k % 8 || a.n % 4) return false;
  if (a.batch > 65535) return false;
  if (!aligned(a.a, 16) || !aligned(a.b, 16)) return false;
  if (a.lda % 8 || a.ldb % 8 || a.stride_a % 8 || a.stride_b % 8) return false;
  const int csz = a.c_dtype == MFX_F32 ? 16 : 8;  // a run of 4 outputs
  if (!aligned(a.c, csz) || a.ldc % 4 || a.stride_c % 4) return false;
  // Byte offsets a load forms, per operand tile (32-bit lane offsets).
  const int64_t lim = 1LL << 31;
  const int64_t a_off = a.trans_a ? (a.k * a.lda + a.m) * 2 : ((int64_t)kBM * a.lda + a.k) * 2;
  const int64_t b_off = a.trans_b ? ((int64_t)kBN * a.ldb + a.k) * 2 : (a.k * a.ldb + a.n) * 2;
  if (a_off >= lim || b_off >= lim) return false;
  if (a.m >= lim || a.n >= lim || a.k >= lim) return false;
  const int64_t tiles = ((a.m + kBM - 1) / kBM) * ((a.n + kBN - 1) / kBN);
  return tiles < lim;
}

int gemm16_launch(const mfx_gemm_args& a, hipStream_t s) {
  Params p;
  p.a = static_cast<const bf16*>(a.a);
  p.b = static_cast<const bf16*>(a.b);
  p.c = a.c;
  p.sa = a.stride_a;
  p.sb = a.stride_b;
  p.sc = a.stride_c;
  p.M = (int)a.m;
  p.N = (int)a.n;
  p.K = (int)a.k;
  p.lda = (int)a.lda;
  p.ldb = (int)a.ldb;
  p.ldc = (int)a.ldc;
  p.tiles_m = (int)((a.m + kBM - 1) / kBM);
  p.tiles_n = (int)((a.n + kBN - 1) / kBN);
  // Split K when the output tiles number fewer than the CUs and there is K
  // to spread (each range keeps at least 4 k-tiles), up to two workgroups
  // per CU.  (With one tile per CU or more, the partials' extra traffic
  // costs more than the idle half of the CUs: [8192, 512, 2048] runs 33 us
  // whole and 36 us in two ranges.)
  const int nkt = (int)((a.k + kBK - 1) / kBK);
  const int64_t wgs = (int64_t)p.tiles_m * p.tiles_n * a.batch;
  const int64_t cus = device_cu_count();
  const int64_t want = 2 * cus;
  int splits = 1;
  if (wgs < cus) {
    const int64_t by_wgs = (want + wgs - 1) / wgs;
    const int by_k = nkt / 4;
    splits = (int)(by_wgs < by_k ? by_wgs : by_k);
    if (splits < 1) splits = 1;
  }
  p.kt_per_split = (nkt + splits - 1) / splits;
  p.splits = (nkt + p.kt_per_split - 1) / p.kt_per_split;  // no empty range
  p.part = nullptr;
  if (p.splits > 1) {
    const size_t bytes = (size_t)a.batch * p.splits * a.m * a.n * sizeof(float);
    p.part = static_cast<float*>(device_scratch(bytes, s));
    if (!p.part) return MFX_E_HIP;
  }
  return a.dtype == MFX_F16 ? launch_e<1>(p, a, s) : launch_e<0>(p, a, s);
}

}  // namespace mfx
