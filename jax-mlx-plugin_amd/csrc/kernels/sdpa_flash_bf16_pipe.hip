// Flash attention forward without an additive mask (causal or not), bf16
// inputs, fp32 accumulation, gfx950 MFMA, software-pipelined per wavefront.
//
// Workgroup = 4 wavefronts = 128 query rows of one (batch, head); each
// wavefront owns 32 query rows, held as the B operand of S^T = K Q^T in
// registers.  K and V tiles of 64 keys stream through two LDS stages each by
// LDS-DMA (buffer_load ... lds); one vmcnt wait + barrier per tile publishes
// them.  The products and the operand layouts are those of the masked kernel
// (sdpa_flash_bf16.hip): S^T = K Q^T and O^T = V^T P^T on
// v_mfma_f32_32x32x16_bf16, P taken from the S^T accumulator, V^T fragments
// from transposing LDS reads.
//
// The difference is the schedule and the softmax's vector work.  There is
// no per-tile row max: a row's exp2 base is its first tile's max, and a tile
// whose row sum passes kSumCap (a score more than 11 above the base, in log2
// units) takes a rare path that raises the base, rescales O and l, and
// recomputes that tile's P.  Per tile and wavefront the vector work is 32
// FMA + exp2, 16 bf16 packs and 16 dot2 row sums, spread evenly over the 32
// MFMAs (the exp2 is the one costly instruction: about 2.5 ns per MFMA it
// shares a slot with, where FMAs and packs are free):
//   phase A: S(t+1) = K(t+1) Q^T, with the exp2 of keys 32-63 of S(t)
//            between the MFMAs;
//   phase B: O^T += V^T(t) P(t)^T, with the exp2 of keys 0-31 of S(t+1)
//            between the MFMAs.
// The LDS operand reads are inline asm issued a fixed distance ahead of their
// MFMAs, each followed by an lgkmcnt wait that counts the reads issued after
// it (LDS reads complete in order); the compiler therefore adds no waits of
// its own for the LDS-DMA into the other stage.  sched_barrier fences keep
// this interleave as written.
//
// A wavefront's last tile runs outside the loop (tile_last: no S of a next
// tile), its registers moved to the even-tile set and its V stage a runtime
// offset, so the loop keeps its two tile bodies and the kernel stays
// spill-free.
//
// MT != 0 adds an additive mask that does not vary along query rows (element
// strides [b, h, 0, key]: padding masks, per-head key biases) of type f32
// (MT 1), bf16 (2) or f16 (3).  Wavefront 0 loads a tile's 64 values one
// tile ahead (one lane per key, issued with the K DMA), converts them to raw
// score units (mask_log2 / (scale * log2 e), finite values held at or above
// -2^30 in log2 units, -inf kept) and writes them to a 64-float LDS row before the
// barrier that publishes the tile.  The S products of the tile start from
// that row instead of zero (the MFMA's accumulator input), so S comes out as
// Q K^T + mask / (scale * log2 e) and the exp2, row-max, rebase and row-sum
// code runs unchanged, with no vector work for the mask.  Masks that vary
// along query rows run on the kernel of sdpa_flash_bf16.hip.  No spill is allowed here: the inline-asm LDS reads complete
// after the asm statement, and a spill or copy of a destination register
// placed before its lgkmcnt wait would save the value before it arrives.
//
// Built with -DMFX_PHASE_TIMERS (build.py --phase-timers, a separate
// diagnostic library), every wavefront also records where its time goes:
// s_memrealtime stamps (100 MHz) at its start, when its first tiles have
// landed, at its loop entry and at its end, and s_memtime (shader clock)
// sums over its phases -- S MFMAs with the exp2 of the previous tile (A), the
// row-sum check (C), PV MFMAs (B), the barrier with the next tiles' DMA issue
// (S) and the last tile -- read at points where none of its inline-asm LDS
// reads is outstanding.  mfx_phase_timers_read() copies the records out;
// jax-mlx-plugin_amd/phase_budget.py turns them into the per-tile budget.
#include <type_traits>

#include "sdpa_elem.h"
#include "sdpa_tiles.h"

#if defined(MFX_PHASE_TIMERS)
#define PHASE(...) __VA_ARGS__
#else
#define PHASE(...)
#endif

namespace mfx {

#if defined(MFX_PHASE_TIMERS)
// One record of kPhaseFields u64 per wavefront (blockIdx.x * 4 + wave).
constexpr int kPhaseRecords = 1 << 15;
constexpr int kPhaseFields = 20;
__device__ unsigned long long g_phase_records[kPhaseRecords * kPhaseFields];

struct PhaseClock {
  // 32-bit fields keep the kernel's SGPR budget: cycle sums of one
  // wavefront stay far below 2^32, and realtime stamps keep their low word
  // (the host rebuilds them from the 64-bit end stamp).
  unsigned rt_start, rt_ready = 0, rt_loop = 0, c_start, c_loop = 0;
  unsigned cyc_a = 0, cyc_check = 0, cyc_b = 0, cyc_sync = 0, cyc_last = 0;
  unsigned tiles = 0, rebases = 0, cyc_vmwait = 0, cyc_barrier = 0, cyc_dma_k = 0;
  __device__ static unsigned now() { return (unsigned)__builtin_amdgcn_s_memtime(); }
  __device__ static unsigned real() { return (unsigned)__builtin_amdgcn_s_memrealtime(); }
  __device__ PhaseClock() : rt_start(real()), c_start(now()) {}
  // Fields: 0 ids (XCC id, HW_ID, (batch*H + head), q-block), 1-3 realtime
  // start / first tiles landed / loop entry (low words), 4 realtime end
  // (64 bits), 5-9 cycles of phases A / check / B / barrier+DMA / last tile,
  // 10 tiles in the loop, 11 rebases, 12 total cycles, 13 cycles before the
  // loop, 14 (workgroup tiles, wavefront tiles), 15 cycles of the epilogue,
  // 16 / 17 cycles of the barrier phase spent in its vmcnt wait / s_barrier,
  // 18 cycles of issuing the K tile's DMA (the rest of the phase issues V's).
  __device__ void write(int lane, int rec, int bh, int mblk, int N, int nw, unsigned c_epi) const {
    unsigned xcc, hwid;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hwid));
    const unsigned c_end = now();
    const unsigned long long rt_end = __builtin_amdgcn_s_memrealtime();
    if (lane != 0 || rec >= kPhaseRecords) return;
    unsigned long long* r = g_phase_records + (size_t)rec * kPhaseFields;
    r[0] = (unsigned long long)(xcc & 0xff) | ((unsigned long long)hwid << 8) | ((unsigned long long)bh << 40) |
           ((unsigned long long)(mblk & 0xff) << 56);
    r[1] = rt_start;
    r[2] = rt_ready;
    r[3] = rt_loop;
    r[4] = rt_end;
    r[5] = cyc_a;
    r[6] = cyc_check;
    r[7] = cyc_b;
    r[8] = cyc_sync;
    r[9] = cyc_last;
    r[10] = tiles;
    r[11] = rebases;
    r[12] = c_end - c_start;
    r[13] = c_loop - c_start;
    r[14] = ((unsigned long long)(unsigned)N << 32) | (unsigned)nw;
    r[15] = c_end - c_epi;
    r[16] = cyc_vmwait;
    r[17] = cyc_barrier;
    r[18] = cyc_dma_k;
  }
};
#endif

namespace {

constexpr int kBM = 128;  // query rows per workgroup
constexpr int kBN = 64;   // keys per tile
constexpr int kNW = 4;    // wavefronts per workgroup
constexpr int kNT = kNW * 64;
constexpr int kPfK = 4;   // K operand reads issued ahead of their S MFMA
constexpr int kPfV = 4;   // V read pairs issued ahead of their PV MFMA
constexpr int kHeadGroup = 4;  // heads whose q-blocks an XCD issues together

using tiles::kSlack;
// Row-sum cap of one tile (32 keys per lane), kMaxP of the element type: a
// sum above it (or NaN) means a score passed the base by more than
// log2(kMaxP / 32) = 11 (bf16) or 10 (f16) > kSlack.
using tiles::s16x4;
using tiles::tile_swz;
using tiles::wait_dma;
using tiles::ds_b128;
using tiles::ds_tr;
using tiles::lgkm_tie;
using tiles::fence;
using tiles::static_for;

// K / V tile loader: rows [t*kBN, t*kBN + kBN) of one (batch, head) into a
// swizzled LDS tile.  Instruction i of a wavefront covers rows
// i*STEP + wave*RPI + lane/DCH of the tile.  One buffer resource spans this
// head's elements, from its first row's first feature to its last row's
// last feature (row_elems = the head size, which is below D when rows load
// tile-wide); the tile, instruction and lane offsets all go into the
// per-lane offset, which the hardware range-checks, so rows past Tk and the
// last row's features past the head read as zeros and no address leaves the
// tensor (with heads interleaved in a row, the last head's tile-wide last
// row would otherwise run past the tensor's end).
template <int D>
struct Loader {
  static constexpr int DCH = D / 8;
  static constexpr int RPI = 64 / DCH;
  static constexpr int LOADS = kBN * DCH / (64 * kNW);
  static constexpr int STEP = kNW * RPI;
  static_assert(STEP % tiles::kSwzPeriod<D> == 0 && kBN % tiles::kSwzPeriod<D> == 0, "one offset per lane");
#if defined(__HIP_DEVICE_COMPILE__)
  __amdgpu_buffer_rsrc_t rsrc;
#endif
  uint32_t voff;
  uint32_t tile_bytes;
  uint32_t step_bytes;
  __device__ __forceinline__ Loader(const bf16* b, int64_t row_stride, int Tk, int row_elems, int wave, int lane) {
    tile_bytes = (uint32_t)(kBN * row_stride * 2);
    step_bytes = (uint32_t)(STEP * row_stride * 2);
    const int row = wave * RPI + lane / DCH, slot = lane % DCH;
    voff = (uint32_t)(((int64_t)row * row_stride + (slot ^ tile_swz<D>(row)) * 8) * 2);
#if defined(__HIP_DEVICE_COMPILE__)
    const int64_t extent = Tk > 0 ? ((int64_t)(Tk - 1) * row_stride + row_elems) * 2 : 0;
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(b), (short)0, (int)extent, 0x00020000);
#endif
  }
  __device__ __forceinline__ void load(int t, bf16* lds, int wave) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t vo = voff + (uint32_t)t * tile_bytes;
#pragma unroll
    for (int i = 0; i < LOADS; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (tiles::lds_void_t*)(lds + (kNW * i + wave) * 64 * 8), 16,
                                               vo + (uint32_t)i * step_bytes, 0, 0, 0);
#endif
  }
};

// lgkmcnt of the wait before S MFMA j (MS per tile, reads pf ahead) and
// before PV MFMA j (MP per tile, read pairs pf ahead): the reads issued
// after the one the MFMA needs.
constexpr int wait_k(int j, int MS, int pf) { return pf < MS - 1 - j ? pf : MS - 1 - j; }
constexpr int wait_v(int j, int MP, int pf) { return 2 * (pf < MP - 1 - j ? pf : MP - 1 - j); }

// D: features per row of the LDS tiles (64 or 128); DV <= D: the head size,
// a multiple of 32.  Rows are loaded D wide, and only features below DV
// reach an MFMA: S contracts over DV features (DV/16 k-steps) and O has DV/32
// feature blocks, so the features DV .. D-1 of a tile (the next row's first
// elements, or zeros past the tensor) are never read from LDS.  (256-wide
// rows do not fit: the loop's state passes 512 registers.)
template <int D, int DV, bool CAUSAL, int MT, int E>
__global__ __launch_bounds__(kNT, 2) void flash_bf16_pipe_kernel(SdpaParams p) {
  static_assert(DV % 32 == 0 && DV <= D && D - DV < 64, "head size");
  constexpr int TILE = kBN * D;     // elements of one K or V tile
  constexpr int TB = TILE * 2;      // its bytes
  constexpr int MS = 2 * (DV / 16);  // S MFMAs per tile
  constexpr int MP = 4 * (DV / 32);  // PV MFMAs per tile
  // LDS read offsets are 16-bit immediates: tiles wider than 128 features
  // would put the V stages past 64 KB, addressed from a per-lane base that
  // includes their start.
  constexpr int VA0 = D > 128 ? 2 * TB : 0;
  constexpr bool MASK = MT != 0;
  // Operand reads ahead of their MFMA: 2, 4 and 6 measured alike on config
  // 3; a masked kernel keeps 2 for the registers its mask rows take.
  constexpr int PFK = MASK ? 2 : kPfK, PFV = MASK ? 2 : kPfV;
  constexpr float kSumCap = kMaxP<E>;
  static_assert(MS >= 4 && MP >= 4, "the 8 exp2 pairs of a phase spread over its MFMAs");
  __shared__ __attribute__((aligned(16))) bf16 smem[4 * TILE];  // K0 K1 V0 V1
  // Mask rows (raw score units) of the tiles in K stages 0 / 1 (MASK only):
  // an array of its own, so the compiler's reads of it need no wait for the
  // K/V DMA into smem.
  __shared__ __attribute__((aligned(16))) float mrow_lds[MASK ? 2 : 1][kBN];

  PHASE(PhaseClock ph;)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;

  const int nmb = (p.Tq + kBM - 1) / kBM;
  const int BH = p.B * p.Hq;
  const int id = blockIdx.x;
  int bh, mblk;
  if ((BH & 7) == 0) {
    // Blocks are dealt to the 8 XCDs round-robin.  Each XCD works through
    // its heads in groups: all q-blocks of a group are issued together,
    // longest first, so they stream the group's K/V tiles at about the same
    // time and mostly hit the XCD's L2.
    const int hg = ((BH >> 3) % kHeadGroup) == 0 ? kHeadGroup : 1;
    const int xcd = id & 7, slot = id >> 3;
    const int grp = slot / (hg * nmb), r = slot % (hg * nmb);
    bh = (grp * hg + r % hg) * 8 + xcd;
    mblk = nmb - 1 - r / hg;
  } else {
    bh = id % BH;
    mblk = nmb - 1 - id / BH;
  }
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h / p.group;
  const bf16* qp = static_cast<const bf16*>(p.q) + b * p.qs[0] + h * p.qs[1];
  const bf16* kp = static_cast<const bf16*>(p.k) + b * p.ks[0] + hk * p.ks[1];
  const bf16* vp = static_cast<const bf16*>(p.v) + b * p.vs[0] + hk * p.vs[1];
  bf16* op = static_cast<bf16*>(p.out) + b * p.os[0] + h * p.os[1];
  const int64_t qs2 = p.qs[2], os2 = p.os[2];
  const int Tq = p.Tq, Tk = p.Tk;
  // Mask row of this (batch, head): element offset of key 0 (MASK only).
  const int64_t mrow = MASK ? b * p.ms[0] + h * p.ms[1] : 0;
  // Raw mask value of key t*kBN + lane (keys past Tk read the last key's:
  // they are masked per element anyway).
  // The lane index goes through an opaque copy here and in mask_store, so
  // the per-lane addresses are formed at each use rather than hoisted and
  // kept in registers across the loop (they serve wavefront 0 only).
  auto mask_raw = [&](int t) -> float {
    int l = lane;
    asm volatile("" : "+v"(l));
    const int64_t key = min(t * kBN + l, Tk - 1);
    if constexpr (MASK) return load_mask_t<MT>(p.mask, mrow + key * p.ms[3]);
    return 0.f;
  };
  // Wavefront 0: converts a raw mask value to score units and stores it as
  // key `lane` of mask row `stage`: log2 units held at or above -2^30, then
  // divided by scale * log2(e); -inf stays -inf.  The floor outweighs any
  // score (a key at it gets weight 0 beside a real one) and is absorbed by
  // the scores it is added to (|s * scale * log2 e| <= 64), so keys at it
  // hold equal S values; and since |floor| < 2^31 the exp2 FMA's rounding
  // residual stays below 64, the same for equal S values: a row whose keys
  // all carry the floor (JAX's finite -0.7 * FLT_MAX mask) gets equal finite
  // weights, the mean of V, where the softmax of where(mask, s, floor) does.
  const float inv_sl2 = p.inv_scale_log2;
  auto mask_store = [&](float raw, int stage) {
    if constexpr (MASK) {
      int l = lane;
      asm volatile("" : "+v"(l));
      const float m = mask_log2(raw);
      mrow_lds[stage][l] = m == -INFINITY ? m : fmaxf(m, -1073741824.f) * inv_sl2;
    }
  };
  // Accumulator seed of S chain mt (32-key block) for the tile in `stage`:
  // element i is key mt*32 + (i/4)*8 + half*4 + i%4 of the row.
  auto mask_seed = [&](int stage, int mt) -> f32x16 {
    f32x16 r = {};
    if constexpr (MASK) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const f32x4 m = *reinterpret_cast<const f32x4*>(&mrow_lds[stage][mt * 32 + g4 * 8 + half * 4]);
#pragma unroll
        for (int e = 0; e < 4; ++e) r[g4 * 4 + e] = m[e];
      }
    }
    return r;
  };

  const int q0 = mblk * kBM + wave * 32;  // first query row of this wavefront (uniform)
  const int qi = q0 + l32;

  // Tiles of the workgroup (N) and of this wavefront (nw).
  int kv_end = Tk;
  if (CAUSAL) kv_end = min(Tk, min(Tq, (mblk + 1) * kBM));
  const int N = (kv_end + kBN - 1) / kBN;
  int nw = 0;
  if (q0 < Tq) {
    const int e = CAUSAL ? min(Tk, min(Tq - 1, q0 + 31) + 1) : Tk;
    nw = (e + kBN - 1) / kBN;
  }
  // Tile t needs per-element masking (ragged end, causal diagonal).
  auto edge = [&](int t) { return (t + 1) * kBN > Tk || (CAUSAL && t * kBN + kBN - 1 > q0); };

  const Loader<D> kload(kp, p.ks[2], Tk, DV, wave, lane), vload(vp, p.vs[2], Tk, DV, wave, lane);
  bf16* const kst[2] = {smem, smem + TILE};
  bf16* const vst[2] = {smem + 2 * TILE, smem + 3 * TILE};
  // Raw mask value of the next tile wavefront 0 converts at the next barrier.
  float mraw = 0.f;
  if (MASK && wave == 0 && N > 0) {
    mask_store(mask_raw(0), 0);
    if (N > 1) mraw = mask_raw(1);
  }
  if (N > 0) {
    kload.load(0, kst[0], wave);
    if (N > 1) kload.load(1, kst[1], wave);
    vload.load(0, vst[0], wave);
  }

  // Q rows as the B operand (rows past Tq read a valid row and are zeroed).
  bf16x8 qf[DV / 16];
  {
    const bf16* qrow = qp + (int64_t)min(qi, Tq - 1) * qs2 + half * 8;
#pragma unroll
    for (int kk = 0; kk < DV / 16; ++kk) {
      u32x4 raw = *reinterpret_cast<const u32x4*>(qrow + kk * 16);
      if (qi >= Tq) raw = u32x4{0u, 0u, 0u, 0u};
      qf[kk] = __builtin_bit_cast(bf16x8, raw);
    }
  }

  // LDS byte addresses of the operand reads; the stage, the 32-key block of
  // the K tile and the 16-key step of the V tile are immediate offsets.
  const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)smem;
  uint32_t ka[DV / 16];
  {
    const int k_sw = tile_swz<D>(l32);
#pragma unroll
    for (int kk = 0; kk < DV / 16; ++kk) ka[kk] = base + (uint32_t)((l32 * D + ((kk * 2 + half) ^ k_sw) * 8) * 2);
  }
  uint32_t va[DV / 32][2];
  {
    // Transposing reads: 16 lanes x 4 keys per read; k-slots 0-3 are keys
    // 4*half + e of the 16-key step, slots 4-7 the same + 8.
    const int tj = lane & 15, tg = (lane >> 4) & 1;
    const int v_row = 4 * half + (tj >> 2);
    const int v_sw = tile_swz<D>(v_row), v_sw8 = tile_swz<D>(v_row + 8);
    const int v_chunk = tg * 2 + ((tj & 3) >> 1);
    const int v_sub = (tj & 1) * 4;
#pragma unroll
    for (int dt = 0; dt < DV / 32; ++dt) {
      va[dt][0] = base + VA0 + (uint32_t)((v_row * D + v_sub + ((dt * 4 + v_chunk) ^ v_sw) * 8) * 2);
      va[dt][1] = base + VA0 + (uint32_t)(((v_row + 8) * D + v_sub + ((dt * 4 + v_chunk) ^ v_sw8) * 8) * 2);
    }
  }

  f32x16 o[DV / 32];
#pragma unroll
  for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
  // Running exp2 base of the row (log2 units, shared by lanes l and l^32),
  // -base for the exp2 FMA, and the lane's partial row sum.
  float b_run = 0.f, nbase = 0.f, l_run = 0.f;
  const float sl2 = p.scale_log2;  // > 0 (checked on the host)
  f32x16 s0[2], s1[2];   // S^T of two tiles: 2 x 32 keys, lane = query
  u32x4 pf0[2], pf1[2];  // P of keys 0-31 (16-key steps 0, 1) of even / odd tiles, bf16 pairs
  u32x4 pb[2];           // P of keys 32-63 (steps 2, 3) of the current tile
  float lf = 0.f;        // row-sum part of keys 0-31 of the next tile

  // Masks S of tile t per element where keys pass Tk or the diagonal.
  auto mask_tile = [&](f32x16 (&s)[2], int t) {
    const int kb = t * kBN;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb + mt * 32 + (i >> 2) * 8 + half * 4 + (i & 3);
        if (key >= Tk || (CAUSAL && key > qi)) s[mt][i] = -INFINITY;
      }
  };
  // Row max of S: 32 in-lane values, then lanes l and l^32.
  auto row_max = [&](f32x16 (&s)[2]) -> float {
    float m0 = -INFINITY, m1 = -INFINITY;
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      const float x = s[g >> 3][(g & 7) * 2], y = s[g >> 3][(g & 7) * 2 + 1];
      if (g & 1) m1 = fmaxf(m1, fmaxf(x, y));
      else m0 = fmaxf(m0, fmaxf(x, y));
    }
    const float mx = fmaxf(m0, m1);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
  };
  // exp2 of pair g of S (keys 2g, 2g+1 of the lane's 32) into P (element
  // type E) and the row sum of exactly those rounded values.
  auto exp_pair = [&](f32x16 (&s)[2], int g, u32x4 (&dst)[2], float& acc) {
    const int mt = g >> 3, i = (g & 7) * 2;
    const float p0 = __builtin_amdgcn_exp2f(fmaf(s[mt][i], sl2, nbase));
    const float p1 = __builtin_amdgcn_exp2f(fmaf(s[mt][i + 1], sl2, nbase));
    const uint32_t wu = pack2<E>(p0, p1);
    acc = dot2<E>(wu, acc);
    // Keeps the work in this MFMA's slot: without a use here the compiler
    // sinks it past the branches between the phases, behind the MFMAs.
    asm volatile("" ::"v"(wu), "v"(acc));
    dst[i >> 3][(i & 7) >> 1] = wu;
  };
  // A tile whose row sum passed kSumCap has a score above the base by more
  // than log2(kSumCap / 32) > kSlack: raise the base of such rows to their
  // max, rescale O and l to it, and recompute the tile's P.  Returns the
  // tile's new row sum.
  auto rebase = [&](f32x16 (&sc)[2], u32x4 (&pc)[2]) -> float {
    const float rel = row_max(sc) * sl2 - b_run;
    const float d = rel > kSlack ? rel : 0.f;
    float alpha;
    if constexpr (MASK) {
      // Scores at the mask floor sit near -2^30 in log2 units, where b_run + d
      // can round back to b_run: scale by the change that happened.
      const float nb = b_run + d;
      alpha = __builtin_amdgcn_exp2f(b_run - nb);
      b_run = nb;
    } else {
      alpha = __builtin_amdgcn_exp2f(-d);
      b_run += d;
    }
    nbase = -b_run;
    l_run *= alpha;
#pragma unroll
    for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int g = 0; g < 8; ++g) exp_pair(sc, g, pc, a0);
#pragma unroll
    for (int g = 8; g < 16; ++g) exp_pair(sc, g, pb, a1);
    return a0 + a1;
  };

  // S of the tile in K stage 0, not interleaved (before the loop).
  auto s_plain = [&](f32x16 (&s)[2]) {
    bf16x8 kr[MS];
#pragma unroll
    for (int j = 0; j < MS; ++j) {
      if ((j & 1) == 0) ds_b128<0>(kr[j], ka[j >> 1]);
      else ds_b128<32 * D * 2>(kr[j], ka[j >> 1]);
    }
#pragma unroll
    for (int j = 0; j < MS; ++j) lgkm_tie<0>(kr[j]);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) s[mt] = mask_seed(0, mt);
#pragma unroll
    for (int j = 0; j < MS; ++j) s[j & 1] = mfma16<E>(kr[j], qf[j >> 1], s[j & 1]);
  };

  // One tile t: K stage KS holds tile t+1, V stage VS tile t; sc = S(t)
  // (keys 0-31 already exponentiated into pc), sn receives S(t+1).
  //   phase A: the S(t+1) MFMAs, with the exp2 of keys 32-63 of S(t) between them;
  //   phase B: the PV(t) MFMAs, with the exp2 of keys 0-31 of S(t+1) (into pn) between them.
  // The row-sum check between the phases runs the rebase before P(t) is used.
  auto tile = [&](f32x16 (&sc)[2], f32x16 (&sn)[2], u32x4 (&pc)[2], u32x4 (&pn)[2], int t, auto ks_tag,
                  auto vs_tag) {
    constexpr int KS = decltype(ks_tag)::value;
    constexpr int VB = (2 + decltype(vs_tag)::value) * TB - VA0;
    bf16x8 kr[MS];
    s16x4 vr[MP][2];
    auto rdk = [&](auto j_tag) {  // S MFMA j: 32-key block j & 1, d-slice j >> 1
      constexpr int j = decltype(j_tag)::value;
      if constexpr ((j & 1) == 0) ds_b128<KS * TB>(kr[j], ka[j >> 1]);
      else ds_b128<KS * TB + 32 * D * 2>(kr[j], ka[j >> 1]);
    };
    auto rdv = [&](auto j_tag) {  // PV MFMA j: d-block j % (DV/32), 16-key step j / (DV/32)
      constexpr int j = decltype(j_tag)::value;
      constexpr int dt = j % (DV / 32), ks = j / (DV / 32);
      ds_tr<VB + ks * 16 * D * 2>(vr[j][0], va[dt][0]);
      ds_tr<VB + ks * 16 * D * 2>(vr[j][1], va[dt][1]);
    };
    float ls = 0.f;
    PHASE(const unsigned c0 = PhaseClock::now(); fence();)
    // S(t+1) starts from tile t+1's mask row (zero without a mask); the
    // second chain's seed is read once the first MFMA is issued.
    const f32x16 seed0 = mask_seed((t + 1) & 1, 0);
    f32x16 seed1 = {};
    static_for<0, PFK>(rdk);
    fence();
    static_for<0, MS>([&](auto j_tag) {
      constexpr int j = decltype(j_tag)::value;
      if constexpr (j + PFK < MS) rdk(std::integral_constant<int, j + PFK>{});
      lgkm_tie<wait_k(j, MS, PFK)>(kr[j]);
      if constexpr (j < 2) {
        sn[j & 1] = mfma16<E>(kr[j], qf[j >> 1], j ? seed1 : seed0);
        if constexpr (MASK && j == 0) seed1 = mask_seed((t + 1) & 1, 1);
      } else {
        sn[j & 1] = mfma16<E>(kr[j], qf[j >> 1], sn[j & 1]);
      }
#pragma unroll
      for (int g = 8 + j * 8 / MS; g < 8 + (j + 1) * 8 / MS; ++g) exp_pair(sc, g, pb, ls);
      fence();
    });
    PHASE(const unsigned c1 = PhaseClock::now(); fence();)
    if (t + 1 < nw && edge(t + 1)) mask_tile(sn, t + 1);
    float lt = lf + ls;
    if (__builtin_amdgcn_ballot_w64(!(lt <= kSumCap))) {
      lt = rebase(sc, pc);
      PHASE(++ph.rebases;)
    }
    l_run += lt;
    lf = 0.f;
    PHASE(fence(); const unsigned c2 = PhaseClock::now(); fence();)
    static_for<0, PFV>(rdv);
    fence();
    static_for<0, MP>([&](auto j_tag) {
      constexpr int j = decltype(j_tag)::value;
      constexpr int dt = j % (DV / 32), ks = j / (DV / 32);
      if constexpr (j + PFV < MP) rdv(std::integral_constant<int, j + PFV>{});
      lgkm_tie<wait_v(j, MP, PFV)>(vr[j][0], vr[j][1]);
      const bf16x8 a =
          __builtin_bit_cast(bf16x8, __builtin_shufflevector(vr[j][0], vr[j][1], 0, 1, 2, 3, 4, 5, 6, 7));
      const u32x4 pbk = ks < 2 ? pc[ks & 1] : pb[ks & 1];
      o[dt] = mfma16<E>(a, __builtin_bit_cast(bf16x8, pbk), o[dt]);
#pragma unroll
      for (int g = j * 8 / MP; g < (j + 1) * 8 / MP; ++g) exp_pair(sn, g, pn, lf);
      fence();
    });
    PHASE(const unsigned c3 = PhaseClock::now(); ph.cyc_a += c1 - c0; ph.cyc_check += c2 - c1;
          ph.cyc_b += c3 - c2; ++ph.tiles; fence();)
  };
  // A wavefront's last tile t: no S(t+1) and no exp2 of it; the exp2 of keys
  // 32-63 of S(t), the row-sum check and the PV(t) MFMAs as in tile().
  auto tile_last = [&](f32x16 (&sc)[2], u32x4 (&pc)[2], int vs_bytes) {
    s16x4 vr[MP][2];
    auto rdv = [&](auto j_tag) {
      constexpr int j = decltype(j_tag)::value;
      constexpr int dt = j % (DV / 32), ks = j / (DV / 32);
      ds_tr<2 * TB - VA0 + ks * 16 * D * 2>(vr[j][0], va[dt][0] + vs_bytes);
      ds_tr<2 * TB - VA0 + ks * 16 * D * 2>(vr[j][1], va[dt][1] + vs_bytes);
    };
    static_for<0, PFV>(rdv);
    fence();
    float ls = 0.f;
#pragma unroll
    for (int g = 8; g < 16; ++g) exp_pair(sc, g, pb, ls);
    float lt = lf + ls;
    if (__builtin_amdgcn_ballot_w64(!(lt <= kSumCap))) lt = rebase(sc, pc);
    l_run += lt;
    lf = 0.f;
    static_for<0, MP>([&](auto j_tag) {
      constexpr int j = decltype(j_tag)::value;
      constexpr int dt = j % (DV / 32), ks = j / (DV / 32);
      if constexpr (j + PFV < MP) rdv(std::integral_constant<int, j + PFV>{});
      lgkm_tie<wait_v(j, MP, PFV)>(vr[j][0], vr[j][1]);
      const bf16x8 a =
          __builtin_bit_cast(bf16x8, __builtin_shufflevector(vr[j][0], vr[j][1], 0, 1, 2, 3, 4, 5, 6, 7));
      const u32x4 pbk = ks < 2 ? pc[ks & 1] : pb[ks & 1];
      o[dt] = mfma16<E>(a, __builtin_bit_cast(bf16x8, pbk), o[dt]);
      fence();
    });
  };

  wait_dma();
  __syncthreads();
  PHASE(ph.rt_ready = PhaseClock::real();)
  if (nw > 0) {
    s_plain(s0);
    if (edge(0)) mask_tile(s0, 0);
    const float mx = row_max(s0);
    b_run = mx == -INFINITY ? 0.f : mx * sl2;
    nbase = -b_run;
#pragma unroll
    for (int g = 0; g < 8; ++g) exp_pair(s0, g, pf0, lf);
  }
  PHASE(fence(); ph.rt_loop = PhaseClock::real(); ph.c_loop = PhaseClock::now(); fence();)
  // Iteration t: K(t+1) in K stage (t+1)&1, V(t) in V stage t&1; loads K(t+2)
  // into K stage t&1 and V(t+1) into V stage (t+1)&1, whose previous tiles
  // every wavefront has finished reading at the barrier.
  // Every wavefront passes N barriers: tiles 0 .. nw-2 in the pipelined
  // loop, tile nw-1 by tile_last, then barrier-only iterations that keep
  // issuing the workgroup's loads.
  auto sync_load = [&](int t) {
    PHASE(const unsigned c0 = PhaseClock::now(); fence();)
    wait_dma();
    // Wavefront 0 publishes mask row t+1 with this barrier (its stage held
    // row t-1, last read before the previous barrier).
    if (MASK && wave == 0 && t + 1 < N) mask_store(mraw, (t + 1) & 1);
    PHASE(fence(); const unsigned cw = PhaseClock::now(); fence();)
    __syncthreads();
    if (MASK && wave == 0 && t + 2 < N) mraw = mask_raw(t + 2);
    PHASE(fence(); const unsigned cb = PhaseClock::now(); ph.cyc_vmwait += cw - c0; ph.cyc_barrier += cb - cw;
          fence();)
    if (t + 2 < N) kload.load(t + 2, (t & 1) ? kst[1] : kst[0], wave);
    PHASE(fence(); const unsigned ck = PhaseClock::now(); ph.cyc_dma_k += ck - cb; fence();)
    if (t + 1 < N) vload.load(t + 1, (t & 1) ? vst[0] : vst[1], wave);
    PHASE(fence(); ph.cyc_sync += PhaseClock::now() - c0;)
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  int last = -1;
  for (int t = 0; t < nw; t += 2) {
    if (t + 1 >= nw) {
      last = t;
      break;
    }
    sync_load(t);
    tile(s0, s1, pf0, pf1, t, I1{}, I0{});
    if (t + 2 >= nw) {
      last = t + 1;
      break;
    }
    sync_load(t + 1);
    tile(s1, s0, pf1, pf0, t + 1, I0{}, I1{});
  }
  int t = 0;
  if (last >= 0) {
    if (last & 1) {
      s0[0] = s1[0];
      s0[1] = s1[1];
      pf0[0] = pf1[0];
      pf0[1] = pf1[1];
    }
    sync_load(last);
    PHASE(const unsigned cl = PhaseClock::now(); fence();)
    tile_last(s0, pf0, (last & 1) * TB);
    PHASE(fence(); ph.cyc_last += PhaseClock::now() - cl;)
    t = last + 1;
  }
  for (; t < N; ++t) sync_load(t);

  PHASE(fence(); const unsigned c_epi = PhaseClock::now(); fence();)
  const float lt = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = 1.0f / lt;
  if (p.lse && half == 0 && qi < Tq) p.lse[(int64_t)bh * Tq + qi] = b_run + __log2f(lt);
  // Lane (l32, half) holds features dt*32 + g*8 + half*4 + e of row qi.
  // (Row addresses are formed from an opaque copy of the row index here, so
  // they are not hoisted into the tile loop, where more live registers
  // would spill.)
  int qo = qi;
  asm volatile("" : "+v"(qo));
  fence();
  {
    // Through LDS, so each store instruction writes whole rows: the K stages
    // are free (after the last barrier no wavefront reads them -- a last
    // tile reads V only, mask rows have an array of their own -- and no DMA
    // writes them), 32 rows x DV per wavefront.  16-byte chunk c of row r
    // sits at slot c ^ (r & SWZ), a permutation within each group of SWZ + 1
    // chunks (so 12-chunk rows, head size 96, stay inside the row), which
    // keeps the 8-byte writes and the row-contiguous 16-byte reads to a few
    // lanes per bank.  Output rows are 16-byte aligned (checked on the host).
    constexpr int CPR = DV / 8;    // 16-byte chunks per row: 4, 8, 12, 16
    constexpr int RPS = 64 / CPR;  // whole rows per store instruction
    constexpr int SWZ = CPR % 16 == 0 ? 15 : CPR % 8 == 0 ? 7 : 3;
    bf16* const st = smem + wave * 32 * DV;
    const int r0 = qo - q0;  // = l32
#pragma unroll
    for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = store_e<E>(o[dt][g * 4 + e] * inv);
        const int c = dt * 4 + g;
        *reinterpret_cast<u16x4*>(st + r0 * DV + (c ^ (r0 & SWZ)) * 8 + half * 4) = w;
      }
#pragma unroll
    for (int k = 0; k < (32 + RPS - 1) / RPS; ++k) {
      const int r = k * RPS + lane / CPR, c = lane % CPR;
      if (lane < RPS * CPR && r < 32) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(st + r * DV + (c ^ (r & SWZ)) * 8);
        // Whole lines, written once: streamed past the L2 (so the kernel's
        // end has no output lines to write back).
        if (q0 + r < Tq)
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(op + (int64_t)(q0 + r) * os2 + c * 8));
      }
    }
  }
  PHASE(fence(); ph.write(lane, id * kNW + wave, bh, mblk, N, nw, c_epi);)
}

template <int D, int DV, bool CAUSAL, int MT, int E>
int launch_t(const SdpaParams& p, hipStream_t s) {
  const int nmb = (p.Tq + kBM - 1) / kBM;
  const int64_t blocks = (int64_t)nmb * p.B * p.Hq;
  hipLaunchKernelGGL((flash_bf16_pipe_kernel<D, DV, CAUSAL, MT, E>), dim3((unsigned)blocks), dim3(kNT), 0, s, p);
  return launch_status("flash_bf16_pipe_kernel");
}

template <int D, int DV, int MT, int E>
int launch_c(const SdpaParams& p, hipStream_t s) {
  return p.causal ? launch_t<D, DV, true, MT, E>(p, s) : launch_t<D, DV, false, MT, E>(p, s);
}

template <int D, int DV, int E>
int launch_m(const SdpaParams& p, hipStream_t s) {
  if (!p.mask) return launch_c<D, DV, 0, E>(p, s);
#if defined(MFX_PHASE_TIMERS)
  // The diagnostic build instruments the mask-free kernels only.
  return fail(MFX_E_UNSUPPORTED, "phase-timer build: masked attention is not instrumented");
#else
  if (p.mask_dtype == MFX_F32) return launch_c<D, DV, 1, E>(p, s);
  if (p.mask_dtype == MFX_BF16) return launch_c<D, DV, 2, E>(p, s);
  return launch_c<D, DV, 3, E>(p, s);
#endif
}

#if defined(MFX_PIPE_WIDE)
// Head sizes 32 (64-wide tiles) and 96 (128-wide tiles).
template <int E>
int launch_d(const SdpaParams& p, hipStream_t s) {
  if (p.D == 32) return launch_m<64, 32, E>(p, s);
  return launch_m<128, 96, E>(p, s);
}
#else
template <int E>
int launch_d(const SdpaParams& p, hipStream_t s) {
  if (p.D == 128) return launch_m<128, 128, E>(p, s);
  if (p.D == 64) return launch_m<64, 64, E>(p, s);
  return launch_flash_bf16_pipe_wide(p, s);
}
#endif

}  // namespace

#if defined(MFX_PIPE_WIDE)
// Head sizes 32 and 96 of launch_flash_bf16_pipe (their kernels are
// instantiated in a translation unit of their own, so the two compile in
// parallel).
int launch_flash_bf16_pipe_wide(const SdpaParams& p, hipStream_t s) {
  return p.dtype == MFX_F16 ? launch_d<1>(p, s) : launch_d<0>(p, s);
}
#else
// Flash attention without an additive mask or with one that does not vary
// along query rows, p.ms[2] == 0 (the caller checked flash_bf16_supports);
// q, k, v and out all bf16 or all f16 (p.dtype); head size 32, 64, 96 or
// 128.
int launch_flash_bf16_pipe(const SdpaParams& p, hipStream_t s) {
  return p.dtype == MFX_F16 ? launch_d<1>(p, s) : launch_d<0>(p, s);
}
#endif

}  // namespace mfx

#if defined(MFX_PHASE_TIMERS)
// Diagnostic build only: copies up to max_records phase records (16 u64 each,
// fields as PhaseClock::write) to host memory after the device is idle and
// returns how many the device array holds; clear != 0 zeroes the array
// afterwards.  Not part of the product's C ABI.
extern "C" __attribute__((visibility("default"))) int64_t mfx_phase_timers_read(void* host, int64_t max_records,
                                                                                int clear) {
  if (hipDeviceSynchronize() != hipSuccess) return -1;
  void* dev = nullptr;
  if (hipGetSymbolAddress(&dev, HIP_SYMBOL(mfx::g_phase_records)) != hipSuccess) return -1;
  const int64_t n = max_records < mfx::kPhaseRecords ? max_records : mfx::kPhaseRecords;
  if (host && n > 0 &&
      hipMemcpy(host, dev, (size_t)n * mfx::kPhaseFields * 8, hipMemcpyDeviceToHost) != hipSuccess)
    return -1;
  if (clear && hipMemset(dev, 0, sizeof(mfx::g_phase_records)) != hipSuccess) return -1;
  if (hipDeviceSynchronize() != hipSuccess) return -1;
  return mfx::kPhaseRecords;
}
#endif
