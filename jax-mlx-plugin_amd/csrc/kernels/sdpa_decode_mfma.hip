// Split-KV attention for few query rows per kv head on the matrix cores
// (GQA / MQA decode, bf16).
//
// The R = (Hq/Hkv) * Tq query rows that share one kv head (R <= 32) are the
// columns of one 32-wide MFMA operand, so every K/V row is read from HBM once
// for all of them:
//   S^T = K Q^T   A = K tile rows (LDS), B = the R query rows (registers,
//                 zero-padded to 32 columns): v_mfma_f32_32x32x16_bf16.
//   O^T = V^T P^T A = transposing LDS reads of the V tile, B = P straight
//                 from the S^T accumulator (same key permutation), as in the
//                 prefill kernel.
// The padding wastes MFMA work that costs a few microseconds against the
// tens of microseconds the K/V bytes take: the kernel is HBM-bound.
//
// Work is balanced over the valid bytes, not over Tk.  A first kernel lists,
// per (batch, kv head), the 32-key tiles holding at least one visible key
// (additive mask not -inf for some row, key < Tk, causal limit).  The W
// wavefronts of the main kernel then split the concatenation of all lists
// into W equal contiguous ranges, so a batch with a long valid cache gets
// proportionally more wavefronts and every wavefront streams the same number
// of tiles.  A range may cross (batch, kv head) boundaries: each segment of
// it writes one partial (m, l, O) per row into slot (wavefront + bhk), which
// is unique because ranges are ordered, and the combine kernel merges the
// slots of the wavefronts whose range meets that bhk.
//
// K/V tiles stream through three swizzled LDS stages by asynchronous LDS-DMA
// loads; while one tile is computed, the next two are in flight.  The
// additive mask of a tile travels the same way: its values are gathered by
// LDS-DMA (one 4-byte slot per key and row, 16-bit types zero-extended) into
// the tail of the tile's V stage, so every load of the stream is an LDS-DMA
// whose completion the explicit vmcnt waits account for.  (Mask values
// loaded into registers instead make the compiler's wait insertion lose
// track of them across the rotating stages and drain the whole queue before
// each tile.)
//
// Optional fused RMSNorm of the query rows (reference chain rms_norm -> sdpa
// of GQA decode): q is normalised in fp32 and rounded to bf16 before it is
// used, exactly as the unfused graph rounds the RMSNorm output.
#include <type_traits>

#include "sdpa_elem.h"
#include "sdpa_tiles.h"

#if defined(MFX_PHASE_TIMERS)
#define PHASE(...) __VA_ARGS__
#else
#define PHASE(...)
#endif

namespace mfx {
namespace {

using tiles::kSlack;
using tiles::lds_void_t;
using tiles::s16x4;
using tiles::tile_swz;
using tiles::fence;

constexpr int kDN = 32;  // keys per tile: three stages = 48 KB of LDS per workgroup at d = 128
constexpr int kMT = kDN / 32;
constexpr int kKS = kDN / 16;
constexpr int kStages = 3;

// Mask slots (4 bytes each) per stage: the tile's keys once when the mask is
// the same for every query row of a kv head (MB), else once per row (up to
// 32 rows).  One LDS-DMA instruction fills 64 slots.
template <int MT, bool MB>
constexpr int mask_slots() { return MT == 0 ? 0 : (MB ? 64 : 32 * kDN); }

// LDS bytes of one workgroup of the main kernel.
template <int D, int MT, bool MB>
constexpr int stage_lds_bytes() { return kStages * (2 * kDN * D * 2 + 4 * mask_slots<MT, MB>()); }

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* ptr) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)ptr;
}

// s_waitcnt lgkmcnt(0) that the values read by inline-asm LDS loads depend
// on, so no use of them is scheduled before it.  The memory clobber keeps
// later writes to the stage (the next LDS-DMA into it) after the reads.
__device__ __forceinline__ void lgkm_wait_tied(bf16x8 (&a)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7])
               :
               : "memory");
}
__device__ __forceinline__ void lgkm_wait_tied(bf16x8 (&a)[4]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]) : : "memory");
}
__device__ __forceinline__ void lgkm_wait_tied(s16x4 (&v)[4][2][2]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(v[0][0][0]), "+v"(v[0][0][1]), "+v"(v[0][1][0]), "+v"(v[0][1][1]), "+v"(v[1][0][0]),
                 "+v"(v[1][0][1]), "+v"(v[1][1][0]), "+v"(v[1][1][1]), "+v"(v[2][0][0]), "+v"(v[2][0][1]),
                 "+v"(v[2][1][0]), "+v"(v[2][1][1]), "+v"(v[3][0][0]), "+v"(v[3][0][1]), "+v"(v[3][1][0]),
                 "+v"(v[3][1][1])
               :
               : "memory");
}
__device__ __forceinline__ void lgkm_wait_tied(s16x4 (&v)[2][2][2]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(v[0][0][0]), "+v"(v[0][0][1]), "+v"(v[0][1][0]), "+v"(v[0][1][1]), "+v"(v[1][0][0]),
                 "+v"(v[1][0][1]), "+v"(v[1][1][0]), "+v"(v[1][1][1])
               :
               : "memory");
}

// The same for other fragment counts (head sizes 32 and 96): the wait, then
// one tie per register, all volatile and so kept in this order.
template <int N>
__device__ __forceinline__ void lgkm_wait_tied_n(bf16x8 (&a)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(a[i]));
}
template <int N>
__device__ __forceinline__ void lgkm_wait_tied_n(s16x4 (&v)[N][2][2]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(v[i][j >> 1][j & 1]));
}
template <int N>
__device__ __forceinline__ void wait_frags(bf16x8 (&a)[N]) {
  if constexpr (N == 8 || N == 4) lgkm_wait_tied(a);
  else lgkm_wait_tied_n(a);
}
template <int N>
__device__ __forceinline__ void wait_frags(s16x4 (&v)[N][2][2]) {
  if constexpr (N == 4 || N == 2) lgkm_wait_tied(v);
  else lgkm_wait_tied_n(v);
}

// s_waitcnt vmcnt(N) with the other counters left alone (N < 64).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Lists, per (batch, kv head), the tiles holding a key some row can see.
// One workgroup per bhk.  Phase 1 reads the mask coalesced: thread t checks
// keys j*256 + t (j = 0, 1, ...), so the 32 keys of a tile sit in 32
// consecutive lanes and one ballot per load gives two tiles' flags, which go
// to LDS.  Phase 2 compacts the flagged tiles in tile order (one thread per
// tile, a ballot per wavefront and a prefix over the four wavefronts).  The
// mask is read per row of the group only when it varies over heads or query
// positions.
template <int MT, bool CAUSAL>
__global__ __launch_bounds__(256) void decode_tiles_kernel(SdpaParams p) {
  constexpr bool MASK = MT != 0;
  constexpr int kPass = 256;  // tiles flagged per pass (256 * 32 keys)
  __shared__ int flag[kPass];
  __shared__ int wave_n[4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int bhk = blockIdx.x;
  const int b = bhk / p.Hkv, hk = bhk % p.Hkv;
  const int Tq = p.Tq, R = p.group * Tq, Tk = p.Tk;
  const int kend = CAUSAL ? min(Tk, Tq) : Tk;  // keys past this are never visible
  const int ntile = (Tk + kDN - 1) / kDN;
  int* list = p.tile_list + (int64_t)bhk * p.tiles_cap;
  const bool bcast = !MASK || ((p.ms[1] == 0 || p.group == 1) && (p.ms[2] == 0 || Tq == 1));
  const int rows = bcast ? 1 : R;
  int n = 0;  // tiles listed so far (uniform)
  for (int t0 = 0; t0 < ntile; t0 += kPass) {
    // Phase 1: flags of tiles t0 .. t0 + kPass - 1.
    // All kB loads of a thread's keys are in flight together.
    constexpr int kB = kPass * kDN / 256;
    bool ok[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) ok[u] = t0 * kDN + u * 256 + tid < kend;
    if constexpr (MASK) {
      bool any[kB];
#pragma unroll
      for (int u = 0; u < kB; ++u) any[u] = false;
      for (int r = 0; r < rows; ++r) {
        const int h2 = hk * p.group + r / Tq, t2 = r % Tq;
        const int64_t mrow = b * p.ms[0] + (bcast ? 0 : h2 * p.ms[1] + t2 * p.ms[2]);
        float mvv[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) {
          const int key = min(t0 * kDN + u * 256 + tid, Tk - 1);
          mvv[u] = load_mask_t<MT>(p.mask, mrow + (int64_t)key * p.ms[3]);
        }
#pragma unroll
        for (int u = 0; u < kB; ++u) {
          const int key = t0 * kDN + u * 256 + tid;
          any[u] = any[u] | ((mvv[u] != -INFINITY) & (bcast | !CAUSAL | (key <= t2)));
        }
      }
#pragma unroll
      for (int u = 0; u < kB; ++u) ok[u] = ok[u] & any[u];
    }
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const uint64_t bal = __ballot(ok[u]);
      // lanes 0-31 / 32-63 of wavefront wv hold tile u*8 + wv*2 + 0 / 1
      if (lane == 0) {
        flag[u * 8 + wv * 2] = (bal & 0xffffffffull) != 0;
        flag[u * 8 + wv * 2 + 1] = (bal >> 32) != 0;
      }
    }
    __syncthreads();
    // Phase 2: compaction in tile order.
    const bool listed = t0 + tid < ntile && flag[tid];
    const uint64_t bal = __ballot(listed);
    if (lane == 0) wave_n[wv] = __popcll(bal);
    __syncthreads();
    int before = n;
    for (int i = 0; i < wv; ++i) before += wave_n[i];
    const int total = wave_n[0] + wave_n[1] + wave_n[2] + wave_n[3];
    if (listed) list[before + __popcll(bal & ((1ull << lane) - 1))] = t0 + tid;
    n += total;
    __syncthreads();
  }
  if (tid == 0) p.tile_count[bhk] = n;
}

// First element of wavefront w's range of the concatenated tile lists.
__device__ __forceinline__ int64_t range_start(int w, int64_t T, int W) { return (int64_t)w * T / W; }

// D: features per row of the LDS tiles (64 or 128); DV <= D: the head size
// (a multiple of 32).  Rows load D wide and only features below DV reach an
// MFMA, as in the pipelined prefill kernel.
#if defined(MFX_PHASE_TIMERS)
// Diagnostic build: one record of kDecPhaseFields u64 per decode wavefront
// (blockIdx.x): 0 ids (XCC id, HW_ID, wavefront), 1-5 realtime stamps (low
// words, 100 MHz) at its start, when its range is found, when the first
// segment's first tiles are issued, at its first tile, at the end of its last
// segment's tiles, 6 realtime end (64 bits), 7 tiles, 8 segments, 9 total
// cycles, 10 cycles in the tile loops.  The kernel's SGPRs are all taken, so
// the values wait in per-lane LDS words until the end; every stamp is taken
// where none of the kernel's inline-asm LDS reads is outstanding.
constexpr int kDecPhaseRecords = 1 << 15;
constexpr int kDecPhaseFields = 12;
__device__ unsigned long long g_dec_phase_records[kDecPhaseRecords * kDecPhaseFields];
enum DecPhaseSlot { kDpStart, kDpRange, kDpIssue, kDpFirst, kDpStreamEnd, kDpTiles, kDpSegs, kDpCStart, kDpCStream,
                    kDpCLoop, kDecPhaseSlots };
#endif

template <int D, int DV, int MT, bool MB, bool CAUSAL, int E>
__global__ __launch_bounds__(64) void decode_mfma_kernel(SdpaParams p) {
  static_assert(DV % 32 == 0 && DV <= D && D - DV < 64, "head size");
  constexpr bool MASK = MT != 0;
  using Loader = tiles::TileLoader<D, kDN, 1>;
  constexpr int kMS = mask_slots<MT, MB>();
  constexpr int kMI = kMS / 64;  // mask LDS-DMA instructions per tile
  // Each V stage is followed by the tile's mask slots (kMS 4-byte slots).
  constexpr int kVN = kDN * D + 2 * kMS;
  __shared__ __attribute__((aligned(16))) bf16 k0[kDN * D];
  __shared__ __attribute__((aligned(16))) bf16 v0[kVN];
  __shared__ __attribute__((aligned(16))) bf16 k1[kDN * D];
  __shared__ __attribute__((aligned(16))) bf16 v1[kVN];
  __shared__ __attribute__((aligned(16))) bf16 k2[kDN * D];
  __shared__ __attribute__((aligned(16))) bf16 v2[kVN];

  const int lane = threadIdx.x;
  const int half = lane >> 5, col = lane & 31;
  const int w = blockIdx.x, W = gridDim.x;
#if defined(MFX_PHASE_TIMERS)
  __shared__ unsigned dph[kDecPhaseSlots * 64];
  auto dslot = [&](int f) -> unsigned& { return dph[f * 64 + lane]; };
  auto dnow = []() { return (unsigned)__builtin_amdgcn_s_memtime(); };
  auto dreal = []() { return (unsigned)__builtin_amdgcn_s_memrealtime(); };
  for (int f = 0; f < kDecPhaseSlots; ++f) dslot(f) = 0;
  dslot(kDpStart) = dreal();
  dslot(kDpCStart) = dnow();
#endif
  const int BHk = p.B * p.Hkv;
  const int Tq = p.Tq, R = p.group * Tq, Tk = p.Tk;
  const float sl2 = p.scale_log2;  // > 0 (checked on the host)
  // Bytes the mask spans (strides >= 0 and the span < 2^31, checked on the
  // host): the extent of the mask gathers' buffer resource.
  [[maybe_unused]] const int mspan = MASK ? (int)(((int64_t)(p.B - 1) * p.ms[0] + (int64_t)(p.Hq - 1) * p.ms[1] +
                                  (int64_t)(p.Tq - 1) * p.ms[2] + (int64_t)(Tk - 1) * p.ms[3] + 1) *
                                 (MT == 1 ? 4 : 2))
                            : 0;

  // Total listed tiles and this wavefront's range [s, e) of them, then the
  // bhk holding element s and the first element P of its list.  Up to
  // 64 * kNC counts are held in registers (lane l of chunk c: bhk c*64 + l),
  // all loaded in one round trip; larger grids read them 64 per load.
  constexpr int kNC = 4;
  const bool in_regs = BHk <= 64 * kNC;
  int creg[kNC];
#pragma unroll
  for (int c = 0; c < kNC; ++c) creg[c] = in_regs && c * 64 + lane < BHk ? p.tile_count[c * 64 + lane] : 0;
  auto chunk = [&](int i0) __attribute__((always_inline)) {
    if (in_regs) {
      const int c = i0 >> 6;
      return c == 0 ? creg[0] : c == 1 ? creg[1] : c == 2 ? creg[2] : creg[3];
    }
    return i0 + lane < BHk ? p.tile_count[i0 + lane] : 0;
  };
  // Tile count of bhk i (uniform).
  auto count_of = [&](int i) __attribute__((always_inline)) {
    return in_regs ? __builtin_amdgcn_readlane(chunk(i & ~63), i & 63) : p.tile_count[i];
  };
  int64_t T = 0;
  for (int i0 = 0; i0 < BHk; i0 += 64) {
    int c = chunk(i0);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off, 64);
    T += __builtin_amdgcn_readfirstlane(c);
  }
  int64_t s = range_start(w, T, W);
  const int64_t e = range_start(w + 1, T, W);
  if (s >= e) return;
  // Inclusive prefix sums across lanes, then the first lane whose prefix
  // passes s.
  int bhk = 0;
  int64_t P = 0;
  for (int i0 = 0; i0 < BHk; i0 += 64) {
    const int c = chunk(i0);
    int incl = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off, 64);
      if (lane >= off) incl += t;
    }
    const uint64_t hit = __ballot(P + incl > s);
    if (hit) {
      const int l0 = __builtin_ctzll(hit);
      bhk = i0 + l0;
      P += __builtin_amdgcn_readlane(incl - c, l0);
      break;
    }
    P += __builtin_amdgcn_readlane(incl, 63);
  }
  PHASE(fence(); dslot(kDpRange) = dreal(); fence();)

  // Per-lane byte offsets of the operand reads within a tile (the same
  // patterns as the prefill kernel).
  uint32_t k_addr[DV / 16];
  uint32_t v_addr[DV / 32][2];
  {
    const int k_sw = tile_swz<D>(col);
#pragma unroll
    for (int kk = 0; kk < DV / 16; ++kk) k_addr[kk] = (uint32_t)((col * D + ((kk * 2 + half) ^ k_sw) * 8) * 2);
    const int tj = lane & 15, tg = (lane >> 4) & 1;
    const int v_row = 4 * half + (tj >> 2);
    const int v_sw = tile_swz<D>(v_row), v_sw8 = tile_swz<D>(v_row + 8);
    const int v_chunk = tg * 2 + ((tj & 3) >> 1);
    const int v_sub = (tj & 1) * 4;
#pragma unroll
    for (int dt = 0; dt < DV / 32; ++dt) {
      v_addr[dt][0] = (uint32_t)((v_row * D + v_sub + ((dt * 4 + v_chunk) ^ v_sw) * 8) * 2);
      v_addr[dt][1] = (uint32_t)(((v_row + 8) * D + v_sub + ((dt * 4 + v_chunk) ^ v_sw8) * 8) * 2);
    }
  }
  const bool qvalid = col < R;
  const int rr = qvalid ? col : 0;

  // One segment per (batch, kv head) the range meets.  At most BHk
  // iterations; every iteration advances s by at least one tile.
  for (int guard = 0; guard < BHk && s < e; ++guard) {
    const int cnt = count_of(bhk);
    const int64_t seg_end = e < P + cnt ? e : P + cnt;
    const int* lst = p.tile_list + (int64_t)bhk * p.tiles_cap + (s - P);
    const int ntl = (int)(seg_end - s);
    // The segment's tile indices live in VGPRs, entries [wb, wb + 64),
    // [wb + 64, wb + 128) and [wb + 128, wb + 192), read with readlane: no
    // memory round trip sits between a tile and the DMA of the tile two
    // places later.  When tile i leaves the first register the window moves
    // by 64, and the new third register is loaded 64 tiles before any entry
    // of it is read (its load only lengthens the vmcnt waits below).
    auto list_at = [&](int j) { return j < ntl ? lst[j] : 0; };
    int w0 = list_at(lane), w1 = list_at(64 + lane), w2 = list_at(128 + lane);
    int wb = 0;
    auto tile_at = [&](int i) __attribute__((always_inline)) {
      const int r = i - wb;
      return r < 64 ? __builtin_amdgcn_readlane(w0, r) : __builtin_amdgcn_readlane(w1, r - 64);
    };
    const int b = bhk / p.Hkv, hk = bhk % p.Hkv;
    const int hq = hk * p.group + rr / Tq, tq = rr % Tq;

    // This lane's query column and RMSNorm weight slice: loaded here and
    // used once the segment's first tiles are in flight, so their round trip
    // overlaps the tiles'.  Lane holds d = kk*16 + half*8 + e; lanes col and
    // col+32 hold one row.  (The weight is 16-byte aligned, checked on the
    // host.)
    const bool qnorm = p.q_rms_eps >= 0.f;
    const bf16* wq = static_cast<const bf16*>(p.q_rms_weight);
    bf16x8 qf[DV / 16], wf[DV / 16];
    {
      const bf16* qrow = static_cast<const bf16*>(p.q) + b * p.qs[0] + hq * p.qs[1] + tq * p.qs[2] + half * 8;
#pragma unroll
      for (int kk = 0; kk < DV / 16; ++kk) qf[kk] = *reinterpret_cast<const bf16x8*>(qrow + kk * 16);
      if (qnorm && wq) {
#pragma unroll
        for (int kk = 0; kk < DV / 16; ++kk) wf[kk] = *reinterpret_cast<const bf16x8*>(wq + kk * 16 + half * 8);
      }
    }
    // Mask element offset of the row each lane gathers in each mask
    // instruction: slot j*64 + lane holds key (lane & 31) of row 2j + half
    // (row 0 with MB; rows past R repeat row R - 1).  Offsets fit 31 bits
    // (checked on the host).
    [[maybe_unused]] constexpr int esz = MT == 1 ? 4 : 2;
    int mrow[kMI > 0 ? kMI : 1];
#pragma unroll
    for (int j = 0; j < kMI; ++j) {
      const int r = MB ? 0 : min(2 * j + half, R - 1);
      mrow[j] = (int)(b * p.ms[0] + (hk * p.group + r / Tq) * p.ms[1] + (r % Tq) * p.ms[2]);
    }

    const bf16* kp = static_cast<const bf16*>(p.k) + b * p.ks[0] + hk * p.ks[1];
    const bf16* vp = static_cast<const bf16*>(p.v) + b * p.vs[0] + hk * p.vs[1];
    const Loader kload(kp, p.ks[2], Tk, DV, 0, lane), vload(vp, p.vs[2], Tk, DV, 0, lane);

    f32x16 o[DV / 32];
#pragma unroll
    for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
    float b_run = -INFINITY, l_run = 0.f;

    // Mask gather of tile gt into the slots after V stage vd: instruction j
    // writes slots j*64 .. j*64+63.  Keys past Tk are clamped to the last
    // key (they are masked by the key < Tk test).  The resource spans the
    // mask's extent, so every gathered offset is range-checked.
    auto issue_mask = [&](int gt, bf16* vd) __attribute__((always_inline)) {
#if defined(__HIP_DEVICE_COMPILE__)
      if constexpr (MASK) {
        const int64_t key = min(gt * kDN + col, Tk - 1);
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.mask), (short)0,
                                                                             mspan, 0x00020000);
        char* md = reinterpret_cast<char*>(vd + kDN * D);
#pragma unroll
        for (int j = 0; j < kMI; ++j) {
          const uint32_t voff = (uint32_t)((mrow[j] + key * p.ms[3]) * esz);
          if constexpr (esz == 4)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(md + j * 256), 4, voff, 0, 0, 0);
          else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(md + j * 256), 2, voff, 0, 0, 0);
        }
      }
#endif
    };
    auto issue = [&](int gt, bf16* kd, bf16* vd) __attribute__((always_inline)) {
      kload.load(gt, kd, 0);
      vload.load(gt, vd, 0);
      issue_mask(gt, vd);
    };
    // Vector-memory operations one tile's loads add to the in-order count.
    constexpr int kOps = 2 * Loader::LOADS + kMI;
    // This lane's mask row in the slots (rows past R read row 0; their
    // columns are never stored).
    const int mslot = MB ? half * 4 : rr * kDN + half * 4;

    // Tile list entry i from stage (kc, vc) while entry i+2 (if any) is
    // issued into (kn, vn): three stages, two tiles in flight.  The
    // restrict-qualified stage pointers scope this tile's accesses, so the
    // compiler's LDS-DMA tracking does not make the operand reads wait for
    // the later tiles' loads.
    auto body = [&](int i, const bf16* __restrict__ kc, const bf16* __restrict__ vc, bf16* __restrict__ kn,
                    bf16* __restrict__ vn) __attribute__((always_inline)) {
      if (i - wb >= 64) {
        wb += 64;
        w0 = w1;
        w1 = w2;
        w2 = list_at(wb + 128 + lane);
      }
      const int kb = tile_at(i) * kDN;
      if (i + 2 < ntl) {
        issue(tile_at(i + 2), kn, vn);
        // The count field holds at most 63: waiting for one more operation
        // than the two later tiles' loads is still correct.
        wait_vm<(2 * kOps < 64 ? 2 * kOps : 63)>();
      } else if (i + 1 < ntl) {
        wait_vm<kOps>();
      } else {
        wait_vm<0>();
      }
      // Log2-domain mask values of this lane's 16 keys (S^T entry i holds
      // key (i >> 2) * 8 + half * 4 + (i & 3)).
      float mv[kMT][16];
      if constexpr (MASK) {
        const uint32_t* mc = reinterpret_cast<const uint32_t*>(vc + kDN * D) + mslot;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const u32x4 w4 = *reinterpret_cast<const u32x4*>(mc + g * 8);
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) {
            float f;
            if constexpr (MT == 1) f = __uint_as_float(w4[e2]);
            else if constexpr (MT == 2) f = __uint_as_float(w4[e2] << 16);
            else f = static_cast<float>(__builtin_bit_cast(_Float16, (uint16_t)w4[e2]));
            mv[0][g * 4 + e2] = mask_log2(f);
          }
        }
      }
      // K operand reads, all issued before one wait, as inline asm: the
      // vmcnt wait above already covers this stage's loads, and the
      // compiler's LDS-DMA tracking, which does not tell this stage from the
      // one just issued, would also wait for the later tile's K loads.
      f32x16 sc[kMT];
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt) {
        bf16x8 ka[DV / 16];
        const uint32_t kbase = lds_addr(kc) + mt * 32 * D * 2;
#pragma unroll
        for (int kk = 0; kk < DV / 16; ++kk)
          asm volatile("ds_read_b128 %0, %1" : "=v"(ka[kk]) : "v"(kbase + k_addr[kk]));
        wait_frags(ka);
#pragma unroll
        for (int i = 0; i < 16; ++i) sc[mt][i] = 0.f;
#pragma unroll
        for (int kk = 0; kk < DV / 16; ++kk)
          sc[mt] = mfma16<E>(ka[kk], qf[kk], sc[mt]);
      }
      // V^T operand reads (transposing), issued now so that their latency
      // overlaps the softmax; inline asm for the same reason as the K reads.
      static_assert(kKS == 2, "two 16-key halves per tile");
      s16x4 vr[DV / 32][kKS][2];
      {
        const uint32_t vbase = lds_addr(vc);
#pragma unroll
        for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(vr[dt][0][h]) : "v"(vbase + v_addr[dt][h]));
            asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                         : "=v"(vr[dt][1][h])
                         : "v"(vbase + v_addr[dt][h]), "i"(16 * D * 2));
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = kb + mt * 32 + (i >> 2) * 8 + half * 4 + (i & 3);
          float x = sc[mt][i] * sl2;
          if constexpr (MASK) x += mv[mt][i];
          if (key >= Tk || (CAUSAL && key > tq)) x = -INFINITY;
          sc[mt][i] = x;
          mx = fmaxf(mx, x);
        }
      {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
        mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      }
      const bool need = mx > b_run + kSlack;
      if (__ballot(need)) {
        const float nb = need ? mx : b_run;
        const float alpha = need ? __builtin_amdgcn_exp2f(b_run - nb) : 1.f;
        b_run = nb;
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
      }
      const float nbase = b_run == -INFINITY ? 0.f : -b_run;
      bf16x8 pb[kKS];
      if constexpr (E == 0) {
#pragma unroll
        for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            pb[mt * 2 + (i >> 3)][i & 7] = f32_elem<E>(__builtin_amdgcn_exp2f(sc[mt][i] + nbase));
        float l0 = 0.f, l1 = 0.f;
#pragma unroll
        for (int j = 0; j < kKS; ++j) {
          const bf16x8 wv = pb[j];
          l0 = dot2_at<E>(wv, 0, l0);
          l1 = dot2_at<E>(wv, 2, l1);
          l0 = dot2_at<E>(wv, 4, l0);
          l1 = dot2_at<E>(wv, 6, l1);
        }
        l_run += l0 + l1;
      } else {
        // f16: pairs packed into dwords first (per-element inserts and dot2
        // operands compile to wrong row sums for f16).
        u32x4 pw[kKS];
        float l0 = 0.f, l1 = 0.f;
#pragma unroll
        for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
          for (int i = 0; i < 16; i += 2) {
            const uint32_t w = pack2<E>(__builtin_amdgcn_exp2f(sc[mt][i] + nbase),
                                        __builtin_amdgcn_exp2f(sc[mt][i + 1] + nbase));
            pw[mt * 2 + (i >> 3)][(i & 7) >> 1] = w;
            if ((i & 2) == 0) l0 = dot2<E>(w, l0);
            else l1 = dot2<E>(w, l1);
          }
#pragma unroll
        for (int j = 0; j < kKS; ++j) pb[j] = __builtin_bit_cast(bf16x8, pw[j]);
        l_run += l0 + l1;
      }
      wait_frags(vr);
#pragma unroll
      for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
        for (int ks = 0; ks < kKS; ++ks) {
          const bf16x8 a =
              __builtin_bit_cast(bf16x8, __builtin_shufflevector(vr[dt][ks][0], vr[dt][ks][1], 0, 1, 2, 3, 4, 5, 6, 7));
          o[dt] = mfma16<E>(a, pb[ks], o[dt]);
        }
    };

    // The segment's tiles in list order, three per iteration (stages 0, 1,
    // 2).  The stages of the previous segment are idle: its last body waited
    // for every load and its reads precede this segment's first DMA in
    // program order.
    issue(tile_at(0), k0, v0);
    if (ntl > 1) issue(tile_at(1), k1, v1);
    PHASE(fence(); if (dslot(kDpSegs) == 0) dslot(kDpIssue) = dreal(); fence();)
    // Rows past R are zero (never stored); optional RMSNorm in fp32, rounded
    // to bf16 as the unfused graph rounds its output.
#pragma unroll
    for (int kk = 0; kk < DV / 16; ++kk)
      if (!qvalid) qf[kk] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
    if (qnorm && E == 0) {
      float ss = 0.f;
#pragma unroll
      for (int kk = 0; kk < DV / 16; ++kk)
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2) {
          const float x = static_cast<float>(qf[kk][e2]);
          ss += x * x;
        }
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
      ss = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
      const float inv = rsqrtf(ss / (float)DV + p.q_rms_eps);
#pragma unroll
      for (int kk = 0; kk < DV / 16; ++kk)
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2) {
          const float wv = wq ? static_cast<float>(wf[kk][e2]) : 1.f;
          qf[kk][e2] = static_cast<bf16>(static_cast<float>(qf[kk][e2]) * inv * wv);
        }
    } else if (qnorm) {
      // f16: whole fragments converted (see frag_f32_f16).
      float ss = 0.f;
#pragma unroll
      for (int kk = 0; kk < DV / 16; ++kk) {
        float x[8];
        frag_f32_f16(qf[kk], x);
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2) ss += x[e2] * x[e2];
      }
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
      ss = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
      const float inv = rsqrtf(ss / (float)DV + p.q_rms_eps);
#pragma unroll
      for (int kk = 0; kk < DV / 16; ++kk) {
        float x[8], w[8];
        frag_f32_f16(qf[kk], x);
        if (wq) frag_f32_f16(wf[kk], w);
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2) x[e2] = x[e2] * inv * (wq ? w[e2] : 1.f);
        qf[kk] = f32_frag_f16(x);
      }
    }
    PHASE(fence(); if (dslot(kDpSegs) == 0) dslot(kDpFirst) = dreal(); dslot(kDpCLoop) = dnow(); fence();)
    for (int i = 0; i < ntl; i += 3) {
      body(i, k0, v0, k2, v2);
      if (i + 1 >= ntl) break;
      body(i + 1, k1, v1, k0, v0);
      if (i + 2 >= ntl) break;
      body(i + 2, k2, v2, k1, v1);
    }
    PHASE(fence(); dslot(kDpStreamEnd) = dreal(); dslot(kDpCStream) += dnow() - dslot(kDpCLoop);
          dslot(kDpTiles) += (unsigned)ntl; dslot(kDpSegs) += 1u; fence();)

    // Lanes col and col+32 hold the two halves of each row's keys.
    float lt;
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
      lt = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    if (qvalid) {
      float* part = p.partial + ((int64_t)(w + bhk) * R + rr) * (DV + 2);
      if (half == 0) {
        part[0] = b_run;
        part[1] = lt;
      }
#pragma unroll
      for (int dt = 0; dt < DV / 32; ++dt)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq)
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) part[2 + dt * 32 + gq * 8 + half * 4 + e2] = o[dt][gq * 4 + e2];
    }
    s = seg_end;
    P += cnt;
    ++bhk;
    while (s < e && bhk < BHk && count_of(bhk) == 0) ++bhk;
  }
#if defined(MFX_PHASE_TIMERS)
  {
    fence();
    unsigned xcc, hwid;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hwid));
    const unsigned c_end = dnow();
    const unsigned long long rt_end = __builtin_amdgcn_s_memrealtime();
    if (lane == 0 && w < kDecPhaseRecords) {
      unsigned long long* r = g_dec_phase_records + (size_t)w * kDecPhaseFields;
      r[0] = (unsigned long long)(xcc & 0xff) | ((unsigned long long)hwid << 8) | ((unsigned long long)w << 40);
      r[1] = dslot(kDpStart);
      r[2] = dslot(kDpRange);
      r[3] = dslot(kDpIssue);
      r[4] = dslot(kDpFirst);
      r[5] = dslot(kDpStreamEnd);
      r[6] = rt_end;
      r[7] = dslot(kDpTiles);
      r[8] = dslot(kDpSegs);
      r[9] = c_end - dslot(kDpCStart);
      r[10] = dslot(kDpCStream);
    }
  }
#endif
}

// Merges the partial (m, l, O) rows of each output row: one wavefront per
// row.  The slots of bhk are w + bhk for the wavefronts w whose non-empty
// range meets bhk's list; lanes load the slots' (m, l) 64 at a time and
// reduce them, then every lane accumulates its features over the slots with
// sixteen slots' loads in flight (the first sixteen issued together with the
// (m, l) loads).  A row with no listed tile (every key masked) is NaN, as the
// unfused softmax.
template <typename OT, int D>
__global__ __launch_bounds__(256) void decode_bal_combine_kernel(SdpaParams p) {
  constexpr int NQ = (D + 63) / 64;  // features per lane (lane + 64 q < D)
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (b*Hq + h)*Tq + t
  const int64_t rows_total = (int64_t)p.B * p.Hq * p.Tq;
  if (row >= rows_total) return;
  const int tq = (int)(row % p.Tq);
  const int bh = (int)(row / p.Tq);
  const int b = bh / p.Hq, h = bh % p.Hq;
  const int hk = h / p.group;
  const int bhk = b * p.Hkv + hk;
  const int R = p.group * p.Tq;
  const int rr = (h % p.group) * p.Tq + tq;
  const int W = p.num_splits, BHk = p.B * p.Hkv;
  // T = all listed tiles, P = those of the bhks before this one, cnt =
  // this bhk's.  The counts are read 256 at a time: four loads per lane in
  // flight together.
  const int cnt = p.tile_count[bhk];
  int64_t T = 0, P = 0;
  for (int i0 = 0; i0 < BHk; i0 += 256) {
    int c[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * 64 + lane;
      c[u] = i < BHk ? p.tile_count[i] : 0;
    }
    int ct = 0, cp = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      ct += c[u];
      cp += i0 + u * 64 + lane < bhk ? c[u] : 0;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      ct += __shfl_xor(ct, off, 64);
      cp += __shfl_xor(cp, off, 64);
    }
    T += ct;
    P += cp;
  }
  OT* orow = static_cast<OT*>(p.out) + b * p.os[0] + h * p.os[1] + tq * p.os[2];
  if (cnt == 0) {
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      if ((D % 64 == 0 || lane + 64 * q < D)) orow[lane + 64 * q] = from_f32<OT>(__builtin_nanf(""));
    return;
  }
  // Wavefronts whose range [start(w), start(w+1)) meets [P, P + cnt).
  int lo = (int)(P * W / T);
  while (lo > 0 && range_start(lo, T, W) > P) --lo;
  while (range_start(lo + 1, T, W) <= P) ++lo;
  int hi = (int)((P + cnt - 1) * W / T);
  while (hi + 1 < W && range_start(hi + 1, T, W) < P + cnt) ++hi;
  while (range_start(hi, T, W) >= P + cnt) --hi;
  const int nslot = hi - lo + 1;
  auto slot_ptr = [&](int k) { return p.partial + ((int64_t)(lo + k + bhk) * R + rr) * (D + 2); };
  // The features of the first 16 slots, loaded before (and in flight with)
  // the slots' (m, l) below.
  float vf[16][NQ];
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const float* pk = slot_ptr(min(u, nslot - 1));
#pragma unroll
    for (int q = 0; q < NQ; ++q) vf[u][q] = (D % 64 == 0 || lane + 64 * q < D) ? pk[2 + lane + 64 * q] : 0.f;
  }
  // Lane k of a 64-slot chunk holds slot k0 + k: whether its wavefront's
  // range is non-empty (the next lane's start differs) and its (m, l).
  auto lane_slot = [&](int k0, float& mk, float& lk) {
    const int k = k0 + lane;
    const int64_t rs = range_start(lo + min(k, nslot), T, W);
    const int64_t rn = __shfl_down(rs, 1, 64);
    const int64_t re = lane == 63 ? range_start(lo + min(k + 1, nslot), T, W) : rn;
    mk = -INFINITY;
    lk = 0.f;
    if (k < nslot && rs < re) {
      const float2 ml = *reinterpret_cast<const float2*>(slot_ptr(k));
      mk = ml.x;
      lk = ml.y;
    }
  };
  // Row maximum and the rescaled l over all slots.
  float m = -INFINITY, l = 0.f, mk0 = -INFINITY;
  for (int k0 = 0; k0 < nslot; k0 += 64) {
    float mk, lk;
    lane_slot(k0, mk, lk);
    if (k0 == 0) mk0 = mk;
    const float mc = group_max<64>(mk);
    const float mn = fmaxf(m, mc);
    const float bn = mn == -INFINITY ? 0.f : mn;
    l = l * __builtin_amdgcn_exp2f(m - bn) + group_sum<64>(lk * __builtin_amdgcn_exp2f(mk - bn));
    m = mn;
  }
  const float base = m == -INFINITY ? 0.f : m;
  // O: each slot's features weighted by its uniform scale (read from the
  // lane that holds it).  A slot of weight 0 adds nothing; an empty range's
  // slot was never written, so its contents are not read into the sum
  // (0 * NaN).
  float acc[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) acc[q] = 0.f;
  auto accumulate = [&](const float (&v)[16][NQ], float sc, int j0, int n) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int su = j0 + u < n ? __builtin_amdgcn_readlane(__float_as_int(sc), j0 + u) : 0;
      const float scu = __int_as_float(su);
#pragma unroll
      for (int q = 0; q < NQ; ++q) acc[q] = scu != 0.f ? fmaf(v[u][q], scu, acc[q]) : acc[q];
    }
  };
  accumulate(vf, __builtin_amdgcn_exp2f(mk0 - base), 0, min(64, nslot));
  // Slots past the first 16, sixteen slots' loads in flight.
  for (int k0 = 0; k0 < nslot; k0 += 64) {
    float mk = mk0, lk;
    if (k0 > 0) lane_slot(k0, mk, lk);
    const float sc = __builtin_amdgcn_exp2f(mk - base);  // 0 for empty slots
    const int n = min(64, nslot - k0);
    for (int j0 = k0 == 0 ? 16 : 0; j0 < n; j0 += 16) {
      float v[16][NQ];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float* pk = slot_ptr(k0 + min(j0 + u, n - 1));
#pragma unroll
        for (int q = 0; q < NQ; ++q) v[u][q] = (D % 64 == 0 || lane + 64 * q < D) ? pk[2 + lane + 64 * q] : 0.f;
      }
      accumulate(v, sc, j0, n);
    }
  }
  const float inv = 1.0f / l;
#pragma unroll
  for (int q = 0; q < NQ; ++q)
    if ((D % 64 == 0 || lane + 64 * q < D)) orow[lane + 64 * q] = from_f32<OT>(acc[q] * inv);
}

// Whether every query row of a kv head sees the same mask row (the mask is
// broadcast over heads of a group and over query positions, or those have
// extent 1).
bool mask_rows_shared(const SdpaParams& p) {
  return (p.ms[1] == 0 || p.group == 1) && (p.ms[2] == 0 || p.Tq == 1);
}

template <int D, int DV, int MT, bool MB, bool CAUSAL, int E>
int launch_t(const SdpaParams& p, hipStream_t s) {
  hipLaunchKernelGGL((decode_tiles_kernel<MT, CAUSAL>), dim3((unsigned)(p.B * p.Hkv)), dim3(256), 0, s, p);
  int rc = launch_status("decode_tiles_kernel");
  if (rc != MFX_OK) return rc;
  hipLaunchKernelGGL((decode_mfma_kernel<D, DV, MT, MB, CAUSAL, E>), dim3((unsigned)p.num_splits), dim3(64), 0, s,
                     p);
  if ((rc = launch_status("decode_mfma_kernel")) != MFX_OK) return rc;
  const unsigned blocks = (unsigned)(((int64_t)p.B * p.Hq * p.Tq + 3) / 4);
  using OT = std::conditional_t<E == 0, bf16, _Float16>;
  hipLaunchKernelGGL((decode_bal_combine_kernel<OT, DV>), dim3(blocks), dim3(256), 0, s, p);
  return launch_status("decode_bal_combine_kernel");
}

template <int D, int DV, int MT, bool CAUSAL, int E>
int launch_m(const SdpaParams& p, hipStream_t s) {
  if constexpr (MT == 0) return launch_t<D, DV, 0, true, CAUSAL, E>(p, s);
  else
    return mask_rows_shared(p) ? launch_t<D, DV, MT, true, CAUSAL, E>(p, s)
                               : launch_t<D, DV, MT, false, CAUSAL, E>(p, s);
}

template <int D, int DV, bool CAUSAL, int E>
int launch_c(const SdpaParams& p, hipStream_t s) {
  switch (p.mask ? mask_code(p.mask_dtype) : 0) {
    case 1: return launch_m<D, DV, 1, CAUSAL, E>(p, s);
    case 2: return launch_m<D, DV, 2, CAUSAL, E>(p, s);
    case 3: return launch_m<D, DV, 3, CAUSAL, E>(p, s);
    default: return launch_m<D, DV, 0, CAUSAL, E>(p, s);
  }
}

template <int D, int DV, int E>
int launch_e(const SdpaParams& p, hipStream_t s) {
  return p.causal ? launch_c<D, DV, true, E>(p, s) : launch_c<D, DV, false, E>(p, s);
}

template <int D, int DV>
int launch_d(const SdpaParams& p, hipStream_t s) {
  return p.dtype == MFX_F16 ? launch_e<D, DV, 1>(p, s) : launch_e<D, DV, 0>(p, s);
}

template <int D>
int lds_bytes_d(const SdpaParams& p) {
  if (!p.mask) return stage_lds_bytes<D, 0, true>();
  return mask_rows_shared(p) ? stage_lds_bytes<D, 1, true>() : stage_lds_bytes<D, 1, false>();
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace

#if defined(MFX_DECODE_WIDE)
// Head sizes 32 (64-wide tiles) and 96 (128-wide tiles) of
// launch_decode_mfma, instantiated in a translation unit of their own.
int launch_decode_mfma_wide(const SdpaParams& p, hipStream_t s) {
  return p.D == 32 ? launch_d<64, 32>(p, s) : launch_d<128, 96>(p, s);
}
#else
bool decode_mfma_supports(const SdpaParams& p) {
  if (p.dtype != MFX_BF16 && p.dtype != MFX_F16) return false;
  if (!(p.scale_log2 > 0.f)) return false;
  if (p.D != p.Dv || (p.D != 32 && p.D != 64 && p.D != 96 && p.D != 128)) return false;
  if (p.group * p.Tq > 32) return false;
  if ((int64_t)p.B * p.Hkv * ((p.Tk + kDN - 1) / kDN) >= (1LL << 31)) return false;  // tile lists
  // Buffer-resource extents span Tk forward rows of at least D elements each.
  if (p.ks[2] < p.D || p.vs[2] < p.Dv) return false;
  if ((int64_t)p.Tk * p.ks[2] * 2 >= (1LL << 31) || (int64_t)p.Tk * p.vs[2] * 2 >= (1LL << 31)) return false;
  if (!aligned16(p.q) || !aligned16(p.k) || !aligned16(p.v)) return false;
  for (int i = 0; i < 3; ++i)
    if (p.qs[i] % 8 || p.ks[i] % 8 || p.vs[i] % 8) return false;
  if (p.q_rms_eps >= 0.f && p.q_rms_weight && !aligned16(p.q_rms_weight)) return false;
  if (p.mask) {
    // The mask is gathered through a buffer resource with 32-bit offsets.
    int64_t span = 1;
    const int64_t ext[4] = {p.B, p.Hq, p.Tq, p.Tk};
    for (int i = 0; i < 4; ++i) {
      if (p.ms[i] < 0) return false;
      span += (ext[i] - 1) * p.ms[i];
    }
    if (span * (p.mask_dtype == MFX_F32 ? 4 : 2) >= (1LL << 31)) return false;
  }
  return true;
}

int decode_mfma_tile() { return kDN; }

int decode_mfma_resident(const SdpaParams& p) {
  // Workgroups (one wavefront each) that fit the 160 KB of LDS of a CU, on
  // 256 CUs.
  const int lds = p.D > 64 ? lds_bytes_d<128>(p) : lds_bytes_d<64>(p);
  return 256 * (160 * 1024 / lds);
}

size_t decode_mfma_workspace(const SdpaParams& p, int W) {
  const int64_t bhk = (int64_t)p.B * p.Hkv;
  const int64_t cap = (p.Tk + kDN - 1) / kDN;
  const size_t lists = (size_t)(bhk * cap + bhk) * sizeof(int);
  const size_t parts = (size_t)(W + bhk) * p.group * p.Tq * (p.Dv + 2) * sizeof(float);
  return (lists + 255) / 256 * 256 + parts;
}

void decode_mfma_bind(SdpaParams& p, int W, void* ws) {
  const int64_t bhk = (int64_t)p.B * p.Hkv;
  const int64_t cap = (p.Tk + kDN - 1) / kDN;
  char* base = static_cast<char*>(ws);
  p.tile_list = reinterpret_cast<int*>(base);
  p.tile_count = p.tile_list + bhk * cap;
  p.tiles_cap = (int)cap;
  const size_t lists = (size_t)(bhk * cap + bhk) * sizeof(int);
  p.partial = reinterpret_cast<float*>(base + (lists + 255) / 256 * 256);
  p.num_splits = W;
}

int launch_decode_mfma(const SdpaParams& p, hipStream_t s) {
  if (p.D == 128) return launch_d<128, 128>(p, s);
  if (p.D == 64) return launch_d<64, 64>(p, s);
  return launch_decode_mfma_wide(p, s);
}
#endif

}  // namespace mfx

#if defined(MFX_PHASE_TIMERS) && !defined(MFX_DECODE_WIDE)
// Diagnostic build only: copies up to max_records decode phase records
// (kDecPhaseFields u64 each, fields as written at the end of
// decode_mfma_kernel) to host memory after the device is idle and returns how
// many the device array holds; clear != 0 zeroes the array afterwards.  Not
// part of the product's C ABI.
extern "C" __attribute__((visibility("default"))) int64_t mfx_decode_phase_timers_read(void* host,
                                                                                       int64_t max_records,
                                                                                       int clear) {
  if (hipDeviceSynchronize() != hipSuccess) return -1;
  void* dev = nullptr;
  if (hipGetSymbolAddress(&dev, HIP_SYMBOL(mfx::g_dec_phase_records)) != hipSuccess) return -1;
  const int64_t n = max_records < mfx::kDecPhaseRecords ? max_records : mfx::kDecPhaseRecords;
  if (host && n > 0 &&
      hipMemcpy(host, dev, (size_t)n * mfx::kDecPhaseFields * 8, hipMemcpyDeviceToHost) != hipSuccess)
    return -1;
  if (clear && hipMemset(dev, 0, sizeof(mfx::g_dec_phase_records)) != hipSuccess) return -1;
  if (hipDeviceSynchronize() != hipSuccess) return -1;
  return mfx::kDecPhaseRecords;
}
#endif
