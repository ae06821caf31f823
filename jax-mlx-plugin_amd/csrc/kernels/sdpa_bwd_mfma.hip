// Flash-attention backward on the matrix cores: bf16 or f16 inputs, head size
// 64 or 128 (D == Dv), fp32 accumulation, v_mfma_f32_32x32x16_bf16 (f16: the
// _f16 form) throughout.
//
// Two kernels, each owning its outputs (deterministic, no atomics):
//
// dkdv: workgroup = 4 wavefronts = 128 keys of one (batch, kv head); each
//   wavefront owns 32 keys.  Its K and V rows stay in registers as the B
//   operands; Q and dO stream through LDS in 64-query tiles (LDS-DMA, two
//   stages) over every query head of the kv head's group, with the rows'
//   lse / delta riding along as two 256-byte DMA rows.  Per 32-query block:
//     S  = Q K^T     A = Q tile rows        B = K (registers)
//     dP = dO V^T    A = dO tile rows       B = V (registers)
//   The 32x32 accumulators give lane l key (l % 32) and 16 query rows, so
//     P  = exp2(S * s * log2e - lse_q),  dS = P * (dP - delta_q)
//   are per-element lane work, and both feed the next products as B operands
//   straight from registers (contraction over queries, permuted identically
//   in A and B, as in the forward kernel's P V product):
//     dV^T += dO^T P   A = dO^T from the transposing LDS read
//     dK^T += Q^T dS   A = Q^T  from the transposing LDS read
//
// dq: workgroup = 4 wavefronts = 128 queries of one (batch, head), each
//   owning 32; Q and dO rows in registers, K and V stream in 64-key tiles as
//   in the forward kernel.  It runs first and also produces each row's
//   delta = rowsum(dO * O) for the dkdv kernel:
//     S^T = K Q^T, dP^T = V dO^T   (lane = query: lse / delta are scalars)
//     dQ^T += K^T dS^T             A = K^T from the transposing LDS read
//
// Tiles use the forward kernel's XOR swizzle, so every operand read is bank
// conflict free; causal tiles that see nothing are skipped, diagonal and
// ragged tiles mask per element.
//
// Built with -DMFX_PHASE_TIMERS (build.py phase_timers, a separate
// diagnostic library), every wavefront of the dK/dV kernel also records
// where its time goes: s_memrealtime stamps (100 MHz) at its start, at its
// loop entry and at its end, and s_memtime (shader clock) sums over its
// X phases (S / dP MFMAs), its Y | V phases (dV / dK MFMAs with the next
// block's exp2 / dS work), its barriers (vmcnt wait, s_barrier, the next
// tile's DMA issue) and its last Y, read where none of its inline-asm LDS
// reads is outstanding and summed in LDS (its SGPRs are all taken).  mfx_bwd_phase_timers_read() copies the records
// out; jax-mlx-plugin_amd/phase_budget.py --kernel dkdv turns them into the
// per-block budget.
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
// One record of kBwdPhaseFields u64 per dK/dV wavefront (blockIdx.x * 4 + wave).
constexpr int kBwdPhaseRecords = 1 << 15;
constexpr int kBwdPhaseFields = 16;
__device__ unsigned long long g_bwd_phase_records[kBwdPhaseRecords * kBwdPhaseFields];

// The kernel's SGPRs are all taken, so the running sums live in LDS: slot f
// of wavefront w is 64 words (one per lane, all equal), added to with
// ds_add_u32 at points where none of the kernel's inline-asm LDS reads is
// outstanding (an older LDS operation still in flight only makes their
// counted lgkmcnt waits stricter).
enum BwdPhaseSlot {
  kPhX, kPhYV, kPhSync, kPhVmwait, kPhBarrier, kPhLast, kPhBlocks, kPhEdges, kPhTiles,
  kPhRtStart, kPhCStart, kPhRtLoop, kPhCLoop, kPhCEpi, kBwdPhaseSlots
};
__device__ __forceinline__ unsigned ph_now() { return (unsigned)__builtin_amdgcn_s_memtime(); }
__device__ __forceinline__ unsigned ph_real() { return (unsigned)__builtin_amdgcn_s_memrealtime(); }
#endif

namespace {

constexpr int kNT = 256;  // 4 wavefronts
constexpr int kTile = 64;  // streamed rows per tile (queries in dkdv, keys in dq)
constexpr int kRows = 128;  // owned rows per workgroup (keys in dkdv, queries in dq)

using tiles::lds_s16x4_t;
using tiles::s16x4;
using tiles::tile_swz;
using tiles::wait_dma;
using tiles::ds_b128;
using tiles::ds_tr;
using tiles::lgkm_tie;
using tiles::fence;
using tiles::static_for;
template <int D>
using Loader = tiles::TileLoader<D, kTile, kNT / 64>;

// A operand of a 32 x 16 block of the transposed tile: rows d = dt*32 + l32
// of the tile's [rows x D] storage, k-slots = tile rows ks*16 + {4*half + e,
// 4*half + 8 + e} (e < 4), the order in which a 32x32 accumulator's 16 rows
// per lane pair are packed into the two k-steps of a B operand.
template <int D>
struct TrReader {
  int row, sw, sw8, chunk, sub;
  __device__ __forceinline__ TrReader(int lane) {
    const int half = lane >> 5, tj = lane & 15, tg = (lane >> 4) & 1;
    row = 4 * half + (tj >> 2);
    sw = tile_swz<D>(row);
    sw8 = tile_swz<D>(row + 8);
    chunk = tg * 2 + ((tj & 3) >> 1);
    sub = (tj & 1) * 4;
  }
  __device__ __forceinline__ bf16x8 read(const bf16* tile, int ks, int dt) const {
    const bf16* rows = tile + (ks * 16 + row) * D + sub;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(rows + ((dt * 4 + chunk) ^ sw) * 8));
    const s16x4 hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(rows + 8 * D + ((dt * 4 + chunk) ^ sw8) * 8));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};

// A operand of tile rows mt*32 + l32, feature chunk kk (16 features).
template <int D>
__device__ __forceinline__ bf16x8 row_frag(const bf16* tile, int mt, int kk, int l32, int half, int sw) {
  return *reinterpret_cast<const bf16x8*>(&tile[(mt * 32 + l32) * D + ((kk * 2 + half) ^ sw) * 8]);
}

// Row `r` (clamped into range, zero past `n`) as D/16 B-operand fragments:
// fragment kk holds features kk*16 + half*8 .. +7.
template <int D>
__device__ __forceinline__ void load_frags(const bf16* base, int64_t stride, int r, int n, int half, bf16x8* f) {
  const bf16* row = base + (int64_t)min(r, n - 1) * stride + half * 8;
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    u32x4 raw = *reinterpret_cast<const u32x4*>(row + kk * 16);
    if (r >= n) raw = u32x4{0u, 0u, 0u, 0u};
    f[kk] = __builtin_bit_cast(bf16x8, raw);
  }
}

// ----------------------------------------------------------------- dK, dV

// dK / dV run one wavefront per SIMD at d = 128 (the 32 keys' K and V
// operands and dK / dV accumulators alone take 192 registers), so the
// kernel overlaps its own vector and matrix work: per 32-query block i,
//   X(i):        S(i) and dP(i) MFMAs (Q / dO row fragments streamed ahead);
//   Y(i-1) | V(i): the dV and dK MFMAs of block i-1, with the exp2 / dS
//                work of block i (V) placed between them.
// Y(i-1) reads block i-1's Q / dO tile, which may be the previous tile, so
// tiles cycle through three LDS stages (one workgroup per CU has the LDS).
// Every block runs, also those a causal mask hides from this wavefront's
// keys: their P and dS are masked to zero, no branch breaks the pipeline,
// and the wavefront with the most visible blocks sets the pace anyway.
constexpr int kKvPf = 2;   // operand reads issued ahead of their MFMAs
constexpr int kKvStages = 3;
constexpr int kDkdvHeadGroup = 2;  // kv heads whose key blocks an XCD runs together

template <int D, bool CAUSAL, bool MASK, int E>
__global__ __launch_bounds__(kNT, 1) void bwd_dkdv_mfma(SdpaBwdParams p) {
  constexpr int TILE = kTile * D;    // elements of one Q or dO tile
  constexpr int TB = TILE * 2;       // its bytes
  constexpr int NK = D / 16;         // S (and dP) MFMAs per block
  constexpr int NT = 2 * (D / 32);   // dV (and dK) MFMAs per block
  constexpr int GB = kKvStages * TB;           // byte offset of the dO stages
  constexpr int LB = 2 * kKvStages * TB;       // byte offset of the lse / delta rows
  constexpr int LS = 2 * kTile * 4;            // their bytes per stage (lse | delta)
  __shared__ __attribute__((aligned(16))) char smem[LB + kKvStages * LS];
#if defined(MFX_PHASE_TIMERS)
  __shared__ unsigned ph_lds[4 * kBwdPhaseSlots * 64];
  const int ph_lane = threadIdx.x & 63, ph_wave = threadIdx.x >> 6;
  auto ph_slot = [&](int f) -> unsigned& { return ph_lds[(ph_wave * kBwdPhaseSlots + f) * 64 + ph_lane]; };
  auto ph_add = [&](int f, unsigned v) {
    __hip_atomic_fetch_add(&ph_slot(f), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  for (int f = 0; f < kBwdPhaseSlots; ++f) ph_slot(f) = 0;
  ph_slot(kPhRtStart) = ph_real();
  ph_slot(kPhCStart) = ph_now();
#endif

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;

  const int BHk = p.B * p.Hkv;
  const int nkb = (p.Tk + kRows - 1) / kRows;
  const int id = blockIdx.x;
  int bhk, kblk;
  if ((BHk & 7) == 0 && ((BHk >> 3) % kDkdvHeadGroup) == 0) {
    // Blocks are dealt to the 8 XCDs round-robin.  Each XCD takes its kv
    // heads in groups whose key blocks all run together (2 heads x 16 key
    // blocks fill an XCD's 32 CUs at config 3), so the group's Q / dO tiles,
    // which every key block of a head reads, stay in the XCD's L2.  Key
    // blocks in ascending order within a group: under a causal mask the
    // first key blocks see the most queries.
    const int hg = kDkdvHeadGroup, xcd = id & 7, slot = id >> 3;
    const int grp = slot / (hg * nkb), r = slot % (hg * nkb);
    bhk = (grp * hg + r % hg) * 8 + xcd;
    kblk = r / hg;
  } else {
    // Key blocks in ascending order, longest first.
    bhk = id % BHk;
    kblk = id / BHk;
  }
  const int b = bhk / p.Hkv, hk = bhk % p.Hkv;
  const int Tq = p.Tq, Tk = p.Tk, G = p.group;
  const int kw = kblk * kRows + wave * 32;  // this wave's first key
  const int key = kw + l32;

  const bf16* kp = static_cast<const bf16*>(p.k) + b * p.ks[0] + hk * p.ks[1];
  const bf16* vp = static_cast<const bf16*>(p.v) + b * p.vs[0] + hk * p.vs[1];
  // Query heads hk*G .. hk*G + G-1 share one resource; tile (g, qt) starts
  // g * qs[1] + qt * 64 * qs[2] elements past the group's first head.
  const bf16* qp = static_cast<const bf16*>(p.q) + b * p.qs[0] + (int64_t)hk * G * p.qs[1];
  const bf16* gp = static_cast<const bf16*>(p.dout) + b * p.dos[0] + (int64_t)hk * G * p.dos[1];
  const int64_t rbase = ((int64_t)b * p.Hq + (int64_t)hk * G) * Tq;  // lse / delta row of (g=0, q=0)
  const float* lsep = p.lse + rbase;
  const float* dlp = p.delta + rbase;
  const int st_bytes = G * Tq * 4;

  const int qt0 = CAUSAL ? (kblk * kRows) / kTile : 0;
  const int nqt = (Tq + kTile - 1) / kTile;
  const int per_head = nqt > qt0 ? nqt - qt0 : 0;
  const int ntiles = G * per_head;

  // Resource extents end with the last element of the group's last row, so
  // rows past Tq read zeros or (inside the span) rows of the next head,
  // which are masked.
  Loader<D> qload(qp, p.qs[2], 0, D, wave, lane), gload(gp, p.dos[2], 0, D, wave, lane);
  qload.nbytes = (int)(((int64_t)(G - 1) * p.qs[1] + (int64_t)(Tq - 1) * p.qs[2] + D) * 2);
  gload.nbytes = (int)(((int64_t)(G - 1) * p.dos[1] + (int64_t)(Tq - 1) * p.dos[2] + D) * 2);
  auto tile_head = [&](int t) { return t / per_head; };
  auto tile_q = [&](int t) { return qt0 + t % per_head; };
  auto issue = [&](int t, int st) {
    const int g = tile_head(t), qt = tile_q(t);
    qload.load_at((uint32_t)(((int64_t)g * p.qs[1] + (int64_t)qt * kTile * p.qs[2]) * 2),
                  reinterpret_cast<bf16*>(smem + st * TB), wave);
    gload.load_at((uint32_t)(((int64_t)g * p.dos[1] + (int64_t)qt * kTile * p.dos[2]) * 2),
                  reinterpret_cast<bf16*>(smem + GB + st * TB), wave);
    const uint32_t soff = (uint32_t)(((int64_t)g * Tq + (int64_t)qt * kTile) * 4);
    float* sl = reinterpret_cast<float*>(smem + LB + st * LS);
    if (wave == 0) tiles::load_row64_f32(lsep, st_bytes, soff, sl, lane);
    if (wave == 1) tiles::load_row64_f32(dlp, st_bytes, soff, sl + kTile, lane);
  };
  if (ntiles > 0) issue(0, 0);

  bf16x8 kf[D / 16], vf[D / 16];
  load_frags<D>(kp, p.ks[2], key, Tk, half, kf);
  load_frags<D>(vp, p.vs[2], key, Tk, half, vf);

  f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) dk[dt][i] = dv[dt][i] = 0.f;

  const float sl2 = p.scale_log2;
  // LDS byte addresses of the operand reads (stage, 32-query block and
  // 16-query step are immediate offsets).
  const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)smem;
  uint32_t ra[D / 16], rg[D / 16];  // row l32 of a 32-query block, feature chunk kk (Q | dO)
  {
    const int rsw = tile_swz<D>(l32);
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      ra[kk] = base + (uint32_t)((l32 * D + ((kk * 2 + half) ^ rsw) * 8) * 2);
      rg[kk] = ra[kk] + GB;
    }
  }
  uint32_t ta[D / 32][2], tg[D / 32][2];  // transposing reads (the order of TrReader), Q | dO
  {
    const int tj = lane & 15, tgi = (lane >> 4) & 1;
    const int r = 4 * half + (tj >> 2);
    const int sw = tile_swz<D>(r), sw8 = tile_swz<D>(r + 8);
    const int chunk = tgi * 2 + ((tj & 3) >> 1), sub = (tj & 1) * 4;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      ta[dt][0] = base + (uint32_t)((r * D + sub + ((dt * 4 + chunk) ^ sw) * 8) * 2);
      ta[dt][1] = base + (uint32_t)(((r + 8) * D + sub + ((dt * 4 + chunk) ^ sw8) * 8) * 2);
      tg[dt][0] = ta[dt][0] + GB;
      tg[dt][1] = ta[dt][1] + GB;
    }
  }
  const uint32_t la = base + LB + half * 16;  // lse | delta of rows 4*half ..

  f32x16 s, dp;         // S and dP of the block in flight
  u32x4 pd[2][2][2];    // [block parity][P | dS][16-query step]: bf16 pairs

  // X: S = Q K^T and dP = dO V^T of block (ST, MT), MFMAs alternating.
  auto X = [&](auto st_tag, auto mt_tag) __attribute__((always_inline)) {
    constexpr int ST = decltype(st_tag)::value, MT = decltype(mt_tag)::value;
    constexpr int O = ST * TB + MT * 32 * D * 2;
    bf16x8 qr[NK], gr[NK];
    auto rd = [&](auto j_tag) {
      constexpr int j = decltype(j_tag)::value;
      ds_b128<O>(qr[j], ra[j]);
      ds_b128<O>(gr[j], rg[j]);
    };
    static_for<0, kKvPf>(rd);
    fence();
    static_for<0, NK>([&](auto j_tag) {
      constexpr int j = decltype(j_tag)::value;
      if constexpr (j + kKvPf < NK) rd(std::integral_constant<int, j + kKvPf>{});
      constexpr int ahead = 2 * (kKvPf < NK - 1 - j ? kKvPf : NK - 1 - j);
      lgkm_tie<ahead + 1>(qr[j]);
      if constexpr (j == 0)
        s = mfma16<E>(qr[j], kf[j], f32x16{});
      else
        s = mfma16<E>(qr[j], kf[j], s);
      lgkm_tie<ahead>(gr[j]);
      if constexpr (j == 0)
        dp = mfma16<E>(gr[j], vf[j], f32x16{});
      else
        dp = mfma16<E>(gr[j], vf[j], dp);
      fence();
    });
  };

  // Y | V: dV^T += dO^T P and dK^T += Q^T dS of block (PS, PM) (P and dS in
  // pd[PM]), with (VAL) the P / dS of block (ST, MT) -- from s and dp -- into
  // pd[MT] between the MFMAs.  q0b: the block's first query; g: its head.
  auto YV = [&](auto ps_tag, auto pm_tag, auto st_tag, auto mt_tag, auto edge_tag, auto val_tag, int q0b, int g)
      __attribute__((always_inline)) {
    constexpr int PS = decltype(ps_tag)::value, PM = decltype(pm_tag)::value;
    constexpr int ST = decltype(st_tag)::value, MT = decltype(mt_tag)::value;
    constexpr bool EDGE = decltype(edge_tag)::value, VAL = decltype(val_tag)::value;
    // lse | delta of this lane's 16 rows of block (ST, MT): rows r*8 + 4*half + e.
    f32x4 lq[4], dq4[4];
    if constexpr (VAL) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(lq[r]) : "v"(la), "i"(ST * LS + (MT * 32 + r * 8) * 4));
        asm volatile("ds_read_b128 %0, %1 offset:%2"
                     : "=v"(dq4[r])
                     : "v"(la), "i"(ST * LS + kTile * 4 + (MT * 32 + r * 8) * 4));
      }
    }
    // MFMA j: dV for j even, dK for j odd; d-block (j/2) % (D/32), step (j/2) / (D/32).
    s16x4 tr[2 * NT][2];
    auto rdt = [&](auto j_tag) {
      constexpr int j = decltype(j_tag)::value;
      constexpr int m = j >> 1, dt = m % (D / 32), ks = m / (D / 32);
      constexpr int O = PS * TB + (PM * 2 + ks) * 16 * D * 2;
      if constexpr ((j & 1) == 0) {
        ds_tr<O>(tr[j][0], tg[dt][0]);
        ds_tr<O>(tr[j][1], tg[dt][1]);
      } else {
        ds_tr<O>(tr[j][0], ta[dt][0]);
        ds_tr<O>(tr[j][1], ta[dt][1]);
      }
    };
    static_for<0, kKvPf>(rdt);
    fence();
    static_for<0, 2 * NT>([&](auto j_tag) {
      constexpr int j = decltype(j_tag)::value;
      constexpr int m = j >> 1, dt = m % (D / 32), ks = m / (D / 32);
      if constexpr (j + kKvPf < 2 * NT) rdt(std::integral_constant<int, j + kKvPf>{});
      lgkm_tie<2 * (kKvPf < 2 * NT - 1 - j ? kKvPf : 2 * NT - 1 - j)>(tr[j][0], tr[j][1]);
      if constexpr (VAL && j == 0) {
        // The lse / delta reads were issued before every operand read: the
        // wait above covered them.
        asm volatile("" : "+v"(lq[0]), "+v"(lq[1]), "+v"(lq[2]), "+v"(lq[3]));
        asm volatile("" : "+v"(dq4[0]), "+v"(dq4[1]), "+v"(dq4[2]), "+v"(dq4[3]));
      }
      const bf16x8 a =
          __builtin_bit_cast(bf16x8, __builtin_shufflevector(tr[j][0], tr[j][1], 0, 1, 2, 3, 4, 5, 6, 7));
      if constexpr ((j & 1) == 0)
        dv[dt] = mfma16<E>(a, __builtin_bit_cast(bf16x8, pd[PM][0][ks]), dv[dt]);
      else
        dk[dt] = mfma16<E>(a, __builtin_bit_cast(bf16x8, pd[PM][1][ks]), dk[dt]);
      if constexpr (VAL) {
        // Entry pairs (2k, 2k+1) of block (ST, MT), 8 over the 2*NT MFMAs.
#pragma unroll
        for (int k = j * 8 / (2 * NT); k < (j + 1) * 8 / (2 * NT); ++k) {
          float sv[2] = {s[2 * k], s[2 * k + 1]}, dv2[2] = {dp[2 * k], dp[2 * k + 1]};
          // Inputs taken here, so the work stays in this MFMA's slot.
          asm volatile("" : "+v"(sv[0]), "+v"(sv[1]), "+v"(dv2[0]), "+v"(dv2[1]));
          float pr[2], ds[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int i = 2 * k + u, r = i >> 2, e = i & 3;
            const int q = q0b + r * 8 + half * 4 + e;
            float x = fmaf(sv[u], sl2, -lq[r][e]);
            if constexpr (MASK) {
              if (q < Tq && key < Tk)
                x += mask_log2(load_mask(p.mask, p.mask_dtype,
                                        b * p.ms[0] + (int64_t)(hk * G + g) * p.ms[1] + (int64_t)q * p.ms[2] +
                                            (int64_t)key * p.ms[3]));
            }
            pr[u] = __builtin_amdgcn_exp2f(x);
            if constexpr (EDGE) {
              if (q >= Tq || (CAUSAL && key > q)) pr[u] = 0.f;
            }
            ds[u] = pr[u] * (dv2[u] - dq4[r][e]);
          }
          const uint32_t up = pack2<E>(pr[0], pr[1]), ud = pack2<E>(ds[0], ds[1]);
          asm volatile("" ::"v"(up), "v"(ud));
          pd[MT][0][k >> 2][k & 3] = up;
          pd[MT][1][k >> 2][k & 3] = ud;
        }
      }
      fence();
    });
  };

  // Block (ST, MT) of tile t after block (PS, PM): X, then Y | V.
  auto step = [&](int t, auto ps_tag, auto pm_tag, auto st_tag, auto mt_tag) __attribute__((always_inline)) {
    constexpr int MT = decltype(mt_tag)::value;
    const int g = tile_head(t), q0b = tile_q(t) * kTile + MT * 32;
    PHASE(fence(); const unsigned c0 = ph_now(); fence();)
    X(st_tag, mt_tag);
    PHASE(fence(); const unsigned c1 = ph_now(); fence();)
    const bool edge = (q0b + 32 > Tq) || (CAUSAL && q0b < kw + 31);
    if (edge)
      YV(ps_tag, pm_tag, st_tag, mt_tag, std::true_type{}, std::true_type{}, q0b, g);
    else
      YV(ps_tag, pm_tag, st_tag, mt_tag, std::false_type{}, std::true_type{}, q0b, g);
    PHASE(fence(); const unsigned c2 = ph_now(); ph_add(kPhX, c1 - c0); ph_add(kPhYV, c2 - c1);
          ph_add(kPhBlocks, 1u); ph_add(kPhEdges, edge ? 1u : 0u); fence();)
  };
  // Tile t in stage ST, the previous tile in stage PS.
  auto tile = [&](int t, auto st_tag, auto ps_tag) __attribute__((always_inline)) {
    constexpr int ST = decltype(st_tag)::value;
    PHASE(fence(); const unsigned c0 = ph_now(); fence();)
    wait_dma();
    PHASE(fence(); const unsigned cw = ph_now(); fence();)
    __syncthreads();
    PHASE(fence(); const unsigned cb = ph_now(); fence();)
    // Stage (ST+1) % 3 last held tile t-2, whose last block's Y ran during
    // tile t-1, before this barrier.
    if (t + 1 < ntiles) issue(t + 1, (ST + 1) % kKvStages);
    PHASE(fence(); const unsigned ci = ph_now(); ph_add(kPhSync, ci - c0); ph_add(kPhVmwait, cw - c0);
          ph_add(kPhBarrier, cb - cw); ph_add(kPhTiles, 1u); fence();)
    step(t, ps_tag, std::integral_constant<int, 1>{}, st_tag, std::integral_constant<int, 0>{});
    step(t, st_tag, std::integral_constant<int, 0>{}, st_tag, std::integral_constant<int, 1>{});
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;

  PHASE(fence(); ph_slot(kPhRtLoop) = ph_real(); ph_slot(kPhCLoop) = ph_now(); fence();)
  if (ntiles > 0) {
    // The first block's Y is a no-op: zero P / dS against tile 0's rows.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int k = 0; k < 2; ++k) pd[1][i][k] = u32x4{0u, 0u, 0u, 0u};
    tile(0, I0{}, I0{});
    for (int t = 1;; t += 3) {
      if (t >= ntiles) break;
      tile(t, I1{}, I0{});
      if (t + 1 >= ntiles) break;
      tile(t + 1, I2{}, I1{});
      if (t + 2 >= ntiles) break;
      tile(t + 2, I0{}, I2{});
    }
    // The last block's Y.
    PHASE(fence(); const unsigned cl = ph_now(); fence();)
    const int ls = (ntiles - 1) % kKvStages;
    if (ls == 0)
      YV(I0{}, I1{}, I0{}, I0{}, std::false_type{}, std::false_type{}, 0, 0);
    else if (ls == 1)
      YV(I1{}, I1{}, I0{}, I0{}, std::false_type{}, std::false_type{}, 0, 0);
    else
      YV(I2{}, I1{}, I0{}, I0{}, std::false_type{}, std::false_type{}, 0, 0);
    PHASE(fence(); ph_add(kPhLast, ph_now() - cl); fence();)
  }

  PHASE(fence(); ph_slot(kPhCEpi) = ph_now(); fence();)
  // Every wavefront's last Y has read its Q / dO stage: the stages take the
  // dK and dV rows on their way out.  (The first key comes from an opaque
  // copy here, so no address is hoisted into the loop.)
  __syncthreads();
  {
    int k0 = kw;
    asm volatile("" : "+v"(k0));
    const int nvalid = min(max(Tk - k0, 0), 32);
    bf16* const st = reinterpret_cast<bf16*>(smem) + wave * 2 * 32 * D;
    store_rows_lds<D, E>(st, static_cast<bf16*>(p.dk) + b * p.dks[0] + hk * p.dks[1] + (int64_t)k0 * p.dks[2],
                         p.dks[2], nvalid, dk, l32, half, lane, p.scale);
    store_rows_lds<D, E>(st + 32 * D,
                         static_cast<bf16*>(p.dv) + b * p.dvs[0] + hk * p.dvs[1] + (int64_t)k0 * p.dvs[2],
                         p.dvs[2], nvalid, dv, l32, half, lane, 1.f);
  }
#if defined(MFX_PHASE_TIMERS)
  {
    // Fields: 0 ids (XCC id, HW_ID, (batch*Hkv + kv head), key block), 1 / 2
    // realtime start / loop entry (low words), 3 realtime end (64 bits), 4-9
    // cycles of the X phases / Y | V phases / barrier phases (all) / their
    // vmcnt waits / their s_barrier / the last Y, 10 blocks, 11 blocks with
    // per-element masking, 12 total cycles, 13 cycles before the loop, 14
    // cycles of the epilogue, 15 tiles.
    fence();
    unsigned xcc, hwid;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hwid));
    const unsigned c_end = ph_now();
    const unsigned long long rt_end = __builtin_amdgcn_s_memrealtime();
    const int rec = id * 4 + wave;
    if (lane == 0 && rec < kBwdPhaseRecords) {
      unsigned long long* r = g_bwd_phase_records + (size_t)rec * kBwdPhaseFields;
      r[0] = (unsigned long long)(xcc & 0xff) | ((unsigned long long)hwid << 8) | ((unsigned long long)bhk << 40) |
             ((unsigned long long)(kblk & 0xff) << 56);
      r[1] = ph_slot(kPhRtStart);
      r[2] = ph_slot(kPhRtLoop);
      r[3] = rt_end;
      r[4] = ph_slot(kPhX);
      r[5] = ph_slot(kPhYV);
      r[6] = ph_slot(kPhSync);
      r[7] = ph_slot(kPhVmwait);
      r[8] = ph_slot(kPhBarrier);
      r[9] = ph_slot(kPhLast);
      r[10] = ph_slot(kPhBlocks);
      r[11] = ph_slot(kPhEdges);
      r[12] = c_end - ph_slot(kPhCStart);
      r[13] = ph_slot(kPhCLoop) - ph_slot(kPhCStart);
      r[14] = c_end - ph_slot(kPhCEpi);
      r[15] = ph_slot(kPhTiles);
    }
  }
#endif
}

// ----------------------------------------------------------------------- dQ

// Operand reads issued ahead of their MFMAs in the dQ kernel (K / V row
// fragment pairs, transposed K fragment pairs).
constexpr int kDqPf = 2;

template <int D, bool CAUSAL, bool MASK, int E>
__global__ __launch_bounds__(kNT, 2) void bwd_dq_mfma(SdpaBwdParams p) {
  constexpr int TILE = kTile * D;  // elements of one K or V tile
  constexpr int TB = TILE * 2;     // its bytes
  constexpr int NK = D / 16;       // S (and dP) MFMAs per 32-key block
  constexpr int NT = 2 * (D / 32);  // dQ MFMAs per 32-key block
  __shared__ __attribute__((aligned(16))) bf16 smem[4 * TILE];  // K0 V0 K1 V1

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;

  const int nmb = (p.Tq + kRows - 1) / kRows;
  const int BH = p.B * p.Hq;
  const int id = blockIdx.x;
  int bh, mblk;
  if ((BH & 7) == 0) {
    // Heads dealt to the 8 XCDs round-robin, longest causal q-block first.
    const int xcd = id & 7, slot = id >> 3, bpx = BH >> 3;
    bh = (slot % bpx) * 8 + xcd;
    mblk = nmb - 1 - slot / bpx;
  } else {
    bh = id % BH;
    mblk = nmb - 1 - id / BH;
  }
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h / p.group;
  const int Tq = p.Tq, Tk = p.Tk;
  const int q0 = mblk * kRows + wave * 32;
  const int qi = q0 + l32;

  const bf16* kp = static_cast<const bf16*>(p.k) + b * p.ks[0] + hk * p.ks[1];
  const bf16* vp = static_cast<const bf16*>(p.v) + b * p.vs[0] + hk * p.vs[1];
  int kv_end = Tk;
  if (CAUSAL) kv_end = min(Tk, min(Tq, (mblk + 1) * kRows));
  const int ntiles = (kv_end + kTile - 1) / kTile;
  const Loader<D> kload(kp, p.ks[2], Tk, D, wave, lane), vload(vp, p.vs[2], Tk, D, wave, lane);
  auto issue = [&](int t, int st) {
    kload.load(t, smem + (2 * st) * TILE, wave);
    vload.load(t, smem + (2 * st + 1) * TILE, wave);
  };
  if (ntiles > 0) issue(0, 0);

  bf16x8 qf[D / 16], gf[D / 16];
  load_frags<D>(static_cast<const bf16*>(p.q) + b * p.qs[0] + h * p.qs[1], p.qs[2], qi, Tq, half, qf);
  load_frags<D>(static_cast<const bf16*>(p.dout) + b * p.dos[0] + h * p.dos[1], p.dos[2], qi, Tq, half, gf);
  const int64_t row = (int64_t)bh * Tq + min(qi, Tq - 1);
  const float lse = p.lse[row];
  // delta = rowsum(dO * O): this lane's 64 features, then its partner's.
  float dl;
  {
    bf16x8 of[D / 16];
    load_frags<D>(static_cast<const bf16*>(p.o) + b * p.os[0] + h * p.os[1], p.os[2], qi, Tq, half, of);
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      if constexpr (E == 0) {
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          a0 = fmaf(elem_f32<E>(gf[kk][e]), elem_f32<E>(of[kk][e]), a0);
          a1 = fmaf(elem_f32<E>(gf[kk][e + 1]), elem_f32<E>(of[kk][e + 1]), a1);
        }
      } else {
        float gv[8], ov[8];
        frag_f32_f16(gf[kk], gv);
        frag_f32_f16(of[kk], ov);
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          a0 = fmaf(gv[e], ov[e], a0);
          a1 = fmaf(gv[e + 1], ov[e + 1], a1);
        }
      }
    }
    dl = a0 + a1;
    dl += __shfl_xor(dl, 32, 64);
  }
  if (half == 0 && qi < Tq) p.delta[row] = dl;

  f32x16 dq[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) dq[dt][i] = 0.f;

  const float sl2 = p.scale_log2;
  // LDS byte addresses of the operand reads; the stage, the 32-key block and
  // the 16-key step are immediate offsets.
  const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)smem;
  uint32_t ra[D / 16];  // row l32 of a 32-key block, feature chunk kk
  {
    const int rsw = tile_swz<D>(l32);
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) ra[kk] = base + (uint32_t)((l32 * D + ((kk * 2 + half) ^ rsw) * 8) * 2);
  }
  uint32_t ta[D / 32][2];  // transposing reads of K (the order of TrReader)
  {
    const int tj = lane & 15, tg = (lane >> 4) & 1;
    const int r = 4 * half + (tj >> 2);
    const int sw = tile_swz<D>(r), sw8 = tile_swz<D>(r + 8);
    const int chunk = tg * 2 + ((tj & 3) >> 1), sub = (tj & 1) * 4;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      ta[dt][0] = base + (uint32_t)((r * D + sub + ((dt * 4 + chunk) ^ sw) * 8) * 2);
      ta[dt][1] = base + (uint32_t)(((r + 8) * D + sub + ((dt * 4 + chunk) ^ sw8) * 8) * 2);
    }
  }

  // One 32-key block (MT) of the tile in stage ST:
  //   S^T = K Q^T and dP^T = V dO^T, their MFMAs alternating, K and V row
  //   fragments read kDqPf pairs ahead; dS = P (dP - delta); then
  //   dQ^T += K^T dS^T with the transposed K fragments read kDqPf ahead.
  auto block = [&](auto st_tag, auto mt_tag, int kb, auto edge_tag) __attribute__((always_inline)) {
    constexpr int ST = decltype(st_tag)::value, MT = decltype(mt_tag)::value;
    constexpr bool EDGE = decltype(edge_tag)::value;
    constexpr int KO = 2 * ST * TB + MT * 32 * D * 2;  // K rows of this block
    constexpr int VO = KO + TB;                        // V rows
    constexpr int KT = 2 * ST * TB;                    // K tile (transposing reads)
    bf16x8 kf[NK], vf[NK];
    auto rd = [&](auto j_tag) {
      constexpr int j = decltype(j_tag)::value;
      ds_b128<KO>(kf[j], ra[j]);
      ds_b128<VO>(vf[j], ra[j]);
    };
    f32x16 s, dp;
    static_for<0, kDqPf>(rd);
    fence();
    static_for<0, NK>([&](auto j_tag) {
      constexpr int j = decltype(j_tag)::value;
      if constexpr (j + kDqPf < NK) rd(std::integral_constant<int, j + kDqPf>{});
      constexpr int ahead = 2 * (kDqPf < NK - 1 - j ? kDqPf : NK - 1 - j);
      lgkm_tie<ahead + 1>(kf[j]);
      if constexpr (j == 0)
        s = mfma16<E>(kf[j], qf[j], f32x16{});
      else
        s = mfma16<E>(kf[j], qf[j], s);
      lgkm_tie<ahead>(vf[j]);
      if constexpr (j == 0)
        dp = mfma16<E>(vf[j], gf[j], f32x16{});
      else
        dp = mfma16<E>(vf[j], gf[j], dp);
      fence();
    });
    bf16x8 db[2];
    float dsv[16];  // f16: dS before its rounding, packed by pairs below
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int key = kb + MT * 32 + (i >> 2) * 8 + half * 4 + (i & 3);
      float x = s[i] * sl2;
      if constexpr (MASK) {
        if (qi < Tq && key < Tk)
          x += mask_log2(load_mask(p.mask, p.mask_dtype,
                                  b * p.ms[0] + (int64_t)h * p.ms[1] + (int64_t)qi * p.ms[2] +
                                      (int64_t)key * p.ms[3]));
      }
      float pr = __builtin_amdgcn_exp2f(x - lse);
      if constexpr (EDGE) {
        if (key >= Tk || (CAUSAL && key > qi)) pr = 0.f;
      }
      if constexpr (E == 0) db[i >> 3][i & 7] = f32_elem<E>(pr * (dp[i] - dl));
      else dsv[i] = pr * (dp[i] - dl);
    }
    if constexpr (E != 0) {
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        float t[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) t[e] = dsv[h2 * 8 + e];
        db[h2] = f32_frag_f16(t);
      }
    }
    // dQ MFMA j: d-block j % (D/32), 16-key step j / (D/32) of this block.
    s16x4 tr[NT][2];
    auto rdt = [&](auto j_tag) {
      constexpr int j = decltype(j_tag)::value;
      constexpr int dt = j % (D / 32), ks = j / (D / 32);
      ds_tr<KT + (MT * 2 + ks) * 16 * D * 2>(tr[j][0], ta[dt][0]);
      ds_tr<KT + (MT * 2 + ks) * 16 * D * 2>(tr[j][1], ta[dt][1]);
    };
    static_for<0, kDqPf>(rdt);
    fence();
    static_for<0, NT>([&](auto j_tag) {
      constexpr int j = decltype(j_tag)::value;
      constexpr int dt = j % (D / 32), ks = j / (D / 32);
      if constexpr (j + kDqPf < NT) rdt(std::integral_constant<int, j + kDqPf>{});
      lgkm_tie<2 * (kDqPf < NT - 1 - j ? kDqPf : NT - 1 - j)>(tr[j][0], tr[j][1]);
      const bf16x8 a =
          __builtin_bit_cast(bf16x8, __builtin_shufflevector(tr[j][0], tr[j][1], 0, 1, 2, 3, 4, 5, 6, 7));
      dq[dt] = mfma16<E>(a, db[ks], dq[dt]);
      fence();
    });
  };

  auto step = [&](int t, auto st_tag) __attribute__((always_inline)) {
    const int kb = t * kTile;
    if (q0 >= Tq) return;
    static_for<0, 2>([&](auto mt_tag) {
      constexpr int MT = decltype(mt_tag)::value;
      const int k0r = kb + MT * 32;
      if (k0r >= Tk || (CAUSAL && k0r > q0 + 31)) return;  // nothing of this block is visible
      const bool edge = (k0r + 32 > Tk) || (CAUSAL && k0r + 31 > q0);
      if (edge)
        block(st_tag, mt_tag, kb, std::true_type{});
      else
        block(st_tag, mt_tag, kb, std::false_type{});
    });
  };

  wait_dma();
  __syncthreads();
  for (int t = 0; t < ntiles; t += 2) {
    if (t + 1 < ntiles) issue(t + 1, 1);
    step(t, std::integral_constant<int, 0>{});
    wait_dma();
    __syncthreads();
    if (t + 1 >= ntiles) break;
    if (t + 2 < ntiles) issue(t + 2, 0);
    step(t + 1, std::integral_constant<int, 1>{});
    wait_dma();
    __syncthreads();
  }

  // Every step ended at a barrier after its reads and with no load in
  // flight: the stages take the dQ rows on their way out.  (The first row
  // comes from an opaque copy here, so no address is hoisted into the loop.)
  {
    int r0 = q0;
    asm volatile("" : "+v"(r0));
    const int nvalid = min(max(Tq - r0, 0), 32);
    store_rows_lds<D, E>(smem + wave * 32 * D,
                         static_cast<bf16*>(p.dq) + b * p.dqs[0] + h * p.dqs[1] + (int64_t)r0 * p.dqs[2], p.dqs[2],
                         nvalid, dq, l32, half, lane, p.scale);
  }
}

template <int D, bool CAUSAL, bool MASK, int E>
int launch_t(const SdpaBwdParams& p, hipStream_t s) {
  const int64_t q_blocks = (int64_t)p.B * p.Hq * ((p.Tq + kRows - 1) / kRows);
  hipLaunchKernelGGL((bwd_dq_mfma<D, CAUSAL, MASK, E>), dim3((unsigned)q_blocks), dim3(kNT), 0, s, p);
  if (int rc = launch_status("bwd_dq_mfma")) return rc;
  const int64_t kv_blocks = (int64_t)p.B * p.Hkv * ((p.Tk + kRows - 1) / kRows);
  hipLaunchKernelGGL((bwd_dkdv_mfma<D, CAUSAL, MASK, E>), dim3((unsigned)kv_blocks), dim3(kNT), 0, s, p);
  return launch_status("bwd_dkdv_mfma");
}

template <int D, int E>
int launch_d(const SdpaBwdParams& p, hipStream_t s) {
  const bool m = p.mask != nullptr;
  if (p.causal) return m ? launch_t<D, true, true, E>(p, s) : launch_t<D, true, false, E>(p, s);
  return m ? launch_t<D, false, true, E>(p, s) : launch_t<D, false, false, E>(p, s);
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace

bool bwd_mfma_supports(const SdpaBwdParams& p) {
  if (p.dtype != MFX_BF16 && p.dtype != MFX_F16) return false;
  if (p.D != p.Dv || (p.D != 64 && p.D != 128)) return false;
  if (!(p.scale_log2 > 0.f)) return false;
  // p.o is null until launch when O is recomputed (then it is the
  // workspace: 256-byte aligned, contiguous).
  const void* ptrs[8] = {p.q, p.k, p.v, p.dout, p.dq, p.dk, p.dv, p.o};
  for (const void* ptr : ptrs)
    if (!aligned16(ptr)) return false;
  for (int i = 0; i < 3; ++i)
    if (p.qs[i] % 8 || p.ks[i] % 8 || p.vs[i] % 8 || p.dos[i] % 8 || p.dqs[i] % 8 || p.dks[i] % 8 ||
        p.dvs[i] % 8 || p.os[i] % 8)
      return false;
  // K / V / Q / dO rows are read through buffer resources whose extents
  // assume rows of at least D elements (rows past the end then read zeros).
  if (p.ks[2] < p.D || p.vs[2] < p.Dv || p.qs[2] < p.D || p.dos[2] < p.Dv) return false;
  // Buffer-resource extents are 31-bit: one kv head's K / V rows, and the
  // query rows (and lse / delta) of all heads of one group.
  const int64_t lim = 1LL << 31;
  if ((int64_t)p.Tk * p.ks[2] * 2 >= lim || (int64_t)p.Tk * p.vs[2] * 2 >= lim) return false;
  if (((int64_t)(p.group - 1) * p.qs[1] + (int64_t)p.Tq * p.qs[2] + p.D) * 2 >= lim) return false;
  if (((int64_t)(p.group - 1) * p.dos[1] + (int64_t)p.Tq * p.dos[2] + p.D) * 2 >= lim) return false;
  // Tile offsets in bytes stay below 2^31 as well.
  if ((int64_t)p.qs[1] < 0 || p.qs[2] < 0 || p.dos[1] < 0 || p.dos[2] < 0) return false;
  if ((int64_t)p.group * p.Tq * 4 >= lim) return false;
  if ((int64_t)p.B * p.Hq * ((p.Tq + kRows - 1) / kRows) >= lim) return false;
  return true;
}

int launch_bwd_mfma(const SdpaBwdParams& p, hipStream_t s) {
  if (p.dtype == MFX_F16) return p.D == 128 ? launch_d<128, 1>(p, s) : launch_d<64, 1>(p, s);
  return p.D == 128 ? launch_d<128, 0>(p, s) : launch_d<64, 0>(p, s);
}

}  // namespace mfx

#if defined(MFX_PHASE_TIMERS)
// Diagnostic build only: copies up to max_records dK/dV phase records
// (kBwdPhaseFields u64 each, fields as written at the end of bwd_dkdv_mfma) to host memory
// after the device is idle and returns how many the device array holds;
// clear != 0 zeroes the array afterwards.  Not part of the product's C ABI.
extern "C" __attribute__((visibility("default"))) int64_t mfx_bwd_phase_timers_read(void* host, int64_t max_records,
                                                                                    int clear) {
  if (hipDeviceSynchronize() != hipSuccess) return -1;
  void* dev = nullptr;
  if (hipGetSymbolAddress(&dev, HIP_SYMBOL(mfx::g_bwd_phase_records)) != hipSuccess) return -1;
  const int64_t n = max_records < mfx::kBwdPhaseRecords ? max_records : mfx::kBwdPhaseRecords;
  if (host && n > 0 &&
      hipMemcpy(host, dev, (size_t)n * mfx::kBwdPhaseFields * 8, hipMemcpyDeviceToHost) != hipSuccess)
    return -1;
  if (clear && hipMemset(dev, 0, sizeof(mfx::g_bwd_phase_records)) != hipSuccess) return -1;
  if (hipDeviceSynchronize() != hipSuccess) return -1;
  return mfx::kBwdPhaseRecords;
}
#endif
