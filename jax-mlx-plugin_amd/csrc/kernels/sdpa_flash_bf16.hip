// Flash attention forward with an additive mask, bf16 inputs, fp32
// accumulation, gfx950 MFMA.  (Mask-free calls go to the software-pipelined
// kernel in sdpa_flash_bf16_pipe.hip.)
//
// Workgroup = 4 wavefronts = 128 query rows of one (batch, head); each
// wavefront owns 32 query rows.  K/V stream through LDS in 64-key tiles, two
// stages: while tile t is computed, tile t+1 is copied global -> LDS by the
// asynchronous LDS-DMA loads (buffer_load_dwordx4 ... lds: no registers, no
// VALU), and one vmcnt wait + barrier per tile publishes it.
//
// Both products use v_mfma_f32_32x32x16_bf16 and are arranged so that the
// online softmax needs almost no cross-lane traffic:
//   S^T = K Q^T   A = K tile rows (from LDS), B = Q rows (registers).  The
//                 32x32 accumulator gives lane l query (l % 32) and 16 keys,
//                 so a query's row max / sum is 16 in-lane values plus one
//                 exchange with lane l ^ 32.
//   O^T = V^T P^T A = V^T fragments read from the row-major V tile with the
//                 transposing LDS read (ds_read_b64_tr_b16: 16 lanes x 4
//                 keys per read), B = P taken straight from the S^T
//                 accumulator: the contraction index (key) is permuted
//                 identically in A and B, so the accumulator registers are
//                 already the B operand.
// Each lane also owns one query of O^T, so the online-softmax rescale is a
// per-lane scalar multiply, and it is lazy (see kSlack).
//
// Tiles are row-major with 16-byte chunks XOR-swizzled per row, so the K
// operand reads (8 lanes on 8 rows) and the transposing V reads (4 rows x 32
// bytes per 16 lanes) are bank-conflict free; the DMA writes 1 KiB runs.
//
// Causal tiles past a wavefront's last query are skipped; the blockIdx ->
// (head, q-block) map keeps the q-blocks of one head on one XCD (blocks are
// dealt to the 8 XCDs round-robin) and issues each XCD's blocks longest
// first, which balances the causal triangle across the CUs.
#include <type_traits>

#include "sdpa_elem.h"
#include "sdpa_tiles.h"

namespace mfx {
namespace {

constexpr int kBM = 128;  // query rows per workgroup
constexpr int kBN = 64;        // keys per tile
constexpr int kMT = kBN / 32;  // 32-key score blocks per tile
constexpr int kKS = kBN / 16;  // 16-key PV steps per tile
constexpr int kNT = 256;  // threads per workgroup

using tiles::kSlack;
using tiles::lds_s16x4_t;
using tiles::s16x4;
using tiles::tile_swz;
using tiles::wait_dma;
using tiles::fence;
template <int D>
using TileLoader = tiles::TileLoader<D, kBN, kNT / 64>;

// D = 256: one workgroup per CU (four 32 KB tiles; O, Q and S of a wavefront
// take ~300 registers).
template <int D, bool CAUSAL, bool MASK, int E>
__global__ __launch_bounds__(kNT, D > 128 ? 1 : 2) void flash_bf16_kernel(SdpaParams p) {
  __shared__ __attribute__((aligned(16))) bf16 k0[kBN * D];
  __shared__ __attribute__((aligned(16))) bf16 v0[kBN * D];
  __shared__ __attribute__((aligned(16))) bf16 k1[kBN * D];
  __shared__ __attribute__((aligned(16))) bf16 v1[kBN * D];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;
  const int l32 = lane & 31;

  const int nmb = (p.Tq + kBM - 1) / kBM;
  const int BH = p.B * p.Hq;
  const int id = blockIdx.x;
  int bh, mblk;
  if ((BH & 7) == 0) {
    // Blocks are dealt to the 8 XCDs round-robin; within an XCD the issue
    // order is longest causal q-block first across all of its heads (LPT
    // list scheduling), so the short blocks fill the tail.
    const int xcd = id & 7, slot = id >> 3, bpx = BH >> 3;
    bh = (slot % bpx) * 8 + xcd;
    mblk = nmb - 1 - slot / bpx;
  } else {
    bh = id % BH;
    mblk = nmb - 1 - id / BH;
  }
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h / p.group;
  const bf16* qp = static_cast<const bf16*>(p.q) + b * p.qs[0] + h * p.qs[1];
  const bf16* kp = static_cast<const bf16*>(p.k) + b * p.ks[0] + hk * p.ks[1];
  const bf16* vp = static_cast<const bf16*>(p.v) + b * p.vs[0] + hk * p.vs[1];
  bf16* op = static_cast<bf16*>(p.out) + b * p.os[0] + h * p.os[1];
  const int64_t qs2 = p.qs[2], ks2 = p.ks[2], vs2 = p.vs[2], os2 = p.os[2];
  const int Tq = p.Tq, Tk = p.Tk;

  const int q0 = mblk * kBM + wave * 32;
  const int qi = q0 + l32;

  int kv_end = Tk;
  // D = 256 compiles only the causal form (the other spills at this width):
  // key j is visible to query i when j <= i + co, co = 0 for a causal call
  // and 2^30 (every key) otherwise.
  const int co = !p.causal ? (1 << 30) : 0;
  if (CAUSAL) kv_end = min(Tk, min(Tq + co, (mblk + 1) * kBM + co));
  const int ntiles = (kv_end + kBN - 1) / kBN;
  const TileLoader<D> kload(kp, ks2, Tk, D, wave, lane), vload(vp, vs2, Tk, D, wave, lane);
  auto issue = [&](int t, bf16* kl, bf16* vl) {
    kload.load(t, kl, wave);
    vload.load(t, vl, wave);
  };
  if (ntiles > 0) issue(0, k0, v0);

  // Rows past Tq load a valid row and are zeroed, so no load is predicated.
  bf16x8 qf[D / 16];
  {
    const bf16* qrow = qp + (int64_t)min(qi, Tq - 1) * qs2 + half * 8;
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      u32x4 raw = *reinterpret_cast<const u32x4*>(qrow + kk * 16);
      if (qi >= Tq) raw = u32x4{0u, 0u, 0u, 0u};
      qf[kk] = __builtin_bit_cast(bf16x8, raw);
    }
  }

  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
  // Running exp2 base (log2 units, shared by lanes l and l^32) and the
  // lane's partial row sum.
  float b_run = -INFINITY, l_run = 0.f;
  const float sl2 = p.scale_log2;  // > 0 (checked on the host)

  // Per-lane LDS offsets (bf16 elements) of the operand reads.
  const int k_off = l32 * D;            // + mt*32*D, chunk (kk*2 + half) ^ k_sw
  const int k_sw = tile_swz<D>(l32);
  const int tj = lane & 15, tg = (lane >> 4) & 1;
  const int v_row = 4 * half + (tj >> 2);  // + ks*16 + 8*r
  const int v_sw = tile_swz<D>(v_row), v_sw8 = tile_swz<D>(v_row + 8);
  const int v_chunk = tg * 2 + ((tj & 3) >> 1);  // + dt*4
  const int v_sub = (tj & 1) * 4;

  // One 64-key tile for this wave's 32 queries.  EDGE tiles (ragged end,
  // causal diagonal) mask per element; interior tiles do no mask work.
  auto compute = [&](const bf16* kl, const bf16* vl, int kb, auto edge_tag) {
    constexpr bool EDGE = decltype(edge_tag)::value;
    // D = 256: the phases of a tile (S, softmax, PV) and the tiles stay
    // apart, so no tile's fragments are live across another's.
    if constexpr (D > 128) fence();
    f32x16 s[kMT];
    // The two waves of a SIMD alternate between MFMA blocks and softmax
    // work; raising a wave's priority for its MFMA blocks lets the arbiter
    // keep the matrix core fed while the other wave's vector work fills in.
    __builtin_amdgcn_s_setprio(3);
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[mt][i] = 0.f;
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(&kl[mt * 32 * D + k_off + ((kk * 2 + half) ^ k_sw) * 8]);
        s[mt] = mfma16<E>(a, qf[kk], s[mt]);
        // D = 256: at most four operand reads run ahead of their MFMAs (all
        // of a tile's at once do not fit the registers).
        if constexpr (D > 128)
          if ((kk & 3) == 3) fence();
      }
    }
    __builtin_amdgcn_s_setprio(0);
    if constexpr (D > 128) fence();
    // MASK: scores move to the log2 domain here (scale and mask folded);
    // otherwise they stay raw and the scale is folded into the exp2 FMA.
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float x = s[mt][i];
        const int key = kb + mt * 32 + (i >> 2) * 8 + half * 4 + (i & 3);
        if constexpr (MASK) {
          x *= sl2;
          if (qi < Tq && key < Tk)
            x += mask_log2(load_mask(p.mask, p.mask_dtype,
                                    b * p.ms[0] + h * p.ms[1] + qi * p.ms[2] + key * p.ms[3]));
        }
        if constexpr (EDGE) {
          if (key >= Tk || (CAUSAL && key > qi + co)) x = -INFINITY;
        }
        s[mt][i] = x;
        mx = fmaxf(mx, x);
      }
    // Lanes l and l^32 hold the two halves of one query's keys.
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    const float m_l2 = MASK ? mx : mx * sl2;
    const bool need = m_l2 > b_run + kSlack;
    if (__ballot(need)) {
      const float nb = need ? m_l2 : b_run;
      const float alpha = need ? __builtin_amdgcn_exp2f(b_run - nb) : 1.f;
      b_run = nb;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
    }
    const float nbase = b_run == -INFINITY ? 0.f : -b_run;
    auto pexp = [&](int mt, int i) {
      return MASK ? __builtin_amdgcn_exp2f(s[mt][i] + nbase) : __builtin_amdgcn_exp2f(fmaf(s[mt][i], sl2, nbase));
    };
    // P rounded to the element type and the row sum of exactly the rounded
    // values the PV product consumes, two per instruction.
    bf16x8 pb[kKS];
    float l0 = 0.f, l1 = 0.f;
    if constexpr (E == 0) {
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) pb[mt * 2 + (i >> 3)][i & 7] = f32_elem<E>(pexp(mt, i));
#pragma unroll
      for (int j = 0; j < kKS; ++j) {
        const bf16x8 w = pb[j];
        l0 = dot2_at<E>(w, 0, l0);
        l1 = dot2_at<E>(w, 2, l1);
        l0 = dot2_at<E>(w, 4, l0);
        l1 = dot2_at<E>(w, 6, l1);
      }
    } else {
      // f16: pairs packed into dwords first.  (Element inserts into the
      // 16-bit vector followed by per-element dot2 operands compile to
      // wrong row sums for f16: pairs built from one value twice.)
      u32x4 pw[kKS];
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          const uint32_t w = pack2<E>(pexp(mt, i), pexp(mt, i + 1));
          pw[mt * 2 + (i >> 3)][(i & 7) >> 1] = w;
          if ((i & 2) == 0) l0 = dot2<E>(w, l0);
          else l1 = dot2<E>(w, l1);
        }
#pragma unroll
      for (int j = 0; j < kKS; ++j) pb[j] = __builtin_bit_cast(bf16x8, pw[j]);
    }
    l_run += l0 + l1;
    if constexpr (D > 128) fence();
    __builtin_amdgcn_s_setprio(3);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int ks = 0; ks < kKS; ++ks) {
        // k-slots 0-3: keys ks*16 + 4*half + e; slots 4-7: the same + 8.
        const bf16* v_rows = vl + (ks * 16 + v_row) * D + v_sub;
        const s16x4 lo =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(v_rows + ((dt * 4 + v_chunk) ^ v_sw) * 8));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4_t*)(v_rows + 8 * D + ((dt * 4 + v_chunk) ^ v_sw8) * 8));
        const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        o[dt] = mfma16<E>(a, pb[ks], o[dt]);
        if constexpr (D > 128)
          if ((ks & 1) == 1) fence();
      }
    if constexpr (D > 128) fence();
  };

  auto step = [&](int t, const bf16* kl, const bf16* vl) {
    const int kb = t * kBN;
    if (q0 >= Tq || (CAUSAL && kb > q0 + 31 + co)) return;  // nothing of this tile is visible
    const bool edge = (kb + kBN > Tk) || (CAUSAL && kb + kBN - 1 > q0 + co);
    if (edge)
      compute(kl, vl, kb, std::true_type{});
    else
      compute(kl, vl, kb, std::false_type{});
  };

  wait_dma();
  __syncthreads();
  // Two stages with distinct LDS arrays (so the compiler's LDS-DMA tracking
  // sees that the loads in flight never alias the tile being read).
  // The restrict-qualified parameters give every access of one iteration
  // scoped no-alias metadata, so the waitcnt pass does not make the tile's
  // reads wait for the next tile's LDS-DMA writes.
  auto iter = [&](int t, const bf16* __restrict__ kc, const bf16* __restrict__ vc, bf16* __restrict__ kn,
                  bf16* __restrict__ vn) {
    if (t + 1 < ntiles) issue(t + 1, kn, vn);
    step(t, kc, vc);
  };
  for (int t = 0; t < ntiles; t += 2) {
    iter(t, k0, v0, k1, v1);
    wait_dma();
    __syncthreads();
    if (t + 1 >= ntiles) break;
    iter(t + 1, k1, v1, k0, v0);
    wait_dma();
    __syncthreads();
  }

  const float lt = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = 1.0f / lt;
  if (p.lse && half == 0 && qi < Tq) p.lse[(int64_t)bh * Tq + qi] = b_run + __log2f(lt);
  if constexpr (D <= 128) {
    // Every iteration ended at a barrier after its reads and with no load in
    // flight: the tile arrays take the output rows on their way out (k0
    // holds wavefronts 0 and 1, v0 wavefronts 2 and 3), stored as whole
    // rows streamed past the L2.  (The first row comes from an opaque copy,
    // so no address is hoisted into the loop.)  At D = 256, one workgroup per
    // CU, nothing would cover the LDS round trip: 8-byte pieces there.
    int r0 = q0;
    asm volatile("" : "+v"(r0));
    store_rows_lds<D, E>((wave < 2 ? k0 : v0) + (wave & 1) * 32 * D, op + (int64_t)r0 * os2, os2,
                         min(max(Tq - r0, 0), 32), o, l32, half, lane, inv);
  } else if (qi < Tq) {
    bf16* orow = op + qi * os2;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = store_e<E>(o[dt][g * 4 + e] * inv);
        *reinterpret_cast<u16x4*>(orow + dt * 32 + g * 8 + half * 4) = w;
      }
  }
}

template <int D, bool CAUSAL, bool MASK, int E>
int launch_t(const SdpaParams& p, hipStream_t s) {
  const int nmb = (p.Tq + kBM - 1) / kBM;
  const int64_t blocks = (int64_t)nmb * p.B * p.Hq;
  hipLaunchKernelGGL((flash_bf16_kernel<D, CAUSAL, MASK, E>), dim3((unsigned)blocks), dim3(kNT), 0, s, p);
  return launch_status("flash_bf16_kernel");
}

template <int D, int E>
int launch_d(const SdpaParams& p, hipStream_t s) {
  return launch_t<D, true, true, E>(p, s);
}

// Head size 256, every mask form (the pipelined kernel stops at 128): the
// causal instantiations serve non-causal calls too (through the kernel's
// causal offset).
template <int E>
int launch_256(const SdpaParams& p, hipStream_t s) {
  return p.mask ? launch_t<256, true, true, E>(p, s) : launch_t<256, true, false, E>(p, s);
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace

bool flash_bf16_supports(const SdpaParams& p) {
  if (p.dtype != MFX_BF16 && p.dtype != MFX_F16) return false;
  if (!(p.scale_log2 > 0.f)) return false;  // the exp2 FMA folds a positive scale
  // K/V rows are read through one buffer resource per head ending at its
  // last row's last feature, range-checked on 31-bit lane offsets: row
  // strides of at least D (rows past Tk then start at or past the extent and
  // read as zeros; a smaller stride, such as 0 for a broadcast view, would
  // leave rows past Tk inside it).
  if (p.ks[2] < p.D || p.vs[2] < p.Dv) return false;
  if ((int64_t)p.Tk * p.ks[2] * 2 >= (1LL << 31) || (int64_t)p.Tk * p.vs[2] * 2 >= (1LL << 31)) return false;
  if (p.D != p.Dv || (p.D != 32 && p.D != 64 && p.D != 96 && p.D != 128 && p.D != 256)) return false;
  // Masks that vary along query rows run on this file's kernel: head sizes
  // 64, 128 and 256 only.
  if (p.mask && p.ms[2] != 0 && p.Tq > 1 && p.D != 64 && p.D != 128 && p.D != 256) return false;
  if (!aligned16(p.q) || !aligned16(p.k) || !aligned16(p.v) || !aligned16(p.out)) return false;
  for (int i = 0; i < 3; ++i)
    if (p.qs[i] % 8 || p.ks[i] % 8 || p.vs[i] % 8 || p.os[i] % 8) return false;  // 16-byte rows
  return true;
}

int launch_flash_bf16(const SdpaParams& p, hipStream_t s) {
  // Without an additive mask, or with one that does not vary along query
  // rows, the software-pipelined kernel runs (sdpa_flash_bf16_pipe.hip);
  // this file's kernel serves masks with a query-row stride, and head size
  // 256 in every form.  (With one query row the pipelined kernel's mask row
  // is that row.)
  if (p.D == 256) return p.dtype == MFX_F16 ? launch_256<1>(p, s) : launch_256<0>(p, s);
  if (!p.mask || p.ms[2] == 0 || p.Tq == 1) return launch_flash_bf16_pipe(p, s);
  if (p.dtype == MFX_F16) return p.D == 128 ? launch_d<128, 1>(p, s) : launch_d<64, 1>(p, s);
  return p.D == 128 ? launch_d<128, 0>(p, s) : launch_d<64, 0>(p, s);
}

}  // namespace mfx
