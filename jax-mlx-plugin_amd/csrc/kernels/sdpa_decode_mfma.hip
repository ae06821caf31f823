// Split-KV attention for few query rows per kv head on the matrix cores
// (GQA / MQA decode, bf16).
//
// The R = (Hq/Hkv) * Tq query rows that share one kv head (R <= 32) are the
// columns of one 32-wide MFMA operand, so every K/V row is read from HBM once
// for all of them.  The grid is (B*Hkv, W): W wavefronts (one per workgroup)
// share a kv head and wavefront j takes the 32-key tiles j, j+W, j+2W, ...,
// so every wavefront gets an equal share of a valid prefix (a length-masked
// cache) and the partial results of the W wavefronts merge at the end:
//   S^T = K Q^T   A = K tile rows (LDS), B = the R query rows (registers,
//                 zero-padded to 32 columns): v_mfma_f32_32x32x16_bf16.
//   O^T = V^T P^T A = transposing LDS reads of the V tile, B = P straight
//                 from the S^T accumulator (same key permutation), as in the
//                 prefill kernel.
// The padding wastes MFMA work that costs a few microseconds against the
// tens of microseconds the K/V bytes take: the kernel is HBM-bound.
//
// K/V tiles stream through two swizzled LDS stages by asynchronous LDS-DMA
// loads; while one tile is computed, the next valid tile is in flight.  A
// prepass marks the tiles that hold at least one visible key (additive mask
// not -inf for some row, key < Tk, causal limit), and only those are
// loaded, so a padded KV cache costs the bytes of its valid prefix.  The W
// partials (m, l, O) of a row merge in the split-KV combine kernel.
//
// Optional fused RMSNorm of the query rows (reference chain rms_norm -> sdpa
// of GQA decode): q is normalised in fp32 and rounded to bf16 before it is
// used, exactly as the unfused graph rounds the RMSNorm output.
#include <type_traits>

#include "sdpa_tiles.h"

namespace mfx {
namespace {

using tiles::kSlack;
using tiles::lds_s16x4_t;
using tiles::s16x4;
using tiles::tile_swz;

constexpr int kDN = 32;  // keys per tile: 32 KB of LDS per workgroup, five per CU
constexpr int kMT = kDN / 32;
constexpr int kKS = kDN / 16;
constexpr int kMaxTiles = 64;  // per wavefront: width of the valid-tile bitmap

// s_waitcnt vmcnt(N) with the other counters left alone (N < 64).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

template <int D, bool MASK, bool CAUSAL>
__global__ __launch_bounds__(64) void decode_mfma_kernel(SdpaParams p) {
  using Loader = tiles::TileLoader<D, kDN, 1>;
  __shared__ __attribute__((aligned(16))) bf16 k0[kDN * D];
  __shared__ __attribute__((aligned(16))) bf16 v0[kDN * D];
  __shared__ __attribute__((aligned(16))) bf16 k1[kDN * D];
  __shared__ __attribute__((aligned(16))) bf16 v1[kDN * D];

  const int lane = threadIdx.x;
  const int half = lane >> 5, col = lane & 31;
  const int split = blockIdx.y, bhk = blockIdx.x;  // split = this wavefront's tile phase j
  const int W = p.num_splits;
  const int b = bhk / p.Hkv, hk = bhk % p.Hkv;
  const int Tq = p.Tq, R = p.group * Tq, Tk = p.Tk;

  // This lane's query column (rows past R are zero and never stored).
  const bool qvalid = col < R;
  const int rr = qvalid ? col : 0;
  const int hq = hk * p.group + rr / Tq, tq = rr % Tq;

  bf16x8 qf[D / 16];
  {
    const bf16* qrow = static_cast<const bf16*>(p.q) + b * p.qs[0] + hq * p.qs[1] + tq * p.qs[2] + half * 8;
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      u32x4 raw = *reinterpret_cast<const u32x4*>(qrow + kk * 16);
      if (!qvalid) raw = u32x4{0u, 0u, 0u, 0u};
      qf[kk] = __builtin_bit_cast(bf16x8, raw);
    }
  }
  if (p.q_rms_eps >= 0.f) {
    // Lane holds d = kk*16 + half*8 + e; lanes col and col+32 hold one row.
    float ss = 0.f;
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = static_cast<float>(qf[kk][e]);
        ss += x * x;
      }
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
    ss = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    const float inv = rsqrtf(ss / (float)D + p.q_rms_eps);
    const bf16* w = static_cast<const bf16*>(p.q_rms_weight);
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float t = static_cast<float>(qf[kk][e]) * inv;
        if (w) t *= static_cast<float>(w[kk * 16 + half * 8 + e]);
        qf[kk][e] = static_cast<bf16>(t);
      }
  }
  const float sl2 = p.scale_log2;  // > 0 (checked on the host)

  // This wavefront's tiles: global tile split + W*i, i = 0 .. ntile-1.
  const int tiles_total = (Tk + kDN - 1) / kDN;
  const int ntile = split < tiles_total ? (tiles_total - split + W - 1) / W : 0;  // <= kMaxTiles (host)
  int64_t m_base = 0;
  if constexpr (MASK) m_base = b * p.ms[0] + hq * p.ms[1] + tq * p.ms[2];

  // Prepass: bit i set when local tile i holds a key some row can see.  Lane
  // l checks key (l % 32) of local tile 2c + l/32; the loads of all chunks
  // are issued eight at a time, so the whole prepass costs one or two round
  // trips.  A mask that does not vary over heads and query positions is
  // checked once per key, otherwise once per (row, key).
  uint64_t vbits = 0;
  {
    const bool bcast = !MASK || ((p.ms[1] == 0 || p.group == 1) && (p.ms[2] == 0 || Tq == 1));
    const int nchunk = (ntile + 1) / 2;
    for (int c0 = 0; c0 < nchunk; c0 += 8) {
      bool ok[8];
      int keyj[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = 2 * (c0 + j) + (lane >> 5);
        const int key = (split + W * i) * kDN + (lane & 31);
        keyj[j] = min(key, Tk - 1);
        ok[j] = i < ntile && key < Tk;
        if (CAUSAL) ok[j] = ok[j] && key <= Tq - 1;
      }
      if constexpr (MASK) {
        if (bcast) {
          float mvv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) mvv[j] = load_mask(p.mask, p.mask_dtype, b * p.ms[0] + (int64_t)keyj[j] * p.ms[3]);
#pragma unroll
          for (int j = 0; j < 8; ++j) ok[j] = ok[j] && mvv[j] != -INFINITY;
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            bool any = false;
            for (int r = 0; r < R; ++r) {
              const int h2 = hk * p.group + r / Tq, t2 = r % Tq;
              const float mvv = load_mask(p.mask, p.mask_dtype,
                                          b * p.ms[0] + h2 * p.ms[1] + t2 * p.ms[2] + (int64_t)keyj[j] * p.ms[3]);
              any |= mvv != -INFINITY && (!CAUSAL || keyj[j] <= t2);
            }
            ok[j] = ok[j] && any;
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint64_t bal = __ballot(ok[j]);
        const int i = 2 * (c0 + j);
        if ((bal & 0xffffffffull) && i < kMaxTiles) vbits |= 1ull << i;
        if ((bal >> 32) && i + 1 < kMaxTiles) vbits |= 1ull << (i + 1);
      }
    }
  }

  const bf16* kp = static_cast<const bf16*>(p.k) + b * p.ks[0] + hk * p.ks[1];
  const bf16* vp = static_cast<const bf16*>(p.v) + b * p.vs[0] + hk * p.vs[1];
  const Loader kload(kp, p.ks[2], Tk, 0, lane), vload(vp, p.vs[2], Tk, 0, lane);
  auto gtile = [&](int i) { return split + W * i; };

  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
  float b_run = -INFINITY, l_run = 0.f;

  // Per-lane byte offsets of the operand reads within a tile (the same
  // patterns as the prefill kernel).
  uint32_t k_addr[D / 16];
  uint32_t v_addr[D / 32][2];
  {
    const int k_sw = tile_swz<D>(col);
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) k_addr[kk] = (uint32_t)((col * D + ((kk * 2 + half) ^ k_sw) * 8) * 2);
    const int tj = lane & 15, tg = (lane >> 4) & 1;
    const int v_row = 4 * half + (tj >> 2);
    const int v_sw = tile_swz<D>(v_row), v_sw8 = tile_swz<D>(v_row + 8);
    const int v_chunk = tg * 2 + ((tj & 3) >> 1);
    const int v_sub = (tj & 1) * 4;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      v_addr[dt][0] = (uint32_t)((v_row * D + v_sub + ((dt * 4 + v_chunk) ^ v_sw) * 8) * 2);
      v_addr[dt][1] = (uint32_t)(((v_row + 8) * D + v_sub + ((dt * 4 + v_chunk) ^ v_sw8) * 8) * 2);
    }
  }

  // Mask values of tile tn in the S^T lane layout (keys past Tk clamped:
  // they are masked by the key < Tk test).
  float mv_next[kMT][16];
  auto load_tile_mask = [&](int tn) __attribute__((always_inline)) {
    const int kb = gtile(tn) * kDN;
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = min(kb + mt * 32 + (i >> 2) * 8 + half * 4 + (i & 3), Tk - 1);
        mv_next[mt][i] = kLog2e * load_mask(p.mask, p.mask_dtype, m_base + (int64_t)key * p.ms[3]);
      }
  };

  auto next_tile = [&](int t) -> int {
    const uint64_t rest = t + 1 < 64 ? (vbits >> (t + 1)) : 0;
    return rest ? t + 1 + __builtin_ctzll(rest) : -1;
  };

  // Tile t from stage (kc, vc) while tile tn (if any) is issued into
  // (kn, vn).  The restrict-qualified stage pointers scope this tile's
  // accesses, so the compiler's LDS-DMA tracking does not make the operand
  // reads wait for the next tile's loads.
  auto body = [&](int t, int tn, const bf16* __restrict__ kc, const bf16* __restrict__ vc, bf16* __restrict__ kn,
                  bf16* __restrict__ vn) __attribute__((always_inline)) {
    const int kb = gtile(t) * kDN;
    // This tile's mask values arrived with its K/V; the next tile's are
    // issued after its DMA, so one in-order vmcnt wait covers this tile.
    float mv[kMT][16];
    if constexpr (MASK) {
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) mv[mt][i] = mv_next[mt][i];
    }
    if (tn >= 0) {
      kload.load(gtile(tn), kn, 0);
      vload.load(gtile(tn), vn, 0);
      if constexpr (MASK) {
        load_tile_mask(tn);
        wait_vm<2 * Loader::LOADS + 16 * kMT>();
      } else {
        wait_vm<2 * Loader::LOADS>();
      }
    } else {
      wait_vm<0>();
    }
    f32x16 s[kMT];
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[mt][i] = 0.f;
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const char*>(kc) + k_addr[kk] +
                                                          mt * 32 * D * 2);
        s[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], s[mt], 0, 0, 0);
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb + mt * 32 + (i >> 2) * 8 + half * 4 + (i & 3);
        float x = s[mt][i] * sl2;
        if constexpr (MASK) x += mv[mt][i];
        if (key >= Tk || (CAUSAL && key > tq)) x = -INFINITY;
        s[mt][i] = x;
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
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
    }
    const float nbase = b_run == -INFINITY ? 0.f : -b_run;
    bf16x8 pb[kKS];
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        pb[mt * 2 + (i >> 3)][i & 7] = static_cast<bf16>(__builtin_amdgcn_exp2f(s[mt][i] + nbase));
    {
      const bf16x2 one = {static_cast<bf16>(1.f), static_cast<bf16>(1.f)};
      float l0 = 0.f, l1 = 0.f;
#pragma unroll
      for (int j = 0; j < kKS; ++j) {
        const bf16x8 w = pb[j];
        l0 = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{w[0], w[1]}, one, l0, false);
        l1 = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{w[2], w[3]}, one, l1, false);
        l0 = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{w[4], w[5]}, one, l0, false);
        l1 = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{w[6], w[7]}, one, l1, false);
      }
      l_run += l0 + l1;
    }
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int ks = 0; ks < kKS; ++ks) {
        const char* vb = reinterpret_cast<const char*>(vc) + ks * 16 * D * 2;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vb + v_addr[dt][0]));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vb + v_addr[dt][1]));
        const bf16x8 a = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[ks], o[dt], 0, 0, 0);
      }
  };

  int t = vbits ? __builtin_ctzll(vbits) : -1;
  if (t >= 0) {
    kload.load(gtile(t), k0, 0);
    vload.load(gtile(t), v0, 0);
    if constexpr (MASK) load_tile_mask(t);
  }
  // Two tiles per iteration (stage 0, stage 1), at most kMaxTiles tiles.
  for (int it = 0; it < kMaxTiles && t >= 0; it += 2) {
    int tn = next_tile(t);
    body(t, tn, k0, v0, k1, v1);
    if (tn < 0) break;
    t = tn;
    tn = next_tile(t);
    body(t, tn, k1, v1, k0, v0);
    t = tn;
  }

  // Lanes col and col+32 hold the two halves of each row's keys.
  float lt;
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
    lt = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if (!qvalid) return;
  if (p.num_splits == 1) {
    const float inv = 1.0f / lt;
    bf16* orow = static_cast<bf16*>(p.out) + b * p.os[0] + hq * p.os[1] + tq * p.os[2];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
#pragma unroll
        for (int e = 0; e < 4; ++e) orow[dt * 32 + gq * 8 + half * 4 + e] = static_cast<bf16>(o[dt][gq * 4 + e] * inv);
  } else {
    const int64_t rows_total = (int64_t)p.B * p.Hq * Tq;
    const int64_t row = ((int64_t)b * p.Hq + hq) * Tq + tq;
    float* part = p.partial + ((int64_t)split * rows_total + row) * (D + 2);
    if (half == 0) {
      part[0] = b_run;
      part[1] = lt;
    }
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
#pragma unroll
        for (int e = 0; e < 4; ++e) part[2 + dt * 32 + gq * 8 + half * 4 + e] = o[dt][gq * 4 + e];
  }
}

template <int D, bool MASK, bool CAUSAL>
int launch_t(const SdpaParams& p, hipStream_t s) {
  dim3 grid((unsigned)(p.B * p.Hkv), (unsigned)p.num_splits);  // (kv heads, W)
  hipLaunchKernelGGL((decode_mfma_kernel<D, MASK, CAUSAL>), grid, dim3(64), 0, s, p);
  int rc = launch_status("decode_mfma_kernel");
  if (rc != MFX_OK || p.num_splits == 1) return rc;
  return launch_decode_combine(p, s);
}

template <int D>
int launch_d(const SdpaParams& p, hipStream_t s) {
  const bool m = p.mask != nullptr;
  if (p.causal) return m ? launch_t<D, true, true>(p, s) : launch_t<D, false, true>(p, s);
  return m ? launch_t<D, true, false>(p, s) : launch_t<D, false, false>(p, s);
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace

bool decode_mfma_supports(const SdpaParams& p) {
  if (p.dtype != MFX_BF16) return false;
  if (!(p.scale_log2 > 0.f)) return false;
  if (p.D != p.Dv || (p.D != 64 && p.D != 128)) return false;
  if (p.group * p.Tq > 32) return false;
  if ((int64_t)(p.Tk + kMaxTiles * kDN - 1) / (kMaxTiles * kDN) > 65535) return false;  // grid y = W
  if ((int64_t)p.Tk * p.ks[2] * 2 >= (1LL << 31) || (int64_t)p.Tk * p.vs[2] * 2 >= (1LL << 31)) return false;
  if (!aligned16(p.q) || !aligned16(p.k) || !aligned16(p.v)) return false;
  for (int i = 0; i < 3; ++i)
    if (p.qs[i] % 8 || p.ks[i] % 8 || p.vs[i] % 8) return false;
  if (p.q_rms_eps >= 0.f && p.q_rms_weight && !aligned16(p.q_rms_weight)) return false;
  return true;
}

int decode_mfma_tile() { return kDN; }
int decode_mfma_max_tiles() { return kMaxTiles; }

int launch_decode_mfma(const SdpaParams& p, hipStream_t s) {
  return p.D == 128 ? launch_d<128>(p, s) : launch_d<64>(p, s);
}

}  // namespace mfx
