// Flash attention forward, bf16 inputs, fp32 accumulation, gfx950 MFMA.
//
// Workgroup = 4 wavefronts = 128 query rows of one (batch, head); each
// wavefront owns 32 query rows.  K/V stream through LDS in 64-key tiles,
// double-buffered, with the global loads of tile t+1 in flight while tile t
// is computed.
//
// Both products use v_mfma_f32_32x32x16_bf16 and are arranged so that the
// online softmax needs almost no cross-lane traffic:
//   S^T = K Q^T   A = K tile rows (from LDS), B = Q rows (registers).  The
//                 32x32 accumulator gives lane l query (l % 32) and 16 keys,
//                 so a query's row max / sum is 16 in-lane values plus one
//                 exchange with lane l ^ 32.
//   O^T = V^T P^T A = V^T (LDS holds the V tile transposed), B = P taken
//                 straight from the S^T accumulator: the contraction index
//                 (key) is permuted identically in A and B, so the
//                 accumulator registers are already the B operand.
// Each lane also owns one query of O^T, so the online-softmax rescale is a
// per-lane scalar multiply.
//
// Causal tiles past a wavefront's last query are skipped; the blockIdx ->
// (head, q-block) map runs the longest causal blocks first and keeps the
// q-blocks of one head on one XCD (blocks are dealt to the 8 XCDs
// round-robin), so its K/V stay in that XCD's L2.
#include "sdpa_common.h"

namespace mfx {
namespace {

constexpr int kBM = 128;  // query rows per workgroup
constexpr int kBN = 64;   // keys per tile
constexpr int kNT = 256;  // threads per workgroup

template <int D>
struct Cfg {
  static constexpr int KROW = D + 8;                  // bf16 per K row in LDS (16 B pad)
  static constexpr int VROW = kBN + 4;                // bf16 per V^T row in LDS (8 B pad)
  static constexpr int CH = kBN * D / 8 / kNT;        // 16-byte chunks per thread per tile
  static constexpr int DCH = D / 8;                   // 16-byte chunks per row
};

__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return (a & 0xffffu) | (b << 16);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return (a >> 16) | (b & 0xffff0000u);
}

template <int D, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(kNT, 2) void flash_bf16_kernel(SdpaParams p) {
  using C = Cfg<D>;
  __shared__ __attribute__((aligned(16))) bf16 k_lds[2][kBN * C::KROW];
  __shared__ __attribute__((aligned(16))) bf16 vt_lds[2][D * C::VROW];

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
    const int xcd = id & 7, slot = id >> 3;
    bh = (slot / nmb) * 8 + xcd;
    mblk = nmb - 1 - slot % nmb;
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

  int kv_end = Tk;
  if (CAUSAL) kv_end = min(Tk, min(Tq, (mblk + 1) * kBM));
  const int ntiles = (kv_end + kBN - 1) / kBN;

  u32x4 kreg[C::CH];
  u32x4 vreg[C::CH];
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  const int vdc = tid % C::DCH;  // V chunk column (d / 8)
  const int vkg = tid / C::DCH;  // V key group (C::CH keys)

  auto gload = [&](int t) {
    const int kb = t * kBN;
#pragma unroll
    for (int i = 0; i < C::CH; ++i) {
      const int c = tid + i * kNT;
      const int row = c / C::DCH, col = c % C::DCH;
      const int key = kb + row;
      u32x4 raw = *reinterpret_cast<const u32x4*>(kp + (int64_t)min(key, Tk - 1) * ks2 + col * 8);
      kreg[i] = key < Tk ? raw : zero4;
    }
#pragma unroll
    for (int r = 0; r < C::CH; ++r) {
      const int key = kb + vkg * C::CH + r;
      u32x4 raw = *reinterpret_cast<const u32x4*>(vp + (int64_t)min(key, Tk - 1) * vs2 + vdc * 8);
      vreg[r] = key < Tk ? raw : zero4;
    }
  };

  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < C::CH; ++i) {
      const int c = tid + i * kNT;
      const int row = c / C::DCH, col = c % C::DCH;
      *reinterpret_cast<u32x4*>(&k_lds[buf][row * C::KROW + col * 8]) = kreg[i];
    }
    // Transpose: vreg[r] holds d = vdc*8 .. +7 of key vkg*CH + r.
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      bf16* dst = &vt_lds[buf][(vdc * 8 + j) * C::VROW + vkg * C::CH];
      uint32_t w[C::CH];
#pragma unroll
      for (int r = 0; r < C::CH; ++r) {
        w[r] = vreg[r][j >> 1];
      }
      if constexpr (C::CH == 4) {
        u32x2 pk;
        pk[0] = (j & 1) ? pack_hi(w[0], w[1]) : pack_lo(w[0], w[1]);
        pk[1] = (j & 1) ? pack_hi(w[2], w[3]) : pack_lo(w[2], w[3]);
        *reinterpret_cast<u32x2*>(dst) = pk;
      } else {
        *reinterpret_cast<uint32_t*>(dst) = (j & 1) ? pack_hi(w[0], w[1]) : pack_lo(w[0], w[1]);
      }
    }
  };

  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float sl2 = p.scale_log2;

  if (ntiles > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) gload(t + 1);
    const int kb = t * kBN;
    const bool active = (q0 < Tq) && (!CAUSAL || kb <= q0 + 31);
    if (active) {
      f32x16 s[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) s[mt][i] = 0.f;
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(
              &k_lds[buf][(mt * 32 + l32) * C::KROW + kk * 16 + half * 8]);
          s[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], s[mt], 0, 0, 0);
        }
      }
      const bool edge = (kb + kBN > Tk) || (CAUSAL && kb + kBN - 1 > q0);
      float mx = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float x = s[mt][i] * sl2;
          const int key = kb + mt * 32 + (i >> 2) * 8 + half * 4 + (i & 3);
          if constexpr (MASK) {
            if (qi < Tq && key < Tk)
              x += kLog2e * load_mask(p.mask, p.mask_dtype,
                                      b * p.ms[0] + h * p.ms[1] + qi * p.ms[2] + key * p.ms[3]);
          }
          if (edge && (key >= Tk || (CAUSAL && key > qi))) x = -INFINITY;
          s[mt][i] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float base = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - base);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
      bf16x8 pb[4];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float pv = __builtin_amdgcn_exp2f(s[mt][i] - base);
          l_run += pv;
          pb[mt * 2 + (i >> 3)][i & 7] = static_cast<bf16>(pv);
        }
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16* vr = &vt_lds[buf][(dt * 32 + l32) * C::VROW + ks * 16 + half * 4];
          const bf16x4 lo = *reinterpret_cast<const bf16x4*>(vr);
          const bf16x4 hi = *reinterpret_cast<const bf16x4*>(vr + 8);
          const bf16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[ks], o[dt], 0, 0, 0);
        }
    }
    if (t + 1 < ntiles) lstore(buf ^ 1);
    __syncthreads();
  }

  const float lt = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = 1.0f / lt;
  if (qi < Tq) {
    bf16* orow = op + qi * os2;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = static_cast<bf16>(o[dt][g * 4 + e] * inv);
        *reinterpret_cast<bf16x4*>(orow + dt * 32 + g * 8 + half * 4) = w;
      }
  }
}

template <int D, bool CAUSAL, bool MASK>
int launch_t(const SdpaParams& p, hipStream_t s) {
  const int nmb = (p.Tq + kBM - 1) / kBM;
  const int64_t blocks = (int64_t)nmb * p.B * p.Hq;
  hipLaunchKernelGGL((flash_bf16_kernel<D, CAUSAL, MASK>), dim3((unsigned)blocks), dim3(kNT), 0,
                     s, p);
  return launch_status("flash_bf16_kernel");
}

template <int D>
int launch_d(const SdpaParams& p, hipStream_t s) {
  const bool m = p.mask != nullptr;
  if (p.causal) return m ? launch_t<D, true, true>(p, s) : launch_t<D, true, false>(p, s);
  return m ? launch_t<D, false, true>(p, s) : launch_t<D, false, false>(p, s);
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace

bool flash_bf16_supports(const SdpaParams& p) {
  if (p.dtype != MFX_BF16) return false;
  if (p.D != p.Dv || (p.D != 64 && p.D != 128)) return false;
  if (!aligned16(p.q) || !aligned16(p.k) || !aligned16(p.v) || !aligned16(p.out)) return false;
  for (int i = 0; i < 3; ++i)
    if (p.qs[i] % 8 || p.ks[i] % 8 || p.vs[i] % 8 || p.os[i] % 4) return false;
  if (p.os[2] % 4) return false;
  return true;
}

int launch_flash_bf16(const SdpaParams& p, hipStream_t s) {
  if (p.D == 128) return launch_d<128>(p, s);
  return launch_d<64>(p, s);
}

}  // namespace mfx
