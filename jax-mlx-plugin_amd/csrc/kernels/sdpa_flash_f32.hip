// Flash attention forward, fp32 end to end, gfx950 fp32 MFMA
// (v_mfma_f32_32x32x2_f32: true fp32 products, no reduced-precision inputs).
//
// Same dataflow as the bf16 kernel: 4 wavefronts x 32 query rows per
// workgroup, S^T = K Q^T so a query's softmax lives in one lane pair, and
// O^T = V^T P^T with P consumed straight from the S^T accumulator.  With a
// K-depth of 2 per MFMA the contraction index of both products is permuted
// so that every LDS read is a 16-byte (K) or conflict-free 4-byte (V) access
// and V needs no transpose.  Tiles are 32 keys, double-buffered through LDS.
#include "sdpa_common.h"

namespace mfx {
namespace {

constexpr int kBM = 128;
constexpr int kBN = 32;
constexpr int kNT = 256;

template <int D>
struct Cfg {
  static constexpr int KROW = D + 4;               // floats per K row (16 B pad)
  static constexpr int VROW = D + 8;               // floats per V row (32 B pad)
  static constexpr int DCH = D / 4;                // 16-byte chunks per row
  static constexpr int CH = kBN * DCH / kNT;       // chunks per thread per tile
};

template <int D, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(kNT, 2) void flash_f32_kernel(SdpaParams p) {
  using C = Cfg<D>;
  __shared__ __attribute__((aligned(16))) float k_lds[2][kBN * C::KROW];
  __shared__ __attribute__((aligned(16))) float v_lds[2][kBN * C::VROW];

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
  const float* qp = static_cast<const float*>(p.q) + b * p.qs[0] + h * p.qs[1];
  const float* kp = static_cast<const float*>(p.k) + b * p.ks[0] + hk * p.ks[1];
  const float* vp = static_cast<const float*>(p.v) + b * p.vs[0] + hk * p.vs[1];
  float* op = static_cast<float*>(p.out) + b * p.os[0] + h * p.os[1];
  const int64_t qs2 = p.qs[2], ks2 = p.ks[2], vs2 = p.vs[2], os2 = p.os[2];
  const int Tq = p.Tq, Tk = p.Tk;

  const int q0 = mblk * kBM + wave * 32;
  const int qi = q0 + l32;

  // qf[c*4+e] = Q[qi][c*8 + half*4 + e]: the k-slot (half) of MFMA step
  // (c, e) is feature c*8 + half*4 + e, matched by the K reads below.
  float qf[D / 2];
  {
    const float* qrow = qp + (int64_t)min(qi, Tq - 1) * qs2 + half * 4;
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
      f32x4 t = *reinterpret_cast<const f32x4*>(qrow + c * 8);
      if (qi >= Tq) t = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) qf[c * 4 + e] = t[e];
    }
  }

  int kv_end = Tk;
  if (CAUSAL) kv_end = min(Tk, min(Tq, (mblk + 1) * kBM));
  const int ntiles = (kv_end + kBN - 1) / kBN;

  f32x4 kreg[C::CH], vreg[C::CH];
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  auto gload = [&](int t) {
    const int kb = t * kBN;
#pragma unroll
    for (int i = 0; i < C::CH; ++i) {
      const int c = tid + i * kNT;
      const int row = c / C::DCH, col = c % C::DCH;
      const int key = kb + row;
      const int64_t kr = (int64_t)min(key, Tk - 1);
      f32x4 a = *reinterpret_cast<const f32x4*>(kp + kr * ks2 + col * 4);
      f32x4 v = *reinterpret_cast<const f32x4*>(vp + kr * vs2 + col * 4);
      kreg[i] = key < Tk ? a : zero4;
      vreg[i] = key < Tk ? v : zero4;
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < C::CH; ++i) {
      const int c = tid + i * kNT;
      const int row = c / C::DCH, col = c % C::DCH;
      *reinterpret_cast<f32x4*>(&k_lds[buf][row * C::KROW + col * 4]) = kreg[i];
      *reinterpret_cast<f32x4*>(&v_lds[buf][row * C::VROW + col * 4]) = vreg[i];
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
      f32x16 s;
#pragma unroll
      for (int i = 0; i < 16; ++i) s[i] = 0.f;
#pragma unroll
      for (int c = 0; c < D / 8; ++c) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(&k_lds[buf][l32 * C::KROW + c * 8 + half * 4]);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          s = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], qf[c * 4 + e], s, 0, 0, 0);
      }
      const bool edge = (kb + kBN > Tk) || (CAUSAL && kb + kBN - 1 > q0);
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float x = s[i] * sl2;
        const int key = kb + (i >> 2) * 8 + half * 4 + (i & 3);
        if constexpr (MASK) {
          if (qi < Tq && key < Tk)
            x += mask_log2(load_mask(p.mask, p.mask_dtype,
                                    b * p.ms[0] + h * p.ms[1] + qi * p.ms[2] + key * p.ms[3]));
        }
        if (edge && (key >= Tk || (CAUSAL && key > qi))) x = -INFINITY;
        s[i] = x;
        mx = fmaxf(mx, x);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float base = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2f(m_run - base);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        s[i] = exp2f(s[i] - base);
        l_run += s[i];
      }
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kl = (i >> 2) * 8 + half * 4 + (i & 3);
          const float a = v_lds[buf][kl * C::VROW + dt * 32 + l32];
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, s[i], o[dt], 0, 0, 0);
        }
    }
    if (t + 1 < ntiles) lstore(buf ^ 1);
    __syncthreads();
  }

  const float lt = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = 1.0f / lt;
  if (p.lse && half == 0 && qi < Tq) p.lse[(int64_t)bh * Tq + qi] = m_run + __log2f(lt);
  if (qi < Tq) {
    float* orow = op + qi * os2;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = o[dt][g * 4 + e] * inv;
        *reinterpret_cast<f32x4*>(orow + dt * 32 + g * 8 + half * 4) = w;
      }
  }
}

template <int D, bool CAUSAL, bool MASK>
int launch_t(const SdpaParams& p, hipStream_t s) {
  const int nmb = (p.Tq + kBM - 1) / kBM;
  const int64_t blocks = (int64_t)nmb * p.B * p.Hq;
  hipLaunchKernelGGL((flash_f32_kernel<D, CAUSAL, MASK>), dim3((unsigned)blocks), dim3(kNT), 0, s,
                     p);
  return launch_status("flash_f32_kernel");
}

template <int D>
int launch_d(const SdpaParams& p, hipStream_t s) {
  const bool m = p.mask != nullptr;
  if (p.causal) return m ? launch_t<D, true, true>(p, s) : launch_t<D, true, false>(p, s);
  return m ? launch_t<D, false, true>(p, s) : launch_t<D, false, false>(p, s);
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace

bool flash_f32_supports(const SdpaParams& p) {
  if (p.dtype != MFX_F32) return false;
  if (p.D != p.Dv || (p.D != 64 && p.D != 128)) return false;
  if (!aligned16(p.q) || !aligned16(p.k) || !aligned16(p.v) || !aligned16(p.out)) return false;
  for (int i = 0; i < 3; ++i)
    if (p.qs[i] % 4 || p.ks[i] % 4 || p.vs[i] % 4 || p.os[i] % 4) return false;
  return true;
}

int launch_flash_f32(const SdpaParams& p, hipStream_t s) {
  if (p.D == 128) return launch_d<128>(p, s);
  return launch_d<64>(p, s);
}

}  // namespace mfx
