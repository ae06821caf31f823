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

// 8-byte raw buffer load, bound to the LLVM intrinsic itself: this
// compiler's __builtin_amdgcn_raw_buffer_load_b64 lowers to a 4-byte load.
typedef float mfx_f32x2 __attribute__((ext_vector_type(2)));
__device__ mfx_f32x2 mfx_raw_buffer_load_f32x2(__amdgpu_buffer_rsrc_t rsrc, int voffset, int soffset, int aux) __asm(
    "llvm.amdgcn.raw.ptr.buffer.load.v2f32");

namespace mfx {
namespace {

constexpr int kBM = 128;
constexpr int kBN = 32;
constexpr int kNT = 256;

}  // namespace

// The key-split variant when 128-row workgroups would number fewer than two
// per CU and each wavefront of the split still has at most a few tiles.  Its
// buffer loads need rows that do not overlap (sequence stride >= D, so the
// rows past the end fall outside a tile's byte range) and 32 rows within a
// 32-bit byte range.
bool flash_f32_use_split(const SdpaParams& p) {
  const int64_t wgs = (int64_t)((p.Tq + 127) / 128) * p.B * p.Hq;
  if (p.D > 128) return false;  // head size 256: the row-block kernel only
  for (int64_t st : {p.qs[2], p.ks[2], p.vs[2]})
    if (st < p.D || st >= (int64_t(1) << 24)) return false;
  return wgs < 2LL * device_cu_count() && p.Tk <= 32 * 4 * 8;
}

namespace {

// Bytes from the first to the last valid element of `rows` rows of D floats
// at `stride` floats apart (0 when no row is valid).
template <int D>
__device__ __forceinline__ int rows_extent(int rows, int64_t stride) {
  return rows > 0 ? (int)(((int64_t)(rows - 1) * stride + D) * 4) : 0;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t f32_rsrc(const float* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, bytes, 0x00020000);
}

__device__ __forceinline__ f32x4 ld4(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

template <int D, bool MASK>
struct Cfg {
  static constexpr int KROW = D + 4;               // floats per K row (16 B pad)
  static constexpr int VROW = D + 8;               // floats per V row (32 B pad)
  static constexpr int DCH = D / 4;                // 16-byte chunks per row
  // Keys per LDS stage: two 32-key sub-tiles per barrier at D = 64 without
  // a mask (70 KB of LDS per workgroup, two workgroups per CU), one
  // otherwise (the masked kernel's extra state would spill).
  static constexpr int KS = (D == 64 && !MASK) ? 64 : 32;
  static constexpr int NSUB = KS / kBN;
  static constexpr int CH = KS * DCH / kNT;        // chunks per thread per stage
};

// Two workgroups per CU (256 VGPRs) except masked D = 96 and 128, whose
// extra mask state would spill at that bound, and D = 256 (Q and O alone
// take 256 registers; 134 KB of LDS).
template <int D, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(kNT, (D >= 256 || (D >= 96 && MASK)) ? 1 : 2) void flash_f32_kernel(SdpaParams p) {
  using C = Cfg<D, MASK>;
  __shared__ __attribute__((aligned(16))) float k_lds[2][C::KS * C::KROW];
  __shared__ __attribute__((aligned(16))) float v_lds[2][C::KS * C::VROW];

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

  // The exponent scale enters as |scale_log2| with its sign folded into Q
  // (negating Q negates every score exactly), so a row's largest scaled
  // score is |scale_log2| times its largest raw score.
  const float sl2 = fabsf(p.scale_log2);
  const float qsign = p.scale_log2 < 0.f ? -1.f : 1.f;

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
      for (int e = 0; e < 4; ++e) qf[c * 4 + e] = t[e] * qsign;
    }
  }

  int kv_end = Tk;
  if (CAUSAL) kv_end = min(Tk, min(Tq, (mblk + 1) * kBM));
  const int nstages = (kv_end + C::KS - 1) / C::KS;

  // K/V stages come through buffer resources spanning exactly the stage's
  // valid rows: rows past Tk read as zero (sequence stride >= D) or as
  // valid rows (overlapping rows), whose scores are masked either way.
  // Every lane's byte offsets are fixed for the whole kernel; the stage
  // moves the resource base.
  int koff[C::CH], voff[C::CH];
#pragma unroll
  for (int i = 0; i < C::CH; ++i) {
    const int c = tid + i * kNT;
    const int row = c / C::DCH, col = c % C::DCH;
    koff[i] = (int)((row * ks2 + col * 4) * 4);
    voff[i] = (int)((row * vs2 + col * 4) * 4);
  }
  f32x4 kreg[C::CH], vreg[C::CH];
  auto gload = [&](int st) {
    const int kb = st * C::KS;
    const int rows = min(C::KS, Tk - kb);
    const auto rk = f32_rsrc(kp + (int64_t)kb * ks2, rows_extent<D>(rows, ks2));
    const auto rv = f32_rsrc(vp + (int64_t)kb * vs2, rows_extent<D>(rows, vs2));
#pragma unroll
    for (int i = 0; i < C::CH; ++i) {
      kreg[i] = ld4(rk, koff[i]);
      vreg[i] = ld4(rv, voff[i]);
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
  // m_run: the exponent base of a row (log2 units), which trails the row's
  // running maximum by at most kSlack, so every exp2 is at most 2^kSlack.
  // O and l are rescaled only when some row's maximum passes its base by
  // more than that (a wavefront-uniform branch, rare after the first tile).
  constexpr float kSlack = 8.f;
  float m_run = -INFINITY, l_run = 0.f;

  if (nstages > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();

  for (int st = 0; st < nstages; ++st) {
    const int buf = st & 1;
    if (st + 1 < nstages) gload(st + 1);
#pragma unroll
    for (int u = 0; u < C::NSUB; ++u) {
      const int kb = st * C::KS + u * kBN;
      const float* kt = &k_lds[buf][u * kBN * C::KROW];
      const float* vt = &v_lds[buf][u * kBN * C::VROW];
      const bool active = kb < kv_end && (q0 < Tq) && (!CAUSAL || kb <= q0 + 31);
      if (active) {
        f32x16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.f;
        __builtin_amdgcn_s_setprio(3);
#pragma unroll
        for (int c = 0; c < D / 8; ++c) {
          const f32x4 a = *reinterpret_cast<const f32x4*>(&kt[l32 * C::KROW + c * 8 + half * 4]);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], qf[c * 4 + e], s, 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
        // Tiles with masked keys (additive mask, past Tk, causal diagonal)
        // form the scaled scores one by one; the others keep the raw scores
        // and fold the scale into the exponent's fma.
        const bool scaled = MASK || (kb + kBN > Tk) || (CAUSAL && kb + kBN - 1 > q0);
        float mx;
        if (scaled) {
          mx = -INFINITY;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            float x = s[i] * sl2;
            const int key = kb + (i >> 2) * 8 + half * 4 + (i & 3);
            if constexpr (MASK) {
              if (qi < Tq && key < Tk)
                x += mask_log2(load_mask(p.mask, p.mask_dtype,
                                        b * p.ms[0] + h * p.ms[1] + qi * p.ms[2] + key * p.ms[3]));
            }
            if (key >= Tk || (CAUSAL && key > qi)) x = -INFINITY;
            s[i] = x;
            mx = fmaxf(mx, x);
          }
        } else {
          float r = s[0];
#pragma unroll
          for (int i = 1; i < 16; ++i) r = fmaxf(r, s[i]);
          mx = r * sl2;
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const bool grow = mx > m_run + kSlack;
        if (__ballot(grow)) {
          const float m_new = grow ? mx : m_run;
          const float alpha = grow ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;
          m_run = m_new;
          l_run *= alpha;
#pragma unroll
          for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
        }
        const float base = m_run == -INFINITY ? 0.f : m_run;
        if (scaled) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            s[i] = __builtin_amdgcn_exp2f(s[i] - base);
            l_run += s[i];
          }
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            s[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], sl2, -base));
            l_run += s[i];
          }
        }
        __builtin_amdgcn_s_setprio(3);
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int kl = (i >> 2) * 8 + half * 4 + (i & 3);
            const float a = vt[kl * C::VROW + dt * 32 + l32];
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, s[i], o[dt], 0, 0, 0);
          }
        __builtin_amdgcn_s_setprio(0);
      }
    }
    if (st + 1 < nstages) lstore(buf ^ 1);
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

// Short-sequence variant: a workgroup owns 32 query rows and its 4
// wavefronts split the keys (wavefront w takes the 32-key tiles w, w+4, ...),
// each reading its K rows and V columns straight from global memory into
// MFMA operands (no LDS staging, no barrier in the loop).  The four partial
// (max, sum, O) triples merge through LDS at the end.  Used when the
// 128-row workgroups of flash_f32_kernel would leave most CUs idle (few
// heads times short sequences, e.g. [8,8,128,64]): it launches 4x the
// workgroups and 16x the wavefronts per query.
//
// Loads go through raw buffer resources spanning exactly the valid rows of
// one tile, so rows past Tq / Tk read as zero with no clamp or select, and
// every per-lane offset is fixed for the whole kernel (the tile moves the
// resource base, a scalar operation).
constexpr int kSW = 4;  // wavefronts (key splits) per workgroup

// NDT consecutive floats (NDT = 2 or 4).
template <int NDT>
__device__ __forceinline__ void ldn(__amdgpu_buffer_rsrc_t r, int off, float (&v)[NDT]) {
  if constexpr (NDT == 2) {
    const mfx_f32x2 x = mfx_raw_buffer_load_f32x2(r, off, 0, 0);
    v[0] = x[0];
    v[1] = x[1];
  } else {
    const f32x4 x = ld4(r, off);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = x[j];
  }
}

template <int D, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(64 * kSW) void flash_f32_split_kernel(SdpaParams p) {
  __shared__ float red_m[kSW][32], red_l[kSW][32];
  // [split][query][feature]; a 4-float pad keeps the 16-byte rows of one
  // ds_write_b128 on distinct banks.
  __shared__ __align__(16) float o_part[kSW][32][D + 4];
  __shared__ __align__(16) float q_lds[32][D + 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int l32 = lane & 31;

  const int nmb = (p.Tq + 31) / 32;
  const int bh = blockIdx.x / nmb, mblk = blockIdx.x % nmb;
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h / p.group;
  const float* qp = static_cast<const float*>(p.q) + b * p.qs[0] + h * p.qs[1];
  const float* kp = static_cast<const float*>(p.k) + b * p.ks[0] + hk * p.ks[1];
  const float* vp = static_cast<const float*>(p.v) + b * p.vs[0] + hk * p.vs[1];
  float* op = static_cast<float*>(p.out) + b * p.os[0] + h * p.os[1];
  const int64_t qs2 = p.qs[2], ks2 = p.ks[2], vs2 = p.vs[2], os2 = p.os[2];
  const int Tq = p.Tq, Tk = p.Tk;
  const int q0 = mblk * 32;
  const int qi = q0 + l32;

  int kv_end = Tk;
  if (CAUSAL) kv_end = min(Tk, min(Tq, q0 + 32));
  const int ntiles = (kv_end + 31) / 32;

  // Operand layouts as in flash_f32_kernel: the k-slot of MFMA step (c, e)
  // is feature c*8 + half*4 + e (Q row qi, K row kb + l32); for P^T slot i
  // the lane supplies the scores s[i] of keys key(i) = (i>>2)*8 + half*4 +
  // (i&3).  Row r of output tile dt (an O^T row) is feature r*NDT + dt, so a
  // lane's V^T operands for one key, V[kb + key(i)][l32*NDT + dt] over dt,
  // are NDT consecutive floats: one load per key.
  constexpr int NDT = D / 32;
  const int voff_k = (int)((l32 * ks2 + half * 4) * 4);
  int voff_v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) voff_v[i] = (int)((((i >> 2) * 8 + half * 4 + (i & 3)) * vs2 + l32 * NDT) * 4);
  float qf[D / 2];
  f32x4 kr[D / 8];
  float vr[16][NDT];
  auto issue_k = [&](int t) {
    const auto r = f32_rsrc(kp + (int64_t)t * 32 * ks2, rows_extent<D>(min(32, Tk - t * 32), ks2));
#pragma unroll
    for (int c = 0; c < D / 8; ++c) kr[c] = ld4(r, voff_k + c * 32);
  };
  auto issue_v = [&](int t) {
    const auto r = f32_rsrc(vp + (int64_t)t * 32 * vs2, rows_extent<D>(min(32, Tk - t * 32), vs2));
#pragma unroll
    for (int i = 0; i < 16; ++i) ldn<NDT>(r, voff_v[i], vr[i]);
  };
  // The four wavefronts share one copy of the 32 query rows: wavefront w
  // fetches rows 8w..8w+7 (lane -> row 8w + lane/8, 4 features at
  // (lane%8)*4 + 32j) into LDS and each then reads its MFMA operands back.
  {
    const auto r = f32_rsrc(qp + (int64_t)q0 * qs2, rows_extent<D>(min(32, Tq - q0), qs2));
    const int row = wave * 8 + (lane >> 3), col = (lane & 7) * 4;
    const int voff = (int)((row * qs2 + col) * 4);
#pragma unroll
    for (int j = 0; j < D / 32; ++j)
      *reinterpret_cast<f32x4*>(&q_lds[row][col + j * 32]) = ld4(r, voff + j * 128);
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < D / 8; ++c) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(&q_lds[l32][c * 8 + half * 4]);
#pragma unroll
    for (int e = 0; e < 4; ++e) qf[c * 4 + e] = t[e];
  }
  // Pipeline: K(t + kSW) is fetched once the S products of tile t are
  // issued and V(t + kSW) once its PV products are, so each fetch overlaps
  // the other half of the tile.  The scheduling fences keep the compiler
  // from sinking the loads next to their first use.  The first fetch is
  // unconditional (a wavefront without a tile fetches the last one and
  // skips the loop): behind a branch, the counter waits of the loop's first
  // products would have to assume the loads were skipped and wait for all
  // but the Q fetches.
  issue_k(min(wave, ntiles - 1));
  issue_v(min(wave, ntiles - 1));
  __builtin_amdgcn_sched_barrier(0);

  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float sl2 = p.scale_log2;
  const int64_t mrow = MASK ? b * p.ms[0] + h * p.ms[1] + (int64_t)min(qi, Tq - 1) * p.ms[2] : 0;

  for (int t = wave; t < ntiles; t += kSW) {
    const int kb = t * 32;
    const bool more = t + kSW < ntiles;
    f32x16 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.f;
#pragma unroll
    for (int c = 0; c < D / 8; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[c][e], qf[c * 4 + e], s, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (more) issue_k(t + kSW);
    __builtin_amdgcn_sched_barrier(0);
    const bool edge = (kb + 32 > Tk) || (CAUSAL && kb + 31 > q0);
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float x = s[i] * sl2;
      const int key = kb + (i >> 2) * 8 + half * 4 + (i & 3);
      if constexpr (MASK) {
        if (key < Tk) x += mask_log2(load_mask(p.mask, p.mask_dtype, mrow + key * p.ms[3]));
      }
      if (edge && (key >= Tk || (CAUSAL && key > qi))) x = -INFINITY;
      s[i] = x;
      mx = fmaxf(mx, x);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float base = m_new == -INFINITY ? 0.f : m_new;
    if (t != wave) {  // nothing accumulated before a wavefront's first tile
      const float alpha = __builtin_amdgcn_exp2f(m_run - base);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
    }
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = __builtin_amdgcn_exp2f(s[i] - base);
      l_run += s[i];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vr[i][dt], s[i], o[dt], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (more) issue_v(t + kSW);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Merge the kSW partials: per query row, M = max of the running maxima
  // (log2 units), L = sum_w l_w 2^(m_w - M), O = sum_w O_w 2^(m_w - M) / L.
  // Each wavefront scales its own O by 2^(m_w - M) / L before the exchange,
  // so the cross-wavefront step is a plain sum.  A row with no visible key
  // (L = 0) comes out as 0/0, as a softmax over an all -inf row does.
  const float lw = l_run + __shfl_xor(l_run, 32, 64);
  if (half == 0) {
    red_m[wave][l32] = m_run;
    red_l[wave][l32] = lw;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kSW; ++w) M = fmaxf(M, red_m[w][l32]);
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < kSW; ++w) {
    const float mw = red_m[w][l32];
    L += mw == -INFINITY ? 0.f : red_l[w][l32] * __builtin_amdgcn_exp2f(mw - M);
  }
  const float f = (m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - M)) / L;
  // Lane (half, l32) holds tile rows g*8 + half*4 + e (e = 0..3) of query
  // l32 in o[dt][g*4 + e], i.e. features (g*8 + half*4)*NDT + e*NDT + dt:
  // 4*NDT consecutive features per g.
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    float run[4 * NDT];
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) run[e * NDT + dt] = o[dt][g * 4 + e] * f;
#pragma unroll
    for (int j = 0; j < NDT; ++j)
      *reinterpret_cast<f32x4*>(&o_part[wave][l32][(g * 8 + half * 4) * NDT + j * 4]) =
          f32x4{run[j * 4], run[j * 4 + 1], run[j * 4 + 2], run[j * 4 + 3]};
  }
  if (p.lse && wave == 0 && half == 0 && qi < Tq) p.lse[(int64_t)bh * Tq + qi] = M + __log2f(L);
  __syncthreads();
  constexpr int C4 = D / 4;  // float4 columns per row
#pragma unroll
  for (int idx = tid; idx < 32 * C4; idx += 64 * kSW) {
    const int q = idx / C4, c = idx % C4;
    f32x4 acc = *reinterpret_cast<const f32x4*>(&o_part[0][q][c * 4]);
#pragma unroll
    for (int w = 1; w < kSW; ++w) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(&o_part[w][q][c * 4]);
      acc[0] += t[0];
      acc[1] += t[1];
      acc[2] += t[2];
      acc[3] += t[3];
    }
    if (q0 + q < Tq) *reinterpret_cast<f32x4*>(op + (int64_t)(q0 + q) * os2 + c * 4) = acc;
  }
}

template <int D, bool CAUSAL, bool MASK>
int launch_split(const SdpaParams& p, hipStream_t s) {
  const int64_t blocks = (int64_t)((p.Tq + 31) / 32) * p.B * p.Hq;
  hipLaunchKernelGGL((flash_f32_split_kernel<D, CAUSAL, MASK>), dim3((unsigned)blocks), dim3(64 * kSW), 0, s, p);
  return launch_status("flash_f32_split_kernel");
}

template <int D, bool CAUSAL, bool MASK>
int launch_t(const SdpaParams& p, hipStream_t s) {
  if constexpr (D <= 128)
    if (flash_f32_use_split(p)) return launch_split<D, CAUSAL, MASK>(p, s);
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
  if (p.D != p.Dv || (p.D != 32 && p.D != 64 && p.D != 96 && p.D != 128 && p.D != 256)) return false;
  if (!aligned16(p.q) || !aligned16(p.k) || !aligned16(p.v) || !aligned16(p.out)) return false;
  for (int i = 0; i < 3; ++i)
    if (p.qs[i] % 4 || p.ks[i] % 4 || p.vs[i] % 4 || p.os[i] % 4) return false;
  // K/V stages (up to 64 rows) are read through buffer resources with
  // 32-bit lane offsets.
  for (int64_t st : {p.ks[2], p.vs[2]})
    if (st < 0 || st >= (int64_t(1) << 23)) return false;
  return true;
}

int launch_flash_f32(const SdpaParams& p, hipStream_t s) {
  switch (p.D) {
    case 32: return launch_d<32>(p, s);
    case 96: return launch_d<96>(p, s);
    case 128: return launch_d<128>(p, s);
    case 256: return launch_d<256>(p, s);
    default: return launch_d<64>(p, s);
  }
}

}  // namespace mfx
