// Split-KV attention for few query rows per kv head (GQA / MQA decode).
//
// The R = (Hq/Hkv) * Tq query rows that share one kv head are processed
// together, so each K/V row is read from HBM once for all of them.  Keys are
// split over a grid of (splits, B*Hkv) workgroups; inside a workgroup, groups
// of LPK lanes own one key row each (16-byte loads, a 256-byte bf16 row per
// 16-lane group), walking U consecutive keys per step.  Each group keeps an
// online softmax per query row; the groups of a workgroup merge through LDS
// and the splits merge in decode_combine_kernel.
//
// The path is HBM-bound: keys whose additive mask is -inf for every row (and
// keys past a causal limit) are skipped before their K/V bytes are loaded, so
// a padded cache costs only the bytes of its valid prefix.
//
// Optional fused RMSNorm of the query rows (reference chain rms_norm -> sdpa
// of GQA decode): q is normalised in fp32, rounded to the input type, then
// scaled by scale*log2(e) for exp2-based softmax.
#include "sdpa_common.h"

namespace mfx {
namespace {

constexpr int kNT = 256;
constexpr int kU = 4;  // consecutive keys per group step

template <typename T>
struct Lanes {
  static constexpr int ELEMS = 16 / sizeof(T);
};

template <typename T>
__device__ __forceinline__ void unpack(const u32x4& w, float* out);
template <>
__device__ __forceinline__ void unpack<bf16>(const u32x4& w, float* out) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void unpack<_Float16>(const u32x4& w, float* out) {
  // Halves taken with integer shifts: a bit_cast of each dword to a 2 x f16
  // vector compiles (f16 -> f32 folded into v_fma_mix) to products that all
  // read the first dword.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t x = w[i];
    out[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, (uint16_t)(x & 0xffffu)));
    out[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, (uint16_t)(x >> 16)));
  }
}
template <>
__device__ __forceinline__ void unpack<float>(const u32x4& w, float* out) {
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(w[i]);
}

template <typename T, int D, int R, bool MASK, bool CAUSAL>
__global__ __launch_bounds__(kNT) void decode_kernel(SdpaParams p) {
  constexpr int E = Lanes<T>::ELEMS;
  constexpr int LPK = D / E;
  constexpr int GROUPS = kNT / LPK;
  __shared__ float lds_o[GROUPS * R * D];
  __shared__ float lds_ml[GROUPS * R * 2];

  const int tid = threadIdx.x;
  const int li = tid % LPK;
  const int g = tid / LPK;
  const int split = blockIdx.x;
  const int bhk = blockIdx.y;
  const int b = bhk / p.Hkv, hk = bhk % p.Hkv;
  const int Tq = p.Tq;
  const int rows = p.group * Tq;

  int hq[R], tr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int rr = r < rows ? r : rows - 1;
    hq[r] = hk * p.group + rr / Tq;
    tr[r] = rr % Tq;
  }

  // Query rows in fp32, optional RMSNorm, folded softmax scale.
  float qv[R][E];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const T* qrow = static_cast<const T*>(p.q) + b * p.qs[0] + hq[r] * p.qs[1] + tr[r] * p.qs[2];
    u32x4 w = *reinterpret_cast<const u32x4*>(qrow + li * E);
    unpack<T>(w, qv[r]);
  }
  if (p.q_rms_eps >= 0.f) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) ss += qv[r][e] * qv[r][e];
      ss = group_sum<LPK>(ss);
      const float inv = rsqrtf(ss / (float)D + p.q_rms_eps);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        float t = qv[r][e] * inv;
        if (p.q_rms_weight) t *= to_f32(static_cast<const T*>(p.q_rms_weight)[li * E + e]);
        qv[r][e] = to_f32(from_f32<T>(t));
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int e = 0; e < E; ++e) qv[r][e] *= p.scale_log2;

  const T* kp = static_cast<const T*>(p.k) + b * p.ks[0] + hk * p.ks[1] + li * E;
  const T* vp = static_cast<const T*>(p.v) + b * p.vs[0] + hk * p.vs[1] + li * E;
  const int64_t ks2 = p.ks[2], vs2 = p.vs[2];
  const int kbeg = split * p.split_len;
  const int kend = min(p.Tk, kbeg + p.split_len);

  float m[R], l[R], o[R][E];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) o[r][e] = 0.f;
  }

  for (int base = kbeg + g * kU; base < kend; base += GROUPS * kU) {
    float mv[kU][R];
    bool use[kU];
    bool any = false;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int key = base + u;
      bool uu = false;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float x = (key < kend && r < rows) ? 0.f : -INFINITY;
        if constexpr (MASK) {
          if (x == 0.f)
            x = mask_log2(load_mask(p.mask, p.mask_dtype,
                                   b * p.ms[0] + hq[r] * p.ms[1] + tr[r] * p.ms[2] + key * p.ms[3]));
        }
        if (CAUSAL && key > tr[r]) x = -INFINITY;
        mv[u][r] = x;
        uu |= x != -INFINITY;
      }
      use[u] = uu;
      any |= uu;
    }
    if (!any) continue;  // uniform across the LPK lanes of the group

    u32x4 kw[kU], vw[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (use[u]) {
        kw[u] = *reinterpret_cast<const u32x4*>(kp + (int64_t)(base + u) * ks2);
        vw[u] = *reinterpret_cast<const u32x4*>(vp + (int64_t)(base + u) * vs2);
      } else {
        kw[u] = u32x4{0u, 0u, 0u, 0u};
        vw[u] = u32x4{0u, 0u, 0u, 0u};
      }
    }

    float s[kU][R];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      float kf[E];
      unpack<T>(kw[u], kf);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) acc += qv[r][e] * kf[e];
        s[u][r] = acc;
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int r = 0; r < R; ++r) s[u][r] = group_sum<LPK>(s[u][r]) + mv[u][r];

#pragma unroll
    for (int r = 0; r < R; ++r) {
      float mx = s[0][r];
#pragma unroll
      for (int u = 1; u < kU; ++u) mx = fmaxf(mx, s[u][r]);
      const float m_new = fmaxf(m[r], mx);
      const float bse = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m[r] - bse);
      m[r] = m_new;
      l[r] *= alpha;
#pragma unroll
      for (int e = 0; e < E; ++e) o[r][e] *= alpha;
#pragma unroll
      for (int u = 0; u < kU; ++u) s[u][r] = __builtin_amdgcn_exp2f(s[u][r] - bse);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      float vf[E];
      unpack<T>(vw[u], vf);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        l[r] += s[u][r];
#pragma unroll
        for (int e = 0; e < E; ++e) o[r][e] += s[u][r] * vf[e];
      }
    }
  }

  // Merge the GROUPS partial softmaxes of this workgroup.
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int e = 0; e < E; ++e) lds_o[(g * R + r) * D + li * E + e] = o[r][e];
    if (li == 0) {
      lds_ml[(g * R + r) * 2] = m[r];
      lds_ml[(g * R + r) * 2 + 1] = l[r];
    }
  }
  __syncthreads();

  const int rows_total = p.B * p.Hq * Tq;
  for (int idx = tid; idx < rows * D; idx += kNT) {
    const int r = idx / D, d = idx % D;
    float M = -INFINITY;
    for (int gg = 0; gg < GROUPS; ++gg) M = fmaxf(M, lds_ml[(gg * R + r) * 2]);
    const float bse = M == -INFINITY ? 0.f : M;
    float L = 0.f, O = 0.f;
    for (int gg = 0; gg < GROUPS; ++gg) {
      const float w = __builtin_amdgcn_exp2f(lds_ml[(gg * R + r) * 2] - bse);
      L += w * lds_ml[(gg * R + r) * 2 + 1];
      O += w * lds_o[(gg * R + r) * D + d];
    }
    const int hqr = hk * p.group + r / Tq, t = r % Tq;
    const int64_t row = ((int64_t)b * p.Hq + hqr) * Tq + t;
    if (p.num_splits == 1) {
      T* orow = static_cast<T*>(p.out) + b * p.os[0] + hqr * p.os[1] + t * p.os[2];
      orow[d] = from_f32<T>(O / L);
    } else {
      float* part = p.partial + ((int64_t)split * rows_total + row) * (D + 2);
      if (d == 0) {
        part[0] = M;
        part[1] = L;
      }
      part[2 + d] = O;
    }
  }
}

// Merges the split partials (m, l, O) of one output row per wavefront: lane
// s holds split s's (m, l) (64 splits per pass), the base and the weights
// come from two wave reductions, and each lane then sums its D/64 output
// columns over the splits with the weights broadcast from their lanes.
template <typename T>
__global__ __launch_bounds__(256) void decode_combine_kernel(SdpaParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (b*Hq + h)*Tq + t
  const int64_t rows_total = (int64_t)p.B * p.Hq * p.Tq;
  if (row >= rows_total) return;
  const int D = p.Dv, S = p.num_splits;
  const int64_t stride = rows_total * (D + 2);
  const float* base = p.partial + row * (D + 2);
  float M = -INFINITY;
  for (int s0 = 0; s0 < S; s0 += 64)
    if (s0 + lane < S) M = fmaxf(M, base[(s0 + lane) * stride]);
  M = group_max<64>(M);
  const float bse = M == -INFINITY ? 0.f : M;
  float L = 0.f;
  for (int s0 = 0; s0 < S; s0 += 64)
    if (s0 + lane < S) L += __builtin_amdgcn_exp2f(base[(s0 + lane) * stride] - bse) * base[(s0 + lane) * stride + 1];
  L = group_sum<64>(L);
  const int t = (int)(row % p.Tq);
  const int bh = (int)(row / p.Tq);
  const int b = bh / p.Hq, h = bh % p.Hq;
  T* orow = static_cast<T*>(p.out) + b * p.os[0] + h * p.os[1] + t * p.os[2];
  float acc[4] = {0.f, 0.f, 0.f, 0.f};  // columns lane, lane+64, ... (D <= 256)
  const int nc = (D + 63) / 64;
  for (int s0 = 0; s0 < S; s0 += 64) {
    const float w = s0 + lane < S ? __builtin_amdgcn_exp2f(base[(s0 + lane) * stride] - bse) : 0.f;
    const int n = min(64, S - s0);
    // Sixteen splits per batch: their loads are independent and issued
    // together, so a row costs a few L2 round trips, not one per split.
    for (int j0 = 0; j0 < n; j0 += 16) {
      float ov[16][4];
#pragma unroll
      for (int j = 0; j < 16; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c)
          ov[j][c] = (j0 + j < n && c < nc && c * 64 + lane < D) ? base[(s0 + j0 + j) * stride + 2 + c * 64 + lane] : 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float wj = __shfl(w, min(j0 + j, 63), 64);
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] += wj * ov[j][c];
      }
    }
  }
  const float inv = 1.0f / L;
#pragma unroll
  for (int c = 0; c < 4; ++c)
    if (c * 64 + lane < D) orow[c * 64 + lane] = from_f32<T>(acc[c] * inv);
}

template <typename T, int D, int R, bool MASK, bool CAUSAL>
int launch_t(const SdpaParams& p, hipStream_t s) {
  dim3 grid((unsigned)p.num_splits, (unsigned)(p.B * p.Hkv));
  hipLaunchKernelGGL((decode_kernel<T, D, R, MASK, CAUSAL>), grid, dim3(kNT), 0, s, p);
  int rc = launch_status("decode_kernel");
  if (rc != MFX_OK || p.num_splits == 1) return rc;
  return launch_decode_combine(p, s);
}

template <typename T, int D, int R>
int launch_r(const SdpaParams& p, hipStream_t s) {
  const bool m = p.mask != nullptr;
  if (p.causal) return m ? launch_t<T, D, R, true, true>(p, s) : launch_t<T, D, R, false, true>(p, s);
  return m ? launch_t<T, D, R, true, false>(p, s) : launch_t<T, D, R, false, false>(p, s);
}

template <typename T, int D>
int launch_d(const SdpaParams& p, hipStream_t s) {
  const int rows = p.group * p.Tq;
  if (rows <= 1) return launch_r<T, D, 1>(p, s);
  if (rows <= 2) return launch_r<T, D, 2>(p, s);
  if (rows <= 4) return launch_r<T, D, 4>(p, s);
  return launch_r<T, D, 8>(p, s);
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace

bool decode_supports(const SdpaParams& p) {
  if (p.dtype != MFX_BF16 && p.dtype != MFX_F16 && p.dtype != MFX_F32) return false;
  if (p.D != p.Dv || (p.D != 64 && p.D != 128)) return false;
  if (p.group * p.Tq > 8) return false;
  if (!aligned16(p.q) || !aligned16(p.k) || !aligned16(p.v)) return false;
  const int e = p.dtype == MFX_F32 ? 4 : 8;
  for (int i = 0; i < 3; ++i)
    if (p.qs[i] % e || p.ks[i] % e || p.vs[i] % e) return false;
  return true;
}

int launch_decode_combine(const SdpaParams& p, hipStream_t s) {
  const unsigned blocks = (unsigned)(((int64_t)p.B * p.Hq * p.Tq + 3) / 4);
  if (p.dtype == MFX_BF16)
    hipLaunchKernelGGL((decode_combine_kernel<bf16>), dim3(blocks), dim3(256), 0, s, p);
  else if (p.dtype == MFX_F16)
    hipLaunchKernelGGL((decode_combine_kernel<_Float16>), dim3(blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((decode_combine_kernel<float>), dim3(blocks), dim3(256), 0, s, p);
  return launch_status("decode_combine_kernel");
}

int launch_decode(const SdpaParams& p, hipStream_t s) {
  if (p.dtype == MFX_BF16) return p.D == 128 ? launch_d<bf16, 128>(p, s) : launch_d<bf16, 64>(p, s);
  if (p.dtype == MFX_F16) return p.D == 128 ? launch_d<_Float16, 128>(p, s) : launch_d<_Float16, 64>(p, s);
  return p.D == 128 ? launch_d<float, 128>(p, s) : launch_d<float, 64>(p, s);
}

}  // namespace mfx
