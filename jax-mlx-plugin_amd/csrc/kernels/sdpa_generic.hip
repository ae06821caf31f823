// Shape-general SDPA: any head size up to 256, any strides whose feature
// stride is 1, f32, bf16 or f16, causal / additive mask / GQA / fused q RMSNorm.
// One wavefront per query row; keys stream in chunks of 64 (one score per
// lane, online softmax per chunk), values accumulate with each lane owning
// features lane, lane+64, ...  This kernel covers the shapes the MFMA and
// split-KV kernels do not take; it is correct, not fast.
#include "sdpa_common.h"

namespace mfx {
namespace {

constexpr int kMaxD = 256;

template <typename T>
__global__ __launch_bounds__(64) void generic_kernel(SdpaParams p) {
  __shared__ float q_lds[kMaxD];
  __shared__ float p_lds[64];
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int t = (int)(row % p.Tq);
  const int bh = (int)(row / p.Tq);
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h / p.group;
  const int D = p.D, Dv = p.Dv;

  const T* qrow = static_cast<const T*>(p.q) + b * p.qs[0] + h * p.qs[1] + t * p.qs[2];
  float ss = 0.f;
  for (int d = lane; d < D; d += 64) {
    const float x = to_f32(qrow[d]);
    q_lds[d] = x;
    ss += x * x;
  }
  ss = group_sum<64>(ss);
  __syncthreads();
  if (p.q_rms_eps >= 0.f) {
    const float inv = rsqrtf(ss / (float)D + p.q_rms_eps);
    for (int d = lane; d < D; d += 64) {
      float x = q_lds[d] * inv;
      if (p.q_rms_weight) x *= to_f32(static_cast<const T*>(p.q_rms_weight)[d]);
      q_lds[d] = to_f32(from_f32<T>(x));
    }
    __syncthreads();
  }

  const T* kbase = static_cast<const T*>(p.k) + b * p.ks[0] + hk * p.ks[1];
  const T* vbase = static_cast<const T*>(p.v) + b * p.vs[0] + hk * p.vs[1];
  float o[kMaxD / 64];
#pragma unroll
  for (int j = 0; j < kMaxD / 64; ++j) o[j] = 0.f;
  float m = -INFINITY, l = 0.f;

  for (int kb = 0; kb < p.Tk; kb += 64) {
    const int key = kb + lane;
    float s = -INFINITY;
    if (key < p.Tk && !(p.causal && key > t)) {
      const T* krow = kbase + (int64_t)key * p.ks[2];
      float acc = 0.f;
      for (int d = 0; d < D; ++d) acc += q_lds[d] * to_f32(krow[d]);
      s = acc * p.scale_log2;
      if (p.mask)
        s += mask_log2(load_mask(p.mask, p.mask_dtype,
                                b * p.ms[0] + h * p.ms[1] + t * p.ms[2] + key * p.ms[3]));
    }
    const float mx = group_max<64>(s);
    const float m_new = fmaxf(m, mx);
    const float bse = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m - bse);
    const float pk = exp2f(s - bse);
    m = m_new;
    l = l * alpha + group_sum<64>(pk);
#pragma unroll
    for (int j = 0; j < kMaxD / 64; ++j) o[j] *= alpha;
    p_lds[lane] = pk;
    __syncthreads();
    const int n = min(64, p.Tk - kb);
    for (int j = 0; j < n; ++j) {
      const float pj = p_lds[j];
      const T* vrow = vbase + (int64_t)(kb + j) * p.vs[2];
#pragma unroll
      for (int jj = 0; jj < kMaxD / 64; ++jj) {
        const int d = lane + jj * 64;
        if (d < Dv) o[jj] += pj * to_f32(vrow[d]);
      }
    }
    __syncthreads();
  }
  if (p.lse && lane == 0) p.lse[row] = m + __log2f(l);
  T* orow = static_cast<T*>(p.out) + b * p.os[0] + h * p.os[1] + t * p.os[2];
#pragma unroll
  for (int jj = 0; jj < kMaxD / 64; ++jj) {
    const int d = lane + jj * 64;
    if (d < Dv) orow[d] = from_f32<T>(o[jj] / l);
  }
}

}  // namespace

int launch_generic(const SdpaParams& p, hipStream_t s) {
  if (p.D > kMaxD || p.Dv > kMaxD)
    return fail(MFX_E_UNSUPPORTED, "head size above 256 is not supported");
  const int64_t rows = (int64_t)p.B * p.Hq * p.Tq;
  if (p.dtype == MFX_BF16)
    hipLaunchKernelGGL((generic_kernel<bf16>), dim3((unsigned)rows), dim3(64), 0, s, p);
  else if (p.dtype == MFX_F16)
    hipLaunchKernelGGL((generic_kernel<_Float16>), dim3((unsigned)rows), dim3(64), 0, s, p);
  else
    hipLaunchKernelGGL((generic_kernel<float>), dim3((unsigned)rows), dim3(64), 0, s, p);
  return launch_status("generic_kernel");
}

}  // namespace mfx
