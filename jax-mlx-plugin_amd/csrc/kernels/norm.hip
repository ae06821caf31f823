// Row-reduction kernels for gfx950: LayerNorm, RMSNorm and softmax over the
// last axis.
//
// A row is owned by 16 or 64 lanes of one wavefront (rows up to 1024
// 16-byte vectors, i.e. 4096 f32 / 8192 bf16 or f16 elements) or by a 256-thread
// workgroup (up to 4096 vectors); longer or unaligned rows take a looped
// fallback.  Each element is read from HBM once and written once -- the HBM
// roofline's algorithmic traffic.
#include "rowvec.h"

namespace mfx {
namespace {

using namespace rowvec;

enum class RowOp { kLayerNorm, kRmsNorm, kSoftmax, kLogSoftmax };

constexpr bool is_softmax(RowOp op) { return op == RowOp::kSoftmax || op == RowOp::kLogSoftmax; }

// One row per LANES threads (16 or 64 lanes of one wavefront, or a whole
// 256-thread workgroup).  Each lane loads NV 16-byte vectors with consecutive
// lanes on consecutive vectors, so every load instruction of a wavefront
// covers 1 KiB of contiguous row data, and all of a row's loads are in flight
// before the first reduction.  The gamma / beta slices a lane needs are
// loaded as vectors of their storage type PT right after the row (L2 hits
// after the first rows), so the epilogue is pure FMA work.  The row stays in
// registers: LayerNorm is two-pass (mean, then sum of squared deviations)
// without re-reading HBM, so each element is read once and written once.
template <typename T, typename PT, int LANES, int NV, RowOp OP>
__global__ __launch_bounds__(kBlock) void row_kernel(
    const T* __restrict__ x, T* __restrict__ y, const void* __restrict__ gamma,
    const void* __restrict__ beta, int64_t rows, int n, int64_t xs, int64_t ys, float eps) {
  constexpr int VEC = Vec16<T>::N;
  typedef typename Vec16<T>::type V;
  constexpr int ROWS_PER_BLOCK = kBlock / LANES;
  constexpr bool kParams = !is_softmax(OP);
  __shared__ float lds[kBlock / 64];

  const int lane = threadIdx.x % LANES;
  const int64_t row = (int64_t)blockIdx.x * ROWS_PER_BLOCK + threadIdx.x / LANES;
  const bool row_ok = row < rows;
  const int nvec = n / VEC;

  const V* xr = reinterpret_cast<const V*>(x + (row_ok ? row : 0) * xs);
  float v[NV][VEC];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = i * LANES + lane;
    if (row_ok && vi < nvec) {
      unpack16<T>(xr[vi], v[i]);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[i][j] = is_softmax(OP) ? -INFINITY : 0.f;
    }
  }
  float gv[kParams ? NV : 1][VEC], bv[kParams && OP == RowOp::kLayerNorm ? NV : 1][VEC];
  if constexpr (kParams) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int vi = min(i * LANES + lane, nvec - 1);
      if (gamma) load_params<PT, VEC>(gamma, vi * VEC, gv[i]);
      else
#pragma unroll
        for (int j = 0; j < VEC; ++j) gv[i][j] = 1.f;
      if constexpr (OP == RowOp::kLayerNorm) {
        if (beta) load_params<PT, VEC>(beta, vi * VEC, bv[i]);
        else
#pragma unroll
          for (int j = 0; j < VEC; ++j) bv[i][j] = 0.f;
      }
    }
  }

  const float inv_n = 1.0f / (float)n;
  float scale_or_max = 0.f, shift = 0.f;
  if constexpr (OP == RowOp::kLayerNorm) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) s += v[i][j];
    const float mean = row_reduce<LANES, false>(s, lds) * inv_n;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const bool in = (i * LANES + lane) < nvec;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float d = v[i][j] - mean;
        q += in ? d * d : 0.f;
      }
    }
    const float var = row_reduce<LANES, false>(q, lds) * inv_n;
    scale_or_max = rsqrtf(var + eps);
    shift = mean;
  } else if constexpr (OP == RowOp::kRmsNorm) {
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) q += v[i][j] * v[i][j];
    const float ms = row_reduce<LANES, false>(q, lds) * inv_n;
    scale_or_max = rsqrtf(ms + eps);
  } else {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) m = fmaxf(m, v[i][j]);
    m = row_reduce<LANES, true>(m, lds);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float e = __expf(v[i][j] - m);
        if constexpr (OP == RowOp::kSoftmax) v[i][j] = e;
        s += e;
      }
    s = row_reduce<LANES, false>(s, lds);
    // softmax: 1 / sum;  log-softmax: the total shift max + log(sum).
    scale_or_max = OP == RowOp::kSoftmax ? 1.0f / s : m + logf(s);
  }

  if (!row_ok) return;
  V* yr = reinterpret_cast<V*>(y + row * ys);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = i * LANES + lane;
    if (vi >= nvec) continue;
    float o[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      if constexpr (OP == RowOp::kSoftmax) {
        o[j] = v[i][j] * scale_or_max;
      } else if constexpr (OP == RowOp::kLogSoftmax) {
        o[j] = v[i][j] - scale_or_max;
      } else if constexpr (OP == RowOp::kLayerNorm) {
        o[j] = fmaf((v[i][j] - shift) * scale_or_max, gv[i][j], bv[i][j]);
      } else {
        o[j] = v[i][j] * scale_or_max * gv[i][j];
      }
    }
    yr[vi] = pack16<T>(o);
  }
}

// Fallback for rows that are not 16-byte vectorisable or longer than the
// register-resident variants: one workgroup per row, scalar strided loops,
// three passes over the row.
template <typename T, RowOp OP>
__global__ __launch_bounds__(kBlock) void row_kernel_looped(
    const T* __restrict__ x, T* __restrict__ y, const void* __restrict__ gamma,
    const void* __restrict__ beta, int pdt, int64_t rows, int64_t n, int64_t xs,
    int64_t ys, float eps) {
  __shared__ float lds[kBlock / 64];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * xs;
  T* yr = y + row * ys;
  float a = 0.f, b = 0.f;
  if constexpr (OP == RowOp::kLayerNorm) {
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += kBlock) s += to_f32(xr[i]);
    const float mean = row_reduce<kBlock, false>(s, lds) / (float)n;
    float q = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += kBlock) {
      const float d = to_f32(xr[i]) - mean;
      q += d * d;
    }
    a = rsqrtf(row_reduce<kBlock, false>(q, lds) / (float)n + eps);
    b = mean;
  } else if constexpr (OP == RowOp::kRmsNorm) {
    float q = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += kBlock) {
      const float t = to_f32(xr[i]);
      q += t * t;
    }
    a = rsqrtf(row_reduce<kBlock, false>(q, lds) / (float)n + eps);
  } else {
    float m = -INFINITY;
    for (int64_t i = threadIdx.x; i < n; i += kBlock) m = fmaxf(m, to_f32(xr[i]));
    m = row_reduce<kBlock, true>(m, lds);
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += kBlock) s += __expf(to_f32(xr[i]) - m);
    s = row_reduce<kBlock, false>(s, lds);
    a = OP == RowOp::kSoftmax ? 1.0f / s : logf(s);
    b = m;
  }
  for (int64_t i = threadIdx.x; i < n; i += kBlock) {
    float t = to_f32(xr[i]);
    if constexpr (OP == RowOp::kSoftmax) {
      t = __expf(t - b) * a;
    } else if constexpr (OP == RowOp::kLogSoftmax) {
      t = t - (b + a);
    } else {
      t = (t - b) * a;
      if (gamma) t *= load_param(gamma, pdt, (int)i);
      if (OP == RowOp::kLayerNorm && beta) t += load_param(beta, pdt, (int)i);
    }
    yr[i] = from_f32<T>(t);
  }
}

template <typename T, typename PT, int LANES, int NV, RowOp OP>
int launch_rows(const mfx_norm_args& a, hipStream_t s) {
  constexpr int rpb = kBlock / LANES;
  const int64_t blocks = (a.rows + rpb - 1) / rpb;
  hipLaunchKernelGGL((row_kernel<T, PT, LANES, NV, OP>), dim3((unsigned)blocks), dim3(kBlock), 0, s,
                     static_cast<const T*>(a.x), static_cast<T*>(a.y), a.gamma, a.beta, a.rows, (int)a.n,
                     a.x_row_stride, a.y_row_stride, a.eps);
  return launch_status("row_kernel");
}

template <typename T, typename PT, RowOp OP>
int dispatch_vec(const mfx_norm_args& a, hipStream_t s, int64_t nvec) {
  if (nvec <= 16) return launch_rows<T, PT, 16, 1, OP>(a, s);
  if (nvec <= 32) return launch_rows<T, PT, 16, 2, OP>(a, s);
  if (nvec <= 64) return launch_rows<T, PT, 16, 4, OP>(a, s);
  if (nvec <= 128) return launch_rows<T, PT, 64, 2, OP>(a, s);
  if (nvec <= 256) return launch_rows<T, PT, 64, 4, OP>(a, s);
  if (nvec <= 512) return launch_rows<T, PT, 64, 8, OP>(a, s);
  if (nvec <= 1024) return launch_rows<T, PT, 64, 16, OP>(a, s);
  if (nvec <= 2048) return launch_rows<T, PT, 256, 8, OP>(a, s);
  return launch_rows<T, PT, 256, 16, OP>(a, s);
}

template <typename T, RowOp OP>
int dispatch_typed(const mfx_norm_args& a, hipStream_t s) {
  constexpr int VEC = Vec16<T>::N;
  const bool params = !is_softmax(OP) && (a.gamma || (OP == RowOp::kLayerNorm && a.beta));
  // Parameter vectors are read at element offsets that are multiples of VEC.
  const int pbytes = a.param_dtype == MFX_F32 ? 4 : 2;
  const bool params_aligned = !params || ((!a.gamma || (uintptr_t)a.gamma % (VEC * pbytes > 16 ? 16 : VEC * pbytes) == 0) &&
                                          (!a.beta || (uintptr_t)a.beta % (VEC * pbytes > 16 ? 16 : VEC * pbytes) == 0));
  const bool aligned = (a.n % VEC == 0) && (a.x_row_stride % VEC == 0) &&
                       (a.y_row_stride % VEC == 0) &&
                       ((uintptr_t)a.x % 16 == 0) && ((uintptr_t)a.y % 16 == 0) && params_aligned;
  const int64_t nvec = a.n / VEC;
  // Vector kernels read parameters stored as f32 or as bf16; f16 rows also
  // take f16 parameters.  Other pairings run the looped kernel.
  constexpr bool kF16 = std::is_same<T, _Float16>::value;
  const bool pvec = !params || a.param_dtype == MFX_F32 || a.param_dtype == (kF16 ? MFX_F16 : MFX_BF16);
  if (aligned && nvec <= 4096 && pvec) {
    if (params && a.param_dtype != MFX_F32) {
      if constexpr (kF16) return dispatch_vec<T, _Float16, OP>(a, s, nvec);
      else return dispatch_vec<T, bf16, OP>(a, s, nvec);
    }
    return dispatch_vec<T, float, OP>(a, s, nvec);
  }
  hipLaunchKernelGGL((row_kernel_looped<T, OP>), dim3((unsigned)a.rows), dim3(kBlock), 0, s,
                     static_cast<const T*>(a.x), static_cast<T*>(a.y), a.gamma, a.beta,
                     a.param_dtype, a.rows, a.n, a.x_row_stride, a.y_row_stride, a.eps);
  return launch_status("row_kernel_looped");
}

template <RowOp OP>
int dispatch(const mfx_norm_args* a, void* stream) {
  if (!a) return fail(MFX_E_INVALID, "null args");
  if (a->rows < 0 || a->n <= 0) return fail(MFX_E_INVALID, "rows must be >= 0 and n > 0");
  if (a->rows == 0) return MFX_OK;
  if (!a->x || !a->y) return fail(MFX_E_INVALID, "x and y must be non-null");
  if (a->x_row_stride < a->n || a->y_row_stride < a->n)
    return fail(MFX_E_INVALID, "row strides must be >= n");
  if (a->rows > 0x7fffffffLL) return fail(MFX_E_UNSUPPORTED, "too many rows");
  if (a->n > 0x7fffffffLL) return fail(MFX_E_UNSUPPORTED, "row too long");
  if ((a->gamma || a->beta) && a->param_dtype != MFX_F32 && a->param_dtype != MFX_BF16 && a->param_dtype != MFX_F16)
    return fail(MFX_E_UNSUPPORTED, "param_dtype must be f32, bf16 or f16");
  if (!is_softmax(OP) && !(a->eps >= 0.f))
    return fail(MFX_E_INVALID, "eps must be >= 0");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (a->dtype) {
    case MFX_F32: return dispatch_typed<float, OP>(*a, s);
    case MFX_BF16: return dispatch_typed<bf16, OP>(*a, s);
    case MFX_F16: return dispatch_typed<_Float16, OP>(*a, s);
    default: return fail(MFX_E_UNSUPPORTED, "dtype must be f32, bf16 or f16");
  }
}

}  // namespace
}  // namespace mfx

extern "C" {

int mfx_layer_norm(const mfx_norm_args* args, void* stream) {
  return mfx::dispatch<mfx::RowOp::kLayerNorm>(args, stream);
}

int mfx_rms_norm(const mfx_norm_args* args, void* stream) {
  return mfx::dispatch<mfx::RowOp::kRmsNorm>(args, stream);
}

int mfx_softmax(const mfx_norm_args* args, void* stream) {
  return mfx::dispatch<mfx::RowOp::kSoftmax>(args, stream);
}

int mfx_log_softmax(const mfx_norm_args* args, void* stream) {
  return mfx::dispatch<mfx::RowOp::kLogSoftmax>(args, stream);
}

}  // extern "C"
