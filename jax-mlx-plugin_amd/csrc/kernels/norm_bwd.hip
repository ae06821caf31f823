// LayerNorm backward over the last axis, the arithmetic of the reference's
// custom_call @mlx_layer_norm_bwd (src/jax_mlx_pjrt.cpp:8237-8281, an
// mx::vjp of fast::layer_norm; closed form src/jax_mlx/layer_norm.py:59-76):
//
//   xhat = (x - mean) * inv,  inv = 1 / sqrt(var + eps)   (population var)
//   dxh  = dy * gamma
//   dx   = inv * (dxh - mean(dxh) - xhat * mean(dxh * xhat))
//   dgamma = sum_rows(dy * xhat),  dbeta = sum_rows(dy)
//
// Pass 1 (ln_bwd_rows): a row is owned by 16 / 64 lanes of a wavefront or by
// a 256-thread workgroup, as in the forward kernel; 16- and 64-lane groups
// take rows in pairs with both rows' loads in flight together.  x and dy are
// read once into registers as 16-byte vectors; mean and variance are recomputed from x
// (two passes over registers), dx is written once.  Each lane keeps running
// dgamma / dbeta sums for the columns it owns across every row its group
// visits, and the workgroup folds its groups into one fp32 partial row pair
// (workspace [G][2][n]).  Pass 2 (ln_bwd_params) sums the G partials per
// column.  HBM traffic: x and dy read once, dx written once, plus
// 2 * G * n * 4 bytes of partials written and read back.
#include "rowvec.h"

namespace mfx {
namespace {

using namespace rowvec;

constexpr int kMaxPartials = 1024;
constexpr int kParamWaves = 16;

template <typename T, typename PT, int LANES, int NV>
__global__ __launch_bounds__(kBlock) void ln_bwd_rows(
    const T* __restrict__ x, const T* __restrict__ dy, T* __restrict__ dx,
    const void* __restrict__ gamma, float* __restrict__ partial, int64_t rows, int n,
    int64_t xs, int64_t gs, int64_t dxs, float eps) {
  constexpr int VEC = Vec16<T>::N;
  typedef typename Vec16<T>::type V;
  constexpr int RPB = kBlock / LANES;
  __shared__ float lds[2 * (kBlock / 64)];
  __shared__ float fold[RPB > 1 ? RPB * LANES * NV * VEC : 1];

  const int lane = threadIdx.x % LANES;
  const int grp = threadIdx.x / LANES;
  const int nvec = n / VEC;
  const float inv_n = 1.0f / (float)n;

  float gv[NV][VEC];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = min(i * LANES + lane, nvec - 1);
    if (gamma) load_params<PT, VEC>(gamma, vi * VEC, gv[i]);
    else
#pragma unroll
      for (int j = 0; j < VEC; ++j) gv[i][j] = 1.f;
  }
  float ag[NV][VEC], ab[NV][VEC];
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int j = 0; j < VEC; ++j) ag[i][j] = ab[i][j] = 0.f;

  // With 16 or 64 lanes per row, rows come in pairs (row, row + stride): both
  // rows' x and dy loads are issued before either row's reductions, so a
  // wavefront keeps two rows of reads in flight.  With LANES == 256 the
  // whole workgroup owns each row and the reductions synchronise through
  // LDS, so the loop bound is uniform per workgroup.
  const int64_t stride = (int64_t)gridDim.x * RPB;
  auto load_row = [&](int64_t row, bool valid, float (&xv)[NV][VEC], float (&g)[NV][VEC]) {
    const V* xr = reinterpret_cast<const V*>(x + row * xs);
    const V* gr = reinterpret_cast<const V*>(dy + row * gs);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int vi = i * LANES + lane;
      if (valid && vi < nvec) {
        unpack16<T>(xr[vi], xv[i]);
        unpack16<T>(gr[vi], g[i]);
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) xv[i][j] = g[i][j] = 0.f;
      }
    }
  };
  auto finish_row = [&](int64_t row, bool valid, float (&xv)[NV][VEC], float (&g)[NV][VEC]) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) s += xv[i][j];
    const float mean = row_reduce<LANES, false>(s, lds) * inv_n;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const bool in = (i * LANES + lane) < nvec;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        xv[i][j] = in ? xv[i][j] - mean : 0.f;
        q += xv[i][j] * xv[i][j];
      }
    }
    const float inv = rsqrtf(row_reduce<LANES, false>(q, lds) * inv_n + eps);
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        xv[i][j] *= inv;  // xhat (0 for an absent row, whose dy is 0 too)
        const float d = g[i][j] * gv[i][j];
        s1 += d;
        s2 += d * xv[i][j];
        ag[i][j] = fmaf(g[i][j], xv[i][j], ag[i][j]);
        ab[i][j] += g[i][j];
      }
    row_reduce_sum2<LANES>(s1, s2, lds);
    const float m1 = s1 * inv_n, m2 = s2 * inv_n;
    if (!valid) return;
    V* dr = reinterpret_cast<V*>(dx + row * dxs);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int vi = i * LANES + lane;
      if (vi >= nvec) continue;
      float o[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) o[j] = inv * (g[i][j] * gv[i][j] - m1 - xv[i][j] * m2);
      dr[vi] = pack16<T>(o);
    }
  };
  if constexpr (LANES <= 64) {
    for (int64_t row = (int64_t)blockIdx.x * RPB + grp; row < rows; row += 2 * stride) {
      const bool second = row + stride < rows;
      float xa[NV][VEC], ga[NV][VEC], xb[NV][VEC], gb[NV][VEC];
      load_row(row, true, xa, ga);
      load_row(row + stride, second, xb, gb);
      finish_row(row, true, xa, ga);
      finish_row(row + stride, second, xb, gb);
    }
  } else {
    // A 256-lane row already has 256 x NV 16-byte loads in flight, and a
    // second row's registers would cost occupancy.
    for (int64_t row = blockIdx.x; row < rows; row += stride) {
      const V* xr = reinterpret_cast<const V*>(x + row * xs);
      const V* gr = reinterpret_cast<const V*>(dy + row * gs);
      float xv[NV][VEC], g[NV][VEC];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int vi = i * LANES + lane;
        if (vi < nvec) {
          unpack16<T>(xr[vi], xv[i]);
          unpack16<T>(gr[vi], g[i]);
        } else {
#pragma unroll
          for (int j = 0; j < VEC; ++j) xv[i][j] = g[i][j] = 0.f;
        }
      }
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j) s += xv[i][j];
      const float mean = row_reduce<LANES, false>(s, lds) * inv_n;
      float q = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const bool in = (i * LANES + lane) < nvec;
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          xv[i][j] = in ? xv[i][j] - mean : 0.f;
          q += xv[i][j] * xv[i][j];
        }
      }
      const float inv = rsqrtf(row_reduce<LANES, false>(q, lds) * inv_n + eps);
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          xv[i][j] *= inv;  // xhat
          const float d = g[i][j] * gv[i][j];
          s1 += d;
          s2 += d * xv[i][j];
          ag[i][j] = fmaf(g[i][j], xv[i][j], ag[i][j]);
          ab[i][j] += g[i][j];
        }
      row_reduce_sum2<LANES>(s1, s2, lds);
      const float m1 = s1 * inv_n, m2 = s2 * inv_n;
      V* dr = reinterpret_cast<V*>(dx + row * dxs);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int vi = i * LANES + lane;
        if (vi >= nvec) continue;
        float o[VEC];
#pragma unroll
        for (int j = 0; j < VEC; ++j) o[j] = inv * (g[i][j] * gv[i][j] - m1 - xv[i][j] * m2);
        dr[vi] = pack16<T>(o);
      }
    }
  }

  if (!partial) return;
  float* pg = partial + (int64_t)blockIdx.x * 2 * n;
  float* pb = pg + n;
  if constexpr (RPB == 1) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int vi = i * LANES + lane;
      if (vi >= nvec) continue;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        pg[vi * VEC + j] = ag[i][j];
        pb[vi * VEC + j] = ab[i][j];
      }
    }
  } else {
    // Fold the RPB groups: fold[grp][column], columns of this group's lanes.
    constexpr int W = LANES * NV * VEC;  // columns one group covers (>= n)
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
      for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j)
          fold[grp * W + (i * LANES + lane) * VEC + j] = pass == 0 ? ag[i][j] : ab[i][j];
      __syncthreads();
      float* dst = pass == 0 ? pg : pb;
      for (int c = threadIdx.x; c < n; c += kBlock) {
        float t = 0.f;
#pragma unroll
        for (int r = 0; r < RPB; ++r) t += fold[r * W + c];
        dst[c] = t;
      }
      __syncthreads();
    }
  }
}

// Rows that are unaligned or longer than the register-resident variants: the
// workgroup walks rows blockIdx.x, blockIdx.x + G, ...; thread t owns columns
// t, t + 256, ... of the block's partial rows, which it updates in place
// (no other thread touches them).
template <typename T>
__global__ __launch_bounds__(kBlock) void ln_bwd_rows_looped(
    const T* __restrict__ x, const T* __restrict__ dy, T* __restrict__ dx,
    const void* __restrict__ gamma, int pdt, float* __restrict__ partial, int64_t rows,
    int64_t n, int64_t xs, int64_t gs, int64_t dxs, float eps) {
  __shared__ float lds[kBlock / 64];
  float* pg = partial ? partial + (int64_t)blockIdx.x * 2 * n : nullptr;
  float* pb = pg ? pg + n : nullptr;
  if (pg)
    for (int64_t c = threadIdx.x; c < n; c += kBlock) pg[c] = pb[c] = 0.f;
  const float inv_n = 1.0f / (float)n;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const T* xr = x + row * xs;
    const T* gr = dy + row * gs;
    float s = 0.f;
    for (int64_t c = threadIdx.x; c < n; c += kBlock) s += to_f32(xr[c]);
    const float mean = row_reduce<kBlock, false>(s, lds) * inv_n;
    float q = 0.f;
    for (int64_t c = threadIdx.x; c < n; c += kBlock) {
      const float d = to_f32(xr[c]) - mean;
      q += d * d;
    }
    const float inv = rsqrtf(row_reduce<kBlock, false>(q, lds) * inv_n + eps);
    float s1 = 0.f, s2 = 0.f;
    for (int64_t c = threadIdx.x; c < n; c += kBlock) {
      const float xh = (to_f32(xr[c]) - mean) * inv;
      const float g = to_f32(gr[c]);
      const float d = g * (gamma ? load_param(gamma, pdt, (int)c) : 1.f);
      s1 += d;
      s2 += d * xh;
      if (pg) {
        pg[c] = fmaf(g, xh, pg[c]);
        pb[c] += g;
      }
    }
    const float m1 = row_reduce<kBlock, false>(s1, lds) * inv_n;
    const float m2 = row_reduce<kBlock, false>(s2, lds) * inv_n;
    T* dr = dx + row * dxs;
    for (int64_t c = threadIdx.x; c < n; c += kBlock) {
      const float xh = (to_f32(xr[c]) - mean) * inv;
      const float d = to_f32(gr[c]) * (gamma ? load_param(gamma, pdt, (int)c) : 1.f);
      dr[c] = from_f32<T>(inv * (d - m1 - xh * m2));
    }
  }
}

// dgamma[c] = sum_p partial[p][0][c], dbeta[c] = sum_p partial[p][1][c]:
// 64 columns per workgroup, its 16 wavefronts split the partial rows.
template <typename PT>
__global__ __launch_bounds__(64 * kParamWaves) void ln_bwd_params(
    const float* __restrict__ partial, int G, int64_t n, PT* __restrict__ dgamma,
    PT* __restrict__ dbeta) {
  __shared__ float red[2][kParamWaves][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  float sg = 0.f, sb = 0.f;
  if (c < n) {
    for (int p = w; p < G; p += kParamWaves) {
      sg += partial[(int64_t)p * 2 * n + c];
      sb += partial[(int64_t)p * 2 * n + n + c];
    }
  }
  red[0][w][lane] = sg;
  red[1][w][lane] = sb;
  __syncthreads();
  if (w == 0 && c < n) {
    float tg = 0.f, tb = 0.f;
#pragma unroll
    for (int i = 0; i < kParamWaves; ++i) {
      tg += red[0][i][lane];
      tb += red[1][i][lane];
    }
    if (dgamma) dgamma[c] = from_f32<PT>(tg);
    if (dbeta) dbeta[c] = from_f32<PT>(tb);
  }
}

struct BwdPlan {
  bool vector = false;
  int lanes = 0, nv = 0;
  int64_t groups = 0;  // G: workgroups of pass 1 = partial row pairs
};

int vec_of(int dt) { return dt == MFX_F32 ? 4 : 8; }

BwdPlan plan_bwd(const mfx_norm_bwd_args& a) {
  BwdPlan p;
  const int VEC = vec_of(a.dtype);
  const int es = a.dtype == MFX_F32 ? 4 : 2;
  const int pbytes = a.param_dtype == MFX_F32 ? 4 : 2;
  const int palign = VEC * pbytes > 16 ? 16 : VEC * pbytes;
  const bool aligned = a.n % VEC == 0 && a.x_row_stride % VEC == 0 && a.dy_row_stride % VEC == 0 &&
                       a.dx_row_stride % VEC == 0 && (uintptr_t)a.x % 16 == 0 &&
                       (uintptr_t)a.dy % 16 == 0 && (uintptr_t)a.dx % 16 == 0 &&
                       (!a.gamma || (uintptr_t)a.gamma % palign == 0) &&
                       // Vector kernels read gamma stored as f32 or as bf16
                       // (f16 rows: f32 or f16).
                       (!a.gamma || a.param_dtype == MFX_F32 ||
                        a.param_dtype == (a.dtype == MFX_F16 ? MFX_F16 : MFX_BF16));
  const int64_t nvec = a.n / VEC;
  (void)es;
  // Register budget: at most 16 fp32 values per lane per row array.
  const int maxnv = 16 / VEC;
  static const int kLanes[3] = {16, 64, 256};
  if (aligned) {
    for (int li = 0; li < 3 && !p.vector; ++li)
      for (int nv = 1; nv <= maxnv; nv *= 2)
        if (nvec <= (int64_t)kLanes[li] * nv) {
          p.vector = true;
          p.lanes = kLanes[li];
          p.nv = nv;
          break;
        }
  }
  const int64_t rpb = p.vector ? kBlock / p.lanes : 1;
  // At least two rows per group, at most kMaxPartials partial row pairs.
  int64_t g = (a.rows + 2 * rpb - 1) / (2 * rpb);
  p.groups = g < 1 ? 1 : (g > kMaxPartials ? kMaxPartials : g);
  return p;
}

template <typename T, typename PT, int LANES, int NV>
void launch_rows_bwd(const mfx_norm_bwd_args& a, const BwdPlan& p, float* partial, hipStream_t s) {
  hipLaunchKernelGGL((ln_bwd_rows<T, PT, LANES, NV>), dim3((unsigned)p.groups), dim3(kBlock), 0, s,
                     static_cast<const T*>(a.x), static_cast<const T*>(a.dy), static_cast<T*>(a.dx),
                     a.gamma, partial, a.rows, (int)a.n, a.x_row_stride, a.dy_row_stride, a.dx_row_stride,
                     a.eps);
}

template <typename T, typename PT>
void dispatch_rows_bwd(const mfx_norm_bwd_args& a, const BwdPlan& p, float* partial, hipStream_t s) {
  constexpr int VEC = Vec16<T>::N;
#define MFX_LN_BWD_CASE(L, N)                                             \
  if (p.lanes == L && p.nv == N) {                                        \
    if constexpr (N * VEC <= 16) return launch_rows_bwd<T, PT, L, N>(a, p, partial, s); \
  }
  MFX_LN_BWD_CASE(16, 1)
  MFX_LN_BWD_CASE(16, 2)
  MFX_LN_BWD_CASE(16, 4)
  MFX_LN_BWD_CASE(64, 1)
  MFX_LN_BWD_CASE(64, 2)
  MFX_LN_BWD_CASE(64, 4)
  MFX_LN_BWD_CASE(256, 1)
  MFX_LN_BWD_CASE(256, 2)
  MFX_LN_BWD_CASE(256, 4)
#undef MFX_LN_BWD_CASE
}

size_t partial_bytes(const mfx_norm_bwd_args& a, const BwdPlan& p) {
  if ((!a.dgamma && !a.dbeta) || a.rows == 0) return 0;
  return (size_t)p.groups * 2 * (size_t)a.n * sizeof(float);
}

const char* validate(const mfx_norm_bwd_args* a) {
  if (!a) return "null args";
  if (a->rows < 0 || a->n <= 0) return "rows must be >= 0 and n > 0";
  if (a->rows > 0x7fffffffLL || a->n > 0x7fffffffLL) return "rows or n too large";
  if (a->rows > 0 && (!a->x || !a->dy || !a->dx)) return "x, dy and dx must be non-null";
  if (a->x_row_stride < a->n || a->dy_row_stride < a->n || a->dx_row_stride < a->n)
    return "row strides must be >= n";
  if (a->dtype != MFX_F32 && a->dtype != MFX_BF16 && a->dtype != MFX_F16) return "dtype must be f32, bf16 or f16";
  if ((a->gamma || a->dgamma || a->dbeta) && a->param_dtype != MFX_F32 && a->param_dtype != MFX_BF16 &&
      a->param_dtype != MFX_F16)
    return "param_dtype must be f32, bf16 or f16";
  if (!(a->eps >= 0.f)) return "eps must be >= 0";
  return nullptr;
}

}  // namespace
}  // namespace mfx

extern "C" {

size_t mfx_layer_norm_bwd_workspace_size(const mfx_norm_bwd_args* args) {
  using namespace mfx;
  if (validate(args)) return 0;
  return partial_bytes(*args, plan_bwd(*args));
}

int mfx_layer_norm_bwd(const mfx_norm_bwd_args* args, void* stream) {
  using namespace mfx;
  if (const char* e = validate(args)) return fail(MFX_E_INVALID, e);
  const mfx_norm_bwd_args& a = *args;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const BwdPlan p = plan_bwd(a);
  const size_t need = a.rows ? partial_bytes(a, p) : 0;
  float* partial = nullptr;
  if (need) {
    if (a.workspace) {
      if (a.workspace_bytes < need)
        return fail(MFX_E_WORKSPACE, "workspace smaller than mfx_layer_norm_bwd_workspace_size()");
      if ((uintptr_t)a.workspace % 4) return fail(MFX_E_INVALID, "workspace must be 4-byte aligned");
      partial = static_cast<float*>(a.workspace);
    } else {
      partial = static_cast<float*>(device_scratch(need, s));
      if (!partial) return MFX_E_HIP;
    }
  }
  if (a.rows == 0) {
    // Empty batch: the parameter gradients are empty sums (pass 2 with G = 0).
  } else if (p.vector) {
    const bool p16 = a.param_dtype != MFX_F32 && a.gamma;  // the row type's 16-bit kind (plan_bwd)
    if (a.dtype == MFX_F32) {
      if (p16) dispatch_rows_bwd<float, bf16>(a, p, partial, s);
      else dispatch_rows_bwd<float, float>(a, p, partial, s);
    } else if (a.dtype == MFX_F16) {
      if (p16) dispatch_rows_bwd<_Float16, _Float16>(a, p, partial, s);
      else dispatch_rows_bwd<_Float16, float>(a, p, partial, s);
    } else {
      if (p16) dispatch_rows_bwd<bf16, bf16>(a, p, partial, s);
      else dispatch_rows_bwd<bf16, float>(a, p, partial, s);
    }
    if (int rc = launch_status("ln_bwd_rows")) return rc;
  } else {
    if (a.dtype == MFX_F32)
      hipLaunchKernelGGL((ln_bwd_rows_looped<float>), dim3((unsigned)p.groups), dim3(kBlock), 0, s,
                         static_cast<const float*>(a.x), static_cast<const float*>(a.dy),
                         static_cast<float*>(a.dx), a.gamma, a.param_dtype, partial, a.rows, a.n,
                         a.x_row_stride, a.dy_row_stride, a.dx_row_stride, a.eps);
    else if (a.dtype == MFX_F16)
      hipLaunchKernelGGL((ln_bwd_rows_looped<_Float16>), dim3((unsigned)p.groups), dim3(kBlock), 0, s,
                         static_cast<const _Float16*>(a.x), static_cast<const _Float16*>(a.dy),
                         static_cast<_Float16*>(a.dx), a.gamma, a.param_dtype, partial, a.rows, a.n,
                         a.x_row_stride, a.dy_row_stride, a.dx_row_stride, a.eps);
    else
      hipLaunchKernelGGL((ln_bwd_rows_looped<bf16>), dim3((unsigned)p.groups), dim3(kBlock), 0, s,
                         static_cast<const bf16*>(a.x), static_cast<const bf16*>(a.dy),
                         static_cast<bf16*>(a.dx), a.gamma, a.param_dtype, partial, a.rows, a.n,
                         a.x_row_stride, a.dy_row_stride, a.dx_row_stride, a.eps);
    if (int rc = launch_status("ln_bwd_rows_looped")) return rc;
  }
  if (!a.dgamma && !a.dbeta) return MFX_OK;
  const int G = a.rows == 0 ? 0 : (int)p.groups;
  const unsigned blocks = (unsigned)((a.n + 63) / 64);
  if (a.param_dtype == MFX_F32)
    hipLaunchKernelGGL((ln_bwd_params<float>), dim3(blocks), dim3(64 * kParamWaves), 0, s, partial, G, a.n,
                       static_cast<float*>(a.dgamma), static_cast<float*>(a.dbeta));
  else if (a.param_dtype == MFX_F16)
    hipLaunchKernelGGL((ln_bwd_params<_Float16>), dim3(blocks), dim3(64 * kParamWaves), 0, s, partial, G, a.n,
                       static_cast<_Float16*>(a.dgamma), static_cast<_Float16*>(a.dbeta));
  else
    hipLaunchKernelGGL((ln_bwd_params<bf16>), dim3(blocks), dim3(64 * kParamWaves), 0, s, partial, G, a.n,
                       static_cast<bf16*>(a.dgamma), static_cast<bf16*>(a.dbeta));
  return launch_status("ln_bwd_params");
}

}  // extern "C"
