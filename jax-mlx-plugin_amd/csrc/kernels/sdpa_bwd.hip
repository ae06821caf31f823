// mfx_sdpa_bwd: argument validation, the recomputed forward pass, the
// delta = rowsum(dO * O) pass and the shape-general backward kernels.
//
// Backward of out = softmax(s * Q K^T + M) V (reference closed form
// src/jax_mlx/sdpa.py:65-87, extended with the causal / additive masks and
// GQA of the forward):
//   P = exp2(s * log2e * Q K^T + log2e * M - lse)    (lse: row log2-sum-exp2)
//   dV = P^T dO,  dP = dO V^T,  dS = P * (dP - delta),  delta = rowsum(dO * O)
//   dQ = s * dS K,  dK = s * dS^T Q
// Order of work: forward (O and lse into the workspace), delta, then dK / dV
// and dQ (the matrix-core dQ kernel computes delta itself and runs before
// dK / dV, which read it).  dK / dV are owned per key row (summing the
// group's query heads) and dQ per query row, so no output is accumulated by
// two workgroups and the result is deterministic.
//
// The shape-general kernels here take any head size up to 256, f32, bf16 or
// f16, and every mask; one wavefront owns one output row and walks the other
// axis in chunks of 64 (one score per lane), then accumulates its row with
// lanes over features.  They are correct, not fast: bf16 and f16 with head
// size 64 / 128 run on the matrix-core kernels (sdpa_bwd_mfma.hip), and head
// sizes 32 / 96 too, on copies of q, k, v, dO and O zero-padded to 64 / 128
// features in the workspace (the padded features add zero to every score and
// to delta, and their gradients, zero, are not copied out).
#include <algorithm>
#include <cmath>

#include "sdpa_common.h"

namespace mfx {
namespace {

constexpr int kMaxD = 256;
constexpr int kFeat = kMaxD / 64;

template <typename T>
__global__ __launch_bounds__(256) void bwd_delta_kernel(SdpaBwdParams p, float* delta) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t rows = (int64_t)p.B * p.Hq * p.Tq;
  if (row >= rows) return;
  const int t = (int)(row % p.Tq);
  const int bh = (int)(row / p.Tq);
  const int b = bh / p.Hq, h = bh % p.Hq;
  const T* orow = static_cast<const T*>(p.o) + b * p.os[0] + h * p.os[1] + t * p.os[2];
  const T* grow = static_cast<const T*>(p.dout) + b * p.dos[0] + h * p.dos[1] + t * p.dos[2];
  float s = 0.f;
  for (int d = lane; d < p.Dv; d += 64) s += to_f32(orow[d]) * to_f32(grow[d]);
  s = group_sum<64>(s);
  if (lane == 0) delta[row] = s;
}

// Log2-domain score of (query i of head h, key j) given the dot product.
__device__ __forceinline__ float bwd_score(const SdpaBwdParams& p, float dot, int b, int h, int i, int j) {
  float x = dot * p.scale_log2;
  if (p.mask) x += mask_log2(load_mask(p.mask, p.mask_dtype, b * p.ms[0] + h * p.ms[1] + i * p.ms[2] + j * p.ms[3]));
  return x;
}

// dQ: one wavefront per query row (b, h, i).
template <typename T>
__global__ __launch_bounds__(64) void bwd_dq_generic(SdpaBwdParams p) {
  __shared__ float q_lds[kMaxD];
  __shared__ float g_lds[kMaxD];
  __shared__ float ds_lds[64];
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int i = (int)(row % p.Tq);
  const int bh = (int)(row / p.Tq);
  const int b = bh / p.Hq, h = bh % p.Hq, hk = h / p.group;
  const T* qrow = static_cast<const T*>(p.q) + b * p.qs[0] + h * p.qs[1] + i * p.qs[2];
  const T* grow = static_cast<const T*>(p.dout) + b * p.dos[0] + h * p.dos[1] + i * p.dos[2];
  for (int d = lane; d < p.D; d += 64) q_lds[d] = to_f32(qrow[d]);
  for (int d = lane; d < p.Dv; d += 64) g_lds[d] = to_f32(grow[d]);
  __syncthreads();
  const float lse = p.lse[row], dl = p.delta[row];
  const T* kbase = static_cast<const T*>(p.k) + b * p.ks[0] + hk * p.ks[1];
  const T* vbase = static_cast<const T*>(p.v) + b * p.vs[0] + hk * p.vs[1];
  float acc[kFeat];
#pragma unroll
  for (int f = 0; f < kFeat; ++f) acc[f] = 0.f;
  const int kend = p.causal ? min(p.Tk, i + 1) : p.Tk;
  for (int kb = 0; kb < kend; kb += 64) {
    const int j = kb + lane;
    float ds = 0.f;
    if (j < kend) {
      const T* krow = kbase + (int64_t)j * p.ks[2];
      const T* vrow = vbase + (int64_t)j * p.vs[2];
      float s = 0.f, dp = 0.f;
      for (int d = 0; d < p.D; ++d) s += q_lds[d] * to_f32(krow[d]);
      for (int d = 0; d < p.Dv; ++d) dp += g_lds[d] * to_f32(vrow[d]);
      const float pr = exp2f(bwd_score(p, s, b, h, i, j) - lse);
      ds = pr * (dp - dl);
    }
    ds_lds[lane] = ds;
    __syncthreads();
    const int n = min(64, kend - kb);
    for (int jj = 0; jj < n; ++jj) {
      const float w = ds_lds[jj];
      const T* krow = kbase + (int64_t)(kb + jj) * p.ks[2];
#pragma unroll
      for (int f = 0; f < kFeat; ++f) {
        const int d = lane + f * 64;
        if (d < p.D) acc[f] += w * to_f32(krow[d]);
      }
    }
    __syncthreads();
  }
  T* out = static_cast<T*>(p.dq) + b * p.dqs[0] + h * p.dqs[1] + i * p.dqs[2];
#pragma unroll
  for (int f = 0; f < kFeat; ++f) {
    const int d = lane + f * 64;
    if (d < p.D) out[d] = from_f32<T>(acc[f] * p.scale);
  }
}

// dK and dV: one wavefront per key row (b, hk, j), over every query row of
// the group's heads that sees key j.
template <typename T>
__global__ __launch_bounds__(64) void bwd_dkdv_generic(SdpaBwdParams p) {
  __shared__ float k_lds[kMaxD];
  __shared__ float v_lds[kMaxD];
  __shared__ float p_lds[64];
  __shared__ float ds_lds[64];
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int j = (int)(row % p.Tk);
  const int bhk = (int)(row / p.Tk);
  const int b = bhk / p.Hkv, hk = bhk % p.Hkv;
  const T* krow = static_cast<const T*>(p.k) + b * p.ks[0] + hk * p.ks[1] + j * p.ks[2];
  const T* vrow = static_cast<const T*>(p.v) + b * p.vs[0] + hk * p.vs[1] + j * p.vs[2];
  for (int d = lane; d < p.D; d += 64) k_lds[d] = to_f32(krow[d]);
  for (int d = lane; d < p.Dv; d += 64) v_lds[d] = to_f32(vrow[d]);
  __syncthreads();
  float dk[kFeat], dv[kFeat];
#pragma unroll
  for (int f = 0; f < kFeat; ++f) dk[f] = dv[f] = 0.f;
  const int qstart = p.causal ? j : 0;
  for (int g = 0; g < p.group; ++g) {
    const int h = hk * p.group + g;
    const T* qbase = static_cast<const T*>(p.q) + b * p.qs[0] + h * p.qs[1];
    const T* gbase = static_cast<const T*>(p.dout) + b * p.dos[0] + h * p.dos[1];
    const int64_t rbase = ((int64_t)b * p.Hq + h) * p.Tq;
    for (int qb = qstart; qb < p.Tq; qb += 64) {
      const int i = qb + lane;
      float pr = 0.f, ds = 0.f;
      if (i < p.Tq) {
        const T* qrow = qbase + (int64_t)i * p.qs[2];
        const T* grow = gbase + (int64_t)i * p.dos[2];
        float s = 0.f, dp = 0.f;
        for (int d = 0; d < p.D; ++d) s += to_f32(qrow[d]) * k_lds[d];
        for (int d = 0; d < p.Dv; ++d) dp += to_f32(grow[d]) * v_lds[d];
        pr = exp2f(bwd_score(p, s, b, h, i, j) - p.lse[rbase + i]);
        ds = pr * (dp - p.delta[rbase + i]);
      }
      p_lds[lane] = pr;
      ds_lds[lane] = ds;
      __syncthreads();
      const int n = min(64, p.Tq - qb);
      for (int ii = 0; ii < n; ++ii) {
        const float pw = p_lds[ii], dw = ds_lds[ii];
        const T* qrow = qbase + (int64_t)(qb + ii) * p.qs[2];
        const T* grow = gbase + (int64_t)(qb + ii) * p.dos[2];
#pragma unroll
        for (int f = 0; f < kFeat; ++f) {
          const int d = lane + f * 64;
          if (d < p.D) dk[f] += dw * to_f32(qrow[d]);
          if (d < p.Dv) dv[f] += pw * to_f32(grow[d]);
        }
      }
      __syncthreads();
    }
  }
  T* dko = static_cast<T*>(p.dk) + b * p.dks[0] + hk * p.dks[1] + j * p.dks[2];
  T* dvo = static_cast<T*>(p.dv) + b * p.dvs[0] + hk * p.dvs[1] + j * p.dvs[2];
#pragma unroll
  for (int f = 0; f < kFeat; ++f) {
    const int d = lane + f * 64;
    if (d < p.D) dko[d] = from_f32<T>(dk[f] * p.scale);
    if (d < p.Dv) dvo[d] = from_f32<T>(dv[f]);
  }
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Copies rows [rows][D] (element strides s0..s2 over (b, h, t), feature
// stride 1) into contiguous rows of Dp >= D features, the rest zero; or back
// (unpad: the first D features of each contiguous row to the strided rows).
// One thread per 16-byte chunk (D and Dp multiples of 8 elements).
template <bool UNPAD>
__global__ __launch_bounds__(256) void pad_rows_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                       int64_t rows, int D, int Dp, int H, int T, int64_t s0,
                                                       int64_t s1, int64_t s2) {
  const int cpr = Dp / 8;  // chunks per padded row
  const int64_t n = rows * cpr;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / cpr;
    const int c = (int)(i % cpr) * 8;
    const int t = (int)(r % T);
    const int64_t bh = r / T;
    const int64_t strided = (bh / H) * s0 + (bh % H) * s1 + t * s2 + c;
    if constexpr (UNPAD) {
      if (c < D) *reinterpret_cast<uint4*>(dst + strided) = *reinterpret_cast<const uint4*>(src + r * Dp + c);
    } else {
      uint4 v = {0u, 0u, 0u, 0u};
      if (c < D) v = *reinterpret_cast<const uint4*>(src + strided);
      *reinterpret_cast<uint4*>(dst + r * Dp + c) = v;
    }
  }
}

struct BwdPlan {
  SdpaBwdParams p{};
  SdpaParams fwd{};
  bool mfma = false;
  size_t o_bytes = 0, row_bytes = 0;  // workspace: O, then lse, then delta
  // Head size 32 / 96 on the matrix-core kernels: pp is p on rows padded to
  // dp features (q, k, v, dO, O and dq, dk, dv in the workspace after
  // delta; pointers bound at launch).
  int dp = 0;
  SdpaBwdParams pp{};
  size_t q_pad = 0, kv_pad = 0;  // bytes of one padded [B,Hq,Tq,dp] / [B,Hkv,Tk,dp] tensor
};

int make_bwd_plan(const mfx_sdpa_bwd_args* a, BwdPlan& out) {
  if (!a) return fail(MFX_E_INVALID, "null args");
  if (!a->q || !a->k || !a->v || !a->dout || !a->dq || !a->dk || !a->dv)
    return fail(MFX_E_INVALID, "q, k, v, dout, dq, dk and dv must be non-null");
  if (a->B <= 0 || a->Hq <= 0 || a->Hkv <= 0 || a->Tq <= 0 || a->Tk <= 0 || a->D <= 0 || a->Dv <= 0)
    return fail(MFX_E_INVALID, "B, Hq, Hkv, Tq, Tk, D and Dv must all be positive");
  if (a->Hq % a->Hkv != 0) return fail(MFX_E_INVALID, "Hq must be a multiple of Hkv");
  const int64_t lim = 0x7fffffffLL;
  if (a->B * a->Hq * a->Tq > lim || a->B * a->Hkv * a->Tk > lim)
    return fail(MFX_E_UNSUPPORTED, "problem too large for one launch");
  const int64_t* st[8] = {a->q_strides, a->k_strides, a->v_strides, a->do_strides,
                          a->dq_strides, a->dk_strides, a->dv_strides, nullptr};
  for (int i = 0; st[i]; ++i)
    if (st[i][3] != 1) return fail(MFX_E_INVALID, "feature (last) strides must be 1");
  if (a->dtype != MFX_F32 && a->dtype != MFX_BF16 && a->dtype != MFX_F16)
    return fail(MFX_E_UNSUPPORTED, "dtype must be f32, bf16 or f16");
  if (a->mask && a->mask_dtype != MFX_F32 && a->mask_dtype != MFX_BF16 && a->mask_dtype != MFX_F16)
    return fail(MFX_E_UNSUPPORTED, "mask dtype must be f32, bf16 or f16");
  if (!std::isfinite(a->scale)) return fail(MFX_E_INVALID, "scale must be finite");
  if ((a->fwd_out != nullptr) != (a->fwd_lse != nullptr))
    return fail(MFX_E_INVALID, "fwd_out and fwd_lse are passed together or not at all");
  const bool saved = a->fwd_out != nullptr;
  if (saved && a->fwd_out_strides[3] != 1) return fail(MFX_E_INVALID, "fwd_out feature stride must be 1");
  if (a->D > kMaxD || a->Dv > kMaxD) return fail(MFX_E_UNSUPPORTED, "head size above 256 is not supported");

  SdpaBwdParams& p = out.p;
  p.q = a->q;
  p.k = a->k;
  p.v = a->v;
  p.dout = a->dout;
  p.mask = a->mask;
  p.dq = a->dq;
  p.dk = a->dk;
  p.dv = a->dv;
  for (int i = 0; i < 4; ++i) {
    p.qs[i] = a->q_strides[i];
    p.ks[i] = a->k_strides[i];
    p.vs[i] = a->v_strides[i];
    p.dos[i] = a->do_strides[i];
    p.dqs[i] = a->dq_strides[i];
    p.dks[i] = a->dk_strides[i];
    p.dvs[i] = a->dv_strides[i];
    p.ms[i] = a->mask ? a->mask_strides[i] : 0;
  }
  p.B = (int)a->B;
  p.Hq = (int)a->Hq;
  p.Hkv = (int)a->Hkv;
  p.Tq = (int)a->Tq;
  p.Tk = (int)a->Tk;
  p.D = (int)a->D;
  p.Dv = (int)a->Dv;
  p.group = (int)(a->Hq / a->Hkv);
  p.mask_dtype = a->mask_dtype;
  p.dtype = a->dtype;
  p.causal = a->causal ? 1 : 0;
  p.scale = a->scale;
  p.scale_log2 = a->scale * kLog2e;
  // O: the caller's forward output, or the recomputed one (contiguous, in
  // the workspace, bound at launch).
  for (int i = 0; i < 4; ++i)
    p.os[i] = saved ? a->fwd_out_strides[i]
                    : (i == 0 ? (int64_t)p.Hq * p.Tq * p.Dv : i == 1 ? (int64_t)p.Tq * p.Dv : i == 2 ? p.Dv : 1);
  if (saved) {
    p.o = a->fwd_out;
    p.lse = a->fwd_lse;
  }

  const int64_t rows = (int64_t)p.B * p.Hq * p.Tq;
  out.o_bytes = saved ? 0 : align256((size_t)rows * p.Dv * dtype_size(p.dtype));
  out.row_bytes = align256((size_t)rows * sizeof(float));

  // The forward pass that regenerates O and lse: the flash kernels where they
  // apply (never the decode kernels, which do not produce lse), else generic.
  SdpaParams& f = out.fwd;
  f.q = p.q;
  f.k = p.k;
  f.v = p.v;
  f.mask = p.mask;
  for (int i = 0; i < 4; ++i) {
    f.qs[i] = p.qs[i];
    f.ks[i] = p.ks[i];
    f.vs[i] = p.vs[i];
    f.ms[i] = p.ms[i];
  }
  f.os[0] = (int64_t)p.Hq * p.Tq * p.Dv;
  f.os[1] = (int64_t)p.Tq * p.Dv;
  f.os[2] = p.Dv;
  f.os[3] = 1;
  f.B = p.B;
  f.Hq = p.Hq;
  f.Hkv = p.Hkv;
  f.Tq = p.Tq;
  f.Tk = p.Tk;
  f.D = p.D;
  f.Dv = p.Dv;
  f.group = p.group;
  f.mask_dtype = p.mask_dtype;
  f.dtype = p.dtype;
  f.causal = p.causal;
  f.scale_log2 = p.scale_log2;
  f.inv_scale_log2 = p.scale_log2 != 0.f ? 1.f / p.scale_log2 : 0.f;
  f.q_rms_eps = -1.f;
  f.num_splits = 1;
  f.split_len = p.Tk;
  out.mfma = bwd_mfma_supports(p);
  // The copies move 16-byte chunks: every tensor 16-byte aligned with
  // strides of whole chunks (the recomputed O is the workspace's).
  auto chunked = [&]() {
    const void* ptrs[8] = {p.q, p.k, p.v, p.dout, p.dq, p.dk, p.dv, saved ? p.o : nullptr};
    for (const void* ptr : ptrs)
      if ((uintptr_t)ptr % 16) return false;
    for (int i = 0; i < 3; ++i)
      if (p.qs[i] % 8 || p.ks[i] % 8 || p.vs[i] % 8 || p.dos[i] % 8 || p.os[i] % 8 || p.dqs[i] % 8 ||
          p.dks[i] % 8 || p.dvs[i] % 8)
        return false;
    return true;
  };
  if (!out.mfma && (p.dtype == MFX_BF16 || p.dtype == MFX_F16) && p.D == p.Dv && (p.D == 32 || p.D == 96) &&
      chunked()) {
    // The matrix-core kernels on zero-padded copies: contiguous rows of dp
    // features (pointers null until launch; the workspace is 256-byte
    // aligned and every region a multiple of 256 bytes).
    SdpaBwdParams pp = p;
    const int dp = p.D == 32 ? 64 : 128;
    pp.D = pp.Dv = dp;
    const int64_t qst[4] = {(int64_t)p.Hq * p.Tq * dp, (int64_t)p.Tq * dp, dp, 1};
    const int64_t kst[4] = {(int64_t)p.Hkv * p.Tk * dp, (int64_t)p.Tk * dp, dp, 1};
    for (int i = 0; i < 4; ++i) {
      pp.qs[i] = pp.dos[i] = pp.os[i] = pp.dqs[i] = qst[i];
      pp.ks[i] = pp.vs[i] = pp.dks[i] = pp.dvs[i] = kst[i];
    }
    pp.q = pp.k = pp.v = pp.dout = pp.o = nullptr;
    pp.dq = pp.dk = pp.dv = nullptr;
    if (bwd_mfma_supports(pp)) {
      out.dp = dp;
      out.pp = pp;
      out.q_pad = align256((size_t)rows * dp * 2);
      out.kv_pad = align256((size_t)p.B * p.Hkv * p.Tk * dp * 2);
    }
  }
  return MFX_OK;
}

// Workspace: O (recomputed), lse, delta; with padding, then Q, dO, O, dQ
// (q_pad each) and K, V, dK, dV (kv_pad each).
size_t bwd_workspace(const BwdPlan& pl) {
  return pl.o_bytes + 2 * pl.row_bytes + (pl.dp ? 4 * pl.q_pad + 4 * pl.kv_pad : 0);
}

// Pads (or unpads) one [B, H, T, D] tensor with element strides st.
int pad_rows(const void* src, void* dst, const BwdPlan& pl, int H, int T, const int64_t* st, bool unpad,
             hipStream_t s) {
  const int64_t rows = (int64_t)pl.p.B * H * T;
  const int64_t chunks = rows * (pl.dp / 8);
  const unsigned blocks = (unsigned)std::min<int64_t>((chunks + 255) / 256, 4096);
  if (unpad)
    hipLaunchKernelGGL((pad_rows_kernel<true>), dim3(blocks), dim3(256), 0, s, static_cast<const uint16_t*>(src),
                       static_cast<uint16_t*>(dst), rows, pl.p.D, pl.dp, H, T, st[0], st[1], st[2]);
  else
    hipLaunchKernelGGL((pad_rows_kernel<false>), dim3(blocks), dim3(256), 0, s, static_cast<const uint16_t*>(src),
                       static_cast<uint16_t*>(dst), rows, pl.p.D, pl.dp, H, T, st[0], st[1], st[2]);
  return launch_status("pad_rows_kernel");
}

}  // namespace
}  // namespace mfx

extern "C" {

size_t mfx_sdpa_bwd_workspace_size(const mfx_sdpa_bwd_args* args) {
  mfx::BwdPlan pl;
  if (mfx::make_bwd_plan(args, pl) != MFX_OK) return 0;
  return mfx::bwd_workspace(pl);
}

const char* mfx_sdpa_bwd_kernel_name(const mfx_sdpa_bwd_args* args) {
  mfx::BwdPlan pl;
  if (mfx::make_bwd_plan(args, pl) != MFX_OK) return nullptr;
  if (pl.dp) {
    static const char* const padded[2][2] = {{"mfma_bf16_d32", "mfma_bf16_d96"}, {"mfma_f16_d32", "mfma_f16_d96"}};
    return padded[pl.p.dtype == MFX_F16][pl.p.D == 96];
  }
  if (!pl.mfma) return "generic";
  if (pl.p.dtype == MFX_F16) return pl.p.D == 128 ? "mfma_f16_d128" : "mfma_f16_d64";
  return pl.p.D == 128 ? "mfma_bf16_d128" : "mfma_bf16_d64";
}

int mfx_sdpa_bwd(const mfx_sdpa_bwd_args* args, void* stream) {
  using namespace mfx;
  BwdPlan pl;
  int rc = make_bwd_plan(args, pl);
  if (rc != MFX_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t need = bwd_workspace(pl);
  char* ws = nullptr;
  if (args->workspace) {
    if (args->workspace_bytes < need)
      return fail(MFX_E_WORKSPACE, "workspace smaller than mfx_sdpa_bwd_workspace_size()");
    if ((uintptr_t)args->workspace % 256) return fail(MFX_E_INVALID, "workspace must be 256-byte aligned");
    ws = static_cast<char*>(args->workspace);
  } else {
    ws = static_cast<char*>(device_scratch(need, s));
    if (!ws) return MFX_E_HIP;
  }
  SdpaBwdParams& p = pl.p;
  SdpaParams& f = pl.fwd;
  float* delta = reinterpret_cast<float*>(ws + pl.o_bytes + pl.row_bytes);
  p.delta = delta;
  if (!args->fwd_out) {
    // Recompute O and lse into the workspace.
    f.out = ws;
    f.lse = reinterpret_cast<float*>(ws + pl.o_bytes);
    p.o = f.out;
    p.lse = f.lse;
    if (flash_bf16_supports(f)) rc = launch_flash_bf16(f, s);
    else if (flash_f32_supports(f)) rc = launch_flash_f32(f, s);
    else rc = launch_generic(f, s);
    if (rc != MFX_OK) return rc;
  }

  if (pl.mfma) return launch_bwd_mfma(p, s);
  if (pl.dp) {
    // Zero-padded copies in, the matrix-core kernels, the gradients out.
    char* w = ws + pl.o_bytes + 2 * pl.row_bytes;
    SdpaBwdParams& pp = pl.pp;
    void* qp = w;
    void* dop = w + pl.q_pad;
    void* op = w + 2 * pl.q_pad;
    void* dqp = w + 3 * pl.q_pad;
    char* wk = w + 4 * pl.q_pad;
    void* kp = wk;
    void* vp = wk + pl.kv_pad;
    void* dkp = wk + 2 * pl.kv_pad;
    void* dvp = wk + 3 * pl.kv_pad;
    if ((rc = pad_rows(p.q, qp, pl, p.Hq, p.Tq, p.qs, false, s)) != MFX_OK) return rc;
    if ((rc = pad_rows(p.dout, dop, pl, p.Hq, p.Tq, p.dos, false, s)) != MFX_OK) return rc;
    if ((rc = pad_rows(p.o, op, pl, p.Hq, p.Tq, p.os, false, s)) != MFX_OK) return rc;
    if ((rc = pad_rows(p.k, kp, pl, p.Hkv, p.Tk, p.ks, false, s)) != MFX_OK) return rc;
    if ((rc = pad_rows(p.v, vp, pl, p.Hkv, p.Tk, p.vs, false, s)) != MFX_OK) return rc;
    pp.q = qp;
    pp.dout = dop;
    pp.o = op;
    pp.k = kp;
    pp.v = vp;
    pp.dq = dqp;
    pp.dk = dkp;
    pp.dv = dvp;
    pp.lse = p.lse;
    pp.delta = p.delta;
    if ((rc = launch_bwd_mfma(pp, s)) != MFX_OK) return rc;
    if ((rc = pad_rows(dqp, p.dq, pl, p.Hq, p.Tq, p.dqs, true, s)) != MFX_OK) return rc;
    if ((rc = pad_rows(dkp, p.dk, pl, p.Hkv, p.Tk, p.dks, true, s)) != MFX_OK) return rc;
    return pad_rows(dvp, p.dv, pl, p.Hkv, p.Tk, p.dvs, true, s);
  }
  const int64_t rows = (int64_t)p.B * p.Hq * p.Tq;
  const unsigned dblocks = (unsigned)((rows + 3) / 4);
  if (p.dtype == MFX_BF16)
    hipLaunchKernelGGL((bwd_delta_kernel<bf16>), dim3(dblocks), dim3(256), 0, s, p, delta);
  else if (p.dtype == MFX_F16)
    hipLaunchKernelGGL((bwd_delta_kernel<_Float16>), dim3(dblocks), dim3(256), 0, s, p, delta);
  else
    hipLaunchKernelGGL((bwd_delta_kernel<float>), dim3(dblocks), dim3(256), 0, s, p, delta);
  if ((rc = launch_status("bwd_delta_kernel")) != MFX_OK) return rc;
  const unsigned kv_rows = (unsigned)((int64_t)p.B * p.Hkv * p.Tk);
  if (p.dtype == MFX_BF16) {
    hipLaunchKernelGGL((bwd_dkdv_generic<bf16>), dim3(kv_rows), dim3(64), 0, s, p);
    hipLaunchKernelGGL((bwd_dq_generic<bf16>), dim3((unsigned)rows), dim3(64), 0, s, p);
  } else if (p.dtype == MFX_F16) {
    hipLaunchKernelGGL((bwd_dkdv_generic<_Float16>), dim3(kv_rows), dim3(64), 0, s, p);
    hipLaunchKernelGGL((bwd_dq_generic<_Float16>), dim3((unsigned)rows), dim3(64), 0, s, p);
  } else {
    hipLaunchKernelGGL((bwd_dkdv_generic<float>), dim3(kv_rows), dim3(64), 0, s, p);
    hipLaunchKernelGGL((bwd_dq_generic<float>), dim3((unsigned)rows), dim3(64), 0, s, p);
  }
  return launch_status("bwd generic kernels");
}

}  // extern "C"
