// mfx_sdpa_fwd: argument validation, kernel selection and workspace layout;
// mfx_sdpa_fwd_noalloc: the same with the workspace in a static device array.
#include <cmath>
#include <mutex>
#include <string>
#include <vector>

#include "sdpa_common.h"

// Workspace of mfx_sdpa_fwd_noalloc (split-KV partials and tile lists, or a
// normalised copy of q): one copy per device, held until the process ends.
// Host code never passes `scratch` itself to a kernel (on the host it names
// a stand-in, not the device copy): it uses the per-device address that
// hipGetSymbolAddress returns.
static __device__ __align__(256) char scratch[MFX_SDPA_NOALLOC_SCRATCH_BYTES];

namespace mfx {
namespace {

enum class Kind { kFlashBf16, kFlashF32, kDecode, kDecodeMfma, kGeneric };

struct Plan {
  SdpaParams p{};
  Kind kind = Kind::kGeneric;
  size_t partial_bytes = 0;  // split-KV partials
  size_t qnorm_bytes = 0;    // normalised q for kernels without fused RMSNorm
  int decode_waves = 0;      // MFMA decode: wavefronts of the main kernel
};

int make_plan(const mfx_sdpa_args* a, Plan& out) {
  if (!a) return fail(MFX_E_INVALID, "null args");
  if (!a->q || !a->k || !a->v || !a->out) return fail(MFX_E_INVALID, "q, k, v and out must be non-null");
  if (a->B <= 0 || a->Hq <= 0 || a->Hkv <= 0 || a->Tq <= 0 || a->Tk <= 0 || a->D <= 0 || a->Dv <= 0)
    return fail(MFX_E_INVALID, "B, Hq, Hkv, Tq, Tk, D and Dv must all be positive");
  if (a->Hq % a->Hkv != 0) return fail(MFX_E_INVALID, "Hq must be a multiple of Hkv");
  const int64_t lim = 0x7fffffffLL;
  if (a->B * a->Hq * a->Tq > lim || a->Tk > lim || a->B * a->Hkv > 65535)
    return fail(MFX_E_UNSUPPORTED, "problem too large for one launch");
  if (a->q_strides[3] != 1 || a->k_strides[3] != 1 || a->v_strides[3] != 1 || a->o_strides[3] != 1)
    return fail(MFX_E_INVALID, "feature (last) strides must be 1");
  if (a->dtype != MFX_F32 && a->dtype != MFX_BF16 && a->dtype != MFX_F16)
    return fail(MFX_E_UNSUPPORTED, "dtype must be f32, bf16 or f16");
  if (a->mask && a->mask_dtype != MFX_F32 && a->mask_dtype != MFX_BF16 && a->mask_dtype != MFX_F16)
    return fail(MFX_E_UNSUPPORTED, "mask dtype must be f32, bf16 or f16");
  if (!std::isfinite(a->scale)) return fail(MFX_E_INVALID, "scale must be finite");
  if (a->D > 256 || a->Dv > 256) return fail(MFX_E_UNSUPPORTED, "head size above 256 is not supported");

  SdpaParams& p = out.p;
  p.q = a->q;
  p.k = a->k;
  p.v = a->v;
  p.out = a->out;
  p.mask = a->mask;
  p.q_rms_weight = a->q_rms_weight;
  for (int i = 0; i < 4; ++i) {
    p.qs[i] = a->q_strides[i];
    p.ks[i] = a->k_strides[i];
    p.vs[i] = a->v_strides[i];
    p.os[i] = a->o_strides[i];
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
  p.scale_log2 = a->scale * kLog2e;
  p.inv_scale_log2 = p.scale_log2 != 0.f ? 1.f / p.scale_log2 : 0.f;
  p.q_rms_eps = a->q_rms_eps;
  p.num_splits = 1;
  p.split_len = p.Tk;
  // The row log-sum-exp output, for a backward pass: the split-KV decode
  // kernels do not form it, so a request for it takes the flash / generic
  // kernels.
  p.lse = a->lse;
  const bool decode_ok = a->lse == nullptr;

  if (decode_ok && p.Tq <= 4 && decode_mfma_supports(p)) {
    // W wavefronts split the listed (visible) tiles of all kv heads into
    // equal ranges: as many as stay resident at once, at most one per tile.
    out.kind = Kind::kDecodeMfma;
    const int64_t tiles = (int64_t)p.B * p.Hkv * ((p.Tk + decode_mfma_tile() - 1) / decode_mfma_tile());
    const int64_t resident = decode_mfma_resident(p);
    out.decode_waves = (int)(tiles < resident ? tiles : resident);
    out.partial_bytes = decode_mfma_workspace(p, out.decode_waves);
    return MFX_OK;
  }
  if (decode_ok && p.Tq <= 4 && decode_supports(p)) {
    out.kind = Kind::kDecode;
    const int pairs = p.B * p.Hkv;
    int splits = (2048 + pairs - 1) / pairs;
    const int max_splits = (p.Tk + 255) / 256;
    splits = splits < 1 ? 1 : (splits > max_splits ? max_splits : splits);
    int len = (p.Tk + splits - 1) / splits;
    len = (len + 63) / 64 * 64;
    splits = (p.Tk + len - 1) / len;
    p.num_splits = splits;
    p.split_len = len;
    if (splits > 1)
      out.partial_bytes = (size_t)splits * p.B * p.Hq * p.Tq * (p.Dv + 2) * sizeof(float);
    return MFX_OK;
  }
  if (p.q_rms_eps >= 0.f) out.qnorm_bytes = (size_t)p.B * p.Hq * p.Tq * p.D * dtype_size(p.dtype);
  if (flash_bf16_supports(p)) {
    out.kind = Kind::kFlashBf16;
  } else if (flash_f32_supports(p)) {
    out.kind = Kind::kFlashF32;
  } else {
    out.kind = Kind::kGeneric;
  }
  return MFX_OK;
}

const char* kind_name(const Plan& pl) {
  switch (pl.kind) {
    case Kind::kFlashBf16: {
      static const char* const names[2][5] = {
          {"flash_bf16_d32", "flash_bf16_d64", "flash_bf16_d96", "flash_bf16_d128", "flash_bf16_d256"},
          {"flash_f16_d32", "flash_f16_d64", "flash_f16_d96", "flash_f16_d128", "flash_f16_d256"}};
      const int d = pl.p.D;
      return names[pl.p.dtype == MFX_F16][d == 32 ? 0 : d == 64 ? 1 : d == 96 ? 2 : d == 128 ? 3 : 4];
    }
    case Kind::kFlashF32: {
      static const char* const names[2][5] = {
          {"flash_f32_d32", "flash_f32_d64", "flash_f32_d96", "flash_f32_d128", "flash_f32_d256"},
          {"flash_f32_split_d32", "flash_f32_split_d64", "flash_f32_split_d96", "flash_f32_split_d128", ""}};
      const int d = pl.p.D;
      return names[flash_f32_use_split(pl.p)][d == 32 ? 0 : d == 64 ? 1 : d == 96 ? 2 : d == 128 ? 3 : 4];
    }
    case Kind::kDecode: return "decode_splitkv";
    case Kind::kDecodeMfma: return "decode_splitkv_mfma";
    default: return "generic";
  }
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Device address of `scratch` on the current device, looked up once per
// device (the first mfx_sdpa_fwd_noalloc call there) and kept.
std::mutex g_scratch_addr_mu;
std::vector<void*> g_scratch_addr;  // indexed by device ordinal

int noalloc_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_scratch_addr_mu);
  if ((size_t)dev >= g_scratch_addr.size()) g_scratch_addr.resize(dev + 1, nullptr);
  if (!g_scratch_addr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!ptr) return fail(MFX_E_HIP, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_addr[dev] = ptr;
  }
  *out = g_scratch_addr[dev];
  return MFX_OK;
}

}  // namespace
}  // namespace mfx

extern "C" {

size_t mfx_sdpa_workspace_size(const mfx_sdpa_args* args) {
  mfx::Plan pl;
  if (mfx::make_plan(args, pl) != MFX_OK) return 0;
  return mfx::align256(pl.partial_bytes) + mfx::align256(pl.qnorm_bytes);
}

const char* mfx_sdpa_kernel_name(const mfx_sdpa_args* args) {
  mfx::Plan pl;
  if (mfx::make_plan(args, pl) != MFX_OK) return nullptr;
  return mfx::kind_name(pl);
}

int mfx_sdpa_fwd(const mfx_sdpa_args* args, void* stream) {
  using namespace mfx;
  Plan pl;
  int rc = make_plan(args, pl);
  if (rc != MFX_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t need = align256(pl.partial_bytes) + align256(pl.qnorm_bytes);
  char* ws = nullptr;
  if (need > 0) {
    if (args->workspace) {
      if (args->workspace_bytes < need)
        return fail(MFX_E_WORKSPACE, "workspace smaller than mfx_sdpa_workspace_size()");
      ws = static_cast<char*>(args->workspace);
    } else {
      ws = static_cast<char*>(device_scratch(need, s));
      if (!ws) return MFX_E_HIP;
    }
  }
  SdpaParams& p = pl.p;
  if (pl.kind == Kind::kDecodeMfma) decode_mfma_bind(p, pl.decode_waves, ws);
  else if (pl.partial_bytes) p.partial = reinterpret_cast<float*>(ws);
  if (pl.qnorm_bytes) {
    // Kernels without a fused q RMSNorm read a normalised copy of q.
    void* qn = ws + align256(pl.partial_bytes);
    for (int64_t bb = 0; bb < p.B; ++bb) {
      mfx_norm_args na{};
      na.x = static_cast<const char*>(p.q) + bb * p.qs[0] * dtype_size(p.dtype);
      na.y = static_cast<char*>(qn) + bb * (int64_t)p.Hq * p.Tq * p.D * dtype_size(p.dtype);
      na.gamma = p.q_rms_weight;
      na.n = p.D;
      na.eps = p.q_rms_eps;
      na.dtype = p.dtype;
      na.param_dtype = p.dtype;
      if (p.qs[1] == (int64_t)p.Tq * p.qs[2]) {
        na.rows = (int64_t)p.Hq * p.Tq;
        na.x_row_stride = p.qs[2];
        na.y_row_stride = p.D;
        rc = mfx_rms_norm(&na, stream);
        if (rc != MFX_OK) return rc;
      } else {
        for (int64_t hh = 0; hh < p.Hq; ++hh) {
          na.x = static_cast<const char*>(p.q) + (bb * p.qs[0] + hh * p.qs[1]) * dtype_size(p.dtype);
          na.y = static_cast<char*>(qn) + ((bb * p.Hq + hh) * (int64_t)p.Tq * p.D) * dtype_size(p.dtype);
          na.rows = p.Tq;
          na.x_row_stride = p.qs[2];
          na.y_row_stride = p.D;
          rc = mfx_rms_norm(&na, stream);
          if (rc != MFX_OK) return rc;
        }
      }
    }
    p.q = qn;
    p.qs[0] = (int64_t)p.Hq * p.Tq * p.D;
    p.qs[1] = (int64_t)p.Tq * p.D;
    p.qs[2] = p.D;
    p.qs[3] = 1;
    p.q_rms_eps = -1.f;
  }
  switch (pl.kind) {
    case Kind::kFlashBf16: return launch_flash_bf16(p, s);
    case Kind::kFlashF32: return launch_flash_f32(p, s);
    case Kind::kDecode: return launch_decode(p, s);
    case Kind::kDecodeMfma: return launch_decode_mfma(p, s);
    default: return launch_generic(p, s);
  }
}

int mfx_sdpa_fwd_noalloc(const mfx_sdpa_args* args, void* stream) {
  using namespace mfx;
  Plan pl;
  int rc = make_plan(args, pl);
  if (rc != MFX_OK) return rc;
  const size_t need = align256(pl.partial_bytes) + align256(pl.qnorm_bytes);
  if (need > MFX_SDPA_NOALLOC_SCRATCH_BYTES)
    return fail(MFX_E_WORKSPACE, "mfx_sdpa_fwd_noalloc: these arguments need " + std::to_string(need) +
                                     " bytes of workspace, above the " +
                                     std::to_string((size_t)MFX_SDPA_NOALLOC_SCRATCH_BYTES) +
                                     " bytes of its static scratch; call mfx_sdpa_fwd with a workspace");
  mfx_sdpa_args a = *args;
  a.workspace = nullptr;
  a.workspace_bytes = 0;
  if (need > 0) {
    rc = noalloc_scratch(&a.workspace);
    if (rc != MFX_OK) return rc;
    a.workspace_bytes = MFX_SDPA_NOALLOC_SCRATCH_BYTES;
  }
  return mfx_sdpa_fwd(&a, stream);
}

}  // extern "C"
