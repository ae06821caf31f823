// Launch-side description of one SDPA call, shared by the SDPA kernels.
#pragma once

#include "common.h"

namespace mfx {

// All strides in elements, ordered (batch, head, seq, feature).
struct SdpaParams {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const void* mask;
  const void* q_rms_weight;
  float* partial;  // split-KV partials: [splits][B*Hq*Tq][Dv + 2]
  int64_t qs[4], ks[4], vs[4], os[4], ms[4];
  int B, Hq, Hkv, Tq, Tk, D, Dv;
  int group;         // Hq / Hkv
  int mask_dtype;
  int dtype;
  int causal;
  float scale_log2;  // scale * log2(e)
  float q_rms_eps;   // < 0: no RMSNorm on q
  int num_splits;    // split-KV decode only: partials per row
  int split_len;     // keys per split (VALU decode; the MFMA decode interleaves tiles)
};

// Kernel families; each returns MFX_OK or an error code after launching.
int launch_flash_bf16(const SdpaParams& p, hipStream_t s);
int launch_flash_f32(const SdpaParams& p, hipStream_t s);
int launch_decode(const SdpaParams& p, hipStream_t s);
int launch_decode_mfma(const SdpaParams& p, hipStream_t s);
int launch_decode_combine(const SdpaParams& p, hipStream_t s);  // merges split partials
int launch_generic(const SdpaParams& p, hipStream_t s);

bool flash_bf16_supports(const SdpaParams& p);
bool flash_f32_supports(const SdpaParams& p);
bool decode_supports(const SdpaParams& p);
bool decode_mfma_supports(const SdpaParams& p);
int decode_mfma_tile();       // keys per tile of the MFMA decode
int decode_mfma_max_tiles();  // tiles one of its wavefronts can own

// Loads one additive-mask element as fp32.
__device__ __forceinline__ float load_mask(const void* m, int dt, int64_t off) {
  if (dt == MFX_F32) return static_cast<const float*>(m)[off];
  if (dt == MFX_BF16) return static_cast<float>(static_cast<const bf16*>(m)[off]);
  return static_cast<float>(static_cast<const _Float16*>(m)[off]);
}

}  // namespace mfx
