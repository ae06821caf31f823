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
  float inv_scale_log2;  // 1 / scale_log2 (0 when scale_log2 is 0)
  float q_rms_eps;   // < 0: no RMSNorm on q
  int num_splits;    // split-KV decode only: partials per row
  int split_len;     // keys per split (VALU decode; the MFMA decode interleaves tiles)
  // MFMA decode work lists (workspace): per (batch, kv head) the indices of
  // the key tiles with a visible key, tile_list[bhk * tiles_cap + i], and
  // their number tile_count[bhk].
  int* tile_list;
  int* tile_count;
  int tiles_cap;
  // Optional: row log-sum-exp of the scaled scores in log2 units,
  // lse[(b * Hq + h) * Tq + i] = log2(sum_j exp2(s_ij)), written by the
  // flash and generic kernels when non-null (the backward pass reads it).
  float* lse;
};

// Backward pass (mfx_sdpa_bwd).  o / lse come from the recomputed forward
// pass or from the caller's forward call: o [B][Hq][Tq][Dv] of `dtype` at
// element strides os (feature stride 1), lse and delta [B][Hq][Tq] fp32
// (log2 units for lse; delta = rowsum(dO * o)).
struct SdpaBwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const void* mask;
  void* dq;
  void* dk;
  void* dv;
  const float* lse;
  float* delta;  // written by the delta pass or by the matrix-core dQ kernel
  int64_t qs[4], ks[4], vs[4], dos[4], dqs[4], dks[4], dvs[4], ms[4], os[4];
  int B, Hq, Hkv, Tq, Tk, D, Dv;
  int group;
  int mask_dtype;
  int dtype;
  int causal;
  float scale;
  float scale_log2;
};

bool bwd_mfma_supports(const SdpaBwdParams& p);
// dQ (which also computes delta from O and dO), then dK and dV.
int launch_bwd_mfma(const SdpaBwdParams& p, hipStream_t s);

// Kernel families; each returns MFX_OK or an error code after launching.
int launch_flash_bf16(const SdpaParams& p, hipStream_t s);
int launch_flash_bf16_pipe(const SdpaParams& p, hipStream_t s);  // no mask
int launch_flash_bf16_pipe_wide(const SdpaParams& p, hipStream_t s);  // head sizes 32, 96
int launch_flash_f32(const SdpaParams& p, hipStream_t s);
int launch_decode(const SdpaParams& p, hipStream_t s);
int launch_decode_mfma(const SdpaParams& p, hipStream_t s);
int launch_decode_mfma_wide(const SdpaParams& p, hipStream_t s);  // head sizes 32, 96
int launch_decode_combine(const SdpaParams& p, hipStream_t s);  // merges split partials
int launch_generic(const SdpaParams& p, hipStream_t s);

bool flash_bf16_supports(const SdpaParams& p);
bool flash_f32_supports(const SdpaParams& p);
bool flash_f32_use_split(const SdpaParams& p);  // the key-split variant runs
bool decode_supports(const SdpaParams& p);
bool decode_mfma_supports(const SdpaParams& p);
int decode_mfma_tile();  // keys per tile of the MFMA decode
// Wavefronts of the MFMA decode that are resident at once (its LDS per
// workgroup against the 160 KB of a CU, on 256 CUs).
int decode_mfma_resident(const SdpaParams& p);
// Workspace bytes of the MFMA decode with W wavefronts: tile lists, counts and
// the (W + B*Hkv) * R partial rows.
size_t decode_mfma_workspace(const SdpaParams& p, int W);
// Lays the MFMA decode's work lists and partials out in `ws` (which holds
// decode_mfma_workspace bytes) and sets p.num_splits = W.
void decode_mfma_bind(SdpaParams& p, int W, void* ws);

// Mask element type as a compile-time code: 1 f32, 2 bf16, 3 f16 (0: no
// mask).  Typed loads keep the conversion out of a runtime branch, so the
// compiler need not wait for the load inside it.
inline int mask_code(int dt) { return dt == MFX_F32 ? 1 : dt == MFX_BF16 ? 2 : 3; }
template <int MT>
__device__ __forceinline__ float load_mask_t(const void* m, int64_t off) {
  if constexpr (MT == 1) return static_cast<const float*>(m)[off];
  else if constexpr (MT == 2) return static_cast<float>(static_cast<const bf16*>(m)[off]);
  else return static_cast<float>(static_cast<const _Float16*>(m)[off]);
}

// An additive-mask value in log2 units.  Finite values below kMaskMin are
// raised to it first, so the product with log2(e) stays finite: JAX masks with
// the finite value -0.7 * FLT_MAX (and finfo.min is common), whose product with
// log2(e) would round to -inf.  With the clamp a row whose keys all carry such
// a value has equal scores and returns the mean of V, as jnp.where-then-softmax
// does; with -inf it would be 0/0.  -inf itself (and NaN) pass through.
constexpr float kMaskMin = -2.3e38f;  // above -FLT_MAX / log2(e) = -2.3586e38
__device__ __forceinline__ float mask_log2(float m) {
  return kLog2e * ((m < kMaskMin && m != -INFINITY) ? kMaskMin : m);
}

// Loads one additive-mask element as fp32.
__device__ __forceinline__ float load_mask(const void* m, int dt, int64_t off) {
  if (dt == MFX_F32) return static_cast<const float*>(m)[off];
  if (dt == MFX_BF16) return static_cast<float>(static_cast<const bf16*>(m)[off]);
  return static_cast<float>(static_cast<const _Float16*>(m)[off]);
}

}  // namespace mfx
