/*
 * mfx_kernels.h — thin C-ABI over the hand-written gfx950 HIP kernels of the
 * fused SDPA / LayerNorm / RMSNorm path (libmfx_kernels.so).
 *
 * Plain pointers, sizes and POD argument structs; no C++ or torch types.  Every
 * entry point validates its arguments on the host, enqueues its kernels on
 * `stream` (a hipStream_t, NULL = the default stream) and returns 0, or a
 * negative MFX_E* code with a message readable through mfx_last_error() on the
 * calling thread.  Device pointers must come from hipMalloc (or a view into
 * such an allocation).  Calls are asynchronous with respect to the host.
 *
 * The reference runs the same arithmetic through MLX's fused Metal ops; each
 * entry point names the reference call it replaces.
 */
#ifndef MFX_KERNELS_H_
#define MFX_KERNELS_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (subset of PJRT_Buffer_Type that the kernels compute on). */
enum {
  MFX_F32 = 0,
  MFX_BF16 = 1,
  MFX_F16 = 2,
};

/* Return codes. */
enum {
  MFX_OK = 0,
  MFX_E_INVALID = -1,     /* bad argument (shape, stride, dtype, null pointer) */
  MFX_E_UNSUPPORTED = -2, /* valid but not implemented by any kernel */
  MFX_E_HIP = -3,         /* a HIP runtime call failed */
  MFX_E_WORKSPACE = -4,   /* caller workspace too small */
};

/* Message for the last non-zero return on this thread ("" if none). */
const char* mfx_last_error(void);

/* Library version, and number of HIP devices visible (0 without a GPU). */
int mfx_version(void);
int mfx_device_count(void);

/*
 * Row normalisation over the last axis of a [rows, n] view.
 *   x / y     : rows spaced x_row_stride / y_row_stride elements apart,
 *               elements contiguous within a row; dtype `dtype`.
 *   gamma/beta: [n] vectors of `param_dtype`, each may be NULL.
 *   LayerNorm : y = (x - mean) / sqrt(var + eps) * gamma + beta, population
 *               variance computed two-pass in fp32 registers.
 *   RMSNorm   : y = x / sqrt(mean(x^2) + eps) * gamma  (beta ignored).
 * y may alias x when the strides are equal.
 */
typedef struct {
  const void* x;
  void* y;
  const void* gamma;
  const void* beta;
  int64_t rows;
  int64_t n;
  int64_t x_row_stride;
  int64_t y_row_stride;
  float eps;
  int32_t dtype;
  int32_t param_dtype;
} mfx_norm_args;

/* Replaces mlx::core::fast::layer_norm (reference src/jax_mlx_pjrt.cpp:4436,
 * 8228): the mlx.layer_norm synthetic op (:4430-4437) and the
 * custom_call @mlx_layer_norm target (:8207-8236). */
int mfx_layer_norm(const mfx_norm_args* args, void* stream);

/* Replaces mlx::core::fast::rms_norm (reference src/jax_mlx_pjrt.cpp:4428),
 * the mlx.rms_norm synthetic op (:4422-4429). */
int mfx_rms_norm(const mfx_norm_args* args, void* stream);

/*
 * Row softmax over the last axis of a [rows, n] view (same layout rules as
 * mfx_norm_args; gamma/beta/eps unused).  An all -inf row gives NaN, as
 * exp(x - max(x)) / sum does.
 * Replaces mlx::core::softmax for the mlx.softmax synthetic op (reference
 * src/jax_mlx_pjrt.cpp:4408-4417, matched at :1857-2044).
 */
int mfx_softmax(const mfx_norm_args* args, void* stream);

/*
 * Scaled dot-product attention, out = softmax(scale * Q K^T + M) V.
 *
 * Logical shapes q [B, Hq, Tq, D], k [B, Hkv, Tk, D], v [B, Hkv, Tk, Dv],
 * out [B, Hq, Tq, Dv]; every tensor is described by element strides in
 * (batch, head, seq, feature) order, so BHTD and BTNH (JAX
 * dot_product_attention) buffers are both passed without a copy.  The feature
 * stride must be 1.  Query head h reads kv head h / (Hq / Hkv) (GQA / MQA).
 *
 * M is the sum of:
 *   causal != 0 : key j is visible to query i iff j <= i (top-left aligned,
 *                 jax.nn.dot_product_attention's is_causal);
 *   mask        : optional additive tensor of `mask_dtype`, read at
 *                 b*ms[0] + h*ms[1] + i*ms[2] + j*ms[3] (0 strides
 *                 broadcast); -inf entries remove keys.
 * A query row with every key removed yields NaN (0/0), as the unfused
 * softmax does.
 *
 * q_rms_eps >= 0 applies RMSNorm over D to each query row first (rounded to
 * `dtype`, optionally times q_rms_weight[D] of `dtype`), which fuses the
 * RMSNorm(q) -> SDPA chain of GQA decode.  Pass a negative value to disable.
 *
 * dtype is MFX_F32 or MFX_BF16 (fp32 accumulation for both; bf16
 * probabilities feed the PV product in the bf16 path, as JAX's attention
 * casts them to the value dtype).
 *
 * workspace: split-KV decode keeps per-split partial results there.  Query
 * the size with mfx_sdpa_workspace_size(); pass NULL to let the library use a
 * per-device buffer it allocates once and reuses (calls that overlap on one
 * device then serialise on that buffer's stream order).
 *
 * Replaces mlx::core::fast::scaled_dot_product_attention (reference
 * src/jax_mlx_pjrt.cpp:4444 for mlx.sdpa, :8138 for custom_call @mlx_sdpa).
 */
typedef struct {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const void* mask;
  const void* q_rms_weight;
  void* workspace;
  size_t workspace_bytes;
  int64_t B, Hq, Hkv, Tq, Tk, D, Dv;
  int64_t q_strides[4];
  int64_t k_strides[4];
  int64_t v_strides[4];
  int64_t o_strides[4];
  int64_t mask_strides[4];
  float scale;
  float q_rms_eps;
  int32_t causal;
  int32_t dtype;
  int32_t mask_dtype;
  int32_t reserved;
} mfx_sdpa_args;

int mfx_sdpa_fwd(const mfx_sdpa_args* args, void* stream);

/* Bytes of workspace mfx_sdpa_fwd needs for these arguments (0 if none). */
size_t mfx_sdpa_workspace_size(const mfx_sdpa_args* args);

/* Which kernel mfx_sdpa_fwd would launch for these arguments, as a static
 * string ("flash_bf16_d128", "decode_splitkv", ...), or NULL if invalid. */
const char* mfx_sdpa_kernel_name(const mfx_sdpa_args* args);

#ifdef __cplusplus
}
#endif

#endif /* MFX_KERNELS_H_ */
