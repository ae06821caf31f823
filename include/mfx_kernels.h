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
 *               elements contiguous within a row; dtype `dtype` (MFX_F32,
 *               MFX_BF16 or MFX_F16; fp32 arithmetic).
 *   gamma/beta: [n] vectors of `param_dtype` (any of the three), each may
 *               be NULL.
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
 * Row log-softmax over the last axis, y = (x - max) - log(sum(exp(x - max))),
 * same layout rules as mfx_softmax.  Replaces the reference's special-cased
 * callee @log_softmax (src/jax_mlx_pjrt.cpp:5624-5641, an mlx max / exp /
 * sum / log composition) for jax.nn.log_softmax's lowering.
 */
int mfx_log_softmax(const mfx_norm_args* args, void* stream);

/*
 * LayerNorm backward over the last axis of [rows, n] views (feature stride 1,
 * one row stride per tensor), for y = (x - mean) / sqrt(var + eps) * gamma + b
 * with the population variance:
 *   dx     = (dxh - mean(dxh) - xhat * mean(dxh * xhat)) / sqrt(var + eps),
 *            xhat = (x - mean) / sqrt(var + eps), dxh = dy * gamma;
 *   dgamma = sum over rows of dy * xhat;  dbeta = sum over rows of dy.
 * gamma NULL means gamma = 1; dgamma / dbeta NULL skip that output.  x, dy and
 * dx have `dtype`; gamma, dgamma and dbeta have `param_dtype`.  Sums run in
 * fp32.  The parameter sums go through a workspace of
 * mfx_layer_norm_bwd_workspace_size() bytes (NULL: library scratch).
 * Replaces mx::vjp of fast::layer_norm behind custom_call
 * @mlx_layer_norm_bwd (reference src/jax_mlx_pjrt.cpp:8237-8281; closed form
 * src/jax_mlx/layer_norm.py:59-76).
 */
typedef struct {
  const void* x;
  const void* gamma;
  const void* dy;
  void* dx;
  void* dgamma;
  void* dbeta;
  void* workspace;
  size_t workspace_bytes;
  int64_t rows;
  int64_t n;
  int64_t x_row_stride;
  int64_t dy_row_stride;
  int64_t dx_row_stride;
  float eps;
  int32_t dtype;
  int32_t param_dtype;
  int32_t reserved;
} mfx_norm_bwd_args;

int mfx_layer_norm_bwd(const mfx_norm_bwd_args* args, void* stream);

/* Bytes of workspace mfx_layer_norm_bwd needs for these arguments. */
size_t mfx_layer_norm_bwd_workspace_size(const mfx_norm_bwd_args* args);

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
 * A query row with every key removed by -inf yields NaN (0/0), as the
 * unfused softmax does.  Finite mask values below -2.3e38 (JAX's
 * -0.7 * FLT_MAX, finfo.min) are raised to -2.3e38 so that scaling them
 * stays finite: a row whose keys all carry such a value returns the mean of
 * V, as jnp.where(mask, s, finite) then softmax does.
 *
 * q_rms_eps >= 0 applies RMSNorm over D to each query row first (rounded to
 * `dtype`, optionally times q_rms_weight[D] of `dtype`), which fuses the
 * RMSNorm(q) -> SDPA chain of GQA decode.  Pass a negative value to disable.
 *
 * dtype is MFX_F32, MFX_BF16 or MFX_F16 (fp32 accumulation for all; the
 * 16-bit paths feed probabilities rounded to `dtype` to the PV product, as
 * JAX's attention casts them to the value dtype).  Head sizes D == Dv of 32,
 * 64, 96, 128 and 256 run on the matrix-core kernels (mfx_sdpa_kernel_name
 * names the one a call takes); any other up to 256 on a per-row kernel.
 *
 * lse (optional output): the row log-sum-exp of the scaled, masked scores in
 * log2 units, lse[(b * Hq + h) * Tq + i] = log2(sum_j exp2(log2e * (scale *
 * q_i.k_j + M_ij))), fp32 -- what mfx_sdpa_bwd needs (fwd_lse) to skip its
 * recomputed forward pass.  When it is set the split-KV decode kernels (which
 * do not form it) are not used.  NULL: not written.
 *
 * workspace: split-KV decode keeps per-split partial results there.  Query
 * the size with mfx_sdpa_workspace_size(); pass NULL to let the library use a
 * buffer of its own for this device and stream (calls on one stream share it
 * in stream order, calls on different streams get different buffers; when it
 * must grow the library allocates a larger one and keeps the old one until
 * the process ends, so it neither waits nor frees memory queued work may
 * read, but it does call hipMalloc: callers that cannot allocate pass a
 * workspace or use mfx_sdpa_fwd_noalloc).
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
  float* lse;
} mfx_sdpa_args;

int mfx_sdpa_fwd(const mfx_sdpa_args* args, void* stream);

/* Bytes of workspace mfx_sdpa_fwd needs for these arguments (0 if none). */
size_t mfx_sdpa_workspace_size(const mfx_sdpa_args* args);

/*
 * mfx_sdpa_fwd without any allocation, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference: it is
 * an addition of this library for those callers.
 *
 * Same arguments and results as mfx_sdpa_fwd, except that args->workspace is
 * ignored: the workspace is a static device array of
 * MFX_SDPA_NOALLOC_SCRATCH_BYTES per device, held until the process ends.
 * Arguments whose mfx_sdpa_workspace_size() exceeds it are rejected with
 * MFX_E_WORKSPACE before anything is launched.  The entry point calls no
 * hipMalloc / hipFree.  Every call on a device shares that device's array, so
 * calls that overlap on one device (different streams, or host threads
 * without ordering) race; calls ordered on one stream do not.  The array
 * keeps the last call's contents; nothing in it needs to start at zero.
 */
#define MFX_SDPA_NOALLOC_SCRATCH_BYTES (16u << 20)
int mfx_sdpa_fwd_noalloc(const mfx_sdpa_args* args, void* stream);

/* Which kernel mfx_sdpa_fwd would launch for these arguments, as a static
 * string ("flash_bf16_d128", "decode_splitkv", ...), or NULL if invalid. */
const char* mfx_sdpa_kernel_name(const mfx_sdpa_args* args);

/*
 * SDPA backward: given dO = dL/d(out) of out = softmax(scale * Q K^T + M) V,
 *   P = softmax(scale * Q K^T + M),  dP = dO V^T,
 *   dS = P * (dP - rowsum(dO * out)),
 *   dV = P^T dO,  dQ = scale * dS K,  dK = scale * dS^T Q,
 * with dK / dV of a kv head summed over its Hq / Hkv query heads (GQA).
 * Shapes, strides (feature stride 1), causal and mask follow mfx_sdpa_args;
 * dq / dk / dv have q / k / v's logical shapes and their own strides, and
 * every tensor has `dtype` (fp32 accumulation).  The forward pass is
 * recomputed into the workspace (out and the row log-sum-exp), so only the
 * inputs are needed -- unless the caller passes the forward's own results:
 * fwd_out (out of mfx_sdpa_fwd on the same inputs, `dtype`, strides
 * fwd_out_strides) and fwd_lse (that call's lse output), both or neither;
 * with both, the recompute is skipped.  The gradients then equal the
 * recomputing call's bit for bit whenever the forward ran the kernel the
 * recompute runs (out 16-byte aligned with strides a multiple of 8 -- every
 * output the plugin's planner allocates).  A plan that
 * runs a forward and its backward passes them along; the reference's
 * custom_call @mlx_sdpa_bwd interface (q, k, v, grad_out) has no slot for
 * them, and its mx::vjp recomputes.  Workspace:
 * mfx_sdpa_bwd_workspace_size() bytes, or NULL for library scratch.
 * Deterministic: no atomics.
 * Replaces mx::vjp of fast::scaled_dot_product_attention behind custom_call
 * @mlx_sdpa_bwd (reference src/jax_mlx_pjrt.cpp:8151-8206; closed form
 * src/jax_mlx/sdpa.py:65-87).
 */
typedef struct {
  const void* q;
  const void* k;
  const void* v;
  const void* dout;
  const void* mask;
  void* dq;
  void* dk;
  void* dv;
  void* workspace;
  size_t workspace_bytes;
  int64_t B, Hq, Hkv, Tq, Tk, D, Dv;
  int64_t q_strides[4];
  int64_t k_strides[4];
  int64_t v_strides[4];
  int64_t do_strides[4];
  int64_t dq_strides[4];
  int64_t dk_strides[4];
  int64_t dv_strides[4];
  int64_t mask_strides[4];
  float scale;
  int32_t causal;
  int32_t dtype;
  int32_t mask_dtype;
  const void* fwd_out;
  const float* fwd_lse;
  int64_t fwd_out_strides[4];
} mfx_sdpa_bwd_args;

int mfx_sdpa_bwd(const mfx_sdpa_bwd_args* args, void* stream);

/* Bytes of workspace mfx_sdpa_bwd needs for these arguments: the recomputed
 * out, lse and delta, and for bf16 / f16 at head size 32 / 96 (D == Dv,
 * tensors 16-byte aligned with strides a multiple of 8) the copies of q, k,
 * v, dO, out and the gradients zero-padded to 64 / 128 features that the
 * matrix-core kernels run on. */
size_t mfx_sdpa_bwd_workspace_size(const mfx_sdpa_bwd_args* args);

/* Which backward kernels mfx_sdpa_bwd would launch ("mfma_bf16_d128",
 * "mfma_bf16_d96" (through the padded copies), "generic", ...), or NULL if
 * the arguments are invalid. */
const char* mfx_sdpa_bwd_kernel_name(const mfx_sdpa_bwd_args* args);

/* ==========================================================================
 * Generic ops: the graph regions the pattern matcher does not fuse.
 * The reference evaluates these op by op with MLX (reference
 * src/jax_mlx_pjrt.cpp:4396-4666, 4808-5009, 5298-5341, 5455-5560,
 * 5738-5747); here a run of elementwise / broadcast / transpose / convert /
 * select / compare / iota ops becomes one fused loop kernel.
 * ========================================================================== */

/* Element types of the generic ops (the three float codes above, plus): */
enum {
  MFX_I32 = 3,
  MFX_PRED = 4, /* one byte, 0 or 1 */
  MFX_I64 = 5,
  MFX_U8 = 6,
  MFX_I8 = 7,
  MFX_U32 = 8,
  MFX_F64 = 9,
};

#define MFX_MAX_RANK 8
#define MFX_EW_MAX_INPUTS 8
#define MFX_EW_MAX_REGS 32
#define MFX_EW_MAX_INSTRS 64

/* Instruction set of a fused elementwise program.  Registers hold fp32;
 * integer values are exact up to 2^24 (the index arithmetic of masks). */
enum {
  MFX_EW_LOAD = 0, /* r[dst] = input[a] at the current output index */
  MFX_EW_CONST,    /* r[dst] = imm */
  MFX_EW_IOTA,     /* r[dst] = coordinate of the output index along dim a */
  /* unary: r[dst] = f(r[a]) */
  MFX_EW_NEG,
  MFX_EW_ABS,
  MFX_EW_EXP,
  MFX_EW_EXPM1,
  MFX_EW_LOG,
  MFX_EW_LOG1P,
  MFX_EW_SQRT,
  MFX_EW_RSQRT,
  MFX_EW_TANH,
  MFX_EW_LOGISTIC,
  MFX_EW_ERF,
  MFX_EW_SIN,
  MFX_EW_COS,
  MFX_EW_FLOOR,
  MFX_EW_CEIL,
  MFX_EW_ROUND_NE,
  MFX_EW_SIGN,
  MFX_EW_NOT,        /* logical not (pred) or bitwise not (int flag) */
  MFX_EW_ROUND_BF16, /* round to the nearest bf16 value (a convert to bf16) */
  MFX_EW_ROUND_F16,
  MFX_EW_TO_INT,     /* truncate toward zero (a convert float -> int) */
  MFX_EW_IS_FINITE,
  MFX_EW_COPY,
  /* binary: r[dst] = f(r[a], r[b]) */
  MFX_EW_ADD,
  MFX_EW_SUB,
  MFX_EW_MUL,
  MFX_EW_DIV, /* int flag: truncating division */
  MFX_EW_MAX, /* NaN-propagating, as stablehlo.maximum */
  MFX_EW_MIN,
  MFX_EW_POW,
  MFX_EW_REM,
  MFX_EW_AND,
  MFX_EW_OR,
  MFX_EW_XOR,
  MFX_EW_EQ,
  MFX_EW_NE,
  MFX_EW_LT,
  MFX_EW_LE,
  MFX_EW_GT,
  MFX_EW_GE,
  MFX_EW_ATAN2,
  /* ternary */
  MFX_EW_SELECT, /* r[dst] = r[a] != 0 ? r[b] : r[c] */
  MFX_EW_CLAMP,  /* r[dst] = min(max(r[b], r[a]), r[c]) */
  MFX_EW_NUM_OPS
};

#define MFX_EW_FLAG_INT 1 /* integer semantics for DIV / REM / AND / OR / XOR / NOT */

typedef struct {
  uint8_t op;
  uint8_t dst;
  uint8_t a;
  uint8_t b;
  uint8_t c;
  uint8_t flags;
  uint8_t pad[2];
  float imm;
} mfx_ew_instr;

typedef struct {
  const void* data;
  int32_t dtype;
  int32_t pad;
  int64_t strides[MFX_MAX_RANK]; /* element strides per output dim; 0 broadcasts */
} mfx_ew_input;

/* out[idx] = program(inputs at idx) for every index of a [dims] output,
 * stored as out_dtype at element offset sum(idx[d] * out_strides[d]), or
 * contiguously (row-major) when every out_strides entry is 0. */
typedef struct {
  void* out;
  int32_t out_dtype;
  int32_t rank;
  int64_t dims[MFX_MAX_RANK];
  int64_t out_strides[MFX_MAX_RANK];
  int32_t num_inputs;
  int32_t num_instrs;
  int32_t result;
  int32_t pad;
  mfx_ew_input inputs[MFX_EW_MAX_INPUTS];
  mfx_ew_instr code[MFX_EW_MAX_INSTRS];
} mfx_ew_program;

int mfx_elementwise(const mfx_ew_program* prog, void* stream);

/* Compiles, ahead of its first mfx_elementwise call, the native kernel of a
 * program (hipRTC, gfx950): the instruction sequence, dtypes, dims and
 * strides become constants of a generated kernel, cached per device.  Data
 * pointers may be null here; their alignment, when given, selects the
 * vector-load variant (16-byte aligned is assumed for null ones).
 * mfx_elementwise uses the compiled kernel when one exists (compiling it on
 * first use otherwise) and its interpreter for programs hipRTC rejects;
 * MFX_EW_JIT=0 in the environment selects the interpreter always.
 * No counterpart in the reference: it replaces the per-op MLX kernels that
 * mx::compile fuses (src/jax_mlx_pjrt.cpp:9063-9081). */
int mfx_ew_prepare(const mfx_ew_program* prog);

/* Selects compiled kernels (on != 0, the default unless MFX_EW_JIT=0) or the
 * interpreter for mfx_elementwise; returns the previous setting.  Process
 * wide; for tests and measurements that compare the two paths. */
int mfx_ew_jit_enable(int on);

enum { MFX_RED_SUM = 0, MFX_RED_MAX = 1, MFX_RED_MIN = 2, MFX_RED_PROD = 3 };

/* out[kept...] = init (op) reduce_{dims d with bit d of reduce_mask}(in),
 * accumulated in fp32 and stored contiguously over the kept dims in order
 * (reference reduce handler src/jax_mlx_pjrt.cpp:4896-4999). */
typedef struct {
  const void* in;
  void* out;
  int32_t in_dtype;
  int32_t out_dtype;
  int32_t rank;
  int32_t op;
  int64_t dims[MFX_MAX_RANK];
  int64_t strides[MFX_MAX_RANK];
  uint32_t reduce_mask;
  float init;
} mfx_reduce_args;

int mfx_reduce(const mfx_reduce_args* args, void* stream);

/* Batched GEMM, row-major: for each batch i,
 *   C_i[m,n] = sum_k op(A_i)[m,k] * op(B_i)[k,n]
 * with A_i at a + i*stride_a stored [m][k] (lda) or, if trans_a, [k][m];
 * B_i at b + i*stride_b stored [k][n] (ldb) or, if trans_b, [n][k].
 * fp32 accumulation; a/b share `dtype`, c has `c_dtype`.  f32 products
 * without transposes whose A and B rows are 16-byte aligned (k % 4 == 0,
 * lda and ldb multiples of 4, even n) run on the hand-written f32 MFMA tile
 * kernel; bf16 / f16 products in any transpose combination (k % 8 == 0,
 * n % 4 == 0, A and B 16-byte aligned with lda, ldb and batch strides
 * multiples of 8, c rows 4-element aligned) on the hand-written 16-bit MFMA
 * tile kernel; every other case on rocBLAS (mfx_gemm_kernel_name tells
 * which).  The 16-bit kernel splits K over workgroups when the output tiles
 * are too few to fill the device (a weight gradient x^T dy): fp32 partials in
 * the library's scratch for the call's stream, summed in a fixed order (the
 * result is deterministic).  That scratch is allocated on first use per
 * stream and size: a call captured into a graph needs an eager call of the
 * same or a larger split size on the capturing stream first.
 * Replaces the dot_general lowering (reference src/jax_mlx_pjrt.cpp:4577-4666). */
typedef struct {
  const void* a;
  const void* b;
  void* c;
  int32_t dtype;
  int32_t c_dtype;
  int64_t batch, m, n, k;
  int64_t lda, ldb, ldc;
  int64_t stride_a, stride_b, stride_c;
  int32_t trans_a;
  int32_t trans_b;
} mfx_gemm_args;

int mfx_gemm(const mfx_gemm_args* args, void* stream);

/* Name of the kernel mfx_gemm runs for args (no device needed; pointers are
 * read for their alignment): "gemm_f32_tile", "gemm_bf16_tile",
 * "gemm_f16_tile" (hand-written MFMA kernels) or "rocblas".  For tests and
 * traces. */
const char* mfx_gemm_kernel_name(const mfx_gemm_args* args);

/* GEMM with a fused elementwise epilogue: out = epi(inputs) where epi's
 * input `c_input` is the GEMM result C = A B, read at the program's output
 * index (contiguous strides, fp32; its data pointer and gemm->c are
 * ignored): C is never stored.  The program's output index space must be C's
 * [batch * m, n] (rank-1..8 dims whose trailing dims span exactly n) with a
 * contiguous output aligned to two elements; gemm must be an f32 row-major
 * product the tile kernel handles (no transposes, k % 4 == 0, n % 4 == 0, lda and
 * ldb multiples of 4 -- so n % 4 == 0 for a contiguous B -- A and B 16-byte
 * aligned, ldc = n, stride_c = m * n).  The kernel is generated from the program and compiled
 * with hipRTC for gfx950 on first use (cached per device and program); the
 * arithmetic is that of mfx_elementwise, so the result equals mfx_gemm
 * followed by mfx_elementwise bit for bit.  Returns MFX_E_UNSUPPORTED for
 * pairs it cannot fuse (run the two calls instead).
 * Replaces the MLX matmul + fused elementwise kernels that mx::compile
 * produces for a dot_general and its consumers (reference
 * src/jax_mlx_pjrt.cpp:4577-4666 and 9063-9081). */
int mfx_gemm_ew(const mfx_gemm_args* gemm, const mfx_ew_program* epi, int c_input, void* stream);

/* Host-only check (no device needed) that mfx_gemm_ew accepts the pair; the
 * pointers are read for their alignment only. */
int mfx_gemm_ew_check(const mfx_gemm_args* gemm, const mfx_ew_program* epi, int c_input);

/* Compiles the fused kernel ahead of its first mfx_gemm_ew call (needs a
 * current device). */
int mfx_gemm_ew_prepare(const mfx_gemm_args* gemm, const mfx_ew_program* epi, int c_input);

/* Diagnostic: writes the generated source of the fused kernel (which
 * includes "gemm_f32_tile.h") into buf (NUL-terminated, truncated to
 * size) and returns its full length, or -1 when the pair cannot be fused. */
int64_t mfx_gemm_ew_source(const mfx_gemm_args* gemm, const mfx_ew_program* epi, int c_input, char* buf,
                           int64_t size);

#ifdef __cplusplus
}
#endif

#endif /* MFX_KERNELS_H_ */
