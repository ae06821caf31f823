// mfx_gemm: batched strided GEMM for the dot_general ops.
//
// f32 row-major products without transposes (the dense layers of a
// transformer) run on the hand-written f32 MFMA tile kernel (gemm_f32.hip),
// bf16 / f16 products in any transpose combination on the 16-bit one
// (gemm16.hip); every other case goes to rocBLAS's gemm_strided_batched_ex
// with fp32 accumulation, issuing row-major C = op(A) op(B) as the
// column-major product C^T = op(B)^T op(A)^T.
#include <rocblas/rocblas.h>

#include <mutex>
#include <vector>

#include "common.h"
#include "gemm16.h"
#include "gemm_f32.h"

namespace mfx {
namespace {

std::mutex g_mu;
std::vector<rocblas_handle> g_handles;  // per device ordinal

int handle_for_current_device(rocblas_handle* out) {
  int dev = 0;
  MFX_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_mu);
  if ((size_t)dev >= g_handles.size()) g_handles.resize(dev + 1, nullptr);
  if (!g_handles[dev]) {
    rocblas_handle h = nullptr;
    if (rocblas_create_handle(&h) != rocblas_status_success)
      return fail(MFX_E_HIP, "rocblas_create_handle failed");
    g_handles[dev] = h;
  }
  *out = g_handles[dev];
  return MFX_OK;
}

bool to_rocblas(int dt, rocblas_datatype* out) {
  switch (dt) {
    case MFX_F32: *out = rocblas_datatype_f32_r; return true;
    case MFX_BF16: *out = rocblas_datatype_bf16_r; return true;
    case MFX_F16: *out = rocblas_datatype_f16_r; return true;
    default: return false;
  }
}

}  // namespace
}  // namespace mfx

extern "C" int mfx_gemm(const mfx_gemm_args* a, void* stream) {
  using namespace mfx;
  if (!a || !a->a || !a->b || !a->c) return fail(MFX_E_INVALID, "null gemm args");
  if (a->batch <= 0 || a->m <= 0 || a->n <= 0 || a->k < 0)
    return fail(MFX_E_INVALID, "gemm dims must be positive");
  const int64_t lim = 0x7fffffffLL;
  if (a->m > lim || a->n > lim || a->k > lim || a->batch > lim || a->lda > lim || a->ldb > lim ||
      a->ldc > lim)
    return fail(MFX_E_UNSUPPORTED, "gemm dims exceed 32-bit rocBLAS limits");
  rocblas_datatype ab_t, c_t;
  if (!to_rocblas(a->dtype, &ab_t) || !to_rocblas(a->c_dtype, &c_t))
    return fail(MFX_E_UNSUPPORTED, "gemm dtype must be f32, bf16 or f16");
  const int64_t a_cols = a->trans_a ? a->m : a->k;
  const int64_t b_cols = a->trans_b ? a->k : a->n;
  if (a->lda < a_cols || a->ldb < b_cols || a->ldc < a->n)
    return fail(MFX_E_INVALID, "gemm leading dimension too small");
  if (gemm_f32_supported(*a)) return gemm_f32_launch(*a, static_cast<hipStream_t>(stream));
  if (gemm16_supported(*a)) return gemm16_launch(*a, static_cast<hipStream_t>(stream));
  rocblas_handle h;
  int rc = handle_for_current_device(&h);
  if (rc != MFX_OK) return rc;
  if (rocblas_set_stream(h, static_cast<hipStream_t>(stream)) != rocblas_status_success)
    return fail(MFX_E_HIP, "rocblas_set_stream failed");
  const float alpha = 1.0f, beta = 0.0f;
  if (a->k == 0) {
    // Empty contraction: C = 0.
    for (int64_t i = 0; i < a->batch; ++i)
      for (int64_t r = 0; r < a->m; ++r)
        MFX_HIP_CHECK(hipMemsetAsync(static_cast<char*>(a->c) + (i * a->stride_c + r * a->ldc) * dtype_size(a->c_dtype),
                                     0, a->n * dtype_size(a->c_dtype), static_cast<hipStream_t>(stream)));
    return MFX_OK;
  }
  const rocblas_operation opB = a->trans_b ? rocblas_operation_transpose : rocblas_operation_none;
  const rocblas_operation opA = a->trans_a ? rocblas_operation_transpose : rocblas_operation_none;
  rocblas_status st = rocblas_gemm_strided_batched_ex(
      h, opB, opA, (rocblas_int)a->n, (rocblas_int)a->m, (rocblas_int)a->k, &alpha, a->b, ab_t,
      (rocblas_int)a->ldb, a->stride_b, a->a, ab_t, (rocblas_int)a->lda, a->stride_a, &beta, a->c, c_t,
      (rocblas_int)a->ldc, a->stride_c, a->c, c_t, (rocblas_int)a->ldc, a->stride_c, (rocblas_int)a->batch,
      rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  if (st != rocblas_status_success)
    return fail(MFX_E_HIP, std::string("rocblas_gemm_strided_batched_ex: ") + rocblas_status_to_string(st));
  return MFX_OK;
}

extern "C" const char* mfx_gemm_kernel_name(const mfx_gemm_args* a) {
  if (!a) return "invalid";
  if (mfx::gemm_f32_supported(*a)) return "gemm_f32_tile";
  if (mfx::gemm16_supported(*a)) return a->dtype == MFX_F16 ? "gemm_f16_tile" : "gemm_bf16_tile";
  return "rocblas";
}
