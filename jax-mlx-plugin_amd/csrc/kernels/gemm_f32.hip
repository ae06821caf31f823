// Hand-written f32 GEMM for mfx_gemm (row-major, no transposes), on the tile
// kernel of gemm_f32_tile.h with a plain store.  gemm_jit.cpp builds the
// same tile kernel with a fused elementwise epilogue.
#include "gemm_f32.h"

#include "common.h"

namespace mfx {
namespace {

using mfx_gemm_tile::Params;
using mfx_gemm_tile::StoreEpilogue;

template <int BM, int BN, int S, int MINB>
__global__ __launch_bounds__(mfx_gemm_tile::threads(BM, BN), MINB) void gemm_f32_kernel(Params p) {
  mfx_gemm_tile::gemm_tile<BM, BN, S, StoreEpilogue>(p, StoreEpilogue::Args{});
}

bool aligned(const void* p, uintptr_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

}  // namespace

bool gemm_f32_supported(const mfx_gemm_args& a) {
  if (a.dtype != MFX_F32 || a.c_dtype != MFX_F32 || a.trans_a || a.trans_b) return false;
  if (a.batch < 1 || a.batch > 65535 || a.m < 1 || a.n < 1 || a.k < 0) return false;
  if (a.k % 4 || a.n % 4 || a.lda % 4 || a.ldb % 4 || a.ldc % 2) return false;
  if (a.lda < a.k || a.ldb < a.n || a.ldc < a.n) return false;
  if (a.stride_a % 4 || a.stride_b % 4 || a.stride_c % 2) return false;
  if (!aligned(a.a, 16) || !aligned(a.b, 16) || !aligned(a.c, 8)) return false;
  const int64_t lim = 0x7fffffffLL;
  if (a.m > lim || a.n > lim || a.k > lim || a.ldc > lim) return false;
  // Byte offsets of one k-tile load stay below 2^31 (A: a block of rows from
  // its first row; B: the whole operand plus one k-tile and one tile width).
  if ((int64_t)kGemmF32BM * a.lda * 4 + (a.k + 64) * 4 > lim) return false;
  if ((a.k + 64) * a.ldb * 4 + (a.n + kGemmF32BN) * 4 > lim) return false;
  const int64_t tiles = ((a.m + kGemmF32BM - 1) / kGemmF32BM) * ((a.n + kGemmF32BN - 1) / kGemmF32BN);
  return tiles <= lim;
}

Params gemm_f32_params(const mfx_gemm_args& a) {
  Params p{};
  p.a = static_cast<const float*>(a.a);
  p.b = static_cast<const float*>(a.b);
  p.c = static_cast<float*>(a.c);
  p.sa = a.stride_a;
  p.sb = a.stride_b;
  p.sc = a.stride_c;
  p.M = (int)a.m;
  p.N = (int)a.n;
  p.K = (int)a.k;
  p.lda = (int)a.lda;
  p.ldb = (int)a.ldb;
  p.ldc = (int)a.ldc;
  p.tiles_m = (int)((a.m + kGemmF32BM - 1) / kGemmF32BM);
  p.tiles_n = (int)((a.n + kGemmF32BN - 1) / kGemmF32BN);
  return p;
}

int gemm_f32_launch(const mfx_gemm_args& a, hipStream_t stream) {
  const Params p = gemm_f32_params(a);
  constexpr int kThreads = mfx_gemm_tile::threads(kGemmF32BM, kGemmF32BN);
  hipLaunchKernelGGL((gemm_f32_kernel<kGemmF32BM, kGemmF32BN, kGemmF32Stages, kGemmF32MinBlocks>),
                     dim3((unsigned)(p.tiles_m * p.tiles_n), (unsigned)a.batch, 1), dim3(kThreads), 0, stream, p);
  return launch_status("gemm_f32_kernel");
}

}  // namespace mfx
