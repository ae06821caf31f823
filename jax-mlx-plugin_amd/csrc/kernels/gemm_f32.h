// Host side of the hand-written f32 GEMM (gemm_f32.hip) and of its fused
// elementwise-epilogue variant (gemm_jit.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include "gemm_f32_tile.h"
#include "mfx_kernels.h"

namespace mfx {

// Tile configuration: 64 x 128 workgroup tiles of four 32 x 64 wavefront
// blocks, two LDS stages (48 KB), three workgroups per CU.
constexpr int kGemmF32BM = 64;
constexpr int kGemmF32BN = 128;
constexpr int kGemmF32Stages = 2;
constexpr int kGemmF32MinBlocks = 3;

// True when the tile kernel handles `a`: f32 in and out, row-major A[m][k]
// and B[k][n], K % 4 == 0, N % 4 == 0, leading dims and batch strides that keep
// A and B rows 16-byte aligned, and 32-bit load offsets.
bool gemm_f32_supported(const mfx_gemm_args& a);

// Kernel parameters of `a` (requires gemm_f32_supported(a)); grid
// (tiles_m * tiles_n, batch) of mfx_gemm_tile::threads(BM, BN) threads.
mfx_gemm_tile::Params gemm_f32_params(const mfx_gemm_args& a);

// Launches the plain tile kernel (requires gemm_f32_supported(a)).
int gemm_f32_launch(const mfx_gemm_args& a, hipStream_t stream);

}  // namespace mfx
