// Host side of the bf16 / f16 GEMM tile kernel (gemm16.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "mfx_kernels.h"

namespace mfx {

// True when the 16-bit tile kernel handles `a`: A and B bf16 or f16 (one
// type), C f32, bf16 or f16; any of the four transpose combinations; K > 0
// and K % 8 == 0, N % 4 == 0; A and B 16-byte aligned with leading dims and
// batch strides multiples of 8 elements; C rows 4-element aligned; the byte
// offsets a tile load forms below 2^31.
bool gemm16_supported(const mfx_gemm_args& a);

// Launches it (requires gemm16_supported(a)).
int gemm16_launch(const mfx_gemm_args& a, hipStream_t stream);

}  // namespace mfx
