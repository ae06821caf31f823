// Device math shared by the elementwise interpreter (generic.hip) and the
// hipRTC-generated kernels (ew_jit.cpp, gemm_jit.cpp), which compile this
// header's text: one definition, so every path gives the same bits.
// Self-contained (no includes), and written with explicit fused multiply-adds
// so the result does not depend on the compiler's contraction setting (the
// library is built with hipcc's default, the generated kernels with
// -ffp-contract=off).
#pragma once

// tanh(x) within 4 ulp (measured against fp64 over all f32 magnitudes,
// tests/test_kernels_gpu.py).  For |x| >= 0.55: (1 - e) / (1 + e) with
// e = exp(-2|x|) = exp2(-2|x| / ln 2) on the hardware exp2 and reciprocal
// (e <= 1/3, so neither 1 - e nor 1 + e loses bits to cancellation; e
// underflows to 0 past |x| ~ 44, giving +-1).  For |x| < 0.55: x + x^3 P(x^2)
// with P the degree-4 polynomial minimising the relative error of tanh on
// that interval (fitted in fp64, 0.8 ulp in fp32 Horner form).  Replaces the
// library tanhf (about 25 instructions with range reduction) by 17.
__device__ __forceinline__ float mfx_tanh(float x) {
  const float a = __builtin_fabsf(x), s = x * x;
  float p = __builtin_fmaf(-0.006274502258747816f, s, 0.02107185311615467f);
  p = __builtin_fmaf(p, s, -0.053852349519729614f);
  p = __builtin_fmaf(p, s, 0.13332585990428925f);
  p = __builtin_fmaf(p, s, -0.33333316445350647f);
  const float small = __builtin_fmaf(a * s, p, a);
  const float e = __builtin_amdgcn_exp2f(a * -2.8853900817779268f);
  const float big = (1.0f - e) * __builtin_amdgcn_rcpf(1.0f + e);
  // Both branches are computed on |x|; the sign goes on last (tanh(-0) = -0).
  return __builtin_copysignf(a < 0.55f ? small : big, x);
}
