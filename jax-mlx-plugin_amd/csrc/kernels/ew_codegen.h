// Source generation shared by the hipRTC kernels of fused elementwise
// programs (ew_jit.cpp) and of GEMMs with a fused elementwise epilogue
// (gemm_jit.cpp): the fp32 expression of each program instruction, written
// with the same library functions and rounding as the interpreter in
// generic.hip, so every path gives the same bits for the same program.
#pragma once

#include <cmath>
#include <cstdio>
#include <string>

#include "mfx_kernels.h"

namespace mfx {
namespace ewgen {

inline int bytes_of(int dt) {
  switch (dt) {
    case MFX_F32: case MFX_I32: case MFX_U32: return 4;
    case MFX_BF16: case MFX_F16: return 2;
    case MFX_PRED: case MFX_U8: case MFX_I8: return 1;
    case MFX_I64: case MFX_F64: return 8;
    default: return 0;
  }
}

// Device helpers every generated source starts with.
inline const char* preamble() {
  return "__device__ __forceinline__ float nan_max(float a, float b) {"
         " return (a != a || b != b) ? __builtin_nanf(\"\") : fmaxf(a, b); }\n"
         "__device__ __forceinline__ float nan_min(float a, float b) {"
         " return (a != a || b != b) ? __builtin_nanf(\"\") : fminf(a, b); }\n";
}

// Exact fp32 literal.
inline std::string flit(float v) {
  if (std::isnan(v)) return "__builtin_nanf(\"\")";
  if (std::isinf(v)) return v > 0 ? "__builtin_inff()" : "(-__builtin_inff())";
  char buf[64];
  std::snprintf(buf, sizeof(buf), "%af", (double)v);
  return std::string("(") + buf + ")";
}

inline const char* ctype(int dt) {
  switch (dt) {
    case MFX_F32: return "float";
    case MFX_BF16: return "__bf16";
    case MFX_F16: return "_Float16";
    case MFX_I32: return "int";
    case MFX_PRED: case MFX_U8: return "unsigned char";
    case MFX_I8: return "signed char";
    case MFX_I64: return "long long";
    case MFX_U32: return "unsigned int";
    case MFX_F64: return "double";
    default: return nullptr;
  }
}

// Expression of the stored value for out dtype dt given fp32 expression v.
inline std::string store_expr(int dt, const std::string& v) {
  switch (dt) {
    case MFX_F32: return v;
    case MFX_BF16: return "(__bf16)(" + v + ")";
    case MFX_F16: return "(_Float16)(" + v + ")";
    case MFX_I32: return "(int)(" + v + ")";
    case MFX_PRED: return "(unsigned char)((" + v + ") != 0.f ? 1 : 0)";
    case MFX_U8: return "(unsigned char)(" + v + ")";
    case MFX_I8: return "(signed char)(" + v + ")";
    case MFX_I64: return "(long long)(" + v + ")";
    case MFX_U32: return "(unsigned int)(" + v + ")";
    case MFX_F64: return "(double)(" + v + ")";
    default: return v;
  }
}

// fp32 expression of instruction `in` with operand expressions a, b, c.
inline bool op_expr(const mfx_ew_instr& in, const std::string& a, const std::string& b, const std::string& c,
             std::string& out) {
  const bool is_int = in.flags & MFX_EW_FLAG_INT;
  switch (in.op) {
    case MFX_EW_NEG: out = "(-" + a + ")"; return true;
    case MFX_EW_ABS: out = "fabsf(" + a + ")"; return true;
    case MFX_EW_EXP: out = "expf(" + a + ")"; return true;
    case MFX_EW_EXPM1: out = "expm1f(" + a + ")"; return true;
    case MFX_EW_LOG: out = "logf(" + a + ")"; return true;
    case MFX_EW_LOG1P: out = "log1pf(" + a + ")"; return true;
    case MFX_EW_SQRT: out = "sqrtf(" + a + ")"; return true;
    case MFX_EW_RSQRT: out = "(1.0f / sqrtf(" + a + "))"; return true;
    case MFX_EW_TANH: out = "tanhf(" + a + ")"; return true;
    case MFX_EW_LOGISTIC: out = "(1.0f / (1.0f + expf(-" + a + ")))"; return true;
    case MFX_EW_ERF: out = "erff(" + a + ")"; return true;
    case MFX_EW_SIN: out = "sinf(" + a + ")"; return true;
    case MFX_EW_COS: out = "cosf(" + a + ")"; return true;
    case MFX_EW_FLOOR: out = "floorf(" + a + ")"; return true;
    case MFX_EW_CEIL: out = "ceilf(" + a + ")"; return true;
    case MFX_EW_ROUND_NE: out = "rintf(" + a + ")"; return true;
    case MFX_EW_SIGN: out = "(" + a + " > 0.f ? 1.f : (" + a + " < 0.f ? -1.f : " + a + "))"; return true;
    case MFX_EW_NOT:
      out = is_int ? "((float)(~(int)" + a + "))" : "(" + a + " == 0.f ? 1.f : 0.f)";
      return true;
    case MFX_EW_ROUND_BF16: out = "((float)(__bf16)" + a + ")"; return true;
    case MFX_EW_ROUND_F16: out = "((float)(_Float16)" + a + ")"; return true;
    case MFX_EW_TO_INT: out = "truncf(" + a + ")"; return true;
    case MFX_EW_IS_FINITE: out = "(__builtin_isfinite(" + a + ") ? 1.f : 0.f)"; return true;
    case MFX_EW_COPY: out = a; return true;
    case MFX_EW_ADD: out = "(" + a + " + " + b + ")"; return true;
    case MFX_EW_SUB: out = "(" + a + " - " + b + ")"; return true;
    case MFX_EW_MUL: out = "(" + a + " * " + b + ")"; return true;
    case MFX_EW_DIV: out = is_int ? "truncf(" + a + " / " + b + ")" : "(" + a + " / " + b + ")"; return true;
    case MFX_EW_MAX: out = "nan_max(" + a + ", " + b + ")"; return true;
    case MFX_EW_MIN: out = "nan_min(" + a + ", " + b + ")"; return true;
    case MFX_EW_POW: out = "powf(" + a + ", " + b + ")"; return true;
    case MFX_EW_REM: out = "fmodf(" + a + ", " + b + ")"; return true;
    case MFX_EW_AND:
      out = is_int ? "((float)((int)" + a + " & (int)" + b + "))" : "((" + a + " != 0.f && " + b + " != 0.f) ? 1.f : 0.f)";
      return true;
    case MFX_EW_OR:
      out = is_int ? "((float)((int)" + a + " | (int)" + b + "))" : "((" + a + " != 0.f || " + b + " != 0.f) ? 1.f : 0.f)";
      return true;
    case MFX_EW_XOR:
      out = is_int ? "((float)((int)" + a + " ^ (int)" + b + "))"
                   : "(((" + a + " != 0.f) != (" + b + " != 0.f)) ? 1.f : 0.f)";
      return true;
    case MFX_EW_EQ: out = "(" + a + " == " + b + " ? 1.f : 0.f)"; return true;
    case MFX_EW_NE: out = "(" + a + " != " + b + " ? 1.f : 0.f)"; return true;
    case MFX_EW_LT: out = "(" + a + " < " + b + " ? 1.f : 0.f)"; return true;
    case MFX_EW_LE: out = "(" + a + " <= " + b + " ? 1.f : 0.f)"; return true;
    case MFX_EW_GT: out = "(" + a + " > " + b + " ? 1.f : 0.f)"; return true;
    case MFX_EW_GE: out = "(" + a + " >= " + b + " ? 1.f : 0.f)"; return true;
    case MFX_EW_ATAN2: out = "atan2f(" + a + ", " + b + ")"; return true;
    case MFX_EW_SELECT: out = "(" + a + " != 0.f ? " + b + " : " + c + ")"; return true;
    case MFX_EW_CLAMP: out = "nan_min(nan_max(" + b + ", " + a + "), " + c + ")"; return true;
    default: return false;
  }
}

}  // namespace ewgen
}  // namespace mfx
