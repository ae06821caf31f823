// Native kernels for fused elementwise programs, generated from the program
// and compiled for gfx950 at run time with hipRTC.
//
// The interpreter in generic.hip decodes each instruction per element group
// and is bound by that dispatch, not by HBM.  Here the program becomes
// straight-line code: the instruction sequence, the input / output dtypes and
// every dim and stride are compile-time constants, so a kernel is loads, the
// arithmetic of the program, and stores.  Each thread handles V consecutive
// elements of the innermost dim (V = 4 when the output is contiguous and the
// inner dim a multiple of four), with 16-byte loads for contiguous aligned
// f32 inputs, 8-byte for bf16, one load for inputs broadcast along the inner
// dim, and per-element loads otherwise.
//
// The arithmetic is that of the interpreter, written with the same library
// functions and rounding (expf, tanhf, ... ; bf16 conversion rounds to
// nearest even), so both paths give the same bits.
//
// Compiled kernels are cached per device and program signature (the program
// with its data pointers removed, plus the alignment class of each pointer).
// A program hipRTC cannot compile returns false and runs on the interpreter.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <sstream>
#include <string>
#include <unordered_map>

#include "common.h"
#include "ew_codegen.h"
#include "ew_index.h"

namespace mfx {

// Used by mfx_elementwise (generic.hip).
bool ew_jit_launch(const mfx_ew_program& p, hipStream_t s, int* rc);
int ew_jit_prepare(const mfx_ew_program& p);

namespace {

using namespace ewgen;

constexpr int kThreads = kEwThreads;

struct JitKernel {
  hipModule_t module = nullptr;
  hipFunction_t fn = nullptr;
  int64_t work_items = 0;  // threads of work (grid-stride loop over them)
};

struct Layout {
  int V = 1;           // elements per thread along the inner dim
  bool strided = false;  // output at sum(idx * out_strides)
  int mode[MFX_EW_MAX_INPUTS] = {};  // 0 vector, 1 broadcast, 2 scalar (V = 4 only)
};

std::mutex g_mu;
std::unordered_map<std::string, JitKernel> g_cache;  // key: device + signature
std::unordered_map<std::string, bool> g_failed;      // signatures hipRTC rejected

// 1: compiled kernels, 0: interpreter only; -1 until first read (then the
// MFX_EW_JIT environment variable decides, default on).
std::atomic<int> g_jit{-1};

bool jit_enabled() {
  int v = g_jit.load(std::memory_order_relaxed);
  if (v < 0) {
    const char* e = std::getenv("MFX_EW_JIT");
    v = (e && e[0] == '0') ? 0 : 1;
    int expected = -1;
    g_jit.compare_exchange_strong(expected, v);
    v = g_jit.load(std::memory_order_relaxed);
  }
  return v != 0;
}

Layout layout_of(const mfx_ew_program& p) {
  Layout L;
  for (int d = 0; d < p.rank; ++d) L.strided |= p.out_strides[d] != 0;
  const int last = p.rank - 1;
  const bool fp = [&] {
    if (p.out_dtype != MFX_F32 && p.out_dtype != MFX_BF16) return false;
    for (int i = 0; i < p.num_inputs; ++i)
      if (p.inputs[i].dtype != MFX_F32 && p.inputs[i].dtype != MFX_BF16) return false;
    return true;
  }();
  const int osz = bytes_of(p.out_dtype);
  if (fp && !L.strided && p.rank >= 1 && p.dims[last] % 4 == 0 && (uintptr_t)p.out % (size_t)(osz * 4) == 0) {
    L.V = 4;
    for (int i = 0; i < p.num_inputs; ++i) {
      const mfx_ew_input& in = p.inputs[i];
      int m = 2;
      if (in.strides[last] == 0) {
        m = 1;
      } else if (in.strides[last] == 1) {
        bool aligned = (uintptr_t)in.data % (size_t)(bytes_of(in.dtype) * 4) == 0;
        for (int d = 0; d < last; ++d) aligned = aligned && in.strides[d] % 4 == 0;
        if (aligned) m = 0;
      }
      L.mode[i] = m;
    }
  }
  return L;
}

// Program identity without its data pointers.
std::string signature(const mfx_ew_program& p, const Layout& L) {
  mfx_ew_program q = p;
  q.out = nullptr;
  for (int i = 0; i < MFX_EW_MAX_INPUTS; ++i) q.inputs[i].data = nullptr;
  for (int i = q.num_inputs; i < MFX_EW_MAX_INPUTS; ++i) std::memset(&q.inputs[i], 0, sizeof(q.inputs[i]));
  for (int pc = q.num_instrs; pc < MFX_EW_MAX_INSTRS; ++pc) std::memset(&q.code[pc], 0, sizeof(q.code[pc]));
  for (int d = q.rank; d < MFX_MAX_RANK; ++d) q.dims[d] = q.out_strides[d] = 0;
  std::string s(reinterpret_cast<const char*>(&q), sizeof(q));
  s.push_back((char)L.V);
  for (int i = 0; i < p.num_inputs; ++i) s.push_back((char)L.mode[i]);
  return s;
}

std::string gen_source(const mfx_ew_program& p, const Layout& L, int64_t& work_items) {
  const int R = p.rank, last = R - 1, V = L.V;
  int64_t numel = 1;
  for (int d = 0; d < R; ++d) numel *= p.dims[d];
  // Work items: V-element chunks along the inner dim.
  const int64_t inner = R > 0 ? p.dims[last] : 1;
  const int64_t inner_chunks = V == 4 ? inner / 4 : inner;
  work_items = V == 4 ? numel / 4 : numel;
  const bool wide = ew_needs_wide_index(work_items);
  const char* IDX = wide ? "long long" : "int";
  std::ostringstream o;
  o << "typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));\n" << ewgen::preamble();
  o << "struct Args { void* out; const void* in[" << MFX_EW_MAX_INPUTS << "]; };\n";
  o << "extern \"C\" __global__ __launch_bounds__(" << kThreads << ") void mfx_ew_kernel(const Args args) {\n";
  o << "  for (" << IDX << " c = (" << IDX << ")blockIdx.x * " << kThreads << " + threadIdx.x; c < (" << IDX << ")"
    << work_items << "LL; c += (" << IDX << ")gridDim.x * " << kThreads << ") {\n";
  // Coordinates k<d> of the first element of the chunk.
  if (R > 0) {
    o << "    " << IDX << " rem = c;\n";
    if (V == 4) {
      o << "    const " << IDX << " k" << last << " = (rem % " << inner_chunks << "LL) * 4; rem /= " << inner_chunks
        << "LL;\n";
    } else {
      o << "    const " << IDX << " k" << last << " = rem % " << inner << "LL; rem /= " << inner << "LL;\n";
    }
    for (int d = last - 1; d >= 0; --d) {
      if (d == 0)
        o << "    const " << IDX << " k0 = rem;\n";
      else
        o << "    const " << IDX << " k" << d << " = rem % " << p.dims[d] << "LL; rem /= " << p.dims[d] << "LL;\n";
    }
  }
  auto offset = [&](const int64_t* strides) {
    std::ostringstream e;
    e << "(long long)0";
    for (int d = 0; d < R; ++d)
      if (strides[d] != 0) e << " + (long long)k" << d << " * " << strides[d] << "LL";
    return e.str();
  };
  // Inputs: x<i>_<e>.
  for (int i = 0; i < p.num_inputs; ++i) {
    const mfx_ew_input& in = p.inputs[i];
    const char* t = ctype(in.dtype);
    if (!t) return "";
    o << "    const " << t << "* in" << i << " = static_cast<const " << t << "*>(args.in[" << i << "]) + ("
      << offset(in.strides) << ");\n";
    if (V == 4 && L.mode[i] == 0) {
      if (in.dtype == MFX_F32) {
        o << "    const float4 w" << i << " = *reinterpret_cast<const float4*>(in" << i << ");\n";
        o << "    const float x" << i << "_0 = w" << i << ".x, x" << i << "_1 = w" << i << ".y, x" << i << "_2 = w" << i
          << ".z, x" << i << "_3 = w" << i << ".w;\n";
      } else {
        o << "    const uint2 w" << i << " = *reinterpret_cast<const uint2*>(in" << i << ");\n";
        o << "    const float x" << i << "_0 = __uint_as_float(w" << i << ".x << 16), x" << i
          << "_1 = __uint_as_float(w" << i << ".x & 0xffff0000u), x" << i << "_2 = __uint_as_float(w" << i
          << ".y << 16), x" << i << "_3 = __uint_as_float(w" << i << ".y & 0xffff0000u);\n";
      }
    } else if (V == 4 && L.mode[i] == 1) {
      o << "    const float x" << i << "_b = (float)in" << i << "[0];\n";
      for (int e = 0; e < 4; ++e) o << "    const float x" << i << "_" << e << " = x" << i << "_b;\n";
    } else {
      for (int e = 0; e < V; ++e)
        o << "    const float x" << i << "_" << e << " = (float)in" << i << "[" << (int64_t)e * in.strides[last]
          << "LL];\n";
    }
  }
  // Program: register r's current value per element is a named value.
  std::string cur[MFX_EW_MAX_REGS][4];
  int tmp = 0;
  for (int pc = 0; pc < p.num_instrs; ++pc) {
    const mfx_ew_instr& in = p.code[pc];
    for (int e = 0; e < V; ++e) {
      std::string expr;
      if (in.op == MFX_EW_LOAD) {
        expr = "x" + std::to_string(in.a) + "_" + std::to_string(e);
      } else if (in.op == MFX_EW_CONST) {
        expr = flit(in.imm);
      } else if (in.op == MFX_EW_IOTA) {
        expr = "(float)(k" + std::to_string(in.a) + (in.a == last && e > 0 ? " + " + std::to_string(e) : "") + ")";
      } else {
        const std::string& a = cur[in.a][e];
        const std::string& b = cur[in.b < MFX_EW_MAX_REGS ? in.b : 0][e];
        const std::string& c = cur[in.c < MFX_EW_MAX_REGS ? in.c : 0][e];
        if (!op_expr(in, a, b, c, expr)) return "";
      }
      const std::string name = "t" + std::to_string(tmp++);
      o << "    const float " << name << " = " << expr << ";\n";
      cur[in.dst][e] = name;
    }
  }
  // Store.
  const char* ot = ctype(p.out_dtype);
  if (!ot) return "";
  if (V == 4) {
    o << "    " << ot << "* out = static_cast<" << ot << "*>(args.out) + (long long)c * 4;\n";
    const std::string* r = cur[p.result];
    if (p.out_dtype == MFX_F32) {
      o << "    *reinterpret_cast<float4*>(out) = make_float4(" << r[0] << ", " << r[1] << ", " << r[2] << ", " << r[3]
        << ");\n";
    } else {
      o << "    bf16x4 ow; ow[0] = (__bf16)" << r[0] << "; ow[1] = (__bf16)" << r[1] << "; ow[2] = (__bf16)" << r[2]
        << "; ow[3] = (__bf16)" << r[3] << ";\n";
      o << "    *reinterpret_cast<bf16x4*>(out) = ow;\n";
    }
  } else {
    o << "    " << ot << "* out = static_cast<" << ot << "*>(args.out) + ("
      << (L.strided ? offset(p.out_strides) : std::string("(long long)c")) << ");\n";
    o << "    *out = " << store_expr(p.out_dtype, cur[p.result][0]) << ";\n";
  }
  o << "  }\n}\n";
  return o.str();
}

int device_id() {
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess) return -1;
  return d;
}

// Compiles (or finds) the kernel of p; nullptr if it cannot be compiled.
const JitKernel* get_kernel(const mfx_ew_program& p, const Layout& L) {
  const int dev = device_id();
  if (dev < 0) return nullptr;
  const std::string sig = signature(p, L);
  const std::string key = std::to_string(dev) + ":" + sig;
  std::lock_guard<std::mutex> lock(g_mu);
  auto it = g_cache.find(key);
  if (it != g_cache.end()) return &it->second;
  if (g_failed.count(sig)) return nullptr;
  int64_t work = 0;
  const std::string src = gen_source(p, L, work);
  if (src.empty()) {
    g_failed[sig] = true;
    return nullptr;
  }
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "mfx_ew.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
    g_failed[sig] = true;
    return nullptr;
  }
  // Same code generation constraints as the library's own kernels, and no
  // contraction of a multiply and an add into one fma: each StableHLO op
  // rounds on its own, as in the interpreter.
  const char* opts[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  const hiprtcResult cr = hiprtcCompileProgram(prog, (int)(sizeof(opts) / sizeof(opts[0])), opts);
  size_t code_size = 0;
  std::string code;
  if (cr == HIPRTC_SUCCESS && hiprtcGetCodeSize(prog, &code_size) == HIPRTC_SUCCESS && code_size > 0) {
    code.resize(code_size);
    if (hiprtcGetCode(prog, &code[0]) != HIPRTC_SUCCESS) code.clear();
  }
  if (cr != HIPRTC_SUCCESS && std::getenv("MFX_EW_JIT_LOG")) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n, '\0');
    hiprtcGetProgramLog(prog, &log[0]);
    std::fprintf(stderr, "mfx_ew_jit: compile failed:\n%s\n%s\n", log.c_str(), src.c_str());
  }
  hiprtcDestroyProgram(&prog);
  if (code.empty()) {
    g_failed[sig] = true;
    return nullptr;
  }
  JitKernel k;
  if (hipModuleLoadData(&k.module, code.data()) != hipSuccess) {
    (void)hipGetLastError();
    g_failed[sig] = true;
    return nullptr;
  }
  if (hipModuleGetFunction(&k.fn, k.module, "mfx_ew_kernel") != hipSuccess) {
    (void)hipGetLastError();
    (void)hipModuleUnload(k.module);
    g_failed[sig] = true;
    return nullptr;
  }
  k.work_items = work;
  return &(g_cache[key] = k);
}

}  // namespace

bool ew_jit_launch(const mfx_ew_program& p, hipStream_t s, int* rc) {
  if (!jit_enabled()) return false;
  const Layout L = layout_of(p);
  const JitKernel* k = get_kernel(p, L);
  if (!k) return false;
  struct {
    void* out;
    const void* in[MFX_EW_MAX_INPUTS];
  } args{};
  args.out = p.out;
  for (int i = 0; i < p.num_inputs; ++i) args.in[i] = p.inputs[i].data;
  size_t size = sizeof(args);
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &args, HIP_LAUNCH_PARAM_BUFFER_SIZE, &size, HIP_LAUNCH_PARAM_END};
  const unsigned blocks = (unsigned)ew_blocks(k->work_items);
  const hipError_t e = hipModuleLaunchKernel(k->fn, blocks, 1, 1, kThreads, 1, 1, 0, s, nullptr, config);
  *rc = e == hipSuccess ? MFX_OK : hip_fail(e, "mfx_ew_kernel");
  return true;
}

int ew_jit_prepare(const mfx_ew_program& p) {
  if (!jit_enabled()) return MFX_OK;
  return get_kernel(p, layout_of(p)) ? MFX_OK : fail(MFX_E_UNSUPPORTED, "elementwise program not compiled");
}

}  // namespace mfx

extern "C" int mfx_ew_jit_enable(int on) {
  const int prev = mfx::jit_enabled() ? 1 : 0;
  mfx::g_jit.store(on ? 1 : 0, std::memory_order_relaxed);
  return prev;
}
