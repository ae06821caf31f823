// Generic ops for the graph regions the pattern matcher leaves unfused:
//   mfx_elementwise  one loop kernel runs a whole fused elementwise program
//                    (loads with broadcast strides, arithmetic, compare,
//                    select, iota, converts) per output element;
//   mfx_reduce       strided reduction over any subset of axes.
// Both are HBM-bound loop kernels; the host collapses contiguous dims so the
// common cases run with rank 1 or 2 index arithmetic.
#include <cstring>

#include "common.h"

namespace mfx {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float load_elem(const void* p, int dt, int64_t off) {
  switch (dt) {
    case MFX_F32: return static_cast<const float*>(p)[off];
    case MFX_BF16: return static_cast<float>(static_cast<const bf16*>(p)[off]);
    case MFX_F16: return static_cast<float>(static_cast<const _Float16*>(p)[off]);
    case MFX_I32: return (float)static_cast<const int32_t*>(p)[off];
    case MFX_PRED:
    case MFX_U8: return (float)static_cast<const uint8_t*>(p)[off];
    case MFX_I8: return (float)static_cast<const int8_t*>(p)[off];
    case MFX_I64: return (float)static_cast<const int64_t*>(p)[off];
    case MFX_U32: return (float)static_cast<const uint32_t*>(p)[off];
    case MFX_F64: return (float)static_cast<const double*>(p)[off];
    default: return 0.f;
  }
}

__device__ __forceinline__ void store_elem(void* p, int dt, int64_t off, float v) {
  switch (dt) {
    case MFX_F32: static_cast<float*>(p)[off] = v; break;
    case MFX_BF16: static_cast<bf16*>(p)[off] = static_cast<bf16>(v); break;
    case MFX_F16: static_cast<_Float16*>(p)[off] = static_cast<_Float16>(v); break;
    case MFX_I32: static_cast<int32_t*>(p)[off] = (int32_t)v; break;
    case MFX_PRED: static_cast<uint8_t*>(p)[off] = v != 0.f ? 1 : 0; break;
    case MFX_U8: static_cast<uint8_t*>(p)[off] = (uint8_t)v; break;
    case MFX_I8: static_cast<int8_t*>(p)[off] = (int8_t)v; break;
    case MFX_I64: static_cast<int64_t*>(p)[off] = (int64_t)v; break;
    case MFX_U32: static_cast<uint32_t*>(p)[off] = (uint32_t)v; break;
    case MFX_F64: static_cast<double*>(p)[off] = (double)v; break;
    default: break;
  }
}

__device__ __forceinline__ float nan_max(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
}
__device__ __forceinline__ float nan_min(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : fminf(a, b);
}

__device__ __forceinline__ float apply(const mfx_ew_instr& in, const float* r, int64_t idx_unused) {
  const float a = r[in.a];
  const bool is_int = in.flags & MFX_EW_FLAG_INT;
  switch (in.op) {
    case MFX_EW_NEG: return -a;
    case MFX_EW_ABS: return fabsf(a);
    case MFX_EW_EXP: return expf(a);
    case MFX_EW_EXPM1: return expm1f(a);
    case MFX_EW_LOG: return logf(a);
    case MFX_EW_LOG1P: return log1pf(a);
    case MFX_EW_SQRT: return sqrtf(a);
    case MFX_EW_RSQRT: return 1.0f / sqrtf(a);
    case MFX_EW_TANH: return tanhf(a);
    case MFX_EW_LOGISTIC: return 1.0f / (1.0f + expf(-a));
    case MFX_EW_ERF: return erff(a);
    case MFX_EW_SIN: return sinf(a);
    case MFX_EW_COS: return cosf(a);
    case MFX_EW_FLOOR: return floorf(a);
    case MFX_EW_CEIL: return ceilf(a);
    case MFX_EW_ROUND_NE: return rintf(a);
    case MFX_EW_SIGN: return a > 0.f ? 1.f : (a < 0.f ? -1.f : a);
    case MFX_EW_NOT: return is_int ? (float)(~(int32_t)a) : (a == 0.f ? 1.f : 0.f);
    case MFX_EW_ROUND_BF16: return static_cast<float>(static_cast<bf16>(a));
    case MFX_EW_ROUND_F16: return static_cast<float>(static_cast<_Float16>(a));
    case MFX_EW_TO_INT: return truncf(a);
    case MFX_EW_IS_FINITE: return isfinite(a) ? 1.f : 0.f;
    case MFX_EW_COPY: return a;
    default: break;
  }
  const float b = r[in.b];
  switch (in.op) {
    case MFX_EW_ADD: return a + b;
    case MFX_EW_SUB: return a - b;
    case MFX_EW_MUL: return a * b;
    case MFX_EW_DIV: return is_int ? truncf(a / b) : a / b;
    case MFX_EW_MAX: return nan_max(a, b);
    case MFX_EW_MIN: return nan_min(a, b);
    case MFX_EW_POW: return powf(a, b);
    case MFX_EW_REM: return fmodf(a, b);
    case MFX_EW_AND: return is_int ? (float)((int32_t)a & (int32_t)b) : ((a != 0.f && b != 0.f) ? 1.f : 0.f);
    case MFX_EW_OR: return is_int ? (float)((int32_t)a | (int32_t)b) : ((a != 0.f || b != 0.f) ? 1.f : 0.f);
    case MFX_EW_XOR: return is_int ? (float)((int32_t)a ^ (int32_t)b) : (((a != 0.f) != (b != 0.f)) ? 1.f : 0.f);
    case MFX_EW_EQ: return a == b ? 1.f : 0.f;
    case MFX_EW_NE: return a != b ? 1.f : 0.f;
    case MFX_EW_LT: return a < b ? 1.f : 0.f;
    case MFX_EW_LE: return a <= b ? 1.f : 0.f;
    case MFX_EW_GT: return a > b ? 1.f : 0.f;
    case MFX_EW_GE: return a >= b ? 1.f : 0.f;
    case MFX_EW_ATAN2: return atan2f(a, b);
    default: break;
  }
  const float c = r[in.c];
  switch (in.op) {
    case MFX_EW_SELECT: return a != 0.f ? b : c;
    case MFX_EW_CLAMP: return nan_min(nan_max(b, a), c);
    default: return 0.f;
  }
}

template <typename IDX>
__global__ __launch_bounds__(kThreads) void ew_kernel(const mfx_ew_program prog, IDX numel, int strided_out) {
  float r[MFX_EW_MAX_REGS];
  for (IDX idx = (IDX)blockIdx.x * kThreads + threadIdx.x; idx < numel;
       idx += (IDX)gridDim.x * kThreads) {
    IDX coord[MFX_MAX_RANK];
    {
      IDX rem = idx;
      for (int d = prog.rank - 1; d >= 0; --d) {
        const IDX n = (IDX)prog.dims[d];
        coord[d] = rem % n;
        rem /= n;
      }
    }
    for (int pc = 0; pc < prog.num_instrs; ++pc) {
      const mfx_ew_instr in = prog.code[pc];
      float v;
      if (in.op == MFX_EW_LOAD) {
        const mfx_ew_input& src = prog.inputs[in.a];
        int64_t off = 0;
        for (int d = 0; d < prog.rank; ++d) off += (int64_t)coord[d] * src.strides[d];
        v = load_elem(src.data, src.dtype, off);
      } else if (in.op == MFX_EW_CONST) {
        v = in.imm;
      } else if (in.op == MFX_EW_IOTA) {
        v = (float)coord[in.a];
      } else {
        v = apply(in, r, 0);
      }
      r[in.dst] = v;
    }
    int64_t out_off = (int64_t)idx;
    if (strided_out) {
      out_off = 0;
      for (int d = 0; d < prog.rank; ++d) out_off += (int64_t)coord[d] * prog.out_strides[d];
    }
    store_elem(prog.out, prog.out_dtype, out_off, r[prog.result]);
  }
}

// Kept dims (kd, ks) and reduced dims (rd, rs) with their input strides.
struct ReduceMeta {
  int64_t m[32];  // kd[8], ks[8], rd[8], rs[8]
};

// One output per thread: suits many outputs with short reductions.
__global__ __launch_bounds__(kThreads) void reduce_thread_kernel(
    const void* in, void* out, int in_dt, int out_dt, int op, float init, int nk,
    const ReduceMeta meta, int nr, int64_t K, int64_t R) {
  const int64_t* m = meta.m;
  for (int64_t o = (int64_t)blockIdx.x * kThreads + threadIdx.x; o < K; o += (int64_t)gridDim.x * kThreads) {
    int64_t base = 0, rem = o;
    for (int d = nk - 1; d >= 0; --d) {
      base += (rem % m[d]) * m[8 + d];
      rem /= m[d];
    }
    float acc = init;
    for (int64_t j = 0; j < R; ++j) {
      int64_t off = base, rj = j;
      for (int d = nr - 1; d >= 0; --d) {
        off += (rj % m[16 + d]) * m[24 + d];
        rj /= m[16 + d];
      }
      const float x = load_elem(in, in_dt, off);
      switch (op) {
        case MFX_RED_SUM: acc += x; break;
        case MFX_RED_MAX: acc = nan_max(acc, x); break;
        case MFX_RED_MIN: acc = nan_min(acc, x); break;
        default: acc *= x; break;
      }
    }
    store_elem(out, out_dt, o, acc);
  }
}

// One output per workgroup: long reductions.
__global__ __launch_bounds__(kThreads) void reduce_block_kernel(
    const void* in, void* out, int in_dt, int out_dt, int op, float init, int nk,
    const ReduceMeta meta, int nr, int64_t K, int64_t R) {
  const int64_t* m = meta.m;
  __shared__ float part[kThreads / 64];
  const float ident = op == MFX_RED_SUM ? 0.f : op == MFX_RED_MAX ? -INFINITY : op == MFX_RED_MIN ? INFINITY : 1.f;
  for (int64_t o = blockIdx.x; o < K; o += gridDim.x) {
    int64_t base = 0, rem = o;
    for (int d = nk - 1; d >= 0; --d) {
      base += (rem % m[d]) * m[8 + d];
      rem /= m[d];
    }
    float acc = ident;
    for (int64_t j = threadIdx.x; j < R; j += kThreads) {
      int64_t off = base, rj = j;
      for (int d = nr - 1; d >= 0; --d) {
        off += (rj % m[16 + d]) * m[24 + d];
        rj /= m[16 + d];
      }
      const float x = load_elem(in, in_dt, off);
      switch (op) {
        case MFX_RED_SUM: acc += x; break;
        case MFX_RED_MAX: acc = nan_max(acc, x); break;
        case MFX_RED_MIN: acc = nan_min(acc, x); break;
        default: acc *= x; break;
      }
    }
    for (int off = 32; off > 0; off >>= 1) {
      const float y = __shfl_xor(acc, off, 64);
      switch (op) {
        case MFX_RED_SUM: acc += y; break;
        case MFX_RED_MAX: acc = nan_max(acc, y); break;
        case MFX_RED_MIN: acc = nan_min(acc, y); break;
        default: acc *= y; break;
      }
    }
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = init;
      for (int w = 0; w < kThreads / 64; ++w) {
        switch (op) {
          case MFX_RED_SUM: t += part[w]; break;
          case MFX_RED_MAX: t = nan_max(t, part[w]); break;
          case MFX_RED_MIN: t = nan_min(t, part[w]); break;
          default: t *= part[w]; break;
        }
      }
      store_elem(out, out_dt, o, t);
    }
    __syncthreads();
  }
}

bool valid_dtype(int dt) { return dt >= MFX_F32 && dt <= MFX_F64; }

// Merges adjacent output dims whose strides allow it for every input.
void collapse(mfx_ew_program& p) {
  if (p.rank <= 1) return;
  int w = 0;
  for (int d = 1; d < p.rank; ++d) {
    bool ok = true;
    for (int i = 0; i < p.num_inputs && ok; ++i)
      ok = p.inputs[i].strides[w] == p.inputs[i].strides[d] * p.dims[d];
    // IOTA reads coordinates: keep dims it refers to.
    for (int pc = 0; pc < p.num_instrs && ok; ++pc)
      if (p.code[pc].op == MFX_EW_IOTA) ok = false;
    if (ok) {
      p.dims[w] *= p.dims[d];
      for (int i = 0; i < p.num_inputs; ++i) p.inputs[i].strides[w] = p.inputs[i].strides[d];
    } else {
      ++w;
      p.dims[w] = p.dims[d];
      for (int i = 0; i < p.num_inputs; ++i) p.inputs[i].strides[w] = p.inputs[i].strides[d];
    }
  }
  p.rank = w + 1;
}

}  // namespace
}  // namespace mfx

extern "C" {

int mfx_elementwise(const mfx_ew_program* prog_in, void* stream) {
  using namespace mfx;
  if (!prog_in) return fail(MFX_E_INVALID, "null program");
  mfx_ew_program p = *prog_in;
  if (p.rank < 0 || p.rank > MFX_MAX_RANK) return fail(MFX_E_INVALID, "rank out of range");
  if (p.num_inputs < 0 || p.num_inputs > MFX_EW_MAX_INPUTS) return fail(MFX_E_INVALID, "too many inputs");
  if (p.num_instrs <= 0 || p.num_instrs > MFX_EW_MAX_INSTRS) return fail(MFX_E_INVALID, "bad instruction count");
  if (p.result < 0 || p.result >= MFX_EW_MAX_REGS) return fail(MFX_E_INVALID, "bad result register");
  if (!p.out || !valid_dtype(p.out_dtype)) return fail(MFX_E_INVALID, "bad output");
  int64_t numel = 1;
  for (int d = 0; d < p.rank; ++d) {
    if (p.dims[d] < 0) return fail(MFX_E_INVALID, "negative dim");
    numel *= p.dims[d];
  }
  for (int i = 0; i < p.num_inputs; ++i)
    if (!p.inputs[i].data || !valid_dtype(p.inputs[i].dtype)) return fail(MFX_E_INVALID, "bad input");
  bool written[MFX_EW_MAX_REGS] = {};
  for (int pc = 0; pc < p.num_instrs; ++pc) {
    const mfx_ew_instr& in = p.code[pc];
    if (in.op >= MFX_EW_NUM_OPS || in.dst >= MFX_EW_MAX_REGS)
      return fail(MFX_E_INVALID, "bad instruction");
    if (in.op == MFX_EW_LOAD && in.a >= p.num_inputs) return fail(MFX_E_INVALID, "load of a missing input");
    if (in.op == MFX_EW_IOTA && in.a >= p.rank) return fail(MFX_E_INVALID, "iota dim out of range");
    const int nsrc = in.op <= MFX_EW_IOTA ? 0 : in.op <= MFX_EW_COPY ? 1 : in.op <= MFX_EW_ATAN2 ? 2 : 3;
    const uint8_t srcs[3] = {in.a, in.b, in.c};
    for (int s = 0; s < nsrc; ++s)
      if (srcs[s] >= MFX_EW_MAX_REGS || !written[srcs[s]])
        return fail(MFX_E_INVALID, "instruction reads an unwritten register");
    written[in.dst] = true;
  }
  if (!written[p.result]) return fail(MFX_E_INVALID, "result register never written");
  if (numel == 0) return MFX_OK;
  int strided = 0;
  for (int d = 0; d < p.rank; ++d) strided |= p.out_strides[d] != 0;
  if (strided) {
    // Out-of-place layout: keep the dims as given (no collapsing).
  } else {
    collapse(p);
  }
  const int64_t blocks64 = (numel + kThreads - 1) / kThreads;
  const unsigned blocks = (unsigned)(blocks64 < 65536 ? blocks64 : 65536);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (numel < (1LL << 31))
    hipLaunchKernelGGL((ew_kernel<int32_t>), dim3(blocks), dim3(kThreads), 0, s, p, (int32_t)numel, strided);
  else
    hipLaunchKernelGGL((ew_kernel<int64_t>), dim3(blocks), dim3(kThreads), 0, s, p, numel, strided);
  return launch_status("ew_kernel");
}

int mfx_reduce(const mfx_reduce_args* a, void* stream) {
  using namespace mfx;
  if (!a || !a->in || !a->out) return fail(MFX_E_INVALID, "null reduce args");
  if (a->rank < 0 || a->rank > MFX_MAX_RANK) return fail(MFX_E_INVALID, "rank out of range");
  if (!valid_dtype(a->in_dtype) || !valid_dtype(a->out_dtype)) return fail(MFX_E_INVALID, "bad dtype");
  if (a->op < MFX_RED_SUM || a->op > MFX_RED_PROD) return fail(MFX_E_INVALID, "bad reduce op");
  ReduceMeta rm{};
  int64_t* meta = rm.m;
  int nk = 0, nr = 0;
  int64_t K = 1, R = 1;
  for (int d = 0; d < a->rank; ++d) {
    if (a->dims[d] < 0) return fail(MFX_E_INVALID, "negative dim");
    if (a->reduce_mask & (1u << d)) {
      meta[16 + nr] = a->dims[d];
      meta[24 + nr] = a->strides[d];
      ++nr;
      R *= a->dims[d];
    } else {
      meta[nk] = a->dims[d];
      meta[8 + nk] = a->strides[d];
      ++nk;
      K *= a->dims[d];
    }
  }
  if (K == 0) return MFX_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (R <= 64 || K >= 65536) {
    const int64_t b64 = (K + kThreads - 1) / kThreads;
    const unsigned blocks = (unsigned)(b64 < 65536 ? b64 : 65536);
    hipLaunchKernelGGL(reduce_thread_kernel, dim3(blocks), dim3(kThreads), 0, s, a->in, a->out, a->in_dtype,
                       a->out_dtype, a->op, a->init, nk, rm, nr, K, R);
  } else {
    const unsigned blocks = (unsigned)(K < 65536 ? K : 65536);
    hipLaunchKernelGGL(reduce_block_kernel, dim3(blocks), dim3(kThreads), 0, s, a->in, a->out, a->in_dtype,
                       a->out_dtype, a->op, a->init, nk, rm, nr, K, R);
  }
  return launch_status("reduce_kernel");
}

}  // extern "C"
