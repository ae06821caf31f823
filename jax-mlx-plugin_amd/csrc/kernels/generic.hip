// Generic ops for the graph regions the pattern matcher leaves unfused:
//   mfx_elementwise  one loop kernel runs a whole fused elementwise program
//                    (loads with broadcast strides, arithmetic, compare,
//                    select, iota, converts) per output element;
//   mfx_reduce       strided reduction over any subset of axes.
// Both are HBM-bound loop kernels; the host collapses contiguous dims so the
// common cases run with rank 1 or 2 index arithmetic.
#include <cstring>

#include "common.h"
#include "ew_math.h"

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

// Result of one arithmetic instruction for NV elements; opnd(e, k) is operand
// k (0: a, 1: b, 2: c) of element e.  The switch on the (uniform) opcode
// runs once for all NV elements.
#define MFX_EW_UN(expr)                    \
  _Pragma("unroll") for (int e = 0; e < NV; ++e) { \
    const float a = opnd(e, 0);            \
    v[e] = (expr);                         \
  }                                        \
  return;
#define MFX_EW_BIN(expr)                   \
  _Pragma("unroll") for (int e = 0; e < NV; ++e) { \
    const float a = opnd(e, 0), b = opnd(e, 1); \
    v[e] = (expr);                         \
  }                                        \
  return;
// Library math (tens of instructions each) runs as a rolled loop so the
// kernel keeps one copy of it.
#define MFX_EW_UN_SLOW(expr)               \
  _Pragma("nounroll") for (int e = 0; e < NV; ++e) { \
    const float a = opnd(e, 0);            \
    v[e] = (expr);                         \
  }                                        \
  return;
#define MFX_EW_BIN_SLOW(expr)              \
  _Pragma("nounroll") for (int e = 0; e < NV; ++e) { \
    const float a = opnd(e, 0), b = opnd(e, 1); \
    v[e] = (expr);                         \
  }                                        \
  return;
#define MFX_EW_TER(expr)                   \
  _Pragma("unroll") for (int e = 0; e < NV; ++e) { \
    const float a = opnd(e, 0), b = opnd(e, 1), c = opnd(e, 2); \
    v[e] = (expr);                         \
  }                                        \
  return;

template <int NV, typename Opnd>
__device__ __forceinline__ void apply_n(const mfx_ew_instr& in, Opnd&& opnd, float* v) {
  const bool is_int = in.flags & MFX_EW_FLAG_INT;
  switch (in.op) {
    case MFX_EW_NEG: MFX_EW_UN(-a)
    case MFX_EW_ABS: MFX_EW_UN(fabsf(a))
    case MFX_EW_EXP: MFX_EW_UN_SLOW(expf(a))
    case MFX_EW_EXPM1: MFX_EW_UN_SLOW(expm1f(a))
    case MFX_EW_LOG: MFX_EW_UN_SLOW(logf(a))
    case MFX_EW_LOG1P: MFX_EW_UN_SLOW(log1pf(a))
    case MFX_EW_SQRT: MFX_EW_UN(sqrtf(a))
    case MFX_EW_RSQRT: MFX_EW_UN(1.0f / sqrtf(a))
    case MFX_EW_TANH: MFX_EW_UN(mfx_tanh(a))
    case MFX_EW_LOGISTIC: MFX_EW_UN_SLOW(1.0f / (1.0f + expf(-a)))
    case MFX_EW_ERF: MFX_EW_UN_SLOW(erff(a))
    case MFX_EW_SIN: MFX_EW_UN_SLOW(sinf(a))
    case MFX_EW_COS: MFX_EW_UN_SLOW(cosf(a))
    case MFX_EW_FLOOR: MFX_EW_UN(floorf(a))
    case MFX_EW_CEIL: MFX_EW_UN(ceilf(a))
    case MFX_EW_ROUND_NE: MFX_EW_UN(rintf(a))
    case MFX_EW_SIGN: MFX_EW_UN(a > 0.f ? 1.f : (a < 0.f ? -1.f : a))
    case MFX_EW_NOT: MFX_EW_UN(is_int ? (float)(~(int32_t)a) : (a == 0.f ? 1.f : 0.f))
    case MFX_EW_ROUND_BF16: MFX_EW_UN(static_cast<float>(static_cast<bf16>(a)))
    case MFX_EW_ROUND_F16: MFX_EW_UN(static_cast<float>(static_cast<_Float16>(a)))
    case MFX_EW_TO_INT: MFX_EW_UN(truncf(a))
    case MFX_EW_IS_FINITE: MFX_EW_UN(isfinite(a) ? 1.f : 0.f)
    case MFX_EW_COPY: MFX_EW_UN(a)
    case MFX_EW_ADD: MFX_EW_BIN(a + b)
    case MFX_EW_SUB: MFX_EW_BIN(a - b)
    case MFX_EW_MUL: MFX_EW_BIN(a * b)
    case MFX_EW_DIV: MFX_EW_BIN(is_int ? truncf(a / b) : a / b)
    case MFX_EW_MAX: MFX_EW_BIN(nan_max(a, b))
    case MFX_EW_MIN: MFX_EW_BIN(nan_min(a, b))
    case MFX_EW_POW: MFX_EW_BIN_SLOW(powf(a, b))
    case MFX_EW_REM: MFX_EW_BIN_SLOW(fmodf(a, b))
    case MFX_EW_AND: MFX_EW_BIN(is_int ? (float)((int32_t)a & (int32_t)b) : ((a != 0.f && b != 0.f) ? 1.f : 0.f))
    case MFX_EW_OR: MFX_EW_BIN(is_int ? (float)((int32_t)a | (int32_t)b) : ((a != 0.f || b != 0.f) ? 1.f : 0.f))
    case MFX_EW_XOR: MFX_EW_BIN(is_int ? (float)((int32_t)a ^ (int32_t)b) : (((a != 0.f) != (b != 0.f)) ? 1.f : 0.f))
    case MFX_EW_EQ: MFX_EW_BIN(a == b ? 1.f : 0.f)
    case MFX_EW_NE: MFX_EW_BIN(a != b ? 1.f : 0.f)
    case MFX_EW_LT: MFX_EW_BIN(a < b ? 1.f : 0.f)
    case MFX_EW_LE: MFX_EW_BIN(a <= b ? 1.f : 0.f)
    case MFX_EW_GT: MFX_EW_BIN(a > b ? 1.f : 0.f)
    case MFX_EW_GE: MFX_EW_BIN(a >= b ? 1.f : 0.f)
    case MFX_EW_ATAN2: MFX_EW_BIN_SLOW(atan2f(a, b))
    case MFX_EW_SELECT: MFX_EW_TER(a != 0.f ? b : c)
    case MFX_EW_CLAMP: MFX_EW_TER(nan_min(nan_max(b, a), c))
    default:
#pragma unroll
      for (int e = 0; e < NV; ++e) v[e] = 0.f;
      return;
  }
}
#undef MFX_EW_UN
#undef MFX_EW_BIN
#undef MFX_EW_TER
#undef MFX_EW_UN_SLOW
#undef MFX_EW_BIN_SLOW

__device__ __forceinline__ float apply(const mfx_ew_instr& in, const float* r) {
  float v;
  apply_n<1>(in, [&](int, int k) { return r[k == 0 ? in.a : k == 1 ? in.b : in.c]; }, &v);
  return v;
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
        v = apply(in, r);
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

// Four consecutive elements of the innermost (collapsed) dim per thread and
// iteration: the output coordinates are decomposed once per four elements,
// each instruction is decoded once per four elements, and the loads and the
// store move four elements per instruction where the layout allows.  Input
// i's access mode is two bits of `modes`: 0 = contiguous along the inner dim
// and aligned for a vector load of its dtype, 1 = inner stride 0 (one value
// for all four), 2 = anything else (four scalar loads).  The output is
// contiguous, its inner dim a multiple of four and its pointer aligned for a
// four-element store.
constexpr int kV = 4;

// Inputs of the four-wide kernel are f32 or bf16 (checked on the host).
__device__ __forceinline__ void load4(const void* p, int dt, int64_t off, int64_t step, int mode, float* v) {
  if (dt == MFX_F32) {
    const float* f = static_cast<const float*>(p) + off;
    if (mode == 0) {
      const float4 w = *reinterpret_cast<const float4*>(f);
      v[0] = w.x; v[1] = w.y; v[2] = w.z; v[3] = w.w;
    } else if (mode == 1) {
      v[0] = v[1] = v[2] = v[3] = f[0];
    } else {
#pragma unroll
      for (int e = 0; e < kV; ++e) v[e] = f[e * step];
    }
    return;
  }
  const bf16* h = static_cast<const bf16*>(p) + off;
  if (mode == 0) {
    const uint2 w = *reinterpret_cast<const uint2*>(h);
    v[0] = __uint_as_float(w.x << 16); v[1] = __uint_as_float(w.x & 0xffff0000u);
    v[2] = __uint_as_float(w.y << 16); v[3] = __uint_as_float(w.y & 0xffff0000u);
  } else if (mode == 1) {
    v[0] = v[1] = v[2] = v[3] = static_cast<float>(h[0]);
  } else {
#pragma unroll
    for (int e = 0; e < kV; ++e) v[e] = static_cast<float>(h[e * step]);
  }
}

// Output of the four-wide kernel is f32 or bf16 (checked on the host).
__device__ __forceinline__ void store4(void* p, int dt, int64_t off, const float* v) {
  if (dt == MFX_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + off) = make_float4(v[0], v[1], v[2], v[3]);
    return;
  }
  bf16x4 w;
#pragma unroll
  for (int e = 0; e < kV; ++e) w[e] = static_cast<bf16>(v[e]);
  *reinterpret_cast<bf16x4*>(static_cast<bf16*>(p) + off) = w;
}

// The program's registers live in LDS, one 16-byte slot (four elements) per
// thread and register: lds[reg][thread] as float4, so every operand read and
// result write is one conflict-free ds_read_b128 / ds_write_b128 whose
// address is the thread's slot plus a uniform register offset.  (A register
// file indexed by a runtime register number cannot stay in VGPRs: the
// compiler lowers such accesses to select chains or scratch memory.)
template <typename IDX, int NREG>
__global__ __launch_bounds__(kThreads) void ew_kernel_v4(const mfx_ew_program prog, IDX nchunks, IDX inner_chunks,
                                                         uint32_t modes) {
  __shared__ float4 regs[NREG][kThreads];
  float4* mine = &regs[0][threadIdx.x];
  auto rd = [&](int i) __attribute__((always_inline)) { return mine[i * kThreads]; };
  auto wr = [&](int i, const float* v) __attribute__((always_inline)) {
    mine[i * kThreads] = make_float4(v[0], v[1], v[2], v[3]);
  };
  const int last = prog.rank - 1;
  for (IDX c = (IDX)blockIdx.x * kThreads + threadIdx.x; c < nchunks; c += (IDX)gridDim.x * kThreads) {
    IDX here[MFX_MAX_RANK];
    {
      const IDX outer = c / inner_chunks;
      IDX rem = outer;
      for (int d = last - 1; d >= 0; --d) {
        const IDX n = (IDX)prog.dims[d];
        here[d] = rem % n;
        rem /= n;
      }
      here[last] = (c - outer * inner_chunks) * kV;
    }
    // Every input is loaded before the program runs, so all loads of a
    // chunk are in flight together.
    float li[MFX_EW_MAX_INPUTS][kV];
#pragma unroll
    for (int i = 0; i < MFX_EW_MAX_INPUTS; ++i) {
      if (i < prog.num_inputs) {
        const mfx_ew_input& src = prog.inputs[i];
        int64_t off = 0;
        for (int d = 0; d <= last; ++d) off += (int64_t)here[d] * src.strides[d];
        load4(src.data, src.dtype, off, src.strides[last], (modes >> (2 * i)) & 3, li[i]);
      }
    }
    for (int pc = 0; pc < prog.num_instrs; ++pc) {
      const mfx_ew_instr in = prog.code[pc];
      float v[kV];
      if (in.op == MFX_EW_LOAD) {
        // Uniform branch on the input index keeps li in fixed registers.
#pragma unroll
        for (int i = 0; i < MFX_EW_MAX_INPUTS; ++i)
          if (in.a == i) {
#pragma unroll
            for (int e = 0; e < kV; ++e) v[e] = li[i][e];
          }
      } else if (in.op == MFX_EW_CONST) {
        v[0] = v[1] = v[2] = v[3] = in.imm;
      } else if (in.op == MFX_EW_IOTA) {
        const float base = (float)here[in.a];
#pragma unroll
        for (int e = 0; e < kV; ++e) v[e] = in.a == last ? base + (float)e : base;
      } else {
        const float4 a = rd(in.a);
        const float4 b = in.op > MFX_EW_COPY ? rd(in.b) : a;
        const float4 cc = in.op > MFX_EW_ATAN2 ? rd(in.c) : a;
        const float av[kV] = {a.x, a.y, a.z, a.w}, bv[kV] = {b.x, b.y, b.z, b.w}, cv[kV] = {cc.x, cc.y, cc.z, cc.w};
        auto opnd = [&](int e, int k) __attribute__((always_inline)) {
          return k == 0 ? av[e] : k == 1 ? bv[e] : cv[e];
        };
        apply_n<kV>(in, opnd, v);
      }
      wr(in.dst, v);
    }
    const float4 r = rd(prog.result);
    const float o[kV] = {r.x, r.y, r.z, r.w};
    store4(prog.out, prog.out_dtype, (int64_t)c * kV, o);
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

int dtype_bytes_of(int dt) {
  switch (dt) {
    case MFX_F32: case MFX_I32: case MFX_U32: return 4;
    case MFX_BF16: case MFX_F16: return 2;
    case MFX_PRED: case MFX_U8: case MFX_I8: return 1;
    case MFX_I64: case MFX_F64: return 8;
    default: return 0;
  }
}

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

// Native kernels generated per program (ew_jit.cpp).
bool ew_jit_launch(const mfx_ew_program& p, hipStream_t s, int* rc);
int ew_jit_prepare(const mfx_ew_program& p);

namespace {

// Validates prog_in and returns in p the program to run: dims collapsed
// where every input's strides allow it (contiguous outputs only).  Sets
// numel; returns MFX_OK or an error.
int normalise(const mfx_ew_program* prog_in, mfx_ew_program& p, int64_t& numel, bool need_ptrs) {
  if (!prog_in) return fail(MFX_E_INVALID, "null program");
  p = *prog_in;
  if (p.rank < 0 || p.rank > MFX_MAX_RANK) return fail(MFX_E_INVALID, "rank out of range");
  if (p.num_inputs < 0 || p.num_inputs > MFX_EW_MAX_INPUTS) return fail(MFX_E_INVALID, "too many inputs");
  if (p.num_instrs <= 0 || p.num_instrs > MFX_EW_MAX_INSTRS) return fail(MFX_E_INVALID, "bad instruction count");
  if (p.result < 0 || p.result >= MFX_EW_MAX_REGS) return fail(MFX_E_INVALID, "bad result register");
  if ((need_ptrs && !p.out) || !valid_dtype(p.out_dtype)) return fail(MFX_E_INVALID, "bad output");
  numel = 1;
  for (int d = 0; d < p.rank; ++d) {
    if (p.dims[d] < 0) return fail(MFX_E_INVALID, "negative dim");
    numel *= p.dims[d];
  }
  for (int i = 0; i < p.num_inputs; ++i)
    if ((need_ptrs && !p.inputs[i].data) || !valid_dtype(p.inputs[i].dtype)) return fail(MFX_E_INVALID, "bad input");
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
  int strided = 0;
  for (int d = 0; d < p.rank; ++d) strided |= p.out_strides[d] != 0;
  // A strided (out-of-place) output keeps the dims as given.
  if (!strided) collapse(p);
  return MFX_OK;
}

}  // namespace
}  // namespace mfx

extern "C" {

int mfx_ew_prepare(const mfx_ew_program* prog_in) {
  using namespace mfx;
  mfx_ew_program p;
  int64_t numel = 0;
  const int rc = normalise(prog_in, p, numel, false);
  if (rc != MFX_OK || numel == 0) return rc;
  return ew_jit_prepare(p);
}

int mfx_elementwise(const mfx_ew_program* prog_in, void* stream) {
  using namespace mfx;
  mfx_ew_program p;
  int64_t numel = 0;
  int rc = normalise(prog_in, p, numel, true);
  if (rc != MFX_OK || numel == 0) return rc;
  int strided = 0;
  for (int d = 0; d < p.rank; ++d) strided |= p.out_strides[d] != 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The program's own compiled kernel when hipRTC builds it; the
  // interpreter below otherwise.
  if (ew_jit_launch(p, s, &rc)) return rc;
  // Four elements per thread when the output is contiguous with an inner
  // dim that is a multiple of four.
  const int last = p.rank - 1;
  const int osz = dtype_bytes_of(p.out_dtype);
  bool fp_only = p.out_dtype == MFX_F32 || p.out_dtype == MFX_BF16;
  for (int i = 0; i < p.num_inputs; ++i)
    fp_only = fp_only && (p.inputs[i].dtype == MFX_F32 || p.inputs[i].dtype == MFX_BF16);
  if (fp_only && !strided && p.rank >= 1 && p.dims[last] % kV == 0 && osz > 0 &&
      (uintptr_t)p.out % (size_t)(osz * kV > 16 ? 16 : osz * kV) == 0) {
    uint32_t modes = 0;
    for (int i = 0; i < p.num_inputs; ++i) {
      const mfx_ew_input& in = p.inputs[i];
      const int isz = dtype_bytes_of(in.dtype);
      int mode = 2;
      if (in.strides[last] == 0) {
        mode = 1;
      } else if (in.strides[last] == 1) {
        bool aligned = (uintptr_t)in.data % (size_t)(isz * kV) == 0;
        for (int d = 0; d < last; ++d) aligned = aligned && in.strides[d] % kV == 0;
        if (aligned) mode = 0;
      }
      modes |= (uint32_t)mode << (2 * i);
    }
    const int64_t chunks = numel / kV;
    const int64_t inner_chunks = p.dims[last] / kV;
    int nreg = p.result + 1;
    for (int pc = 0; pc < p.num_instrs; ++pc) nreg = nreg > p.code[pc].dst + 1 ? nreg : p.code[pc].dst + 1;
    // One chunk per thread (up to 2^24 workgroups, then a grid-stride loop).
    const int64_t b64 = (chunks + kThreads - 1) / kThreads;
    const unsigned g = (unsigned)(b64 < (1 << 24) ? b64 : (1 << 24));
    const bool small = numel < (1LL << 31);
#define MFX_EW_V4(N)                                                                                      \
    if (small)                                                                                            \
      hipLaunchKernelGGL((ew_kernel_v4<int32_t, N>), dim3(g), dim3(kThreads), 0, s, p, (int32_t)chunks,   \
                         (int32_t)inner_chunks, modes);                                                  \
    else                                                                                                  \
      hipLaunchKernelGGL((ew_kernel_v4<int64_t, N>), dim3(g), dim3(kThreads), 0, s, p, chunks,           \
                         inner_chunks, modes);
    if (nreg <= 4) {
      MFX_EW_V4(4)
    } else if (nreg <= 8) {
      MFX_EW_V4(8)
    } else if (nreg <= 16) {
      MFX_EW_V4(16)
    } else {
      MFX_EW_V4(MFX_EW_MAX_REGS)
    }
#undef MFX_EW_V4
    return launch_status("ew_kernel_v4");
  }
  const int64_t blocks64 = (numel + kThreads - 1) / kThreads;
  const unsigned blocks = (unsigned)(blocks64 < 65536 ? blocks64 : 65536);
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
