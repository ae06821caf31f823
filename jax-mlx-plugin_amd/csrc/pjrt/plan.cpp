// Launch planner / executor for a rewritten module (see plan.h).
//
// Elementwise fusion: every value that must exist in memory (function result,
// operand of a GEMM / reduce / fused op, or an arithmetic value with several
// uses) is the root of one mfx_elementwise program; its expression tree
// inlines single-use arithmetic, converts, broadcasts, transposes, slices,
// unit reshapes, iotas and splat constants, with each leaf load given strides
// over the root's coordinates.  GEMM and reduce read transposed / broadcast /
// sliced operands in place through strides; a dot operand whose strides fit
// no GEMM layout is first copied to a canonical [batch, rows, cols] buffer.
#include "plan.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <set>
#include <sstream>

namespace mfxp {

int mfx_dtype(DType t) {
  switch (t) {
    case DType::kF32: return MFX_F32;
    case DType::kBF16: return MFX_BF16;
    case DType::kF16: return MFX_F16;
    case DType::kI32: return MFX_I32;
    case DType::kPred: return MFX_PRED;
    case DType::kI64: return MFX_I64;
    case DType::kU8: return MFX_U8;
    case DType::kI8: return MFX_I8;
    case DType::kU32: return MFX_U32;
    case DType::kF64: return MFX_F64;
    default: return -1;
  }
}

namespace {

struct Restart {
  int value;
};

const std::map<std::string, int>& unary_ops() {
  static const std::map<std::string, int> m = {
      {"stablehlo.negate", MFX_EW_NEG},
      {"stablehlo.abs", MFX_EW_ABS},
      {"stablehlo.exponential", MFX_EW_EXP},
      {"stablehlo.exponential_minus_one", MFX_EW_EXPM1},
      {"stablehlo.log", MFX_EW_LOG},
      {"stablehlo.log_plus_one", MFX_EW_LOG1P},
      {"stablehlo.sqrt", MFX_EW_SQRT},
      {"stablehlo.rsqrt", MFX_EW_RSQRT},
      {"stablehlo.tanh", MFX_EW_TANH},
      {"stablehlo.logistic", MFX_EW_LOGISTIC},
      {"chlo.erf", MFX_EW_ERF},
      {"stablehlo.sine", MFX_EW_SIN},
      {"stablehlo.cosine", MFX_EW_COS},
      {"stablehlo.floor", MFX_EW_FLOOR},
      {"stablehlo.ceil", MFX_EW_CEIL},
      {"stablehlo.round_nearest_even", MFX_EW_ROUND_NE},
      {"stablehlo.sign", MFX_EW_SIGN},
      {"stablehlo.not", MFX_EW_NOT},
      {"stablehlo.is_finite", MFX_EW_IS_FINITE},
      {"stablehlo.optimization_barrier", MFX_EW_COPY},
  };
  return m;
}

const std::map<std::string, int>& binary_ops() {
  static const std::map<std::string, int> m = {
      {"stablehlo.add", MFX_EW_ADD},          {"stablehlo.subtract", MFX_EW_SUB},
      {"stablehlo.multiply", MFX_EW_MUL},     {"stablehlo.divide", MFX_EW_DIV},
      {"stablehlo.maximum", MFX_EW_MAX},      {"stablehlo.minimum", MFX_EW_MIN},
      {"stablehlo.power", MFX_EW_POW},        {"stablehlo.remainder", MFX_EW_REM},
      {"stablehlo.and", MFX_EW_AND},          {"stablehlo.or", MFX_EW_OR},
      {"stablehlo.xor", MFX_EW_XOR},          {"stablehlo.atan2", MFX_EW_ATAN2},
  };
  return m;
}

bool is_int_type(DType t) { return !is_float(t) && t != DType::kPred && t != DType::kInvalid; }

int64_t elem_bytes(int mfx_code) {
  switch (mfx_code) {
    case MFX_F32: case MFX_I32: case MFX_U32: return 4;
    case MFX_BF16: case MFX_F16: return 2;
    case MFX_I64: case MFX_F64: return 8;
    default: return 1;
  }
}

enum class Cls { kArith, kView, kGen, kOther };

Cls classify(const Node& n) {
  const std::string& op = n.op;
  if (unary_ops().count(op) || binary_ops().count(op) || op == "stablehlo.compare" ||
      op == "stablehlo.select" || op == "stablehlo.clamp" || op == "stablehlo.convert")
    return Cls::kArith;
  if (op == "stablehlo.broadcast_in_dim" || op == "stablehlo.transpose" || op == "stablehlo.reshape" ||
      op == "stablehlo.slice")
    return Cls::kView;
  if (op == "stablehlo.iota" || op == "stablehlo.constant") return Cls::kGen;
  return Cls::kOther;
}

// Coordinate of one dim of a value as an affine function of root coordinates.
struct Lin {
  std::vector<int64_t> coef;
  int64_t off = 0;
};
using CMap = std::vector<Lin>;

struct ProgIn {
  int value;
  int64_t off;
  std::vector<int64_t> strides;
};

// Compiles the native kernel of an elementwise program at plan time, so the
// first Execute does not wait for it.  The placeholder pointers carry the
// alignment the run-time ones will have (buffers are 256-byte aligned; an
// input read at an element offset keeps that offset's alignment).  A program
// the compiler rejects runs on the interpreter: the result is ignored.
static void prepare_elementwise(const mfx_ew_program& prog, const std::vector<ProgIn>& ins) {
  mfx_ew_program p = prog;
  constexpr uintptr_t kBase = 1u << 20;
  p.out = reinterpret_cast<void*>(kBase);
  for (size_t i = 0; i < ins.size() && i < (size_t)MFX_EW_MAX_INPUTS; ++i)
    p.inputs[i].data = reinterpret_cast<const void*>(kBase + (uintptr_t)(ins[i].off * elem_bytes(p.inputs[i].dtype)));
  (void)mfx_ew_prepare(&p);
}

struct ProgBuild {
  int root = -1;
  int rank = 0;
  std::vector<mfx_ew_instr> code;  // dst = SSA index (reassigned later)
  std::vector<ProgIn> ins;
  std::map<std::string, int> memo;
};

class Planner {
 public:
  Planner(const Function& f, Plan& p) : f_(f), plan_(p) {}

  void build() {
    nvals_ = (int)f_.values.size();
    for (int v : f_.params) plan_.params_.push_back(f_.type(v));
    for (int v : f_.results) plan_.results_.push_back(f_.type(v));
    for (const Node& n : f_.nodes)
      if (classify(n) == Cls::kOther) check_supported(n);
    uses_.assign(nvals_, 0);
    for (const Node& n : f_.nodes)
      for (int v : n.in) uses_[v]++;
    for (int v : f_.results) uses_[v]++;
    need_.assign(nvals_, 0);
    for (int v : f_.results) need_[v] = 1;
    for (const Node& n : f_.nodes) {
      if (classify(n) != Cls::kOther) continue;
      for (int v : operand_needs(n)) need_[v] = 1;
    }
    mark_shared_values();
    // Programs may discover more values that must be materialised: iterate.
    for (int round = 0;; ++round) {
      if (round > 4 * nvals_ + 8) throw ParseError("planner did not converge");
      try {
        emit_all();
        break;
      } catch (const Restart& r) {
        need_[r.value] = 1;
      }
    }
    assign_locations();
  }

 private:
  const Function& f_;
  Plan& plan_;
  int nvals_ = 0;
  std::vector<int> uses_;
  std::vector<char> need_;
  // Per emitted step: values read and written (value ids; temps >= nvals_).
  struct StepIO {
    std::vector<int> reads, writes;
  };
  std::vector<StepIO> io_;
  // Launch arguments of GEMM and elementwise steps (by step index), for the
  // pass that fuses an elementwise program into the GEMM it consumes.
  struct GemmMeta {
    mfx_gemm_args g;
    int64_t aoff, boff;  // byte offsets into the A / B values
    int av, bv, out_v;
  };
  struct EwMeta {
    mfx_ew_program prog;
    std::vector<ProgIn> ins;
    int out_value;
  };
  std::map<size_t, GemmMeta> gemm_meta_;
  std::map<size_t, EwMeta> ew_meta_;
  // Launch arguments of SDPA forward / backward steps (by step index), for
  // the pass that hands a forward's output and row log-sum-exp to the
  // backward of the same attention.
  struct SdpaMeta {
    mfx_sdpa_args a;
    int q, k, v, out_v, mask, wq, ws_v;
    size_t ws;
    int64_t qo, ko, vo, mo;
  };
  struct SdpaBwdMeta {
    mfx_sdpa_bwd_args a;
    int q, k, v, g, dq, dk, dv, ws_v;
    size_t ws;
  };
  std::map<size_t, SdpaMeta> sdpa_meta_;
  std::map<size_t, SdpaBwdMeta> sdpa_bwd_meta_;
  std::vector<Type> temp_types_;
  std::vector<int64_t> temp_bytes_;
  std::shared_ptr<std::vector<Loc>> loc_ = std::make_shared<std::vector<Loc>>();

  const Type& ty(int v) const {
    return v < nvals_ ? f_.values[v].type : temp_types_[v - nvals_];
  }
  const Node* def(int v) const {
    if (v >= nvals_) return nullptr;
    int d = f_.values[v].def;
    return d < 0 ? nullptr : &f_.nodes[d];
  }
  int64_t bytes_of(int v) const {
    if (v >= nvals_ && temp_bytes_[v - nvals_] >= 0) return temp_bytes_[v - nvals_];
    return ty(v).bytes();
  }
  int new_temp(const Type& t, int64_t bytes = -1) {
    temp_types_.push_back(t);
    temp_bytes_.push_back(bytes);
    return nvals_ + (int)temp_types_.size() - 1;
  }

  // Plan-time bounds proof: every element a step will touch, given its dims,
  // strides and offset, lies inside the buffer of the value it names.  A
  // planning mistake then fails Compile instead of faulting on the device.
  int64_t numel_of(int v) const {
    const int64_t eb = dtype_bytes(ty(v).dtype);
    return eb > 0 ? bytes_of(v) / eb : 0;
  }
  void check_access(const char* what, int v, int64_t off, const std::vector<int64_t>& dims,
                    const std::vector<int64_t>& strides) const {
    int64_t lo = off, hi = off;
    for (size_t d = 0; d < dims.size(); ++d) {
      if (dims[d] <= 0) return;  // nothing is accessed
      const int64_t span = (dims[d] - 1) * strides[d];
      if (span < 0) lo += span;
      else hi += span;
    }
    if (lo < 0 || hi >= numel_of(v))
      throw ParseError(std::string("internal: planned ") + what + " access [" + std::to_string(lo) + ", " +
                       std::to_string(hi) + "] lies outside a buffer of " + std::to_string(numel_of(v)) +
                       " elements");
  }
  void check_access(const char* what, int v, int64_t off, const int64_t* dims, const int64_t* strides,
                    int rank) const {
    check_access(what, v, off, std::vector<int64_t>(dims, dims + rank),
                 std::vector<int64_t>(strides, strides + rank));
  }
  void check_dense(const char* what, int v, int64_t numel) const {
    if (numel > numel_of(v))
      throw ParseError(std::string("internal: planned ") + what + " of " + std::to_string(numel) +
                       " elements exceeds its buffer of " + std::to_string(numel_of(v)));
  }

  static void check_supported(const Node& n) {
    static const std::set<std::string> ok = {
        "stablehlo.dot_general", "stablehlo.dot", "stablehlo.reduce", "mfx.sdpa", "mfx.layer_norm",
        "mfx.rms_norm", "mfx.softmax", "mfx.log_softmax", "mfx.layer_norm_bwd", "mfx.sdpa_bwd",
        "stablehlo.concatenate"};
    if (!ok.count(n.op)) {
      std::string what = n.op;
      if (n.op == "stablehlo.custom_call") what += " @" + n.strs.at("target");
      throw ParseError("unsupported op " + what + " (not on the fused SDPA / norm path)");
    }
  }

  // Values an Other node reads from memory directly (after view tracing).
  // A multi-use arithmetic value needs its own buffer only when the
  // expression trees of two different programs reach it; uses inside one
  // tree share one interpreter register through the builder's memo.  Marking
  // a value changes the trees, so iterate to a fixed point.
  void mark_shared_values() {
    auto inner = [&](int u) {
      const Node* d = def(u);
      return d && !need_[u] && classify(*d) != Cls::kOther;
    };
    for (int round = 0; round < 4 * nvals_ + 8; ++round) {
      std::vector<int> owner(nvals_, -1);  // root reaching it; -2: several roots
      for (int r = 0; r < nvals_; ++r) {
        const Node* dr = def(r);
        if (!need_[r] || !dr || classify(*dr) == Cls::kOther) continue;
        std::vector<int> stack(dr->in.begin(), dr->in.end());
        while (!stack.empty()) {
          const int u = stack.back();
          stack.pop_back();
          if (!inner(u) || owner[u] == r) continue;
          if (owner[u] == -2) continue;
          if (owner[u] >= 0) {
            owner[u] = -2;
            continue;
          }
          owner[u] = r;
          for (int w : def(u)->in) stack.push_back(w);
        }
      }
      bool changed = false;
      for (const Node& n : f_.nodes) {
        if (classify(n) != Cls::kArith) continue;
        for (int v : n.out)
          if (uses_[v] > 1 && !need_[v] && owner[v] == -2) {
            need_[v] = 1;
            changed = true;
          }
      }
      if (!changed) return;
    }
  }

  std::vector<int> operand_needs(const Node& n) {
    std::vector<int> r;
    if (n.op == "stablehlo.dot_general" || n.op == "stablehlo.dot" || n.op == "stablehlo.reduce") {
      for (size_t i = 0; i < n.in.size(); ++i) {
        if (n.op == "stablehlo.reduce" && i == 1) continue;  // init: a constant
        r.push_back(trace_view(f_, n.in[i], true).base);
      }
    } else {
      r = n.in;
    }
    return r;
  }

  // ---- expression building ----
  static std::string key(int v, const CMap& m) {
    std::string k = std::to_string(v);
    for (const Lin& l : m) {
      k += "|" + std::to_string(l.off);
      for (int64_t c : l.coef) k += "," + std::to_string(c);
    }
    return k;
  }

  int emit(ProgBuild& pb, uint8_t op, int a = 0, int b = 0, int c = 0, float imm = 0.f, uint8_t flags = 0) {
    mfx_ew_instr in{};
    in.op = op;
    in.a = (uint8_t)a;
    in.b = (uint8_t)b;
    in.c = (uint8_t)c;
    in.imm = imm;
    in.flags = flags;
    pb.code.push_back(in);
    if (pb.code.size() > 200) throw Restart{pb.root};  // unreachable in practice
    return (int)pb.code.size() - 1;
  }

  int load(ProgBuild& pb, int v, const CMap& m) {
    auto cs = contiguous_strides(ty(v).dims);
    ProgIn in{v, 0, std::vector<int64_t>(pb.rank, 0)};
    for (size_t d = 0; d < m.size(); ++d) {
      in.off += cs[d] * m[d].off;
      for (int r = 0; r < pb.rank; ++r) in.strides[r] += cs[d] * m[d].coef[r];
    }
    int idx = -1;
    for (size_t i = 0; i < pb.ins.size(); ++i)
      if (pb.ins[i].value == v && pb.ins[i].off == in.off && pb.ins[i].strides == in.strides) idx = (int)i;
    if (idx < 0) {
      pb.ins.push_back(in);
      idx = (int)pb.ins.size() - 1;
    }
    // The LOAD operand is an input index, not an SSA value.
    mfx_ew_instr ld{};
    ld.op = MFX_EW_LOAD;
    ld.a = (uint8_t)idx;
    pb.code.push_back(ld);
    return (int)pb.code.size() - 1;
  }

  int build(ProgBuild& pb, int v, const CMap& m) {
    std::string k = key(v, m);
    auto it = pb.memo.find(k);
    if (it != pb.memo.end()) return it->second;
    int r = build_uncached(pb, v, m);
    pb.memo[k] = r;
    return r;
  }

  int build_uncached(ProgBuild& pb, int v, const CMap& m) {
    const Node* n = def(v);
    const bool is_root = v == pb.root;
    if (!n || (need_[v] && !is_root)) {
      if (n && n->op == "stablehlo.constant" && n->literal->splat) return emit(pb, MFX_EW_CONST, 0, 0, 0, (float)n->literal->values[0]);
      return load(pb, v, m);
    }
    Cls cl = classify(*n);
    const Type& t = ty(v);
    if (cl == Cls::kOther) return load(pb, v, m);
    if (cl == Cls::kGen) {
      if (n->op == "stablehlo.constant") {
        if (n->literal->splat) return emit(pb, MFX_EW_CONST, 0, 0, 0, (float)n->literal->values[0]);
        if (is_root) {
          // A non-splat constant as a root: copy from its uploaded buffer.
          throw ParseError("internal: constant root");
        }
        return load(pb, v, m);  // constants always have a buffer
      }
      // iota: the coordinate along its dim must be one root coordinate.
      int d = (int)n->ints.at("dim").at(0);
      const Lin& l = m[d];
      int which = -1, nz = 0;
      for (int r = 0; r < pb.rank; ++r)
        if (l.coef[r] != 0) {
          ++nz;
          which = r;
        }
      if (nz == 0) return emit(pb, MFX_EW_CONST, 0, 0, 0, (float)l.off);
      if (nz == 1 && l.coef[which] == 1 && l.off == 0) return emit(pb, MFX_EW_IOTA, which);
      if (is_root) throw ParseError("internal: iota root map");
      throw Restart{v};
    }
    if (cl == Cls::kView) {
      int x = n->in[0];
      const Type& xt = ty(x);
      CMap mx(xt.rank(), Lin{std::vector<int64_t>(pb.rank, 0), 0});
      if (n->op == "stablehlo.broadcast_in_dim") {
        const auto& bd = n->ints.at("dims");
        for (int i = 0; i < xt.rank(); ++i)
          if (!(xt.dims[i] == 1 && t.dims[bd[i]] != 1)) mx[i] = m[bd[i]];
      } else if (n->op == "stablehlo.transpose") {
        const auto& perm = n->ints.at("dims");
        for (size_t i = 0; i < perm.size(); ++i) mx[perm[i]] = m[i];
      } else if (n->op == "stablehlo.slice") {
        const auto& st = n->ints.at("start");
        const auto& sd = n->ints.at("stride");
        for (int i = 0; i < xt.rank(); ++i) {
          mx[i] = m[i];
          for (auto& c : mx[i].coef) c *= sd[i];
          mx[i].off = m[i].off * sd[i] + st[i];
        }
      } else {  // reshape
        std::vector<int> xs, vs;
        for (int i = 0; i < xt.rank(); ++i)
          if (xt.dims[i] != 1) xs.push_back(i);
        for (int i = 0; i < t.rank(); ++i)
          if (t.dims[i] != 1) vs.push_back(i);
        bool unit_only = xs.size() == vs.size();
        for (size_t i = 0; unit_only && i < xs.size(); ++i) unit_only = xt.dims[xs[i]] == t.dims[vs[i]];
        if (unit_only) {
          for (size_t i = 0; i < xs.size(); ++i) mx[xs[i]] = m[vs[i]];
        } else {
          // Same elements in the same row-major order: read x's buffer linearly.
          const Node* xn = def(x);
          bool has_buf = !xn || need_[x] || classify(*xn) == Cls::kOther ||
                         (xn->op == "stablehlo.constant" && !xn->literal->splat);
          if (!has_buf) throw Restart{x};
          auto cs = contiguous_strides(t.dims);
          Lin lin{std::vector<int64_t>(pb.rank, 0), 0};
          for (int d = 0; d < t.rank(); ++d) {
            lin.off += cs[d] * m[d].off;
            for (int r = 0; r < pb.rank; ++r) lin.coef[r] += cs[d] * m[d].coef[r];
          }
          // Express as a rank-1 view of x.
          CMap flat(1, lin);
          Type ft;
          ft.dtype = xt.dtype;
          ft.dims = {xt.numel()};
          int fv = flat_alias(x, ft);
          return load(pb, fv, flat);
        }
      }
      return build(pb, x, mx);
    }
    // Arithmetic.
    const std::string& op = n->op;
    if (op == "stablehlo.convert") {
      int a = build(pb, n->in[0], m);
      DType from = ty(n->in[0]).dtype, to = t.dtype;
      if (to == DType::kBF16 && from != DType::kBF16) return emit(pb, MFX_EW_ROUND_BF16, a);
      if (to == DType::kF16 && from != DType::kF16) return emit(pb, MFX_EW_ROUND_F16, a);
      if (is_int_type(to) && is_float(from)) return emit(pb, MFX_EW_TO_INT, a);
      if (to == DType::kPred && from != DType::kPred) {
        int z = emit(pb, MFX_EW_CONST, 0, 0, 0, 0.f);
        return emit(pb, MFX_EW_NE, a, z);
      }
      return a;
    }
    std::vector<int> args;
    for (int in : n->in) {
      const Type& it = ty(in);
      if (it.rank() == 0 && t.rank() > 0) {
        args.push_back(build(pb, in, CMap{}));
      } else {
        args.push_back(build(pb, in, m));
      }
    }
    const uint8_t iflag = is_int_type(ty(n->in[0]).dtype) ? MFX_EW_FLAG_INT : 0;
    auto u = unary_ops().find(op);
    if (u != unary_ops().end()) return emit(pb, (uint8_t)u->second, args[0], 0, 0, 0.f, iflag);
    auto b = binary_ops().find(op);
    if (b != binary_ops().end()) return emit(pb, (uint8_t)b->second, args[0], args[1], 0, 0.f, iflag);
    if (op == "stablehlo.compare") {
      const std::string& d = n->strs.at("comparison_direction");
      uint8_t code = d == "EQ" ? MFX_EW_EQ : d == "NE" ? MFX_EW_NE : d == "LT" ? MFX_EW_LT
                   : d == "LE" ? MFX_EW_LE : d == "GT" ? MFX_EW_GT : MFX_EW_GE;
      return emit(pb, code, args[0], args[1]);
    }
    if (op == "stablehlo.select") return emit(pb, MFX_EW_SELECT, args[0], args[1], args[2]);
    if (op == "stablehlo.clamp") return emit(pb, MFX_EW_CLAMP, args[0], args[1], args[2]);
    throw ParseError("internal: unhandled elementwise op " + op);
  }

  // A rank-1 alias value for reading x linearly (same location as x).
  std::map<int, int> flat_alias_;
  std::vector<std::pair<int, int>> aliases_;  // (alias value, of value)
  int flat_alias(int x, const Type& ft) {
    auto it = flat_alias_.find(x);
    if (it != flat_alias_.end()) return it->second;
    int a = new_temp(ft);
    flat_alias_[x] = a;
    aliases_.push_back({a, x});
    return a;
  }

  // Converts SSA-indexed code into a program with at most 32 live registers.
  bool finalize(ProgBuild& pb, int result, mfx_ew_program& prog) {
    const int n = (int)pb.code.size();
    if (n > MFX_EW_MAX_INSTRS || pb.ins.size() > MFX_EW_MAX_INPUTS) return false;
    auto nsrc = [](uint8_t op) { return op <= MFX_EW_IOTA ? 0 : op <= MFX_EW_COPY ? 1 : op <= MFX_EW_ATAN2 ? 2 : 3; };
    std::vector<int> last(n, -1);
    for (int i = 0; i < n; ++i) {
      const mfx_ew_instr& in = pb.code[i];
      const int srcs[3] = {in.a, in.b, in.c};
      for (int s = 0; s < nsrc(in.op); ++s) last[srcs[s]] = i;
    }
    last[result] = n;
    std::vector<int> reg(n, -1);
    std::vector<int> free_regs;
    for (int r = MFX_EW_MAX_REGS - 1; r >= 0; --r) free_regs.push_back(r);
    std::vector<mfx_ew_instr> out;
    for (int i = 0; i < n; ++i) {
      mfx_ew_instr in = pb.code[i];
      const int ns = nsrc(in.op);
      int srcs[3] = {in.a, in.b, in.c};
      for (int s = 0; s < ns; ++s) srcs[s] = reg[srcs[s]];
      // Free sources whose last use is this instruction (before allocating dst).
      for (int s = 0; s < ns; ++s) {
        int orig = s == 0 ? pb.code[i].a : s == 1 ? pb.code[i].b : pb.code[i].c;
        if (last[orig] == i && std::find(free_regs.begin(), free_regs.end(), reg[orig]) == free_regs.end())
          free_regs.push_back(reg[orig]);
      }
      if (free_regs.empty()) return false;
      if (last[i] < 0) {
        // Dead value (memoised but unused): still needs a register slot briefly.
      }
      reg[i] = free_regs.back();
      free_regs.pop_back();
      if (last[i] < 0) free_regs.push_back(reg[i]);
      if (ns >= 1) in.a = (uint8_t)srcs[0];
      if (ns >= 2) in.b = (uint8_t)srcs[1];
      if (ns >= 3) in.c = (uint8_t)srcs[2];
      in.dst = (uint8_t)reg[i];
      out.push_back(in);
    }
    std::memset(&prog, 0, sizeof prog);
    prog.rank = pb.rank;
    prog.num_instrs = (int)out.size();
    for (int i = 0; i < prog.num_instrs; ++i) prog.code[i] = out[i];
    prog.result = reg[result];
    prog.num_inputs = (int)pb.ins.size();
    return true;
  }

  // Emits the program computing value `root` into its own buffer.
  void emit_program(int root, int out_value) {
    const Type& t = ty(root);
    if (t.rank() > MFX_MAX_RANK) throw ParseError("rank above 8 is not supported");
    if (mfx_dtype(t.dtype) < 0) throw ParseError("unsupported element type " + std::string(dtype_name(t.dtype)));
    ProgBuild pb;
    pb.root = root;
    pb.rank = t.rank();
    CMap id(t.rank(), Lin{std::vector<int64_t>(t.rank(), 0), 0});
    for (int d = 0; d < t.rank(); ++d) id[d].coef[d] = 1;
    int result = build(pb, root, id);
    if (pb.code.empty()) result = emit(pb, MFX_EW_CONST);
    mfx_ew_program prog;
    if (!finalize(pb, result, prog)) {
      // Too large: materialise the largest direct operand and retry.
      const Node* n = def(root);
      int pick = -1;
      if (n)
        for (int in : n->in)
          if (!need_[in] && def(in) && classify(*def(in)) != Cls::kOther) pick = in;
      if (pick < 0) throw ParseError("elementwise program exceeds the interpreter limits");
      throw Restart{pick};
    }
    prog.out_dtype = mfx_dtype(t.dtype);
    for (int d = 0; d < t.rank(); ++d) prog.dims[d] = t.dims[d];
    for (size_t i = 0; i < pb.ins.size(); ++i) {
      int dt = mfx_dtype(ty(pb.ins[i].value).dtype);
      if (dt < 0) throw ParseError("unsupported element type in elementwise input");
      prog.inputs[i].dtype = dt;
      for (int d = 0; d < pb.rank; ++d) prog.inputs[i].strides[d] = pb.ins[i].strides[d];
      check_access("elementwise load", pb.ins[i].value, pb.ins[i].off, prog.dims, prog.inputs[i].strides, pb.rank);
    }
    check_dense("elementwise result", out_value, t.numel());
    prepare_elementwise(prog, pb.ins);
    auto ins = pb.ins;
    StepIO io;
    for (auto& in : ins) io.reads.push_back(in.value);
    io.writes.push_back(out_value);
    Step s;
    s.kind = "elementwise";
    s.label = def(root) ? def(root)->op : "param";
    s.bytes = (double)t.bytes();
    auto loc = loc_;
    Plan* plan = &plan_;
    ew_meta_[plan_.steps_.size()] = EwMeta{prog, ins, out_value};
    s.run = [prog, ins, out_value, loc, plan](const ExecBuffers& b, std::string& err) {
      mfx_ew_program p = prog;
      p.out = plan->ptr((*loc)[out_value], b);
      for (size_t i = 0; i < ins.size(); ++i) {
        char* base = (char*)plan->ptr((*loc)[ins[i].value], b);
        p.inputs[i].data = base + ins[i].off * elem_bytes(p.inputs[i].dtype);
      }
      int rc = mfx_elementwise(&p, b.stream);
      if (rc != MFX_OK) err = mfx_last_error();
      return rc;
    };
    plan_.steps_.push_back(std::move(s));
    io_.push_back(io);
  }

  // ---- non-elementwise steps ----

  struct Grouped {
    int64_t size = 1, stride = 0;
  };
  // Collapses dims (in the given order) into one extent + stride, if the
  // strides are mutually contiguous (unit dims ignored).
  static bool group(const std::vector<int64_t>& dims, const std::vector<int64_t>& strides,
                    const std::vector<int64_t>& which, Grouped& g) {
    g = Grouped{};
    int64_t expect = -1;
    for (size_t i = which.size(); i-- > 0;) {
      int64_t d = dims[which[i]], s = strides[which[i]];
      if (d == 1) continue;
      if (expect < 0) {
        g.stride = s;
      } else if (s != expect) {
        return false;
      }
      g.size *= d;
      expect = s * d;
    }
    if (expect < 0) g.stride = 0;
    return true;
  }

  void emit_gemm(const Node& n) {
    std::vector<int64_t> lb, rb, lc, rc;
    if (n.op == "stablehlo.dot") {
      lc = {(int64_t)ty(n.in[0]).rank() - 1};
      rc = {0};
    } else {
      auto get = [&](const char* k) {
        auto it = n.ints.find(k);
        return it == n.ints.end() ? std::vector<int64_t>{} : it->second;
      };
      lb = get("lhs_batching_dims");
      rb = get("rhs_batching_dims");
      lc = get("lhs_contracting_dims");
      rc = get("rhs_contracting_dims");
    }
    const int out_v = n.out[0];
    int lhs = n.in[0], rhs = n.in[1];
    const Type& lt = ty(lhs);
    const Type& rt = ty(rhs);
    std::vector<int64_t> lf, rf;
    for (int i = 0; i < lt.rank(); ++i)
      if (std::find(lb.begin(), lb.end(), i) == lb.end() && std::find(lc.begin(), lc.end(), i) == lc.end())
        lf.push_back(i);
    for (int i = 0; i < rt.rank(); ++i)
      if (std::find(rb.begin(), rb.end(), i) == rb.end() && std::find(rc.begin(), rc.end(), i) == rc.end())
        rf.push_back(i);
    DType cd = ty(out_v).dtype;
    DType ad = lt.dtype == rt.dtype ? lt.dtype : DType::kF32;
    if (ad != DType::kF32 && ad != DType::kBF16 && ad != DType::kF16)
      throw ParseError("dot_general on " + std::string(dtype_name(ad)) + " is not supported");
    if (cd != DType::kF32 && cd != DType::kBF16 && cd != DType::kF16)
      throw ParseError("dot_general result type " + std::string(dtype_name(cd)) + " is not supported");
    // Operand A as [batch, M, K]; B as [batch, K, N].
    struct Opnd {
      int value;
      int64_t offset;
      Grouped b, m, k;  // for B: m plays N
      bool trans;
      int64_t ld;
    };
    auto layout = [&](int v, const std::vector<int64_t>& bd, const std::vector<int64_t>& fd,
                      const std::vector<int64_t>& kd, bool is_a, Opnd& o) -> bool {
      if (ty(v).dtype != ad) return false;
      StridedView sv;
      if (v < nvals_) {
        sv = trace_view(f_, v, true);
      } else {
        sv.base = v;
        sv.dims = ty(v).dims;
        sv.strides = contiguous_strides(sv.dims);
      }
      Grouped gb, gf, gk;
      if (!group(sv.dims, sv.strides, bd, gb) || !group(sv.dims, sv.strides, fd, gf) ||
          !group(sv.dims, sv.strides, kd, gk))
        return false;
      o.value = sv.base;
      o.offset = sv.offset;
      o.b = gb;
      o.m = gf;
      o.k = gk;
      // A row-major [m][k]: k unit stride (ld = m stride) or, transposed, m unit stride.
      int64_t fs = gf.size > 1 ? gf.stride : 0, ks = gk.size > 1 ? gk.stride : 0;
      if (ks == 1 || (ks == 0 && gk.size <= 1)) {
        o.trans = !is_a;
        o.ld = std::max<int64_t>(fs, gk.size);
        if (fs == 0) o.ld = gk.size;
        return o.ld >= gk.size && (gf.size <= 1 || fs >= gk.size);
      }
      if (fs == 1 || (fs == 0 && gf.size <= 1)) {
        o.trans = is_a;
        o.ld = std::max<int64_t>(ks, gf.size);
        return ks >= gf.size;
      }
      return false;
    };
    Opnd A{}, B{};
    bool okA = layout(lhs, lb, lf, lc, true, A);
    bool okB = layout(rhs, rb, rf, rc, false, B);
    auto canon = [&](int v, const std::vector<int64_t>& bd, const std::vector<int64_t>& fd,
                     const std::vector<int64_t>& kd, bool is_a) {
      // Copy to a contiguous [b..., f..., k...] (A) or [b..., k..., f...] (B) buffer.
      std::vector<int64_t> perm = bd;
      if (is_a) {
        perm.insert(perm.end(), fd.begin(), fd.end());
        perm.insert(perm.end(), kd.begin(), kd.end());
      } else {
        perm.insert(perm.end(), kd.begin(), kd.end());
        perm.insert(perm.end(), fd.begin(), fd.end());
      }
      const Type& vt = ty(v);
      Type tt;
      tt.dtype = ad;
      for (int64_t p : perm) tt.dims.push_back(vt.dims[p]);
      int tmp = new_temp(tt);
      // Program: out[i...] = v[permuted i...]
      canon_copy(v, perm, tmp);
      return tmp;
    };
    std::vector<int64_t> nb, nf, nk;
    for (size_t i = 0; i < lb.size(); ++i) nb.push_back((int64_t)i);
    if (!okA) {
      int t = canon(lhs, lb, lf, lc, true);
      std::vector<int64_t> f2, k2;
      for (size_t i = 0; i < lf.size(); ++i) f2.push_back((int64_t)(lb.size() + i));
      for (size_t i = 0; i < lc.size(); ++i) k2.push_back((int64_t)(lb.size() + lf.size() + i));
      if (!layout(t, nb, f2, k2, true, A)) throw ParseError("internal: canonical A layout");
    }
    if (!okB) {
      int t = canon(rhs, rb, rf, rc, false);
      std::vector<int64_t> k2, f2;
      for (size_t i = 0; i < rc.size(); ++i) k2.push_back((int64_t)(rb.size() + i));
      for (size_t i = 0; i < rf.size(); ++i) f2.push_back((int64_t)(rb.size() + rc.size() + i));
      if (!layout(t, nb, f2, k2, false, B)) throw ParseError("internal: canonical B layout");
    }
    const int64_t batch = std::max<int64_t>(A.b.size, 1), M = A.m.size, K = A.k.size, N = B.m.size;
    if (B.k.size != K || std::max<int64_t>(B.b.size, 1) != batch)
      throw ParseError("dot_general operand extents disagree");
    mfx_gemm_args g{};
    g.dtype = mfx_dtype(ad);
    g.c_dtype = mfx_dtype(cd);
    g.batch = batch;
    g.m = M;
    g.n = N;
    g.k = K;
    g.lda = A.ld;
    g.ldb = B.ld;
    g.ldc = N;
    g.stride_a = A.b.size > 1 ? A.b.stride : 0;
    g.stride_b = B.b.size > 1 ? B.b.stride : 0;
    g.stride_c = M * N;
    g.trans_a = A.trans ? 1 : 0;
    g.trans_b = B.trans ? 1 : 0;
    // Row-major A(m, k) sits at m*lda + k, or k*lda + m when transposed;
    // B(k, n) at k*ldb + n, or n*ldb + k when transposed.
    check_access("gemm A", A.value, A.offset, {batch, M, K},
                 {g.stride_a, A.trans ? 1 : g.lda, A.trans ? g.lda : 1});
    check_access("gemm B", B.value, B.offset, {batch, K, N},
                 {g.stride_b, B.trans ? 1 : g.ldb, B.trans ? g.ldb : 1});
    check_dense("gemm C", out_v, batch * M * N);
    // Row-major B[k][n] wants n unit stride; `layout` reports trans when k is unit.
    StepIO io;
    io.reads = {A.value, B.value};
    io.writes = {out_v};
    const int64_t aoff = A.offset * dtype_bytes(ad), boff = B.offset * dtype_bytes(ad);
    const int av = A.value, bv = B.value;
    auto loc = loc_;
    Plan* plan = &plan_;
    Step s;
    s.kind = "gemm";
    s.label = "dot_general " + std::to_string(batch) + "x" + std::to_string(M) + "x" + std::to_string(N) + "x" +
              std::to_string(K);
    s.flops = 2.0 * batch * M * N * K;
    gemm_meta_[plan_.steps_.size()] = GemmMeta{g, aoff, boff, av, bv, out_v};
    s.run = [g, aoff, boff, av, bv, out_v, loc, plan](const ExecBuffers& b, std::string& err) {
      mfx_gemm_args a = g;
      a.a = (char*)plan->ptr((*loc)[av], b) + aoff;
      a.b = (char*)plan->ptr((*loc)[bv], b) + boff;
      a.c = plan->ptr((*loc)[out_v], b);
      int rc = mfx_gemm(&a, b.stream);
      if (rc != MFX_OK) err = mfx_last_error();
      return rc;
    };
    plan_.steps_.push_back(std::move(s));
    io_.push_back(io);
  }

  // tmp[i...] = v at permuted coordinates (perm[j] = source dim of tmp dim j).
  void canon_copy(int v, const std::vector<int64_t>& perm, int tmp) {
    const Type& tt = ty(tmp);
    StridedView sv = trace_view(f_, v, true);
    mfx_ew_program prog{};
    prog.rank = tt.rank();
    for (int d = 0; d < tt.rank(); ++d) {
      prog.dims[d] = tt.dims[d];
      prog.inputs[0].strides[d] = sv.strides[perm[d]];
    }
    prog.num_inputs = 1;
    prog.inputs[0].dtype = mfx_dtype(ty(sv.base).dtype);
    prog.num_instrs = 1;
    prog.code[0].op = MFX_EW_LOAD;
    prog.code[0].dst = 0;
    prog.code[0].a = 0;
    prog.result = 0;
    prog.out_dtype = mfx_dtype(tt.dtype);
    const int base = sv.base;
    check_access("canonical copy load", base, sv.offset, prog.dims, prog.inputs[0].strides, prog.rank);
    check_dense("canonical copy", tmp, tt.numel());
    const int64_t off = sv.offset * dtype_bytes(ty(sv.base).dtype);
    auto loc = loc_;
    Plan* plan = &plan_;
    Step s;
    s.kind = "elementwise";
    s.label = "canonical copy for dot_general";
    s.bytes = (double)tt.bytes();
    s.run = [prog, base, off, tmp, loc, plan](const ExecBuffers& b, std::string& err) {
      mfx_ew_program p = prog;
      p.inputs[0].data = (char*)plan->ptr((*loc)[base], b) + off;
      p.out = plan->ptr((*loc)[tmp], b);
      int rc = mfx_elementwise(&p, b.stream);
      if (rc != MFX_OK) err = mfx_last_error();
      return rc;
    };
    plan_.steps_.push_back(std::move(s));
    io_.push_back(StepIO{{base}, {tmp}});
  }

  void emit_reduce(const Node& n) {
    if (n.in.size() != 2 || n.out.size() != 1) throw ParseError("multi-operand reduce is not supported");
    const std::string& kind = n.strs.at("reduce");
    int op = kind == "stablehlo.add" ? MFX_RED_SUM : kind == "stablehlo.maximum" ? MFX_RED_MAX
           : kind == "stablehlo.minimum" ? MFX_RED_MIN : kind == "stablehlo.multiply" ? MFX_RED_PROD : -1;
    if (op < 0) throw ParseError("reduce with " + kind + " is not supported");
    const Node* init = def(n.in[1]);
    if (!init || init->op != "stablehlo.constant") throw ParseError("reduce init must be a constant");
    StridedView sv = trace_view(f_, n.in[0], true);
    if ((int)sv.dims.size() > MFX_MAX_RANK) throw ParseError("reduce rank above 8");
    mfx_reduce_args a{};
    a.rank = (int)sv.dims.size();
    a.op = op;
    a.init = (float)init->literal->values[0];
    for (int d = 0; d < a.rank; ++d) {
      a.dims[d] = sv.dims[d];
      a.strides[d] = sv.strides[d];
    }
    for (int64_t d : n.ints.at("dimensions")) a.reduce_mask |= 1u << d;
    a.in_dtype = mfx_dtype(ty(sv.base).dtype);
    a.out_dtype = mfx_dtype(ty(n.out[0]).dtype);
    if (a.in_dtype < 0 || a.out_dtype < 0) throw ParseError("reduce dtype not supported");
    const int base = sv.base, out_v = n.out[0];
    check_access("reduce input", base, sv.offset, a.dims, a.strides, a.rank);
    check_dense("reduce result", out_v, ty(out_v).numel());
    const int64_t off = sv.offset * dtype_bytes(ty(base).dtype);
    auto loc = loc_;
    Plan* plan = &plan_;
    Step s;
    s.kind = "reduce";
    s.label = kind;
    s.run = [a, base, off, out_v, loc, plan](const ExecBuffers& b, std::string& err) {
      mfx_reduce_args r = a;
      r.in = (char*)plan->ptr((*loc)[base], b) + off;
      r.out = plan->ptr((*loc)[out_v], b);
      int rc = mfx_reduce(&r, b.stream);
      if (rc != MFX_OK) err = mfx_last_error();
      return rc;
    };
    plan_.steps_.push_back(std::move(s));
    io_.push_back(StepIO{{base}, {out_v}});
  }

  void emit_norm(const Node& n) {
    const int x = n.in[0], out_v = n.out[0];
    const Type& t = ty(x);
    int gamma = -1, beta = -1;
    int k = 1;
    if (n.ints.count("has_gamma") && n.ints.at("has_gamma").at(0)) gamma = n.in[k++];
    if (n.ints.count("has_beta") && n.ints.at("has_beta").at(0)) beta = n.in[k++];
    mfx_norm_args a{};
    a.n = t.rank() ? t.dims.back() : 1;
    a.rows = a.n ? t.numel() / a.n : 0;
    a.x_row_stride = a.y_row_stride = a.n;
    a.eps = n.nums.count("eps") ? (float)n.nums.at("eps") : 0.f;
    a.dtype = mfx_dtype(t.dtype);
    a.param_dtype = gamma >= 0 ? mfx_dtype(ty(gamma).dtype) : beta >= 0 ? mfx_dtype(ty(beta).dtype) : a.dtype;
    if (gamma >= 0 && beta >= 0 && ty(gamma).dtype != ty(beta).dtype) throw ParseError("gamma/beta dtypes differ");
    check_dense("norm input", x, a.rows * a.n);
    check_dense("norm result", out_v, a.rows * a.n);
    if (gamma >= 0) check_dense("norm gamma", gamma, a.n);
    if (beta >= 0) check_dense("norm beta", beta, a.n);
    int which = n.op == "mfx.layer_norm" ? 0 : n.op == "mfx.rms_norm" ? 1 : n.op == "mfx.softmax" ? 2 : 3;
    auto loc = loc_;
    Plan* plan = &plan_;
    Step s;
    s.kind = n.op.substr(4);
    s.label = n.op;
    s.bytes = 2.0 * t.bytes();
    s.run = [a, x, out_v, gamma, beta, which, loc, plan](const ExecBuffers& b, std::string& err) {
      mfx_norm_args r = a;
      r.x = plan->ptr((*loc)[x], b);
      r.y = plan->ptr((*loc)[out_v], b);
      r.gamma = gamma >= 0 ? plan->ptr((*loc)[gamma], b) : nullptr;
      r.beta = beta >= 0 ? plan->ptr((*loc)[beta], b) : nullptr;
      int rc = which == 0   ? mfx_layer_norm(&r, b.stream)
               : which == 1 ? mfx_rms_norm(&r, b.stream)
               : which == 2 ? mfx_softmax(&r, b.stream)
                            : mfx_log_softmax(&r, b.stream);
      if (rc != MFX_OK) err = mfx_last_error();
      return rc;
    };
    plan_.steps_.push_back(std::move(s));
    StepIO io{{x}, {out_v}};
    if (gamma >= 0) io.reads.push_back(gamma);
    if (beta >= 0) io.reads.push_back(beta);
    io_.push_back(io);
  }

  // custom_call @mlx_layer_norm_bwd: (x, gamma, dy) -> (dx, dgamma, dbeta).
  void emit_norm_bwd(const Node& n) {
    const int x = n.in[0], gamma = n.in[1], dy = n.in[2];
    const int dx = n.out[0], dg = n.out[1], db = n.out[2];
    const Type& t = ty(x);
    mfx_norm_bwd_args a{};
    a.n = t.dims.back();
    a.rows = a.n ? t.numel() / a.n : 0;
    a.x_row_stride = a.dy_row_stride = a.dx_row_stride = a.n;
    a.eps = (float)n.nums.at("eps");
    a.dtype = mfx_dtype(t.dtype);
    a.param_dtype = mfx_dtype(ty(dg).dtype);
    if (ty(dy).dtype != t.dtype || ty(dx).dtype != t.dtype || ty(gamma).dtype != ty(dg).dtype)
      throw ParseError("mlx_layer_norm_bwd: x / grad_out / dx and weight / dweight dtypes must match");
    if (a.dtype != MFX_F32 && a.dtype != MFX_BF16 && a.dtype != MFX_F16)
      throw ParseError("mlx_layer_norm_bwd: x must be f32, bf16 or f16");
    if (a.param_dtype != MFX_F32 && a.param_dtype != MFX_BF16 && a.param_dtype != MFX_F16)
      throw ParseError("mlx_layer_norm_bwd: weight must be f32, bf16 or f16");
    check_dense("norm bwd x", x, a.rows * a.n);
    check_dense("norm bwd dy", dy, a.rows * a.n);
    check_dense("norm bwd dx", dx, a.rows * a.n);
    check_dense("norm bwd gamma", gamma, a.n);
    check_dense("norm bwd dgamma", dg, a.n);
    check_dense("norm bwd dbeta", db, a.n);
    mfx_norm_bwd_args probe = a;
    probe.x = probe.dy = probe.gamma = (void*)0x10000;
    probe.dx = probe.dgamma = probe.dbeta = (void*)0x10000;
    const size_t ws = mfx_layer_norm_bwd_workspace_size(&probe);
    int ws_v = -1;
    if (ws > 0) {
      Type wt;
      wt.dtype = DType::kU8;
      wt.dims = {(int64_t)ws};
      ws_v = new_temp(wt);
    }
    auto loc = loc_;
    Plan* plan = &plan_;
    Step s;
    s.kind = "layer_norm_bwd";
    s.label = "mfx.layer_norm_bwd";
    s.bytes = 3.0 * t.bytes();
    s.run = [a, x, gamma, dy, dx, dg, db, ws_v, ws, loc, plan](const ExecBuffers& b, std::string& err) {
      mfx_norm_bwd_args r = a;
      r.x = plan->ptr((*loc)[x], b);
      r.gamma = plan->ptr((*loc)[gamma], b);
      r.dy = plan->ptr((*loc)[dy], b);
      r.dx = plan->ptr((*loc)[dx], b);
      r.dgamma = plan->ptr((*loc)[dg], b);
      r.dbeta = plan->ptr((*loc)[db], b);
      if (ws_v >= 0) {
        r.workspace = plan->ptr((*loc)[ws_v], b);
        r.workspace_bytes = ws;
      }
      int rc = mfx_layer_norm_bwd(&r, b.stream);
      if (rc != MFX_OK) err = mfx_last_error();
      return rc;
    };
    plan_.steps_.push_back(std::move(s));
    StepIO io{{x, gamma, dy}, {dx, dg, db}};
    if (ws_v >= 0) io.writes.push_back(ws_v);
    io_.push_back(io);
  }

  // custom_call @mlx_sdpa_bwd: BTNH (q, k, v, dO) -> (dq, dk, dv).
  void emit_sdpa_bwd(const Node& n) {
    const auto& sh = n.ints.at("shape");
    const int64_t B = sh[0], N = sh[1], K = sh[2], T = sh[3], S = sh[4], H = sh[5], Hv = sh[6];
    mfx_sdpa_bwd_args a{};
    a.B = B;
    a.Hq = N;
    a.Hkv = K;
    a.Tq = T;
    a.Tk = S;
    a.D = H;
    a.Dv = Hv;
    auto btnh = [](int64_t* st, int64_t t, int64_t heads, int64_t d) {
      st[0] = t * heads * d;
      st[1] = d;
      st[2] = heads * d;
      st[3] = 1;
    };
    btnh(a.q_strides, T, N, H);
    btnh(a.dq_strides, T, N, H);
    btnh(a.k_strides, S, K, H);
    btnh(a.dk_strides, S, K, H);
    btnh(a.v_strides, S, K, Hv);
    btnh(a.dv_strides, S, K, Hv);
    btnh(a.do_strides, T, N, Hv);
    a.scale = (float)n.nums.at("scale");
    const DType dt = ty(n.in[0]).dtype;
    a.dtype = mfx_dtype(dt);
    for (int v : n.in)
      if (ty(v).dtype != dt) throw ParseError("mlx_sdpa_bwd operands must share one dtype");
    for (int v : n.out)
      if (ty(v).dtype != dt) throw ParseError("mlx_sdpa_bwd results must have the operands' dtype");
    if (a.dtype != MFX_F32 && a.dtype != MFX_BF16 && a.dtype != MFX_F16)
      throw ParseError("mlx_sdpa_bwd: dtype must be f32, bf16 or f16");
    for (int i = 0; i < 4; ++i) check_dense("sdpa bwd operand", n.in[i], ty(n.in[i]).numel());
    for (int i = 0; i < 3; ++i) check_dense("sdpa bwd result", n.out[i], ty(n.out[i]).numel());
    mfx_sdpa_bwd_args probe = a;
    probe.q = probe.k = probe.v = probe.dout = (void*)0x10000;
    probe.dq = probe.dk = probe.dv = (void*)0x10000;
    const size_t ws = mfx_sdpa_bwd_workspace_size(&probe);
    if (!ws) throw ParseError(std::string("mlx_sdpa_bwd: ") + mfx_last_error());
    Type wt;
    wt.dtype = DType::kU8;
    wt.dims = {(int64_t)ws};
    const int ws_v = new_temp(wt);
    const SdpaBwdMeta m{a, n.in[0], n.in[1], n.in[2], n.in[3], n.out[0], n.out[1], n.out[2], ws_v, ws};
    sdpa_bwd_meta_[plan_.steps_.size()] = m;
    plan_.steps_.push_back(sdpa_bwd_step(m, -1, -1));
    io_.push_back(StepIO{{m.q, m.k, m.v, m.g}, {m.dq, m.dk, m.dv, m.ws_v}});
  }

  // The backward step; with fwd_out >= 0 it reads that forward output and
  // the row log-sum-exp in value lse instead of recomputing them.
  Step sdpa_bwd_step(const SdpaBwdMeta& m, int fwd_out, int lse) {
    auto loc = loc_;
    Plan* plan = &plan_;
    const mfx_sdpa_bwd_args& a = m.a;
    const double B = a.B, N = a.Hq, T = a.Tq, S = a.Tk, H = a.D, Hv = a.Dv;
    Step s;
    s.kind = "sdpa_bwd";
    s.label = fwd_out >= 0 ? "mfx.sdpa_bwd (forward's out and lse)" : "mfx.sdpa_bwd";
    // backward (S, dP, dV, dK, and S, dP, dQ), plus the recomputed forward (S, PV)
    s.flops = 2.0 * B * N * T * S * (4 * H + 3 * Hv) + (fwd_out >= 0 ? 0.0 : 2.0 * B * N * T * S * (H + Hv));
    s.run = [m, fwd_out, lse, loc, plan](const ExecBuffers& b, std::string& err) {
      mfx_sdpa_bwd_args r = m.a;
      r.q = plan->ptr((*loc)[m.q], b);
      r.k = plan->ptr((*loc)[m.k], b);
      r.v = plan->ptr((*loc)[m.v], b);
      r.dout = plan->ptr((*loc)[m.g], b);
      r.dq = plan->ptr((*loc)[m.dq], b);
      r.dk = plan->ptr((*loc)[m.dk], b);
      r.dv = plan->ptr((*loc)[m.dv], b);
      r.workspace = plan->ptr((*loc)[m.ws_v], b);
      r.workspace_bytes = m.ws;
      if (fwd_out >= 0) {
        r.fwd_out = plan->ptr((*loc)[fwd_out], b);
        r.fwd_lse = static_cast<const float*>(plan->ptr((*loc)[lse], b));
      }
      int rc = mfx_sdpa_bwd(&r, b.stream);
      if (rc != MFX_OK) err = mfx_last_error();
      return rc;
    };
    return s;
  }

  void emit_sdpa(const Node& n) {
    const auto& sh = n.ints.at("shape");
    mfx_sdpa_args a{};
    a.B = sh[0];
    a.Hq = sh[1];
    a.Hkv = sh[2];
    a.Tq = sh[3];
    a.Tk = sh[4];
    a.D = sh[5];
    a.Dv = sh[6];
    for (int i = 0; i < 4; ++i) {
      a.q_strides[i] = n.ints.at("q_strides")[i];
      a.k_strides[i] = n.ints.at("k_strides")[i];
      a.v_strides[i] = n.ints.at("v_strides")[i];
      a.o_strides[i] = n.ints.at("o_strides")[i];
    }
    a.scale = (float)n.nums.at("scale");
    a.causal = (int32_t)n.ints.at("causal").at(0);
    const int q = n.in[0], k = n.in[1], v = n.in[2], out_v = n.out[0];
    const DType dt = ty(q).dtype;
    a.dtype = mfx_dtype(dt);
    a.q_rms_eps = n.ints.count("q_rms") ? (float)n.nums.at("q_rms_eps") : -1.f;
    int wq = n.ints.count("q_rms_weight_index") ? n.in[n.ints.at("q_rms_weight_index").at(0)] : -1;
    std::vector<int64_t> offs = n.ints.count("offsets") ? n.ints.at("offsets") : std::vector<int64_t>{0, 0, 0, 0};
    const int mask_kind = (int)n.ints.at("mask_kind").at(0);
    int mask = -1;
    int64_t moff = 0;
    if (mask_kind) {
      for (int i = 0; i < 4; ++i) a.mask_strides[i] = n.ints.at("mask_strides")[i];
      mask = n.in[3];
      moff = offs[3];
      if (mask_kind == 2) {
        // Boolean predicate -> additive fp32 mask (0 where kept, `neg` where not).
        Type mt = ty(mask);
        Type ft;
        ft.dtype = DType::kF32;
        ft.dims = mt.dims;
        int tmp = new_temp(ft);
        mfx_ew_program prog{};
        prog.rank = mt.rank();
        auto cs = contiguous_strides(mt.dims);
        for (int d = 0; d < mt.rank(); ++d) {
          prog.dims[d] = mt.dims[d];
          prog.inputs[0].strides[d] = cs[d];
        }
        prog.num_inputs = 1;
        prog.inputs[0].dtype = mfx_dtype(mt.dtype);
        prog.code[0] = mfx_ew_instr{MFX_EW_LOAD, 0, 0, 0, 0, 0, {0, 0}, 0.f};
        prog.code[1] = mfx_ew_instr{MFX_EW_CONST, 1, 0, 0, 0, 0, {0, 0}, 0.f};
        prog.code[2] = mfx_ew_instr{MFX_EW_CONST, 2, 0, 0, 0, 0, {0, 0}, (float)n.nums.at("mask_neg")};
        prog.code[3] = mfx_ew_instr{MFX_EW_SELECT, 3, 0, 1, 2, 0, {0, 0}, 0.f};
        prog.num_instrs = 4;
        prog.result = 3;
        prog.out_dtype = MFX_F32;
        if (prog.rank > MFX_MAX_RANK) throw ParseError("mask rank above 8");
        auto loc = loc_;
        Plan* plan = &plan_;
        Step s;
        s.kind = "elementwise";
        s.label = "attention mask to additive";
        const int pred = mask;
        s.run = [prog, pred, tmp, loc, plan](const ExecBuffers& b, std::string& err) {
          mfx_ew_program p = prog;
          p.inputs[0].data = plan->ptr((*loc)[pred], b);
          p.out = plan->ptr((*loc)[tmp], b);
          int rc = mfx_elementwise(&p, b.stream);
          if (rc != MFX_OK) err = mfx_last_error();
          return rc;
        };
        plan_.steps_.push_back(std::move(s));
        io_.push_back(StepIO{{pred}, {tmp}});
        mask = tmp;
        a.mask_dtype = MFX_F32;
      } else {
        a.mask_dtype = mfx_dtype(ty(mask).dtype);
      }
    }
    // Workspace (split-KV partials, a normalised copy of q) from the arena.
    // The kernel is chosen at run time from the operands' alignment, so the
    // size is the larger of two probes: every buffer 256-byte aligned (arena
    // and pool buffers) plus each operand's element offset, and every operand
    // one element off 16-byte alignment (a caller's view of odd alignment).
    const int pb = dtype_bytes(dt);
    const int64_t mb = mask >= 0 ? dtype_bytes(ty(mask).dtype) : 0;
    size_t ws = 0;
    for (int64_t skew : {(int64_t)0, (int64_t)1}) {
      mfx_sdpa_args probe = a;
      const uintptr_t base = 0x10000;
      probe.q = (void*)(base + (offs[0] + skew) * pb);
      probe.k = (void*)(base + (offs[1] + skew) * pb);
      probe.v = (void*)(base + (offs[2] + skew) * pb);
      probe.out = (void*)base;
      probe.mask = mask >= 0 ? (void*)(base + (moff + skew) * mb) : nullptr;
      probe.q_rms_weight = wq >= 0 ? (void*)base : nullptr;
      ws = std::max(ws, mfx_sdpa_workspace_size(&probe));
    }
    int ws_v = -1;
    if (ws > 0) {
      Type wt;
      wt.dtype = DType::kU8;
      wt.dims = {(int64_t)ws};
      ws_v = new_temp(wt);
    }
    if (ty(k).dtype != dt || ty(v).dtype != dt || ty(out_v).dtype != dt)
      throw ParseError("internal: sdpa operand dtypes differ");
    check_access("sdpa q", q, offs[0], {a.B, a.Hq, a.Tq, a.D}, std::vector<int64_t>(a.q_strides, a.q_strides + 4));
    check_access("sdpa k", k, offs[1], {a.B, a.Hkv, a.Tk, a.D}, std::vector<int64_t>(a.k_strides, a.k_strides + 4));
    check_access("sdpa v", v, offs[2], {a.B, a.Hkv, a.Tk, a.Dv},
                 std::vector<int64_t>(a.v_strides, a.v_strides + 4));
    check_access("sdpa out", out_v, 0, {a.B, a.Hq, a.Tq, a.Dv}, std::vector<int64_t>(a.o_strides, a.o_strides + 4));
    if (mask >= 0)
      check_access("sdpa mask", mask, moff, {a.B, a.Hq, a.Tq, a.Tk},
                   std::vector<int64_t>(a.mask_strides, a.mask_strides + 4));
    if (wq >= 0) check_dense("sdpa q-norm weight", wq, a.D);
    const int eb = dtype_bytes(dt);
    const int64_t mo = moff * (mask >= 0 ? dtype_bytes(ty(mask).dtype) : 0);
    const SdpaMeta m{a, q, k, v, out_v, mask, wq, ws_v, ws, offs[0] * eb, offs[1] * eb, offs[2] * eb, mo};
    sdpa_meta_[plan_.steps_.size()] = m;
    plan_.steps_.push_back(sdpa_step(m, -1));
    StepIO io{{q, k, v}, {out_v}};
    if (mask >= 0) io.reads.push_back(mask);
    if (wq >= 0) io.reads.push_back(wq);
    if (ws_v >= 0) io.writes.push_back(ws_v);
    io_.push_back(io);
  }

  // The forward step; with lse >= 0 it also writes the row log-sum-exp there.
  Step sdpa_step(const SdpaMeta& m, int lse) {
    auto loc = loc_;
    Plan* plan = &plan_;
    const mfx_sdpa_args& a = m.a;
    Step s;
    s.kind = "sdpa";
    s.label = std::string(a.causal ? "sdpa causal" : "sdpa") + (lse >= 0 ? " (+ lse)" : "");
    double keys = a.causal ? (double)a.Tq * (a.Tq + 1) / 2.0 : (double)a.Tq * a.Tk;
    s.flops = 2.0 * a.B * a.Hq * keys * (a.D + a.Dv);
    s.run = [m, lse, loc, plan](const ExecBuffers& b, std::string& err) {
      mfx_sdpa_args r = m.a;
      r.q = (char*)plan->ptr((*loc)[m.q], b) + m.qo;
      r.k = (char*)plan->ptr((*loc)[m.k], b) + m.ko;
      r.v = (char*)plan->ptr((*loc)[m.v], b) + m.vo;
      r.out = plan->ptr((*loc)[m.out_v], b);
      r.mask = m.mask >= 0 ? (char*)plan->ptr((*loc)[m.mask], b) + m.mo : nullptr;
      r.q_rms_weight = m.wq >= 0 ? plan->ptr((*loc)[m.wq], b) : nullptr;
      if (m.ws_v >= 0) {
        r.workspace = plan->ptr((*loc)[m.ws_v], b);
        r.workspace_bytes = m.ws;
      }
      if (lse >= 0) r.lse = static_cast<float*>(plan->ptr((*loc)[lse], b));
      int rc = mfx_sdpa_fwd(&r, b.stream);
      if (rc != MFX_OK) err = mfx_last_error();
      return rc;
    };
    return s;
  }

  // A backward step whose q, k and v are the operands of an earlier forward
  // step with the same shape, scale and no mask, causal limit or q RMSNorm
  // (a training step's attention and its gradient): the forward also writes
  // its row log-sum-exp, and the backward reads it and the forward's output
  // instead of recomputing both (same forward kernel, so the same bits).
  // Several backward steps of one forward (two VJPs with different
  // cotangents, a Jacobian) share the one lse value that forward writes.
  void link_sdpa_backward() {
    std::map<size_t, int> fwd_lse;  // forward step index -> its lse value
    for (auto& bw : sdpa_bwd_meta_) {
      const SdpaBwdMeta& m = bw.second;
      const mfx_sdpa_bwd_args& ba = m.a;
      if (ba.mask || ba.causal) continue;
      for (auto& fw : sdpa_meta_) {
        if (fw.first >= bw.first) break;
        const SdpaMeta& f = fw.second;
        const mfx_sdpa_args& fa = f.a;
        if (resolve_alias(f.q) != resolve_alias(m.q) || resolve_alias(f.k) != resolve_alias(m.k) ||
            resolve_alias(f.v) != resolve_alias(m.v))
          continue;
        if (f.qo || f.ko || f.vo || f.mask >= 0 || fa.causal || fa.q_rms_eps >= 0.f || f.wq >= 0) continue;
        if (fa.B != ba.B || fa.Hq != ba.Hq || fa.Hkv != ba.Hkv || fa.Tq != ba.Tq || fa.Tk != ba.Tk || fa.D != ba.D ||
            fa.Dv != ba.Dv || fa.scale != ba.scale || fa.dtype != ba.dtype)
          continue;
        bool same = true;
        for (int i = 0; i < 4; ++i)
          same = same && fa.q_strides[i] == ba.q_strides[i] && fa.k_strides[i] == ba.k_strides[i] &&
                 fa.v_strides[i] == ba.v_strides[i];
        if (!same) continue;
        // Backward workspace without the recomputed output.
        mfx_sdpa_bwd_args probe = ba;
        probe.q = probe.k = probe.v = probe.dout = (void*)0x10000;
        probe.dq = probe.dk = probe.dv = (void*)0x10000;
        probe.fwd_out = (void*)0x10000;
        probe.fwd_lse = (const float*)0x10000;
        for (int i = 0; i < 4; ++i) probe.fwd_out_strides[i] = fa.o_strides[i];
        const size_t ws = mfx_sdpa_bwd_workspace_size(&probe);
        if (!ws) continue;
        int lse;
        auto linked = fwd_lse.find(fw.first);
        if (linked != fwd_lse.end()) {
          lse = linked->second;
        } else {
          Type lt;
          lt.dtype = DType::kF32;
          lt.dims = {fa.B * fa.Hq * fa.Tq};
          lse = new_temp(lt);
          fwd_lse[fw.first] = lse;
          plan_.steps_[fw.first] = sdpa_step(f, lse);
          io_[fw.first].writes.push_back(lse);
        }
        Type wt;
        wt.dtype = DType::kU8;
        wt.dims = {(int64_t)ws};
        SdpaBwdMeta mb = m;
        mb.a.fwd_out_strides[0] = fa.o_strides[0];
        mb.a.fwd_out_strides[1] = fa.o_strides[1];
        mb.a.fwd_out_strides[2] = fa.o_strides[2];
        mb.a.fwd_out_strides[3] = fa.o_strides[3];
        mb.ws_v = new_temp(wt);
        mb.ws = ws;
        plan_.steps_[bw.first] = sdpa_bwd_step(mb, f.out_v, lse);
        io_[bw.first] = StepIO{{mb.q, mb.k, mb.v, mb.g, f.out_v, lse}, {mb.dq, mb.dk, mb.dv, mb.ws_v}};
        break;
      }
    }
  }

  void emit_concat(const Node& n) {
    const int out_v = n.out[0];
    const Type& ot = ty(out_v);
    int64_t dim = n.ints.at("dimension").empty() ? 0 : n.ints.at("dimension")[0];
    auto cs = contiguous_strides(ot.dims);
    int64_t pos = 0;
    for (int in : n.in) {
      const Type& it = ty(in);
      mfx_ew_program prog{};
      prog.rank = it.rank();
      auto ics = contiguous_strides(it.dims);
      for (int d = 0; d < it.rank(); ++d) {
        prog.dims[d] = it.dims[d];
        prog.inputs[0].strides[d] = ics[d];
        prog.out_strides[d] = cs[d];
      }
      prog.num_inputs = 1;
      prog.inputs[0].dtype = mfx_dtype(it.dtype);
      prog.code[0] = mfx_ew_instr{MFX_EW_LOAD, 0, 0, 0, 0, 0, {0, 0}, 0.f};
      prog.num_instrs = 1;
      prog.result = 0;
      prog.out_dtype = mfx_dtype(ot.dtype);
      check_dense("concatenate operand", in, it.numel());
      check_access("concatenate store", out_v, pos * cs[dim], prog.dims, prog.out_strides, prog.rank);
      const int64_t off = pos * cs[dim] * dtype_bytes(ot.dtype);
      pos += it.dims[dim];
      auto loc = loc_;
      Plan* plan = &plan_;
      Step s;
      s.kind = "elementwise";
      s.label = "concatenate";
      s.run = [prog, in, out_v, off, loc, plan](const ExecBuffers& b, std::string& err) {
        mfx_ew_program p = prog;
        p.inputs[0].data = plan->ptr((*loc)[in], b);
        p.out = (char*)plan->ptr((*loc)[out_v], b) + off;
        int rc = mfx_elementwise(&p, b.stream);
        if (rc != MFX_OK) err = mfx_last_error();
        return rc;
      };
      plan_.steps_.push_back(std::move(s));
      io_.push_back(StepIO{{in}, {out_v}});
    }
  }

  void emit_all() {
    plan_.steps_.clear();
    io_.clear();
    gemm_meta_.clear();
    ew_meta_.clear();
    sdpa_meta_.clear();
    sdpa_bwd_meta_.clear();
    temp_types_.clear();
    temp_bytes_.clear();
    flat_alias_.clear();
    aliases_.clear();
    alias_of_.clear();
    result_copy_.clear();
    for (const Node& n : f_.nodes) {
      Cls cl = classify(n);
      if (cl == Cls::kOther) {
        if (n.op == "stablehlo.dot_general" || n.op == "stablehlo.dot") emit_gemm(n);
        else if (n.op == "stablehlo.reduce") emit_reduce(n);
        else if (n.op == "mfx.sdpa") emit_sdpa(n);
        else if (n.op == "stablehlo.concatenate") emit_concat(n);
        else if (n.op == "mfx.layer_norm_bwd") emit_norm_bwd(n);
        else if (n.op == "mfx.sdpa_bwd") emit_sdpa_bwd(n);
        else emit_norm(n);
        continue;
      }
      for (int v : n.out) {
        if (!need_[v]) continue;
        if (n.op == "stablehlo.constant" && !n.literal->splat) continue;  // uploaded buffer
        // A materialised reshape / same-type convert of a materialised value
        // shares its buffer (results keep their own buffers).
        if ((n.op == "stablehlo.reshape" ||
             (n.op == "stablehlo.convert" && ty(n.in[0]).dtype == ty(v).dtype)) &&
            !is_result(v) && has_buffer(n.in[0])) {
          alias_of_[v] = n.in[0];
          continue;
        }
        emit_program(v, v);
      }
    }
    // Results that are parameters / constants / duplicates: copy into outputs.
    std::set<int> seen;
    for (size_t j = 0; j < f_.results.size(); ++j) {
      int v = f_.results[j];
      const Node* n = def(v);
      bool produced = n && !(n->op == "stablehlo.constant" && !n->literal->splat);
      if (!produced || seen.count(v) || alias_of_.count(v)) {
        int tmp = new_temp(ty(v));
        result_copy_[j] = tmp;
        emit_copy(v, tmp);
      }
      seen.insert(v);
    }
    link_sdpa_backward();  // rewrites steps in place: before the pass that merges steps
    fuse_gemm_epilogues();
  }

  // A GEMM step followed by an elementwise step that is the only reader of
  // the GEMM result, at the result's own index, becomes one launch: the tile
  // kernel evaluates the program on its accumulators (mfx_gemm_ew) and the
  // GEMM result gets no buffer.  Run-time pointers the fused kernel does not
  // take (alignment) fall back to the GEMM writing into the program's f32
  // output, then the program in place there: same values, two launches.
  void fuse_gemm_epilogues() {
    std::vector<Step> steps;
    std::vector<StepIO> io;
    const size_t n = plan_.steps_.size();
    for (size_t i = 0; i < n; ++i) {
      if (i + 1 < n && try_fuse(i, steps, io)) {
        ++i;
        continue;
      }
      steps.push_back(std::move(plan_.steps_[i]));
      io.push_back(io_[i]);
    }
    plan_.steps_ = std::move(steps);
    io_ = std::move(io);
  }

  bool try_fuse(size_t i, std::vector<Step>& steps, std::vector<StepIO>& io) {
    auto gi = gemm_meta_.find(i);
    auto ei = ew_meta_.find(i + 1);
    if (gi == gemm_meta_.end() || ei == ew_meta_.end()) return false;
    const GemmMeta G = gi->second;
    const EwMeta E = ei->second;
    const int gv = resolve_alias(G.out_v);
    if (E.prog.out_dtype != MFX_F32) return false;
    for (int r : f_.results)
      if (resolve_alias(r) == gv) return false;
    for (size_t j = 0; j < io_.size(); ++j) {
      if (j == i + 1) continue;
      for (int v : io_[j].reads)
        if (resolve_alias(v) == gv) return false;
    }
    int ci = -1;
    for (size_t k = 0; k < E.ins.size(); ++k) {
      if (resolve_alias(E.ins[k].value) != gv) continue;
      if (ci >= 0 || E.ins[k].off != 0) return false;
      ci = (int)k;
    }
    if (ci < 0) return false;
    // Plan-time check with placeholder pointers of the run-time alignment
    // (buffers are 256-byte aligned; views keep their byte offsets).
    constexpr uintptr_t kBase = 1u << 20;
    mfx_gemm_args g = G.g;
    g.a = reinterpret_cast<const void*>(kBase + (uintptr_t)G.aoff);
    g.b = reinterpret_cast<const void*>(kBase + (uintptr_t)G.boff);
    g.c = nullptr;
    mfx_ew_program p = E.prog;
    p.out = reinterpret_cast<void*>(kBase);
    for (size_t k = 0; k < E.ins.size(); ++k)
      p.inputs[k].data =
          reinterpret_cast<const void*>(kBase + (uintptr_t)(E.ins[k].off * elem_bytes(p.inputs[k].dtype)));
    if (mfx_gemm_ew_check(&g, &p, ci) != MFX_OK) return false;
    (void)mfx_gemm_ew_prepare(&g, &p, ci);  // compiles now when a device is current
    Step s;
    s.kind = "gemm_ew";
    s.label = plan_.steps_[i].label + " + " + plan_.steps_[i + 1].label;
    s.flops = plan_.steps_[i].flops;
    s.bytes = plan_.steps_[i + 1].bytes;
    auto loc = loc_;
    Plan* plan = &plan_;
    const mfx_gemm_args g0 = G.g;
    const mfx_ew_program p0 = E.prog;
    const std::vector<ProgIn> ins = E.ins;
    const int out_value = E.out_value;
    s.run = [G, g0, p0, ins, ci, out_value, loc, plan](const ExecBuffers& b, std::string& err) {
      mfx_gemm_args a = g0;
      a.a = (char*)plan->ptr((*loc)[G.av], b) + G.aoff;
      a.b = (char*)plan->ptr((*loc)[G.bv], b) + G.boff;
      a.c = nullptr;
      mfx_ew_program p = p0;
      p.out = plan->ptr((*loc)[out_value], b);
      for (size_t k = 0; k < ins.size(); ++k) {
        if ((int)k == ci) continue;
        char* base = (char*)plan->ptr((*loc)[ins[k].value], b);
        p.inputs[k].data = base + ins[k].off * elem_bytes(p.inputs[k].dtype);
      }
      int rc = mfx_gemm_ew(&a, &p, ci, b.stream);
      if (rc == MFX_E_UNSUPPORTED) {
        a.c = p.out;
        rc = mfx_gemm(&a, b.stream);
        if (rc == MFX_OK) {
          p.inputs[ci].data = p.out;
          rc = mfx_elementwise(&p, b.stream);
        }
      }
      if (rc != MFX_OK) err = mfx_last_error();
      return rc;
    };
    StepIO sio;
    sio.reads = {G.av, G.bv};
    for (size_t k = 0; k < ins.size(); ++k)
      if ((int)k != ci) sio.reads.push_back(ins[k].value);
    sio.writes = {out_value};
    steps.push_back(std::move(s));
    io.push_back(sio);
    return true;
  }

  std::map<int, int> alias_of_;
  std::map<size_t, int> result_copy_;

  bool is_result(int v) const { return std::find(f_.results.begin(), f_.results.end(), v) != f_.results.end(); }
  bool has_buffer(int v) const {
    const Node* n = def(v);
    if (!n) return true;
    if (n->op == "stablehlo.constant") return !n->literal->splat;
    return need_[v] || classify(*n) == Cls::kOther;
  }

  void emit_copy(int src, int dst) {
    auto loc = loc_;
    Plan* plan = &plan_;
    const int64_t nbytes = ty(src).bytes();
    Step s;
    s.kind = "copy";
    s.label = "result copy";
    s.run = [src, dst, nbytes, loc, plan](const ExecBuffers& b, std::string& err) {
      if (nbytes == 0) return (int)MFX_OK;
      hipError_t e = hipMemcpyAsync(plan->ptr((*loc)[dst], b), plan->ptr((*loc)[src], b), nbytes,
                                    hipMemcpyDeviceToDevice, b.stream);
      if (e != hipSuccess) {
        err = std::string("hipMemcpyAsync: ") + hipGetErrorString(e);
        return (int)MFX_E_HIP;
      }
      return (int)MFX_OK;
    };
    plan_.steps_.push_back(std::move(s));
    io_.push_back(StepIO{{src}, {dst}});
  }

  // ---- locations ----
  void assign_locations() {
    const int total = nvals_ + (int)temp_types_.size();
    loc_->assign(total, Loc{});
    for (size_t i = 0; i < f_.params.size(); ++i) (*loc_)[f_.params[i]] = Loc{Loc::kParam, (int)i, 0};
    // Constants with buffers.
    for (const Node& n : f_.nodes)
      if (n.op == "stablehlo.constant" && !n.literal->splat) {
        plan_.const_host_.push_back(n.literal);
        (*loc_)[n.out[0]] = Loc{Loc::kConst, (int)plan_.const_host_.size() - 1, 0};
      }
    // Outputs.
    for (size_t j = 0; j < f_.results.size(); ++j) {
      auto it = result_copy_.find(j);
      int v = it != result_copy_.end() ? it->second : f_.results[j];
      (*loc_)[v] = Loc{Loc::kOutput, (int)j, 0};
    }
    // Liveness over steps for arena values.
    std::vector<int> first(total, -1), last(total, -1);
    for (size_t s = 0; s < io_.size(); ++s) {
      for (int v : io_[s].writes) {
        v = resolve_alias(v);
        if (first[v] < 0) first[v] = (int)s;
        last[v] = std::max(last[v], (int)s);
      }
      for (int v : io_[s].reads) {
        v = resolve_alias(v);
        if (first[v] < 0) first[v] = (int)s;
        last[v] = std::max(last[v], (int)s);
      }
    }
    struct Block {
      int64_t off, size;
      int until;
    };
    std::vector<Block> live;
    int64_t top = 0;
    auto align = [](int64_t x) { return (x + 255) / 256 * 256; };
    for (size_t s = 0; s < io_.size(); ++s) {
      // Retire blocks whose last use is before this step.
      live.erase(std::remove_if(live.begin(), live.end(), [&](const Block& b) { return b.until < (int)s; }),
                 live.end());
      for (int v0 : io_[s].writes) {
        int v = resolve_alias(v0);
        if ((*loc_)[v].kind != Loc::kNone || first[v] != (int)s) continue;
        int64_t size = align(std::max<int64_t>(bytes_of(v), 1));
        // First fit between live blocks.
        std::sort(live.begin(), live.end(), [](const Block& a, const Block& b) { return a.off < b.off; });
        int64_t cand = 0;
        for (const Block& b : live) {
          if (cand + size <= b.off) break;
          cand = std::max(cand, b.off + b.size);
        }
        live.push_back(Block{cand, size, last[v]});
        top = std::max(top, cand + size);
        (*loc_)[v] = Loc{Loc::kArena, 0, cand};
      }
    }
    // Aliases share their source's location.
    for (auto& kv : alias_of_) (*loc_)[kv.first] = (*loc_)[resolve_alias(kv.second)];
    for (auto& pr : aliases_) (*loc_)[pr.first] = (*loc_)[resolve_alias(pr.second)];
    for (int v = 0; v < total; ++v) {
      if ((*loc_)[v].kind != Loc::kNone) continue;
      // Values never read or written by a step (unused) stay unplaced.
    }
    plan_.arena_bytes_ = (size_t)top;
    for (size_t s = 0; s < io_.size() && s < plan_.steps_.size(); ++s) {
      plan_.steps_[s].reads.clear();
      plan_.steps_[s].writes.clear();
      for (int v : io_[s].reads) plan_.steps_[s].reads.push_back(resolve_alias(v));
      for (int v : io_[s].writes) plan_.steps_[s].writes.push_back(resolve_alias(v));
    }
    // Every value a step touches must be placed.
    for (auto& io : io_)
      for (auto* vec : {&io.reads, &io.writes})
        for (int v : *vec)
          if ((*loc_)[resolve_alias(v)].kind == Loc::kNone)
            throw ParseError("internal: value " + std::to_string(v) + " has no location");
  }

  int resolve_alias(int v) const {
    for (int guard = 0; guard < 64; ++guard) {
      auto it = alias_of_.find(v);
      if (it != alias_of_.end()) {
        v = it->second;
        continue;
      }
      bool found = false;
      for (auto& pr : aliases_)
        if (pr.first == v) {
          v = pr.second;
          found = true;
          break;
        }
      if (!found) return v;
    }
    return v;
  }
};

// IEEE binary16 bits of x, rounded to nearest even.
uint16_t f32_to_f16_bits(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const int32_t exp = (int32_t)((u >> 23) & 0xff) - 127 + 15;
  uint32_t man = u & 0x7fffffu;
  if (((u >> 23) & 0xff) == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
  if (exp >= 31) return (uint16_t)(sign | 0x7c00u);
  if (exp <= 0) {
    if (exp < -10) return (uint16_t)sign;
    man |= 0x800000u;
    const int shift = 14 - exp;
    uint32_t half = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1), mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1))) ++half;
    return (uint16_t)(sign | half);
  }
  uint32_t h = ((uint32_t)exp << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;
  return (uint16_t)(sign | h);
}

}  // namespace

std::unique_ptr<Plan> Plan::build(const Function& f) {
  std::unique_ptr<Plan> p(new Plan());
  Planner pl(f, *p);
  pl.build();
  return p;
}

Plan::~Plan() {
  for (void* d : const_dev_)
    if (d) (void)hipFree(d);
  if (arena_) (void)hipFree(arena_);
}

double Plan::total_flops() const {
  double t = 0;
  for (const Step& s : steps_) t += s.flops;
  return t;
}

void* Plan::ptr(const Loc& l, const ExecBuffers& b) const {
  switch (l.kind) {
    case Loc::kParam: return (char*)b.params.at(l.index) + l.offset;
    case Loc::kConst: return (char*)const_dev_.at(l.index) + l.offset;
    case Loc::kArena: return (char*)b.arena + l.offset;
    case Loc::kOutput: return (char*)b.outputs.at(l.index) + l.offset;
    default: return nullptr;
  }
}

int Plan::prepare(std::string& err) {
  std::lock_guard<std::mutex> lock(mu_);
  if (prepared_) return MFX_OK;
  for (auto& lit : const_host_) {
    const Type& t = lit->type;
    const int64_t n = t.numel();
    std::vector<uint8_t> host((size_t)std::max<int64_t>(t.bytes(), 1));
    for (int64_t i = 0; i < n; ++i) {
      double v = lit->at(i);
      uint8_t* p = host.data() + i * dtype_bytes(t.dtype);
      switch (t.dtype) {
        case DType::kF32: { float x = (float)v; std::memcpy(p, &x, 4); break; }
        case DType::kF64: std::memcpy(p, &v, 8); break;
        case DType::kBF16: {
          float x = (float)v;
          uint32_t u;
          std::memcpy(&u, &x, 4);
          uint32_t r = ((u >> 16) & 1) + 0x7fff;
          uint16_t h = (uint16_t)((u + r) >> 16);
          if (std::isnan(x)) h = 0x7fc0;
          std::memcpy(p, &h, 2);
          break;
        }
        case DType::kF16: {
          uint16_t h = f32_to_f16_bits((float)v);
          std::memcpy(p, &h, 2);
          break;
        }
        case DType::kI32: case DType::kU32: { int32_t x = (int32_t)(int64_t)v; std::memcpy(p, &x, 4); break; }
        case DType::kI64: case DType::kU64: { int64_t x = (int64_t)v; std::memcpy(p, &x, 8); break; }
        case DType::kI16: case DType::kU16: { int16_t x = (int16_t)(int64_t)v; std::memcpy(p, &x, 2); break; }
        default: { uint8_t x = (uint8_t)(int64_t)v; *p = x; break; }
      }
    }
    void* d = nullptr;
    hipError_t e = hipMalloc(&d, host.size());
    if (e == hipSuccess) e = hipMemcpy(d, host.data(), host.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      err = std::string("uploading constants: ") + hipGetErrorString(e);
      return MFX_E_HIP;
    }
    const_dev_.push_back(d);
  }
  if (arena_bytes_) {
    hipError_t e = hipMalloc(&arena_, arena_bytes_);
    if (e != hipSuccess) {
      err = std::string("arena allocation: ") + hipGetErrorString(e);
      return MFX_E_HIP;
    }
  }
  prepared_ = true;
  return MFX_OK;
}

int Plan::run(ExecBuffers& b, std::string& err) {
  int rc = prepare(err);
  if (rc != MFX_OK) return rc;
  std::lock_guard<std::mutex> lock(mu_);
  b.arena = arena_;
  for (size_t i = 0; i < steps_.size(); ++i) {
    rc = steps_[i].run(b, err);
    if (rc != MFX_OK) {
      err = "step " + std::to_string(i) + " (" + steps_[i].kind + ": " + steps_[i].label + "): " + err;
      return rc;
    }
  }
  return MFX_OK;
}

std::string Plan::summary_json() const {
  std::ostringstream o;
  o << "{\"arena_bytes\": " << arena_bytes_ << ", \"steps\": [";
  for (size_t i = 0; i < steps_.size(); ++i)
  {
    o << (i ? ", " : "") << "{\"kind\": \"" << steps_[i].kind << "\", \"label\": \"" << steps_[i].label
      << "\", \"flops\": " << steps_[i].flops;
    for (int w = 0; w < 2; ++w) {
      const std::vector<int>& vs = w ? steps_[i].writes : steps_[i].reads;
      o << (w ? ", \"writes\": [" : ", \"reads\": [");
      for (size_t j = 0; j < vs.size(); ++j) o << (j ? ", " : "") << vs[j];
      o << "]";
    }
    o << "}";
  }
  o << "]}";
  return o.str();
}

}  // namespace mfxp
