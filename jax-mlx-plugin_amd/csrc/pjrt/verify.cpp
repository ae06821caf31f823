// Structural checks of a parsed module, run before the rewriter and planner.
//
// The rewriter and planner index shapes and attribute lists by each other
// (broadcast dims by operand rank, permutations by result dims, slice bounds
// by operand dims, ...).  A module from jaxlib satisfies StableHLO's own
// verifier, but text handed to Client_Compile directly need not, so every
// such relation is checked here once and a violation becomes a ParseError
// (INVALID_ARGUMENT at the C API) instead of an out-of-range access later.
#include <algorithm>
#include <set>
#include <string>

#include "ir.h"

namespace mfxp {
namespace {

constexpr int64_t kMaxDim = int64_t(1) << 40;
constexpr int64_t kMaxElems = int64_t(1) << 48;

[[noreturn]] void bad(const Node& n, const std::string& what) { throw ParseError(n.op + ": " + what); }

const std::vector<int64_t>& ints(const Node& n, const char* key) {
  auto it = n.ints.find(key);
  if (it == n.ints.end()) bad(n, std::string("missing attribute '") + key + "'");
  return it->second;
}

void check_type(const Type& t, const std::string& where) {
  if (t.dtype == DType::kInvalid) throw ParseError(where + ": value without an element type");
  int64_t n = 1;
  for (int64_t d : t.dims) {
    if (d < 0 || d > kMaxDim) throw ParseError(where + ": dimension " + std::to_string(d) + " out of range");
    if (d != 0 && n > kMaxElems / d) throw ParseError(where + ": more than 2^48 elements");
    n *= d;
  }
}

// Each entry of `dims` lies in [0, rank) and appears once.
void check_axes(const Node& n, const std::vector<int64_t>& dims, int rank, const char* what) {
  std::set<int64_t> seen;
  for (int64_t d : dims) {
    if (d < 0 || d >= rank) bad(n, std::string(what) + " " + std::to_string(d) + " outside rank " + std::to_string(rank));
    if (!seen.insert(d).second) bad(n, std::string(what) + " " + std::to_string(d) + " repeated");
  }
}

std::vector<int64_t> opt_ints(const Node& n, const char* key) {
  auto it = n.ints.find(key);
  return it == n.ints.end() ? std::vector<int64_t>{} : it->second;
}

// Operand count of an elementwise op (0: any), or -1 for other ops.
int elementwise_arity(const std::string& op) {
  static const std::set<std::string> unary = {
      "stablehlo.convert", "stablehlo.negate", "stablehlo.abs", "stablehlo.exponential",
      "stablehlo.exponential_minus_one", "stablehlo.log", "stablehlo.log_plus_one", "stablehlo.logistic",
      "stablehlo.tanh", "stablehlo.sqrt", "stablehlo.rsqrt", "stablehlo.sine", "stablehlo.cosine",
      "stablehlo.floor", "stablehlo.ceil", "stablehlo.sign", "stablehlo.not", "stablehlo.is_finite",
      "stablehlo.round_nearest_even", "stablehlo.atan"};
  static const std::set<std::string> binary = {
      "stablehlo.add", "stablehlo.subtract", "stablehlo.multiply", "stablehlo.divide", "stablehlo.maximum",
      "stablehlo.minimum", "stablehlo.power", "stablehlo.remainder", "stablehlo.atan2", "stablehlo.and",
      "stablehlo.or", "stablehlo.xor", "stablehlo.compare"};
  if (unary.count(op)) return 1;
  if (binary.count(op)) return 2;
  if (op == "stablehlo.select" || op == "stablehlo.clamp") return 3;
  if (op == "stablehlo.optimization_barrier") return 0;
  return -1;
}

void verify_node(const Function& f, const Node& n) {
  for (int v : n.in)
    if (v < 0 || v >= (int)f.values.size()) bad(n, "operand out of range");
  for (int v : n.out)
    if (v < 0 || v >= (int)f.values.size()) bad(n, "result out of range");
  for (int v : n.out) check_type(f.type(v), n.op + " result %" + f.values[v].name);
  auto in_t = [&](size_t i) -> const Type& {
    if (i >= n.in.size()) bad(n, "too few operands");
    return f.type(n.in[i]);
  };
  auto out_t = [&](size_t i) -> const Type& {
    if (i >= n.out.size()) bad(n, "too few results");
    return f.type(n.out[i]);
  };
  const std::string& op = n.op;

  if (const int arity = elementwise_arity(op); arity >= 0) {
    if (n.in.empty() || n.out.empty()) bad(n, "needs operands and a result");
    if (arity > 0 && ((int)n.in.size() != arity || n.out.size() != 1))
      bad(n, "takes " + std::to_string(arity) + " operand(s) and one result");
    const Type& o = out_t(0);
    for (size_t i = 0; i < n.in.size(); ++i) {
      const Type& t = in_t(i);
      // select's predicate and clamp's bounds may be scalars.
      const bool scalar_ok = (op == "stablehlo.select" && i == 0) || (op == "stablehlo.clamp" && i != 1);
      if (t.dims != o.dims && !(scalar_ok && t.rank() == 0))
        bad(n, "operand " + std::to_string(i) + " " + t.str() + " does not match result " + o.str());
    }
    if (op == "stablehlo.optimization_barrier" && n.in.size() != n.out.size()) bad(n, "operand / result count");
    return;
  }
  if (op == "stablehlo.broadcast_in_dim") {
    const Type &x = in_t(0), &o = out_t(0);
    const auto& d = ints(n, "dims");
    if ((int)d.size() != x.rank()) bad(n, "broadcast dims size differs from operand rank");
    check_axes(n, d, o.rank(), "broadcast dimension");
    for (int i = 0; i < x.rank(); ++i)
      if (x.dims[i] != 1 && x.dims[i] != o.dims[d[i]]) bad(n, "operand dim " + std::to_string(i) + " mismatch");
    return;
  }
  if (op == "stablehlo.transpose") {
    const Type &x = in_t(0), &o = out_t(0);
    const auto& p = ints(n, "dims");
    if ((int)p.size() != x.rank() || o.rank() != x.rank()) bad(n, "permutation size differs from rank");
    check_axes(n, p, x.rank(), "permutation entry");
    for (int i = 0; i < x.rank(); ++i)
      if (o.dims[i] != x.dims[p[i]]) bad(n, "result dims do not follow the permutation");
    return;
  }
  if (op == "stablehlo.reshape") {
    if (in_t(0).numel() != out_t(0).numel()) bad(n, "element count changes");
    return;
  }
  if (op == "stablehlo.slice") {
    const Type &x = in_t(0), &o = out_t(0);
    const auto &st = ints(n, "start"), &li = ints(n, "limit"), &sd = ints(n, "stride");
    if ((int)st.size() != x.rank() || (int)li.size() != x.rank() || (int)sd.size() != x.rank() ||
        o.rank() != x.rank())
      bad(n, "slice bounds size differs from rank");
    for (int i = 0; i < x.rank(); ++i) {
      if (st[i] < 0 || st[i] > li[i] || li[i] > x.dims[i] || sd[i] < 1) bad(n, "slice bounds out of range");
      if (o.dims[i] != (li[i] - st[i] + sd[i] - 1) / sd[i]) bad(n, "result dims do not follow the bounds");
    }
    return;
  }
  if (op == "stablehlo.iota") {
    const auto& d = ints(n, "dim");
    if (d.size() != 1) bad(n, "iota dimension");
    check_axes(n, d, out_t(0).rank(), "iota dimension");
    return;
  }
  if (op == "stablehlo.concatenate") {
    const Type& o = out_t(0);
    const auto& d = ints(n, "dimension");
    if (d.size() != 1) bad(n, "concatenate dimension");
    check_axes(n, d, o.rank(), "concatenate dimension");
    int64_t sum = 0;
    for (size_t i = 0; i < n.in.size(); ++i) {
      const Type& t = in_t(i);
      if (t.rank() != o.rank()) bad(n, "operand rank");
      for (int a = 0; a < o.rank(); ++a)
        if (a != d[0] && t.dims[a] != o.dims[a]) bad(n, "operand dims");
      sum += t.dims[d[0]];
    }
    if (n.in.empty() || sum != o.dims[d[0]]) bad(n, "concatenated size");
    return;
  }
  if (op == "stablehlo.dot_general" || op == "stablehlo.dot") {
    const Type &a = in_t(0), &b = in_t(1), &o = out_t(0);
    std::vector<int64_t> lb, rb, lc, rc;
    if (op == "stablehlo.dot") {
      if (a.rank() < 1 || a.rank() > 2 || b.rank() < 1 || b.rank() > 2) bad(n, "dot operands must be rank 1 or 2");
      lc = {a.rank() - 1};
      rc = {0};
    } else {
      lb = opt_ints(n, "lhs_batching_dims");
      rb = opt_ints(n, "rhs_batching_dims");
      lc = opt_ints(n, "lhs_contracting_dims");
      rc = opt_ints(n, "rhs_contracting_dims");
    }
    if (lb.size() != rb.size() || lc.size() != rc.size()) bad(n, "dimension numbers differ in length");
    std::vector<int64_t> la = lb, ra = rb;
    la.insert(la.end(), lc.begin(), lc.end());
    ra.insert(ra.end(), rc.begin(), rc.end());
    check_axes(n, la, a.rank(), "lhs dimension");
    check_axes(n, ra, b.rank(), "rhs dimension");
    for (size_t i = 0; i < lb.size(); ++i)
      if (a.dims[lb[i]] != b.dims[rb[i]]) bad(n, "batch sizes differ");
    for (size_t i = 0; i < lc.size(); ++i)
      if (a.dims[lc[i]] != b.dims[rc[i]]) bad(n, "contracting sizes differ");
    const int free_rank = (a.rank() - (int)la.size()) + (b.rank() - (int)ra.size());
    if (o.rank() != (int)lb.size() + free_rank) bad(n, "result rank");
    return;
  }
  if (op == "stablehlo.reduce") {
    if (n.in.empty() || n.in.size() % 2 || n.out.size() != n.in.size() / 2) bad(n, "operand / init / result counts");
    const Type& x = in_t(0);
    const auto& d = ints(n, "dimensions");
    check_axes(n, d, x.rank(), "reduce dimension");
    if (out_t(0).rank() != x.rank() - (int)d.size()) bad(n, "result rank");
    return;
  }
  if (op == "stablehlo.constant") {
    if (!n.literal || n.out.size() != 1) bad(n, "constant without a literal");
    if (!n.literal->splat && (int64_t)n.literal->values.size() != out_t(0).numel()) bad(n, "literal size");
    return;
  }
}

// A call's operands and results against the callee's parameters and
// returned values (inlining splices the callee's values in place of the
// call's results, so their types must agree).
void verify_calls(const Module& m, const Function& f) {
  for (const Node& n : f.nodes) {
    if (n.op != "func.call") continue;
    auto it = n.strs.find("callee");
    auto callee = it == n.strs.end() ? nullptr : m.find(it->second);
    if (!callee) throw ParseError("func.call: unknown callee");
    if (callee->params.size() != n.in.size() || callee->results.size() != n.out.size())
      throw ParseError("func.call @" + callee->name + ": operand / result count differs from the callee");
    for (size_t i = 0; i < n.in.size(); ++i)
      if (callee->type(callee->params[i]) != f.type(n.in[i]))
        throw ParseError("func.call @" + callee->name + ": operand " + std::to_string(i) + " type differs");
    for (size_t i = 0; i < n.out.size(); ++i)
      if (callee->type(callee->results[i]) != f.type(n.out[i]))
        throw ParseError("func.call @" + callee->name + ": result " + std::to_string(i) + " type differs");
  }
}

void verify_function(const Function& f) {
  for (size_t v = 0; v < f.values.size(); ++v) check_type(f.values[v].type, f.name + " value %" + f.values[v].name);
  for (int r : f.results)
    if (r < 0 || r >= (int)f.values.size()) throw ParseError(f.name + ": returned value out of range");
  for (const Node& n : f.nodes) {
    verify_node(f, n);
    for (const auto& r : n.regions)
      if (r) verify_function(*r);
  }
}

}  // namespace

void verify_module(const Module& m) {
  for (const auto& f : m.funcs)
    if (f) verify_function(*f);
  for (const auto& f : m.funcs)
    if (f) verify_calls(m, *f);
}

}  // namespace mfxp
