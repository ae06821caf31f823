// SSA graph IR of a StableHLO module, as parsed from MLIR text.
//
// The reference keeps ops as a flat vector of MLXOp records with string-keyed
// attribute maps and recomputes producer/consumer maps inside its matcher
// (reference src/jax_mlx_pjrt.cpp:414-432, 1816-1855).  Here values are typed
// first-class objects with their producer recorded, so the rewriter can ask
// "who defines %x / how many uses does it have" directly, and shapes/dtypes
// travel with every value into the launch planner.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace mfxp {

enum class DType : int8_t {
  kInvalid,
  kPred,
  kI8,
  kI16,
  kI32,
  kI64,
  kU8,
  kU16,
  kU32,
  kU64,
  kF16,
  kBF16,
  kF32,
  kF64,
};

const char* dtype_name(DType t);
DType dtype_from_name(const std::string& s);
int dtype_bytes(DType t);
bool is_float(DType t);

struct Type {
  DType dtype = DType::kInvalid;
  std::vector<int64_t> dims;

  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : dims) n *= d;
    return n;
  }
  int rank() const { return (int)dims.size(); }
  int64_t bytes() const { return numel() * dtype_bytes(dtype); }
  bool operator==(const Type& o) const { return dtype == o.dtype && dims == o.dims; }
  bool operator!=(const Type& o) const { return !(*this == o); }
  std::string str() const;
};

// A dense constant.  Values are kept as doubles (exact for every float type
// and for integers below 2^53); splat constants hold one value.
struct Literal {
  Type type;
  bool splat = true;
  std::vector<double> values;

  double at(int64_t i) const { return splat ? values.at(0) : values.at(i); }
};

struct Function;

struct Node {
  std::string op;          // "stablehlo.add", ..., or a fused op "mfx.sdpa"
  std::vector<int> in;     // operand value ids
  std::vector<int> out;    // result value ids
  std::map<std::string, std::vector<int64_t>> ints;  // dims, batching/contracting dims, ...
  std::map<std::string, std::string> strs;          // comparison_direction, callee, target, ...
  std::map<std::string, double> nums;               // eps, scale, ...
  std::shared_ptr<Literal> literal;                 // stablehlo.constant
  std::vector<std::shared_ptr<Function>> regions;   // reducer bodies
  bool dead = false;
};

struct Value {
  std::string name;  // SSA name without '%', for messages
  Type type;
  int def = -1;      // producing node index, -1 for a function parameter
  int def_result = 0;
};

struct Function {
  std::string name;
  std::vector<int> params;   // value ids
  std::vector<int> results;  // value ids returned
  std::vector<Node> nodes;
  std::vector<Value> values;

  int add_value(const std::string& name, const Type& t) {
    values.push_back(Value{name, t, -1, 0});
    return (int)values.size() - 1;
  }
  const Type& type(int v) const { return values.at(v).type; }
  // Producer node of value v, or nullptr for parameters.
  Node* producer(int v) {
    int d = values.at(v).def;
    return d < 0 ? nullptr : &nodes[d];
  }
};

struct Module {
  std::string name;
  std::vector<std::shared_ptr<Function>> funcs;
  std::shared_ptr<Function> find(const std::string& n) const {
    for (auto& f : funcs)
      if (f->name == n) return f;
    return nullptr;
  }
  std::shared_ptr<Function> main() const {
    auto m = find("main");
    if (!m && !funcs.empty()) m = funcs.front();
    return m;
  }
};

struct ParseError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// Parses the pretty-printed StableHLO text JAX emits (and the generic
// "op"(...) form for the ops the planner knows).  Throws ParseError.
Module parse_module(const std::string& text);

// Structural checks (operand/result shapes against each op's attributes);
// throws ParseError on the first violation.
void verify_module(const Module& m);

// Replaces every func.call by the callee's body (recursively), so fused
// patterns are matched across jax.nn helper boundaries such as @softmax.
void inline_calls(Module& m);

// Fuses attention / normalisation / softmax subgraphs and the reference's
// custom_call targets into mfx.* nodes; returns the number of rewrites.
struct RewriteStats {
  int sdpa = 0, layer_norm = 0, rms_norm = 0, softmax = 0, log_softmax = 0, sigmoid = 0, custom_calls = 0,
      affine_absorbed = 0;
  int total() const { return sdpa + layer_norm + rms_norm + softmax + log_softmax + sigmoid + custom_calls; }
};
RewriteStats rewrite(Function& f);

// Drops dead nodes and recomputes value producers.
void compact(Function& f);

// A strided view of a materialised base value: element (i0, i1, ...) of the
// viewed value lives at base + offset + sum(i_d * strides[d]) (elements).
struct StridedView {
  int base = -1;
  int64_t offset = 0;
  std::vector<int64_t> dims, strides;
};
std::vector<int64_t> contiguous_strides(const std::vector<int64_t>& dims);
// Strides of out_dims viewing the same elements as (in_dims, in_strides), or
// false when the reshape is not expressible as a strided view.
bool reshape_strides(const std::vector<int64_t>& in_dims, const std::vector<int64_t>& in_strides,
                     const std::vector<int64_t>& out_dims, std::vector<int64_t>& out_strides);
// Follows v back through transpose / reshape / slice (and broadcast_in_dim
// when allowed) to the value whose buffer it reads.
StridedView trace_view(const Function& f, int v, bool allow_broadcast);

// Human/JSON readable dump of a function (ops, fused attributes, shapes).
std::string to_json(const Function& f, const RewriteStats* stats);

}  // namespace mfxp
