// StableHLO (MLIR text) -> IR.
//
// A cursor-based recursive-descent parser for the pretty-printed form that
// jax.jit(...).lower(...).as_text() produces: module / func.func /
// stablehlo.* ops with their custom assembly (dims = [...],
// batching_dims = [...] x [...], reduce(... init: ...) applies ...,
// compare GT, ..., custom_call @target(...) {backend_config = "..."}), dense
// literals (decimal, hex bit patterns, hex blobs, nested arrays), reducer
// regions and func.call.  It plays the role of the reference's regex/line
// parser (reference src/mlx_mlir_parser.h:46-616, 1075-2299) but extracts
// every attribute the rewriter checks (dot dimension numbers, reduce kind and
// axes, broadcast dims, literal values, custom_call config) with types on
// every value.  Unknown ops are an error, not a silent pass-through.
#include <cctype>
#include <cmath>
#include <cstring>
#include <sstream>

#include "ir.h"

namespace mfxp {

const char* dtype_name(DType t) {
  switch (t) {
    case DType::kPred: return "i1";
    case DType::kI8: return "i8";
    case DType::kI16: return "i16";
    case DType::kI32: return "i32";
    case DType::kI64: return "i64";
    case DType::kU8: return "ui8";
    case DType::kU16: return "ui16";
    case DType::kU32: return "ui32";
    case DType::kU64: return "ui64";
    case DType::kF16: return "f16";
    case DType::kBF16: return "bf16";
    case DType::kF32: return "f32";
    case DType::kF64: return "f64";
    default: return "invalid";
  }
}

DType dtype_from_name(const std::string& s) {
  static const std::map<std::string, DType> m = {
      {"i1", DType::kPred},  {"i8", DType::kI8},     {"i16", DType::kI16},  {"i32", DType::kI32},
      {"i64", DType::kI64},  {"ui8", DType::kU8},    {"ui16", DType::kU16}, {"ui32", DType::kU32},
      {"ui64", DType::kU64}, {"f16", DType::kF16},   {"bf16", DType::kBF16}, {"f32", DType::kF32},
      {"f64", DType::kF64},  {"si32", DType::kI32},  {"si64", DType::kI64}, {"si8", DType::kI8},
  };
  auto it = m.find(s);
  return it == m.end() ? DType::kInvalid : it->second;
}

int dtype_bytes(DType t) {
  switch (t) {
    case DType::kPred:
    case DType::kI8:
    case DType::kU8: return 1;
    case DType::kI16:
    case DType::kU16:
    case DType::kF16:
    case DType::kBF16: return 2;
    case DType::kI32:
    case DType::kU32:
    case DType::kF32: return 4;
    case DType::kI64:
    case DType::kU64:
    case DType::kF64: return 8;
    default: return 0;
  }
}

bool is_float(DType t) {
  return t == DType::kF16 || t == DType::kBF16 || t == DType::kF32 || t == DType::kF64;
}

std::string Type::str() const {
  std::string s = "tensor<";
  for (int64_t d : dims) s += std::to_string(d) + "x";
  return s + dtype_name(dtype) + ">";
}

namespace {

// Decodes the IEEE bit pattern `bits` of a float element type.
double float_from_bits(DType t, uint64_t bits) {
  if (t == DType::kF32) {
    uint32_t b = (uint32_t)bits;
    float f;
    std::memcpy(&f, &b, 4);
    return f;
  }
  if (t == DType::kF64) {
    double d;
    std::memcpy(&d, &bits, 8);
    return d;
  }
  if (t == DType::kBF16) {
    uint32_t b = (uint32_t)(bits & 0xffff) << 16;
    float f;
    std::memcpy(&f, &b, 4);
    return f;
  }
  if (t == DType::kF16) {
    uint32_t h = (uint32_t)(bits & 0xffff);
    uint32_t sign = (h >> 15) & 1, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    double v;
    if (exp == 0) v = std::ldexp((double)man, -24);
    else if (exp == 31) v = man ? NAN : INFINITY;
    else v = std::ldexp((double)(man | 0x400), (int)exp - 25);
    return sign ? -v : v;
  }
  return (double)bits;
}

class Parser {
 public:
  explicit Parser(const std::string& s) : s_(s) {}

  Module parse() {
    Module m;
    ws();
    // Location aliases (#loc = loc(...)) may precede the module.
    while (peek() == '#') {
      while (!at_end() && s_[p_] != '\n') ++p_;
      ws();
    }
    if (kw("module")) {
      ws();
      if (peek() == '@') m.name = symbol();
      ws();
      if (kw("attributes")) {
        ws();
        skip_balanced();
      }
      ws();
      expect('{');
      while (true) {
        ws();
        if (peek() == '}') {
          ++p_;
          break;
        }
        if (at_end()) fail("unterminated module");
        parse_top(m);
      }
    } else {
      while (true) {
        ws();
        if (at_end()) break;
        parse_top(m);
      }
    }
    if (m.funcs.empty()) fail("no func.func in module");
    return m;
  }

 private:
  const std::string& s_;
  size_t p_ = 0;

  // ---- lexing helpers ----
  bool at_end() const { return p_ >= s_.size(); }
  char peek(size_t o = 0) const { return p_ + o < s_.size() ? s_[p_ + o] : '\0'; }

  [[noreturn]] void fail(const std::string& msg) const {
    size_t line = 1, col = 1;
    for (size_t i = 0; i < p_ && i < s_.size(); ++i) {
      if (s_[i] == '\n') {
        ++line;
        col = 1;
      } else {
        ++col;
      }
    }
    size_t ls = s_.rfind('\n', p_ ? p_ - 1 : 0);
    ls = (ls == std::string::npos) ? 0 : ls + 1;
    size_t le = s_.find('\n', p_);
    std::string ctx = s_.substr(ls, (le == std::string::npos ? s_.size() : le) - ls);
    if (ctx.size() > 160) ctx = ctx.substr(0, 160) + "...";
    throw ParseError("StableHLO parse error at line " + std::to_string(line) + ":" +
                     std::to_string(col) + ": " + msg + "\n  | " + ctx);
  }

  void ws() {
    while (!at_end()) {
      char c = s_[p_];
      if (std::isspace((unsigned char)c)) {
        ++p_;
      } else if (c == '/' && peek(1) == '/') {
        while (!at_end() && s_[p_] != '\n') ++p_;
      } else {
        break;
      }
    }
  }

  bool lit(const char* t) {
    ws();
    size_t n = std::strlen(t);
    if (s_.compare(p_, n, t) == 0) {
      p_ += n;
      return true;
    }
    return false;
  }

  // Keyword: literal followed by a non-identifier character.
  bool kw(const char* t) {
    ws();
    size_t n = std::strlen(t);
    if (s_.compare(p_, n, t) != 0) return false;
    char c = p_ + n < s_.size() ? s_[p_ + n] : '\0';
    if (std::isalnum((unsigned char)c) || c == '_' || c == '.') return false;
    p_ += n;
    return true;
  }

  void expect(char c) {
    ws();
    if (peek() != c) fail(std::string("expected '") + c + "'");
    ++p_;
  }

  bool accept(char c) {
    ws();
    if (peek() == c) {
      ++p_;
      return true;
    }
    return false;
  }

  static bool ident_char(char c) {
    return std::isalnum((unsigned char)c) || c == '_' || c == '.' || c == '$' || c == '-';
  }

  std::string ident() {
    ws();
    size_t b = p_;
    if (!(std::isalpha((unsigned char)peek()) || peek() == '_')) fail("expected identifier");
    while (!at_end() && (std::isalnum((unsigned char)s_[p_]) || s_[p_] == '_' || s_[p_] == '.' ||
                         s_[p_] == '$'))
      ++p_;
    return s_.substr(b, p_ - b);
  }

  std::string ssa() {
    ws();
    if (peek() != '%') fail("expected SSA value");
    ++p_;
    size_t b = p_;
    while (!at_end() && (ident_char(s_[p_]) || s_[p_] == '#')) ++p_;
    if (p_ == b) fail("empty SSA name");
    return s_.substr(b, p_ - b);
  }

  std::string symbol() {
    ws();
    if (peek() != '@') fail("expected @symbol");
    ++p_;
    if (peek() == '"') return str_lit();
    size_t b = p_;
    while (!at_end() && ident_char(s_[p_])) ++p_;
    return s_.substr(b, p_ - b);
  }

  std::string str_lit() {
    ws();
    if (peek() != '"') fail("expected string");
    ++p_;
    std::string out;
    while (!at_end() && s_[p_] != '"') {
      char c = s_[p_++];
      if (c == '\\' && !at_end()) {
        char e = s_[p_++];
        switch (e) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          default:
            if (std::isxdigit((unsigned char)e) && std::isxdigit((unsigned char)peek())) {
              char h[3] = {e, s_[p_++], 0};
              out += (char)std::strtol(h, nullptr, 16);
            } else {
              out += e;
            }
        }
      } else {
        out += c;
      }
    }
    if (at_end()) fail("unterminated string");
    ++p_;
    return out;
  }

  int64_t integer() {
    ws();
    size_t b = p_;
    if (peek() == '-' || peek() == '+') ++p_;
    if (!std::isdigit((unsigned char)peek())) fail("expected integer");
    while (std::isdigit((unsigned char)peek())) ++p_;
    return std::stoll(s_.substr(b, p_ - b));
  }

  std::vector<int64_t> int_list() {
    expect('[');
    std::vector<int64_t> v;
    ws();
    if (accept(']')) return v;
    do {
      v.push_back(integer());
    } while (accept(','));
    expect(']');
    return v;
  }

  // Skips one balanced (), [], {} or <> group starting at the cursor.
  void skip_balanced() {
    ws();
    char open = peek();
    char close = open == '(' ? ')' : open == '[' ? ']' : open == '{' ? '}' : open == '<' ? '>' : 0;
    if (!close) fail("expected a bracketed group");
    int depth = 0;
    while (!at_end()) {
      char c = s_[p_];
      if (c == '"') {
        str_lit();
        continue;
      }
      if (c == '(' || c == '[' || c == '{' || c == '<') ++depth;
      if (c == ')' || c == ']' || c == '}' || c == '>') {
        // "->" inside a group is an arrow, not a closing bracket.
        if (c == '>' && p_ > 0 && s_[p_ - 1] == '-') {
          ++p_;
          continue;
        }
        --depth;
      }
      ++p_;
      if (depth == 0) return;
    }
    fail("unbalanced brackets");
  }

  std::string balanced_text() {
    ws();
    size_t b = p_;
    skip_balanced();
    return s_.substr(b, p_ - b);
  }

  void skip_loc() {
    ws();
    if (s_.compare(p_, 4, "loc(") == 0) {
      p_ += 3;
      skip_balanced();
    }
  }

  // ---- types ----
  Type type() {
    ws();
    Type t;
    if (kw("tensor")) {
      expect('<');
      size_t b = p_;
      int depth = 1;
      while (!at_end() && depth) {
        if (s_[p_] == '<') ++depth;
        if (s_[p_] == '>') --depth;
        ++p_;
      }
      std::string body = s_.substr(b, p_ - b - 1);
      size_t comma = body.find(',');
      if (comma != std::string::npos) body = body.substr(0, comma);  // drop encodings
      size_t pos = 0;
      while (true) {
        size_t x = body.find('x', pos);
        std::string part = body.substr(pos, x == std::string::npos ? std::string::npos : x - pos);
        if (x != std::string::npos && !part.empty() && (std::isdigit((unsigned char)part[0]) || part[0] == '?')) {
          if (part[0] == '?') fail("dynamic shapes are not supported");
          t.dims.push_back(std::stoll(part));
          pos = x + 1;
        } else {
          part = body.substr(pos);
          while (!part.empty() && std::isspace((unsigned char)part.back())) part.pop_back();
          while (!part.empty() && std::isspace((unsigned char)part.front())) part.erase(part.begin());
          t.dtype = dtype_from_name(part);
          if (t.dtype == DType::kInvalid) fail("unsupported element type '" + part + "'");
          break;
        }
      }
      return t;
    }
    if (peek() == '!') fail("unsupported type " + balanced_token());
    std::string name = ident();
    t.dtype = dtype_from_name(name);
    if (t.dtype == DType::kInvalid) fail("unsupported type '" + name + "'");
    return t;
  }

  std::string balanced_token() {
    size_t b = p_;
    while (!at_end() && !std::isspace((unsigned char)s_[p_]) && s_[p_] != ',' && s_[p_] != ')') ++p_;
    return s_.substr(b, p_ - b);
  }

  // ": (T, T) -> T" | ": (T) -> (T, T)" | ": T" | ": T, T"  -> (operand types, result types)
  void signature(std::vector<Type>& ins, std::vector<Type>& outs) {
    expect(':');
    ws();
    if (peek() == '(') {
      ++p_;
      ws();
      if (!accept(')')) {
        do {
          ins.push_back(type());
        } while (accept(','));
        expect(')');
      }
      if (!lit("->")) fail("expected '->'");
      ws();
      if (peek() == '(') {
        ++p_;
        ws();
        if (!accept(')')) {
          do {
            outs.push_back(type());
            ws();
            if (peek() == '{') skip_balanced();
          } while (accept(','));
          expect(')');
        }
      } else {
        outs.push_back(type());
      }
    } else {
      ins.push_back(type());
      while (true) {
        ws();
        if (peek() != ',') break;
        size_t save = p_;
        ++p_;
        ws();
        if (s_.compare(p_, 6, "tensor") == 0) {
          ins.push_back(type());
        } else {
          p_ = save;
          break;
        }
      }
    }
    skip_loc();
  }

  // ---- literals ----
  void literal_values(DType et, const std::string& body, Literal& lit) {
    std::string b = body;
    auto trim = [](std::string x) {
      while (!x.empty() && std::isspace((unsigned char)x.back())) x.pop_back();
      size_t i = 0;
      while (i < x.size() && std::isspace((unsigned char)x[i])) ++i;
      return x.substr(i);
    };
    b = trim(b);
    if (!b.empty() && b[0] == '"') {
      // Hex blob of little-endian elements.
      std::string hex = b.substr(1, b.size() - 2);
      if (hex.rfind("0x", 0) != 0 && hex.rfind("0X", 0) != 0) throw ParseError("bad dense string literal");
      hex = hex.substr(2);
      int eb = dtype_bytes(et);
      if (eb == 0) throw ParseError("unsupported literal element type");
      size_t nbytes = hex.size() / 2;
      std::vector<uint8_t> raw(nbytes);
      for (size_t i = 0; i < nbytes; ++i) raw[i] = (uint8_t)std::stoul(hex.substr(2 * i, 2), nullptr, 16);
      size_t n = nbytes / eb;
      lit.values.clear();
      for (size_t i = 0; i < n; ++i) {
        uint64_t bits = 0;
        std::memcpy(&bits, &raw[i * eb], eb);
        lit.values.push_back(scalar_from_bits(et, bits, eb));
      }
      lit.splat = (n == 1);
      return;
    }
    // Decimal / hex scalars, possibly nested in [ ].
    lit.values.clear();
    std::string tok;
    auto flush = [&]() {
      std::string t = trim(tok);
      tok.clear();
      if (t.empty()) return;
      lit.values.push_back(parse_scalar(et, t));
    };
    bool nested = false;
    for (char c : b) {
      if (c == '[' || c == ']' || c == ',') {
        if (c == '[') nested = true;
        flush();
      } else {
        tok += c;
      }
    }
    flush();
    lit.splat = !nested && lit.values.size() == 1;
    if (lit.values.empty()) throw ParseError("empty dense literal");
  }

  static double scalar_from_bits(DType et, uint64_t bits, int eb) {
    if (is_float(et)) return float_from_bits(et, bits);
    if (et == DType::kPred) return bits ? 1.0 : 0.0;
    bool is_signed = et == DType::kI8 || et == DType::kI16 || et == DType::kI32 || et == DType::kI64;
    if (is_signed && eb < 8 && (bits >> (8 * eb - 1)) & 1) return (double)((int64_t)bits - ((int64_t)1 << (8 * eb)));
    return is_signed ? (double)(int64_t)bits : (double)bits;
  }

  static double parse_scalar(DType et, const std::string& t) {
    if (t == "true") return 1.0;
    if (t == "false") return 0.0;
    if (t.size() > 2 && (t.rfind("0x", 0) == 0 || t.rfind("0X", 0) == 0)) {
      uint64_t bits = std::stoull(t.substr(2), nullptr, 16);
      return scalar_from_bits(et, bits, dtype_bytes(et));
    }
    if (t == "inf" || t == "+inf") return INFINITY;
    if (t == "-inf") return -INFINITY;
    if (t == "nan" || t == "-nan") return NAN;
    return std::strtod(t.c_str(), nullptr);
  }

  // ---- functions and ops ----
  struct Scope {
    Function* f;
    std::map<std::string, int> names;
  };

  int lookup(Scope& sc, const std::string& name) {
    auto it = sc.names.find(name);
    if (it == sc.names.end()) {
      // "%0#0" of a single-result op is "%0".
      size_t hash = name.find('#');
      if (hash != std::string::npos && name.substr(hash) == "#0") {
        it = sc.names.find(name.substr(0, hash));
        if (it != sc.names.end()) return it->second;
      }
      fail("use of undefined value %" + name);
    }
    return it->second;
  }

  void parse_top(Module& m) {
    ws();
    if (s_.compare(p_, 9, "func.func") == 0) {
      m.funcs.push_back(parse_func());
      return;
    }
    // Anything else at module level (e.g. sdy.mesh declarations): skip the line.
    while (!at_end() && s_[p_] != '\n') {
      if (s_[p_] == '{' || s_[p_] == '(' || s_[p_] == '[') {
        skip_balanced();
        continue;
      }
      ++p_;
    }
  }

  std::shared_ptr<Function> parse_func() {
    if (!kw("func.func")) fail("expected func.func");
    kw("public") || kw("private") || kw("nested");
    auto f = std::make_shared<Function>();
    f->name = symbol();
    Scope sc{f.get(), {}};
    expect('(');
    ws();
    if (!accept(')')) {
      do {
        std::string n = ssa();
        expect(':');
        Type t = type();
        ws();
        if (peek() == '{') skip_balanced();
        skip_loc();
        int v = f->add_value(n, t);
        f->params.push_back(v);
        sc.names[n] = v;
      } while (accept(','));
      expect(')');
    }
    std::vector<Type> result_types;
    if (lit("->")) {
      ws();
      if (peek() == '(') {
        ++p_;
        ws();
        if (!accept(')')) {
          do {
            result_types.push_back(type());
            ws();
            if (peek() == '{') skip_balanced();
          } while (accept(','));
          expect(')');
        }
      } else {
        result_types.push_back(type());
      }
    }
    if (kw("attributes")) skip_balanced();
    expect('{');
    parse_block(sc, f->results);
    expect('}');
    skip_loc();
    if (f->results.size() != result_types.size())
      fail("function @" + f->name + " returns a different number of values than declared");
    return f;
  }

  // Parses ops until the block's terminator (return); fills `results`.
  void parse_block(Scope& sc, std::vector<int>& results) {
    while (true) {
      ws();
      if (peek() == '}') fail("block without a return");
      if (kw("return") || kw("func.return") || kw("stablehlo.return") || kw("mhlo.return")) {
        ws();
        if (peek() == '%') {
          do {
            results.push_back(lookup(sc, ssa()));
          } while (accept(','));
          std::vector<Type> ins, outs;
          signature(ins, outs);
        }
        skip_loc();
        return;
      }
      parse_op(sc);
    }
  }

  void parse_op(Scope& sc) {
    Function& f = *sc.f;
    std::vector<std::string> res_names;
    std::vector<int> res_counts;
    ws();
    if (peek() == '%') {
      do {
        std::string n = ssa();
        int count = 1;
        ws();
        if (peek() == ':' && std::isdigit((unsigned char)peek(1))) {
          ++p_;
          count = (int)integer();
        }
        res_names.push_back(n);
        res_counts.push_back(count);
      } while (accept(','));
      expect('=');
    }
    Node node;
    ws();
    bool generic = false;
    if (peek() == '"') {
      node.op = str_lit();
      generic = true;
    } else {
      node.op = ident();
    }
    if (node.op.rfind("mhlo.", 0) == 0) node.op = "stablehlo." + node.op.substr(5);
    std::vector<Type> ins, outs;
    if (generic) {
      parse_generic(sc, node, ins, outs);
    } else {
      parse_pretty(sc, node, ins, outs);
    }
    // Define results.
    int total = 0;
    for (int c : res_counts) total += c;
    if (outs.empty() && total == 1 && !ins.empty()) outs.push_back(ins.back());
    if ((int)outs.size() != total) {
      if (total == 0 && outs.empty()) {
        // an op without results
      } else {
        fail("op " + node.op + " declares " + std::to_string(outs.size()) + " result types for " +
             std::to_string(total) + " results");
      }
    }
    int k = 0;
    int node_index = (int)f.nodes.size();
    for (size_t i = 0; i < res_names.size(); ++i) {
      for (int j = 0; j < res_counts[i]; ++j, ++k) {
        std::string nm = res_counts[i] == 1 ? res_names[i] : res_names[i] + "#" + std::to_string(j);
        int v = f.add_value(nm, outs[k]);
        f.values[v].def = node_index;
        f.values[v].def_result = k;
        node.out.push_back(v);
        sc.names[nm] = v;
      }
    }
    f.nodes.push_back(std::move(node));
  }

  std::vector<int> operands(Scope& sc) {
    std::vector<int> v;
    ws();
    if (peek() != '%') return v;
    do {
      ws();
      if (peek() != '%') break;
      v.push_back(lookup(sc, ssa()));
    } while (accept(','));
    return v;
  }

  // key = value pairs after the operands of pretty ops (dims = [..], ...).
  void keyword_attrs(Node& node) {
    while (true) {
      ws();
      size_t save = p_;
      if (!(std::isalpha((unsigned char)peek()) || peek() == '_')) break;
      std::string key = ident();
      ws();
      if (peek() != '=') {
        p_ = save;
        break;
      }
      ++p_;
      ws();
      if (peek() == '[') {
        size_t save2 = p_;
        ++p_;
        ws();
        bool ints = std::isdigit((unsigned char)peek()) || peek() == '-' || peek() == ']';
        p_ = save2;
        if (ints) {
          std::vector<int64_t> a = int_list();
          if (kw("x")) {
            node.ints["lhs_" + key] = a;
            node.ints["rhs_" + key] = int_list();
          } else {
            node.ints[key] = a;
          }
        } else {
          node.strs[key] = balanced_text();
        }
      } else if (std::isdigit((unsigned char)peek()) || peek() == '-') {
        node.ints[key] = {integer()};
      } else if (peek() == '<' || peek() == '{' || peek() == '(') {
        node.strs[key] = balanced_text();
      } else if (peek() == '"') {
        node.strs[key] = str_lit();
      } else {
        node.strs[key] = ident();
      }
      ws();
      if (peek() == ',') {
        ++p_;
        continue;
      }
      break;
    }
  }

  // Attribute dictionary {k = v, ...}: strings decoded, the rest kept as text.
  void attr_dict(Node& node) {
    expect('{');
    ws();
    if (accept('}')) return;
    do {
      ws();
      std::string key = peek() == '"' ? str_lit() : ident();
      ws();
      if (!accept('=')) {
        node.strs[key] = "true";
        continue;
      }
      ws();
      std::string val;
      if (peek() == '"') {
        val = str_lit();
      } else if (peek() == '[' || peek() == '{' || peek() == '<' || peek() == '(') {
        val = balanced_text();
      } else {
        size_t b = p_;
        while (!at_end() && s_[p_] != ',' && s_[p_] != '}') {
          if (s_[p_] == '<' || s_[p_] == '(' || s_[p_] == '[') {
            skip_balanced();
            continue;
          }
          ++p_;
        }
        val = s_.substr(b, p_ - b);
        while (!val.empty() && std::isspace((unsigned char)val.back())) val.pop_back();
      }
      node.strs[key] = val;
    } while (accept(','));
    expect('}');
  }

  static std::vector<int64_t> ints_in(const std::string& text) {
    // "array<i64: 1, 2>" | "dense<[1, 2]> : tensor<2xi64>" | "[1, 2]"
    std::string t = text;
    size_t colon = t.find("array<");
    if (colon != std::string::npos) {
      size_t c2 = t.find(':', colon);
      t = c2 == std::string::npos ? "" : t.substr(c2 + 1);
    } else {
      size_t tp = t.find(" : ");
      if (tp != std::string::npos) t = t.substr(0, tp);
    }
    std::vector<int64_t> v;
    std::string num;
    for (char c : t) {
      if (std::isdigit((unsigned char)c) || (c == '-' && num.empty())) {
        num += c;
      } else {
        if (!num.empty() && num != "-") v.push_back(std::stoll(num));
        num.clear();
      }
    }
    if (!num.empty() && num != "-") v.push_back(std::stoll(num));
    return v;
  }

  void parse_reduce_pretty(Scope& sc, Node& node, std::vector<Type>& ins, std::vector<Type>& outs) {
    // (%x init: %i), (%y init: %j) applies stablehlo.add across dimensions = [..] : sig
    // or ... across dimensions = [..] : sig reducer(%a: T, %b: T) { ... }
    std::vector<int> vals, inits;
    do {
      expect('(');
      vals.push_back(lookup(sc, ssa()));
      if (!lit("init:")) fail("expected 'init:' in reduce");
      inits.push_back(lookup(sc, ssa()));
      expect(')');
    } while (accept(','));
    node.in = vals;
    node.in.insert(node.in.end(), inits.begin(), inits.end());
    if (kw("applies")) {
      std::string op = ident();
      if (op.rfind("mhlo.", 0) == 0) op = "stablehlo." + op.substr(5);
      node.strs["reduce"] = op;
    }
    if (!kw("across")) fail("expected 'across' in reduce");
    if (!kw("dimensions")) fail("expected 'dimensions' in reduce");
    expect('=');
    node.ints["dimensions"] = int_list();
    ws();
    if (peek() == '{') attr_dict(node);
    signature(ins, outs);
    ws();
    if (kw("reducer")) {
      auto body = std::make_shared<Function>();
      body->name = "reducer";
      Scope bs{body.get(), {}};
      for (int grp = 0; grp < 2; ++grp) {
        ws();
        if (peek() != '(') break;
        expect('(');
        do {
          std::string n = ssa();
          expect(':');
          Type t = type();
          int v = body->add_value(n, t);
          body->params.push_back(v);
          bs.names[n] = v;
        } while (accept(','));
        expect(')');
      }
      expect('{');
      parse_block(bs, body->results);
      expect('}');
      node.regions.push_back(body);
      classify_reducer(node);
    }
    if (!node.strs.count("reduce")) fail("reduce without a recognisable reducer");
  }

  void parse_region(Scope& sc, Node& node) {
    // ({ ^bb0(%a: T, %b: T): ops... stablehlo.return %x : T })
    expect('(');
    while (true) {
      ws();
      if (peek() != '{') break;
      ++p_;
      auto body = std::make_shared<Function>();
      body->name = "region";
      Scope bs{body.get(), {}};
      ws();
      if (peek() == '^') {
        while (!at_end() && s_[p_] != '(') ++p_;
        expect('(');
        ws();
        if (!accept(')')) {
          do {
            std::string n = ssa();
            expect(':');
            Type t = type();
            int v = body->add_value(n, t);
            body->params.push_back(v);
            bs.names[n] = v;
          } while (accept(','));
          expect(')');
        }
        expect(':');
      }
      parse_block(bs, body->results);
      expect('}');
      node.regions.push_back(body);
      if (!accept(',')) break;
    }
    expect(')');
  }

  static void classify_reducer(Node& node) {
    if (node.regions.empty()) return;
    Function& b = *node.regions[0];
    if (b.nodes.size() == 1 && b.results.size() == 1 && b.params.size() == 2) {
      const Node& n = b.nodes[0];
      if (n.in.size() == 2 && n.out.size() == 1 && n.out[0] == b.results[0]) node.strs["reduce"] = n.op;
    }
  }

  void parse_generic(Scope& sc, Node& node, std::vector<Type>& ins, std::vector<Type>& outs) {
    expect('(');
    ws();
    if (!accept(')')) {
      node.in = operands(sc);
      expect(')');
    }
    ws();
    if (peek() == '<' && peek(1) == '{') {
      ++p_;
      attr_dict(node);
      expect('>');
    }
    ws();
    if (peek() == '(') parse_region(sc, node);
    ws();
    if (peek() == '{') attr_dict(node);
    signature(ins, outs);
    // Normalise the generic attribute spellings to the pretty ones.
    auto take = [&](const char* from, const char* to) {
      auto it = node.strs.find(from);
      if (it != node.strs.end()) node.ints[to] = ints_in(it->second);
    };
    take("broadcast_dimensions", "dims");
    take("permutation", "dims");
    take("dimensions", "dimensions");
    take("iota_dimension", "dim");
    if (node.op == "stablehlo.constant") {
      auto it = node.strs.find("value");
      if (it == node.strs.end()) fail("constant without value");
      set_literal(node, it->second, outs.empty() ? Type{} : outs[0]);
    }
    if (node.op == "stablehlo.compare") {
      auto it = node.strs.find("comparison_direction");
      if (it != node.strs.end()) {
        for (const char* d : {"EQ", "NE", "LT", "LE", "GT", "GE"})
          if (it->second.find(d) != std::string::npos) node.strs["comparison_direction"] = d;
      }
    }
    if (node.op == "stablehlo.dot_general") {
      auto it = node.strs.find("dot_dimension_numbers");
      if (it != node.strs.end()) {
        const std::string& t = it->second;
        auto grab = [&](const char* key) {
          size_t k = t.find(key);
          if (k == std::string::npos) return std::vector<int64_t>{};
          size_t b = t.find('[', k), e = t.find(']', b);
          return ints_in(t.substr(b, e - b + 1));
        };
        node.ints["lhs_batching_dims"] = grab("lhs_batching_dimensions");
        node.ints["rhs_batching_dims"] = grab("rhs_batching_dimensions");
        node.ints["lhs_contracting_dims"] = grab("lhs_contracting_dimensions");
        node.ints["rhs_contracting_dims"] = grab("rhs_contracting_dimensions");
      }
    }
    if (node.op == "stablehlo.reduce") {
      classify_reducer(node);
      if (!node.strs.count("reduce")) fail("reduce without a recognisable reducer");
    }
    if (node.op == "stablehlo.concatenate") take("dimension", "dimension");
  }

  void set_literal(Node& node, const std::string& text, const Type& t) {
    // text: dense<...> [: tensor<..>]
    size_t b = text.find("dense<");
    if (b == std::string::npos) fail("unsupported constant literal (only dense<...>)");
    size_t p = b + 6;
    int depth = 1;
    size_t e = p;
    bool in_str = false;
    for (; e < text.size(); ++e) {
      char c = text[e];
      if (c == '"') in_str = !in_str;
      if (in_str) continue;
      if (c == '<') ++depth;
      if (c == '>' && --depth == 0) break;
    }
    auto lit = std::make_shared<Literal>();
    lit->type = t;
    literal_values(t.dtype, text.substr(p, e - p), *lit);
    if (!lit->splat && (int64_t)lit->values.size() != t.numel())
      fail("dense literal has " + std::to_string(lit->values.size()) + " values for " + t.str());
    node.literal = lit;
  }

  void parse_pretty(Scope& sc, Node& node, std::vector<Type>& ins, std::vector<Type>& outs) {
    const std::string& op = node.op;
    if (op == "stablehlo.constant") {
      ws();
      size_t b = p_;
      if (s_.compare(p_, 6, "dense<") != 0) fail("unsupported constant literal (only dense<...>)");
      p_ += 5;
      skip_balanced();
      std::string text = s_.substr(b, p_ - b);
      signature(ins, outs);
      if (outs.empty()) outs = ins;
      set_literal(node, text, outs[0]);
      ins.clear();
      return;
    }
    if (op == "stablehlo.reduce") {
      parse_reduce_pretty(sc, node, ins, outs);
      return;
    }
    if (op == "stablehlo.compare") {
      node.strs["comparison_direction"] = ident();
      expect(',');
      node.in = operands(sc);
      ws();
      if (std::isalpha((unsigned char)peek())) node.strs["compare_type"] = ident();
      signature(ins, outs);
      if (outs.empty()) {
        Type t = ins.at(0);
        t.dtype = DType::kPred;
        outs.push_back(t);
      }
      return;
    }
    if (op == "stablehlo.iota") {
      if (!kw("dim")) fail("expected 'dim' in iota");
      expect('=');
      node.ints["dim"] = {integer()};
      signature(ins, outs);
      if (outs.empty()) outs = ins;
      ins.clear();
      return;
    }
    if (op == "stablehlo.custom_call") {
      node.strs["target"] = symbol();
      expect('(');
      ws();
      if (!accept(')')) {
        node.in = operands(sc);
        expect(')');
      }
      ws();
      if (peek() == '{') attr_dict(node);
      signature(ins, outs);
      return;
    }
    if (op == "func.call" || op == "call") {
      node.op = "func.call";
      node.strs["callee"] = symbol();
      expect('(');
      ws();
      if (!accept(')')) {
        node.in = operands(sc);
        expect(')');
      }
      ws();
      if (peek() == '{') attr_dict(node);
      signature(ins, outs);
      return;
    }
    if (op == "stablehlo.composite") {
      node.strs["name"] = str_lit();
      node.in = operands(sc);
      ws();
      if (peek() == '{') attr_dict(node);
      signature(ins, outs);
      auto it = node.strs.find("decomposition");
      if (it == node.strs.end()) fail("composite without decomposition");
      std::string callee = it->second;
      if (!callee.empty() && callee[0] == '@') callee = callee.substr(1);
      node.op = "func.call";
      node.strs["callee"] = callee;
      return;
    }
    if (op == "stablehlo.slice") {
      node.in = operands(sc);
      ws();
      // [start:limit(:stride), ...]
      expect('[');
      std::vector<int64_t> st, li, sd;
      ws();
      if (!accept(']')) {
        do {
          st.push_back(integer());
          expect(':');
          li.push_back(integer());
          int64_t stride = 1;
          if (accept(':')) stride = integer();
          sd.push_back(stride);
        } while (accept(','));
        expect(']');
      }
      node.ints["start"] = st;
      node.ints["limit"] = li;
      node.ints["stride"] = sd;
      signature(ins, outs);
      return;
    }
    if (op == "stablehlo.while" || op == "stablehlo.case" || op == "stablehlo.if" ||
        op == "stablehlo.sort" || op == "stablehlo.scatter" || op == "stablehlo.reduce_window" ||
        op == "stablehlo.select_and_scatter" || op == "stablehlo.map")
      fail("op " + op + " is outside this plugin's fused-path scope");
    // Generic pretty form: operands, keyword attrs, optional attr dict, signature.
    node.in = operands(sc);
    ws();
    if (peek() == ',') {
      ++p_;
      keyword_attrs(node);
    } else if (std::isalpha((unsigned char)peek())) {
      keyword_attrs(node);
    }
    ws();
    if (peek() == '{') attr_dict(node);
    signature(ins, outs);
    // concatenate's pretty form spells its axis "dim".
    if (op == "stablehlo.concatenate" && node.ints.count("dim")) node.ints["dimension"] = node.ints["dim"];
  }
};

}  // namespace

Module parse_module(const std::string& text) {
  Parser p(text);
  return p.parse();
}

}  // namespace mfxp
