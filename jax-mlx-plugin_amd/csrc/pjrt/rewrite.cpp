// Graph rewriting: call inlining, dead-code elimination and the fused-pattern
// matcher.
//
// The reference's RecognizePatterns (reference src/jax_mlx_pjrt.cpp:
// 1816-2769) walks fixed producer chains from a divide (softmax, SDPA) or a
// multiply (RMSNorm, LayerNorm), rejects a match when an intermediate has an
// outside consumer, and never checks dot dimension numbers.  This rewriter
// instead recognises the *value* each pattern computes:
//   * mean / variance / mean-square / softmax are identified semantically
//     (two-pass and one-pass variance, divide-by-n or multiply-by-1/n,
//     keepdims reshapes, f32 upcasts of bf16 inputs);
//   * SDPA is matched from the PV dot_general back through the softmax to the
//     QK dot_general with the dot dimension numbers checked, transposes and
//     reshapes of q/k/v/out folded into kernel strides (BTNH and BHTD alike),
//     GQA (q reshaped to [.., Hkv, G, ..]) mapped to the kernel's head groups,
//     causal masks recognised by evaluating the mask expression over (t, s),
//     and additive / boolean data masks passed as an additive mask tensor;
//   * a match only replaces the final value; intermediates that other ops
//     still use simply stay alive (dead-code elimination removes the rest),
//     so no match has to be rejected for outside consumers;
//   * LayerNorm absorbs its gamma/beta epilogue and RMSNorm(q) folds into the
//     attention kernel's prologue.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <set>
#include <sstream>

#include "ir.h"

namespace mfxp {
namespace {

bool op_is(const Node* n, const char* name) { return n && n->op == name; }

// Element types the fused kernels read and write (fp32 arithmetic inside).
bool kernel_float(DType t) { return t == DType::kF32 || t == DType::kBF16 || t == DType::kF16; }

std::vector<int> use_counts(const Function& f) {
  std::vector<int> u(f.values.size(), 0);
  for (const Node& n : f.nodes)
    if (!n.dead)
      for (int v : n.in) u[v]++;
  for (int v : f.results) u[v]++;
  return u;
}

struct Ctx {
  Function& f;
  std::vector<int> uses;
  explicit Ctx(Function& fn) : f(fn), uses(use_counts(fn)) {}
  void refresh() { uses = use_counts(f); }

  Node* def(int v) {
    Node* n = f.producer(v);
    return (n && !n->dead) ? n : nullptr;
  }
  const Type& ty(int v) const { return f.values[v].type; }
  int rank(int v) const { return (int)f.values[v].type.dims.size(); }

  // Through value-preserving reshapes / broadcasts (keepdims shapes).
  int strip_shape(int v) {
    for (;;) {
      Node* n = def(v);
      if (n && (n->op == "stablehlo.broadcast_in_dim" || n->op == "stablehlo.reshape")) {
        v = n->in[0];
        continue;
      }
      return v;
    }
  }
  // Through float -> float converts.
  int strip_convert(int v) {
    for (;;) {
      Node* n = def(v);
      if (n && n->op == "stablehlo.convert" && is_float(ty(n->in[0]).dtype) && is_float(ty(v).dtype)) {
        v = n->in[0];
        continue;
      }
      return v;
    }
  }
  int strip_all(int v) {
    for (;;) {
      int w = strip_convert(strip_shape(v));
      if (w == v) return v;
      v = w;
    }
  }
  bool same(int a, int b) { return strip_convert(a) == strip_convert(b); }

  // A splat constant seen through broadcasts / reshapes / converts.
  bool splat(int v, double& out) {
    v = strip_all(v);
    Node* n = def(v);
    if (!op_is(n, "stablehlo.constant") || !n->literal) return false;
    const Literal& l = *n->literal;
    if (!l.splat) {
      for (double x : l.values)
        if (x != l.values[0]) return false;
    }
    out = l.values.at(0);
    return true;
  }
};

bool near(double a, double b) { return std::fabs(a - b) <= 1e-6 * std::max(1.0, std::fabs(b)); }

// ---- reductions / statistics --------------------------------------------------

// v is reduce_<kind>(x) over exactly `axis` (after stripping shape ops).
bool match_reduce(Ctx& c, int v, const char* kind, int& x, int& axis) {
  v = c.strip_all(v);
  Node* n = c.def(v);
  if (!op_is(n, "stablehlo.reduce") || n->in.size() != 2 || n->out.size() != 1) return false;
  auto it = n->strs.find("reduce");
  if (it == n->strs.end() || it->second != kind) return false;
  auto d = n->ints.find("dimensions");
  if (d == n->ints.end() || d->second.size() != 1) return false;
  double init;
  if (!c.splat(n->in[1], init)) return false;
  const std::string k = kind;
  if (k == "stablehlo.add" && init != 0.0) return false;
  if (k == "stablehlo.maximum" && !(std::isinf(init) && init < 0) && init > -1e30) return false;
  x = n->in[0];
  axis = (int)d->second[0];
  return true;
}

// v == mean(x) over `axis`: sum(x)/n or sum(x)*(1/n).
bool match_mean(Ctx& c, int v, int& x, int& axis) {
  v = c.strip_all(v);
  Node* n = c.def(v);
  if (!n || n->in.size() != 2) return false;
  double k;
  if (n->op == "stablehlo.divide") {
    if (!match_reduce(c, n->in[0], "stablehlo.add", x, axis)) return false;
    if (!c.splat(n->in[1], k)) return false;
    return near(k, (double)c.ty(x).dims[axis]);
  }
  if (n->op == "stablehlo.multiply") {
    for (int o = 0; o < 2; ++o) {
      if (match_reduce(c, n->in[o], "stablehlo.add", x, axis) && c.splat(n->in[1 - o], k))
        return near(k * (double)c.ty(x).dims[axis], 1.0);
    }
  }
  return false;
}

// v == t*t (multiply or power 2).
bool match_square(Ctx& c, int v, int& t) {
  Node* n = c.def(c.strip_convert(v));
  if (!n) return false;
  if (n->op == "stablehlo.multiply" && n->in.size() == 2 && c.same(n->in[0], n->in[1])) {
    t = n->in[0];
    return true;
  }
  double e;
  if (n->op == "stablehlo.power" && c.splat(n->in[1], e) && e == 2.0) {
    t = n->in[0];
    return true;
  }
  return false;
}

// v == mean(x) over axis (x compared modulo converts).
bool is_mean_of(Ctx& c, int v, int x, int axis) {
  int mx, ma;
  return match_mean(c, v, mx, ma) && ma == axis && c.same(mx, x);
}

// v == variance of x over axis, population form, two-pass or one-pass.
bool is_var_of(Ctx& c, int v, int x, int axis) {
  v = c.strip_all(v);
  Node* n = c.def(v);
  if (!n) return false;
  double zero;
  if (n->op == "stablehlo.maximum" && n->in.size() == 2) {
    for (int o = 0; o < 2; ++o)
      if (c.splat(n->in[o], zero) && zero == 0.0) return is_var_of(c, n->in[1 - o], x, axis);
    return false;
  }
  // Two-pass: mean(square(x - mean(x))).
  int sq_in, ma;
  if (match_mean(c, v, sq_in, ma) && ma == axis) {
    int t;
    if (match_square(c, sq_in, t)) {
      Node* s = c.def(c.strip_convert(t));
      if (op_is(s, "stablehlo.subtract") && c.same(s->in[0], x) && is_mean_of(c, s->in[1], x, axis)) return true;
    }
    return false;
  }
  // One-pass: mean(x^2) - mean(x)^2.
  if (n->op == "stablehlo.subtract") {
    int t;
    if (!match_mean(c, n->in[0], sq_in, ma) || ma != axis || !match_square(c, sq_in, t) || !c.same(t, x))
      return false;
    int m;
    return match_square(c, c.strip_shape(n->in[1]), m) && is_mean_of(c, m, x, axis);
  }
  return false;
}

// v == rsqrt(stat + eps) (or 1/sqrt); returns stat and eps.
bool match_rsqrt_eps(Ctx& c, int v, int& stat, double& eps) {
  v = c.strip_all(v);
  Node* n = c.def(v);
  int arg;
  if (op_is(n, "stablehlo.rsqrt")) {
    arg = n->in[0];
  } else if (op_is(n, "stablehlo.divide")) {
    double one;
    Node* s = c.def(c.strip_all(n->in[1]));
    if (!c.splat(n->in[0], one) || one != 1.0 || !op_is(s, "stablehlo.sqrt")) return false;
    arg = s->in[0];
  } else {
    return false;
  }
  Node* a = c.def(c.strip_all(arg));
  if (!op_is(a, "stablehlo.add")) return false;
  for (int o = 0; o < 2; ++o) {
    if (c.splat(a->in[o], eps)) {
      stat = a->in[1 - o];
      return true;
    }
  }
  return false;
}

bool match_sqrt_eps(Ctx& c, int v, int& stat, double& eps) {
  Node* s = c.def(c.strip_all(v));
  if (!op_is(s, "stablehlo.sqrt")) return false;
  Node* a = c.def(c.strip_all(s->in[0]));
  if (!op_is(a, "stablehlo.add")) return false;
  for (int o = 0; o < 2; ++o)
    if (c.splat(a->in[o], eps)) {
      stat = a->in[1 - o];
      return true;
    }
  return false;
}

// v is a [C] vector broadcast along the last axis of a rank-r tensor.
bool match_last_axis_vector(Ctx& c, int v, int C, int& vec) {
  Node* n = c.def(v);
  if (!op_is(n, "stablehlo.broadcast_in_dim")) return false;
  int src = n->in[0];
  const auto& bd = n->ints["dims"];
  int r = c.rank(v);
  const Type& st = c.ty(src);
  // Accept [C] with dims=[r-1] or [1,..,1,C] with trailing dims.
  for (int i = 0; i < st.rank(); ++i) {
    bool last = i == st.rank() - 1;
    if (last) {
      if (st.dims[i] != C || bd.at(i) != r - 1) return false;
    } else if (st.dims[i] != 1) {
      return false;
    }
  }
  // Look through a reshape [C] -> [1,..,C].
  Node* rs = c.def(src);
  if (op_is(rs, "stablehlo.reshape") && c.ty(rs->in[0]).numel() == C) src = rs->in[0];
  vec = src;
  return true;
}

// ---- LayerNorm / RMSNorm ------------------------------------------------------

struct NormMatch {
  int x = -1;
  int gamma = -1;  // folded into the normaliser (Flax: rsqrt(var+eps) * scale)
  double eps = 0;
  bool rms = false;
};

// Normaliser factor r of x: rsqrt(stat+eps) or rsqrt(stat+eps)*gamma.
bool match_factor(Ctx& c, int r, int x, int axis, bool rms, NormMatch& m) {
  int stat;
  double eps;
  int rr = c.strip_all(r);
  Node* n = c.def(rr);
  if (op_is(n, "stablehlo.multiply")) {
    int C = (int)c.ty(x).dims.back();
    for (int o = 0; o < 2; ++o) {
      int vec;
      if (match_last_axis_vector(c, n->in[1 - o], C, vec) &&
          match_factor(c, n->in[o], x, axis, rms, m) && m.gamma < 0) {
        m.gamma = vec;
        return true;
      }
    }
    return false;
  }
  if (!match_rsqrt_eps(c, r, stat, eps)) return false;
  if (rms) {
    int sq, ma, t;
    if (!match_mean(c, stat, sq, ma) || ma != axis || !match_square(c, sq, t) || !c.same(t, x)) return false;
  } else if (!is_var_of(c, stat, x, axis)) {
    return false;
  }
  m.eps = eps;
  return true;
}

// v = normalised x: (x - mean) * r, (x - mean) / sqrt(var+eps), x * r, x / sqrt(ms+eps).
bool match_norm(Ctx& c, int v, NormMatch& m) {
  Node* n = c.def(v);
  if (!n || n->in.size() != 2) return false;
  if (!is_float(c.ty(v).dtype) || c.rank(v) < 1) return false;
  const int axis = c.rank(v) - 1;
  if (n->op == "stablehlo.multiply") {
    for (int o = 0; o < 2; ++o) {
      int a = n->in[o], r = n->in[1 - o];
      Node* s = c.def(c.strip_convert(a));
      if (op_is(s, "stablehlo.subtract") && is_mean_of(c, s->in[1], s->in[0], axis)) {
        NormMatch t;
        t.x = s->in[0];
        if (match_factor(c, r, t.x, axis, false, t)) {
          m = t;
          return true;
        }
      }
      // RMS: x * rsqrt(mean(x^2) + eps)
      NormMatch t;
      t.x = a;
      t.rms = true;
      if (c.rank(a) == c.rank(v) && match_factor(c, r, a, axis, true, t)) {
        m = t;
        return true;
      }
    }
  } else if (n->op == "stablehlo.divide") {
    int stat;
    double eps;
    if (!match_sqrt_eps(c, n->in[1], stat, eps)) return false;
    int a = n->in[0];
    Node* s = c.def(c.strip_convert(a));
    if (op_is(s, "stablehlo.subtract") && is_mean_of(c, s->in[1], s->in[0], axis) &&
        is_var_of(c, stat, s->in[0], axis)) {
      m.x = s->in[0];
      m.eps = eps;
      m.rms = false;
      return true;
    }
    int sq, ma, t;
    if (match_mean(c, stat, sq, ma) && ma == axis && match_square(c, sq, t) && c.same(t, a)) {
      m.x = a;
      m.eps = eps;
      m.rms = true;
      return true;
    }
  }
  return false;
}

int single_user(Ctx& c, int v) {
  if (c.uses[v] != 1) return -1;
  for (size_t i = 0; i < c.f.nodes.size(); ++i) {
    const Node& n = c.f.nodes[i];
    if (n.dead) continue;
    for (int u : n.in)
      if (u == v) return (int)i;
  }
  return -1;  // used by the function result
}

int rewrite_norms(Ctx& c, RewriteStats& st) {
  int count = 0;
  for (size_t i = 0; i < c.f.nodes.size(); ++i) {
    Node& n = c.f.nodes[i];
    if (n.dead || n.out.size() != 1) continue;
    if (n.op != "stablehlo.multiply" && n.op != "stablehlo.divide") continue;
    NormMatch m;
    int v = n.out[0];
    if (!match_norm(c, v, m)) continue;
    const int C = (int)c.ty(v).dims.back();
    int gamma = m.gamma, beta = -1;
    int out_v = v;
    // Absorb y*gamma and (+beta) when y feeds only them.
    int u = single_user(c, out_v);
    if (u >= 0 && gamma < 0 && c.f.nodes[u].op == "stablehlo.multiply") {
      Node& mn = c.f.nodes[u];
      int other = mn.in[0] == out_v ? mn.in[1] : mn.in[0];
      int vec;
      if (match_last_axis_vector(c, other, C, vec)) {
        gamma = vec;
        out_v = mn.out[0];
        u = single_user(c, out_v);
      }
    }
    if (!m.rms && u >= 0 && c.f.nodes[u].op == "stablehlo.add") {
      Node& an = c.f.nodes[u];
      int other = an.in[0] == out_v ? an.in[1] : an.in[0];
      int vec;
      if (match_last_axis_vector(c, other, C, vec)) {
        beta = vec;
        out_v = an.out[0];
        u = single_user(c, out_v);
      }
    }
    // Input / output dtype: read x in the dtype the output is stored in.
    int x = m.x;
    const DType od = c.ty(out_v).dtype;
    int xs = c.strip_convert(x);
    if (c.ty(xs).dtype == od) x = xs;
    if (u >= 0 && c.f.nodes[u].op == "stablehlo.convert" && c.ty(c.f.nodes[u].out[0]).dtype == c.ty(xs).dtype &&
        is_float(c.ty(xs).dtype)) {
      // f32 statistics of a bf16 input, converted back: one bf16 kernel.
      out_v = c.f.nodes[u].out[0];
      x = xs;
    }
    if (c.ty(x).dtype != c.ty(out_v).dtype || c.ty(x).dims != c.ty(out_v).dims) continue;
    if (!kernel_float(c.ty(x).dtype)) continue;
    for (int p : {gamma, beta})
      if (p >= 0 && !kernel_float(c.ty(p).dtype)) gamma = beta = -2;
    if (gamma == -2) continue;
    Node fused;
    fused.op = m.rms ? "mfx.rms_norm" : "mfx.layer_norm";
    fused.in = {x};
    fused.ints["has_gamma"] = {gamma >= 0 ? 1 : 0};
    fused.ints["has_beta"] = {beta >= 0 ? 1 : 0};
    if (gamma >= 0) fused.in.push_back(gamma);
    if (beta >= 0) fused.in.push_back(beta);
    fused.nums["eps"] = m.eps;
    fused.out = {out_v};
    int at = c.f.values[out_v].def;
    c.f.nodes[at] = fused;
    if (m.rms) st.rms_norm++;
    else st.layer_norm++;
    if (gamma >= 0 || beta >= 0) st.affine_absorbed++;
    ++count;
    c.refresh();
  }
  return count;
}

// ---- softmax -------------------------------------------------------------------

// The row max of a softmax-style chain: reduce_max over the last axis of x
// [through maximum(-inf, .)], seen through broadcasts.
bool match_row_max(Ctx& c, int v, int xv, int axis) {
  int mv = c.strip_all(v);
  Node* mn = c.def(mv);
  if (op_is(mn, "stablehlo.maximum")) {
    double lo;
    int keep = -1;
    for (int o = 0; o < 2; ++o)
      if (c.splat(mn->in[o], lo) && lo < -1e30) keep = mn->in[1 - o];
    if (keep < 0) return false;
    mv = keep;
  }
  int mx, ma;
  return match_reduce(c, mv, "stablehlo.maximum", mx, ma) && ma == axis && c.same(mx, xv);
}

// v == softmax(x) over the last axis; returns x.
bool match_softmax(Ctx& c, int v, int& x) {
  Node* d = c.def(v);
  if (!op_is(d, "stablehlo.divide")) return false;
  int e = d->in[0];
  Node* en = c.def(c.strip_convert(e));
  if (!op_is(en, "stablehlo.exponential")) return false;
  Node* sub = c.def(c.strip_convert(en->in[0]));
  if (!op_is(sub, "stablehlo.subtract")) return false;
  int xv = sub->in[0];
  const int axis = c.rank(xv) - 1;
  if (axis < 0) return false;
  // Denominator: sum of the same exp over the last axis.
  int sx, sa;
  if (!match_reduce(c, d->in[1], "stablehlo.add", sx, sa) || sa != axis || !c.same(sx, e)) return false;
  if (!match_row_max(c, sub->in[1], xv, axis)) return false;
  x = xv;
  return true;
}

int rewrite_softmax(Ctx& c, RewriteStats& st) {
  int count = 0;
  for (size_t i = 0; i < c.f.nodes.size(); ++i) {
    Node& n = c.f.nodes[i];
    if (n.dead || n.op != "stablehlo.divide" || n.out.size() != 1) continue;
    int x;
    if (!match_softmax(c, n.out[0], x)) continue;
    if (c.ty(x) != c.ty(n.out[0])) continue;
    if (!kernel_float(c.ty(x).dtype)) continue;
    Node fused;
    fused.op = "mfx.softmax";
    fused.in = {x};
    fused.out = n.out;
    n = fused;
    st.softmax++;
    ++count;
    c.refresh();
  }
  return count;
}

// v == log_softmax(x) over the last axis, in jax.nn.log_softmax's form
//   shifted = x - max(x);  v = shifted - log(sum(exp(shifted)))
// (the computation the reference special-cases for callee @log_softmax,
// src/jax_mlx_pjrt.cpp:5624-5641); returns x.
bool match_log_softmax(Ctx& c, int v, int& x) {
  Node* d = c.def(v);
  if (!op_is(d, "stablehlo.subtract")) return false;
  const int shifted = d->in[0];
  Node* sh = c.def(c.strip_convert(shifted));
  if (!op_is(sh, "stablehlo.subtract")) return false;
  const int xv = sh->in[0];
  const int axis = c.rank(xv) - 1;
  if (axis < 0) return false;
  Node* lg = c.def(c.strip_all(d->in[1]));
  if (!op_is(lg, "stablehlo.log")) return false;
  int sx, sa;
  if (!match_reduce(c, lg->in[0], "stablehlo.add", sx, sa) || sa != axis) return false;
  Node* en = c.def(c.strip_convert(sx));
  if (!op_is(en, "stablehlo.exponential") || !c.same(en->in[0], shifted)) return false;
  if (!match_row_max(c, sh->in[1], xv, axis)) return false;
  x = xv;
  return true;
}

int rewrite_log_softmax(Ctx& c, RewriteStats& st) {
  int count = 0;
  for (size_t i = 0; i < c.f.nodes.size(); ++i) {
    Node& n = c.f.nodes[i];
    if (n.dead || n.op != "stablehlo.subtract" || n.out.size() != 1) continue;
    int x;
    if (!match_log_softmax(c, n.out[0], x)) continue;
    if (c.ty(x) != c.ty(n.out[0])) continue;
    if (!kernel_float(c.ty(x).dtype)) continue;
    Node fused;
    fused.op = "mfx.log_softmax";
    fused.in = {x};
    fused.out = n.out;
    n = fused;
    st.log_softmax++;
    ++count;
    c.refresh();
  }
  return count;
}

// 1 / (1 + exp(-x)) -> logistic(x), the reference's sigmoid pattern
// (src/jax_mlx_pjrt.cpp:2046-2164: divide(1, add(1, exp(negate(x))))).  The
// result is one elementwise instruction instead of four; intermediates used
// elsewhere stay computed (the replaced divide is the only node rewritten).
int rewrite_sigmoid(Ctx& c, RewriteStats& st) {
  int count = 0;
  for (size_t i = 0; i < c.f.nodes.size(); ++i) {
    Node& n = c.f.nodes[i];
    if (n.dead || n.op != "stablehlo.divide" || n.out.size() != 1) continue;
    double one;
    if (!c.splat(n.in[0], one) || one != 1.0) continue;
    Node* ad = c.def(n.in[1]);
    if (!op_is(ad, "stablehlo.add")) continue;
    int e = -1;
    for (int o = 0; o < 2; ++o)
      if (c.splat(ad->in[o], one) && one == 1.0) e = ad->in[1 - o];
    Node* en = e >= 0 ? c.def(e) : nullptr;
    if (!op_is(en, "stablehlo.exponential")) continue;
    Node* ng = c.def(en->in[0]);
    if (!op_is(ng, "stablehlo.negate")) continue;
    const int x = ng->in[0];
    if (c.ty(x) != c.ty(n.out[0])) continue;
    Node fused;
    fused.op = "stablehlo.logistic";
    fused.in = {x};
    fused.out = n.out;
    n = fused;
    st.sigmoid++;
    ++count;
    c.refresh();
  }
  return count;
}

// ---- views: transpose / reshape / broadcast folded into strides ------------------

}  // namespace

std::vector<int64_t> contiguous_strides(const std::vector<int64_t>& dims) {
  std::vector<int64_t> s(dims.size(), 1);
  for (int i = (int)dims.size() - 2; i >= 0; --i) s[i] = s[i + 1] * dims[i + 1];
  return s;
}

bool reshape_strides(const std::vector<int64_t>& in_dims, const std::vector<int64_t>& in_strides,
                     const std::vector<int64_t>& out_dims, std::vector<int64_t>& out_strides) {
  int64_t total = 1, total_out = 1;
  for (int64_t x : in_dims) total *= x;
  for (int64_t x : out_dims) total_out *= x;
  if (total != total_out) return false;
  out_strides.assign(out_dims.size(), 0);
  if (total == 0) return true;
  if (in_dims.empty()) return true;  // scalar -> all-unit shape
  // Walk the input from its innermost dim in chunks of mutually contiguous
  // dims; each chunk must be covered exactly by a run of output dims, which
  // then split the chunk with strides relative to its innermost stride.
  int od = (int)out_dims.size() - 1;
  int64_t base = in_strides.back();
  int64_t chunk = 1, covered = 1;
  for (int id = (int)in_dims.size() - 1; id >= 0; --id) {
    chunk *= in_dims[id];
    bool chunk_end = id == 0 || (in_dims[id - 1] != 1 && in_strides[id - 1] != chunk * base);
    if (!chunk_end) continue;
    while (od >= 0 && (covered < chunk || out_dims[od] == 1)) {
      out_strides[od] = covered * base;
      covered *= out_dims[od];
      --od;
    }
    if (covered != chunk) return false;
    if (id > 0) {
      base = in_strides[id - 1];
      chunk = 1;
      covered = 1;
    }
  }
  return od == -1;
}

StridedView trace_view(const Function& f, int v, bool allow_broadcast) {
  const Type& t = f.values[v].type;
  int d = f.values[v].def;
  const Node* n = d < 0 ? nullptr : &f.nodes[d];
  auto leaf = [&]() {
    StridedView b;
    b.base = v;
    b.dims = t.dims;
    b.strides = contiguous_strides(t.dims);
    return b;
  };
  if (!n || n->dead) return leaf();
  StridedView out;
  auto get = [&](const char* k) -> const std::vector<int64_t>& { return n->ints.at(k); };
  if (n->op == "stablehlo.transpose") {
    StridedView x = trace_view(f, n->in[0], allow_broadcast);
    const auto& perm = get("dims");
    out.base = x.base;
    out.offset = x.offset;
    for (size_t i = 0; i < perm.size(); ++i) {
      out.dims.push_back(x.dims[perm[i]]);
      out.strides.push_back(x.strides[perm[i]]);
    }
  } else if (n->op == "stablehlo.reshape" ||
             (n->op == "stablehlo.convert" && f.values[n->in[0]].type.dtype == t.dtype)) {
    StridedView x = trace_view(f, n->in[0], allow_broadcast);
    std::vector<int64_t> st;
    if (!reshape_strides(x.dims, x.strides, t.dims, st)) return leaf();
    out.base = x.base;
    out.offset = x.offset;
    out.dims = t.dims;
    out.strides = st;
  } else if (n->op == "stablehlo.broadcast_in_dim" && allow_broadcast) {
    StridedView x = trace_view(f, n->in[0], allow_broadcast);
    const auto& bd = get("dims");
    out.base = x.base;
    out.offset = x.offset;
    out.dims = t.dims;
    out.strides.assign(t.dims.size(), 0);
    for (size_t i = 0; i < bd.size(); ++i)
      out.strides[bd[i]] = (x.dims[i] == 1 && t.dims[bd[i]] != 1) ? 0 : x.strides[i];
  } else if (n->op == "stablehlo.slice") {
    StridedView x = trace_view(f, n->in[0], allow_broadcast);
    const auto& st = get("start");
    const auto& sd = get("stride");
    out.base = x.base;
    out.offset = x.offset;
    out.dims = t.dims;
    for (size_t i = 0; i < st.size(); ++i) {
      out.offset += st[i] * x.strides[i];
      out.strides.push_back(x.strides[i] * sd[i]);
    }
  } else {
    return leaf();
  }
  return out;
}

namespace {

using View = StridedView;
std::vector<int64_t> contiguous(const std::vector<int64_t>& dims) { return contiguous_strides(dims); }
View trace_view(Ctx& c, int v, bool allow_broadcast) { return mfxp::trace_view(c.f, v, allow_broadcast); }

// ---- mask expressions: causal detection by evaluation over (t, s) -----------------

// Evaluates one row (fixed t, all s) of an elementwise expression that depends
// only on iotas and constants.  role[d] says what dim d of value v follows:
// 0 = the query index t, 1 = the key index s, -1 = a fixed coordinate fixed[d].
// Sets *other when the value would vary along a fixed dim (an iota over it or
// a non-splat constant spanning it), so the caller knows the predicate is not
// the same for every batch/head.  Returns false on a non-constant leaf or an
// op outside the evaluated set.
bool eval_row(Ctx& c, int v, const std::vector<int>& role, const std::vector<int64_t>& fixed, int64_t t,
              int64_t S, std::vector<double>& out, bool* other, int depth = 0) {
  if (depth > 64) return false;
  Node* n = c.def(v);
  if (!n) return false;
  const std::string& op = n->op;
  out.assign((size_t)S, 0.0);
  if (op == "stablehlo.constant") {
    const Literal& l = *n->literal;
    if (l.splat) {
      std::fill(out.begin(), out.end(), l.values[0]);
      return true;
    }
    const auto& dims = l.type.dims;
    auto st = contiguous(dims);
    int64_t base = 0, s_stride = 0;
    for (size_t d = 0; d < dims.size(); ++d) {
      if (role[d] == 0) base += t * st[d];
      else if (role[d] == 1) s_stride += st[d];
      else {
        if (dims[d] > 1) *other = true;
        base += fixed[d] * st[d];
      }
    }
    for (int64_t s = 0; s < S; ++s) out[s] = l.values.at(base + s * s_stride);
    return true;
  }
  if (op == "stablehlo.iota") {
    const int d = (int)n->ints["dim"].at(0);
    if (role[d] == 1)
      for (int64_t s = 0; s < S; ++s) out[s] = (double)s;
    else {
      if (role[d] == -1 && c.ty(v).dims[d] > 1) *other = true;
      std::fill(out.begin(), out.end(), role[d] == 0 ? (double)t : (double)fixed[d]);
    }
    return true;
  }
  if (op == "stablehlo.broadcast_in_dim" || op == "stablehlo.transpose" || op == "stablehlo.reshape") {
    const Type& it = c.ty(n->in[0]);
    std::vector<int> ir(it.dims.size(), -1);
    std::vector<int64_t> ifx(it.dims.size(), 0);
    if (op == "stablehlo.broadcast_in_dim") {
      const auto& bd = n->ints["dims"];
      for (size_t i = 0; i < bd.size(); ++i)
        if (it.dims[i] != 1) {
          ir[i] = role[bd[i]];
          ifx[i] = fixed[bd[i]];
        }
    } else if (op == "stablehlo.transpose") {
      const auto& perm = n->ints["dims"];
      for (size_t i = 0; i < perm.size(); ++i) {
        ir[perm[i]] = role[i];
        ifx[perm[i]] = fixed[i];
      }
    } else {
      // Only reshapes that insert or drop unit dims keep a per-dim mapping.
      const Type& ot = c.ty(v);
      size_t j = 0;
      for (size_t i = 0; i < it.dims.size(); ++i) {
        if (it.dims[i] == 1) continue;
        while (j < ot.dims.size() && ot.dims[j] == 1) ++j;
        if (j == ot.dims.size() || ot.dims[j] != it.dims[i]) return false;
        ir[i] = role[j];
        ifx[i] = fixed[j];
        ++j;
      }
      for (; j < ot.dims.size(); ++j)
        if (ot.dims[j] != 1) return false;
    }
    return eval_row(c, n->in[0], ir, ifx, t, S, out, other, depth + 1);
  }
  if (op == "stablehlo.convert") {
    if (!eval_row(c, n->in[0], role, fixed, t, S, out, other, depth + 1)) return false;
    if (c.ty(v).dtype == DType::kPred)
      for (auto& x : out) x = x != 0.0;
    return true;
  }
  const size_t na = n->in.size();
  if (na < 1 || na > 3) return false;
  std::vector<double> a[3];
  for (size_t i = 0; i < na; ++i)
    if (!eval_row(c, n->in[i], role, fixed, t, S, a[i], other, depth + 1)) return false;
  auto each = [&](auto f) {
    for (int64_t s = 0; s < S; ++s) out[s] = f(s);
  };
  if (op == "stablehlo.compare") {
    const std::string& d = n->strs["comparison_direction"];
    const auto& x = a[0];
    const auto& y = a[1];
    if (d == "EQ") each([&](int64_t s) { return (double)(x[s] == y[s]); });
    else if (d == "NE") each([&](int64_t s) { return (double)(x[s] != y[s]); });
    else if (d == "LT") each([&](int64_t s) { return (double)(x[s] < y[s]); });
    else if (d == "LE") each([&](int64_t s) { return (double)(x[s] <= y[s]); });
    else if (d == "GT") each([&](int64_t s) { return (double)(x[s] > y[s]); });
    else if (d == "GE") each([&](int64_t s) { return (double)(x[s] >= y[s]); });
    else return false;
    return true;
  }
  if (op == "stablehlo.and") each([&](int64_t s) { return (double)(a[0][s] != 0 && a[1][s] != 0); });
  else if (op == "stablehlo.or") each([&](int64_t s) { return (double)(a[0][s] != 0 || a[1][s] != 0); });
  else if (op == "stablehlo.not") each([&](int64_t s) { return (double)(a[0][s] == 0); });
  else if (op == "stablehlo.select") each([&](int64_t s) { return a[0][s] != 0 ? a[1][s] : a[2][s]; });
  else if (op == "stablehlo.add") each([&](int64_t s) { return a[0][s] + a[1][s]; });
  else if (op == "stablehlo.subtract") each([&](int64_t s) { return a[0][s] - a[1][s]; });
  else if (op == "stablehlo.multiply") each([&](int64_t s) { return a[0][s] * a[1][s]; });
  else if (op == "stablehlo.negate") each([&](int64_t s) { return -a[0][s]; });
  else if (op == "stablehlo.maximum") each([&](int64_t s) { return std::max(a[0][s], a[1][s]); });
  else if (op == "stablehlo.minimum") each([&](int64_t s) { return std::min(a[0][s], a[1][s]); });
  else return false;
  return true;
}

// Is predicate p (shape = scores layout) exactly "s <= t" (causal, top-left)
// over dims (t_dim, s_dim) and independent of every other dim?  Every (t, s)
// is evaluated; independence is shown structurally (no iota or non-splat
// constant spans another dim).
bool is_causal_pred(Ctx& c, int p, int t_dim, int s_dim) {
  const Type& pt = c.ty(p);
  const int64_t T = pt.dims[t_dim], S = pt.dims[s_dim];
  std::vector<int> role(pt.dims.size(), -1);
  role[t_dim] = 0;
  role[s_dim] = 1;
  const std::vector<int64_t> fixed(pt.dims.size(), 0);
  std::vector<double> row;
  bool other = false;
  for (int64_t t = 0; t < T; ++t) {
    if (!eval_row(c, p, role, fixed, t, S, row, &other) || other) return false;
    for (int64_t s = 0; s < S; ++s)
      if ((row[s] != 0.0) != (s <= t)) return false;
  }
  return true;
}

// ---- SDPA ------------------------------------------------------------------------

struct Chain {
  int dot = -1;                  // QK dot_general node index
  double scale = 1.0;
  std::vector<int> perm;         // X dim i = dot-result dim perm[i]
  int bias = -1;                 // additive bias value (in its own layout)
  std::vector<int> bias_perm;    // bias dim i = dot-result dim bias_perm[i]
  int pred = -1;                 // select predicate (in its own layout)
  std::vector<int> pred_perm;
  double neg = 0;                // select's masked value
};

// Walks from the softmax input X back to the QK dot_general.
bool trace_scores(Ctx& c, int x, Chain& ch) {
  std::vector<int> perm(c.rank(x));
  for (size_t i = 0; i < perm.size(); ++i) perm[i] = (int)i;
  int v = x;
  for (int guard = 0; guard < 32; ++guard) {
    Node* n = c.def(v);
    if (!n) return false;
    const std::string& op = n->op;
    if (op == "stablehlo.dot_general") {
      ch.dot = c.f.values[v].def;
      ch.perm = perm;
      return true;
    }
    if (op == "stablehlo.convert" && is_float(c.ty(n->in[0]).dtype)) {
      v = n->in[0];
      continue;
    }
    if (op == "stablehlo.transpose") {
      const auto& tp = n->ints["dims"];
      std::vector<int> np(perm.size());
      for (size_t i = 0; i < perm.size(); ++i) np[i] = (int)tp[perm[i]];
      perm = np;
      v = n->in[0];
      continue;
    }
    if (op == "stablehlo.multiply") {
      double k;
      if (c.splat(n->in[1], k)) { ch.scale *= k; v = n->in[0]; continue; }
      if (c.splat(n->in[0], k)) { ch.scale *= k; v = n->in[1]; continue; }
      return false;
    }
    if (op == "stablehlo.divide") {
      double k;
      if (c.splat(n->in[1], k) && k != 0.0) { ch.scale /= k; v = n->in[0]; continue; }
      return false;
    }
    if (op == "stablehlo.add") {
      if (ch.bias >= 0) return false;
      // The bias side is the one that does not lead back to a dot_general.
      for (int o = 0; o < 2; ++o) {
        Chain probe;
        if (trace_scores(c, n->in[o], probe)) {
          ch.bias = n->in[1 - o];
          ch.bias_perm = perm;
          v = n->in[o];
          break;
        }
      }
      if (ch.bias < 0) return false;
      // Scale applied after the bias would scale the bias too.
      if (ch.scale != 1.0) return false;
      continue;
    }
    if (op == "stablehlo.select") {
      if (ch.pred >= 0) return false;
      double neg;
      if (!c.splat(n->in[2], neg) || !(neg < -1e30 || std::isinf(neg))) return false;
      ch.pred = n->in[0];
      ch.pred_perm = perm;
      ch.neg = neg;
      if (ch.scale != 1.0) return false;
      v = n->in[1];
      continue;
    }
    return false;
  }
  return false;
}

// Map (b, h, t, d)-style kernel strides out of a view over labelled dims.
struct Labels {
  int nb = 0;                  // number of batch dims (1 or 2)
  std::vector<int64_t> bdims;  // extents of batch dims
  int64_t G = 1, T = 0, S = 0, D = 0, Dv = 0;
};

int rewrite_sdpa(Ctx& c, RewriteStats& st) {
  int count = 0;
  for (size_t pi = 0; pi < c.f.nodes.size(); ++pi) {
    Node& pv = c.f.nodes[pi];
    if (pv.dead || pv.op != "stablehlo.dot_general" || pv.in.size() != 2) continue;
    // ---- PV dot: lhs = probabilities, rhs = V
    int P = c.strip_convert(pv.in[0]);
    int X;
    if (!match_softmax(c, P, X)) continue;
    Chain ch;
    if (!trace_scores(c, X, ch)) continue;
    // Masks were recorded in the layout where they apply; express their dims
    // as dot-result dims (perm at record time maps X dims to that layout).
    auto to_result = [&](std::vector<int>& lay) {
      if (lay.empty()) return;
      std::vector<int> fixed(lay.size());
      for (size_t i = 0; i < lay.size(); ++i) fixed[lay[i]] = ch.perm[i];
      lay = fixed;
    };
    to_result(ch.pred_perm);
    to_result(ch.bias_perm);
    Node& qk = c.f.nodes[ch.dot];
    auto& qlb = qk.ints["lhs_batching_dims"];
    auto& qrb = qk.ints["rhs_batching_dims"];
    auto& qlc = qk.ints["lhs_contracting_dims"];
    auto& qrc = qk.ints["rhs_contracting_dims"];
    if (qlc.size() != 1 || qrc.size() != 1 || qlb.size() != qrb.size()) continue;
    const int nb = (int)qlb.size();
    if (nb < 1 || nb > 2) continue;
    const Type& qt = c.ty(qk.in[0]);
    const Type& kt = c.ty(qk.in[1]);
    std::vector<int> qfree, kfree;
    for (int i = 0; i < qt.rank(); ++i)
      if (std::find(qlb.begin(), qlb.end(), i) == qlb.end() && i != qlc[0]) qfree.push_back(i);
    for (int i = 0; i < kt.rank(); ++i)
      if (std::find(qrb.begin(), qrb.end(), i) == qrb.end() && i != qrc[0]) kfree.push_back(i);
    if (kfree.size() != 1 || qfree.empty() || qfree.size() > 2) continue;
    // dot-result layout: [batch (nb), qfree..., kfree]
    const int r_rank = nb + (int)qfree.size() + 1;
    const int s_pos = r_rank - 1;
    if ((int)ch.perm.size() != r_rank) continue;
    // Softmax ran over X's last dim: must be the key dim.
    if (ch.perm.back() != s_pos) continue;
    // PV dims: lhs (X layout) batching must be the batch dims in order, contracting the key dim.
    auto& plb = pv.ints["lhs_batching_dims"];
    auto& prb = pv.ints["rhs_batching_dims"];
    auto& plc = pv.ints["lhs_contracting_dims"];
    auto& prc = pv.ints["rhs_contracting_dims"];
    if ((int)plb.size() != nb || prb.size() != plb.size() || plc.size() != 1 || prc.size() != 1) continue;
    if (ch.perm[plc[0]] != s_pos) continue;
    bool ok = true;
    for (int i = 0; i < nb; ++i) ok &= ch.perm[plb[i]] == i;
    if (!ok) continue;
    const Type& vt = c.ty(pv.in[1]);
    std::vector<int> vfree;
    for (int i = 0; i < vt.rank(); ++i)
      if (std::find(prb.begin(), prb.end(), i) == prb.end() && i != prc[0]) vfree.push_back(i);
    if (vfree.size() != 1) continue;
    // PV lhs free dims, in X order, as dot-result dims (query-side free dims).
    std::vector<int> pfree_res;
    for (int i = 0; i < r_rank; ++i)
      if (std::find(plb.begin(), plb.end(), i) == plb.end() && i != plc[0]) pfree_res.push_back(ch.perm[i]);
    // ---- labels
    Labels L;
    L.nb = nb;
    for (int i = 0; i < nb; ++i) {
      if (qt.dims[qlb[i]] != kt.dims[qrb[i]] || kt.dims[qrb[i]] != vt.dims[prb[i]]) ok = false;
      L.bdims.push_back(qt.dims[qlb[i]]);
    }
    L.D = qt.dims[qlc[0]];
    L.S = kt.dims[kfree[0]];
    L.Dv = vt.dims[vfree[0]];
    if (!ok || kt.dims[qrc[0]] != L.D || vt.dims[prc[0]] != L.S) continue;
    // Which query free dim is T (the other, if any, is the GQA group G).
    // Result positions of query free dims: nb .. nb+qfree-1.
    int t_res = nb, g_res = -1;
    bool causal = false;
    if (qfree.size() == 2) {
      t_res = -1;
    }
    // Causal / data masks (in the layout where they were applied).
    auto res_to_pred = [&](const std::vector<int>& lay, int res_dim) {
      for (size_t i = 0; i < lay.size(); ++i)
        if (lay[i] == res_dim) return (int)i;
      return -1;
    };
    int mask_val = -1;
    std::vector<int> mask_perm;
    if (ch.pred >= 0) {
      int sp = res_to_pred(ch.pred_perm, s_pos);
      std::vector<int> cands;
      for (int q = nb; q < nb + (int)qfree.size(); ++q) cands.push_back(q);
      for (int q : cands) {
        if (t_res >= 0 && q != t_res) continue;
        if (is_causal_pred(c, ch.pred, res_to_pred(ch.pred_perm, q), sp)) {
          causal = true;
          t_res = q;
          break;
        }
      }
      if (!causal) {
        mask_val = ch.pred;  // data mask: converted to an additive mask below
        mask_perm = ch.pred_perm;
      }
    }
    if (qfree.size() == 2) {
      if (t_res < 0) {
        // No causal structure: a unit dim is T (decode), else the first.
        int a = nb, b = nb + 1;
        int ta = (int)qt.dims[qfree[0]], tb = (int)qt.dims[qfree[1]];
        t_res = (tb == 1 && ta != 1) ? b : a;
      }
      g_res = t_res == nb ? nb + 1 : nb;
    }
    const int q_t_dim = qfree[t_res - nb];
    const int q_g_dim = g_res >= 0 ? qfree[g_res - nb] : -1;
    L.T = qt.dims[q_t_dim];
    L.G = q_g_dim >= 0 ? qt.dims[q_g_dim] : 1;
    // ---- views of q, k, v
    // Views whose feature dim is not unit-stride read the operand itself,
    // which the planner then materialises contiguously.
    auto unit_view = [&](int val, int feat_dim) {
      View w = trace_view(c, val, false);
      if (w.strides[feat_dim] != 1) {
        w = View{};
        w.base = val;
        w.dims = c.ty(val).dims;
        w.strides = contiguous(w.dims);
      }
      return w;
    };
    View qv = unit_view(qk.in[0], (int)qlc[0]);
    View kv = unit_view(qk.in[1], (int)qrc[0]);
    View vv = unit_view(pv.in[1], vfree[0]);
    auto qs = [&](int dim) { return qv.strides[dim]; };
    // Kernel head index h = hb*G + g with hb the last batch dim.
    const int64_t Hkv_ext = L.bdims[nb - 1];
    // Kernel head h = hb*G + g needs one stride: s_hb == G * s_g.
    auto merge_h = [&](int64_t s_hb, int64_t s_g, int64_t& sh) {
      if (L.G == 1) { sh = s_hb; return true; }
      if (Hkv_ext == 1 || s_hb == L.G * s_g) { sh = s_g; return true; }
      return false;
    };
    int64_t q_sb = nb == 2 ? qs(qlb[0]) : 0, q_sh, q_st = qs(q_t_dim), q_sd = qs(qlc[0]);
    if (!merge_h(qs(qlb[nb - 1]), q_g_dim >= 0 ? qs(q_g_dim) : 0, q_sh)) continue;
    int64_t k_sb = nb == 2 ? kv.strides[qrb[0]] : 0, k_sh = kv.strides[qrb[nb - 1]];
    int64_t k_ss = kv.strides[kfree[0]], k_sd = kv.strides[qrc[0]];
    int64_t v_sb = nb == 2 ? vv.strides[prb[0]] : 0, v_sh = vv.strides[prb[nb - 1]];
    int64_t v_ss = vv.strides[prc[0]], v_sd = vv.strides[vfree[0]];
    if (q_sd != 1 || k_sd != 1 || v_sd != 1) continue;
    // ---- output: PV result [batch (nb), pfree (X order), Dv] -> follow views forward
    int out_v = pv.out[0];
    std::vector<int64_t> out_dims = c.ty(out_v).dims;
    // Follow a single-use chain of transposes / view reshapes.
    std::vector<int> fwd;
    for (int guard = 0; guard < 8; ++guard) {
      int u = single_user(c, out_v);
      if (u < 0) break;
      Node& un = c.f.nodes[u];
      if (un.op != "stablehlo.transpose" && un.op != "stablehlo.reshape") break;
      fwd.push_back(u);
      out_v = un.out[0];
    }
    // Strides of the PV result dims inside out_v's contiguous buffer: walk back.
    std::vector<int64_t> cur_dims = c.ty(out_v).dims, cur_str = contiguous(cur_dims);
    bool view_ok = true;
    for (size_t k = fwd.size(); k-- > 0;) {
      Node& un = c.f.nodes[fwd[k]];
      const Type& in_t = c.ty(un.in[0]);
      if (un.op == "stablehlo.transpose") {
        const auto& perm = un.ints["dims"];
        std::vector<int64_t> s2(perm.size());
        for (size_t i = 0; i < perm.size(); ++i) s2[perm[i]] = cur_str[i];
        cur_str = s2;
      } else {
        std::vector<int64_t> s2;
        if (!reshape_strides(cur_dims, cur_str, in_t.dims, s2)) {
          view_ok = false;
          break;
        }
        cur_str = s2;
      }
      cur_dims = in_t.dims;
    }
    if (!view_ok) {
      out_v = pv.out[0];
      cur_dims = c.ty(out_v).dims;
      cur_str = contiguous(cur_dims);
    }
    // PV result position of the T / G query dims.
    int o_t = -1, o_g = -1;
    for (size_t i = 0; i < pfree_res.size(); ++i) {
      if (pfree_res[i] == t_res) o_t = nb + (int)i;
      if (pfree_res[i] == g_res) o_g = nb + (int)i;
    }
    const int o_d = (int)cur_dims.size() - 1;
    int64_t o_sb = nb == 2 ? cur_str[0] : 0, o_st = cur_str[o_t], o_sd = cur_str[o_d], o_sh;
    if (!merge_h(cur_str[nb - 1], o_g >= 0 ? cur_str[o_g] : 0, o_sh)) continue;
    if (o_sd != 1) continue;
    // ---- mask tensor (bias or predicate), as (b, h, t, s) strides
    int mask_in = -1;
    int64_t mask_off = 0;
    std::vector<int64_t> ms(4, 0);
    auto mask_strides = [&](int val, const std::vector<int>& lay) -> bool {
      View mv = trace_view(c, val, true);
      // dot-result dim -> stride
      std::vector<int64_t> rs(r_rank, 0);
      for (size_t i = 0; i < lay.size(); ++i) rs[lay[i]] = mv.strides[i];
      int64_t sh;
      if (!merge_h(rs[nb - 1], g_res >= 0 ? rs[g_res] : 0, sh)) return false;
      ms = {nb == 2 ? rs[0] : 0, sh, rs[t_res], rs[s_pos]};
      mask_in = mv.base;
      mask_off = mv.offset;
      return true;
    };
    int mask_kind = 0;  // 1 additive bias, 2 boolean predicate
    if (ch.bias >= 0) {
      if (mask_val >= 0) continue;  // bias and data predicate together: leave unfused
      if (!mask_strides(ch.bias, ch.bias_perm)) continue;
      mask_kind = 1;
    } else if (mask_val >= 0) {
      if (!mask_strides(mask_val, mask_perm)) continue;
      mask_kind = 2;
    }
    if (mask_kind) {
      DType md = c.ty(mask_in).dtype;
      if (mask_kind == 1 && !kernel_float(md)) continue;
    }
    DType qd = c.ty(qv.base).dtype, kd = c.ty(kv.base).dtype, vd = c.ty(vv.base).dtype;
    DType od = c.ty(out_v).dtype;
    if (qd != kd || kd != vd || !kernel_float(qd)) continue;
    if (od != qd) {
      // f32 accumulate then convert: absorb a trailing convert to the input dtype.
      int u = single_user(c, out_v);
      if (u >= 0 && c.f.nodes[u].op == "stablehlo.convert" && c.ty(c.f.nodes[u].out[0]).dtype == qd &&
          view_ok) {
        out_v = c.f.nodes[u].out[0];
      } else {
        continue;
      }
    }
    // ---- emit
    Node fused;
    fused.op = "mfx.sdpa";
    fused.in = {qv.base, kv.base, vv.base};
    int64_t Hkv = L.bdims[nb - 1];
    int64_t B = nb == 2 ? L.bdims[0] : 1;
    fused.ints["shape"] = {B, Hkv * L.G, Hkv, L.T, L.S, L.D, L.Dv};
    fused.ints["q_strides"] = {q_sb, q_sh, q_st, q_sd};
    fused.ints["k_strides"] = {k_sb, k_sh, k_ss, k_sd};
    fused.ints["v_strides"] = {v_sb, v_sh, v_ss, v_sd};
    fused.ints["o_strides"] = {o_sb, o_sh, o_st, o_sd};
    fused.ints["causal"] = {causal ? 1 : 0};
    fused.ints["mask_kind"] = {mask_kind};
    fused.ints["offsets"] = {qv.offset, kv.offset, vv.offset, mask_off};
    fused.nums["scale"] = ch.scale;
    fused.nums["mask_neg"] = ch.neg;
    if (mask_kind) {
      fused.in.push_back(mask_in);
      fused.ints["mask_strides"] = ms;
    }
    fused.out = {out_v};
    int at = c.f.values[out_v].def;
    c.f.nodes[at] = fused;
    st.sdpa++;
    ++count;
    c.refresh();
  }
  return count;
}

// RMSNorm(q) -> SDPA: the attention kernel normalises q rows itself.
void fold_rms_into_sdpa(Ctx& c) {
  for (Node& n : c.f.nodes) {
    if (n.dead || n.op != "mfx.sdpa" || n.ints.count("q_rms")) continue;
    int q = n.in[0];
    Node* r = c.def(q);
    if (!op_is(r, "mfx.rms_norm") || c.uses[q] != 1) continue;
    int x = r->in[0];
    if (c.ty(x) != c.ty(q)) continue;
    n.in[0] = x;
    n.nums["q_rms_eps"] = r->nums["eps"];
    n.ints["q_rms"] = {1};
    if (r->ints["has_gamma"].at(0)) {
      int w = r->in[1];
      if (c.ty(w).dtype != c.ty(q).dtype) {
        n.in[0] = q;
        n.ints.erase("q_rms");
        n.nums.erase("q_rms_eps");
        continue;
      }
      n.in.push_back(w);
      n.ints["q_rms_weight_index"] = {(int64_t)n.in.size() - 1};
    }
    c.refresh();
  }
}

// ---- the reference's custom_call targets ---------------------------------------

bool json_number(const std::string& cfg, const std::string& key, double& out) {
  size_t k = cfg.find("\"" + key + "\"");
  if (k == std::string::npos) return false;
  size_t colon = cfg.find(':', k);
  if (colon == std::string::npos) return false;
  const char* s = cfg.c_str() + colon + 1;
  char* end = nullptr;
  double v = std::strtod(s, &end);
  if (end == s || !std::isfinite(v)) throw ParseError("backend_config \"" + key + "\" is not a number: " + cfg);
  out = v;
  return true;
}

int rewrite_custom_calls(Ctx& c, RewriteStats& st) {
  int count = 0;
  for (Node& n : c.f.nodes) {
    if (n.dead || n.op != "stablehlo.custom_call") continue;
    const std::string& target = n.strs["target"];
    const std::string cfg = n.strs.count("backend_config") ? n.strs["backend_config"] : "";
    if (target == "mlx_sdpa") {
      // q (B,T,N,H), k/v (B,S,K,H) contiguous BTNH; out like q.
      if (n.in.size() != 3 || n.out.size() != 1) throw ParseError("mlx_sdpa expects 3 operands and 1 result");
      const Type& qt = c.ty(n.in[0]);
      const Type& kt = c.ty(n.in[1]);
      if (qt.rank() != 4 || kt.rank() != 4) throw ParseError("mlx_sdpa expects rank-4 BTNH operands");
      double scale = 1.0;
      json_number(cfg, "scale", scale);
      int64_t B = qt.dims[0], T = qt.dims[1], N = qt.dims[2], H = qt.dims[3];
      int64_t S = kt.dims[1], K = kt.dims[2];
      const Type& vt = c.ty(n.in[2]);
      if (vt.rank() != 4 || kt.dims[0] != B || kt.dims[3] != H || vt.dims[0] != B || vt.dims[1] != S ||
          vt.dims[2] != K || K <= 0 || N % K != 0)
        throw ParseError("mlx_sdpa operand shapes do not agree");
      if (c.ty(n.out[0]).dims != std::vector<int64_t>{B, T, N, vt.dims[3]})
        throw ParseError("mlx_sdpa result shape does not agree with q and v");
      Node f;
      f.op = "mfx.sdpa";
      f.in = n.in;
      f.out = n.out;
      f.ints["shape"] = {B, N, K, T, S, H, c.ty(n.in[2]).dims[3]};
      f.ints["q_strides"] = {T * N * H, H, N * H, 1};
      f.ints["k_strides"] = {S * K * H, H, K * H, 1};
      f.ints["v_strides"] = {S * K * c.ty(n.in[2]).dims[3], c.ty(n.in[2]).dims[3], K * c.ty(n.in[2]).dims[3], 1};
      int64_t Dv = c.ty(n.out[0]).dims[3];
      f.ints["o_strides"] = {T * N * Dv, Dv, N * Dv, 1};
      f.ints["causal"] = {0};
      f.ints["mask_kind"] = {0};
      f.ints["offsets"] = {0, 0, 0, 0};
      f.nums["scale"] = scale;
      f.nums["mask_neg"] = 0;
      n = f;
      st.custom_calls++;
      st.sdpa++;
      ++count;
    } else if (target == "mlx_layer_norm") {
      if (n.in.size() != 3 || n.out.size() != 1) throw ParseError("mlx_layer_norm expects 3 operands");
      double eps = 1e-5;
      json_number(cfg, "eps", eps);
      Node f;
      f.op = "mfx.layer_norm";
      f.in = n.in;
      f.out = n.out;
      f.ints["has_gamma"] = {1};
      f.ints["has_beta"] = {1};
      f.nums["eps"] = eps;
      n = f;
      st.custom_calls++;
      st.layer_norm++;
      ++count;
    } else if (target == "mlx_sdpa_bwd") {
      // (q, k, v, grad_out) BTNH -> (dq, dk, dv) like the operands
      // (reference src/jax_mlx/sdpa.py:52-60, handler src/jax_mlx_pjrt.cpp:8151-8206).
      if (n.in.size() != 4 || n.out.size() != 3)
        throw ParseError("mlx_sdpa_bwd expects 4 operands and 3 results");
      const Type& qt = c.ty(n.in[0]);
      const Type& kt = c.ty(n.in[1]);
      const Type& vt = c.ty(n.in[2]);
      if (qt.rank() != 4 || kt.rank() != 4 || vt.rank() != 4) throw ParseError("mlx_sdpa_bwd expects rank-4 BTNH operands");
      const int64_t B = qt.dims[0], T = qt.dims[1], N = qt.dims[2], H = qt.dims[3];
      const int64_t S = kt.dims[1], K = kt.dims[2], Hv = vt.dims[3];
      if (kt.dims[0] != B || kt.dims[3] != H || vt.dims[0] != B || vt.dims[1] != S || vt.dims[2] != K ||
          K <= 0 || N % K != 0)
        throw ParseError("mlx_sdpa_bwd operand shapes do not agree");
      if (c.ty(n.in[3]).dims != std::vector<int64_t>{B, T, N, Hv} || c.ty(n.out[0]).dims != qt.dims ||
          c.ty(n.out[1]).dims != kt.dims || c.ty(n.out[2]).dims != vt.dims)
        throw ParseError("mlx_sdpa_bwd grad_out / result shapes do not agree with q, k, v");
      double scale = 1.0;
      json_number(cfg, "scale", scale);
      Node f;
      f.op = "mfx.sdpa_bwd";
      f.in = n.in;
      f.out = n.out;
      f.ints["shape"] = {B, N, K, T, S, H, Hv};
      f.nums["scale"] = scale;
      n = f;
      st.custom_calls++;
      ++count;
    } else if (target == "mlx_layer_norm_bwd") {
      // (x, weight, bias, grad_out) -> (dx, dweight, dbias); bias only fixes
      // the dbias type (reference src/jax_mlx/layer_norm.py:46-56).
      if (n.in.size() != 4 || n.out.size() != 3)
        throw ParseError("mlx_layer_norm_bwd expects 4 operands and 3 results");
      const Type& xt = c.ty(n.in[0]);
      const Type& wt = c.ty(n.in[1]);
      if (xt.rank() < 1 || wt.rank() != 1 || wt.dims[0] != xt.dims.back())
        throw ParseError("mlx_layer_norm_bwd weight must be [N] for x [..., N]");
      if (c.ty(n.in[3]).dims != xt.dims || c.ty(n.out[0]).dims != xt.dims)
        throw ParseError("mlx_layer_norm_bwd grad_out and dx must have x's shape");
      if (c.ty(n.out[1]).dims != wt.dims || c.ty(n.out[2]).dims != wt.dims ||
          c.ty(n.out[1]).dtype != c.ty(n.out[2]).dtype)
        throw ParseError("mlx_layer_norm_bwd dweight and dbias must be [N] of one dtype");
      double eps = 1e-5;
      json_number(cfg, "eps", eps);
      Node f;
      f.op = "mfx.layer_norm_bwd";
      f.in = {n.in[0], n.in[1], n.in[3]};
      f.out = n.out;
      f.nums["eps"] = eps;
      n = f;
      st.custom_calls++;
      ++count;
    }
  }
  if (count) c.refresh();
  return count;
}

}  // namespace

// ---- public entry points ------------------------------------------------------------

void compact(Function& f) {
  // Iterative DCE over nodes whose results are unused.
  bool changed = true;
  while (changed) {
    changed = false;
    std::vector<int> u = use_counts(f);
    for (Node& n : f.nodes) {
      if (n.dead) continue;
      bool used = false;
      for (int v : n.out) used |= u[v] > 0;
      if (!used) {
        n.dead = true;
        changed = true;
      }
    }
  }
  std::vector<Node> live;
  for (Node& n : f.nodes)
    if (!n.dead) live.push_back(std::move(n));
  f.nodes = std::move(live);
  for (Value& v : f.values) v.def = -1;
  for (size_t i = 0; i < f.nodes.size(); ++i)
    for (size_t k = 0; k < f.nodes[i].out.size(); ++k) {
      f.values[f.nodes[i].out[k]].def = (int)i;
      f.values[f.nodes[i].out[k]].def_result = (int)k;
    }
}

void inline_calls(Module& m) {
  for (auto& fp : m.funcs) {
    Function& f = *fp;
    for (int round = 0; round < 64; ++round) {
      bool any = false;
      std::vector<Node> out;
      out.reserve(f.nodes.size());
      for (Node& n : f.nodes) {
        if (n.op != "func.call") {
          out.push_back(std::move(n));
          continue;
        }
        auto callee = m.find(n.strs["callee"]);
        if (!callee) throw ParseError("call to unknown function @" + n.strs["callee"]);
        if (callee.get() == &f) throw ParseError("recursive call to @" + f.name);
        if (callee->params.size() != n.in.size() || callee->results.size() != n.out.size())
          throw ParseError("call to @" + callee->name + " has mismatched arity");
        any = true;
        std::map<int, int> remap;  // callee value -> caller value
        for (size_t i = 0; i < callee->params.size(); ++i) remap[callee->params[i]] = n.in[i];
        for (const Node& cn : callee->nodes) {
          Node copy = cn;
          for (int& v : copy.in) v = remap.at(v);
          for (int& v : copy.out) {
            int nv = f.add_value(callee->values[v].name + "@" + callee->name, callee->values[v].type);
            remap[v] = nv;
            v = nv;
          }
          out.push_back(std::move(copy));
        }
        // Results: alias call outputs to callee results through a copy-free rename.
        for (size_t i = 0; i < n.out.size(); ++i) {
          int src = remap.at(callee->results[i]);
          int dst = n.out[i];
          // Replace uses of dst by src in the rest of the function.
          for (Node& later : f.nodes)
            for (int& v : later.in)
              if (v == dst) v = src;
          for (Node& done : out)
            for (int& v : done.in)
              if (v == dst) v = src;
          for (int& v : f.results)
            if (v == dst) v = src;
        }
      }
      f.nodes = std::move(out);
      for (Value& v : f.values) v.def = -1;
      for (size_t i = 0; i < f.nodes.size(); ++i)
        for (size_t k = 0; k < f.nodes[i].out.size(); ++k) {
          f.values[f.nodes[i].out[k]].def = (int)i;
          f.values[f.nodes[i].out[k]].def_result = (int)k;
        }
      if (!any) break;
    }
  }
}

RewriteStats rewrite(Function& f) {
  RewriteStats st;
  Ctx c(f);
  rewrite_custom_calls(c, st);
  // Attention first: its softmax must not be claimed by the softmax gate.
  rewrite_sdpa(c, st);
  compact(f);
  Ctx c2(f);
  rewrite_norms(c2, st);
  compact(f);
  Ctx c3(f);
  fold_rms_into_sdpa(c3);
  rewrite_softmax(c3, st);
  rewrite_log_softmax(c3, st);
  rewrite_sigmoid(c3, st);
  compact(f);
  return st;
}

std::string to_json(const Function& f, const RewriteStats* stats) {
  std::ostringstream o;
  auto q = [](const std::string& s) {
    std::string r = "\"";
    for (char ch : s) {
      if (ch == '"' || ch == '\\') r += '\\';
      if (ch == '\n') {
        r += "\\n";
        continue;
      }
      r += ch;
    }
    return r + "\"";
  };
  o << "{\"function\": " << q(f.name) << ", \"params\": [";
  for (size_t i = 0; i < f.params.size(); ++i)
    o << (i ? ", " : "") << q(f.values[f.params[i]].type.str());
  o << "], \"results\": [";
  for (size_t i = 0; i < f.results.size(); ++i)
    o << (i ? ", " : "") << q(f.values[f.results[i]].type.str());
  o << "], \"nodes\": [";
  bool first = true;
  for (const Node& n : f.nodes) {
    if (n.dead) continue;
    o << (first ? "" : ", ") << "{\"op\": " << q(n.op) << ", \"in\": [";
    first = false;
    for (size_t i = 0; i < n.in.size(); ++i) o << (i ? ", " : "") << n.in[i];
    o << "], \"out\": [";
    for (size_t i = 0; i < n.out.size(); ++i) o << (i ? ", " : "") << n.out[i];
    o << "], \"out_types\": [";
    for (size_t i = 0; i < n.out.size(); ++i) o << (i ? ", " : "") << q(f.values[n.out[i]].type.str());
    o << "]";
    for (auto& kv : n.ints) {
      o << ", " << q("i:" + kv.first) << ": [";
      for (size_t i = 0; i < kv.second.size(); ++i) o << (i ? ", " : "") << kv.second[i];
      o << "]";
    }
    for (auto& kv : n.nums) {
      char buf[64];
      std::snprintf(buf, sizeof buf, "%.9g", kv.second);
      std::string num = buf;
      if (num == "inf") num = "1e999";
      if (num == "-inf") num = "-1e999";
      if (num == "nan") num = "null";
      o << ", " << q("f:" + kv.first) << ": " << num;
    }
    for (auto& kv : n.strs) o << ", " << q("s:" + kv.first) << ": " << q(kv.second);
    o << "}";
  }
  o << "]";
  if (stats)
    o << ", \"rewrites\": {\"sdpa\": " << stats->sdpa << ", \"layer_norm\": " << stats->layer_norm
      << ", \"rms_norm\": " << stats->rms_norm << ", \"softmax\": " << stats->softmax
      << ", \"log_softmax\": " << stats->log_softmax << ", \"sigmoid\": " << stats->sigmoid
      << ", \"custom_calls\": " << stats->custom_calls << ", \"affine_absorbed\": " << stats->affine_absorbed
      << "}";
  o << "}";
  return o.str();
}

}  // namespace mfxp
