"""StableHLO text modules for the fused-path configurations, written in the
forms jax.jit(...).lower(...).as_text() produces for them.

No jax is installed in this environment (or on the GPU boxes), so the modules
the PJRT plugin is tested with are generated here, op for op in the shapes
JAX's lowering uses:
  * jnp.mean / jnp.var lower to reduce(add) / divide-by-n with keepdims
    broadcast_in_dim; jax.nn.softmax is a jitted helper (func.call @softmax)
    with reduce(max) init -inf, maximum(-inf, .), exp, reduce(add), divide;
  * einsum lowers to dot_general with batching / contracting dims (results
    ordered batch, lhs free, rhs free) plus a transpose where the einsum's
    output order differs;
  * jax.nn.dot_product_attention (xla implementation) reshapes q to
    [B, T, K, G, H], computes 'BTKGH,BSKH->BKGTS' in fp32, scales, masks with
    jnp.where(mask, logits, -0.7 * finfo.max) where the causal mask is
    jnp.tril(ones) built from iota / compare GE, softmaxes, casts to the value
    dtype and computes 'BKGTS,BSKH->BTKGH' before reshaping to [B, T, N, H];
  * the reference's custom_call targets carry {"scale": s} / {"eps": e}
    backend_config JSON (reference src/jax_mlx/sdpa.py:105,
    src/jax_mlx/layer_norm.py:93).
"""
from __future__ import annotations

import math
import struct


def ty(shape, dt):
    if not shape:
        return f"tensor<{dt}>"
    return "tensor<" + "x".join(str(int(s)) for s in shape) + f"x{dt}>"


def f32_lit(x: float, dt: str = "f32") -> str:
    if math.isinf(x):
        bits = {"f32": 0xFF800000 if x < 0 else 0x7F800000, "bf16": 0xFF80 if x < 0 else 0x7F80,
                "f16": 0xFC00 if x < 0 else 0x7C00}[dt]
        width = 8 if dt == "f32" else 4
        return f"0x{bits:0{width}X}"
    return f"{x:.8E}"


class Fn:
    """Accumulates the body of one func.func."""

    def __init__(self, name: str, args, results=None, public=True):
        self.name = name
        self.args = args  # list of (shape, dtype)
        self.lines = []
        self.n = 0
        self.public = public

    def arg(self, i):
        return f"%arg{i}"

    def new(self):
        v = f"%{self.n}"
        self.n += 1
        return v

    def emit(self, rhs: str) -> str:
        v = self.new()
        self.lines.append(f"    {v} = {rhs}")
        return v

    # ---- op helpers (pretty syntax) ----
    def const(self, x, shape=(), dt="f32"):
        lit = "true" if x is True else "false" if x is False else (
            str(int(x)) if dt.startswith("i") or dt.startswith("ui") else f32_lit(float(x), dt))
        return self.emit(f"stablehlo.constant dense<{lit}> : {ty(shape, dt)}")

    def bcast(self, v, src_shape, dims, shape, dt):
        d = ", ".join(str(x) for x in dims)
        return self.emit(f"stablehlo.broadcast_in_dim {v}, dims = [{d}] : ({ty(src_shape, dt)}) -> {ty(shape, dt)}")

    def splat(self, x, shape, dt="f32"):
        c = self.const(x, (), dt)
        return self.bcast(c, (), [], shape, dt)

    def binary(self, op, a, b, shape, dt):
        return self.emit(f"stablehlo.{op} {a}, {b} : {ty(shape, dt)}")

    def unary(self, op, a, shape, dt):
        return self.emit(f"stablehlo.{op} {a} : {ty(shape, dt)}")

    def convert(self, a, shape, src, dst):
        return self.emit(f"stablehlo.convert {a} : ({ty(shape, src)}) -> {ty(shape, dst)}")

    def reshape(self, a, src_shape, shape, dt):
        return self.emit(f"stablehlo.reshape {a} : ({ty(src_shape, dt)}) -> {ty(shape, dt)}")

    def transpose(self, a, src_shape, perm, dt):
        shape = [src_shape[p] for p in perm]
        d = ", ".join(str(p) for p in perm)
        return self.emit(f"stablehlo.transpose {a}, dims = [{d}] : ({ty(src_shape, dt)}) -> {ty(shape, dt)}"), shape

    def reduce(self, a, shape, dims, kind, dt):
        init = self.const(0.0 if kind == "add" else -math.inf, (), dt)
        out = [s for i, s in enumerate(shape) if i not in dims]
        d = ", ".join(str(x) for x in dims)
        return self.emit(f"stablehlo.reduce({a} init: {init}) applies stablehlo.{kind} across dimensions = [{d}] : "
                         f"({ty(shape, dt)}, {ty((), dt)}) -> {ty(out, dt)}"), out

    def dot_general(self, a, b, ashape, bshape, batch, contract, dt, out_dt=None):
        out_dt = out_dt or dt
        ab, bb = batch
        ac, bc = contract
        afree = [i for i in range(len(ashape)) if i not in ab and i not in ac]
        bfree = [i for i in range(len(bshape)) if i not in bb and i not in bc]
        out = [ashape[i] for i in ab] + [ashape[i] for i in afree] + [bshape[i] for i in bfree]
        parts = []
        if ab:
            parts.append(f"batching_dims = [{', '.join(map(str, ab))}] x [{', '.join(map(str, bb))}]")
        parts.append(f"contracting_dims = [{', '.join(map(str, ac))}] x [{', '.join(map(str, bc))}]")
        parts.append("precision = [DEFAULT, DEFAULT]")
        return self.emit(f"stablehlo.dot_general {a}, {b}, {', '.join(parts)} : "
                         f"({ty(ashape, dt)}, {ty(bshape, dt)}) -> {ty(out, out_dt)}"), out

    def call(self, name, args, in_types, out_type):
        return self.emit(f"func.call @{name}({', '.join(args)}) : ({', '.join(in_types)}) -> {out_type}")

    def text(self, ret_vals, ret_types):
        vis = "public" if self.public else "private"
        args = ", ".join(f"%arg{i}: {ty(s, d)}" for i, (s, d) in enumerate(self.args))
        rt = ", ".join(f"{t}" + (' {jax.result_info = "result"}' if self.public else "") for t in ret_types)
        if self.public:
            rt = f"({rt})"
        elif len(ret_types) > 1:
            rt = f"({rt})"
        body = "\n".join(self.lines)
        rv = ", ".join(ret_vals)
        rts = ", ".join(ret_types)
        return f"  func.func {vis} @{self.name}({args}) -> {rt} {{\n{body}\n    return {rv} : {rts}\n  }}"


def module(name: str, funcs) -> str:
    return (f"module @{name} attributes {{mhlo.num_partitions = 1 : i32, mhlo.num_replicas = 1 : i32}} {{\n"
            + "\n".join(funcs) + "\n}\n")


def softmax_fn(shape, dt="f32", name="softmax"):
    """jax.nn.softmax(x, axis=-1) as the private function JAX emits."""
    f = Fn(name, [(shape, dt)], public=False)
    x = f.arg(0)
    r = len(shape) - 1
    m, mshape = f.reduce(x, shape, [r], "maximum", dt)
    ninf = f.splat(-math.inf, mshape, dt)
    m = f.binary("maximum", ninf, m, mshape, dt)
    kshape = list(mshape) + [1]
    m = f.bcast(m, mshape, list(range(r)), kshape, dt)
    m = f.bcast(m, kshape, list(range(r + 1)), shape, dt)
    e = f.unary("exponential", f.binary("subtract", x, m, shape, dt), shape, dt)
    s, sshape = f.reduce(e, shape, [r], "add", dt)
    s = f.bcast(s, sshape, list(range(r)), kshape, dt)
    s = f.bcast(s, kshape, list(range(r + 1)), shape, dt)
    out = f.binary("divide", e, s, shape, dt)
    return f.text([out], [ty(shape, dt)])


def _mean_keepdims(f, x, shape, dt):
    r = len(shape) - 1
    s, sshape = f.reduce(x, shape, [r], "add", dt)
    kshape = list(sshape) + [1]
    s = f.bcast(s, sshape, list(range(r)), kshape, dt)
    n = f.splat(float(shape[-1]), kshape, dt)
    return f.binary("divide", s, n, kshape, dt), kshape


# ---------------------------------------------------------------- norms

def layer_norm_module(shape=(8, 128, 512), eps=1e-5, dt="f32", form="var", affine=True):
    """form "var": (x - mean) / sqrt(var + eps) * w + b with jnp.var
    (src/jax_mlx/layer_norm.py:20-25); "standardize": jax.nn.standardize's
    mean(x^2) - mean^2 then (x - mean) * rsqrt(var + eps); "flax": Flax
    LayerNorm, x upcast to f32 for the statistics, scale folded into the
    rsqrt multiplier, result cast back."""
    shape = list(shape)
    C = shape[-1]
    args = [(shape, dt)] + ([([C], dt), ([C], dt)] if affine else [])
    f = Fn("main", args)
    x = f.arg(0)
    cdt = "f32" if form == "flax" else dt
    if cdt != dt:
        x = f.convert(x, shape, dt, cdt)
    r = len(shape) - 1
    mean, kshape = _mean_keepdims(f, x, shape, cdt)
    if form == "var":
        m2, _ = _mean_keepdims(f, x, shape, cdt)
        cen = f.binary("subtract", x, f.bcast(m2, kshape, list(range(r + 1)), shape, cdt), shape, cdt)
        sq = f.binary("multiply", cen, cen, shape, cdt)
        var, _ = _mean_keepdims(f, sq, shape, cdt)
    else:
        sq = f.binary("multiply", x, x, shape, cdt)
        ex2, _ = _mean_keepdims(f, sq, shape, cdt)
        msq = f.binary("multiply", mean, mean, kshape, cdt)
        var = f.binary("subtract", ex2, msq, kshape, cdt)
        if form == "flax":
            var = f.binary("maximum", f.splat(0.0, kshape, cdt), var, kshape, cdt)
    xc = f.binary("subtract", x, f.bcast(mean, kshape, list(range(r + 1)), shape, cdt), shape, cdt)
    ve = f.binary("add", var, f.splat(eps, kshape, cdt), kshape, cdt)
    if form == "var":
        den = f.bcast(f.unary("sqrt", ve, kshape, cdt), kshape, list(range(r + 1)), shape, cdt)
        y = f.binary("divide", xc, den, shape, cdt)
        if affine:
            y = f.binary("multiply", y, f.bcast(f.arg(1), [C], [r], shape, cdt), shape, cdt)
            y = f.binary("add", y, f.bcast(f.arg(2), [C], [r], shape, cdt), shape, cdt)
    elif form == "standardize":
        mul = f.bcast(f.unary("rsqrt", ve, kshape, cdt), kshape, list(range(r + 1)), shape, cdt)
        y = f.binary("multiply", xc, mul, shape, cdt)
        if affine:
            y = f.binary("multiply", y, f.bcast(f.arg(1), [C], [r], shape, cdt), shape, cdt)
            y = f.binary("add", y, f.bcast(f.arg(2), [C], [r], shape, cdt), shape, cdt)
    else:  # flax
        mul = f.bcast(f.unary("rsqrt", ve, kshape, cdt), kshape, list(range(r + 1)), shape, cdt)
        if affine:
            sc = f.arg(1)
            if dt != cdt:
                sc = f.convert(sc, [C], dt, cdt)
            scb = f.bcast(f.reshape(sc, [C], [1] * r + [C], cdt), [1] * r + [C], list(range(r + 1)), shape, cdt)
            mul = f.binary("multiply", mul, scb, shape, cdt)
        y = f.binary("multiply", xc, mul, shape, cdt)
        if affine:
            bi = f.arg(2)
            if dt != cdt:
                bi = f.convert(bi, [C], dt, cdt)
            bib = f.bcast(f.reshape(bi, [C], [1] * r + [C], cdt), [1] * r + [C], list(range(r + 1)), shape, cdt)
            y = f.binary("add", y, bib, shape, cdt)
        if dt != cdt:
            y = f.convert(y, shape, cdt, dt)
    return module("jit_layer_norm", [f.text([y], [ty(shape, dt)])])


def layer_norm_escape_module(shape=(64, 512), eps=1e-5, dt="f32"):
    """The "var" LayerNorm with its mean and variance also returned (as
    [..., 1]): intermediates of the matched pattern that escape it."""
    shape = list(shape)
    C = shape[-1]
    f = Fn("main", [(shape, dt), ([C], dt), ([C], dt)])
    x = f.arg(0)
    r = len(shape) - 1
    mean, kshape = _mean_keepdims(f, x, shape, dt)
    cen = f.binary("subtract", x, f.bcast(mean, kshape, list(range(r + 1)), shape, dt), shape, dt)
    var, _ = _mean_keepdims(f, f.binary("multiply", cen, cen, shape, dt), shape, dt)
    ve = f.binary("add", var, f.splat(eps, kshape, dt), kshape, dt)
    den = f.bcast(f.unary("sqrt", ve, kshape, dt), kshape, list(range(r + 1)), shape, dt)
    y = f.binary("divide", cen, den, shape, dt)
    y = f.binary("multiply", y, f.bcast(f.arg(1), [C], [r], shape, dt), shape, dt)
    y = f.binary("add", y, f.bcast(f.arg(2), [C], [r], shape, dt), shape, dt)
    return module("jit_layer_norm_stats", [f.text([y, mean, var], [ty(shape, dt), ty(kshape, dt), ty(kshape, dt)])])


def rms_norm_module(shape=(2, 4, 128), eps=1e-6, dt="f32", weight=True, upcast=False):
    shape = list(shape)
    C = shape[-1]
    args = [(shape, dt)] + ([([C], dt)] if weight else [])
    f = Fn("main", args)
    x = f.arg(0)
    cdt = "f32" if upcast else dt
    if upcast:
        x = f.convert(x, shape, dt, cdt)
    r = len(shape) - 1
    ms, kshape = _mean_keepdims(f, f.binary("multiply", x, x, shape, cdt), shape, cdt)
    inv = f.unary("rsqrt", f.binary("add", ms, f.splat(eps, kshape, cdt), kshape, cdt), kshape, cdt)
    y = f.binary("multiply", x, f.bcast(inv, kshape, list(range(r + 1)), shape, cdt), shape, cdt)
    if upcast:
        y = f.convert(y, shape, cdt, dt)
    if weight:
        y = f.binary("multiply", y, f.bcast(f.arg(1), [C], [r], shape, dt), shape, dt)
    return module("jit_rms_norm", [f.text([y], [ty(shape, dt)])])


def softmax_module(shape=(6, 64), dt="f32"):
    shape = list(shape)
    f = Fn("main", [(shape, dt)])
    y = f.call("softmax", [f.arg(0)], [ty(shape, dt)], ty(shape, dt))
    return module("jit_softmax", [f.text([y], [ty(shape, dt)]), softmax_fn(shape, dt)])


def log_softmax_fn(shape, dt="f32", name="log_softmax"):
    """jax.nn.log_softmax(x, axis=-1) as the private function JAX emits:
    x_max = max(x, initial=-inf, keepdims); shifted = x - x_max;
    shifted - log(sum(exp(shifted), keepdims))."""
    f = Fn(name, [(shape, dt)], public=False)
    x = f.arg(0)
    r = len(shape) - 1
    m, mshape = f.reduce(x, shape, [r], "maximum", dt)
    m = f.binary("maximum", f.splat(-math.inf, mshape, dt), m, mshape, dt)
    kshape = list(mshape) + [1]
    m = f.bcast(m, mshape, list(range(r)), kshape, dt)
    shifted = f.binary("subtract", x, f.bcast(m, kshape, list(range(r + 1)), shape, dt), shape, dt)
    e = f.unary("exponential", shifted, shape, dt)
    s, sshape = f.reduce(e, shape, [r], "add", dt)
    s = f.bcast(s, sshape, list(range(r)), kshape, dt)
    lg = f.unary("log", s, kshape, dt)
    out = f.binary("subtract", shifted, f.bcast(lg, kshape, list(range(r + 1)), shape, dt), shape, dt)
    return f.text([out], [ty(shape, dt)])


def log_softmax_module(shape=(6, 64), dt="f32"):
    shape = list(shape)
    f = Fn("main", [(shape, dt)])
    y = f.call("log_softmax", [f.arg(0)], [ty(shape, dt)], ty(shape, dt))
    return module("jit_log_softmax", [f.text([y], [ty(shape, dt)]), log_softmax_fn(shape, dt)])


def sigmoid_silu_module(shape=(16, 256), dt="f32"):
    """Two results: the divide form of the sigmoid the reference matches
    (1 / (1 + exp(-x)), src/jax_mlx_pjrt.cpp:2046-2164) and jax.nn.silu as a
    private @silu function (x * logistic(x))."""
    shape = list(shape)
    f = Fn("main", [(shape, dt)])
    x = f.arg(0)
    den = f.binary("add", f.splat(1.0, shape, dt), f.unary("exponential", f.unary("negate", x, shape, dt), shape, dt),
                   shape, dt)
    sig = f.binary("divide", f.splat(1.0, shape, dt), den, shape, dt)
    si = f.call("silu", [x], [ty(shape, dt)], ty(shape, dt))
    g = Fn("silu", [(shape, dt)], public=False)
    y = g.binary("multiply", g.arg(0), g.unary("logistic", g.arg(0), shape, dt), shape, dt)
    return module("jit_sigmoid_silu", [f.text([sig, si], [ty(shape, dt), ty(shape, dt)]),
                                       g.text([y], [ty(shape, dt)])])


# ---------------------------------------------------------------- attention

def _causal_pred(f, T, S):
    """jnp.tril(jnp.ones((T, S), bool)) as JAX lowers it: iota / add k /
    compare GE / select between broadcast true and false."""
    i0 = f.emit(f"stablehlo.iota dim = 0 : {ty([T, S], 'i32')}")
    k = f.splat(0, [T, S], "i32")
    i0 = f.binary("add", i0, k, [T, S], "i32")
    i1 = f.emit(f"stablehlo.iota dim = 1 : {ty([T, S], 'i32')}")
    tri = f.emit(f"stablehlo.compare  GE, {i0}, {i1},  SIGNED : ({ty([T, S], 'i32')}, {ty([T, S], 'i32')}) -> "
                 f"{ty([T, S], 'i1')}")
    t = f.splat(True, [T, S], "i1")
    fl = f.splat(False, [T, S], "i1")
    return f.emit(f"stablehlo.select {tri}, {t}, {fl} : {ty([T, S], 'i1')}, {ty([T, S], 'i1')}")


def sdpa_bhtd_module(B=8, H=8, T=128, S=None, D=64, dt="f32", causal=False, scale=None, mask_value=None,
                     transposed_k=False, inline_softmax=False, return_probs=False):
    """softmax(einsum('bhtd,bhsd->bhts', q, k) * scale [masked]) @ v in BHTD.
    transposed_k: k passed as [B, H, D, S] and used through a transpose.
    return_probs: the softmax probabilities are a second result."""
    S = S or T
    scale = scale if scale is not None else 1.0 / math.sqrt(D)
    kshape = [B, H, D, S] if transposed_k else [B, H, S, D]
    f = Fn("main", [([B, H, T, D], dt), (kshape, dt), ([B, H, S, D], dt)])
    acc = "f32"
    k = f.arg(1)
    if transposed_k:
        k, _ = f.transpose(k, kshape, [0, 1, 3, 2], dt)
    s, sshape = f.dot_general(f.arg(0), k, [B, H, T, D], [B, H, S, D], ([0, 1], [0, 1]), ([3], [3]), dt, acc)
    s = f.binary("multiply", s, f.splat(scale, sshape, acc), sshape, acc)
    if causal:
        pred = _causal_pred(f, T, S)
        pb = f.bcast(pred, [T, S], [2, 3], sshape, "i1")
        neg = mask_value if mask_value is not None else -math.inf
        s = f.emit(f"stablehlo.select {pb}, {s}, {f.splat(neg, sshape, acc)} : {ty(sshape, 'i1')}, {ty(sshape, acc)}")
    funcs = []
    if inline_softmax:
        # softmax body inlined in main (no func.call)
        r = 3
        m, mshape = f.reduce(s, sshape, [r], "maximum", acc)
        m = f.bcast(m, mshape, [0, 1, 2], sshape, acc)
        e = f.unary("exponential", f.binary("subtract", s, m, sshape, acc), sshape, acc)
        z, zshape = f.reduce(e, sshape, [r], "add", acc)
        p = f.binary("divide", e, f.bcast(z, zshape, [0, 1, 2], sshape, acc), sshape, acc)
    else:
        p = f.call("softmax", [s], [ty(sshape, acc)], ty(sshape, acc))
        funcs.append(softmax_fn(sshape, acc))
    probs = p
    if dt != acc:
        p = f.convert(p, sshape, acc, dt)
    o, oshape = f.dot_general(p, f.arg(2), sshape, [B, H, S, D], ([0, 1], [0, 1]), ([3], [2]), dt)
    if return_probs:
        return module("jit_attention", [f.text([o, probs], [ty(oshape, dt), ty(sshape, acc)])] + funcs)
    return module("jit_attention", [f.text([o], [ty(oshape, dt)])] + funcs)


def dot_product_attention_module(B=4, T=2048, N=32, K=None, H=128, S=None, dt="bf16", is_causal=True, bias=False):
    """jax.nn.dot_product_attention(q, k, v, bias=..., is_causal=...) with the
    xla implementation, q [B, T, N, H], k/v [B, S, K, H] (BTNH)."""
    K = K or N
    S = S or T
    G = N // K
    args = [([B, T, N, H], dt), ([B, S, K, H], dt), ([B, S, K, H], dt)]
    if bias:
        args.append(([B, 1, 1, S], "f32"))
    f = Fn("main", args)
    acc = "f32"
    q = f.reshape(f.arg(0), [B, T, N, H], [B, T, K, G, H], dt)
    s, sshape = f.dot_general(q, f.arg(1), [B, T, K, G, H], [B, S, K, H], ([0, 2], [0, 2]), ([4], [3]), dt, acc)
    # dot result [B, K, T, G, S] -> 'BKGTS'
    s, sshape = f.transpose(s, sshape, [0, 1, 3, 2, 4], acc)
    scale = 1.0 / math.sqrt(H)
    s = f.binary("multiply", s, f.splat(scale, sshape, acc), sshape, acc)
    if bias:
        bb = f.reshape(f.arg(3), [B, 1, 1, S], [B, 1, 1, 1, S], "f32")
        bb = f.bcast(bb, [B, 1, 1, 1, S], [0, 1, 2, 3, 4], sshape, "f32")
        s = f.binary("add", s, bb, sshape, acc)
    if is_causal:
        pred = _causal_pred(f, T, S)
        p5 = f.reshape(pred, [T, S], [1, 1, 1, T, S], "i1")
        p5 = f.bcast(p5, [1, 1, 1, T, S], [0, 1, 2, 3, 4], sshape, "i1")
        ones = f.splat(True, sshape, "i1")
        comb = f.binary("and", ones, p5, sshape, "i1")
        neg = -0.7 * 3.4028234663852886e38
        s = f.emit(f"stablehlo.select {comb}, {s}, {f.splat(neg, sshape, acc)} : {ty(sshape, 'i1')}, {ty(sshape, acc)}")
    p = f.call("softmax", [s], [ty(sshape, acc)], ty(sshape, acc))
    p = f.convert(p, sshape, acc, dt)
    o, oshape = f.dot_general(p, f.arg(2), sshape, [B, S, K, H], ([0, 1], [0, 2]), ([4], [1]), dt)
    # [B, K, G, T, H] -> 'BTKGH' -> [B, T, N, H]
    o, oshape = f.transpose(o, oshape, [0, 3, 1, 2, 4], dt)
    o = f.reshape(o, oshape, [B, T, N, H], dt)
    return module("jit_dot_product_attention",
                  [f.text([o], [ty([B, T, N, H], dt)]), softmax_fn(sshape, acc)])


def gqa_decode_module(B=16, Hq=32, Hkv=8, S=8192, D=128, eps=1e-6, dt="bf16", Tq=1):
    """RMSNorm(q) (f32 statistics, cast back) then grouped attention with an
    additive padding mask: q [B, Hq, Tq, D], k/v [B, Hkv, S, D], mask
    [B, 1, 1, S]."""
    G = Hq // Hkv
    f = Fn("main", [([B, Hq, Tq, D], dt), ([B, Hkv, S, D], dt), ([B, Hkv, S, D], dt), ([B, 1, 1, S], "f32")])
    qshape = [B, Hq, Tq, D]
    qf = f.convert(f.arg(0), qshape, dt, "f32")
    ms, kshape = _mean_keepdims(f, f.binary("multiply", qf, qf, qshape, "f32"), qshape, "f32")
    inv = f.unary("rsqrt", f.binary("add", ms, f.splat(eps, kshape, "f32"), kshape, "f32"), kshape, "f32")
    qn = f.binary("multiply", qf, f.bcast(inv, kshape, [0, 1, 2, 3], qshape, "f32"), qshape, "f32")
    qn = f.convert(qn, qshape, "f32", dt)
    qg = f.reshape(qn, qshape, [B, Hkv, G, Tq, D], dt)
    s, sshape = f.dot_general(qg, f.arg(1), [B, Hkv, G, Tq, D], [B, Hkv, S, D], ([0, 1], [0, 1]), ([4], [3]), dt,
                              "f32")
    s = f.binary("multiply", s, f.splat(1.0 / math.sqrt(D), sshape, "f32"), sshape, "f32")
    mb = f.reshape(f.arg(3), [B, 1, 1, S], [B, 1, 1, 1, S], "f32")
    mb = f.bcast(mb, [B, 1, 1, 1, S], [0, 1, 2, 3, 4], sshape, "f32")
    s = f.binary("add", s, mb, sshape, "f32")
    p = f.call("softmax", [s], [ty(sshape, "f32")], ty(sshape, "f32"))
    p = f.convert(p, sshape, "f32", dt)
    o, oshape = f.dot_general(p, f.arg(2), sshape, [B, Hkv, S, D], ([0, 1], [0, 1]), ([4], [2]), dt)
    o = f.reshape(o, oshape, [B, Hq, Tq, D], dt)
    return module("jit_gqa_decode", [f.text([o], [ty([B, Hq, Tq, D], dt)]), softmax_fn(sshape, "f32")])


def custom_call_sdpa_module(B=2, T=64, N=4, K=None, H=64, S=None, dt="f32", scale=0.125):
    """custom_call @mlx_sdpa as emitted by the reference's lowering
    (src/jax_mlx/sdpa.py:97-112): BTNH operands, {"scale": s}."""
    K = K or N
    S = S or T
    f = Fn("main", [([B, T, N, H], dt), ([B, S, K, H], dt), ([B, S, K, H], dt)])
    cfg = '{\\22scale\\22: ' + repr(float(scale)) + '}'
    o = f.emit(f'stablehlo.custom_call @mlx_sdpa(%arg0, %arg1, %arg2) {{backend_config = "{cfg}"}} : '
               f"({ty([B, T, N, H], dt)}, {ty([B, S, K, H], dt)}, {ty([B, S, K, H], dt)}) -> {ty([B, T, N, H], dt)}")
    return module("jit_mlx_sdpa", [f.text([o], [ty([B, T, N, H], dt)])])


def custom_call_layer_norm_module(shape=(4, 512), eps=1e-5, dt="f32"):
    """custom_call @mlx_layer_norm (src/jax_mlx/layer_norm.py:86-100)."""
    shape = list(shape)
    C = shape[-1]
    f = Fn("main", [(shape, dt), ([C], dt), ([C], dt)])
    cfg = '{\\22eps\\22: ' + repr(float(eps)) + '}'
    o = f.emit(f'stablehlo.custom_call @mlx_layer_norm(%arg0, %arg1, %arg2) {{backend_config = "{cfg}"}} : '
               f"({ty(shape, dt)}, {ty([C], dt)}, {ty([C], dt)}) -> {ty(shape, dt)}")
    return module("jit_mlx_layer_norm", [f.text([o], [ty(shape, dt)])])


def custom_call_sdpa_bwd_module(B=2, T=64, N=4, K=None, H=64, S=None, dt="f32", scale=0.125):
    """custom_call @mlx_sdpa_bwd as emitted by the reference's lowering
    (src/jax_mlx/sdpa.py:114-130): BTNH (q, k, v, grad_out) -> (dq, dk, dv)."""
    K = K or N
    S = S or T
    qt, kt = ty([B, T, N, H], dt), ty([B, S, K, H], dt)
    f = Fn("main", [([B, T, N, H], dt), ([B, S, K, H], dt), ([B, S, K, H], dt), ([B, T, N, H], dt)])
    cfg = '{\\22scale\\22: ' + repr(float(scale)) + '}'
    r = f.new()
    f.lines.append(f'    {r}:3 = stablehlo.custom_call @mlx_sdpa_bwd(%arg0, %arg1, %arg2, %arg3) '
                   f'{{backend_config = "{cfg}"}} : ({qt}, {kt}, {kt}, {qt}) -> ({qt}, {kt}, {kt})')
    return module("jit_mlx_sdpa_bwd", [f.text([f"{r}#0", f"{r}#1", f"{r}#2"], [qt, kt, kt])])


def sdpa_vjp_module(B=2, T=64, N=4, K=None, H=64, S=None, dt="f32", scale=0.125, same_inputs=True,
                    cotangents=1):
    """jax.vjp of the reference's mlx_dot_product_attention (custom_vjp:
    src/jax_mlx/sdpa.py:156-191) inside one jit: custom_call @mlx_sdpa on
    (q, k, v), then @mlx_sdpa_bwd on the saved (q, k, v) and the cotangent
    g.  Results: the attention output and (dq, dk, dv).  same_inputs=False
    feeds the backward q + 0 from a separate argument instead (a different
    q value).  cotangents=2 applies the VJP to a second cotangent (the last
    argument) as well, appending its (dq, dk, dv): two backward steps of one
    forward, as a Jacobian makes."""
    K = K or N
    S = S or T
    qt, kt = ty([B, T, N, H], dt), ty([B, S, K, H], dt)
    args = [([B, T, N, H], dt), ([B, S, K, H], dt), ([B, S, K, H], dt), ([B, T, N, H], dt)]
    if not same_inputs:
        args.append(([B, T, N, H], dt))
    if cotangents == 2:
        args.append(([B, T, N, H], dt))
    f = Fn("main", args)
    cfg = '{\\22scale\\22: ' + repr(float(scale)) + '}'
    o = f.emit(f'stablehlo.custom_call @mlx_sdpa(%arg0, %arg1, %arg2) {{backend_config = "{cfg}"}} : '
               f"({qt}, {kt}, {kt}) -> {qt}")
    qb = "%arg0" if same_inputs else "%arg4"
    res, rts = [o], [qt]
    for c in range(cotangents):
        g = "%arg3" if c == 0 else f"%arg{len(args) - 1}"
        r = f.new()
        f.lines.append(f'    {r}:3 = stablehlo.custom_call @mlx_sdpa_bwd({qb}, %arg1, %arg2, {g}) '
                       f'{{backend_config = "{cfg}"}} : ({qt}, {kt}, {kt}, {qt}) -> ({qt}, {kt}, {kt})')
        res += [f"{r}#0", f"{r}#1", f"{r}#2"]
        rts += [qt, kt, kt]
    return module("jit_mlx_sdpa_vjp", [f.text(res, rts)])


def custom_call_layer_norm_bwd_module(shape=(4, 512), eps=1e-5, dt="f32", pdt=None):
    """custom_call @mlx_layer_norm_bwd (src/jax_mlx/layer_norm.py:102-116):
    (x, weight, bias, grad_out) -> (dx, dweight, dbias)."""
    shape = list(shape)
    pdt = pdt or dt
    C = shape[-1]
    f = Fn("main", [(shape, dt), ([C], pdt), ([C], pdt), (shape, dt)])
    cfg = '{\\22eps\\22: ' + repr(float(eps)) + '}'
    rts = [ty(shape, dt), ty([C], pdt), ty([C], pdt)]
    r = f.new()
    f.lines.append(f'    {r}:3 = stablehlo.custom_call @mlx_layer_norm_bwd(%arg0, %arg1, %arg2, %arg3) '
                   f'{{backend_config = "{cfg}"}} : ({ty(shape, dt)}, {ty([C], pdt)}, {ty([C], pdt)}, '
                   f'{ty(shape, dt)}) -> ({", ".join(rts)})')
    return module("jit_mlx_layer_norm_bwd", [f.text([f"{r}#0", f"{r}#1", f"{r}#2"], rts)])


# ---------------------------------------------------------------- transformer

def elementwise_mix_module(R=64, C=256, dt="f32"):
    """A generic-op region the fused kernels do not cover: bias add through a
    broadcast, the tanh GELU, a product with a transposed operand, and an
    iota / compare / select lower-triangle mask -- one elementwise program."""
    f = Fn("main", [([R, C], dt), ([C], dt), ([C, R], dt)])
    shape = [R, C]
    u = f.binary("add", f.arg(0), f.bcast(f.arg(1), [C], [1], shape, dt), shape, dt)
    u3 = f.binary("multiply", f.binary("multiply", u, u, shape, dt), u, shape, dt)
    inner = f.binary("add", u, f.binary("multiply", f.splat(0.044715, shape, dt), u3, shape, dt), shape, dt)
    inner = f.binary("multiply", f.splat(math.sqrt(2 / math.pi), shape, dt), inner, shape, dt)
    t = f.binary("add", f.splat(1.0, shape, dt), f.unary("tanh", inner, shape, dt), shape, dt)
    g = f.binary("multiply", f.binary("multiply", f.splat(0.5, shape, dt), u, shape, dt), t, shape, dt)
    at, _ = f.transpose(f.arg(2), [C, R], [1, 0], dt)
    y = f.binary("multiply", g, at, shape, dt)
    i0 = f.emit(f"stablehlo.iota dim = 0 : {ty(shape, 'i32')}")
    i1 = f.emit(f"stablehlo.iota dim = 1 : {ty(shape, 'i32')}")
    tri = f.emit(f"stablehlo.compare  GE, {i0}, {i1},  SIGNED : ({ty(shape, 'i32')}, {ty(shape, 'i32')}) -> "
                 f"{ty(shape, 'i1')}")
    o = f.emit(f"stablehlo.select {tri}, {y}, {f.splat(-1.0, shape, dt)} : {ty(shape, 'i1')}, {ty(shape, dt)}")
    return module("jit_elementwise_mix", [f.text([o], [ty(shape, dt)])])


def transformer_module(layers=4, B=32, T=256, d=512, heads=8, mlp=2048, eps=1e-5, dt="f32", causal=False):
    """Pre-LN transformer forward (Flax-style modules under jax.jit):
    x + Attn(LN(x)); x + MLP(LN(x)) with a fused QKV projection split by
    slices, dot_product_attention-style heads, GELU (tanh approximation,
    jax.nn.gelu's default) in the MLP.  Parameters per layer, in order:
    ln1 scale/bias [d], w_qkv [d, 3d], b_qkv [3d], w_o [d, d], b_o [d],
    ln2 scale/bias [d], w1 [d, mlp], b1 [mlp], w2 [mlp, d], b2 [d]."""
    hd = d // heads
    args = [([B, T, d], dt)]
    for _ in range(layers):
        args += [([d], dt), ([d], dt), ([d, 3 * d], dt), ([3 * d], dt), ([d, d], dt), ([d], dt),
                 ([d], dt), ([d], dt), ([d, mlp], dt), ([mlp], dt), ([mlp, d], dt), ([d], dt)]
    f = Fn("main", args)
    x = f.arg(0)
    xs = [B, T, d]
    ai = 1

    def ln(v, g, b):
        mean, kshape = _mean_keepdims(f, v, xs, dt)
        m2, _ = _mean_keepdims(f, v, xs, dt)
        cen = f.binary("subtract", v, f.bcast(m2, kshape, [0, 1, 2], xs, dt), xs, dt)
        var, _ = _mean_keepdims(f, f.binary("multiply", cen, cen, xs, dt), xs, dt)
        xc = f.binary("subtract", v, f.bcast(mean, kshape, [0, 1, 2], xs, dt), xs, dt)
        inv = f.unary("rsqrt", f.binary("add", var, f.splat(eps, kshape, dt), kshape, dt), kshape, dt)
        y = f.binary("multiply", xc, f.bcast(inv, kshape, [0, 1, 2], xs, dt), xs, dt)
        y = f.binary("multiply", y, f.bcast(g, [d], [2], xs, dt), xs, dt)
        return f.binary("add", y, f.bcast(b, [d], [2], xs, dt), xs, dt)

    def dense(v, vshape, w, b, n_out):
        y, yshape = f.dot_general(v, w, vshape, [vshape[-1], n_out], ([], []), ([len(vshape) - 1], [0]), dt)
        return f.binary("add", y, f.bcast(b, [n_out], [len(yshape) - 1], yshape, dt), yshape, dt), yshape

    funcs = []
    for _ in range(layers):
        g1, b1, wqkv, bqkv, wo, bo, g2, b2, w1, bm1, w2, bm2 = (f.arg(ai + i) for i in range(12))
        ai += 12
        h = ln(x, g1, b1)
        qkv, qshape = dense(h, xs, wqkv, bqkv, 3 * d)
        parts = []
        for j in range(3):
            sl = f.emit(f"stablehlo.slice {qkv} [0:{B}, 0:{T}, {j * d}:{(j + 1) * d}] : "
                        f"({ty(qshape, dt)}) -> {ty(xs, dt)}")
            parts.append(f.reshape(sl, xs, [B, T, heads, hd], dt))
        q, k, v = parts
        # 'BTNH,BSNH->BNTS'
        s, sshape = f.dot_general(q, k, [B, T, heads, hd], [B, T, heads, hd], ([0, 2], [0, 2]), ([3], [3]), dt)
        s = f.binary("multiply", s, f.splat(1.0 / math.sqrt(hd), sshape, dt), sshape, dt)
        if causal:
            pred = _causal_pred(f, T, T)
            pb = f.bcast(pred, [T, T], [2, 3], sshape, "i1")
            s = f.emit(f"stablehlo.select {pb}, {s}, {f.splat(-math.inf, sshape, dt)} : {ty(sshape, 'i1')}, "
                       f"{ty(sshape, dt)}")
        p = f.call("softmax", [s], [ty(sshape, dt)], ty(sshape, dt))
        # 'BNTS,BSNH->BNTH' then to BTNH
        o, oshape = f.dot_general(p, v, sshape, [B, T, heads, hd], ([0, 1], [0, 2]), ([3], [1]), dt)
        o, oshape = f.transpose(o, oshape, [0, 2, 1, 3], dt)
        o = f.reshape(o, oshape, xs, dt)
        o, _ = dense(o, xs, wo, bo, d)
        x = f.binary("add", x, o, xs, dt)
        h = ln(x, g2, b2)
        u, ushape = dense(h, xs, w1, bm1, mlp)
        # gelu tanh: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
        x3 = f.binary("multiply", f.binary("multiply", u, u, ushape, dt), u, ushape, dt)
        inner = f.binary("add", u, f.binary("multiply", f.splat(0.044715, ushape, dt), x3, ushape, dt), ushape, dt)
        inner = f.binary("multiply", f.splat(math.sqrt(2.0 / math.pi), ushape, dt), inner, ushape, dt)
        t = f.unary("tanh", inner, ushape, dt)
        g = f.binary("multiply", f.binary("multiply", f.splat(0.5, ushape, dt), u, ushape, dt),
                     f.binary("add", f.splat(1.0, ushape, dt), t, ushape, dt), ushape, dt)
        m, _ = dense(g, ushape, w2, bm2, d)
        x = f.binary("add", x, m, xs, dt)
    funcs.append(softmax_fn([B, heads, T, T], dt))
    return module("jit_transformer", [f.text([x], [ty(xs, dt)])] + funcs)


def dense_module(M=256, K=128, N=192, epilogue="bias", dt="f32", escape=None):
    """One dense layer y = x @ w followed by its epilogue: "bias" (y + b),
    "bias_gelu" (tanh GELU of y + b), "bias_residual" (r + (y + b)).
    escape="result" also returns y; escape="reader" also returns y * 2 (a
    second program reading y).  Arguments: x [M, K], w [K, N], b [N] and, for
    bias_residual, r [M, N]."""
    args = [([M, K], dt), ([K, N], dt), ([N], dt)]
    if epilogue == "bias_residual":
        args.append(([M, N], dt))
    f = Fn("main", args)
    y, ys = f.dot_general(f.arg(0), f.arg(1), [M, K], [K, N], ([], []), ([1], [0]), dt)
    u = f.binary("add", y, f.bcast(f.arg(2), [N], [1], ys, dt), ys, dt)
    if epilogue == "bias_gelu":
        x3 = f.binary("multiply", f.binary("multiply", u, u, ys, dt), u, ys, dt)
        inner = f.binary("add", u, f.binary("multiply", f.splat(0.044715, ys, dt), x3, ys, dt), ys, dt)
        inner = f.binary("multiply", f.splat(math.sqrt(2.0 / math.pi), ys, dt), inner, ys, dt)
        t = f.unary("tanh", inner, ys, dt)
        u = f.binary("multiply", f.binary("multiply", f.splat(0.5, ys, dt), u, ys, dt),
                     f.binary("add", f.splat(1.0, ys, dt), t, ys, dt), ys, dt)
    elif epilogue == "bias_residual":
        u = f.binary("add", f.arg(3), u, ys, dt)
    outs = [u]
    if escape == "result":
        outs.append(y)
    elif escape == "reader":
        outs.append(f.binary("multiply", y, f.splat(2.0, ys, dt), ys, dt))
    return module("jit_dense", [f.text(outs, [ty(ys, dt)] * len(outs))])


def batched_dense_module(Bt=3, M=100, K=64, N=96, dt="f32"):
    """A batched product 'bmk,bkn->bmn' (batching dims 0 x 0) followed by a
    bias add and a tanh GELU over its [Bt, M, N] result.  Arguments:
    x [Bt, M, K], w [Bt, K, N], b [N]."""
    f = Fn("main", [([Bt, M, K], dt), ([Bt, K, N], dt), ([N], dt)])
    y, ys = f.dot_general(f.arg(0), f.arg(1), [Bt, M, K], [Bt, K, N], ([0], [0]), ([2], [1]), dt)
    u = f.binary("add", y, f.bcast(f.arg(2), [N], [2], ys, dt), ys, dt)
    x3 = f.binary("multiply", f.binary("multiply", u, u, ys, dt), u, ys, dt)
    inner = f.binary("add", u, f.binary("multiply", f.splat(0.044715, ys, dt), x3, ys, dt), ys, dt)
    inner = f.binary("multiply", f.splat(math.sqrt(2.0 / math.pi), ys, dt), inner, ys, dt)
    t = f.unary("tanh", inner, ys, dt)
    g = f.binary("multiply", f.binary("multiply", f.splat(0.5, ys, dt), u, ys, dt),
                 f.binary("add", f.splat(1.0, ys, dt), t, ys, dt), ys, dt)
    return module("jit_batched_dense", [f.text([g], [ty(ys, dt)])])


def config4_inputs(seed=4, layers=4, B=32, T=256, d=512, mlp=2048):
    """Arguments of transformer_module in order, as BASELINE config 4 states
    them: x ~ N(0,1), Xavier-uniform weights (U(+-sqrt(6 / (fan_in +
    fan_out)))), zero biases, LayerNorm scales 1 and offsets 0, drawn from
    numpy.random.default_rng(seed) in argument order, generated in f32."""
    import numpy as np

    rng = np.random.default_rng(seed)

    def xavier(fi, fo):
        a = math.sqrt(6.0 / (fi + fo))
        return rng.uniform(-a, a, size=(fi, fo)).astype(np.float32)

    ones = lambda n: np.ones(n, np.float32)  # noqa: E731
    zeros = lambda n: np.zeros(n, np.float32)  # noqa: E731
    out = [rng.standard_normal((B, T, d), dtype=np.float32)]
    for _ in range(layers):
        out += [ones(d), zeros(d), xavier(d, 3 * d), zeros(3 * d), xavier(d, d), zeros(d),
                ones(d), zeros(d), xavier(d, mlp), zeros(mlp), xavier(mlp, d), zeros(d)]
    return out


def transformer_flops(layers=4, B=32, T=256, d=512, heads=8, mlp=2048):
    tok = B * T
    per = 2 * tok * d * 3 * d + 2 * tok * d * d + 2 * tok * d * mlp * 2 + 4 * B * T * T * d
    return layers * per
