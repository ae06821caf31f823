"""Fused LayerNorm primitives for the MI355X plugin.

Same contract as the reference's package (src/jax_mlx/layer_norm.py):

* `mlx_layer_norm` (x, weight, bias; attribute `eps`) -> y over the last
  axis, lowered on the plugin's platform to `custom_call @mlx_layer_norm`
  with backend_config `{"eps": e}` (reference :86-100);
* `mlx_layer_norm_bwd` (x, weight, bias, grad_out; `eps`) -> (dx, dweight,
  dbias), lowered to `custom_call @mlx_layer_norm_bwd` (reference :102-116);
* `mlx_layer_norm(x, weight, bias, eps)`: a `custom_vjp` pairing the two
  (reference :143-160);
* `patch_flax_layer_norm()`: routes flax.nnx.LayerNorm and
  flax.linen.LayerNorm calls that normalise the last axis with both scale and
  bias through it (reference :165-252).

y = (x - mean) / sqrt(var + eps) * weight + bias with the population
variance (reference :20-25).  On other platforms the primitives lower to the
same mathematics written with jax.numpy (`layer_norm_reference` /
`layer_norm_reference_bwd`, which also run on numpy arrays).  jax and flax
are imported only when used.
"""
from __future__ import annotations

import functools
import json

PLATFORM = "mi355x"
_prims: dict = {}


# ---- the mathematics (any array namespace: jax.numpy or numpy) --------------

def layer_norm_reference(xp, x, weight, bias, eps):
    xf = x.astype(xp.float32)
    mu = xf.mean(axis=-1, keepdims=True)
    var = ((xf - mu) ** 2).mean(axis=-1, keepdims=True)
    return ((xf - mu) / xp.sqrt(var + eps) * weight + bias).astype(x.dtype)


def layer_norm_reference_bwd(xp, x, weight, bias, grad_out, eps):
    """(dx, dweight, dbias) with x_hat = (x - mean) * r, r = 1/sqrt(var + eps):
    dbias = sum(g), dweight = sum(g x_hat) over all rows,
    dx = r (g w - mean(g w) - x_hat mean(g w x_hat)) per row."""
    xf = x.astype(xp.float32)
    g = grad_out.astype(xp.float32)
    mu = xf.mean(axis=-1, keepdims=True)
    r = 1.0 / xp.sqrt(((xf - mu) ** 2).mean(axis=-1, keepdims=True) + eps)
    xh = (xf - mu) * r
    rows = tuple(range(x.ndim - 1))
    dbias = g.sum(axis=rows)
    dweight = (g * xh).sum(axis=rows)
    gw = g * weight
    dx = r * (gw - gw.mean(axis=-1, keepdims=True) - xh * (gw * xh).mean(axis=-1, keepdims=True))
    return dx.astype(x.dtype), dweight.astype(weight.dtype), dbias.astype(bias.dtype)


# ---- primitives ---------------------------------------------------------------

def _build():
    if _prims:
        return _prims
    import jax.numpy as jnp
    from jax._src import core
    from jax._src.interpreters import mlir

    fwd = core.Primitive("mlx_layer_norm")
    bwd = core.Primitive("mlx_layer_norm_bwd")
    bwd.multiple_results = True
    fwd.def_impl(lambda x, w, b, *, eps: layer_norm_reference(jnp, x, w, b, eps))
    fwd.def_abstract_eval(lambda x, w, b, *, eps: core.ShapedArray(x.shape, x.dtype))
    bwd.def_impl(lambda x, w, b, g, *, eps: layer_norm_reference_bwd(jnp, x, w, b, g, eps))
    bwd.def_abstract_eval(lambda x, w, b, g, *, eps: (core.ShapedArray(x.shape, x.dtype),
                                                       core.ShapedArray(w.shape, w.dtype),
                                                       core.ShapedArray(b.shape, b.dtype)))
    mlir.register_lowering(fwd, mlir.lower_fun(
        lambda x, w, b, *, eps: layer_norm_reference(jnp, x, w, b, eps), multiple_results=False))
    mlir.register_lowering(bwd, mlir.lower_fun(
        lambda x, w, b, g, *, eps: layer_norm_reference_bwd(jnp, x, w, b, g, eps), multiple_results=True))
    _prims.update(fwd=fwd, bwd=bwd)
    return _prims


def __getattr__(name):
    if name == "mlx_layer_norm_p":
        return _build()["fwd"]
    if name == "mlx_layer_norm_bwd_p":
        return _build()["bwd"]
    raise AttributeError(name)


def _config(eps: float) -> str:
    return json.dumps({"eps": float(eps)})


def register_lowering(platform: str = PLATFORM) -> None:
    """custom_call lowerings of both primitives on the plugin's platform."""
    from jax._src.interpreters import mlir

    prims = _build()

    def fwd_lowering(ctx, x, w, b, *, eps):
        return mlir.custom_call("mlx_layer_norm", result_types=[mlir.aval_to_ir_type(ctx.avals_out[0])],
                                operands=[x, w, b], backend_config=_config(eps)).results

    def bwd_lowering(ctx, x, w, b, g, *, eps):
        return mlir.custom_call("mlx_layer_norm_bwd", result_types=[mlir.aval_to_ir_type(a) for a in ctx.avals_out],
                                operands=[x, w, b, g], backend_config=_config(eps)).results

    mlir.register_lowering(prims["fwd"], fwd_lowering, platform=platform)
    mlir.register_lowering(prims["bwd"], bwd_lowering, platform=platform)


@functools.lru_cache(maxsize=None)
def _fused(eps: float):
    import jax

    prims = _build()

    @jax.custom_vjp
    def layer_norm(x, w, b):
        return prims["fwd"].bind(x, w, b, eps=eps)

    def layer_norm_fwd(x, w, b):
        return layer_norm(x, w, b), (x, w, b)

    def layer_norm_bwd(res, g):
        return tuple(prims["bwd"].bind(*res, g, eps=eps))

    layer_norm.defvjp(layer_norm_fwd, layer_norm_bwd)
    return layer_norm


def mlx_layer_norm(x, weight, bias, eps=1e-5):
    """Fused LayerNorm over the last axis with the fused backward as its VJP
    (reference argument order)."""
    return _fused(float(eps))(x, weight, bias)


def _last_axis_only(axes, ndim) -> bool:
    if isinstance(axes, int):
        axes = (axes,)
    return tuple(a % ndim for a in axes) == (ndim - 1,)


def patch_flax_layer_norm() -> None:
    """Route flax LayerNorm modules (nnx and linen) that normalise only the
    last axis with a scale and a bias through mlx_layer_norm; other
    configurations keep flax's implementation.  A missing flax is ignored."""
    try:
        import flax.nnx as nnx
    except ImportError:
        nnx = None
    if nnx is not None and not getattr(nnx.LayerNorm.__call__, "_mi355x_fused", False):
        nnx_call = nnx.LayerNorm.__call__

        def nnx_layer_norm(self, x, *args, **kwargs):
            scale, bias = getattr(self, "scale", None), getattr(self, "bias", None)
            if (args or kwargs or scale is None or bias is None
                    or not _last_axis_only(getattr(self, "reduction_axes", -1), x.ndim)
                    or not _last_axis_only(getattr(self, "feature_axes", -1), x.ndim)):
                return nnx_call(self, x, *args, **kwargs)
            return mlx_layer_norm(x, scale.value, bias.value, getattr(self, "epsilon", 1e-6))

        nnx_layer_norm._mi355x_fused = True
        nnx.LayerNorm.__call__ = nnx_layer_norm

    try:
        import flax.linen as nn
    except ImportError:
        nn = None
    if nn is not None and not getattr(nn.LayerNorm.__call__, "_mi355x_fused", False):
        linen_call = nn.LayerNorm.__call__

        def linen_layer_norm(self, x, *args, **kwargs):
            if (args or kwargs or not getattr(self, "use_scale", True) or not getattr(self, "use_bias", True)
                    or not _last_axis_only(getattr(self, "reduction_axes", -1), x.ndim)
                    or not _last_axis_only(getattr(self, "feature_axes", -1), x.ndim)):
                return linen_call(self, x, *args, **kwargs)
            features = (x.shape[-1],)
            pdt = getattr(self, "param_dtype", x.dtype)
            scale = self.param("scale", self.scale_init, features, pdt)
            bias = self.param("bias", self.bias_init, features, pdt)
            return mlx_layer_norm(x, scale, bias, getattr(self, "epsilon", 1e-6))

        linen_layer_norm._mi355x_fused = True
        nn.LayerNorm.__call__ = linen_layer_norm
