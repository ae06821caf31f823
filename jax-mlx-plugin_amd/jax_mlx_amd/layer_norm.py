"""`mlx_layer_norm` primitive: fused LayerNorm as a `custom_call`.

Same contract as the reference's primitive (src/jax_mlx/layer_norm.py:20-40,
86-100): operands x, weight, bias; attribute `eps`; lowered to
`stablehlo.custom_call @mlx_layer_norm` with backend_config `{"eps": e}`;
y = (x - mean) / sqrt(var + eps) * weight + bias over the last axis with the
population variance.
"""
from __future__ import annotations

_prims = {}


def _primitive():
    if "fwd" in _prims:
        return _prims["fwd"]
    import jax.numpy as jnp
    from jax._src import core

    p = core.Primitive("mlx_layer_norm")

    def impl(x, weight, bias, *, eps):
        xf = x.astype(jnp.float32)
        mu = xf.mean(-1, keepdims=True)
        var = ((xf - mu) ** 2).mean(-1, keepdims=True)
        return ((xf - mu) / jnp.sqrt(var + eps) * weight + bias).astype(x.dtype)

    p.def_impl(impl)
    p.def_abstract_eval(lambda x, w, b, *, eps: core.ShapedArray(x.shape, x.dtype))
    _prims["fwd"] = p
    return p


def register_lowering(platform: str) -> None:
    from jax._src.interpreters import mlir

    def lowering(ctx, x, w, b, *, eps):
        out = mlir.custom_call("mlx_layer_norm", result_types=[mlir.aval_to_ir_type(ctx.avals_out[0])],
                               operands=[x, w, b], backend_config=f'{{"eps": {float(eps)!r}}}')
        return out.results

    mlir.register_lowering(_primitive(), lowering, platform=platform)


def mlx_layer_norm(x, weight, bias, eps=1e-5):
    """Fused LayerNorm over the last axis (reference argument order)."""
    return _primitive().bind(x, weight, bias, eps=float(eps))
