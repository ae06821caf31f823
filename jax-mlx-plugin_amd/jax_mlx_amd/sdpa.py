"""`mlx_sdpa` primitive: fused attention as a `custom_call` the plugin runs.

Same contract as the reference's primitive (src/jax_mlx/sdpa.py:19-47,
97-112): BTNH query/key/value, one float attribute `scale`, lowered to
`stablehlo.custom_call @mlx_sdpa` with backend_config `{"scale": s}`.  The
plugin's compiler turns that call into its flash kernel (any N/K head ratio).
Off the plugin the primitive evaluates the same formula with jax.numpy.
"""
from __future__ import annotations

_prims = {}


def _primitive():
    if "fwd" in _prims:
        return _prims["fwd"]
    import jax.numpy as jnp
    from jax._src import core

    p = core.Primitive("mlx_sdpa")

    def impl(q, k, v, *, scale):
        # softmax(scale * q k^T) v over BTNH, k/v heads repeated for GQA.
        g = q.shape[2] // k.shape[2]
        kk = jnp.repeat(k, g, axis=2)
        vv = jnp.repeat(v, g, axis=2)
        s = jnp.einsum("btnh,bsnh->bnts", q.astype(jnp.float32), kk.astype(jnp.float32)) * scale
        pr = jnp.exp(s - s.max(-1, keepdims=True))
        pr = pr / pr.sum(-1, keepdims=True)
        return jnp.einsum("bnts,bsnh->btnh", pr, vv.astype(jnp.float32)).astype(q.dtype)

    p.def_impl(impl)
    p.def_abstract_eval(lambda q, k, v, *, scale: core.ShapedArray(q.shape, q.dtype))
    _prims["fwd"] = p
    return p


def register_lowering(platform: str) -> None:
    from jax._src.interpreters import mlir

    def lowering(ctx, q, k, v, *, scale):
        out = mlir.custom_call("mlx_sdpa", result_types=[mlir.aval_to_ir_type(ctx.avals_out[0])],
                               operands=[q, k, v], backend_config=f'{{"scale": {float(scale)!r}}}')
        return out.results

    mlir.register_lowering(_primitive(), lowering, platform=platform)


def mlx_dot_product_attention(query, key, value, scale=None):
    """Fused attention on BTNH arrays (reference name and argument order)."""
    if scale is None:
        scale = query.shape[-1] ** -0.5
    return _primitive().bind(query, key, value, scale=float(scale))
