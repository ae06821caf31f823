"""Fused attention primitives for the MI355X plugin.

Same contract as the reference's package (src/jax_mlx/sdpa.py):

* `mlx_sdpa` (query, key, value; attribute `scale`) -> output, lowered on
  the plugin's platform to `stablehlo.custom_call @mlx_sdpa` with
  backend_config `{"scale": s}` (reference :97-112);
* `mlx_sdpa_bwd` (query, key, value, grad_out; `scale`) -> (dq, dk, dv),
  lowered to `custom_call @mlx_sdpa_bwd` (reference :114-130);
* `mlx_dot_product_attention(query, key, value, scale)`: a `custom_vjp` whose
  forward binds `mlx_sdpa` and whose backward binds `mlx_sdpa_bwd`
  (reference :156-191);
* `patch_jax_dot_product_attention()`: routes `jax.nn.dot_product_attention`
  calls without bias, mask, causal flag, sequence lengths or window to the
  fused pair (reference :194-265).  Unlike the reference it also routes
  grouped-query calls (N a multiple of K): the plugin's kernels take any
  head ratio.  Causal and masked calls keep JAX's own implementation, whose
  StableHLO the plugin's compiler fuses into the causal / masked kernels.

Layout is BTNH ([batch, seq, heads, head_dim]).  On other platforms the
primitives lower to the same mathematics written with jax.numpy
(`attention_reference` / `attention_reference_bwd`, which also run on numpy
arrays).  jax is imported only when a primitive is first used, so this
module imports in processes without jax.
"""
from __future__ import annotations

import functools
import json

PLATFORM = "mi355x"
_prims: dict = {}


# ---- the mathematics (any array namespace: jax.numpy or numpy) --------------

def _grouped(xp, query, key):
    """q [B,T,N,H] -> [B,T,K,G,H] so head n reads kv head n // G."""
    B, T, N, H = query.shape
    K = key.shape[2]
    if K == 0 or N % K:
        raise ValueError(f"query heads ({N}) must be a multiple of key/value heads ({K})")
    return xp.reshape(query, (B, T, K, N // K, H))


def attention_reference(xp, query, key, value, scale):
    """softmax(scale * q k^T) v in fp32, BTNH in and out (GQA by grouping)."""
    q = _grouped(xp, query, key).astype(xp.float32)
    s = xp.einsum("btkgh,bskh->bkgts", q, key.astype(xp.float32)) * scale
    s = s - s.max(axis=-1, keepdims=True)
    p = xp.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    o = xp.einsum("bkgts,bskh->btkgh", p, value.astype(xp.float32))
    return xp.reshape(o, query.shape[:3] + (value.shape[-1],)).astype(query.dtype)


def attention_reference_bwd(xp, query, key, value, grad_out, scale):
    """(dq, dk, dv) of attention_reference for upstream gradient grad_out:
    P = softmax(scale q k^T), dP = g v^T, dS = P (dP - rowsum(P dP)),
    dq = scale dS k, dk = scale dS^T q, dv = P^T g; dk, dv summed over the
    query heads that share a kv head."""
    q = _grouped(xp, query, key).astype(xp.float32)
    g = _grouped(xp, grad_out, key).astype(xp.float32)
    k = key.astype(xp.float32)
    v = value.astype(xp.float32)
    s = xp.einsum("btkgh,bskh->bkgts", q, k) * scale
    s = s - s.max(axis=-1, keepdims=True)
    p = xp.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    dp = xp.einsum("btkgh,bskh->bkgts", g, v)
    ds = p * (dp - (p * dp).sum(axis=-1, keepdims=True))
    dq = xp.einsum("bkgts,bskh->btkgh", ds, k) * scale
    dk = xp.einsum("bkgts,btkgh->bskh", ds, q) * scale
    dv = xp.einsum("bkgts,btkgh->bskh", p, g)
    return (xp.reshape(dq, query.shape).astype(query.dtype), dk.astype(key.dtype), dv.astype(value.dtype))


# ---- primitives ---------------------------------------------------------------

def _build():
    if _prims:
        return _prims
    import jax.numpy as jnp
    from jax._src import core
    from jax._src.interpreters import mlir

    fwd = core.Primitive("mlx_sdpa")
    bwd = core.Primitive("mlx_sdpa_bwd")
    bwd.multiple_results = True

    fwd.def_impl(lambda q, k, v, *, scale: attention_reference(jnp, q, k, v, scale))
    fwd.def_abstract_eval(lambda q, k, v, *, scale: core.ShapedArray(q.shape[:3] + (v.shape[-1],), q.dtype))
    bwd.def_impl(lambda q, k, v, g, *, scale: attention_reference_bwd(jnp, q, k, v, g, scale))
    bwd.def_abstract_eval(lambda q, k, v, g, *, scale: (core.ShapedArray(q.shape, q.dtype),
                                                         core.ShapedArray(k.shape, k.dtype),
                                                         core.ShapedArray(v.shape, v.dtype)))
    # Every other platform lowers the mathematics itself.
    mlir.register_lowering(fwd, mlir.lower_fun(
        lambda q, k, v, *, scale: attention_reference(jnp, q, k, v, scale), multiple_results=False))
    mlir.register_lowering(bwd, mlir.lower_fun(
        lambda q, k, v, g, *, scale: attention_reference_bwd(jnp, q, k, v, g, scale), multiple_results=True))
    _prims.update(fwd=fwd, bwd=bwd)
    return _prims


def __getattr__(name):
    # The reference's module-level names, built on first access.
    if name == "mlx_sdpa_p":
        return _build()["fwd"]
    if name == "mlx_sdpa_bwd_p":
        return _build()["bwd"]
    raise AttributeError(name)


def _config(scale: float) -> str:
    return json.dumps({"scale": float(scale)})


def register_lowering(platform: str = PLATFORM) -> None:
    """custom_call lowerings of both primitives on the plugin's platform."""
    from jax._src.interpreters import mlir

    prims = _build()

    def fwd_lowering(ctx, q, k, v, *, scale):
        return mlir.custom_call("mlx_sdpa", result_types=[mlir.aval_to_ir_type(ctx.avals_out[0])],
                                operands=[q, k, v], backend_config=_config(scale)).results

    def bwd_lowering(ctx, q, k, v, g, *, scale):
        return mlir.custom_call("mlx_sdpa_bwd", result_types=[mlir.aval_to_ir_type(a) for a in ctx.avals_out],
                                operands=[q, k, v, g], backend_config=_config(scale)).results

    mlir.register_lowering(prims["fwd"], fwd_lowering, platform=platform)
    mlir.register_lowering(prims["bwd"], bwd_lowering, platform=platform)


@functools.lru_cache(maxsize=None)
def _fused(scale: float):
    """custom_vjp of fused attention for one scale (scale is static)."""
    import jax

    prims = _build()

    @jax.custom_vjp
    def attention(q, k, v):
        return prims["fwd"].bind(q, k, v, scale=scale)

    def attention_fwd(q, k, v):
        return attention(q, k, v), (q, k, v)

    def attention_bwd(res, g):
        return tuple(prims["bwd"].bind(*res, g, scale=scale))

    attention.defvjp(attention_fwd, attention_bwd)
    return attention


def mlx_dot_product_attention(query, key, value, scale=None):
    """Fused attention on BTNH arrays with the fused backward as its VJP
    (reference name and argument order; scale defaults to 1/sqrt(head_dim))."""
    if scale is None:
        scale = query.shape[-1] ** -0.5
    return _fused(float(scale))(query, key, value)


def routes_to_fused(query, key, *, bias=None, mask=None, is_causal=False, query_seq_lengths=None,
                    key_value_seq_lengths=None, local_window_size=None, return_residual=False) -> bool:
    """Whether patched jax.nn.dot_product_attention sends a call to the fused
    primitives (shapes only; no jax needed)."""
    if bias is not None or mask is not None or is_causal or return_residual:
        return False
    if query_seq_lengths is not None or key_value_seq_lengths is not None or local_window_size is not None:
        return False
    if len(query.shape) not in (3, 4) or len(key.shape) != len(query.shape):
        return False
    N, K = query.shape[-2], key.shape[-2]
    return K > 0 and N % K == 0


def patch_jax_dot_product_attention() -> None:
    """Point jax.nn.dot_product_attention at the fused pair for the calls
    routes_to_fused() accepts; everything else keeps JAX's implementation."""
    import jax.nn as jnn
    from jax._src.nn import functions as nn_functions

    original = nn_functions.dot_product_attention
    if getattr(original, "_mi355x_fused", False):
        return

    def dot_product_attention(query, key, value, bias=None, mask=None, *, scale=None, is_causal=False,
                              query_seq_lengths=None, key_value_seq_lengths=None, local_window_size=None,
                              **kwargs):
        if not routes_to_fused(query, key, bias=bias, mask=mask, is_causal=is_causal,
                               query_seq_lengths=query_seq_lengths, key_value_seq_lengths=key_value_seq_lengths,
                               local_window_size=local_window_size,
                               return_residual=kwargs.get("return_residual", False)):
            return original(query, key, value, bias, mask, scale=scale, is_causal=is_causal,
                            query_seq_lengths=query_seq_lengths, key_value_seq_lengths=key_value_seq_lengths,
                            local_window_size=local_window_size, **kwargs)
        unbatched = query.ndim == 3
        if unbatched:
            query, key, value = query[None], key[None], value[None]
        out = mlx_dot_product_attention(query, key, value, scale)
        return out[0] if unbatched else out

    dot_product_attention._mi355x_fused = True
    dot_product_attention.__wrapped__ = original
    nn_functions.dot_product_attention = dot_product_attention
    jnn.dot_product_attention = dot_product_attention
