"""The JAX-facing package (jax_mlx_amd.plugin / sdpa / layer_norm) without
jax: it imports, declares its `jax_plugins` entry point, emits the
backend_config the plugin's compiler parses, and its fallback mathematics
(which the primitives lower to off the plugin's platform) matches the fp64
oracle.  jax is absent here and on the GPU box, so the jax side itself --
primitives, custom_vjp, lowerings, patches -- is unverified end-to-end.

Reference: src/jax_mlx/sdpa.py:19-31, 65-87, 97-151, 194-265;
src/jax_mlx/layer_norm.py:20-25, 59-76, 86-116, 165-252; setup.py:73-77."""
import importlib
import importlib.util
import math
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]


def test_imports_without_jax():
    for name in ("jax_mlx_amd.plugin", "jax_mlx_amd.sdpa", "jax_mlx_amd.layer_norm"):
        importlib.import_module(name)
    if importlib.util.find_spec("jax") is None:
        assert "jax" not in sys.modules  # nothing above imported it eagerly


def test_entry_point_declared():
    import tomli

    meta = tomli.loads((REPO / "jax-mlx-plugin_amd" / "pyproject.toml").read_text())
    from jax_mlx_amd import plugin

    eps = meta["project"]["entry-points"][plugin.ENTRY_POINT_GROUP]
    assert eps[plugin.ENTRY_POINT_NAME] == "jax_mlx_amd.plugin"
    mod = importlib.import_module(eps[plugin.ENTRY_POINT_NAME])
    assert callable(mod.initialize) and mod.PLATFORM == "mi355x"
    assert "lib/*.so" in meta["tool"]["setuptools"]["package-data"]["jax_mlx_amd"]


def btnh(a):
    return np.ascontiguousarray(a.transpose(0, 2, 1, 3))


@pytest.mark.parametrize("N,K", [(4, 4), (8, 2)])
def test_attention_fallback_matches_oracle(oracle, N, K):
    from jax_mlx_amd import sdpa

    rng = np.random.default_rng(41)
    B, T, S, H = 2, 24, 40, 32
    q = rng.standard_normal((B, T, N, H)).astype(np.float32)
    k = rng.standard_normal((B, S, K, H)).astype(np.float32)
    v = rng.standard_normal((B, S, K, H)).astype(np.float32)
    g = rng.standard_normal((B, T, N, H)).astype(np.float32)
    scale = 0.17
    out = sdpa.attention_reference(np, q, k, v, scale)
    ref = btnh(oracle.sdpa(btnh(q), btnh(k), btnh(v), scale))
    assert out.dtype == np.float32 and np.abs(out - ref).max() <= 1e-5
    grads = sdpa.attention_reference_bwd(np, q, k, v, g, scale)
    refs = [btnh(r) for r in oracle.sdpa_bwd(btnh(q), btnh(k), btnh(v), btnh(g), scale)]
    for a, r in zip(grads, refs):
        assert a.shape == r.shape and np.abs(a - r).max() <= 1e-4 * max(1.0, np.abs(r).max())


def test_layer_norm_fallback_matches_oracle(oracle):
    from jax_mlx_amd import layer_norm as ln

    rng = np.random.default_rng(42)
    x = (rng.standard_normal((3, 5, 64)) * 2 + 0.3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(64)).astype(np.float32)
    b = (0.1 * rng.standard_normal(64)).astype(np.float32)
    g = rng.standard_normal((3, 5, 64)).astype(np.float32)
    y = ln.layer_norm_reference(np, x, w, b, 1e-5)
    assert np.abs(y - oracle.layer_norm(x, w, b, 1e-5)).max() <= 1e-5
    dx, dw, db = ln.layer_norm_reference_bwd(np, x, w, b, g, 1e-5)
    rdx, rdw, rdb = oracle.layer_norm_bwd(x.reshape(-1, 64), w, g.reshape(-1, 64), 1e-5)
    for a, r in ((dx.reshape(-1, 64), rdx), (dw, rdw), (db, rdb)):
        assert np.abs(a - r).max() <= 1e-5 * max(1.0, np.abs(r).max())


def test_routing_of_patched_dot_product_attention():
    from jax_mlx_amd.sdpa import routes_to_fused

    q, k = np.zeros((2, 8, 4, 16)), np.zeros((2, 8, 2, 16))
    assert routes_to_fused(q, k)                           # GQA goes to the fused pair
    assert routes_to_fused(q[0], k[0])                     # unbatched [T, N, H]
    assert not routes_to_fused(q, np.zeros((2, 8, 3, 16)))  # 4 heads over 3 kv heads
    for kw in ({"is_causal": True}, {"mask": q}, {"bias": q}, {"local_window_size": (4, 4)},
               {"query_seq_lengths": q}, {"key_value_seq_lengths": q}, {"return_residual": True}):
        assert not routes_to_fused(q, k, **kw)           # JAX's path (the plugin fuses its HLO)


def _escaped(cfg):
    return cfg.replace('"', "\\22")


@pytest.mark.parametrize("scale", [0.125, 1.0 / math.sqrt(128), 3e-2])
def test_backend_configs_parse_in_the_plugin(scale):
    """The JSON the lowerings emit is what Client_Compile parses."""
    import mlir_modules as M
    from jax_mlx_amd import layer_norm as ln
    from jax_mlx_amd import pjrt
    from jax_mlx_amd import sdpa

    api = pjrt.Api()
    text = M.custom_call_sdpa_module(scale=0.5).replace(_escaped('{"scale": 0.5}'),
                                                        _escaped(sdpa._config(scale)))
    (n,) = [n for n in api.inspect(text)["graph"]["nodes"] if n["op"] == "mfx.sdpa"]
    assert math.isclose(n["f:scale"], scale, rel_tol=1e-6)
    text = M.custom_call_layer_norm_module(eps=0.5).replace(_escaped('{"eps": 0.5}'), _escaped(ln._config(scale)))
    (n,) = [n for n in api.inspect(text)["graph"]["nodes"] if n["op"] == "mfx.layer_norm"]
    assert math.isclose(n["f:eps"], scale, rel_tol=1e-6)
