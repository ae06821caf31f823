"""JAX registration of the MI355X PJRT plugin.

Mirrors the reference's `jax_mlx.plugin` (src/jax_mlx/plugin.py:24-47 and
its `_register_sdpa_lowering`, :113-143): JAX's plugin discovery finds this
module through the `jax_plugins` entry point (pyproject.toml, as the
reference's setup.py:73-77 declares it) and calls `initialize()`, which
registers libpjrt_mi355x.so under the platform name "mi355x", installs the
`custom_call` lowerings of the fused primitives (`mlx_sdpa`, `mlx_sdpa_bwd`,
`mlx_layer_norm`, `mlx_layer_norm_bwd`) for that platform, and patches
`jax.nn.dot_product_attention` and flax's LayerNorm to use them.  jax is
imported lazily, so this module also imports in processes without jax.
"""
from __future__ import annotations

import warnings
from pathlib import Path

PLATFORM = "mi355x"
ENTRY_POINT_GROUP = "jax_plugins"
ENTRY_POINT_NAME = "mi355x_plugin"


def library_path() -> str:
    p = Path(__file__).resolve().parent / "lib" / "libpjrt_mi355x.so"
    if not p.exists():
        raise RuntimeError(f"{p} is not built; run jax-mlx-plugin_amd/build.py")
    return str(p)


def initialize() -> None:
    """Called by JAX's plugin discovery (or by hand before the first jit)."""
    from jax._src import xla_bridge

    xla_bridge.register_plugin(PLATFORM, library_path=library_path())
    from . import layer_norm, sdpa

    sdpa.register_lowering(PLATFORM)
    layer_norm.register_lowering(PLATFORM)
    # The patches are conveniences: a JAX or flax version whose internals
    # differ keeps its own implementations (the plugin still fuses their
    # StableHLO), so a failure here is a warning, not an error.
    for patch in (sdpa.patch_jax_dot_product_attention, layer_norm.patch_flax_layer_norm):
        try:
            patch()
        except Exception as exc:  # noqa: BLE001
            warnings.warn(f"mi355x plugin: {patch.__name__} skipped: {exc}", stacklevel=2)
