"""JAX registration of the MI355X PJRT plugin.

Mirrors the reference's `jax_mlx.plugin` (src/jax_mlx/plugin.py:24-47):
`initialize()` registers libpjrt_mi355x.so with jaxlib under the platform name
"mi355x" and installs the `custom_call` lowerings of the fused primitives
(`mlx_sdpa`, `mlx_layer_norm`) for that platform.  jax is imported lazily, so
this module also imports in processes without jax.
"""
from __future__ import annotations

from pathlib import Path

PLATFORM = "mi355x"


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
