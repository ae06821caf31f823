"""MI355X-native replacement for jax-mlx-plugin's fused SDPA / LayerNorm / RMSNorm path.

Native pieces (built in-tree by jax-mlx-plugin_amd/build.py):
  lib/libmfx_kernels.so   gfx950 HIP kernels behind a C-ABI (include/mfx_kernels.h)
  lib/libpjrt_mi355x.so   PJRT C-API plugin exporting GetPjrtApi (include/pjrt_mi355x.h)

Python modules:
  native      ctypes binding of the kernel C-ABI (torch tensors as device memory)
  pjrt        ctypes driver of the PJRT C API (Client_Create -> Compile -> Execute)
  plugin      JAX plugin registration (`initialize`), active only when jax is importable
  sdpa, layer_norm   custom_call lowerings compatible with the reference's targets
"""
from pathlib import Path

__version__ = "0.1.0"

LIB_DIR = Path(__file__).resolve().parent / "lib"
