"""MLIR bytecode -> text, called by libpjrt_mi355x.so from inside the jaxlib
process (csrc/pjrt/bytecode.cpp).

jaxlib gives PJRT plugins each module as a StableHLO portable artifact; the
plugin's own parser reads MLIR text, so the artifact is deserialised with the
StableHLO bindings jaxlib already ships and printed in the pretty form
(reference route: src/jax_mlx_pjrt.cpp:749-822).  Needs jax / jaxlib, which
only the calling process provides.
"""


def to_text(data: bytes) -> str:
    from jax._src.interpreters import mlir
    from jaxlib.mlir.dialects import stablehlo

    with mlir.make_ir_context() as ctx:
        module = stablehlo.deserialize_portable_artifact(ctx, data)
        return module.operation.get_asm(enable_debug_info=False)
