/*
 * pjrt_mi355x.h — entry points of libpjrt_mi355x.so, the PJRT plugin.
 *
 * GetPjrtApi is the plugin's whole interface to jaxlib (and any other PJRT
 * C-API client): the reference exports exactly this symbol
 * (reference src/jax_mlx_pjrt.cpp:9481-9670) and jax_mlx/plugin.py registers
 * the library with xla_bridge.register_plugin (src/jax_mlx/plugin.py:24-47).
 * The table layout is PJRT C API 0.90 (include/pjrt_abi.h).
 *
 * mfx_pjrt_inspect / mfx_pjrt_free have no counterpart in the reference: they
 * expose, for tests and debugging on machines without a GPU, what Compile
 * does to a StableHLO module (parse, inline calls, fused-pattern rewrite,
 * launch plan), which the reference only prints under MLX_PJRT_DEBUG
 * (src/jax_mlx_pjrt.cpp:2225-2230 and its other debug prints).
 */
#ifndef PJRT_MI355X_H_
#define PJRT_MI355X_H_

#include <stddef.h>

#include "pjrt_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The PJRT function table (static storage, version 0.90). */
const PJRT_Api* GetPjrtApi(void);

/* Parses + rewrites + plans MLIR text without touching a device.  On success
 * returns 0 and *json_out points to a malloc'd JSON document
 * {"graph": {...rewritten main...}, "plan": {...steps...}}; on failure returns
 * a non-zero PJRT_Error_Code and *json_out holds {"error": "..."}.
 * Free the string with mfx_pjrt_free. */
int mfx_pjrt_inspect(const char* mlir_text, size_t size, char** json_out);
void mfx_pjrt_free(char* p);

#ifdef __cplusplus
}
#endif

#endif /* PJRT_MI355X_H_ */
