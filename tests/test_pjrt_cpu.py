"""PJRT plugin tests that need no GPU: the C API table, the exported symbols,
error behaviour without a device, and what Compile's rewriter and planner do
to each module form (through mfx_pjrt_inspect).

The pattern decisions follow the reference's RecognizePatterns cases
(src/jax_mlx_pjrt.cpp:1857-2044 softmax, :2166-2334 RMSNorm, :2336-2487
LayerNorm, :2490-2757 SDPA, :8108-8236 custom calls).  The reference has no
tests of these fusions (its tests/ hold test_compilation_coverage.py,
test_complex.py, test_exhaustive.py and test_exhaustive_while.py, none of
which covers SDPA, LayerNorm or RMSNorm), so the module texts are this
repository's own (tests/mlir_modules.py)."""
import json
import math
import re
import subprocess
from pathlib import Path

import pytest

import mlir_modules as M
from jax_mlx_amd import pjrt

REPO = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def api():
    return pjrt.Api()


def fused(doc):
    return [n for n in doc["graph"]["nodes"] if n["op"].startswith("mfx.")]


def steps(doc):
    return [s["kind"] for s in doc["plan"]["steps"]]


# ------------------------------------------------------------------ C API table

def test_table_order_matches_header(api):
    text = (REPO / "include" / "pjrt_abi.h").read_text()
    body = text[text.index("typedef struct PJRT_Api {"):]
    body = body[:body.index("} PJRT_Api;")]
    names = re.findall(r"PJRT_(?:FN|STUB)\(PJRT_(\w+)\)|void \(\*PJRT_(\w+)\)", body)
    names = [a or b for a, b in names]
    assert names == pjrt.SLOTS
    assert len(names) == 128


def test_table_header(api):
    assert api.version == (0, 90)
    assert api.struct_size == 40 + 8 * len(pjrt.SLOTS)
    assert all(api.slots.values()), [k for k, v in api.slots.items() if not v]


def test_exports():
    out = subprocess.run(["nm", "-D", "--defined-only", str(pjrt.PLUGIN_LIB)], capture_output=True, text=True,
                         check=True).stdout
    syms = {line.split()[-1] for line in out.splitlines() if " T " in line}
    header = (REPO / "include" / "pjrt_mi355x.h").read_text()
    declared = set(re.findall(r"^\S.*?\b(\w+)\(", header, re.M)) - {"defined"}
    assert declared == {"GetPjrtApi", "mfx_pjrt_inspect", "mfx_pjrt_free"}
    assert declared <= syms
    # nothing of the plugin's internals leaks into the dynamic symbol table
    assert syms == declared, syms - declared


C_HOST = r"""
#include <dlfcn.h>
#include <stdio.h>
#include "pjrt_mi355x.h"
int main(int argc, char** argv) {
  void* h = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
  if (!h) return 2;
  const PJRT_Api* (*get)(void) = (const PJRT_Api* (*)(void))dlsym(h, "GetPjrtApi");
  const PJRT_Api* api = get();
  PJRT_Plugin_Initialize_Args init = {PJRT_ABI_SIZE(PJRT_Plugin_Initialize_Args, extension_start)};
  if (api->PJRT_Plugin_Initialize(&init)) return 3;
  PJRT_Client_Create_Args cc = {0};
  cc.struct_size = sizeof cc;
  PJRT_Error* err = api->PJRT_Client_Create(&cc);
  int code = 0;
  if (err) {
    PJRT_Error_GetCode_Args g = {sizeof g, NULL, err, 0};
    api->PJRT_Error_GetCode(&g);
    code = g.code;
    PJRT_Error_Destroy_Args d = {sizeof d, NULL, err};
    api->PJRT_Error_Destroy(&d);
  } else {
    PJRT_Client_Destroy_Args d = {sizeof d, NULL, cc.client};
    api->PJRT_Client_Destroy(&d);
  }
  printf("%d.%d %d\n", api->pjrt_api_version.major_version, api->pjrt_api_version.minor_version, code);
  return 0;
}
"""


def test_c_host_binding(tmp_path):
    """The C host stub of the integration notes compiles against include/ and
    drives the table (Client_Create reports FAILED_PRECONDITION without a GPU)."""
    src = tmp_path / "host.c"
    src.write_text(C_HOST)
    exe = tmp_path / "host"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{REPO / 'include'}", str(src), "-o", str(exe),
                    "-ldl"], check=True)
    out = subprocess.run([str(exe), str(pjrt.PLUGIN_LIB)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    version, code = out.stdout.split()
    assert version == "0.90"
    import torch

    if not torch.cuda.is_available():
        assert int(code) == 9  # FAILED_PRECONDITION


INSPECT_HOST = r"""
#include <dlfcn.h>
#include <stdio.h>
#include <stdlib.h>
/* argv: plugin library, MLIR C-API library to load RTLD_GLOBAL first (or -),
 * file holding the program bytes */
int main(int argc, char** argv) {
  void* capi = NULL;
  if (argc != 4) return 2;
  if (argv[2][0] != '-' && !(capi = dlopen(argv[2], RTLD_NOW | RTLD_GLOBAL))) return 3;
  void* h = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
  if (!h) return 4;
  int (*inspect)(const char*, size_t, char**) = (int (*)(const char*, size_t, char**))dlsym(h, "mfx_pjrt_inspect");
  void (*release)(char*) = (void (*)(char*))dlsym(h, "mfx_pjrt_free");
  FILE* f = fopen(argv[3], "rb");
  if (!f) return 5;
  fseek(f, 0, SEEK_END);
  long n = ftell(f);
  fseek(f, 0, SEEK_SET);
  char* buf = malloc(n ? n : 1);
  if (fread(buf, 1, n, f) != (size_t)n) return 6;
  fclose(f);
  char* json = NULL;
  int rc = inspect(buf, (size_t)n, &json);
  printf("%d\n%s\n", rc, json);
  release(json);
  if (capi) {
    int (*live)(void) = (int (*)(void))dlsym(capi, "mlir_stub_live");
    int (*calls)(void) = (int (*)(void))dlsym(capi, "mlir_stub_calls");
    printf("%d %d\n", live(), calls());
  }
  free(buf);
  return 0;
}
"""


@pytest.fixture(scope="module")
def inspect_host(tmp_path_factory):
    """A C process without Python that inspects a program file through the
    plugin, optionally with the MLIR C-API test double loaded first."""
    d = tmp_path_factory.mktemp("capi")
    (d / "host.c").write_text(INSPECT_HOST)
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", str(d / "host.c"), "-o", str(d / "host"), "-ldl"],
                   check=True)
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-shared", "-fPIC",
                    str(REPO / "tests" / "capi" / "mlir_capi_stub.c"), "-o", str(d / "libmlir_capi_stub.so")],
                   check=True)

    def run(program: bytes, with_capi: bool):
        f = d / "program.bin"
        f.write_bytes(program)
        stub = str(d / "libmlir_capi_stub.so") if with_capi else "-"
        out = subprocess.run([str(d / "host"), str(pjrt.PLUGIN_LIB), stub, str(f)], capture_output=True,
                             text=True, timeout=60)
        assert out.returncode == 0, (out.returncode, out.stderr)
        lines = out.stdout.splitlines()
        doc = json.loads(lines[1])
        counts = tuple(int(x) for x in lines[2].split()) if with_capi else None
        return int(lines[0]), doc, counts

    return run


BYTECODE = b"ML\xefR"


@pytest.mark.parametrize("tag", [b"VHLO:", b"PARSE:"])
def test_bytecode_through_mlir_capi(inspect_host, tag):
    """Route 1 (reference src/jax_mlx_pjrt.cpp:674-745): with the MLIR C API
    in the process, bytecode is deserialised (or, failing that, parsed) and
    printed through it, and the module fuses as its text does.  Every
    context and module the plugin creates is destroyed."""
    text = M.layer_norm_module().encode()
    rc, doc, (live, calls) = inspect_host(BYTECODE + tag + text, True)
    assert rc == 0, doc
    assert doc["source"] == "mlir-capi"
    assert [n["op"] for n in fused(doc)] == [n["op"] for n in fused(inspect_text(text))]
    assert live == 0 and calls == 2


def inspect_text(text: bytes):
    return pjrt.Api().inspect(text)


def test_bytecode_mlir_capi_failure_names_both_routes(inspect_host):
    rc, doc, (live, _) = inspect_host(BYTECODE + b"not an artifact", True)
    assert rc == 3 and live == 0
    assert "MLIR C API could neither deserialize nor parse" in doc["error"]
    assert "no Python interpreter" in doc["error"] and "pass MLIR text" in doc["error"]


def test_bytecode_without_any_mlir_runtime(inspect_host):
    """Route 3: a host with neither the MLIR C API nor Python gets an error
    asking for MLIR text; text itself is accepted there."""
    rc, doc, _ = inspect_host(BYTECODE + b"VHLO:" + M.layer_norm_module().encode(), False)
    assert rc == 3
    assert "no MLIR C API" in doc["error"] and "pass MLIR text instead" in doc["error"]
    rc, doc, _ = inspect_host(M.layer_norm_module().encode(), False)
    assert rc == 0 and doc["source"] == "text"


def test_bytecode_through_python_without_jax(api):
    """Route 2 (reference :749-822) in this Python process, which has no jax:
    the call returns an error naming the missing module (no crash), after
    reporting that no MLIR C API is loaded."""
    with pytest.raises(pjrt.PjrtError) as e:
        api.inspect(BYTECODE + b"VHLO:" + M.layer_norm_module().encode())
    assert e.value.code_name == "INVALID_ARGUMENT"
    assert "no MLIR C API" in e.value.message
    assert "jax_mlx_amd._bytecode.to_text" in e.value.message and "jax" in e.value.message.split("to_text:")[1]


def test_jax_modules_import_without_jax():
    from jax_mlx_amd import layer_norm, plugin, sdpa

    assert Path(plugin.library_path()) == pjrt.PLUGIN_LIB
    assert callable(sdpa.mlx_dot_product_attention) and callable(layer_norm.mlx_layer_norm)


def test_client_create_needs_device(api):
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(pjrt.PjrtError) as e:
        pjrt.Client(api)
    assert e.value.code_name == "FAILED_PRECONDITION"


def test_unimplemented_slot_reports_error(api):
    # a stub slot returns an UNIMPLEMENTED PJRT_Error naming itself
    a = pjrt.new(pjrt.BufferArgs)
    with pytest.raises(pjrt.PjrtError) as e:
        api.call("Client_DmaMap", a)
    assert e.value.code_name == "UNIMPLEMENTED" and "DmaMap" in e.value.message


def test_struct_size_checked(api):
    a = pjrt.new(pjrt.ClientCreateArgs)
    a.struct_size = 8
    with pytest.raises(pjrt.PjrtError) as e:
        api.call("Client_Create", a)
    assert e.value.code_name == "INVALID_ARGUMENT"


# ------------------------------------------------------------ rewriter + planner

@pytest.mark.parametrize("form", ["var", "standardize"])
def test_layer_norm_forms_fuse_with_affine(api, form):
    d = api.inspect(M.layer_norm_module(form=form))
    (n,) = fused(d)
    assert n["op"] == "mfx.layer_norm"
    assert n["i:has_gamma"] == [1] and n["i:has_beta"] == [1]
    assert math.isclose(n["f:eps"], 1e-5, rel_tol=1e-6)
    assert steps(d) == ["layer_norm"] and d["plan"]["arena_bytes"] == 0


def test_layer_norm_flax_bf16(api):
    d = api.inspect(M.layer_norm_module(shape=(4, 64, 256), dt="bf16", form="flax"))
    assert [n["op"] for n in fused(d)] == ["mfx.layer_norm"]
    assert steps(d)[-1] == "layer_norm"


def test_layer_norm_without_affine(api):
    d = api.inspect(M.layer_norm_module(affine=False, eps=1e-6))
    (n,) = fused(d)
    assert n["i:has_gamma"] == [0] and n["i:has_beta"] == [0]
    assert math.isclose(n["f:eps"], 1e-6, rel_tol=1e-6)


def test_layer_norm_intermediate_escapes_stays_computed(api):
    """A matched intermediate (the mean) returned by the function: the
    reference rejects the fusion (hasExternalConsumers,
    src/jax_mlx_pjrt.cpp:1819-1855); this rewriter fuses the normalisation
    and keeps the escaping mean's own ops, so both results are produced."""
    shape = [4, 128]
    f = M.Fn("main", [(shape, "f32")])
    x = f.arg(0)
    mean, ks = M._mean_keepdims(f, x, shape, "f32")
    cen = f.binary("subtract", x, f.bcast(mean, ks, [0, 1], shape, "f32"), shape, "f32")
    var, _ = M._mean_keepdims(f, f.binary("multiply", cen, cen, shape, "f32"), shape, "f32")
    inv = f.unary("rsqrt", f.binary("add", var, f.splat(1e-5, ks, "f32"), ks, "f32"), ks, "f32")
    y = f.binary("multiply", cen, f.bcast(inv, ks, [0, 1], shape, "f32"), shape, "f32")
    text = M.module("m", [f.text([y, mean], [M.ty(shape, "f32"), M.ty(ks, "f32")])])
    d = api.inspect(text)
    assert [n["op"] for n in fused(d)] == ["mfx.layer_norm"]
    assert len(d["graph"]["results"]) == 2
    assert "reduce" in steps(d) and "layer_norm" in steps(d)


def test_rms_norm(api):
    d = api.inspect(M.rms_norm_module())
    (n,) = fused(d)
    assert n["op"] == "mfx.rms_norm" and n["i:has_gamma"] == [1]
    assert math.isclose(n["f:eps"], 1e-6, rel_tol=1e-6)
    d = api.inspect(M.rms_norm_module(dt="bf16", upcast=True))
    assert [n["op"] for n in fused(d)] == ["mfx.rms_norm"]


def test_softmax_through_func_call(api):
    d = api.inspect(M.softmax_module())
    assert [n["op"] for n in fused(d)] == ["mfx.softmax"] and steps(d) == ["softmax"]


def test_log_softmax_through_func_call(api):
    d = api.inspect(M.log_softmax_module((6, 64)))
    (n,) = fused(d)
    assert n["op"] == "mfx.log_softmax"
    assert steps(d) == ["log_softmax"]
    assert d["graph"]["rewrites"]["log_softmax"] == 1


def test_sigmoid_divide_form_and_silu(api):
    d = api.inspect(M.sigmoid_silu_module((16, 256)))
    assert d["graph"]["rewrites"]["sigmoid"] == 1
    ops = [n["op"] for n in d["graph"]["nodes"]]
    assert "stablehlo.divide" not in ops and "stablehlo.exponential" not in ops
    assert ops.count("stablehlo.logistic") == 2  # the rewritten divide and silu's own
    assert steps(d) == ["elementwise", "elementwise"]


def test_softmax_on_leading_axis_is_not_fused(api):
    shape = [64, 6]
    f = M.Fn("main", [(shape, "f32")])
    x = f.arg(0)
    m, ms = f.reduce(x, shape, [0], "maximum", "f32")
    e = f.unary("exponential", f.binary("subtract", x, f.bcast(m, ms, [1], shape, "f32"), shape, "f32"),
                shape, "f32")
    z, zs = f.reduce(e, shape, [0], "add", "f32")
    y = f.binary("divide", e, f.bcast(z, zs, [1], shape, "f32"), shape, "f32")
    d = api.inspect(M.module("m", [f.text([y], [M.ty(shape, "f32")])]))
    assert fused(d) == []
    assert "reduce" in steps(d)


def test_sdpa_config2(api):
    d = api.inspect(M.sdpa_bhtd_module())
    (n,) = fused(d)
    assert n["op"] == "mfx.sdpa"
    assert n["i:shape"] == [8, 8, 8, 128, 128, 64, 64]  # B Hq Hkv Tq Tk D Dv
    assert n["i:causal"] == [0] and n["i:mask_kind"] == [0]
    assert math.isclose(n["f:scale"], 0.125, rel_tol=1e-6)
    assert steps(d) == ["sdpa"]


def test_sdpa_config3_causal_bhtd(api):
    d = api.inspect(M.sdpa_bhtd_module(B=4, H=32, T=2048, D=128, dt="bf16", causal=True))
    (n,) = fused(d)
    assert n["i:causal"] == [1] and n["i:shape"] == [4, 32, 32, 2048, 2048, 128, 128]


def test_sdpa_jax_nn_form_causal(api):
    d = api.inspect(M.dot_product_attention_module())
    (n,) = fused(d)
    assert n["i:causal"] == [1]
    # output written straight into the BTNH result: strides of [B, N, T, H] view
    assert n["i:o_strides"] == [2048 * 32 * 128, 128, 32 * 128, 1]
    assert steps(d) == ["sdpa"]


def test_sdpa_anti_causal_predicate_becomes_mask(api):
    """A lower-right/other predicate is not the causal one: it stays a mask."""
    T = 32
    text = M.sdpa_bhtd_module(B=1, H=2, T=T, D=64, causal=True)
    text = text.replace("GE,", "LE,")
    d = api.inspect(text)
    sd = [n for n in fused(d) if n["op"] == "mfx.sdpa"]
    assert sd and sd[0]["i:causal"] == [0] and sd[0]["i:mask_kind"] == [2]


def test_sdpa_finite_mask_value_falls_back(api):
    """select(pred, s, -1e9) is not treated as causal (the fill is finite):
    the module runs through the generic ops and softmax instead."""
    d = api.inspect(M.sdpa_bhtd_module(B=1, H=2, T=16, D=64, causal=True, mask_value=-1e9))
    assert "mfx.sdpa" not in [n["op"] for n in fused(d)]
    assert steps(d).count("gemm") == 2


@pytest.mark.parametrize("D,dt", [(32, "bf16"), (96, "f16"), (256, "bf16"), (256, "f32"), (80, "bf16")])
def test_sdpa_fuses_at_any_head_size(api, D, dt):
    """The attention match does not depend on the head size: the module is
    one fused step at 32, 96, 256 and at 80 (which the kernel library runs on
    its per-row kernel)."""
    d = api.inspect(M.sdpa_bhtd_module(B=1, H=2, T=64, D=D, dt=dt, causal=True))
    assert [n["op"] for n in fused(d)] == ["mfx.sdpa"]
    assert steps(d) == ["sdpa"]


def test_sdpa_transposed_k(api):
    d = api.inspect(M.sdpa_bhtd_module(transposed_k=True, inline_softmax=True))
    assert [n["op"] for n in fused(d)] == ["mfx.sdpa"]
    assert steps(d) == ["elementwise", "sdpa"]  # k made contiguous first


def test_sdpa_gqa_bias(api):
    d = api.inspect(M.dot_product_attention_module(B=2, T=64, N=8, K=2, H=64, is_causal=False, bias=True))
    (n,) = fused(d)
    assert n["i:shape"][:3] == [2, 8, 2]
    assert n["i:mask_kind"] == [1] and n["i:mask_strides"] == [64, 0, 0, 1]


def test_gqa_decode_with_q_rms(api):
    d = api.inspect(M.gqa_decode_module())
    (n,) = fused(d)
    assert n["i:q_rms"] == [1] and n["i:shape"] == [16, 32, 8, 1, 8192, 128, 128]
    assert n["i:mask_kind"] == [1]
    assert steps(d) == ["sdpa"] and d["plan"]["arena_bytes"] > 0  # split-KV workspace


def test_custom_calls(api):
    d = api.inspect(M.custom_call_sdpa_module(scale=0.2))
    (n,) = fused(d)
    assert n["op"] == "mfx.sdpa" and math.isclose(n["f:scale"], 0.2, rel_tol=1e-6)
    assert n["i:o_strides"] == [64 * 4 * 64, 64, 4 * 64, 1]
    d = api.inspect(M.custom_call_layer_norm_module(eps=1e-3))
    (n,) = fused(d)
    assert n["op"] == "mfx.layer_norm" and math.isclose(n["f:eps"], 1e-3, rel_tol=1e-6)
    d = api.inspect(M.custom_call_layer_norm_bwd_module(shape=(8, 128, 512), eps=1e-4))
    (n,) = fused(d)
    assert n["op"] == "mfx.layer_norm_bwd" and math.isclose(n["f:eps"], 1e-4, rel_tol=1e-6)
    assert steps(d) == ["layer_norm_bwd"] and d["plan"]["arena_bytes"] > 0  # parameter partials
    d = api.inspect(M.custom_call_sdpa_bwd_module(B=2, T=128, N=8, K=2, H=64, scale=0.3))
    (n,) = fused(d)
    assert n["op"] == "mfx.sdpa_bwd" and n["i:shape"] == [2, 8, 2, 128, 128, 64, 64]
    assert math.isclose(n["f:scale"], 0.3, rel_tol=1e-6)
    assert steps(d) == ["sdpa_bwd"] and d["plan"]["arena_bytes"] > 0  # recomputed O, lse, delta


def test_f16_modules_fuse(api):
    """f16 graphs take the same fused kernels as bf16 (the reference hands f16
    to the same MLX fast ops, src/jax_mlx_pjrt.cpp:317-349): LayerNorm (var
    and Flax forms), RMSNorm, softmax, log-softmax, SDPA (BHTD causal, the
    jax.nn form with a bias, GQA decode with q RMSNorm) and both backward
    custom calls."""
    def ops(text):
        return [n["op"] for n in fused(api.inspect(text))]

    assert ops(M.layer_norm_module(dt="f16")) == ["mfx.layer_norm"]
    assert ops(M.layer_norm_module(shape=(4, 64, 256), dt="f16", form="flax")) == ["mfx.layer_norm"]
    assert ops(M.rms_norm_module(dt="f16")) == ["mfx.rms_norm"]
    assert ops(M.rms_norm_module(dt="f16", upcast=True)) == ["mfx.rms_norm"]
    assert ops(M.softmax_module(dt="f16")) == ["mfx.softmax"]
    assert ops(M.log_softmax_module((6, 64), dt="f16")) == ["mfx.log_softmax"]
    d = api.inspect(M.sdpa_bhtd_module(B=2, H=4, T=256, D=128, dt="f16", causal=True))
    (n,) = fused(d)
    assert n["op"] == "mfx.sdpa" and n["i:causal"] == [1] and steps(d) == ["sdpa"]
    assert ops(M.dot_product_attention_module(B=2, T=64, N=8, K=2, H=64, dt="f16", is_causal=False,
                                              bias=True)) == ["mfx.sdpa"]
    assert ops(M.gqa_decode_module(B=2, S=512, dt="f16")) == ["mfx.sdpa"]
    assert ops(M.custom_call_sdpa_bwd_module(dt="f16")) == ["mfx.sdpa_bwd"]
    assert ops(M.custom_call_layer_norm_bwd_module(dt="f16")) == ["mfx.layer_norm_bwd"]


def test_custom_call_sdpa_shape_mismatch(api):
    """mlx_sdpa checks k and v against q as mlx_sdpa_bwd does: a head size or
    sequence length that disagrees, or N not a multiple of K, is a compile
    error rather than a strided read of the wrong elements."""
    def text(q, k, v):
        f = M.Fn("main", [(q, "f32"), (k, "f32"), (v, "f32")])
        o = f.emit(f'stablehlo.custom_call @mlx_sdpa(%arg0, %arg1, %arg2) {{backend_config = "{{}}"}} : '
                   f'({M.ty(q, "f32")}, {M.ty(k, "f32")}, {M.ty(v, "f32")}) -> {M.ty(q, "f32")}')
        return M.module("jit_mlx_sdpa", [f.text([o], [M.ty(q, "f32")])])

    q = [2, 64, 4, 64]
    api.inspect(text(q, [2, 80, 2, 64], [2, 80, 2, 64]))            # GQA, S != T: fine
    bad = [text(q, [2, 64, 2, 32], [2, 64, 2, 64]),                 # head size
           text(q, [2, 64, 2, 64], [2, 48, 2, 64]),                 # k / v lengths
           text(q, [2, 64, 3, 64], [2, 64, 3, 64]),                 # N % K != 0
           text(q, [1, 64, 2, 64], [1, 64, 2, 64])]                 # batch
    for t in bad:
        with pytest.raises(pjrt.PjrtError) as e:
            api.inspect(t)
        assert "mlx_sdpa" in e.value.message


def test_elementwise_index_width_rule(tmp_path):
    """The generated elementwise kernels switch to 64-bit loop indices when the
    grid-stride loop could pass INT32_MAX: work_items - 1 plus one full grid
    stride (at most 2^20 workgroups of 256 threads)."""
    src = tmp_path / "t.cpp"
    src.write_text(r"""
#include "ew_index.h"
#include <cstdio>
#include <initializer_list>
using namespace mfx;
int main() {
  const int64_t stride = kEwMaxBlocks * kEwThreads;           // 2^28
  const int64_t edge = (int64_t)INT32_MAX + 1 - stride;        // largest int-safe work_items
  int bad = 0;
  bad += ew_needs_wide_index(1000);
  bad += ew_needs_wide_index(edge);
  bad += !ew_needs_wide_index(edge + 1);
  bad += !ew_needs_wide_index((1LL << 31) - (1LL << 24));      // the old rule's blind spot
  bad += !ew_needs_wide_index(1LL << 40);
  // Brute force on small grids would take hours; check the arithmetic instead:
  // for every tested size, the last index the loop forms fits an int exactly
  // when the rule says so.
  for (int64_t w : {edge - 1, edge, edge + 1, (int64_t)INT32_MAX, (int64_t)1 << 30}) {
    const int64_t last = (w - 1) + ew_blocks(w) * kEwThreads;
    bad += (last > INT32_MAX) != ew_needs_wide_index(w);
  }
  bad += ew_blocks(0) != 1 || ew_blocks(1) != 1 || ew_blocks(257) != 2 || ew_blocks(1LL << 40) != kEwMaxBlocks;
  std::printf("%d\n", bad);
  return bad;
}
""")
    exe = tmp_path / "t"
    subprocess.run(["g++", "-std=c++17", "-I", str(REPO / "jax-mlx-plugin_amd/csrc/kernels"), str(src), "-o",
                    str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout


def test_structurally_invalid_modules_are_rejected(api):
    """Regression cases the sanitizer fuzz found (each used to read out of
    bounds in the rewriter or planner): the verifier rejects them with
    INVALID_ARGUMENT before either runs."""
    ln = M.layer_norm_module(shape=(4, 64, 128))
    # broadcast_in_dim whose dims list is shorter than the operand rank
    bad_bcast = ln.replace("dims = [0, 1]", "dims = [0]", 1)
    # a softmax body returning a value of another type than its signature
    dpa = M.dot_product_attention_module(B=1, T=64, N=4, H=64)
    bad_return = dpa.replace("return %13 : tensor<1x4x1x64x64xf32>", "return %1 : tensor<1x4x1x64x64xf32>")
    # a binary op with one operand
    bad_arity = dpa.replace("stablehlo.subtract %arg0, %6 :", "stablehlo.subtract %arg0:")
    for text, what in ((bad_bcast, "broadcast"), (bad_return, "func.call"), (bad_arity, "subtract")):
        assert text not in (ln, dpa), what
        with pytest.raises(pjrt.PjrtError) as e:
            api.inspect(text)
        assert e.value.code_name == "INVALID_ARGUMENT" and what in e.value.message, e.value.message


def test_transformer_plan(api):
    d = api.inspect(M.transformer_module(layers=2, B=2, T=64, d=128, heads=4, mlp=256))
    ops = [n["op"] for n in fused(d)]
    assert ops.count("mfx.layer_norm") == 4 and ops.count("mfx.sdpa") == 2
    s = steps(d)
    # every dot_general carries its bias / residual / GELU program as a fused epilogue
    assert s.count("gemm_ew") == 8 and s.count("sdpa") == 2 and s.count("layer_norm") == 4
    assert "gemm" not in s and "elementwise" not in s
    sd = [n for n in fused(d) if n["op"] == "mfx.sdpa"][0]
    assert sd["i:offsets"] == [0, 128, 256, 0]  # q, k, v read in place from the QKV projection


def test_sdpa_vjp_links_forward_and_backward(api):
    """jax.vjp of mlx_dot_product_attention in one module: the forward step
    also writes its row log-sum-exp and the backward reads it and the
    forward's output instead of recomputing them; a backward on another q
    value keeps its recompute."""
    d = api.inspect(M.sdpa_vjp_module())
    assert [s["label"] for s in d["plan"]["steps"]] == ["sdpa (+ lse)", "mfx.sdpa_bwd (forward's out and lse)"]
    d2 = api.inspect(M.sdpa_vjp_module(same_inputs=False))
    assert [s["label"] for s in d2["plan"]["steps"]] == ["sdpa", "mfx.sdpa_bwd"]
    # the recomputed output no longer needs workspace in the arena
    assert d["plan"]["arena_bytes"] < d2["plan"]["arena_bytes"]


def test_sdpa_vjp_two_cotangents_share_the_forward_lse(api):
    """Two backward steps of one forward (a VJP applied to two cotangents):
    the forward writes one lse value and both backward steps read that
    value (a second lse temp would be written by nobody)."""
    d = api.inspect(M.sdpa_vjp_module(cotangents=2))
    st = d["plan"]["steps"]
    assert [s["label"] for s in st] == ["sdpa (+ lse)"] + ["mfx.sdpa_bwd (forward's out and lse)"] * 2
    fw_out, lse = st[0]["writes"]
    for bw in st[1:]:
        assert fw_out in bw["reads"] and lse in bw["reads"]
    assert sum(lse in s["writes"] for s in st) == 1


@pytest.mark.parametrize("epilogue", ["bias", "bias_gelu", "bias_residual"])
def test_dense_epilogue_fuses_into_gemm(api, epilogue):
    """A dot_general whose only reader is one elementwise program at the
    product's own index runs as one fused GEMM launch."""
    d = api.inspect(M.dense_module(epilogue=epilogue))
    assert steps(d) == ["gemm_ew"]


@pytest.mark.parametrize("escape", ["result", "reader"])
def test_dense_epilogue_not_fused_when_product_escapes(api, escape):
    """The product stays materialised when it is also a result, or when a
    second program reads it."""
    s = steps(api.inspect(M.dense_module(epilogue="bias_gelu", escape=escape)))
    assert s[0] == "gemm" and "gemm_ew" not in s and s.count("elementwise") >= 1


def test_batched_dense_epilogue_fuses(api):
    """A batched dot_general ('bmk,bkn->bmn') with its bias + GELU consumer:
    one fused launch over batch * M rows."""
    assert steps(api.inspect(M.batched_dense_module())) == ["gemm_ew"]


def test_dense_epilogue_rules(api):
    """Products the f32 tile kernel does not take keep two steps: bf16
    operands, K not a multiple of 4, odd N."""
    for kw in (dict(dt="bf16"), dict(K=126), dict(N=191)):
        s = steps(api.inspect(M.dense_module(**kw)))
        assert s == ["gemm", "elementwise"], (kw, s)


def test_parse_errors(api):
    with pytest.raises(pjrt.PjrtError) as e:
        api.inspect("module { func.func @main() { stablehlo.while } }")
    assert e.value.code_name == "INVALID_ARGUMENT" and "while" in e.value.message
    with pytest.raises(pjrt.PjrtError):
        api.inspect("not mlir at all")
