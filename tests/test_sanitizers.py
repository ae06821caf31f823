"""The PJRT plugin's host C++ (parser, verifier, rewriter, planner, C API)
under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

1. A driver runs the compile pipeline (mfx_pjrt_inspect) over every module
   form of tests/mlir_modules.py and over a few thousand mutated copies
   (byte flips, deleted / duplicated spans, truncation, extreme numbers,
   swapped lines): each input must be accepted or rejected with an error, and
   no sanitizer may report (a report aborts the driver; leaks are checked at
   exit).
2. The CPU PJRT tests run again against the sanitized plugin library with
   the ASan / UBSan runtimes preloaded.

The builds are host-only g++ builds (tests/sanitize/build_sanitized.py); no
GPU code is compiled with a sanitizer."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

import mlir_modules as M

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO / "tests" / "sanitize"))


@pytest.fixture(scope="module")
def sanitized():
    import build_sanitized

    return build_sanitized.build()


def module_texts():
    return {
        "ln_var": M.layer_norm_module(shape=(4, 64, 128)),
        "ln_std": M.layer_norm_module(shape=(4, 64, 128), form="standardize"),
        "ln_flax": M.layer_norm_module(shape=(4, 64, 128), dt="bf16", form="flax"),
        "ln_escape": M.layer_norm_escape_module(),
        "rms": M.rms_norm_module(),
        "rms_upcast": M.rms_norm_module(dt="bf16", upcast=True),
        "softmax": M.softmax_module(),
        "log_softmax": M.log_softmax_module(),
        "sigmoid_silu": M.sigmoid_silu_module(),
        "sdpa": M.sdpa_bhtd_module(B=1, H=2, T=64),
        "sdpa_causal": M.sdpa_bhtd_module(B=1, H=2, T=64, D=128, dt="bf16", causal=True),
        "sdpa_transposed_k": M.sdpa_bhtd_module(B=1, H=2, T=64, transposed_k=True, inline_softmax=True),
        "sdpa_probs": M.sdpa_bhtd_module(B=1, H=2, T=64, return_probs=True),
        "dpa": M.dot_product_attention_module(B=1, T=64, N=4, H=64),
        "dpa_gqa_bias": M.dot_product_attention_module(B=1, T=64, N=8, K=2, H=64, is_causal=False, bias=True),
        "gqa_decode": M.gqa_decode_module(B=2, Hq=8, Hkv=2, S=256),
        "cc_sdpa": M.custom_call_sdpa_module(),
        "cc_layer_norm": M.custom_call_layer_norm_module(),
        "cc_sdpa_bwd": M.custom_call_sdpa_bwd_module(),
        "cc_layer_norm_bwd": M.custom_call_layer_norm_bwd_module(),
        "elementwise": M.elementwise_mix_module(),
        "transformer": M.transformer_module(layers=1, B=2, T=64, d=128, heads=4, mlp=256),
    }


def env_for_sanitizers():
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=1:allocator_may_return_null=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1"
    return env


@pytest.mark.parametrize("seed", [101, 202, 303])
def test_inspect_pipeline_fuzz(sanitized, tmp_path, seed):
    driver, _ = sanitized
    files = []
    for name, text in module_texts().items():
        f = tmp_path / f"{name}.mlir"
        f.write_text(text)
        files.append(str(f))
    env = env_for_sanitizers()
    env["INSPECT_LAST_INPUT"] = str(tmp_path / "last_input.mlir")
    r = subprocess.run([str(driver), str(seed), "120", *files], capture_output=True, text=True, env=env,
                       timeout=600)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    total, accepted = (int(x) for x in r.stdout.split()[1::2])
    assert total == len(files) * 121 and accepted >= len(files)


def test_pjrt_cpu_tests_under_sanitizers(sanitized):
    _, lib = sanitized
    preload = " ".join(subprocess.run(["gcc", f"-print-file-name={n}"], capture_output=True, text=True,
                                      check=True).stdout.strip() for n in ("libasan.so", "libubsan.so"))
    env = env_for_sanitizers()
    # CPython itself leaks at exit; the driver above checks the plugin's leaks.
    env["ASAN_OPTIONS"] = "detect_leaks=0:verify_asan_link_order=0"
    env["LD_PRELOAD"] = preload
    env["MFX_PJRT_LIB"] = str(lib)
    check = ("import os, sys; sys.path[:0] = ['jax-mlx-plugin_amd']; from jax_mlx_amd import pjrt; "
             "assert pjrt.Api().lib._name == os.environ['MFX_PJRT_LIB']")
    subprocess.run([sys.executable, "-c", check], cwd=REPO, env=env, check=True, timeout=300)
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "tests/test_pjrt_cpu.py",
                        "tests/test_jax_package.py"], cwd=REPO, env=env, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
