"""Host-only sanitizer builds of the PJRT plugin's C++ (csrc/pjrt): test
infrastructure for tests/test_sanitizers.py, outside the product build.

The sources are compiled by g++ (host code; no GPU code is built with a
sanitizer) with AddressSanitizer and UndefinedBehaviorSanitizer, into
    jax-mlx-plugin_amd/_build/asan/inspect_driver       (driver + pipeline)
    jax-mlx-plugin_amd/_build/asan/libpjrt_mi355x.so    (the plugin library)
both linked against the regular libmfx_kernels.so.

    python tests/sanitize/build_sanitized.py
"""
from __future__ import annotations

import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO / "jax-mlx-plugin_amd"))
import build as pkg_build  # noqa: E402

FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
OUT = pkg_build.OBJ_DIR / "asan"


def _objects() -> list[Path]:
    obj_dir = OUT / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    srcs = sorted((pkg_build.CSRC / "pjrt").glob("*.cpp"))
    jobs = [(pkg_build._compile_host, s, obj_dir / (s.stem + ".o"), FLAGS + ["-fvisibility=hidden"]) for s in srcs]
    return pkg_build._parallel(jobs)


def _link(objs, extra, out: Path) -> Path:
    lib = pkg_build.LIB_DIR
    pkg_build._run(["g++", *FLAGS, *extra, *map(str, objs), f"-L{lib}", "-lmfx_kernels", "-L/opt/rocm/lib",
                    "-lamdhip64", f"-Wl,-rpath,{lib}", "-Wl,-rpath,/opt/rocm/lib", "-ldl", "-lpthread", "-o", str(out)])
    return out


def build() -> tuple[Path, Path]:
    objs = _objects()
    drv_obj = OUT / "obj" / "inspect_driver.o"
    pkg_build._compile_host(HERE / "inspect_driver.cpp", drv_obj, FLAGS)
    driver = _link(objs + [drv_obj], [], OUT / "inspect_driver")
    lib = _link(objs, ["-shared", "-fPIC"], OUT / "libpjrt_mi355x.so")
    return driver, lib


if __name__ == "__main__":
    for p in build():
        print(p)
