"""Build recipe for the native libraries of the MI355X fused-path plugin.

    python jax-mlx-plugin_amd/build.py            # build everything
    python jax-mlx-plugin_amd/build.py kernels    # only libmfx_kernels.so

Outputs (in-tree, next to the Python package so they travel with the repo):
    jax_mlx_amd/lib/libmfx_kernels.so   hand-written gfx950 HIP kernels, C-ABI
    jax_mlx_amd/lib/libpjrt_mi355x.so   PJRT C-API plugin (exports GetPjrtApi)

Every HIP translation unit is compiled for gfx950 only, with packed-fp32
instruction selection disabled (-packed-fp32-ops).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO / "include"
LIB_DIR = PKG_DIR / "jax_mlx_amd" / "lib"
OBJ_DIR = PKG_DIR / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]
HOST_CXX_FLAGS = [
    "-O2",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wextra",
    "-Wno-unused-parameter",
    "-D__HIP_PLATFORM_AMD__",
    "-I/opt/rocm/include",
    f"-I{INCLUDE}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = (proc.stdout + proc.stderr).strip()
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    lines = [l for l in out.splitlines() if "packed-fp32-ops" not in l]
    if proc.returncode != 0:
        raise RuntimeError("command failed: " + " ".join(cmd) + "\n" + "\n".join(lines))
    if lines:
        print("\n".join(lines), file=sys.stderr)


# Per-file code-generation options.  sdpa_flash_f32.hip: MFMA accumulators in
# VGPRs rather than AGPRs (its kernels read every accumulator back into VALU
# work -- softmax, rescale, merge -- and the AGPR form adds a move per read).
HIP_FILE_FLAGS = {
    "sdpa_flash_f32.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile_hip(src: Path, obj: Path) -> Path:
    _run([HIPCC, *HIP_FLAGS, *HIP_FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)])
    return obj


def _compile_host(src: Path, obj: Path, extra: list[str]) -> Path:
    _run(["g++", *HOST_CXX_FLAGS, *extra, "-c", str(src), "-o", str(obj)])
    return obj


def _parallel(jobs):
    workers = min(8, max(1, os.cpu_count() or 1))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        futs = [ex.submit(fn, *args) for fn, *args in jobs]
        return [f.result() for f in futs]


def build_kernels() -> Path:
    src_dir = CSRC / "kernels"
    obj_dir = OBJ_DIR / "kernels"
    obj_dir.mkdir(parents=True, exist_ok=True)
    jobs = []
    for src in sorted(src_dir.glob("*.hip")) + sorted(src_dir.glob("*.cpp")):
        jobs.append((_compile_hip, src, obj_dir / (src.stem + ".o")))
    objs = _parallel(jobs)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    out = LIB_DIR / "libmfx_kernels.so"
    tmp = out.with_suffix(".so.tmp")
    vscript = obj_dir / "exports.map"
    vscript.write_text("{ global: mfx_*; local: *; };\n")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs),
          f"-Wl,--version-script={vscript}", "-L/opt/rocm/lib", "-lrocblas", "-lhiprtc",
          "-Wl,-rpath,/opt/rocm/lib", "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_pjrt() -> Path | None:
    src_dir = CSRC / "pjrt"
    srcs = sorted(src_dir.glob("*.cpp"))
    if not srcs:
        return None
    obj_dir = OBJ_DIR / "pjrt"
    obj_dir.mkdir(parents=True, exist_ok=True)
    jobs = [(_compile_host, s, obj_dir / (s.stem + ".o"), ["-fvisibility=hidden"]) for s in srcs]
    objs = _parallel(jobs)
    out = LIB_DIR / "libpjrt_mi355x.so"
    tmp = out.with_suffix(".so.tmp")
    _run(["g++", "-shared", "-fPIC", *map(str, objs), f"-L{LIB_DIR}", "-lmfx_kernels",
          "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath,/opt/rocm/lib",
          "-ldl", "-lpthread", "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build(targets: list[str] | None = None) -> list[Path]:
    targets = targets or ["kernels", "pjrt"]
    built = []
    if "kernels" in targets:
        built.append(build_kernels())
    if "pjrt" in targets:
        p = build_pjrt()
        if p:
            built.append(p)
    return built


def clean() -> None:
    shutil.rmtree(OBJ_DIR, ignore_errors=True)


if __name__ == "__main__":
    args = sys.argv[1:]
    if args == ["clean"]:
        clean()
    else:
        for p in build(args or None):
            print(p)
