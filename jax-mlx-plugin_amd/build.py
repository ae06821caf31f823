"""Build recipe for the native libraries of the MI355X fused-path plugin.

    python jax-mlx-plugin_amd/build.py            # build everything
    python jax-mlx-plugin_amd/build.py kernels    # only libmfx_kernels.so
    python jax-mlx-plugin_amd/build.py phase_timers
        # diagnostic copy of libmfx_kernels.so whose pipelined bf16 flash
        # kernel records per-wavefront phase timings (-DMFX_PHASE_TIMERS),
        # in jax_mlx_amd/lib/phase_timers/; read by phase_budget.py

Outputs (in-tree, next to the Python package so they travel with the repo):
    jax_mlx_amd/lib/libmfx_kernels.so   hand-written gfx950 HIP kernels, C-ABI
    jax_mlx_amd/lib/libpjrt_mi355x.so   PJRT C-API plugin (exports GetPjrtApi)

Every HIP translation unit is compiled for gfx950 only, with packed-fp32
instruction selection disabled (-packed-fp32-ops).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
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


# Kernels whose LDS operand reads are inline asm: the asm statement returns
# before the data arrives (an lgkmcnt wait later ties the registers), so a
# VGPR spill or scratch copy of such a destination would store it early and
# silently corrupt results.  Their build fails if the compiler spills.
NO_SPILL_FILES = {"sdpa_flash_bf16_pipe.hip", "sdpa_flash_pipe_wide.hip", "sdpa_bwd_mfma.hip",
                  "sdpa_decode_mfma.hip", "sdpa_decode_mfma_wide.hip", "gemm16.hip"}
_RESOURCE_REMARK = "-Rpass-analysis=kernel-resource-usage"


def _check_no_spill(src: Path, remarks: str) -> None:
    kernel = "?"
    bad = []
    for line in remarks.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            kernel = m.group(1)
            continue
        m = re.search(r"remark:\s+(VGPRs Spill|ScratchSize \[bytes/lane\]): (\d+)", line)
        if m and int(m.group(2)) > 0:
            bad.append(f"{kernel}: {m.group(1)} {m.group(2)}")
    if bad:
        raise RuntimeError(f"{src.name}: VGPR spills in a kernel with inline-asm LDS reads:\n" + "\n".join(bad))


# LDS-wait check of the same kernels, on their gfx950 assembly (built here
# from source): the compiler's wait insertion does not see loads issued from
# inline asm, so nothing but the code's own lgkmcnt waits keeps a later
# instruction from reading (or a VALU write from clobbering) an LDS read's
# destination before the data arrives.  Per kernel, a dataflow over the basic
# blocks tracks the LDS / scalar-memory operations in flight: LDS operations
# complete in issue order, scalar loads in any order, so `s_waitcnt
# lgkmcnt(N)` is taken to retire the scalar loads first and then the oldest
# LDS operations until N remain.  At a block with
# several predecessors the in-flight lists are aligned from the newest and
# merged register by register.  Any access to a register an LDS read still
# owes is an error, except a later LDS read into it (it completes after).
_VREG = re.compile(r"\b([va])(?:(\d+)|\[(\d+):(\d+)\])")
_LGKM_MAX = 15
_LGKM_SMEM = ("s_load", "s_buffer_load", "s_memtime", "s_memrealtime", "s_sendmsg")


def _vregs(text: str) -> set:
    out = set()
    for m in _VREG.finditer(text):
        if m.group(2) is not None:
            out.add((m.group(1), int(m.group(2))))
        else:
            out.update((m.group(1), r) for r in range(int(m.group(3)), int(m.group(4)) + 1))
    return out


def _lgkm_wait(ins: str):
    m = re.search(r"lgkmcnt\((\d+)\)", ins)
    if m:
        return int(m.group(1))
    m = re.match(r"s_waitcnt\s+(0x[0-9a-fA-F]+|\d+)\s*$", ins)
    if m:
        c = (int(m.group(1), 0) >> 8) & 0xF
        return None if c == 0xF else c
    return None


def _retire(fl: list, keep: int) -> None:
    # what `s_waitcnt lgkmcnt(keep)` guarantees (and what the 4-bit counter
    # forces before an issue past 15 in flight): scalar loads retire first,
    # then LDS operations oldest first
    while len(fl) > keep:
        fl.pop(next((j for j, e in enumerate(fl) if e[0] and not e[1]), 0))


def _merge_inflight(a: tuple, b: tuple) -> tuple:
    n = max(len(a), len(b))
    pad = ((False, frozenset()),)
    a = pad * (n - len(a)) + a
    b = pad * (n - len(b)) + b
    return tuple((x[0] or y[0], x[1] | y[1]) for x, y in zip(a, b))


def _lds_wait_errors(lines: list) -> list:
    blocks = [[None, []]]
    for ln, text in lines:
        code = text.split(";")[0].rstrip()
        if not code.strip():
            continue
        m = re.match(r"^(\.LBB\d+_\d+):", code)
        if m:
            blocks.append([m.group(1), []])
            continue
        ins = code.strip()
        if not ins.startswith("."):
            blocks[-1][1].append((ln, ins))
    label_of = {b[0]: i for i, b in enumerate(blocks) if b[0]}
    errors = []
    state_in = {0: ()}
    work = [0]

    def reach(j: int, state: tuple) -> None:
        merged = state if j not in state_in else _merge_inflight(state_in[j], state)
        if state_in.get(j) != merged:
            state_in[j] = merged
            work.append(j)

    while work:
        i = work.pop()
        fl = list(state_in[i])
        falls_through = True
        for ln, ins in blocks[i][1]:
            mn = ins.split()[0]
            if mn == "s_waitcnt":
                w = _lgkm_wait(ins)
                if w is not None:
                    _retire(fl, w)
                continue
            if mn == "s_branch" or mn.startswith("s_cbranch"):
                if ins.split()[-1] in label_of:
                    reach(label_of[ins.split()[-1]], tuple(fl))
                if mn == "s_branch":
                    falls_through = False
                    break
                continue
            if mn == "s_endpgm":
                falls_through = False
                break
            owed = set().union(*(e[1] for e in fl)) if fl else set()
            ops = ins[len(mn):]
            if mn.startswith("ds_"):
                parts = ops.split(",")
                dest_read = any(t in mn for t in ("read", "load", "_rtn", "permute", "swizzle", "append", "consume"))
                dest = _vregs(parts[0]) if dest_read else set()
                src = _vregs(",".join(parts[1:])) if dest_read else _vregs(ops)
                if src & owed:
                    errors.append(f"line {ln}: {ins}")
                _retire(fl, _LGKM_MAX - 1)
                fl.append((False, frozenset(dest)))
            elif mn.startswith(_LGKM_SMEM):
                _retire(fl, _LGKM_MAX - 1)
                fl.append((True, frozenset()))
            elif _vregs(ops) & owed:
                errors.append(f"line {ln}: {ins}")
        if falls_through and i + 1 < len(blocks):
            reach(i + 1, tuple(fl))
    return sorted(set(errors), key=lambda e: int(e.split()[1].rstrip(":")))


def _check_lds_waits(src: Path, asm: str) -> None:
    bad = []
    name, body = None, []
    for ln, text in enumerate(asm.splitlines(), 1):
        m = re.match(r"^(_Z\S+):", text)
        if m:
            name, body = m.group(1), []
            continue
        if name and text.startswith(".Lfunc_end"):
            bad += [f"{name}: {e}" for e in _lds_wait_errors(body)]
            name = None
        elif name:
            body.append((ln, text))
    if bad:
        raise RuntimeError(f"{src.name}: registers read before their LDS data arrives:\n" + "\n".join(bad[:20]))


def _compile_hip(src: Path, obj: Path) -> Path:
    cmd = [HIPCC, *HIP_FLAGS, f"-I{obj.parent}", *HIP_FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if src.name not in NO_SPILL_FILES:
        _run(cmd)
        return obj
    asm = obj.with_suffix(".s")
    asm_cmd = [HIPCC, *HIP_FLAGS, f"-I{obj.parent}", *HIP_FILE_FLAGS.get(src.name, []), "--cuda-device-only", "-S",
               str(src), "-o", str(asm)]
    asm_proc = subprocess.Popen(asm_cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    proc = subprocess.run([*cmd, _RESOURCE_REMARK], capture_output=True, text=True)
    asm_out = asm_proc.communicate()[0]
    out = proc.stdout + proc.stderr
    if proc.returncode != 0:
        lines = [l for l in out.splitlines() if "packed-fp32-ops" not in l and "remark:" not in l]
        raise RuntimeError("command failed: " + " ".join(cmd) + "\n" + "\n".join(lines))
    _check_no_spill(src, out)
    if asm_proc.returncode != 0:
        raise RuntimeError("command failed: " + " ".join(asm_cmd) + "\n" + asm_out)
    _check_lds_waits(src, asm.read_text())
    return obj


# Headers whose text the library compiles again at run time with hipRTC
# (gemm_jit.cpp): each becomes a generated .inc defining a NUL-terminated
# char array with the header's bytes.
EMBEDDED_HEADERS = {"gemm_f32_tile.h": "kGemmTileSrc", "ew_math.h": "kEwMathSrc"}


def _embed_headers(src_dir: Path, obj_dir: Path) -> None:
    for name, symbol in EMBEDDED_HEADERS.items():
        data = (src_dir / name).read_bytes()
        rows = [", ".join(f"0x{b:02x}" for b in data[i:i + 16]) for i in range(0, len(data), 16)]
        text = (f"// Generated by build.py from {name}; do not edit.\n"
                f"static const char {symbol}[] = {{\n" + ",\n".join(rows) + ",\n0x00};\n")
        out = obj_dir / (Path(name).stem + "_src.inc")
        if not out.exists() or out.read_text() != text:
            out.write_text(text)


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
    _embed_headers(src_dir, obj_dir)
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


PHASE_TIMER_FILES = {"sdpa_flash_bf16_pipe.hip", "sdpa_bwd_mfma.hip", "sdpa_decode_mfma.hip"}


def build_phase_timers() -> Path:
    """libmfx_kernels.so with -DMFX_PHASE_TIMERS on PHASE_TIMER_FILES, linked
    from the regular objects otherwise (built first when missing)."""
    src_dir = CSRC / "kernels"
    obj_dir = OBJ_DIR / "kernels"
    if not (LIB_DIR / "libmfx_kernels.so").exists() or not obj_dir.exists():
        build_kernels()
    t_dir = OBJ_DIR / "kernels_phase_timers"
    t_dir.mkdir(parents=True, exist_ok=True)
    objs = []
    for src in sorted(src_dir.glob("*.hip")) + sorted(src_dir.glob("*.cpp")):
        if src.name in PHASE_TIMER_FILES:
            obj = t_dir / (src.stem + ".o")
            cmd = [HIPCC, *HIP_FLAGS, "-DMFX_PHASE_TIMERS", f"-I{obj_dir}", *HIP_FILE_FLAGS.get(src.name, []),
                   "-c", str(src), "-o", str(obj)]
            proc = subprocess.run([*cmd, _RESOURCE_REMARK], capture_output=True, text=True)
            if proc.returncode != 0:
                raise RuntimeError("command failed: " + " ".join(cmd) + "\n" + proc.stdout + proc.stderr)
            _check_no_spill(src, proc.stdout + proc.stderr)
            objs.append(obj)
        else:
            objs.append(obj_dir / (src.stem + ".o"))
    out_dir = LIB_DIR / "phase_timers"
    out_dir.mkdir(parents=True, exist_ok=True)
    out = out_dir / "libmfx_kernels.so"
    tmp = out.with_suffix(".so.tmp")
    vscript = t_dir / "exports.map"
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
    if "phase_timers" in targets:
        built.append(build_phase_timers())
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
