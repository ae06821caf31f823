"""Per-tile time budget of the pipelined bf16 flash kernel on config 3, and
per-block budget of the SDPA backward's dK/dV kernel on the same shape.

    python jax-mlx-plugin_amd/build.py phase_timers
    python jax-mlx-plugin_amd/phase_budget.py [--json out.json]
    python jax-mlx-plugin_amd/phase_budget.py --kernel dkdv [--json out.json]
    python jax-mlx-plugin_amd/phase_budget.py --kernel decode [--json out.json]

Loads the diagnostic copy of libmfx_kernels.so built with -DMFX_PHASE_TIMERS
(jax_mlx_amd/lib/phase_timers/), runs causal bf16 SDPA on config 3's inputs
([4, 32, 2048, 128], numpy default_rng(3)), and reads the per-wavefront phase
records the kernel writes (sdpa_flash_bf16_pipe.hip, PhaseClock):

- the shader clock under this load (s_memtime cycles over s_memrealtime);
- cycles per 64-key tile and wavefront in each phase of the loop -- A: the S
  MFMAs of the next tile with the exp2 of this one, C: the row-sum check,
  B: the PV MFMAs with the next tile's exp2, S: barrier plus the next tiles'
  DMA issue -- against the MFMA floor (two wavefronts per SIMD, 32 MFMAs
  each per tile, 32 cycles per v_mfma_f32_32x32x16_bf16);
- per-block start (first tiles landed, loop entry), last tile and epilogue;
- SIMD occupancy over the kernel span and the spread between XCDs.

With --kernel dkdv it runs mfx_sdpa_bwd on the same inputs (upstream
gradient drawn fourth, from the forward's output and lse, as bench.py's
config3_sdpa_bwd `from_forward`) and reads the records of bwd_dkdv_mfma
(sdpa_bwd_mfma.hip): cycles per 32-query block and wavefront in its X phase
(the S and dP MFMAs), its Y | V phase (the previous block's dV and dK MFMAs
with this block's exp2 / dS work) and its barrier phase (per 64-query tile:
vmcnt wait, s_barrier, the next tile's DMA issue), against the MFMA floor
(one wavefront per SIMD, 32 MFMAs per block).

With --kernel decode it runs config 5 (GQA decode, q [16,32,1,128] bf16
with RMSNorm, k / v [16,8,8192,128], a length mask, all from
numpy.random.default_rng(5) in bench.py's order) and reads the records of
decode_mfma_kernel (sdpa_decode_mfma.hip): per wavefront, the time to find
its range of the tile lists, to issue its first tiles, until its first tile
and while it streams its tiles, and the spread between XCDs.

The instrumented kernels run a few percent slower than the shipped ones (a
handful of s_memtime reads per tile); shares of the budget are what it is for.
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB = PKG / "jax_mlx_amd" / "lib" / "phase_timers" / "libmfx_kernels.so"
RT_HZ = 100e6          # s_memrealtime frequency
MFMA_CYCLES = 32       # v_mfma_f32_32x32x16_bf16 issue-to-issue on one SIMD
MFMAS_PER_TILE = 32    # per wavefront and 64-key tile at d = 128: 16 for S, 16 for PV
WAVES_PER_SIMD = 2
FIELDS = 20             # u64 per wavefront record (PhaseClock, kPhaseFields)
BWD_FIELDS = 16         # u64 per dK/dV wavefront record (kBwdPhaseFields)
BWD_MFMAS_PER_BLOCK = 32  # S, dP, dV, dK: 8 each per 32-query block at d = 128
DEC_FIELDS = 12         # u64 per decode wavefront record (kDecPhaseFields)
DEC_TILE_BYTES = 2 * 32 * 128 * 2  # K and V of one 32-key tile at d = 128, bf16


def run(steps: int, lib_path: Path = LIB):
    import ctypes

    import torch

    sys.path.insert(0, str(PKG))
    from jax_mlx_amd import native

    lib = native.load(lib_path, make_default=True)
    lib.mfx_phase_timers_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int]
    lib.mfx_phase_timers_read.restype = ctypes.c_int64
    B, H, T, d = 4, 32, 2048, 128
    rng = np.random.default_rng(3)
    q, k, v = (torch.from_numpy(rng.standard_normal((B, H, T, d)).astype(np.float32)).cuda().bfloat16()
               for _ in range(3))
    out = torch.empty_like(q)
    call = lambda: native.sdpa(q, k, v, scale=d ** -0.5, causal=True, out=out)  # noqa: E731
    # Clocks rise under sustained load: 0.25 s of launches first.
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.25:
        for _ in range(10):
            call()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        call()
    e1.record()
    torch.cuda.synchronize()
    avg_us = e0.elapsed_time(e1) * 1e3 / steps
    cap = lib.mfx_phase_timers_read(None, 0, 1)   # clear
    call()
    n = 2048 * 4
    rec = np.zeros((n, FIELDS), dtype=np.uint64)
    got = lib.mfx_phase_timers_read(rec.ctypes.data, n, 0)
    if got < 0 or cap < n:
        raise RuntimeError("reading the phase records failed")
    return rec, avg_us


def occupancy(ids: np.ndarray, rt_start: np.ndarray, rt_end: np.ndarray):
    """Fraction of the span each SIMD holds 0 / 1 / 2 / 3+ wavefronts (from
    HW_ID's SIMD / CU / SA / SE fields and the XCC id), and each XCD's finish
    time after the first wavefront's start (us)."""
    t0 = rt_start.min()
    xcc = (ids & 0xff).astype(np.int64)
    hw = ((ids >> 8) & 0xffffffff).astype(np.int64)
    simd = (xcc << 16) | (((hw >> 13) & 7) << 12) | (((hw >> 12) & 1) << 11) | (((hw >> 8) & 15) << 4) | \
        ((hw >> 4) & 3)
    occ = np.zeros(4)
    for key in np.unique(simd):
        m = simd == key
        ev = sorted([(int(s), 1) for s in rt_start[m]] + [(int(e), -1) for e in rt_end[m]])
        cur, last = 0, int(t0)
        for tm, dlt in ev:
            occ[min(cur, 3)] += tm - last
            cur += dlt
            last = tm
        occ[0] += int(rt_end.max()) - last
    occ /= occ.sum()
    xcd_end = {int(x): (rt_end[xcc == x].max() - t0) / RT_HZ * 1e6 for x in np.unique(xcc)}
    return occ, xcd_end


def run_dkdv(steps: int, lib_path: Path = LIB):
    import ctypes

    import torch

    sys.path.insert(0, str(PKG))
    from jax_mlx_amd import native

    lib = native.load(lib_path, make_default=True)
    lib.mfx_bwd_phase_timers_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int]
    lib.mfx_bwd_phase_timers_read.restype = ctypes.c_int64
    B, H, T, d = 4, 32, 2048, 128
    rng = np.random.default_rng(3)
    q, k, v, g = (torch.from_numpy(rng.standard_normal((B, H, T, d)).astype(np.float32)).cuda().bfloat16()
                  for _ in range(4))
    lse = torch.empty(B * H * T, dtype=torch.float32, device="cuda")
    out = native.sdpa(q, k, v, causal=True, lse=lse)
    ws = torch.empty(native.sdpa_bwd_workspace_size(q, k, v, causal=True, fwd_out=out, fwd_lse=lse),
                     dtype=torch.uint8, device="cuda")
    call = lambda: native.sdpa_bwd(q, k, v, g, causal=True, workspace=ws, fwd_out=out, fwd_lse=lse)  # noqa: E731
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.25:
        call()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        call()
    e1.record()
    torch.cuda.synchronize()
    avg_us = e0.elapsed_time(e1) * 1e3 / steps
    cap = lib.mfx_bwd_phase_timers_read(None, 0, 1)   # clear
    call()
    n = B * H * (T // 128) * 4
    rec = np.zeros((n, BWD_FIELDS), dtype=np.uint64)
    got = lib.mfx_bwd_phase_timers_read(rec.ctypes.data, n, 0)
    if got < 0 or cap < n:
        raise RuntimeError("reading the phase records failed")
    return rec, avg_us


def budget_dkdv(rec: np.ndarray, avg_us: float) -> dict:
    rec = rec[rec[:, 3] != 0]
    if not len(rec):
        raise RuntimeError("no phase records written: the kernel that ran was not the phase-timer build")
    ids, rt_end = rec[:, 0], rec[:, 3].astype(np.int64)
    lo = lambda f: ((rec[:, 3] & 0xffffffff).astype(np.int64) - rec[:, f].astype(np.int64)) % (1 << 32)  # noqa
    rt_start = rt_end - lo(1)
    rt_loop = rt_end - lo(2)
    cyc = {name: rec[:, f].astype(np.float64) for name, f in
           (("X", 4), ("YV", 5), ("S", 6), ("S_vmwait", 7), ("S_barrier", 8), ("last", 9), ("total", 12),
            ("pre", 13), ("epi", 14))}
    blocks, edges, tiles = (rec[:, f].astype(np.float64) for f in (10, 11, 15))
    dur_s = (rt_end - rt_start) / RT_HZ
    clock_mhz = np.median(cyc["total"] / dur_s) / 1e6
    t0 = rt_start.min()
    span_us = (rt_end.max() - t0) / RT_HZ * 1e6
    nb = blocks.sum()
    per_block = {p: float(cyc[p].sum() / nb) for p in ("X", "YV", "S")}
    loop_block = sum(per_block.values())
    floor = BWD_MFMAS_PER_BLOCK * MFMA_CYCLES
    occ, xcd_end = occupancy(ids, rt_start, rt_end)
    us = lambda a: float(np.median(a) / RT_HZ * 1e6)  # noqa: E731
    return {
        "kernel": "bwd_dkdv_mfma<128, causal>",
        "mfx_sdpa_bwd_avg_us_instrumented": round(avg_us, 2),
        "dkdv_span_us": round(span_us, 2),
        "shader_clock_mhz": round(float(clock_mhz), 1),
        "wavefronts": int(len(rec)), "blocks": int(nb), "masked_blocks": int(edges.sum()), "tiles": int(tiles.sum()),
        "cycles_per_block_per_wavefront": {**{k: round(v, 1) for k, v in per_block.items()},
                                           "sum": round(loop_block, 1)},
        "barrier_phase_split_per_block": {
            "vmcnt_wait": round(float(cyc["S_vmwait"].sum() / nb), 1),
            "s_barrier": round(float(cyc["S_barrier"].sum() / nb), 1),
            "dma_issue": round(float((cyc["S"] - cyc["S_vmwait"] - cyc["S_barrier"]).sum() / nb), 1),
            "note": "one barrier per 64-query tile (two blocks)"},
        "mfma_floor_cycles_per_block_per_simd": floor,
        "loop_mfma_fraction": round(floor / loop_block, 4),
        "median_us_start_to_loop": round(us(rt_loop - rt_start), 3),
        "median_cycles_last_y": float(np.median(cyc["last"])),
        "median_cycles_epilogue": float(np.median(cyc["epi"])),
        "simd_occupancy_fraction_0_1_2_3plus_waves": [round(float(x), 4) for x in occ],
        "xcd_finish_us": {k: round(v, 2) for k, v in sorted(xcd_end.items())},
        "xcd_finish_spread_us": round(max(xcd_end.values()) - min(xcd_end.values()), 2),
        "share_of_wavefront_cycles": {
            p: round(float(cyc[p].sum() / cyc["total"].sum()), 4) for p in ("pre", "X", "YV", "S", "last", "epi")},
    }


def run_decode(steps: int, lib_path: Path = LIB):
    import ctypes

    import torch

    sys.path.insert(0, str(PKG))
    from jax_mlx_amd import native

    lib = native.load(lib_path, make_default=True)
    lib.mfx_decode_phase_timers_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int]
    lib.mfx_decode_phase_timers_read.restype = ctypes.c_int64
    rng = np.random.default_rng(5)
    B, Hq, Hkv, d, S = 16, 32, 8, 128, 8192
    draw = lambda shape: torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).cuda().bfloat16()  # noqa
    q = draw((B, Hq, 1, d))
    kvs = [(draw((B, Hkv, S, d)), draw((B, Hkv, S, d)))]
    lens = rng.integers(1024, 8192, size=B, endpoint=True)
    # a second K / V set, alternated as bench.py does, so no call finds its
    # K / V in the 256 MB Infinity Cache
    kvs.append((draw((B, Hkv, S, d)), draw((B, Hkv, S, d))))
    mask = torch.from_numpy(np.where(np.arange(S)[None] < lens[:, None], 0.0, -np.inf)
                            .reshape(B, 1, 1, S).astype(np.float32)).cuda()
    out = torch.empty_like(q)
    it = [0]

    def call():
        k, v = kvs[it[0] % 2]
        it[0] += 1
        native.sdpa(q, k, v, scale=d ** -0.5, mask=mask, q_rms_eps=1e-6, out=out)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.25:
        for _ in range(10):
            call()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        call()
    e1.record()
    torch.cuda.synchronize()
    avg_us = e0.elapsed_time(e1) * 1e3 / steps
    cap = lib.mfx_decode_phase_timers_read(None, 0, 1)   # clear
    call()
    n = 4096
    rec = np.zeros((n, DEC_FIELDS), dtype=np.uint64)
    got = lib.mfx_decode_phase_timers_read(rec.ctypes.data, n, 0)
    if got < 0 or cap < n:
        raise RuntimeError("reading the phase records failed")
    return rec, avg_us, int(lens.sum())


def budget_decode(rec: np.ndarray, avg_us: float, sum_len: int) -> dict:
    rec = rec[rec[:, 6] != 0]
    if not len(rec):
        raise RuntimeError("no phase records written: the kernel that ran was not the phase-timer build")
    ids, rt_end = rec[:, 0], rec[:, 6].astype(np.int64)
    back = lambda f: rt_end - ((rec[:, 6] & 0xffffffff).astype(np.int64) - rec[:, f].astype(np.int64)) % (1 << 32)  # noqa
    rt = {name: back(f) for name, f in (("start", 1), ("range", 2), ("issue", 3), ("first", 4), ("stream_end", 5))}
    tiles = rec[:, 7].astype(np.float64)
    t0 = rt["start"].min()
    span_us = (rt_end.max() - t0) / RT_HZ * 1e6
    us = lambda a: float(np.median(a) / RT_HZ * 1e6)  # noqa: E731
    stream_us = (rt["stream_end"] - rt["first"]) / RT_HZ * 1e6
    xcc = (ids & 0xff).astype(np.int64)
    xcd_stream = {int(x): round(float(np.median(stream_us[xcc == x])), 2) for x in np.unique(xcc)}
    xcd_end = {int(x): round(float((rt_end[xcc == x].max() - t0) / RT_HZ * 1e6), 2) for x in np.unique(xcc)}
    # aggregate rate while streaming: every tile's K / V bytes over the span
    # from the median first tile to the median stream end (the run alternates
    # two K / V sets, so these bytes come from HBM)
    stream_span_s = float(np.median(rt["stream_end"]) - np.median(rt["first"])) / RT_HZ
    clock_mhz = float(np.median(rec[:, 9].astype(np.float64) / ((rt_end - rt["start"]) / RT_HZ)) / 1e6)
    return {
        "kernel": "decode_mfma_kernel<128, f32 mask, shared rows>",
        "call_avg_us_instrumented": round(avg_us, 2),
        "main_kernel_span_us": round(span_us, 2),
        "shader_clock_mhz": round(clock_mhz, 1),
        "wavefronts": int(len(rec)), "tiles": int(tiles.sum()), "mean_tiles_per_wavefront": round(float(tiles.mean()), 2),
        "valid_kv_bytes": 2 * 8 * 128 * 2 * sum_len,
        "median_us": {
            "start_to_range": round(us(rt["range"] - rt["start"]), 3),
            "range_to_first_issue": round(us(rt["issue"] - rt["range"]), 3),
            "first_issue_to_first_tile": round(us(rt["first"] - rt["issue"]), 3),
            "streaming": round(float(np.median(stream_us)), 3),
            "stream_end_to_end": round(us(rt_end - rt["stream_end"]), 3),
            "start_to_end": round(us(rt_end - rt["start"]), 3),
            "last_end_after_first_start": round(span_us, 3)},
        "p10_p90_streaming_us": [round(float(np.percentile(stream_us, 10)), 2),
                                 round(float(np.percentile(stream_us, 90)), 2)],
        "tb_per_s_while_streaming": round(tiles.sum() * DEC_TILE_BYTES / stream_span_s / 1e12, 2),
        "xcd_median_streaming_us": xcd_stream,
        "xcd_finish_us": xcd_end,
        "xcd_finish_spread_us": round(max(xcd_end.values()) - min(xcd_end.values()), 2),
        "segments_per_wavefront_max": int(rec[:, 8].max()),
    }


def budget(rec: np.ndarray, avg_us: float) -> dict:
    rec = rec[rec[:, 4] != 0]
    if not len(rec):
        raise RuntimeError("no phase records written: the kernel that ran was not the phase-timer build")
    ids, rt_end = rec[:, 0], rec[:, 4].astype(np.int64)
    lo = lambda f: ((rec[:, 4] & 0xffffffff).astype(np.int64) - rec[:, f].astype(np.int64)) % (1 << 32)  # noqa
    rt_start = rt_end - lo(1)
    rt_ready = rt_end - lo(2)
    rt_loop = rt_end - lo(3)
    cyc = {name: rec[:, f].astype(np.float64) for name, f in
           (("A", 5), ("C", 6), ("B", 7), ("S", 8), ("last", 9), ("total", 12), ("pre", 13), ("epi", 15),
            ("S_vmwait", 16), ("S_barrier", 17), ("S_dma_k", 18))}
    tiles = rec[:, 10].astype(np.float64)
    rebases = int(rec[:, 11].sum())
    dur_s = (rt_end - rt_start) / RT_HZ
    clock_mhz = np.median(cyc["total"] / dur_s) / 1e6
    t0 = rt_start.min()
    span_us = (rt_end.max() - t0) / RT_HZ * 1e6
    per_tile = {p: float(cyc[p].sum() / tiles.sum()) for p in ("A", "C", "B", "S")}
    loop_tile = sum(per_tile.values())
    floor = MFMAS_PER_TILE * MFMA_CYCLES * WAVES_PER_SIMD
    occ, xcd_end = occupancy(ids, rt_start, rt_end)
    us = lambda a: float(np.median(a) / RT_HZ * 1e6)  # noqa: E731
    return {
        "kernel_avg_us_instrumented": round(avg_us, 2),
        "span_us": round(span_us, 2),
        "shader_clock_mhz": round(float(clock_mhz), 1),
        "wavefronts": int(len(rec)), "loop_tiles": int(tiles.sum()), "rebases": rebases,
        "cycles_per_tile_per_wavefront": {**{k: round(v, 1) for k, v in per_tile.items()},
                                          "sum": round(loop_tile, 1)},
        "barrier_phase_split_per_tile": {
            "vmcnt_wait": round(float(cyc["S_vmwait"].sum() / tiles.sum()), 1),
            "s_barrier": round(float(cyc["S_barrier"].sum() / tiles.sum()), 1),
            "dma_issue": round(float((cyc["S"] - cyc["S_vmwait"] - cyc["S_barrier"]).sum() / tiles.sum()), 1),
            "dma_issue_k_tile": round(float(cyc["S_dma_k"].sum() / tiles.sum()), 1),
            "note": "sums over every barrier a wavefront passes (loop tiles, its last tile, barrier-only "
                    "iterations) divided by its loop tiles"},
        "mfma_floor_cycles_per_tile_per_simd": floor,
        "loop_mfma_fraction": round(floor / loop_tile, 4),
        "median_us_start_to_first_tiles": round(us(rt_ready - rt_start), 3),
        "median_us_start_to_loop": round(us(rt_loop - rt_start), 3),
        "median_us_start_to_loop_first_blocks": round(us((rt_loop - rt_start)[rt_start - t0 < 2 * RT_HZ * 1e-6]), 3),
        "median_us_start_to_loop_later_blocks": round(us((rt_loop - rt_start)[rt_start - t0 >= 2 * RT_HZ * 1e-6]), 3),
        "median_cycles_last_tile": float(np.median(cyc["last"])),
        "median_cycles_epilogue": float(np.median(cyc["epi"])),
        "simd_occupancy_fraction_0_1_2_3plus_waves": [round(float(x), 4) for x in occ],
        "xcd_finish_us": {k: round(v, 2) for k, v in sorted(xcd_end.items())},
        "xcd_finish_spread_us": round(max(xcd_end.values()) - min(xcd_end.values()), 2),
        "share_of_wavefront_cycles": {
            p: round(float(cyc[p].sum() / cyc["total"].sum()), 4) for p in ("pre", "A", "C", "B", "S", "last", "epi")},
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--json", help="also write the budget here")
    ap.add_argument("--lib", type=Path, default=LIB, help="a phase-timer build of libmfx_kernels.so")
    ap.add_argument("--kernel", choices=("flash", "dkdv", "decode"), default="flash",
                    help="flash: the config-3 forward; dkdv: the backward's dK/dV kernel on the same shape; "
                         "decode: config 5's MFMA decode")
    args = ap.parse_args()
    if not args.lib.exists():
        print(f"{args.lib} is not built: python jax-mlx-plugin_amd/build.py phase_timers", file=sys.stderr)
        return 1
    if args.kernel == "dkdv":
        rec, avg_us = run_dkdv(args.steps, args.lib)
        b = budget_dkdv(rec, avg_us)
    elif args.kernel == "decode":
        rec, avg_us, sum_len = run_decode(args.steps, args.lib)
        b = budget_decode(rec, avg_us, sum_len)
    else:
        rec, avg_us = run(args.steps, args.lib)
        b = budget(rec, avg_us)
    print(json.dumps(b, indent=1))
    if args.json:
        Path(args.json).write_text(json.dumps(b, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
