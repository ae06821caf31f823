"""Host-side checks of phase_budget.py's arithmetic (the per-tile / per-block
budgets read from the phase-timer build's records) on synthetic records."""
import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "jax-mlx-plugin_amd"))
import phase_budget as pb  # noqa: E402

RT = pb.RT_HZ


def _ids(xcc, simd, cu):
    # HW_ID: SIMD at bits 4-5, CU at bits 8-11 (SA bit 12, SE bits 13-15 left 0)
    hw = (simd << 4) | (cu << 8)
    return np.uint64(xcc | (hw << 8))


def _dkdv_records():
    # two wavefronts on one SIMD of XCD 0, back to back in time, and one on
    # XCD 1; realtime end stamps cross a 32-bit wrap of the low words
    base = (1 << 32) - 50
    rows = []
    for xcc, start, end, x, yv, s in ((0, 0, 1000, 700, 1300, 500), (0, 1000, 2000, 800, 1200, 400),
                                     (1, 0, 1500, 750, 1250, 450)):
        r = np.zeros(pb.BWD_FIELDS, dtype=np.uint64)
        r[0] = _ids(xcc, 0, 0)
        rt_start, rt_end = base + start, base + end
        r[1] = rt_start & 0xffffffff
        r[2] = (rt_start + 100) & 0xffffffff        # loop entry 1 us after the start
        r[3] = rt_end
        blocks = 10
        r[4], r[5], r[6] = x * blocks, yv * blocks, s * blocks
        r[7], r[8] = 10 * blocks, 20 * blocks      # vmcnt wait, s_barrier
        r[10], r[11], r[15] = blocks, 2, blocks // 2
        r[12] = (end - start) * 24                 # 2.4 GHz: 24 cycles per 100 MHz tick
        r[13], r[14], r[9] = 2000, 3000, 600
        rows.append(r)
    return np.stack(rows)


def test_dkdv_budget_per_block_and_clock():
    b = pb.budget_dkdv(_dkdv_records(), avg_us=500.0)
    per = b["cycles_per_block_per_wavefront"]
    assert per["X"] == pytest.approx(750.0) and per["YV"] == pytest.approx(1250.0) and per["S"] == pytest.approx(450.0)
    assert per["sum"] == pytest.approx(2450.0)
    assert b["loop_mfma_fraction"] == pytest.approx(32 * 32 / 2450.0, abs=1e-4)
    split = b["barrier_phase_split_per_block"]
    assert split["vmcnt_wait"] == 10.0 and split["s_barrier"] == 20.0 and split["dma_issue"] == 420.0
    assert b["shader_clock_mhz"] == pytest.approx(2400.0)
    assert b["blocks"] == 30 and b["masked_blocks"] == 6 and b["tiles"] == 15
    # span: first start to last end across the wrap, in us
    assert b["dkdv_span_us"] == pytest.approx(2000 / RT * 1e6)
    assert b["median_us_start_to_loop"] == pytest.approx(100 / RT * 1e6)


def test_occupancy_counts_waves_per_simd():
    rec = _dkdv_records()
    rt_end = rec[:, 3].astype(np.int64)
    rt_start = rt_end - ((rec[:, 3] & 0xffffffff).astype(np.int64) - rec[:, 1].astype(np.int64)) % (1 << 32)
    occ, xcd_end = pb.occupancy(rec[:, 0], rt_start, rt_end)
    # two SIMDs over a 2000-tick span: XCD 0's SIMD holds one wave throughout;
    # XCD 1's holds one for 1500 ticks and none for 500
    assert occ[1] == pytest.approx(3500 / 4000) and occ[0] == pytest.approx(500 / 4000)
    assert occ[2] == 0 and occ[3] == 0
    assert xcd_end[0] == pytest.approx(2000 / RT * 1e6) and xcd_end[1] == pytest.approx(1500 / RT * 1e6)


def test_dkdv_budget_rejects_empty_records():
    with pytest.raises(RuntimeError, match="phase-timer build"):
        pb.budget_dkdv(np.zeros((4, pb.BWD_FIELDS), dtype=np.uint64), 1.0)


def test_decode_budget_medians_and_rates():
    """Three wavefronts on two XCDs: per-phase medians from the realtime
    stamps (low words rebuilt against the 64-bit end), tiles and the
    streaming rate over the median streaming span."""
    base = (1 << 32) - 30
    rows = []
    # (xcc, start, range, issue, first, stream_end, end, tiles)
    for xcc, st, rg, iss, fi, se, en, t in ((0, 0, 200, 300, 450, 4450, 4500, 20), (0, 10, 210, 320, 460, 4460, 4520, 20),
                                            (1, 0, 250, 350, 500, 5000, 5050, 22)):
        r = np.zeros(pb.DEC_FIELDS, dtype=np.uint64)
        r[0] = _ids(xcc, 0, 0)
        for f, v in ((1, st), (2, rg), (3, iss), (4, fi), (5, se)):
            r[f] = (base + v) & 0xffffffff
        r[6] = base + en
        r[7], r[8] = t, 1
        r[9] = (en - st) * 20                         # 2.0 GHz
        rows.append(r)
    b = pb.budget_decode(np.stack(rows), avg_us=70.0, sum_len=1000)
    m = b["median_us"]
    tick = 1e6 / RT
    assert m["start_to_range"] == pytest.approx(200 * tick)
    assert m["range_to_first_issue"] == pytest.approx(100 * tick)      # 100, 110, 100
    assert m["first_issue_to_first_tile"] == pytest.approx(150 * tick)  # 150, 140, 150
    assert m["streaming"] == pytest.approx(4000 * tick)
    assert b["tiles"] == 62 and b["shader_clock_mhz"] == pytest.approx(2000.0)
    assert b["main_kernel_span_us"] == pytest.approx(5050 * tick)
    # 62 tiles x 16 KB over the median first-tile-to-stream-end span
    span_s = (4460 - 460) / RT
    assert b["tb_per_s_while_streaming"] == pytest.approx(round(62 * pb.DEC_TILE_BYTES / span_s / 1e12, 2))
    assert b["xcd_finish_spread_us"] == pytest.approx(round((5050 - 4520) * tick, 2))
