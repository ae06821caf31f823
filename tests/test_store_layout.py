"""Host-side model of the staged output stores: a wavefront's MFMA
accumulators hold, per lane (l32, half), elements dt*32 + g*8 + half*4 + e
of row l32 (e < 4), and the kernels write them into LDS in XOR-swizzled
16-byte chunks, then read them back row-contiguous so that each store
instruction writes whole rows:

- the pipelined flash kernel (sdpa_flash_bf16_pipe.hip): 32 rows of DV bf16
  per wavefront, chunk c of row r at slot c ^ (r & SWZ), SWZ 3 / 7 / 15 for
  4 / 8 / 12 / 16 chunks per row (a permutation inside each group of SWZ + 1
  chunks, so 12-chunk rows stay inside the row), 64 // CPR rows per store
  instruction with the lanes past RPS * CPR idle;
- store_rows_lds (sdpa_elem.h; the backward's gradients and the
  per-element-mask kernel): D = 64 or 128, slot c ^ (r % CPR);
- the 16-bit tile GEMM (gemm16.hip): a wavefront's 64 x 64 block, 8 chunks
  per row, slot c ^ (r & 7), 8 rows per store instruction.

For every layout the model asserts that the writes cover each (row,
feature) exactly once inside the wavefront's region, that each store
instruction's lanes read exactly what was written for the (row, chunk)
they store, every output element exactly once, and that the write and read
instructions meet at most `max_ways` lanes on one 4-byte LDS bank (64
banks).  CPU only: no kernel runs."""
import collections

import pytest


def _writes(rows, width, swz, blocks_m=1):
    """LDS element index -> (row, feature) written by the accumulator lanes:
    rows `rows` per 32-row block (blocks_m blocks of 32 rows), `width`
    features, chunk c of row r at slot c ^ (r & swz)."""
    lds, banks = {}, []
    for i in range(blocks_m):
        for dt in range(width // 32):
            for g in range(4):
                inst = collections.Counter()
                for half in range(2):
                    for l32 in range(32):
                        r = i * 32 + l32
                        c = dt * 4 + g
                        slot = c ^ (r & swz)
                        assert 0 <= slot < width // 8
                        for e in range(4):
                            idx = r * width + slot * 8 + half * 4 + e
                            assert idx not in lds
                            lds[idx] = (r, dt * 32 + g * 8 + half * 4 + e)
                        # 8 bytes per lane: two 4-byte words
                        w0 = (r * width + slot * 8 + half * 4) // 2
                        inst[w0 % 64] += 1
                        inst[(w0 + 1) % 64] += 1
                banks.append(max(inst.values()))
    assert len(lds) == rows * width
    return lds, max(banks)


def _reads(lds, rows, width, swz):
    """Checks the row-contiguous reads; returns the worst bank multiplicity."""
    cpr = width // 8
    rps = 64 // cpr
    seen, worst = set(), 0
    for k in range((rows + rps - 1) // rps):
        inst = collections.Counter()
        for lane in range(64):
            r, c = k * rps + lane // cpr, lane % cpr
            if lane >= rps * cpr or r >= rows:
                continue
            slot = c ^ (r & swz)
            for e in range(8):
                assert lds[r * width + slot * 8 + e] == (r, c * 8 + e)
                seen.add((r, c * 8 + e))
            w0 = (r * width + slot * 8) // 2
            for q in range(4):
                inst[(w0 + q) % 64] += 1
        worst = max(worst, max(inst.values()))
    assert len(seen) == rows * width
    return worst


@pytest.mark.parametrize("dv", [32, 64, 96, 128])
def test_pipelined_flash_epilogue(dv):
    cpr = dv // 8
    swz = 15 if cpr % 16 == 0 else 7 if cpr % 8 == 0 else 3
    lds, wmax = _writes(32, dv, swz)
    rmax = _reads(lds, 32, dv, swz)
    # the wavefront's 32 x DV region fits its quarter of the two K stages
    # (2 x 64 x D elements, D = 64 for DV <= 64, else 128)
    d = 64 if dv <= 64 else 128
    assert 4 * 32 * dv <= 2 * 64 * d
    assert wmax <= 8 and rmax <= 4, (wmax, rmax)


@pytest.mark.parametrize("d", [64, 128])
def test_store_rows_lds(d):
    swz = d // 8 - 1
    lds, wmax = _writes(32, d, swz)
    rmax = _reads(lds, 32, d, swz)
    assert wmax <= 8 and rmax <= 4, (wmax, rmax)


def test_gemm16_block():
    lds, wmax = _writes(64, 64, 7, blocks_m=2)
    rmax = _reads(lds, 64, 64, 7)
    assert wmax <= 8 and rmax <= 4, (wmax, rmax)


def test_model_catches_an_unswizzled_layout():
    """Without the XOR the 8-byte writes of 32 rows land on the same banks:
    the model's bank count sees it."""
    _, wmax = _writes(32, 128, 0)
    assert wmax >= 16
