"""Host-side model of the K / V tile loads of the bf16 / f16 attention
kernels: `tiles::TileLoader` (jax-mlx-plugin_amd/csrc/kernels/sdpa_tiles.h),
as the MFMA decode (32-key tiles, one wavefront), the per-element-mask flash
kernel and the backward (64-row tiles, four wavefronts) use it, and the
pipelined prefill's `Loader` (sdpa_flash_bf16_pipe.hip), whose addresses are
TileLoader's with one offset per lane (64-key tiles, four wavefronts).

For every (batch, kv head), tile, wavefront, lane and load instruction the
model forms the per-lane byte offset the kernel forms (swizzled 16-byte
chunks, instruction and tile steps, all in the range-checked per-lane
offset) and the resource extent, applies the raw-buffer range check, and
asserts

- every load that returns memory reads 16 bytes inside the tensor, also for
  the last head of a row that interleaves heads (BTNH) when rows load wider
  than the head (head sizes 32 and 96 on 64- / 128-wide tiles);
- every (key, feature) the MFMAs consume (key < Tk, feature < head size)
  comes from exactly that element;
- every row past Tk reads as zero (V rows there meet P = 0, and 0 * NaN
  would not be 0).

`test_model_catches_tensor_end` runs the model on the earlier extent (Tk
rows of the row stride from the head's first element) and shows the last
head's tile-wide last row reading past the tensor.  CPU only: no kernel
runs."""
import numpy as np
import pytest


def _swz(D, r):
    if D >= 128:
        return (r & 3) | (((r ^ (r >> 2)) & 3) << 2)
    return ((r & 3) << 1) | ((r >> 2) & 1)


def _loader(D, BN, NW):
    """Per-lane constants of TileLoader<D, BN, NW>."""
    dch = D // 8
    rpi = 64 // dch
    loads = BN * dch // (64 * NW)
    step = NW * rpi
    period = 16 if D >= 128 else 8
    noff = 1 if step >= period else period // step
    assert loads >= 1 and loads % noff == 0
    return dch, rpi, loads, step, noff


def _tile_loads(D, BN, NW, rs, t):
    """(lds row, source chunk, byte offset from the head's first element) of
    every lane's load of tile t, over all wavefronts and instructions."""
    dch, rpi, loads, step, noff = _loader(D, BN, NW)
    wave, lane = np.meshgrid(np.arange(NW), np.arange(64), indexing="ij")
    wave, lane = wave.ravel(), lane.ravel()
    slot = lane % dch
    voff, rows_j = [], []
    for j in range(noff):
        row = (NW * j + wave) * rpi + lane // dch
        rows_j.append(row)
        voff.append((row * rs + (slot ^ _swz(D, row)) * 8) * 2)
    period_bytes = noff * step * rs * 2
    out = []
    for i in range(loads):
        lds_row = (NW * i + wave) * rpi + lane // dch
        # the swizzle repeats every noff instructions: the source chunk the
        # offset names is the one the LDS row's swizzle expects
        assert np.array_equal(_swz(D, lds_row), _swz(D, rows_j[i % noff]))
        chunk = slot ^ _swz(D, lds_row)
        off = voff[i % noff] + t * BN * rs * 2 + (i // noff) * period_bytes
        out.append((lds_row, chunk, off))
    return out


def _layouts(B, H, T, dv):
    """(name, element strides over (b, h, t), tensor elements)."""
    return [("bhtd", (H * T * dv, T * dv, dv), B * H * T * dv),
            ("btnh", (T * H * dv, dv, H * dv), B * T * H * dv)]


def _check(D, dv, BN, NW, B, H, Tk, new_extent=True):
    """Runs the model; returns the loads that read outside the tensor."""
    bad = []
    for name, (s0, s1, rs), elems in _layouts(B, H, Tk, dv):
        ntiles = (Tk + BN - 1) // BN
        for b in range(B):
            for h in range(H):
                base = b * s0 + h * s1
                extent = ((Tk - 1) * rs + dv) * 2 if new_extent else Tk * rs * 2
                for t in range(ntiles):
                    for lds_row, chunk, off in _tile_loads(D, BN, NW, rs, t):
                        live = off < extent
                        if new_extent:
                            # chunks are 16-byte aligned from the head's
                            # first element and so is the extent
                            assert np.all(~live | (off + 16 <= extent))
                        start = base + off // 2
                        outside = live & ((start < 0) | (start + 8 > elems))
                        if outside.any():
                            bad.append((name, b, h, t))
                        key = t * BN + lds_row
                        used = (key < Tk) & (chunk * 8 < dv)
                        want = (key * rs + chunk * 8) * 2
                        assert np.all(~used | (live & (off == want))), (name, b, h, t)
                        assert not np.any((key >= Tk) & live), (name, b, h, t)
    return bad


# (tile width D, head size dv): rows load D wide, the MFMAs use dv features.
HEADS = [(64, 32), (64, 64), (128, 96), (128, 128)]


@pytest.mark.parametrize("D,dv", HEADS)
@pytest.mark.parametrize("Tk", [1, 31, 64, 100, 130])
def test_prefill_and_backward_tiles(D, dv, Tk):
    """64-key / 64-row tiles over four wavefronts (pipelined prefill Loader,
    per-element-mask kernel, backward Q / dO / K / V tiles)."""
    assert _check(D, dv, 64, 4, B=2, H=3, Tk=Tk) == []


@pytest.mark.parametrize("D,dv", HEADS)
@pytest.mark.parametrize("Tk", [1, 33, 96, 161])
def test_decode_tiles(D, dv, Tk):
    """32-key tiles of one wavefront (MFMA split-KV decode)."""
    assert _check(D, dv, 32, 1, B=2, H=3, Tk=Tk) == []


@pytest.mark.parametrize("D,dv,BN,NW", [(64, 32, 64, 4), (128, 96, 64, 4), (64, 32, 32, 1), (128, 96, 32, 1)])
def test_model_catches_tensor_end(D, dv, BN, NW):
    """The earlier extent (Tk rows of the row stride from the head's first
    element) lets the last head of an interleaved row read its tile-wide last
    row past the tensor's end; head sizes equal to the tile width do not."""
    bad = _check(D, dv, BN, NW, B=2, H=3, Tk=64, new_extent=False)
    assert bad and all(name == "btnh" and b == 1 and h == 2 for name, b, h, _ in bad)
    assert _check(D, D, BN, NW, B=2, H=3, Tk=64, new_extent=False) == []
