"""Host-side model of the f32 GEMM tile kernel's global loads
(jax-mlx-plugin_amd/csrc/kernels/gemm_f32_tile.h, `issue`): for every
workgroup, k-tile, wavefront, lane and load instruction it forms the buffer
resource (base, extent) and the per-lane offset the kernel forms, applies the
hardware's raw-buffer range check (per-lane offset + instruction offset
against the extent; the scalar offset is not checked) and asserts

- every load that returns memory reads 16 bytes inside the operand's
  elements (A: rows < M, columns < K; B: at or before B[K-1][N-1]);
- every (row, k) element the MFMAs consume inside the matrix is loaded from
  exactly that element, and every one outside reads as zero.

The kernel's tile constants are restated here (BM 64, BN 128, 32-wide
k-tiles, four wavefronts); `test_model_catches_scalar_offsets` runs the
model on the earlier form of the loader, whose row and k-tile steps rode in
the unchecked scalar offset, and shows it reads past A and B.
CPU only: no kernel runs."""
import numpy as np
import pytest

BM, BN, BK, NW = 64, 128, 32, 4
A_ROWS = 1024 // (BK * 4)   # A rows per load instruction (8)
B_ROWS = 1024 // (BN * 4)   # B k-rows per load instruction (2)
A_LOADS = BM * BK * 4 // 1024 // NW
B_LOADS = BK * BN * 4 // 1024 // NW
OOR = 0x80000000


def _swz(r):
    return (r & 7) ^ ((r >> 3) & 1)


def _lanes():
    wave, lane = np.meshgrid(np.arange(NW), np.arange(64), indexing="ij")
    return wave.ravel(), lane.ravel()


def _a_loads(M, K, lda, m0, t, scalar_steps=False):
    """(returns_data, byte offset from A[0][0], element row, element col) per
    load of A's k-tile t for the row tile at m0."""
    wave, lane = _lanes()
    a_row = wave * A_ROWS + lane // 8
    chunk = (lane & 7) ^ _swz(a_row)
    a_in = t * BK + chunk * 4 < K
    out = []
    for i in range(A_LOADS):
        if scalar_steps:
            # earlier loader: one resource over rows m0.. (extent (M-m0)*lda*4),
            # row step and k-tile position as the scalar offset
            base = m0 * lda * 4
            extent = (M - m0) * lda * 4
            vo = np.where(a_in, (a_row * lda + chunk * 4) * 4, OOR)
            so = i * NW * A_ROWS * lda * 4 + t * BK * 4
            ok = vo < extent
            addr = base + so + vo
        else:
            rows = min(M - m0, BM)
            base = m0 * lda * 4 + t * BK * 4
            extent = rows * lda * 4 - t * BK * 4
            vo = np.where(a_in, ((i * NW * A_ROWS + a_row) * lda + chunk * 4) * 4, OOR)
            ok = vo < extent
            addr = base + vo
        tile_row = i * NW * A_ROWS + a_row
        out.append((ok, addr, m0 + tile_row, t * BK + chunk * 4))
    return out


def _b_loads(K, N, ldb, n0, t, scalar_steps=False):
    wave, lane = _lanes()
    b_row = wave * B_ROWS + lane // (BN // 4)
    col = n0 + (lane % (BN // 4)) * 4
    out = []
    for i in range(B_LOADS):
        if scalar_steps:
            extent = K * ldb * 4
            vo = (b_row * ldb + col) * 4
            so = (i * NW * B_ROWS + t * BK) * ldb * 4
            ok = vo < extent
            addr = so + vo
        else:
            base = t * BK * ldb * 4
            extent = ((K - 1) * ldb + N) * 4 - base
            vo = ((i * NW * B_ROWS + b_row) * ldb + col) * 4
            ok = vo < extent
            addr = base + vo
        out.append((ok, addr, t * BK + i * NW * B_ROWS + b_row, col))
    return out


def check_gemm_loads(M, N, K, lda, ldb, scalar_steps=False):
    """Raises AssertionError naming the first bad load."""
    a_end = ((M - 1) * lda + K) * 4      # one past A's last element
    b_end = ((K - 1) * ldb + N) * 4      # one past B's last element
    T = (K + BK - 1) // BK
    for m0 in range(0, M, BM):
        for t in range(T):
            for ok, addr, row, col in _a_loads(M, K, lda, m0, t, scalar_steps):
                bad = ok & ((addr < 0) | (addr + 16 > a_end))
                assert not bad.any(), f"A load outside A: m0={m0} t={t} byte {addr[bad][0]} (A ends {a_end})"
                # a load inside the matrix must return data, from its own element
                inside = (row < M) & (col < K)
                assert (ok == inside).all(), f"A range check disagrees with the matrix: m0={m0} t={t}"
                assert (addr[ok] == (row[ok] * lda + col[ok]) * 4).all()
    for n0 in range(0, N, BN):
        for t in range(T):
            for ok, addr, row, col in _b_loads(K, N, ldb, n0, t, scalar_steps):
                bad = ok & ((addr < 0) | (addr + 16 > b_end))
                assert not bad.any(), f"B load outside B: n0={n0} t={t} byte {addr[bad][0]} (B ends {b_end})"
                inside = (row < K) & (col < N)
                # rows past K read zero; columns past N may read the next row (never stored)
                assert not (ok & (row >= K)).any(), f"B row past K returns data: n0={n0} t={t}"
                assert ok[inside].all(), f"B element inside the matrix reads zero: n0={n0} t={t}"
                assert (addr[ok] == (row[ok] * ldb + col[ok]) * 4).all()


# (M, N, K, lda, ldb): config 4's shapes, ragged tiles, padded leading dims,
# K not a multiple of the k-tile, M % 64 in 1..32, one-row A
SHAPES = [(8192, 1536, 512, 512, 1536), (8192, 512, 2048, 2048, 512), (65, 4, 36, 36, 4),
          (65, 128, 36, 40, 132), (1, 128, 4096, 4096, 128), (1000, 132, 36, 36, 132),
          (129, 260, 100, 100, 260), (97, 200, 68, 72, 1536), (64, 128, 32, 32, 128), (33, 8, 4, 4, 8)]


@pytest.mark.parametrize("M,N,K,lda,ldb", SHAPES)
def test_gemm_tile_loads_stay_inside_operands(M, N, K, lda, ldb):
    check_gemm_loads(M, N, K, lda, ldb)


@pytest.mark.parametrize("M,N,K,lda,ldb", [(1, 128, 4096, 4096, 128), (65, 4, 36, 36, 4)])
def test_model_catches_scalar_offsets(M, N, K, lda, ldb):
    """The earlier loader (row step and k-tile position in the scalar
    offset) reads past A or B on these shapes; the model must say so."""
    with pytest.raises(AssertionError, match="outside|past K"):
        check_gemm_loads(M, N, K, lda, ldb, scalar_steps=True)
