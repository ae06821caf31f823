"""GPU tests of the bf16 / f16 GEMM tile kernel (mfx_gemm, gemm16.hip)
through the C-ABI: the four transpose combinations (x W, x W^T, x^T dy,
x^T W^T), f32 and 16-bit outputs, ragged and batched shapes.

Bar: every element within the bound of an fp32 accumulation of exactly
representable products plus the output's rounding,
  |C - ref| <= (K + 2) * 2^-23 * (|op(A)| |op(B)|)[m, n] + u * |ref|[m, n],
u = 0 for f32 outputs, 2^-8 for bf16 and 2^-11 for f16 (unit roundoff), ref
the fp64 product of the 16-bit inputs.  A dropped, doubled or misplaced
k-term (a k slot order that differs between the operands, a wrong swizzle,
a transposed fragment) misses it by orders of magnitude."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch(cuda):
    return cuda


@pytest.fixture(scope="module")
def nt(cuda):
    from jax_mlx_amd import native

    native.load()
    return native


U_OUT = {"f32": 0.0, "bf16": 2.0 ** -8, "f16": 2.0 ** -11}


def _op(x64, trans):
    return np.swapaxes(x64, -1, -2) if trans else x64


def _check(torch, nt, a, b, ta, tb, odt, expect):
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[odt]
    assert nt.gemm_kernel_name(a, b, None, ta, tb) == expect
    out = nt.gemm(a, b, trans_a=ta, trans_b=tb, out_dtype=tdt)
    torch.cuda.synchronize()
    a64 = _op(a.double().cpu().numpy(), ta)
    b64 = _op(b.double().cpu().numpy(), tb)
    k = a64.shape[-1]
    ref = a64 @ b64
    bound = np.abs(a64) @ np.abs(b64) * (k + 2) * 2.0 ** -23 + U_OUT[odt] * np.abs(ref) + 1e-30
    got = out.double().cpu().numpy()
    err = np.abs(got - ref)
    assert np.isfinite(got).all()
    assert (err <= bound).all(), (err / bound).max()
    return out


def _operands(torch, g, m, n, k, ta, tb, dt, batch=None):
    lead = () if batch is None else (batch,)
    ash = lead + ((k, m) if ta else (m, k))
    bsh = lead + ((n, k) if tb else (k, n))
    a = torch.randn(ash, generator=g).to(dt).cuda()
    b = (torch.randn(bsh, generator=g) / k ** 0.5).to(dt).cuda()
    return a, b


# m, n, k multiples of 8 (each is a leading dim in some layout), ragged
# against the 128 x 128 tile and the 64-wide k-tile
SHAPES = [(1000, 136, 40), (136, 264, 104), (64, 128, 64), (8, 128, 4096), (296, 504, 72), (256, 256, 2048),
          (8192, 512, 512)]


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_gemm16_layouts_match_fp64(torch, nt, ta, tb, m, n, k, dt):
    g = torch.Generator(device="cpu").manual_seed(m * 7 + n * 3 + k + 2 * ta + tb)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    a, b = _operands(torch, g, m, n, k, ta, tb, tdt)
    _check(torch, nt, a, b, ta, tb, "f32", f"gemm_{dt}_tile")
    _check(torch, nt, a, b, ta, tb, dt, f"gemm_{dt}_tile")


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm16_batched_shared_and_strided(torch, nt, ta, tb):
    """Batched A and B, batched A with one shared B, and operands that are
    column slices of wider rows (leading dims above the extents)."""
    g = torch.Generator(device="cpu").manual_seed(21 + 2 * ta + tb)
    a, b = _operands(torch, g, 104, 96, 64, ta, tb, torch.bfloat16, batch=3)
    _check(torch, nt, a, b, ta, tb, "bf16", "gemm_bf16_tile")
    b1 = (torch.randn((96, 64) if tb else (64, 96), generator=g) / 8).bfloat16().cuda()
    out = nt.gemm(a, b1, trans_a=ta, trans_b=tb)
    torch.cuda.synchronize()
    for i in range(3):
        a64 = _op(a[i].double().cpu().numpy(), ta)
        b64 = _op(b1.double().cpu().numpy(), tb)
        ref = a64 @ b64
        bound = np.abs(a64) @ np.abs(b64) * 66 * 2.0 ** -23 + 1e-30
        assert (np.abs(out[i].double().cpu().numpy() - ref) <= bound).all()
    wa = torch.randn((200, 88), generator=g).bfloat16().cuda()
    wb = torch.randn((200, 160), generator=g).bfloat16().cuda()
    a2 = wa[:, :64] if not ta else wa[:64, :80]          # [m=200, k=64] or [k=64, m=80]
    b2 = wb[:64, 32:128] if not tb else wb[:96, 8:72]    # [k=64, n=96] or [n=96, k=64]
    _check(torch, nt, a2, b2, ta, tb, "f32", "gemm_bf16_tile")


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("m,n,k", [(72, 128, 40), (136, 8, 72), (8, 136, 4104), (104, 8, 136)])
def test_gemm16_reads_nothing_past_its_operands(torch, nt, ta, tb, m, n, k):
    """A and B each end where a NaN-filled guard region of their allocation
    begins.  Chunks past K of the last k-tile, rows past the last index of
    the last row / column tile and k-rows past K must read as zeros or reach
    only outputs that are never stored: one NaN read into a k column would
    reach every output of its tile (0 * NaN)."""
    g = torch.Generator(device="cpu").manual_seed(m + n + k + 2 * ta + tb)
    guard = 1 << 16
    fa = torch.full((m * k + guard,), float("nan"), dtype=torch.bfloat16)
    fb = torch.full((k * n + guard,), float("nan"), dtype=torch.bfloat16)
    fa[: m * k] = torch.randn(m * k, generator=g).bfloat16()
    fb[: k * n] = (torch.randn(k * n, generator=g) / k ** 0.5).bfloat16()
    fa, fb = fa.cuda(), fb.cuda()
    a = fa[: m * k].view((k, m) if ta else (m, k))
    b = fb[: k * n].view((n, k) if tb else (k, n))
    _check(torch, nt, a, b, ta, tb, "f32", "gemm_bf16_tile")


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_gemm16_16bit_outputs_in_8_byte_pieces(torch, nt, ta, dt):
    """16-bit outputs whose rows are not whole 16-byte chunks take the
    8-byte stores instead of the rows staged through LDS: N % 8 == 4 (B
    transposed, so its rows stay aligned), and an output view 8 bytes past
    a 16-byte boundary with a leading dim of 4 mod 8.  Both against fp64, and
    the view's neighbours untouched."""
    g = torch.Generator(device="cpu").manual_seed(41 + ta)
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16}[dt]
    a, b = _operands(torch, g, 136, 100, 64, ta, True, torch.bfloat16)
    _check(torch, nt, a, b, ta, True, dt, "gemm_bf16_tile")
    a, b = _operands(torch, g, 136, 96, 64, ta, False, torch.bfloat16)
    buf = torch.full((136, 108), 7.0, dtype=tdt, device="cuda")
    out = buf[:, 4:100]  # ldc 108, first element 8 bytes past the row start
    assert out.data_ptr() % 16 == 8 and out.stride(0) % 8 == 4
    # (the Python wrapper writes contiguous outputs: the view's leading dim
    # goes in through the C ABI's ldc)
    args = nt.gemm_args(a, b, out, ta, False)
    args.ldc = out.stride(0)
    assert nt.load().mfx_gemm_kernel_name(ctypes.byref(args)).decode() == "gemm_bf16_tile"
    nt.check(nt.load().mfx_gemm(ctypes.byref(args), nt._stream_handle(a)))
    torch.cuda.synchronize()
    a64, b64 = _op(a.double().cpu().numpy(), ta), b.double().cpu().numpy()
    ref = a64 @ b64
    bound = np.abs(a64) @ np.abs(b64) * 66 * 2.0 ** -23 + U_OUT[dt] * np.abs(ref) + 1e-30
    assert (np.abs(out.double().cpu().numpy() - ref) <= bound).all()
    rest = buf.double().cpu().numpy()
    assert (rest[:, :4] == 7.0).all() and (rest[:, 100:] == 7.0).all()


def test_gemm16_outside_tile_rules_goes_to_rocblas(torch, nt):
    """K % 8 != 0 and N % 4 != 0 stay on rocBLAS, to the same bar."""
    g = torch.Generator(device="cpu").manual_seed(31)
    a = torch.randn(64, 36, generator=g).bfloat16().cuda()
    b = torch.randn(36, 64, generator=g).bfloat16().cuda()
    _check(torch, nt, a, b, False, False, "f32", "rocblas")
    a = torch.randn(64, 32, generator=g).bfloat16().cuda()
    b = torch.randn(32, 66, generator=g).bfloat16().cuda()
    _check(torch, nt, a, b, False, False, "f32", "rocblas")


@pytest.mark.parametrize("ta,tb", [(True, False), (False, False)])
def test_gemm16_split_k(torch, nt, ta, tb):
    """Few output tiles over a long K (a weight gradient x^T dy): the
    k-tiles are split over workgroups whose fp32 partials a second pass sums
    in order.  Batched too (the partials are per batch)."""
    g = torch.Generator(device="cpu").manual_seed(41)
    a, b = _operands(torch, g, 512, 1024, 8192, ta, tb, torch.bfloat16)
    _check(torch, nt, a, b, ta, tb, "bf16", "gemm_bf16_tile")
    _check(torch, nt, a, b, ta, tb, "f32", "gemm_bf16_tile")
    a, b = _operands(torch, g, 136, 128, 3000 - 3000 % 8, ta, tb, torch.bfloat16, batch=2)
    _check(torch, nt, a, b, ta, tb, "f32", "gemm_bf16_tile")
