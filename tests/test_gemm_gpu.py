"""GPU tests of the hand-written f32 GEMM tile kernel (mfx_gemm) and of the
GEMM with a fused elementwise epilogue (mfx_gemm_ew), through the C-ABI.

Bars:
- GEMM: every element within the fp32 accumulation bound
  (K + 2) * 2^-23 * (|A| |B|)[m, n] of the fp64 product (any summation order
  of K fp32 products meets it; a dropped or doubled k-term or a wrong row /
  column misses it by orders of magnitude).
- Fused epilogue: bit-identical to mfx_gemm followed by mfx_elementwise with
  the same program (the two compile the same expression text with the same
  options, on the same accumulator values), and within 2e-5 of the fp64
  program on the fp64 product (O(1) values)."""
import ctypes

import numpy as np
import pytest

import gemm_programs as gp

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch(cuda):
    return cuda


@pytest.fixture(scope="module")
def nt(cuda):
    from jax_mlx_amd import native

    native.load()
    return native


def _bound(a64, b64, k):
    return np.abs(a64) @ np.abs(b64) * (k + 2) * 2.0 ** -23 + 1e-30


def _check_gemm(torch, nt, a, b, expect_kernel):
    assert nt.gemm_kernel_name(a, b) == expect_kernel
    out = nt.gemm(a, b)
    torch.cuda.synchronize()
    a64, b64 = a.double().cpu().numpy(), b.double().cpu().numpy()
    ref = a64 @ b64
    err = np.abs(out.double().cpu().numpy() - ref)
    assert (err <= _bound(a64, b64, a.shape[-1])).all(), err.max()
    return out


# config 4's four dense layers, then ragged and small shapes
SHAPES = [(8192, 1536, 512), (8192, 512, 512), (8192, 2048, 512), (8192, 512, 2048),
          (1000, 132, 36), (64, 128, 32), (65, 4, 4), (129, 260, 100), (1, 128, 4096)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_gemm_tile_matches_fp64(torch, nt, m, n, k):
    g = torch.Generator(device="cpu").manual_seed(m * 7 + n * 3 + k)
    a = torch.randn(m, k, generator=g).cuda()
    b = (torch.randn(k, n, generator=g) / k ** 0.5).cuda()
    _check_gemm(torch, nt, a, b, "gemm_f32_tile")


def test_gemm_tile_batched_and_strided(torch, nt):
    g = torch.Generator(device="cpu").manual_seed(11)
    # batched A and B; batched A with one shared B
    a = torch.randn(3, 100, 64, generator=g).cuda()
    b = torch.randn(3, 64, 96, generator=g).cuda()
    out = _check_gemm(torch, nt, a, b, "gemm_f32_tile")
    for i in range(3):
        ref = a[i].double().cpu().numpy() @ b[i].double().cpu().numpy()
        bound = _bound(a[i].double().cpu().numpy(), b[i].double().cpu().numpy(), 64)
        assert (np.abs(out[i].double().cpu().numpy() - ref) <= bound).all()
    b2 = torch.randn(64, 96, generator=g).cuda()
    out2 = nt.gemm(a, b2)
    torch.cuda.synchronize()
    for i in range(3):
        ref = a[i].double().cpu().numpy() @ b2.double().cpu().numpy()
        bound = _bound(a[i].double().cpu().numpy(), b2.double().cpu().numpy(), 64)
        assert (np.abs(out2[i].double().cpu().numpy() - ref) <= bound).all()
    # A rows padded (lda 80 > K 64), B a column slice (ldb 160 > N 96)
    big_a = torch.randn(200, 80, generator=g).cuda()
    big_b = torch.randn(64, 160, generator=g).cuda()
    _check_gemm(torch, nt, big_a[:, :64], big_b[:, 32:128], "gemm_f32_tile")


@pytest.mark.parametrize("m,n,k", [(65, 128, 36), (65, 4, 36), (1, 128, 4096), (97, 8, 68)])
def test_gemm_tile_reads_nothing_past_its_operands(torch, nt, m, n, k):
    """A and B each end where a NaN-filled guard region of their allocation
    begins.  Rows past M of the last row tile and k-rows past K of the last
    k-tile must read as zeros (buffer range checks), never the guard: one
    NaN read would reach every output of its tile (0 * NaN).  M % 64 in
    1..32 and K % 32 != 0 make both happen."""
    g = torch.Generator(device="cpu").manual_seed(m + n + k)
    guard = 1 << 20
    fa = torch.full((m * k + guard,), float("nan"), dtype=torch.float32)
    fb = torch.full((k * n + guard,), float("nan"), dtype=torch.float32)
    fa[: m * k] = torch.randn(m * k, generator=g)
    fb[: k * n] = torch.randn(k * n, generator=g) / k ** 0.5
    fa, fb = fa.cuda(), fb.cuda()
    a, b = fa[: m * k].view(m, k), fb[: k * n].view(k, n)
    out = _check_gemm(torch, nt, a, b, "gemm_f32_tile")
    assert torch.isfinite(out).all()


def test_gemm_outside_tile_rules_goes_to_rocblas(torch, nt):
    """A rows off 16-byte alignment, and B rows of 130 floats (ldb % 4 != 0):
    rocBLAS, to the same bar."""
    g = torch.Generator(device="cpu").manual_seed(12)
    flat = torch.randn(64 * 32 + 1, generator=g).cuda()
    b = torch.randn(32, 64, generator=g).cuda()
    _check_gemm(torch, nt, flat[1:].view(64, 32), b, "rocblas")
    _check_gemm(torch, nt, torch.randn(100, 36, generator=g).cuda(), torch.randn(36, 130, generator=g).cuda(),
                "rocblas")


def test_gemm_empty_contraction(torch, nt):
    """K = 0: the product is zero (no k-tile runs; the accumulators are
    stored as initialised)."""
    a = torch.zeros(64, 4, device="cuda")[:, :0]
    b = torch.zeros(4, 128, device="cuda")[:0]
    out = torch.full((64, 128), float("nan"), device="cuda")
    g = nt.gemm_args(a, b, out)
    g.a, g.b = a.data_ptr() or 256, b.data_ptr() or 256
    assert nt.load().mfx_gemm_kernel_name(ctypes.byref(g)) == b"gemm_f32_tile"
    nt.check(nt.load().mfx_gemm(ctypes.byref(g), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert (out == 0).all()


def _epilogue_case(torch, nt, name, dims, k, seed):
    prog, ci, extras = gp.PROGRAMS[name](dims)
    rows = int(np.prod(dims[:-1]))
    n = dims[-1]
    g = torch.Generator(device="cpu").manual_seed(seed)
    a = torch.randn(rows, k, generator=g).cuda()
    b = (torch.randn(k, n, generator=g) / k ** 0.5).cuda()
    tensors = []
    for _name, shape, _strides, dt in extras:
        t = torch.randn(shape, generator=g) * 0.5
        if _name == "row_scale":
            t = 1.0 + 0.25 * t
        tensors.append(t.to(getattr(torch, dt)).cuda())
    inputs, it = [], iter(tensors)
    for i in range(prog.num_inputs):
        inputs.append(None if i == ci else next(it))
    return prog, ci, a, b, inputs, tensors


CASES = [("bias_add", [32, 256, 1536], 512), ("bias_residual", [8192, 512], 512),
         ("bias_gelu", [8192, 2048], 512), ("bias_residual", [8192, 512], 2048),
         ("mixed", [3, 5, 64], 36), ("bias_gelu", [7, 132], 100), ("mixed", [4, 33, 260], 64)]


@pytest.mark.parametrize("name,dims,k", CASES)
def test_gemm_epilogue_equals_unfused(torch, nt, name, dims, k):
    prog, ci, a, b, inputs, tensors = _epilogue_case(torch, nt, name, dims, k, seed=len(name) * 100 + k)
    out = torch.full(dims, float("nan"), device="cuda")
    nt.gemm_ew(a, b, prog, ci, inputs, out)
    # unfused: the GEMM result materialised, then the same program over it
    c = nt.gemm(a, b)
    ref = torch.full(dims, float("nan"), device="cuda")
    unfused = list(inputs)
    unfused[ci] = c
    nt.elementwise(prog, unfused, ref)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    # fp64 program on the fp64 product
    c64 = a.double().cpu().numpy() @ b.double().cpu().numpy()
    want = gp.reference(name, c64, [t.double().cpu().numpy() for t in tensors], dims)
    err = np.abs(out.double().cpu().numpy() - want).max()
    assert err <= 2e-5, err


def test_gemm_epilogue_repeat_calls(torch, nt):
    """The cached kernel serves later calls with other pointers and values;
    a smaller shape of the same program compiles its own kernel."""
    for dims, seed in (([64, 384], 1), ([64, 384], 2), ([32, 384], 3)):
        prog, ci, a, b, inputs, tensors = _epilogue_case(torch, nt, "bias_gelu", dims, 64, seed)
        out = torch.empty(dims, device="cuda")
        nt.gemm_ew(a, b, prog, ci, inputs, out)
        torch.cuda.synchronize()
        c64 = a.double().cpu().numpy() @ b.double().cpu().numpy()
        want = gp.reference("bias_gelu", c64, [t.double().cpu().numpy() for t in tensors], dims)
        assert np.abs(out.double().cpu().numpy() - want).max() <= 2e-5


def test_gemm_epilogue_rejects_unaligned(torch, nt):
    prog, ci, a, b, inputs, _ = _epilogue_case(torch, nt, "bias_add", [64, 128], 32, 5)
    flat = torch.zeros(64 * 32 + 1, device="cuda")
    a2 = flat[1:].view(64, 32)
    out = torch.empty(64, 128, device="cuda")
    with pytest.raises(nt.MfxError) as e:
        nt.gemm_ew(a2, b, prog, ci, inputs, out)
    assert e.value.code == -2


def test_gemm_epilogue_batched(torch, nt):
    """Batched product (A [3, 100, 64] with B per batch, and with one shared
    B) under a bias + residual epilogue over the [3, 100, 96] index space:
    the epilogue's row index runs over batch * M; bit-identical to the
    unfused pair and within 2e-5 of fp64."""
    g = torch.Generator(device="cpu").manual_seed(21)
    dims = [3, 100, 96]
    prog, ci, extras = gp.bias_residual(dims)
    bias = torch.randn(96, generator=g).cuda()
    resid = torch.randn(*dims, generator=g).cuda()
    a = torch.randn(3, 100, 64, generator=g).cuda()
    for b in (torch.randn(3, 64, 96, generator=g).cuda(), torch.randn(64, 96, generator=g).cuda()):
        inputs = [None, bias, resid]
        out = torch.full(dims, float("nan"), device="cuda")
        nt.gemm_ew(a, b, prog, ci, inputs, out)
        c = nt.gemm(a, b)
        ref = torch.full(dims, float("nan"), device="cuda")
        nt.elementwise(prog, [c, bias, resid], ref)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        b64 = b.double().cpu().numpy()
        c64 = np.einsum("bmk,bkn->bmn" if b.dim() == 3 else "bmk,kn->bmn", a.double().cpu().numpy(), b64)
        want = gp.reference("bias_residual", c64, [bias.double().cpu().numpy(), resid.double().cpu().numpy()], dims)
        assert np.abs(out.double().cpu().numpy() - want).max() <= 2e-5
