"""CPU checks of libmfx_kernels.so: it loads, exports every entry point that
include/mfx_kernels.h declares, validates arguments on the host and selects
the intended kernel per configuration -- all without touching a GPU."""
import ctypes
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent


def _declared(header: Path) -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(mfx_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def native():
    from jax_mlx_amd import native

    native.load()
    return native


def test_exports_every_declared_symbol(native):
    lib = native.load()
    names = _declared(REPO / "include" / "mfx_kernels.h")
    assert "mfx_sdpa_fwd" in names and "mfx_layer_norm" in names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in mfx_kernels.h but not exported"
    assert lib.mfx_version() >= 1


def _cpu_tensors(torch, *shapes, dtype=None):
    dtype = dtype or torch.bfloat16
    return [torch.zeros(s, dtype=dtype) for s in shapes]


def test_kernel_selection_per_config(native):
    import torch

    # config 3: causal bf16 B4/H32/T2048/d128 -> bf16 MFMA flash kernel
    q, k, v = _cpu_tensors(torch, (4, 32, 2048, 128), (4, 32, 2048, 128), (4, 32, 2048, 128))
    assert native.sdpa_kernel_name(q, k, v, causal=True) == "flash_bf16_d128"
    # config 2: f32 B8/H8/T128/d64 -> fp32 MFMA flash kernel, key-split variant (64 workgroups of
    # 128 rows would leave most CUs idle)
    q, k, v = _cpu_tensors(torch, (8, 8, 128, 64), (8, 8, 128, 64), (8, 8, 128, 64), dtype=torch.float32)
    assert native.sdpa_kernel_name(q, k, v) == "flash_f32_split_d64"
    # config 4's attention (B32, 8 heads, T256): 512 workgroups -> the 128-row kernel
    q, k, v = _cpu_tensors(torch, (32, 8, 256, 64), (32, 8, 256, 64), (32, 8, 256, 64), dtype=torch.float32)
    assert native.sdpa_kernel_name(q, k, v) == "flash_f32_d64"
    # config 5: GQA decode Hq32/Hkv8, Tq=1 -> split-KV decode on the matrix cores
    q, k, v = _cpu_tensors(torch, (16, 32, 1, 128), (16, 8, 8192, 128), (16, 8, 8192, 128))
    assert native.sdpa_kernel_name(q, k, v, q_rms_eps=1e-6) == "decode_splitkv_mfma"
    # the same in f32 -> the vector-ALU split-KV decode
    q, k, v = _cpu_tensors(torch, (2, 8, 1, 128), (2, 2, 512, 128), (2, 2, 512, 128), dtype=torch.float32)
    assert native.sdpa_kernel_name(q, k, v) == "decode_splitkv"
    # up to 32 query rows per kv head (8 heads x 4 positions) stay on the MFMA decode
    q, k, v = _cpu_tensors(torch, (1, 16, 4, 64), (1, 2, 700, 64), (1, 2, 700, 64))
    assert native.sdpa_kernel_name(q, k, v) == "decode_splitkv_mfma"
    # BTNH (JAX layout) views are accepted without a copy
    q, k, v = _cpu_tensors(torch, (2, 256, 8, 64), (2, 256, 8, 64), (2, 256, 8, 64))
    assert native.sdpa_kernel_name(q, k, v, layout="bthd") == "flash_bf16_d64"
    # an odd head size falls to the shape-general kernel
    q, k, v = _cpu_tensors(torch, (1, 2, 33, 80), (1, 2, 33, 80), (1, 2, 33, 80))
    assert native.sdpa_kernel_name(q, k, v) == "generic"


def test_negative_kv_row_strides_leave_buffer_resource_kernels(native):
    """The bf16 flash and MFMA decode kernels read K/V through buffer
    resources spanning a head's Tk rows, range-checked on forward offsets:
    K/V views with negative row strides (possible through the C ABI) must
    select a kernel that addresses K/V with plain pointers instead (the
    shape-general kernel, or for decode the vector-ALU split-KV kernel)."""
    import ctypes

    import torch

    lib = native.load()
    for qs, ks, want, fallback in (((1, 4, 256, 128), (1, 4, 256, 128), "flash_bf16_d128", "generic"),
                                   ((2, 8, 1, 128), (2, 2, 1000, 128), "decode_splitkv_mfma", "decode_splitkv")):
        q, k = _cpu_tensors(torch, qs, ks)
        assert native.sdpa_kernel_name(q, k, k) == want
        a = native.sdpa_args(q, k, k, q)
        a.k_strides[2] = -a.k_strides[2]
        a.v_strides[2] = -a.v_strides[2]
        got = lib.mfx_sdpa_kernel_name(ctypes.byref(a)).decode()
        assert got == fallback, got


def test_short_kv_row_strides_leave_buffer_resource_kernels(native):
    """K/V row strides below D (0 for a broadcast view such as
    torch.expand, or rows that overlap) leave rows past Tk inside a buffer
    resource spanning Tk rows: the bf16 flash, MFMA decode and MFMA backward
    kernels must not take them (shape-general kernel, VALU split-KV decode,
    generic backward)."""
    import ctypes

    import torch

    lib = native.load()
    for qs, ks, want, fallback in (((1, 4, 256, 128), (1, 4, 256, 128), "flash_bf16_d128", "generic"),
                                   ((2, 8, 1, 128), (2, 2, 1000, 128), "decode_splitkv_mfma", "decode_splitkv")):
        for stride in (0, 64):
            for which in ("k", "v"):
                q, k = _cpu_tensors(torch, qs, ks)
                a = native.sdpa_args(q, k, k, q)
                getattr(a, which + "_strides")[2] = stride
                got = lib.mfx_sdpa_kernel_name(ctypes.byref(a)).decode()
                assert got == fallback, (which, stride, got)
    q, k = _cpu_tensors(torch, (1, 4, 256, 128), (1, 4, 256, 128))
    assert native.sdpa_bwd_kernel_name(q, k, k) == "mfma_bf16_d128"
    for which in ("k", "v"):
        a = native.sdpa_bwd_args(q, k, k, q, q, k, k)
        getattr(a, which + "_strides")[2] = 0
        assert lib.mfx_sdpa_bwd_kernel_name(ctypes.byref(a)).decode() == "generic", which


def test_decode_workspace_is_sized(native):
    import torch

    q, k, v = _cpu_tensors(torch, (16, 32, 1, 128), (16, 8, 8192, 128), (16, 8, 8192, 128))
    a = native.sdpa_args(q, k, v, q)
    ws = native.load().mfx_sdpa_workspace_size(ctypes.byref(a))
    # splits * B * Hq * Tq * (Dv + 2) floats, at least two splits here
    assert ws >= 2 * 16 * 32 * 1 * 130 * 4
    q, k, v = _cpu_tensors(torch, (4, 32, 2048, 128), (4, 32, 2048, 128), (4, 32, 2048, 128))
    a = native.sdpa_args(q, k, v, q)
    assert native.load().mfx_sdpa_workspace_size(ctypes.byref(a)) == 0


def test_invalid_arguments_are_rejected_on_host(native):
    import torch

    lib = native.load()
    q, k, v = _cpu_tensors(torch, (1, 3, 4, 64), (1, 2, 4, 64), (1, 2, 4, 64))
    a = native.sdpa_args(q, k, v, q)
    rc = lib.mfx_sdpa_fwd(ctypes.byref(a), None)
    assert rc == -1 and b"multiple of Hkv" in lib.mfx_last_error()
    q, k, v = _cpu_tensors(torch, (1, 2, 4, 64), (1, 2, 4, 64), (1, 2, 4, 64))
    a = native.sdpa_args(q, k, v, q)
    a.q_strides[3] = 2
    assert lib.mfx_sdpa_fwd(ctypes.byref(a), None) == -1
    assert b"feature" in lib.mfx_last_error()
    a = native.sdpa_args(q, k, v, q)
    a.k = None
    assert lib.mfx_sdpa_fwd(ctypes.byref(a), None) == -1
    a = native.sdpa_args(q, k, v, q)
    a.dtype = 7
    assert lib.mfx_sdpa_fwd(ctypes.byref(a), None) == -2
    # Norms: negative eps, short row strides and a null input.
    na = native.NormArgs(x=1, y=1, rows=2, n=8, x_row_stride=8, y_row_stride=8, eps=-1.0,
                         dtype=native.MFX_F32, param_dtype=native.MFX_F32)
    assert lib.mfx_layer_norm(ctypes.byref(na), None) == -1
    na.eps, na.x_row_stride = 1e-5, 4
    assert lib.mfx_rms_norm(ctypes.byref(na), None) == -1
    na.x_row_stride, na.x = 8, None
    assert lib.mfx_softmax(ctypes.byref(na), None) == -1
    # Zero rows is a valid no-op that touches no memory.
    na.x, na.rows = 1, 0
    assert lib.mfx_layer_norm(ctypes.byref(na), None) == 0
    # LayerNorm backward: short strides, null dx, bad dtypes are host errors.
    ba = native.NormBwdArgs(x=16, dy=16, dx=16, rows=4, n=8, x_row_stride=8, dy_row_stride=4,
                            dx_row_stride=8, eps=1e-5, dtype=native.MFX_F32, param_dtype=native.MFX_F32)
    assert lib.mfx_layer_norm_bwd(ctypes.byref(ba), None) == -1
    ba.dy_row_stride, ba.dx = 8, None
    assert lib.mfx_layer_norm_bwd(ctypes.byref(ba), None) == -1
    ba.dx, ba.dtype = 16, 7  # no such element type (f32, bf16 and f16 are taken)
    assert lib.mfx_layer_norm_bwd(ctypes.byref(ba), None) == -1 and b"dtype" in lib.mfx_last_error()


def test_layer_norm_bwd_workspace_is_sized(native):
    import torch

    lib = native.load()
    x = torch.zeros(8 * 128, 512)
    # 1024 rows of 128 vectors: 64 lanes a row, 4 rows a workgroup, 2 rows a
    # group -> 128 partial row pairs of 512 floats.
    assert native.layer_norm_bwd_workspace_size(x) == 128 * 2 * 512 * 4
    assert native.layer_norm_bwd_workspace_size(x, param_grads=False) == 0
    # Partial rows are capped at 1024 however many rows there are.
    big = torch.empty(1 << 20, 64)
    assert native.layer_norm_bwd_workspace_size(big) == 1024 * 2 * 64 * 4
    ba = native.NormBwdArgs(x=16, dy=16, dx=16, dgamma=16, rows=0, n=8, x_row_stride=8,
                            dy_row_stride=8, dx_row_stride=8, eps=1e-5, dtype=native.MFX_F32,
                            param_dtype=native.MFX_F32)
    assert lib.mfx_layer_norm_bwd_workspace_size(ctypes.byref(ba)) == 0


def test_calls_fail_loudly_without_a_gpu(native):
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    x = torch.zeros(4, 8)
    with pytest.raises(ValueError):
        native.layer_norm(x)


# ---------------------------------------------------------------- GEMM

def test_gemm_kernel_selection(native):
    """f32 row-major products without transposes go to the hand-written f32
    MFMA tile kernel, bf16 / f16 products in any transpose combination to the
    16-bit one; what neither takes (K % 4 for f32 and K % 8 for 16-bit, odd
    or N % 4 != 0, rows not 16-byte aligned, transposed f32) to rocBLAS."""
    import torch

    f = torch.float32
    a, b = torch.zeros(8192, 512, dtype=f), torch.zeros(512, 1536, dtype=f)
    assert native.gemm_kernel_name(a, b) == "gemm_f32_tile"
    assert native.gemm_kernel_name(torch.zeros(3, 100, 64, dtype=f), torch.zeros(3, 64, 96, dtype=f)) == "gemm_f32_tile"
    assert native.gemm_kernel_name(torch.zeros(64, 6, dtype=f), torch.zeros(6, 64, dtype=f)) == "rocblas"
    assert native.gemm_kernel_name(torch.zeros(64, 8, dtype=f), torch.zeros(8, 63, dtype=f)) == "rocblas"
    flat = torch.zeros(64 * 8 + 1, dtype=f)
    assert native.gemm_kernel_name(flat[1:].view(64, 8), torch.zeros(8, 64, dtype=f)) == "rocblas"
    assert native.gemm_kernel_name(a.t().contiguous(), b, trans_a=True) == "rocblas"
    for dt, name in ((torch.bfloat16, "gemm_bf16_tile"), (torch.float16, "gemm_f16_tile")):
        a16, b16 = a.to(dt), b.to(dt)
        assert native.gemm_kernel_name(a16, b16) == name
        assert native.gemm_kernel_name(a16, b16.t().contiguous(), trans_b=True) == name          # x W^T
        assert native.gemm_kernel_name(a16.t().contiguous(), b16, trans_a=True) == name          # x^T dy
        assert native.gemm_kernel_name(a16.t().contiguous(), b16.t().contiguous(), trans_a=True,
                                       trans_b=True) == name
        assert native.gemm_kernel_name(torch.zeros(64, 36, dtype=dt), torch.zeros(36, 64, dtype=dt)) == "rocblas"
        assert native.gemm_kernel_name(torch.zeros(64, 32, dtype=dt), torch.zeros(32, 66, dtype=dt)) == "rocblas"
        flat16 = torch.zeros(64 * 32 + 4, dtype=dt)
        assert native.gemm_kernel_name(flat16[4:].view(64, 32), torch.zeros(32, 64, dtype=dt)) == "rocblas"


def _fused_pair(native, name, dims, K):
    import gemm_programs as gp

    prog, ci, extras = gp.PROGRAMS[name](dims)
    rows = 1
    for d in dims[:-1]:
        rows *= d
    g = native.GemmArgs()
    g.a, g.b = 1 << 20, 1 << 21
    g.dtype = g.c_dtype = native.MFX_F32
    g.batch, g.m, g.n, g.k = 1, rows, dims[-1], K
    g.lda, g.ldb, g.ldc, g.stride_c = K, dims[-1], dims[-1], rows * dims[-1]
    prog.out = 1 << 22
    for i in range(prog.num_inputs):
        prog.inputs[i].data = (1 << 23) + 4096 * i
    return g, prog, ci


@pytest.mark.parametrize("name,dims,K", [("bias_gelu", [8192, 2048], 512), ("mixed", [3, 5, 64], 36)])
def test_gemm_epilogue_source_compiles(native, tmp_path, name, dims, K):
    """The generated fused kernel (program as epilogue of the tile kernel)
    compiles for gfx950 with the options hipRTC gets, without spilling."""
    import subprocess

    g, prog, ci = _fused_pair(native, name, dims, K)
    lib = native.load()
    assert lib.mfx_gemm_ew_check(ctypes.byref(g), ctypes.byref(prog), ci) == 0
    src = native.gemm_ew_source(g, prog, ci)
    assert src and "mfx_gemm_ew_kernel" in src
    (tmp_path / "k.hip").write_text(src)
    out = tmp_path / "k.s"
    r = subprocess.run(["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S",
                        "-I", str(REPO / "jax-mlx-plugin_amd/csrc/kernels"), str(tmp_path / "k.hip"), "-o", str(out)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    asm = out.read_text()
    assert re.search(r"\.vgpr_spill_count:\s+0", asm) and "v_mfma_f32_32x32x2_f32" in asm


def test_gemm_epilogue_rejections(native):
    """mfx_gemm_ew_check refuses what the fused kernel cannot do."""
    import gemm_programs as gp

    lib = native.load()

    def rc(g, prog, ci):
        return lib.mfx_gemm_ew_check(ctypes.byref(g), ctypes.byref(prog), ci)

    g, prog, ci = _fused_pair(native, "bias_residual", [256, 192], 128)
    assert rc(g, prog, ci) == 0
    assert rc(g, prog, 7) == -1                       # c_input out of range
    prog.inputs[ci].strides[0], prog.inputs[ci].strides[1] = 1, 256
    assert rc(g, prog, ci) == -2                      # product read transposed
    g, prog, ci = _fused_pair(native, "bias_residual", [256, 192], 128)
    prog.out_strides[0], prog.out_strides[1] = 1, 256
    assert rc(g, prog, ci) == -2                      # strided output
    g, prog, ci = _fused_pair(native, "bias_residual", [256, 192], 128)
    prog.out = (1 << 22) + 4
    assert rc(g, prog, ci) == -2                      # output not aligned to an element pair
    g, prog, ci = _fused_pair(native, "bias_residual", [256, 192], 128)
    g.a = (1 << 20) + 4
    assert rc(g, prog, ci) == -2                      # A rows not 16-byte aligned
    # index space [512, 96]: no dim boundary at N = 192
    prog, ci, _ = gp.bias_add([512, 96])
    g, _, _ = _fused_pair(native, "bias_add", [256, 192], 128)
    prog.out = 1 << 22
    for i in range(prog.num_inputs):
        prog.inputs[i].data = (1 << 23) + 4096 * i
    assert rc(g, prog, ci) == -2


def test_tanh_formula_accuracy():
    """ew_math.h's mfx_tanh restated in numpy fp32 (the header's own
    coefficients, fma as one rounding, exp2 and reciprocal correctly
    rounded): within 2.5 ulp of fp64 tanh on a dense grid of [0, 20] and at
    the 0.55 switch (the six roundings of the exp2 branch reach 2.2 ulp near
    |x| = 1; the polynomial 0.8).  A wrong coefficient or a dropped term fails it by
    orders of magnitude; the GPU test bounds the hardware's exp2 / rcp."""
    import numpy as np

    text = (REPO / "jax-mlx-plugin_amd/csrc/kernels/ew_math.h").read_text()
    nums = [float(v) for v in re.findall(r"(-?\d+\.\d+)f", text)]
    c4, c3, c2, c1, c0 = nums[0], nums[1], nums[2], nums[3], nums[4]
    k, cut = nums[5], nums[-1]
    assert cut == 0.55 and abs(k + 2.0 / np.log(2.0)) < 1e-12
    f32 = np.float32

    def fma(a, b, c):
        return (a.astype(np.float64) * b + c).astype(f32)

    x = np.concatenate([np.linspace(0, 20, 4_000_001, dtype=np.float64).astype(f32),
                        np.nextafter(f32(0.55), f32(0)) + np.arange(-50, 50, dtype=f32) * np.spacing(f32(0.55))])
    s = (x * x).astype(f32)
    p = fma(np.full_like(s, c4), s, f32(c3))
    for c in (c2, c1, c0):
        p = fma(p, s, f32(c))
    small = fma((x * s).astype(f32), p, x)
    e = np.exp2((x * f32(k)).astype(f32).astype(np.float64)).astype(f32)
    big = ((f32(1) - e) * (1.0 / (f32(1) + e).astype(np.float64)).astype(f32)).astype(f32)
    y = np.where(x < f32(cut), small, big)
    ref = np.tanh(x.astype(np.float64))
    ulp = np.abs(y - ref) / np.spacing(np.maximum(np.abs(ref), 1e-38).astype(f32)).astype(np.float64)
    assert ulp.max() <= 2.5, ulp.max()
