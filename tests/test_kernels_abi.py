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
    ba.dx, ba.dtype = 16, native.MFX_F16
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
