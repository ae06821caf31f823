"""ctypes binding of libmfx_kernels.so (the C-ABI declared in include/mfx_kernels.h).

Device memory and the current stream come from torch tensors; the arithmetic is
the library's gfx950 HIP kernels.  There is no fallback: if the library or a
GPU is missing, calls raise.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "lib"
KERNELS_LIB = LIB_DIR / "libmfx_kernels.so"

MFX_F32, MFX_BF16, MFX_F16 = 0, 1, 2
MFX_OK = 0


class MfxError(RuntimeError):
    """A libmfx_kernels.so entry point returned a non-zero code."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"mfx error {code}: {msg}")
        self.code = code


class NormArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("gamma", ctypes.c_void_p),
        ("beta", ctypes.c_void_p),
        ("rows", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("x_row_stride", ctypes.c_int64),
        ("y_row_stride", ctypes.c_int64),
        ("eps", ctypes.c_float),
        ("dtype", ctypes.c_int32),
        ("param_dtype", ctypes.c_int32),
    ]


class NormBwdArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("gamma", ctypes.c_void_p),
        ("dy", ctypes.c_void_p),
        ("dx", ctypes.c_void_p),
        ("dgamma", ctypes.c_void_p),
        ("dbeta", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("rows", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("x_row_stride", ctypes.c_int64),
        ("dy_row_stride", ctypes.c_int64),
        ("dx_row_stride", ctypes.c_int64),
        ("eps", ctypes.c_float),
        ("dtype", ctypes.c_int32),
        ("param_dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


I64x4 = ctypes.c_int64 * 4


class SdpaArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("q_rms_weight", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("B", ctypes.c_int64),
        ("Hq", ctypes.c_int64),
        ("Hkv", ctypes.c_int64),
        ("Tq", ctypes.c_int64),
        ("Tk", ctypes.c_int64),
        ("D", ctypes.c_int64),
        ("Dv", ctypes.c_int64),
        ("q_strides", I64x4),
        ("k_strides", I64x4),
        ("v_strides", I64x4),
        ("o_strides", I64x4),
        ("mask_strides", I64x4),
        ("scale", ctypes.c_float),
        ("q_rms_eps", ctypes.c_float),
        ("causal", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("mask_dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("lse", ctypes.c_void_p),
    ]


class SdpaBwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("dout", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("dq", ctypes.c_void_p),
        ("dk", ctypes.c_void_p),
        ("dv", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("B", ctypes.c_int64),
        ("Hq", ctypes.c_int64),
        ("Hkv", ctypes.c_int64),
        ("Tq", ctypes.c_int64),
        ("Tk", ctypes.c_int64),
        ("D", ctypes.c_int64),
        ("Dv", ctypes.c_int64),
        ("q_strides", I64x4),
        ("k_strides", I64x4),
        ("v_strides", I64x4),
        ("do_strides", I64x4),
        ("dq_strides", I64x4),
        ("dk_strides", I64x4),
        ("dv_strides", I64x4),
        ("mask_strides", I64x4),
        ("scale", ctypes.c_float),
        ("causal", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("mask_dtype", ctypes.c_int32),
        ("fwd_out", ctypes.c_void_p),
        ("fwd_lse", ctypes.c_void_p),
        ("fwd_out_strides", I64x4),
    ]


class GemmArgs(ctypes.Structure):
    """mfx_gemm_args (include/mfx_kernels.h)."""

    _fields_ = [
        ("a", ctypes.c_void_p),
        ("b", ctypes.c_void_p),
        ("c", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("c_dtype", ctypes.c_int32),
        ("batch", ctypes.c_int64),
        ("m", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("k", ctypes.c_int64),
        ("lda", ctypes.c_int64),
        ("ldb", ctypes.c_int64),
        ("ldc", ctypes.c_int64),
        ("stride_a", ctypes.c_int64),
        ("stride_b", ctypes.c_int64),
        ("stride_c", ctypes.c_int64),
        ("trans_a", ctypes.c_int32),
        ("trans_b", ctypes.c_int32),
    ]


MFX_MAX_RANK = 8
MFX_EW_MAX_INPUTS = 8
MFX_EW_MAX_INSTRS = 64

# Elementwise opcodes (enum order of include/mfx_kernels.h).
EW_OPS = ["load", "const", "iota", "neg", "abs", "exp", "expm1", "log", "log1p", "sqrt", "rsqrt", "tanh",
          "logistic", "erf", "sin", "cos", "floor", "ceil", "round_ne", "sign", "not", "round_bf16",
          "round_f16", "to_int", "is_finite", "copy", "add", "sub", "mul", "div", "max", "min", "pow", "rem",
          "and", "or", "xor", "eq", "ne", "lt", "le", "gt", "ge", "atan2", "select", "clamp"]
EW_OP = {name: i for i, name in enumerate(EW_OPS)}


class EwInstr(ctypes.Structure):
    _fields_ = [("op", ctypes.c_uint8), ("dst", ctypes.c_uint8), ("a", ctypes.c_uint8), ("b", ctypes.c_uint8),
                ("c", ctypes.c_uint8), ("flags", ctypes.c_uint8), ("pad", ctypes.c_uint8 * 2),
                ("imm", ctypes.c_float)]


class EwInput(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("pad", ctypes.c_int32),
                ("strides", ctypes.c_int64 * MFX_MAX_RANK)]


class EwProgram(ctypes.Structure):
    """mfx_ew_program (include/mfx_kernels.h)."""

    _fields_ = [("out", ctypes.c_void_p), ("out_dtype", ctypes.c_int32), ("rank", ctypes.c_int32),
                ("dims", ctypes.c_int64 * MFX_MAX_RANK), ("out_strides", ctypes.c_int64 * MFX_MAX_RANK),
                ("num_inputs", ctypes.c_int32), ("num_instrs", ctypes.c_int32), ("result", ctypes.c_int32),
                ("pad", ctypes.c_int32), ("inputs", EwInput * MFX_EW_MAX_INPUTS),
                ("code", EwInstr * MFX_EW_MAX_INSTRS)]


def ew_program(dims, inputs, code, result, out_dtype=MFX_F32):
    """Builds an EwProgram.  inputs: [(dtype_code, strides)] (data pointers
    are set by the caller); code: [(op_name, dst, a, b, c, imm)] with
    trailing fields optional (0, and imm 0.0); result: register of the
    output."""
    p = EwProgram()
    p.out_dtype = out_dtype
    p.rank = len(dims)
    for d, x in enumerate(dims):
        p.dims[d] = x
    p.num_inputs = len(inputs)
    for i, (dt, strides) in enumerate(inputs):
        p.inputs[i].dtype = dt
        for d, x in enumerate(strides):
            p.inputs[i].strides[d] = x
    p.num_instrs = len(code)
    for pc, ins in enumerate(code):
        op, dst, *rest = ins
        a, b, c, imm = list(rest) + [0, 0, 0, 0.0][len(rest):]
        p.code[pc].op = EW_OP[op]
        p.code[pc].dst = dst
        p.code[pc].a = a
        p.code[pc].b = b
        p.code[pc].c = c
        p.code[pc].imm = imm
    p.result = result
    return p


_lib = None


def load(path: str | os.PathLike | None = None, make_default: bool = False) -> ctypes.CDLL:
    """Loads libmfx_kernels.so (once) and declares its signatures.  A `path`
    loads that copy instead (for example the phase-timer build); with
    make_default the module's calls use it from then on."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else KERNELS_LIB
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is not built; run `python jax-mlx-plugin_amd/build.py` (or __graft_entry__.build())")
    lib = ctypes.CDLL(str(p))
    lib.mfx_last_error.restype = ctypes.c_char_p
    lib.mfx_version.restype = ctypes.c_int
    lib.mfx_device_count.restype = ctypes.c_int
    for name in ("mfx_layer_norm", "mfx_rms_norm", "mfx_softmax", "mfx_log_softmax"):
        fn = getattr(lib, name)
        fn.argtypes = [ctypes.POINTER(NormArgs), ctypes.c_void_p]
        fn.restype = ctypes.c_int
    lib.mfx_layer_norm_bwd.argtypes = [ctypes.POINTER(NormBwdArgs), ctypes.c_void_p]
    lib.mfx_layer_norm_bwd.restype = ctypes.c_int
    lib.mfx_layer_norm_bwd_workspace_size.argtypes = [ctypes.POINTER(NormBwdArgs)]
    lib.mfx_layer_norm_bwd_workspace_size.restype = ctypes.c_size_t
    lib.mfx_sdpa_bwd.argtypes = [ctypes.POINTER(SdpaBwdArgs), ctypes.c_void_p]
    lib.mfx_sdpa_bwd.restype = ctypes.c_int
    lib.mfx_sdpa_bwd_workspace_size.argtypes = [ctypes.POINTER(SdpaBwdArgs)]
    lib.mfx_sdpa_bwd_workspace_size.restype = ctypes.c_size_t
    lib.mfx_sdpa_bwd_kernel_name.argtypes = [ctypes.POINTER(SdpaBwdArgs)]
    lib.mfx_sdpa_bwd_kernel_name.restype = ctypes.c_char_p
    lib.mfx_sdpa_fwd.argtypes = [ctypes.POINTER(SdpaArgs), ctypes.c_void_p]
    lib.mfx_sdpa_fwd.restype = ctypes.c_int
    lib.mfx_sdpa_fwd_noalloc.argtypes = [ctypes.POINTER(SdpaArgs), ctypes.c_void_p]
    lib.mfx_sdpa_fwd_noalloc.restype = ctypes.c_int
    lib.mfx_sdpa_workspace_size.argtypes = [ctypes.POINTER(SdpaArgs)]
    lib.mfx_sdpa_workspace_size.restype = ctypes.c_size_t
    lib.mfx_sdpa_kernel_name.argtypes = [ctypes.POINTER(SdpaArgs)]
    lib.mfx_sdpa_kernel_name.restype = ctypes.c_char_p
    lib.mfx_gemm.argtypes = [ctypes.POINTER(GemmArgs), ctypes.c_void_p]
    lib.mfx_gemm.restype = ctypes.c_int
    lib.mfx_gemm_kernel_name.argtypes = [ctypes.POINTER(GemmArgs)]
    lib.mfx_gemm_kernel_name.restype = ctypes.c_char_p
    lib.mfx_gemm_ew.argtypes = [ctypes.POINTER(GemmArgs), ctypes.POINTER(EwProgram), ctypes.c_int, ctypes.c_void_p]
    lib.mfx_gemm_ew.restype = ctypes.c_int
    lib.mfx_gemm_ew_check.argtypes = [ctypes.POINTER(GemmArgs), ctypes.POINTER(EwProgram), ctypes.c_int]
    lib.mfx_gemm_ew_check.restype = ctypes.c_int
    lib.mfx_gemm_ew_prepare.argtypes = [ctypes.POINTER(GemmArgs), ctypes.POINTER(EwProgram), ctypes.c_int]
    lib.mfx_gemm_ew_prepare.restype = ctypes.c_int
    lib.mfx_gemm_ew_source.argtypes = [ctypes.POINTER(GemmArgs), ctypes.POINTER(EwProgram), ctypes.c_int,
                                       ctypes.c_char_p, ctypes.c_int64]
    lib.mfx_gemm_ew_source.restype = ctypes.c_int64
    lib.mfx_elementwise.argtypes = [ctypes.POINTER(EwProgram), ctypes.c_void_p]
    lib.mfx_elementwise.restype = ctypes.c_int
    if path is None or make_default:
        _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != MFX_OK:
        raise MfxError(rc, load().mfx_last_error().decode())


# ---- torch plumbing ------------------------------------------------------------

def _torch():
    import torch  # noqa: PLC0415

    return torch


def dtype_code(dt) -> int:
    torch = _torch()
    if dt == torch.float32:
        return MFX_F32
    if dt == torch.bfloat16:
        return MFX_BF16
    if dt == torch.float16:
        return MFX_F16
    raise TypeError(f"unsupported dtype {dt}")


def _stream_handle(t) -> int:
    torch = _torch()
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_gpu(*ts) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("tensor must live on the GPU (device memory)")


def _rows_view(x):
    """(rows, n, row_stride) of a tensor whose last dim is contiguous and whose
    leading dims collapse to one row index."""
    if x.dim() == 0:
        raise ValueError("scalar input")
    n = x.shape[-1]
    if x.stride(-1) != 1:
        raise ValueError("last dimension must be contiguous")
    rows = x.numel() // n if n else 0
    if x.dim() == 1:
        return 1, n, n
    lead = x.reshape(-1, n) if x.is_contiguous() else None
    if lead is None:
        # Leading dims must still collapse with a single stride.
        try:
            lead = x.view(-1, n)
        except RuntimeError as e:
            raise ValueError("leading dimensions must collapse to one row stride") from e
    return rows, n, lead.stride(0)


def _norm_call(fn_name, x, gamma, beta, eps, out):
    torch = _torch()
    _require_gpu(x, gamma, beta)
    if out is None:
        out = torch.empty_like(x, memory_format=torch.contiguous_format)
    rows, n, xs = _rows_view(x)
    _, _, ys = _rows_view(out)
    pdt = gamma.dtype if gamma is not None else (beta.dtype if beta is not None else x.dtype)
    a = NormArgs(
        x=x.data_ptr(), y=out.data_ptr(),
        gamma=gamma.data_ptr() if gamma is not None else None,
        beta=beta.data_ptr() if beta is not None else None,
        rows=rows, n=n, x_row_stride=xs, y_row_stride=ys, eps=float(eps),
        dtype=dtype_code(x.dtype), param_dtype=dtype_code(pdt))
    check(getattr(load(), fn_name)(ctypes.byref(a), ctypes.c_void_p(_stream_handle(x))))
    return out


def layer_norm(x, gamma=None, beta=None, eps: float = 1e-5, out=None):
    """(x - mean) / sqrt(var + eps) * gamma + beta over the last axis (mfx_layer_norm)."""
    return _norm_call("mfx_layer_norm", x, gamma, beta, eps, out)


def rms_norm(x, weight=None, eps: float = 1e-5, out=None):
    """x / sqrt(mean(x^2) + eps) * weight over the last axis (mfx_rms_norm)."""
    return _norm_call("mfx_rms_norm", x, weight, None, eps, out)


def softmax(x, out=None):
    """Softmax over the last axis (mfx_softmax)."""
    return _norm_call("mfx_softmax", x, None, None, 0.0, out)


def log_softmax(x, out=None):
    """Log-softmax over the last axis (mfx_log_softmax)."""
    return _norm_call("mfx_log_softmax", x, None, None, 0.0, out)


def layer_norm_bwd(x, dy, gamma=None, eps: float = 1e-5, *, param_grads=True, param_dtype=None,
                   dx=None, workspace=None):
    """(dx, dgamma, dbeta) of LayerNorm over the last axis (mfx_layer_norm_bwd).

    dgamma / dbeta have gamma's dtype (or `param_dtype`, default x's dtype when
    gamma is None); with param_grads=False only dx is computed."""
    torch = _torch()
    _require_gpu(x, dy, gamma)
    if dx is None:
        dx = torch.empty_like(x, memory_format=torch.contiguous_format)
    rows, n, xs = _rows_view(x)
    _, _, gs = _rows_view(dy)
    _, _, ds = _rows_view(dx)
    pdt = gamma.dtype if gamma is not None else (param_dtype or x.dtype)
    dg = db = None
    if param_grads:
        dg = torch.empty(n, dtype=pdt, device=x.device)
        db = torch.empty(n, dtype=pdt, device=x.device)
    a = NormBwdArgs(
        x=x.data_ptr(), gamma=gamma.data_ptr() if gamma is not None else None, dy=dy.data_ptr(),
        dx=dx.data_ptr(), dgamma=dg.data_ptr() if dg is not None else None,
        dbeta=db.data_ptr() if db is not None else None, rows=rows, n=n, x_row_stride=xs,
        dy_row_stride=gs, dx_row_stride=ds, eps=float(eps), dtype=dtype_code(x.dtype),
        param_dtype=dtype_code(pdt))
    if workspace is not None:
        a.workspace = workspace.data_ptr()
        a.workspace_bytes = workspace.numel() * workspace.element_size()
    check(load().mfx_layer_norm_bwd(ctypes.byref(a), ctypes.c_void_p(_stream_handle(x))))
    return dx, dg, db


def layer_norm_bwd_workspace_size(x, gamma=None, param_grads=True) -> int:
    """Bytes of workspace mfx_layer_norm_bwd needs (host-only query)."""
    rows, n, xs = _rows_view(x)
    a = NormBwdArgs(x=16, dy=16, dx=16, dgamma=16 if param_grads else None,
                    dbeta=16 if param_grads else None, rows=rows, n=n, x_row_stride=xs,
                    dy_row_stride=n, dx_row_stride=n, eps=1e-5, dtype=dtype_code(x.dtype),
                    param_dtype=dtype_code(gamma.dtype if gamma is not None else x.dtype))
    return int(load().mfx_layer_norm_bwd_workspace_size(ctypes.byref(a)))


def _strides4(t, layout: str):
    s = t.stride()
    if layout == "bhtd":
        return (s[0], s[1], s[2], s[3])
    if layout == "bthd":
        return (s[0], s[2], s[1], s[3])
    raise ValueError(f"layout must be 'bhtd' or 'bthd', got {layout!r}")


def _dims(t, layout):
    if layout == "bhtd":
        return t.shape[0], t.shape[1], t.shape[2], t.shape[3]
    return t.shape[0], t.shape[2], t.shape[1], t.shape[3]


def sdpa_args(q, k, v, out, *, scale=None, causal=False, mask=None, layout="bhtd",
              q_rms_eps=None, q_rms_weight=None, workspace=None, lse=None) -> SdpaArgs:
    B, Hq, Tq, D = _dims(q, layout)
    _, Hkv, Tk, _ = _dims(k, layout)
    Dv = v.shape[-1]
    if scale is None:
        scale = 1.0 / (D ** 0.5)
    a = SdpaArgs()
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    a.B, a.Hq, a.Hkv, a.Tq, a.Tk, a.D, a.Dv = B, Hq, Hkv, Tq, Tk, D, Dv
    a.q_strides = I64x4(*_strides4(q, layout))
    a.k_strides = I64x4(*_strides4(k, layout))
    a.v_strides = I64x4(*_strides4(v, layout))
    a.o_strides = I64x4(*_strides4(out, layout))
    a.scale = float(scale)
    a.causal = 1 if causal else 0
    a.dtype = dtype_code(q.dtype)
    a.q_rms_eps = float(q_rms_eps) if q_rms_eps is not None else -1.0
    a.q_rms_weight = q_rms_weight.data_ptr() if q_rms_weight is not None else None
    if mask is not None:
        m = mask
        while m.dim() < 4:
            m = m.unsqueeze(0)
        if m.dim() != 4:
            raise ValueError("mask must have at most 4 dims [B, H, Tq, Tk]")
        # Broadcast dims (size 1) get stride 0.
        ms = [0 if m.shape[i] == 1 else m.stride(i) for i in range(4)]
        a.mask = m.data_ptr()
        a.mask_strides = I64x4(*ms)
        a.mask_dtype = dtype_code(m.dtype)
    if workspace is not None:
        a.workspace = workspace.data_ptr()
        a.workspace_bytes = workspace.numel() * workspace.element_size()
    if lse is not None:
        if lse.dtype != _torch().float32 or lse.numel() != B * Hq * Tq or not lse.is_contiguous():
            raise ValueError("lse must be a contiguous f32 tensor of B * Hq * Tq elements")
        a.lse = lse.data_ptr()
    return a


def sdpa(q, k, v, *, scale=None, causal=False, mask=None, layout="bhtd", q_rms_eps=None,
         q_rms_weight=None, out=None, workspace=None, lse=None):
    """softmax(scale * Q K^T + mask) V (mfx_sdpa_fwd).

    layout "bhtd": q [B,Hq,Tq,D], k/v [B,Hkv,Tk,D]; "bthd": JAX's BTNH layout.
    lse: optional f32 [B * Hq * Tq] output of the row log-sum-exp (log2
    units), for sdpa_bwd(fwd_out=..., fwd_lse=...).
    """
    torch = _torch()
    _require_gpu(q, k, v, mask, q_rms_weight)
    if out is None:
        shape = list(q.shape)
        shape[-1] = v.shape[-1]
        out = torch.empty(shape, dtype=q.dtype, device=q.device)
    a = sdpa_args(q, k, v, out, scale=scale, causal=causal, mask=mask, layout=layout,
                  q_rms_eps=q_rms_eps, q_rms_weight=q_rms_weight, workspace=workspace, lse=lse)
    check(load().mfx_sdpa_fwd(ctypes.byref(a), ctypes.c_void_p(_stream_handle(q))))
    return out


def sdpa_noalloc(q, k, v, out, *, scale=None, causal=False, mask=None, layout="bhtd", q_rms_eps=None,
                 q_rms_weight=None):
    """sdpa() through mfx_sdpa_fwd_noalloc: no device allocation, the
    workspace is the library's static per-device scratch (at most
    NOALLOC_SCRATCH_BYTES); the caller passes `out`."""
    _require_gpu(q, k, v, out, mask, q_rms_weight)
    a = sdpa_args(q, k, v, out, scale=scale, causal=causal, mask=mask, layout=layout,
                  q_rms_eps=q_rms_eps, q_rms_weight=q_rms_weight)
    check(load().mfx_sdpa_fwd_noalloc(ctypes.byref(a), ctypes.c_void_p(_stream_handle(q))))
    return out


NOALLOC_SCRATCH_BYTES = 16 << 20  # MFX_SDPA_NOALLOC_SCRATCH_BYTES


def sdpa_workspace_size(q, k, v, **kw) -> int:
    """Bytes of workspace mfx_sdpa_fwd needs for these tensors (host-only)."""
    out = kw.pop("out", None)
    a = sdpa_args(q, k, v, out if out is not None else q, **kw)
    return int(load().mfx_sdpa_workspace_size(ctypes.byref(a)))


def sdpa_kernel_name(q, k, v, **kw) -> str:
    """Which kernel mfx_sdpa_fwd picks for these tensors (host-only query)."""
    out = kw.pop("out", None)
    a = sdpa_args(q, k, v, out if out is not None else q, **kw)
    name = load().mfx_sdpa_kernel_name(ctypes.byref(a))
    if name is None:
        raise MfxError(-1, load().mfx_last_error().decode())
    return name.decode()


def sdpa_bwd_args(q, k, v, dout, dq, dk, dv, *, scale=None, causal=False, mask=None, layout="bhtd",
                  workspace=None, fwd_out=None, fwd_lse=None) -> SdpaBwdArgs:
    B, Hq, Tq, D = _dims(q, layout)
    _, Hkv, Tk, _ = _dims(k, layout)
    Dv = v.shape[-1]
    if scale is None:
        scale = 1.0 / (D ** 0.5)
    a = SdpaBwdArgs()
    a.q, a.k, a.v, a.dout = q.data_ptr(), k.data_ptr(), v.data_ptr(), dout.data_ptr()
    a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    a.B, a.Hq, a.Hkv, a.Tq, a.Tk, a.D, a.Dv = B, Hq, Hkv, Tq, Tk, D, Dv
    for name, t in (("q_strides", q), ("k_strides", k), ("v_strides", v), ("do_strides", dout),
                    ("dq_strides", dq), ("dk_strides", dk), ("dv_strides", dv)):
        setattr(a, name, I64x4(*_strides4(t, layout)))
    a.scale = float(scale)
    a.causal = 1 if causal else 0
    a.dtype = dtype_code(q.dtype)
    if mask is not None:
        m = mask
        while m.dim() < 4:
            m = m.unsqueeze(0)
        ms = [0 if m.shape[i] == 1 else m.stride(i) for i in range(4)]
        a.mask = m.data_ptr()
        a.mask_strides = I64x4(*ms)
        a.mask_dtype = dtype_code(m.dtype)
    if workspace is not None:
        a.workspace = workspace.data_ptr()
        a.workspace_bytes = workspace.numel() * workspace.element_size()
    if fwd_out is not None:
        a.fwd_out = fwd_out.data_ptr()
        a.fwd_out_strides = I64x4(*_strides4(fwd_out, layout))
    if fwd_lse is not None:
        a.fwd_lse = fwd_lse.data_ptr()
    return a


def sdpa_bwd(q, k, v, dout, *, scale=None, causal=False, mask=None, layout="bhtd", workspace=None,
             fwd_out=None, fwd_lse=None):
    """(dq, dk, dv) of softmax(scale * Q K^T + mask) V for upstream gradient dout
    (mfx_sdpa_bwd); layouts as sdpa().  fwd_out / fwd_lse: the forward call's
    output and lse on the same inputs (both or neither) to skip the
    recomputed forward pass."""
    torch = _torch()
    _require_gpu(q, k, v, dout, mask, fwd_out, fwd_lse)
    dq, dk, dv = (torch.empty_like(t) for t in (q, k, v))
    a = sdpa_bwd_args(q, k, v, dout, dq, dk, dv, scale=scale, causal=causal, mask=mask, layout=layout,
                      workspace=workspace, fwd_out=fwd_out, fwd_lse=fwd_lse)
    check(load().mfx_sdpa_bwd(ctypes.byref(a), ctypes.c_void_p(_stream_handle(q))))
    return dq, dk, dv


def sdpa_bwd_kernel_name(q, k, v, **kw) -> str:
    """Which backward kernels mfx_sdpa_bwd picks (host-only query)."""
    a = sdpa_bwd_args(q, k, v, q, q, k, v, **kw)
    name = load().mfx_sdpa_bwd_kernel_name(ctypes.byref(a))
    if name is None:
        raise MfxError(-1, load().mfx_last_error().decode())
    return name.decode()


def sdpa_bwd_workspace_size(q, k, v, **kw) -> int:
    a = sdpa_bwd_args(q, k, v, q, q, k, v, **kw)
    return int(load().mfx_sdpa_bwd_workspace_size(ctypes.byref(a)))


# ---- GEMM ----------------------------------------------------------------------

def _matrix(x):
    """(batch, rows, cols, ld, batch_stride) of a 2-D or 3-D tensor whose
    last dim is contiguous."""
    if x.dim() not in (2, 3) or x.stride(-1) != 1:
        raise ValueError("GEMM operands are 2-D or 3-D with a contiguous last dim")
    if x.dim() == 2:
        return 1, x.shape[0], x.shape[1], x.stride(0), 0
    return x.shape[0], x.shape[1], x.shape[2], x.stride(1), x.stride(0)


def gemm_args(a, b, c=None, trans_a=False, trans_b=False):
    """GemmArgs for c = op(a) @ op(b) (row-major, optionally batched; b may
    be 2-D and shared by every batch of a).  trans_a: a is stored [k, m];
    trans_b: b is stored [n, k]."""
    ba, r, s_, lda, sa = _matrix(a)
    m, k = (s_, r) if trans_a else (r, s_)
    bb, r2, s2, ldb, sb = _matrix(b)
    k2, n = (s2, r2) if trans_b else (r2, s2)
    if k2 != k or (bb != ba and bb != 1):
        raise ValueError("GEMM extents disagree")
    g = GemmArgs()
    g.trans_a, g.trans_b = int(trans_a), int(trans_b)
    g.a, g.b = a.data_ptr(), b.data_ptr()
    g.c = c.data_ptr() if c is not None else None
    g.dtype = dtype_code(a.dtype)
    g.c_dtype = dtype_code(c.dtype) if c is not None else MFX_F32
    g.batch, g.m, g.n, g.k = ba, m, n, k
    g.lda, g.ldb, g.ldc = lda, ldb, n
    g.stride_a, g.stride_b, g.stride_c = sa, (sb if bb > 1 else 0), m * n
    return g


def gemm(a, b, out=None, trans_a=False, trans_b=False, out_dtype=None):
    """mfx_gemm: op(a) [(batch,) m, k] @ op(b) [(batch,) k, n] into a new
    contiguous tensor of out_dtype (default f32), or `out`.  trans_a: a is
    stored [(batch,) k, m]; trans_b: b is stored [(batch,) n, k]."""
    torch = _torch()
    _require_gpu(a, b)
    batch = a.shape[0] if a.dim() == 3 else None
    m = a.shape[-1] if trans_a else a.shape[-2]
    n = b.shape[-2] if trans_b else b.shape[-1]
    shape = (batch, m, n) if batch is not None else (m, n)
    if out is None:
        out = torch.empty(shape, dtype=out_dtype or torch.float32, device=a.device)
    g = gemm_args(a, b, out, trans_a, trans_b)
    check(load().mfx_gemm(ctypes.byref(g), _stream_handle(a)))
    return out


def gemm_kernel_name(a, b, out=None, trans_a=False, trans_b=False) -> str:
    """Kernel mfx_gemm runs for op(a) @ op(b): "gemm_f32_tile",
    "gemm_bf16_tile", "gemm_f16_tile" or "rocblas"."""
    return load().mfx_gemm_kernel_name(ctypes.byref(gemm_args(a, b, out, trans_a, trans_b))).decode()


def _bind_inputs(prog, tensors):
    keep = []
    for i, t in enumerate(tensors):
        prog.inputs[i].data = t.data_ptr() if t is not None else None
        keep.append(t)
    return keep


def gemm_ew(a, b, prog, c_input, inputs, out):
    """mfx_gemm_ew: out = prog(inputs) with inputs[c_input] the product a @ b
    (pass None for it)."""
    _require_gpu(a, b, out)
    g = gemm_args(a, b)
    prog.out = out.data_ptr()
    _bind_inputs(prog, inputs)
    check(load().mfx_gemm_ew(ctypes.byref(g), ctypes.byref(prog), c_input, _stream_handle(a)))
    return out


def elementwise(prog, inputs, out):
    """mfx_elementwise: out = prog(inputs)."""
    _require_gpu(out)
    prog.out = out.data_ptr()
    _bind_inputs(prog, inputs)
    check(load().mfx_elementwise(ctypes.byref(prog), _stream_handle(out)))
    return out


def gemm_ew_source(g, prog, c_input) -> str | None:
    """Generated source of the fused kernel (None when the pair is not fused)."""
    lib = load()
    n = lib.mfx_gemm_ew_source(ctypes.byref(g), ctypes.byref(prog), c_input, None, 0)
    if n < 0:
        return None
    buf = ctypes.create_string_buffer(int(n) + 1)
    lib.mfx_gemm_ew_source(ctypes.byref(g), ctypes.byref(prog), c_input, buf, n + 1)
    return buf.value.decode()
