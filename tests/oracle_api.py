"""numpy wrappers of the fp64 CPU oracle (oracle/liboracle.so).

Test infrastructure only: used by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg as the checker, never by the product path.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent.parent
ORACLE_DIR = REPO / "oracle"
LIB = ORACLE_DIR / "liboracle.so"

_lib = None
_dp = ctypes.POINTER(ctypes.c_double)
_i64 = ctypes.c_int64


def _load():
    global _lib
    if _lib is not None:
        return _lib
    src = ORACLE_DIR / "oracle.c"
    if not LIB.exists() or LIB.stat().st_mtime < src.stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    lib = ctypes.CDLL(str(LIB))
    lib.oracle_layer_norm.argtypes = [_dp, _dp, _dp, _i64, _i64, ctypes.c_double, _dp]
    lib.oracle_rms_norm.argtypes = [_dp, _dp, _i64, _i64, ctypes.c_double, _dp]
    lib.oracle_softmax.argtypes = [_dp, _i64, _i64, _dp]
    lib.oracle_log_softmax.argtypes = [_dp, _i64, _i64, _dp]
    lib.oracle_sdpa.argtypes = [_dp, _dp, _dp, _dp, ctypes.POINTER(_i64)] + [_i64] * 7 + [
        ctypes.c_double, ctypes.c_int, _dp]
    lib.oracle_sdpa.restype = ctypes.c_int
    lib.oracle_layer_norm_bwd.argtypes = [_dp, _dp, _dp, _i64, _i64, ctypes.c_double, _dp, _dp, _dp]
    lib.oracle_sdpa_bwd.argtypes = [_dp, _dp, _dp, _dp, _dp, ctypes.POINTER(_i64)] + [_i64] * 7 + [
        ctypes.c_double, ctypes.c_int, _dp, _dp, _dp]
    lib.oracle_sdpa_bwd.restype = ctypes.c_int
    _lib = lib
    return lib


def _c(a):
    if a is None:
        return None, None
    arr = np.ascontiguousarray(np.asarray(a, dtype=np.float64))
    return arr, arr.ctypes.data_as(_dp)


def layer_norm(x, gamma=None, beta=None, eps=1e-5):
    x, xp = _c(x)
    g, gp = _c(gamma)
    b, bp = _c(beta)
    y = np.empty_like(x)
    n = x.shape[-1]
    _load().oracle_layer_norm(xp, gp, bp, x.size // n, n, eps, y.ctypes.data_as(_dp))
    return y


def rms_norm(x, weight=None, eps=1e-5):
    x, xp = _c(x)
    w, wp = _c(weight)
    y = np.empty_like(x)
    n = x.shape[-1]
    _load().oracle_rms_norm(xp, wp, x.size // n, n, eps, y.ctypes.data_as(_dp))
    return y


def softmax(x):
    x, xp = _c(x)
    y = np.empty_like(x)
    n = x.shape[-1]
    _load().oracle_softmax(xp, x.size // n, n, y.ctypes.data_as(_dp))
    return y


def log_softmax(x):
    x, xp = _c(x)
    y = np.empty_like(x)
    n = x.shape[-1]
    _load().oracle_log_softmax(xp, x.size // n, n, y.ctypes.data_as(_dp))
    return y


def _mask4(mask):
    """Broadcast view of an additive mask as (array, strides in elements)."""
    if mask is None:
        return None, None, (_i64 * 4)(0, 0, 0, 0)
    m = np.ascontiguousarray(np.asarray(mask, dtype=np.float64))
    while m.ndim < 4:
        m = m[None]
    st = [0 if m.shape[i] == 1 else m.strides[i] // 8 for i in range(4)]
    return m, m.ctypes.data_as(_dp), (_i64 * 4)(*st)


def sdpa(q, k, v, scale, causal=False, mask=None):
    """BHTD fp64 attention; GQA when k/v have fewer heads than q."""
    q, qp = _c(q)
    k, kp = _c(k)
    v, vp = _c(v)
    m, mp, ms = _mask4(mask)
    B, Hq, Tq, D = q.shape
    _, Hkv, Tk, _ = k.shape
    Dv = v.shape[-1]
    out = np.empty((B, Hq, Tq, Dv))
    rc = _load().oracle_sdpa(qp, kp, vp, mp, ms, B, Hq, Hkv, Tq, Tk, D, Dv, float(scale),
                             1 if causal else 0, out.ctypes.data_as(_dp))
    if rc != 0:
        raise ValueError(f"oracle_sdpa rejected the shapes (rc={rc})")
    return out


def layer_norm_bwd(x, w, g, eps=1e-5):
    x, xp = _c(x)
    w, wp = _c(w)
    g, gp = _c(g)
    n = x.shape[-1]
    dx = np.empty_like(x)
    dw = np.empty(n)
    db = np.empty(n)
    _load().oracle_layer_norm_bwd(xp, wp, gp, x.size // n, n, eps, dx.ctypes.data_as(_dp),
                                  dw.ctypes.data_as(_dp), db.ctypes.data_as(_dp))
    return dx, dw, db


def sdpa_bwd(q, k, v, dout, scale, causal=False, mask=None):
    q, qp = _c(q)
    k, kp = _c(k)
    v, vp = _c(v)
    g, gp = _c(dout)
    m, mp, ms = _mask4(mask)
    B, Hq, Tq, D = q.shape
    _, Hkv, Tk, _ = k.shape
    Dv = v.shape[-1]
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    rc = _load().oracle_sdpa_bwd(qp, kp, vp, gp, mp, ms, B, Hq, Hkv, Tq, Tk, D, Dv, float(scale),
                                 1 if causal else 0, dq.ctypes.data_as(_dp),
                                 dk.ctypes.data_as(_dp), dv.ctypes.data_as(_dp))
    if rc != 0:
        raise ValueError(f"oracle_sdpa_bwd rejected the shapes (rc={rc})")
    return dq, dk, dv
