"""Elementwise programs used as GEMM epilogues in the tests: the consumers
a transformer's dense layers put after their dot_general (bias add; bias add
and residual add; bias add and tanh GELU), plus programs that exercise the
rest of the epilogue generator (iota, bf16 and row-only inputs, rank-3 index
spaces).  Each returns (program, c_input, extra_inputs) where extra_inputs
lists (name, shape, element strides over the program dims, torch dtype name)
for every input besides the GEMM result."""
import math

import numpy as np

from jax_mlx_amd import native as nt

F32, BF16 = nt.MFX_F32, nt.MFX_BF16


def contiguous(dims):
    s, acc = [], 1
    for d in reversed(dims):
        s.append(acc)
        acc *= d
    return list(reversed(s))


def bias_add(dims):
    n = dims[-1]
    bias_strides = [0] * (len(dims) - 1) + [1]
    prog = nt.ew_program(dims, [(F32, contiguous(dims)), (F32, bias_strides)],
                         [("load", 0, 0), ("load", 1, 1), ("add", 2, 0, 1)], 2)
    return prog, 0, [("bias", (n,), bias_strides, "float32")]


def bias_residual(dims):
    n = dims[-1]
    bias_strides = [0] * (len(dims) - 1) + [1]
    prog = nt.ew_program(dims, [(F32, contiguous(dims)), (F32, bias_strides), (F32, contiguous(dims))],
                         [("load", 0, 0), ("load", 1, 1), ("add", 2, 0, 1), ("load", 3, 2), ("add", 4, 3, 2)], 4)
    return prog, 0, [("bias", (n,), bias_strides, "float32"), ("residual", tuple(dims), contiguous(dims), "float32")]


def bias_gelu(dims):
    """0.5 u (1 + tanh(sqrt(2/pi) (u + 0.044715 u^3))), u = C + bias, in the
    instruction order the planner emits for jax.nn.gelu(approximate=True)."""
    n = dims[-1]
    bias_strides = [0] * (len(dims) - 1) + [1]
    code = [("load", 0, 0), ("load", 1, 1), ("add", 2, 0, 1),
            ("mul", 3, 2, 2), ("mul", 4, 3, 2),
            ("const", 5, 0, 0, 0, 0.044715), ("mul", 6, 5, 4), ("add", 7, 2, 6),
            ("const", 8, 0, 0, 0, math.sqrt(2.0 / math.pi)), ("mul", 9, 8, 7), ("tanh", 10, 9),
            ("const", 11, 0, 0, 0, 1.0), ("add", 12, 11, 10),
            ("const", 13, 0, 0, 0, 0.5), ("mul", 14, 13, 2), ("mul", 15, 14, 12)]
    prog = nt.ew_program(dims, [(F32, contiguous(dims)), (F32, bias_strides)], code, 15)
    return prog, 0, [("bias", (n,), bias_strides, "float32")]


def mixed(dims):
    """C * row_scale[row] + bf16 bias[col], then zeroed where the last
    coordinate exceeds the first (iota compare and select)."""
    n = dims[-1]
    r = len(dims)
    bias_strides = [0] * (r - 1) + [1]
    rows = contiguous(dims[:-1])
    row_strides = rows + [0]
    code = [("load", 0, 1), ("load", 1, 2), ("mul", 2, 0, 1), ("load", 3, 0), ("add", 4, 2, 3),
            ("iota", 5, r - 1), ("iota", 6, 0), ("gt", 7, 5, 6), ("const", 8, 0, 0, 0, 0.0),
            ("select", 9, 7, 8, 4)]
    prog = nt.ew_program(dims, [(BF16, bias_strides), (F32, contiguous(dims)), (F32, row_strides)], code, 9)
    return prog, 1, [("bias", (n,), bias_strides, "bfloat16"), ("row_scale", tuple(dims[:-1]), row_strides, "float32")]


PROGRAMS = {"bias_add": bias_add, "bias_residual": bias_residual, "bias_gelu": bias_gelu, "mixed": mixed}


def reference(name, c, extras, dims):
    """fp64 numpy value of program `name` on the GEMM result c [rows, n]
    (float64) and the extra inputs (numpy arrays, in order)."""
    u = c.reshape(dims)
    if name == "bias_add":
        return u + extras[0]
    if name == "bias_residual":
        return extras[1] + (u + extras[0])
    if name == "bias_gelu":
        v = u + extras[0]
        return 0.5 * v * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (v + 0.044715 * v ** 3)))
    if name == "mixed":
        v = u * extras[1][..., None] + extras[0]
        last = np.arange(dims[-1]).reshape([1] * (len(dims) - 1) + [dims[-1]])
        first = np.arange(dims[0]).reshape([dims[0]] + [1] * (len(dims) - 1))
        return np.where(last > first, 0.0, v)
    raise KeyError(name)
