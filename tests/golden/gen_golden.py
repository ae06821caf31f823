"""Generates tests/golden/fixtures.npz: small inputs with expected outputs
computed by independent library routines in float64 (torch CPU:
F.layer_norm, F.rms_norm, torch.softmax, F.scaled_dot_product_attention and
torch.autograd for the backward cases).

The reference's own tests hold no vectors for this path (its suites never call
dot_product_attention / LayerNorm / RMSNorm), so these fixtures pin the fp64
oracle against a second implementation of the same closed forms:
  LayerNorm   src/jax_mlx/layer_norm.py:20-25 (population variance, affine)
  RMSNorm     src/jax_mlx_pjrt.cpp:2166-2169
  softmax     src/jax_mlx_pjrt.cpp:1857-2044
  SDPA        src/jax_mlx/sdpa.py:19-31 plus causal / additive mask / GQA
  backward    src/jax_mlx/layer_norm.py:59-76, src/jax_mlx/sdpa.py:65-87
Inputs are drawn with numpy.random.default_rng(seed) in float32 (rounded to
bfloat16 where the case is bf16), then promoted to float64.

    python tests/golden/gen_golden.py     # rewrites fixtures.npz
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).resolve().parent / "fixtures.npz"


def bf16_round(a: np.ndarray) -> np.ndarray:
    return torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16).to(torch.float64).numpy()


def t64(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


def sdpa_ref(q, k, v, scale, causal=False, mask=None):
    """torch fp64 SDPA in BHTD; GQA through enable_gqa."""
    Hq, Hkv = q.shape[1], k.shape[1]
    kw = {}
    if Hq != Hkv:
        kw["enable_gqa"] = True
    am = None
    if mask is not None:
        am = t64(mask)
    if causal:
        Tq, Tk = q.shape[2], k.shape[2]
        cm = torch.full((Tq, Tk), float("-inf"), dtype=torch.float64).triu(1)
        am = cm if am is None else am + cm
    out = F.scaled_dot_product_attention(t64(q), t64(k), t64(v), attn_mask=am, scale=scale, **kw)
    return out.numpy()


def main() -> None:
    fx: dict[str, np.ndarray] = {}

    # ---- LayerNorm ----
    for name, shape, seed in (("ln_a", (2, 3, 8), 11), ("ln_b", (4, 512), 12)):
        rng = np.random.default_rng(seed)
        x = rng.standard_normal(shape).astype(np.float32)
        g = (1.0 + 0.1 * rng.standard_normal(shape[-1])).astype(np.float32)
        b = (0.1 * rng.standard_normal(shape[-1])).astype(np.float32)
        eps = 1e-5
        y = F.layer_norm(t64(x), (shape[-1],), t64(g), t64(b), eps).numpy()
        fx.update({f"{name}_x": x, f"{name}_gamma": g, f"{name}_beta": b,
                   f"{name}_eps": np.float64(eps), f"{name}_y": y})
        y0 = F.layer_norm(t64(x), (shape[-1],), None, None, eps).numpy()
        fx[f"{name}_y_noaffine"] = y0

    # ---- RMSNorm ----
    rng = np.random.default_rng(21)
    x = rng.standard_normal((2, 4, 128)).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    eps = 1e-6
    fx.update({"rms_x": x, "rms_w": w, "rms_eps": np.float64(eps),
               "rms_y": F.rms_norm(t64(x), (128,), t64(w), eps).numpy(),
               "rms_y_noweight": F.rms_norm(t64(x), (128,), None, eps).numpy()})

    # ---- softmax (with -inf entries; a KAT row of ones) ----
    rng = np.random.default_rng(31)
    x = rng.standard_normal((3, 7)).astype(np.float32)
    x[1, 2] = -np.inf
    x[2, :5] = -np.inf
    fx["softmax_x"] = x
    fx["softmax_y"] = torch.softmax(t64(x), dim=-1).numpy()

    # ---- SDPA ----
    rng = np.random.default_rng(41)
    q = rng.standard_normal((1, 2, 8, 16)).astype(np.float32)
    k = rng.standard_normal((1, 2, 8, 16)).astype(np.float32)
    v = rng.standard_normal((1, 2, 8, 16)).astype(np.float32)
    sc = 1.0 / 4.0
    fx.update({"sdpa_f32_q": q, "sdpa_f32_k": k, "sdpa_f32_v": v, "sdpa_f32_scale": np.float64(sc),
               "sdpa_f32_out": sdpa_ref(q, k, v, sc),
               "sdpa_f32_out_causal": sdpa_ref(q, k, v, sc, causal=True)})

    # Cross attention with Tq != Tk, causal top-left aligned.
    rng = np.random.default_rng(42)
    q = rng.standard_normal((2, 3, 5, 8)).astype(np.float32)
    k = rng.standard_normal((2, 3, 9, 8)).astype(np.float32)
    v = rng.standard_normal((2, 3, 9, 8)).astype(np.float32)
    fx.update({"sdpa_x_q": q, "sdpa_x_k": k, "sdpa_x_v": v, "sdpa_x_scale": np.float64(0.3),
               "sdpa_x_out": sdpa_ref(q, k, v, 0.3),
               "sdpa_x_out_causal": sdpa_ref(q, k, v, 0.3, causal=True)})

    rng = np.random.default_rng(43)
    q = bf16_round(rng.standard_normal((1, 2, 64, 128)).astype(np.float32))
    k = bf16_round(rng.standard_normal((1, 2, 64, 128)).astype(np.float32))
    v = bf16_round(rng.standard_normal((1, 2, 64, 128)).astype(np.float32))
    sc = 1.0 / np.sqrt(128.0)
    fx.update({"sdpa_bf16_q": q, "sdpa_bf16_k": k, "sdpa_bf16_v": v, "sdpa_bf16_scale": np.float64(sc),
               "sdpa_bf16_out_causal": sdpa_ref(q, k, v, sc, causal=True)})

    # GQA decode with a length mask: B=2, Hq=4, Hkv=2, Tq=1, Tk=64.
    rng = np.random.default_rng(44)
    q = bf16_round(rng.standard_normal((2, 4, 1, 32)).astype(np.float32))
    k = bf16_round(rng.standard_normal((2, 2, 64, 32)).astype(np.float32))
    v = bf16_round(rng.standard_normal((2, 2, 64, 32)).astype(np.float32))
    lens = np.array([17, 64])
    mask = np.where(np.arange(64)[None, :] < lens[:, None], 0.0, -np.inf).reshape(2, 1, 1, 64)
    sc = 1.0 / np.sqrt(32.0)
    fx.update({"gqa_q": q, "gqa_k": k, "gqa_v": v, "gqa_mask": mask, "gqa_lens": lens,
               "gqa_scale": np.float64(sc), "gqa_out": sdpa_ref(q, k, v, sc, mask=mask)})

    # ---- backward (torch.autograd in float64) ----
    rng = np.random.default_rng(51)
    x = rng.standard_normal((3, 16))
    w = 1.0 + 0.1 * rng.standard_normal(16)
    b = 0.1 * rng.standard_normal(16)
    g = rng.standard_normal((3, 16))
    xt, wt, bt = (t64(a).requires_grad_() for a in (x, w, b))
    F.layer_norm(xt, (16,), wt, bt, 1e-5).backward(t64(g))
    fx.update({"lnb_x": x, "lnb_w": w, "lnb_b": b, "lnb_g": g, "lnb_eps": np.float64(1e-5),
               "lnb_dx": xt.grad.numpy(), "lnb_dw": wt.grad.numpy(), "lnb_db": bt.grad.numpy()})

    rng = np.random.default_rng(52)
    q = rng.standard_normal((1, 2, 6, 8))
    k = rng.standard_normal((1, 2, 7, 8))
    v = rng.standard_normal((1, 2, 7, 8))
    g = rng.standard_normal((1, 2, 6, 8))
    qt, kt, vt = (t64(a).requires_grad_() for a in (q, k, v))
    F.scaled_dot_product_attention(qt, kt, vt, scale=0.35).backward(t64(g))
    fx.update({"sdpab_q": q, "sdpab_k": k, "sdpab_v": v, "sdpab_g": g, "sdpab_scale": np.float64(0.35),
               "sdpab_dq": qt.grad.numpy(), "sdpab_dk": kt.grad.numpy(), "sdpab_dv": vt.grad.numpy()})

    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(fx)} arrays)")


if __name__ == "__main__":
    main()
