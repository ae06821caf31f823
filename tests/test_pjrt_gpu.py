"""End-to-end parity through the PJRT C API: Client_Compile of StableHLO text,
BufferFromHostBuffer / CreateViewOfDeviceBuffer, LoadedExecutable_Execute,
Buffer_ToHostBuffer -- the path jaxlib drives -- checked against the fp64
oracle.

Bars as in the kernel tests: f32 max-abs <= 1e-5 (norms) / 1e-4 (SDPA);
bf16 ||out - ref||_inf / ||ref||_inf <= 2e-2.  Modules that run through the
generic ops (rocBLAS GEMMs, the elementwise interpreter, reductions) carry the
f32 tolerance stated at each test."""
import math

from pathlib import Path

import numpy as np
import pytest

import mlir_modules as M

pytestmark = pytest.mark.gpu

F32_NORM_TOL = 1e-5
F32_SDPA_TOL = 1e-4
BF16_REL_TOL = 2e-2


@pytest.fixture(scope="module")
def client(cuda):
    from jax_mlx_amd import pjrt

    c = pjrt.Client()
    yield c
    c.destroy()


def bf16_round(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).bfloat16().float().numpy()


def host_arg(a, dt):
    """Host tensor for BufferFromHostBuffer in the module's dtype."""
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return {"bf16": t.bfloat16, "f16": t.half}.get(dt, lambda: t)()


def f16_round(a):
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float64)


def run(client, text, arrays, dts):
    exe = client.compile(text)
    bufs = [client.buffer_from_host(host_arg(a, dt)) for a, dt in zip(arrays, dts)]
    outs = exe.execute(bufs)
    res = [o.to_torch().float().numpy().astype(np.float64) for o in outs]
    for b in bufs + outs:
        b.destroy()
    exe.destroy()
    return res


def rel_inf(out, ref):
    return np.abs(out - ref).max() / np.abs(ref).max()


# ---------------------------------------------------------------- norms

@pytest.mark.parametrize("form", ["var", "standardize"])
def test_layer_norm_config1(client, oracle, form):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((8, 128, 512)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    b = (0.1 * rng.standard_normal(512)).astype(np.float32)
    (y,) = run(client, M.layer_norm_module(form=form), [x, g, b], ["f32"] * 3)
    assert np.abs(y - oracle.layer_norm(x, g, b, 1e-5)).max() <= F32_NORM_TOL


def test_layer_norm_flax_bf16(client, oracle):
    rng = np.random.default_rng(11)
    x = bf16_round(rng.standard_normal((4, 64, 256)) * 2 + 0.5)
    g = bf16_round(1 + 0.1 * rng.standard_normal(256))
    b = bf16_round(0.1 * rng.standard_normal(256))
    (y,) = run(client, M.layer_norm_module(shape=(4, 64, 256), dt="bf16", form="flax"), [x, g, b], ["bf16"] * 3)
    assert rel_inf(y, oracle.layer_norm(x, g, b, 1e-5)) <= BF16_REL_TOL


def test_custom_call_layer_norm(client, oracle):
    rng = np.random.default_rng(12)
    x = rng.standard_normal((4, 512)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    b = (0.1 * rng.standard_normal(512)).astype(np.float32)
    (y,) = run(client, M.custom_call_layer_norm_module(eps=1e-3), [x, g, b], ["f32"] * 3)
    assert np.abs(y - oracle.layer_norm(x, g, b, 1e-3)).max() <= F32_NORM_TOL


@pytest.mark.parametrize("shape,dt,pdt", [((8, 128, 512), "f32", "f32"), ((4, 512), "f32", "f32"),
                                          ((33, 1000), "f32", "f32"), ((16, 64, 768), "bf16", "f32"),
                                          ((16, 64, 768), "bf16", "bf16")])
def test_custom_call_layer_norm_bwd(client, oracle, shape, dt, pdt):
    """custom_call @mlx_layer_norm_bwd (reference src/jax_mlx_pjrt.cpp:8237-8281)
    against the fp64 closed form; f32 bar ||d||_inf <= 1e-5 * max(1, ||ref||_inf)."""
    rng = np.random.default_rng(21)
    x = rng.standard_normal(shape).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(shape[-1])).astype(np.float32)
    b = (0.1 * rng.standard_normal(shape[-1])).astype(np.float32)
    g = rng.standard_normal(shape).astype(np.float32)
    if dt == "bf16":
        x, g = bf16_round(x), bf16_round(g)
    if pdt == "bf16":
        w, b = bf16_round(w), bf16_round(b)
    outs = run(client, M.custom_call_layer_norm_bwd_module(shape, eps=1e-5, dt=dt, pdt=pdt), [x, w, b, g],
               [dt, pdt, pdt, dt])
    n = shape[-1]
    refs = oracle.layer_norm_bwd(x.reshape(-1, n), w, g.reshape(-1, n), 1e-5)
    for o, r in zip(outs, refs):
        o = o.reshape(r.shape)
        if dt == "f32":
            assert np.abs(o - r).max() <= F32_NORM_TOL * max(1.0, np.abs(r).max())
        else:
            assert rel_inf(o, r) <= BF16_REL_TOL


@pytest.mark.parametrize("dt,B,T,N,K,H,S", [("f32", 2, 64, 4, 4, 64, 64), ("bf16", 1, 128, 8, 2, 128, 160),
                                             ("bf16", 2, 96, 4, 4, 64, 96), ("bf16", 1, 100, 4, 2, 96, 130),
                                             ("bf16", 2, 64, 2, 2, 32, 64)])
def test_custom_call_sdpa_bwd(client, oracle, dt, B, T, N, K, H, S):
    """custom_call @mlx_sdpa_bwd (reference src/jax_mlx_pjrt.cpp:8151-8206):
    BTNH gradients against the fp64 closed form."""
    rng = np.random.default_rng(22)
    q = rng.standard_normal((B, T, N, H)).astype(np.float32)
    k = rng.standard_normal((B, S, K, H)).astype(np.float32)
    v = rng.standard_normal((B, S, K, H)).astype(np.float32)
    g = rng.standard_normal((B, T, N, H)).astype(np.float32)
    if dt == "bf16":
        q, k, v, g = (bf16_round(a) for a in (q, k, v, g))
    sc = 1.0 / np.sqrt(H)
    outs = run(client, M.custom_call_sdpa_bwd_module(B, T, N, K, H, S, dt=dt, scale=sc), [q, k, v, g], [dt] * 4)
    tr = lambda a: a.transpose(0, 2, 1, 3)
    refs = [tr(r) for r in oracle.sdpa_bwd(tr(q), tr(k), tr(v), tr(g), sc)]
    for o, r in zip(outs, refs):
        if dt == "f32":
            assert np.abs(o - r).max() <= F32_SDPA_TOL * max(1.0, np.abs(r).max())
        else:
            assert rel_inf(o, r) <= BF16_REL_TOL


@pytest.mark.parametrize("dt,upcast", [("f32", False), ("bf16", True)])
def test_rms_norm(client, oracle, dt, upcast):
    rng = np.random.default_rng(13)
    x = bf16_round(rng.standard_normal((2, 4, 128)))
    w = bf16_round(1 + 0.1 * rng.standard_normal(128))
    (y,) = run(client, M.rms_norm_module(dt=dt, upcast=upcast), [x, w], [dt, dt])
    ref = oracle.rms_norm(x, w, 1e-6)
    if dt == "f32":
        assert np.abs(y - ref).max() <= F32_NORM_TOL
    else:
        assert rel_inf(y, ref) <= BF16_REL_TOL


def test_softmax(client, oracle):
    rng = np.random.default_rng(14)
    x = (rng.standard_normal((6, 64)) * 4).astype(np.float32)
    (y,) = run(client, M.softmax_module(), [x], ["f32"])
    assert np.abs(y - oracle.softmax(x)).max() <= F32_NORM_TOL


# ---------------------------------------------------------------- attention

def test_sdpa_config2(client, oracle):
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal((8, 8, 128, 64)).astype(np.float32) for _ in range(3))
    (o,) = run(client, M.sdpa_bhtd_module(), [q, k, v], ["f32"] * 3)
    assert np.abs(o - oracle.sdpa(q, k, v, 0.125)).max() <= F32_SDPA_TOL


def test_sdpa_causal_bhtd_bf16(client, oracle):
    rng = np.random.default_rng(3)
    q, k, v = (bf16_round(rng.standard_normal((1, 4, 256, 128))) for _ in range(3))
    (o,) = run(client, M.sdpa_bhtd_module(B=1, H=4, T=256, D=128, dt="bf16", causal=True), [q, k, v], ["bf16"] * 3)
    assert rel_inf(o, oracle.sdpa(q, k, v, 1 / math.sqrt(128), causal=True)) <= BF16_REL_TOL


@pytest.mark.parametrize("D,dt", [(32, "bf16"), (96, "bf16"), (256, "bf16"), (96, "f32"), (256, "f32")])
def test_sdpa_head_sizes_through_pjrt(client, oracle, D, dt):
    """The BHTD attention module at head sizes 32, 96 and 256 (bf16) and 96,
    256 (f32), causal, through Client_Compile / Execute: the rewriter fuses
    any head size and the kernel library picks the MFMA kernel for it."""
    rng = np.random.default_rng(95 + D)
    rnd = bf16_round if dt == "bf16" else (lambda a: a.astype(np.float32))
    q, k, v = (rnd(rng.standard_normal((1, 4, 200, D))) for _ in range(3))
    (o,) = run(client, M.sdpa_bhtd_module(B=1, H=4, T=200, D=D, dt=dt, causal=True), [q, k, v], [dt] * 3)
    ref = oracle.sdpa(q, k, v, 1 / math.sqrt(D), causal=True)
    if dt == "bf16":
        assert rel_inf(o, ref) <= BF16_REL_TOL
    else:
        assert np.abs(o - ref).max() <= F32_SDPA_TOL


def _device_bf16(cuda, a):
    return cuda.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda().bfloat16()


def test_sdpa_config3_full_size_through_pjrt(client, oracle, cuda):
    """Config 3 as a jitted module through Client_Compile / Execute at full
    size ([4, 32, 2048, 128] bf16, causal): bit-identical to the direct C-ABI
    call on the same inputs (same kernel and arguments), eight heads (one per
    XCD residue and group slot) against the fp64 oracle, row 0 = v0."""
    from config3_heads import CONFIG3_HEADS
    from jax_mlx_amd import native

    rng = np.random.default_rng(3)
    shape = (4, 32, 2048, 128)
    q, k, v = (bf16_round(rng.standard_normal(shape).astype(np.float32)) for _ in range(3))
    (o,) = run(client, M.sdpa_bhtd_module(B=4, H=32, T=2048, D=128, dt="bf16", causal=True), [q, k, v],
               ["bf16"] * 3)
    direct = native.sdpa(*(_device_bf16(cuda, a) for a in (q, k, v)), scale=128 ** -0.5, causal=True)
    assert np.array_equal(o, direct.float().cpu().numpy().astype(np.float64))
    assert np.array_equal(o[:, :, 0], v[:, :, 0])
    for b, h in CONFIG3_HEADS:
        ref = oracle.sdpa(q[b:b + 1, h:h + 1], k[b:b + 1, h:h + 1], v[b:b + 1, h:h + 1], 128 ** -0.5, causal=True)
        assert rel_inf(o[b:b + 1, h:h + 1], ref) <= BF16_REL_TOL, (b, h)


def test_gqa_decode_config5_full_size_through_pjrt(client, oracle, cuda):
    """Config 5 through PJRT at full size: RMSNorm(q) folded into the GQA
    decode over [16, 8, 8192, 128] K/V with a length mask from
    default_rng(5).  Bit-identical to the direct C-ABI call; every row
    against the fp64 oracle."""
    from jax_mlx_amd import native

    rng = np.random.default_rng(5)
    q = bf16_round(rng.standard_normal((16, 32, 1, 128)).astype(np.float32))
    k = bf16_round(rng.standard_normal((16, 8, 8192, 128)).astype(np.float32))
    v = bf16_round(rng.standard_normal((16, 8, 8192, 128)).astype(np.float32))
    lens = rng.integers(1024, 8192, size=16, endpoint=True)
    mask = np.where(np.arange(8192)[None] < lens[:, None], 0.0, -np.inf).reshape(16, 1, 1, 8192).astype(np.float32)
    (o,) = run(client, M.gqa_decode_module(B=16, S=8192), [q, k, v, mask], ["bf16"] * 3 + ["f32"])
    md = cuda.from_numpy(mask).cuda()
    direct = native.sdpa(*(_device_bf16(cuda, a) for a in (q, k, v)), scale=128 ** -0.5, mask=md, q_rms_eps=1e-6)
    assert np.array_equal(o, direct.float().cpu().numpy().astype(np.float64))
    qn = bf16_round(oracle.rms_norm(q, None, 1e-6).astype(np.float32))
    assert rel_inf(o, oracle.sdpa(qn, k, v, 128 ** -0.5, mask=mask)) <= BF16_REL_TOL


def test_dot_product_attention_btnh_causal(client, oracle):
    """jax.nn.dot_product_attention(is_causal=True) layout: BTNH in and out."""
    rng = np.random.default_rng(3)
    B, T, N, H = 2, 192, 4, 128
    q, k, v = (bf16_round(rng.standard_normal((B, T, N, H))) for _ in range(3))
    (o,) = run(client, M.dot_product_attention_module(B=B, T=T, N=N, H=H), [q, k, v], ["bf16"] * 3)
    t = lambda a: a.transpose(0, 2, 1, 3)
    ref = t(oracle.sdpa(t(q), t(k), t(v), 1 / math.sqrt(H), causal=True))
    assert rel_inf(o, ref) <= BF16_REL_TOL


def test_dot_product_attention_gqa_bias(client, oracle):
    rng = np.random.default_rng(4)
    B, T, N, K, H = 2, 64, 8, 2, 64
    q = bf16_round(rng.standard_normal((B, T, N, H)))
    k, v = (bf16_round(rng.standard_normal((B, T, K, H))) for _ in range(2))
    bias = np.where(rng.random((B, 1, 1, T)) < 0.2, -1e9, 0.0).astype(np.float32)
    bias[:, ..., 0] = 0.0
    (o,) = run(client, M.dot_product_attention_module(B=B, T=T, N=N, K=K, H=H, is_causal=False, bias=True),
               [q, k, v, bias], ["bf16"] * 3 + ["f32"])
    t = lambda a: a.transpose(0, 2, 1, 3)
    ref = t(oracle.sdpa(t(q), t(k), t(v), 1 / math.sqrt(H), mask=bias))
    assert rel_inf(o, ref) <= BF16_REL_TOL


def test_sdpa_predicate_mask(client, oracle):
    """A non-causal predicate (s >= t) runs as a fused boolean mask."""
    rng = np.random.default_rng(5)
    T = 32
    q, k, v = (rng.standard_normal((1, 2, T, 64)).astype(np.float32) for _ in range(3))
    text = M.sdpa_bhtd_module(B=1, H=2, T=T, D=64, causal=True).replace("GE,", "LE,")
    (o,) = run(client, text, [q, k, v], ["f32"] * 3)
    keep = np.triu(np.ones((T, T), bool))
    ref = oracle.sdpa(q, k, v, 0.125, mask=np.where(keep, 0.0, -np.inf)[None, None])
    assert np.abs(o - ref).max() <= F32_SDPA_TOL


def test_sdpa_predicate_mask_fully_masked_row(client, oracle):
    """select(s > t, scores, -0.7 * FLT_MAX), JAX's mask value, fused as a
    boolean mask: row 0 sees no key, so all its scores are equal and it
    returns the mean of V, as the unfused select + softmax does."""
    rng = np.random.default_rng(9)
    T = 48
    q, k, v = (rng.standard_normal((1, 2, T, 64)).astype(np.float32) for _ in range(3))
    text = M.sdpa_bhtd_module(B=1, H=2, T=T, D=64, causal=True, mask_value=-0.7 * 3.4028234663852886e38)
    (o,) = run(client, text.replace("GE,", "GT,"), [q, k, v], ["f32"] * 3)
    keep = np.tril(np.ones((T, T), bool), -1)
    ref = oracle.sdpa(q, k, v, 0.125, mask=np.where(keep, 0.0, -np.inf)[None, None])
    ref[:, :, 0] = v.mean(axis=2)
    assert np.isfinite(o).all()
    assert np.abs(o - ref).max() <= F32_SDPA_TOL


def test_sdpa_finite_mask_through_generic_ops(client, oracle):
    """select(tril, s, -1e9) is not fused: GEMM + select + softmax + GEMM.
    Tolerance: the f32 SDPA bar (rocBLAS f32 GEMMs accumulate in f32)."""
    rng = np.random.default_rng(6)
    q, k, v = (rng.standard_normal((1, 2, 16, 64)).astype(np.float32) for _ in range(3))
    (o,) = run(client, M.sdpa_bhtd_module(B=1, H=2, T=16, D=64, causal=True, mask_value=-1e9), [q, k, v],
               ["f32"] * 3)
    assert np.abs(o - oracle.sdpa(q, k, v, 0.125, causal=True)).max() <= F32_SDPA_TOL


def test_sdpa_transposed_k(client, oracle):
    rng = np.random.default_rng(7)
    q, v = (rng.standard_normal((2, 2, 128, 64)).astype(np.float32) for _ in range(2))
    kt = rng.standard_normal((2, 2, 64, 128)).astype(np.float32)
    (o,) = run(client, M.sdpa_bhtd_module(B=2, H=2, transposed_k=True, inline_softmax=True), [q, kt, v],
               ["f32"] * 3)
    ref = oracle.sdpa(q, np.ascontiguousarray(kt.transpose(0, 1, 3, 2)), v, 0.125)
    assert np.abs(o - ref).max() <= F32_SDPA_TOL


def test_custom_call_sdpa_btnh(client, oracle):
    rng = np.random.default_rng(8)
    q, k, v = (rng.standard_normal((2, 64, 4, 64)).astype(np.float32) for _ in range(3))
    (o,) = run(client, M.custom_call_sdpa_module(scale=0.2), [q, k, v], ["f32"] * 3)
    t = lambda a: a.transpose(0, 2, 1, 3)
    assert np.abs(o - t(oracle.sdpa(t(q), t(k), t(v), 0.2))).max() <= F32_SDPA_TOL


@pytest.mark.parametrize("S", [1024, 8192])
def test_gqa_decode_with_q_rms(client, oracle, S):
    """Config 5's module (RMSNorm(q) + GQA + additive padding mask) at batch 4."""
    rng = np.random.default_rng(5)
    B, Hq, Hkv, D = 4, 32, 8, 128
    q = bf16_round(rng.standard_normal((B, Hq, 1, D)))
    k, v = (bf16_round(rng.standard_normal((B, Hkv, S, D))) for _ in range(2))
    lens = rng.integers(1, S + 1, size=B)
    mask = np.where(np.arange(S)[None, :] < lens[:, None], 0.0, -1e9).astype(np.float32).reshape(B, 1, 1, S)
    (o,) = run(client, M.gqa_decode_module(B=B, S=S), [q, k, v, mask], ["bf16"] * 3 + ["f32"])
    qn = bf16_round(oracle.rms_norm(q, None, 1e-6))
    ref = oracle.sdpa(qn, k, v, 1 / math.sqrt(D), mask=mask)
    assert rel_inf(o, ref) <= BF16_REL_TOL


@pytest.mark.parametrize("shape,dt", [((6, 64), "f32"), ((4, 1000), "f32"), ((16, 2048), "bf16")])
def test_log_softmax_fused(client, oracle, shape, dt):
    rng = np.random.default_rng(23)
    x = rng.standard_normal(shape).astype(np.float32) * 3
    if dt == "bf16":
        x = bf16_round(x)
    (y,) = run(client, M.log_softmax_module(shape, dt), [x], [dt])
    ref = oracle.log_softmax(x)
    if dt == "f32":
        assert np.abs(y - ref).max() <= F32_NORM_TOL * max(1.0, np.abs(ref).max())
    else:
        assert rel_inf(y, ref) <= BF16_REL_TOL


@pytest.mark.parametrize("shape,dt", [((16, 256), "f32"), ((7, 33), "f32"), ((8, 128), "bf16")])
def test_sigmoid_and_silu(client, shape, dt):
    """The sigmoid divide form (rewritten to one logistic instruction) and
    silu through func.call, against numpy fp64: f32 max-abs <= 1e-6 (values
    in [0, 1] and |x|-scaled), bf16 the relative bar."""
    rng = np.random.default_rng(24)
    x = rng.standard_normal(shape).astype(np.float32) * 4
    if dt == "bf16":
        x = bf16_round(x)
    sig, si = run(client, M.sigmoid_silu_module(shape, dt), [x], [dt])
    xs = x.astype(np.float64)
    ref_sig = 1.0 / (1.0 + np.exp(-xs))
    ref_si = xs * ref_sig
    if dt == "f32":
        assert np.abs(sig - ref_sig).max() <= 1e-6
        assert np.abs(si - ref_si).max() <= 1e-6 * max(1.0, np.abs(ref_si).max())
    else:
        assert rel_inf(sig, ref_sig) <= BF16_REL_TOL and rel_inf(si, ref_si) <= BF16_REL_TOL


# ------------------------------------------------------ generic elementwise

@pytest.mark.parametrize("R,C,dt", [(64, 256, "f32"), (33, 77, "f32"), (8, 1024, "bf16"), (5, 12, "bf16"),
                                    (1000, 2048, "f32")])
def test_elementwise_program(client, R, C, dt):
    """One fused elementwise program (broadcast, GELU, transposed operand,
    iota mask) against numpy in fp64.  f32: max-abs <= 1e-5 * max(1, |ref|);
    bf16 (rounded after every op, as the module's bf16 types say): the bf16
    relative bar.  Inner dims that are multiples of four take the four-wide
    interpreter, the others the scalar one."""
    rng = np.random.default_rng(31)
    x = rng.standard_normal((R, C)).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    a = rng.standard_normal((C, R)).astype(np.float32)
    if dt == "bf16":
        x, b, a = (bf16_round(t) for t in (x, b, a))
    (o,) = run(client, M.elementwise_mix_module(R, C, dt), [x, b, a], [dt] * 3)
    u = x.astype(np.float64) + b.astype(np.float64)
    g = 0.5 * u * (1 + np.tanh(math.sqrt(2 / math.pi) * (u + 0.044715 * u ** 3)))
    ref = np.where(np.arange(R)[:, None] >= np.arange(C)[None, :], g * a.T.astype(np.float64), -1.0)
    if dt == "f32":
        assert np.abs(o - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    else:
        assert rel_inf(o, ref) <= BF16_REL_TOL


@pytest.mark.parametrize("case", ["mix_f32_v4", "mix_f32_scalar", "mix_bf16_v4", "mix_bf16_scalar", "sigmoid_bf16",
                                  "transformer"])
def test_compiled_elementwise_matches_interpreter(client, case):
    """The native kernels generated per fused elementwise program (hipRTC) and
    the interpreter give the same bits on the same inputs: same library math,
    bf16 rounding and no fma contraction.  Covers broadcast, transposed and
    iota operands, the four-wide and the scalar layouts, bf16 storage, the
    logistic instruction and a whole transformer module."""
    from jax_mlx_amd import native

    lib = native.load()
    rng = np.random.default_rng(32)
    if case.startswith("mix"):
        R, C = {"mix_f32_v4": (64, 256), "mix_f32_scalar": (33, 77), "mix_bf16_v4": (8, 1024),
                "mix_bf16_scalar": (5, 12)}[case]
        dt = "bf16" if "bf16" in case else "f32"
        arrays = [rng.standard_normal(s).astype(np.float32) for s in ((R, C), (C,), (C, R))]
        if dt == "bf16":
            arrays = [bf16_round(a) for a in arrays]
        text, dts = M.elementwise_mix_module(R, C, dt), [dt] * 3
    elif case == "sigmoid_bf16":
        arrays = [bf16_round(rng.standard_normal((16, 256)).astype(np.float32) * 4)]
        text, dts = M.sigmoid_silu_module((16, 256), "bf16"), ["bf16"]
    else:
        layers, B, T, d, heads, mlp = 2, 2, 64, 128, 4, 256
        x = rng.standard_normal((B, T, d)).astype(np.float32)
        arrays = [x] + [a for p in transformer_params(rng, layers, d, mlp) for a in p]
        text, dts = M.transformer_module(layers=layers, B=B, T=T, d=d, heads=heads, mlp=mlp), ["f32"] * len(arrays)
    prev = lib.mfx_ew_jit_enable(1)
    try:
        compiled = run(client, text, arrays, dts)
        lib.mfx_ew_jit_enable(0)
        interpreted = run(client, text, arrays, dts)
    finally:
        lib.mfx_ew_jit_enable(prev)
    for a, b in zip(compiled, interpreted):
        assert np.array_equal(a, b, equal_nan=True)


# ---------------------------------------------------------------- transformer

def transformer_ref(oracle, x, params, heads, eps=1e-5):
    """fp64 forward of mlir_modules.transformer_module's network."""
    x = x.astype(np.float64)
    B, T, d = x.shape
    hd = d // heads

    def gelu(u):
        return 0.5 * u * (1 + np.tanh(math.sqrt(2 / math.pi) * (u + 0.044715 * u ** 3)))

    for p in params:
        g1, b1, wqkv, bqkv, wo, bo, g2, b2, w1, bm1, w2, bm2 = (a.astype(np.float64) for a in p)
        h = oracle.layer_norm(x, g1, b1, eps)
        qkv = h @ wqkv + bqkv
        q, k, v = (qkv[..., j * d:(j + 1) * d].reshape(B, T, heads, hd).transpose(0, 2, 1, 3) for j in range(3))
        o = oracle.sdpa(q, k, v, 1 / math.sqrt(hd)).transpose(0, 2, 1, 3).reshape(B, T, d)
        x = x + o @ wo + bo
        h = oracle.layer_norm(x, g2, b2, eps)
        x = x + gelu(h @ w1 + bm1) @ w2 + bm2
    return x


def transformer_params(rng, layers, d, mlp):
    out = []
    for _ in range(layers):
        p = [1 + 0.1 * rng.standard_normal(d), 0.1 * rng.standard_normal(d),
             rng.standard_normal((d, 3 * d)) / math.sqrt(d), 0.1 * rng.standard_normal(3 * d),
             rng.standard_normal((d, d)) / math.sqrt(d), 0.1 * rng.standard_normal(d),
             1 + 0.1 * rng.standard_normal(d), 0.1 * rng.standard_normal(d),
             rng.standard_normal((d, mlp)) / math.sqrt(d), 0.1 * rng.standard_normal(mlp),
             rng.standard_normal((mlp, d)) / math.sqrt(mlp), 0.1 * rng.standard_normal(d)]
        out.append([a.astype(np.float32) for a in p])
    return out


def test_transformer_block_f32(client, oracle):
    """Config 4's network at a reduced size (2 layers, B2 T64 d128 h4 mlp256).
    Tolerance 2e-4 max-abs: O(1) activations through 8 f32 GEMMs, 4 LayerNorms
    and 2 attentions (each step within its own f32 bar)."""
    rng = np.random.default_rng(4)
    layers, B, T, d, heads, mlp = 2, 2, 64, 128, 4, 256
    x = rng.standard_normal((B, T, d)).astype(np.float32)
    params = transformer_params(rng, layers, d, mlp)
    flat = [x] + [a for p in params for a in p]
    (y,) = run(client, M.transformer_module(layers=layers, B=B, T=T, d=d, heads=heads, mlp=mlp), flat,
               ["f32"] * len(flat))
    assert np.abs(y - transformer_ref(oracle, x, params, heads)).max() <= 2e-4


def test_transformer_config4_full_size(client, oracle):
    """BASELINE config 4 at its own workload: 4 layers, x [32,256,512], d 512,
    8 heads of 64, MLP 2048, Xavier-uniform weights, zero biases, unit
    LayerNorm scales, inputs from default_rng(4) -- the module bench.py
    times, through Client_Compile / Execute.  Its attention is the flash f32
    kernel reading q/k/v in place from the QKV projection (row stride 1536).
    Batch elements are independent, so batches 0 and 31 are checked against
    the fp64 forward.  Bar: the f32 SDPA bar, 1e-4 max-abs (the same network
    in torch f32 on the CPU is 2.7e-6 from fp64 at ||ref||_inf = 6.8)."""
    arrays = M.config4_inputs(seed=4)
    (y,) = run(client, M.transformer_module(), arrays, ["f32"] * len(arrays))
    assert y.shape == (32, 256, 512) and np.isfinite(y).all()
    params = [arrays[1 + 12 * i:13 + 12 * i] for i in range(4)]
    ref = transformer_ref(oracle, arrays[0][[0, 31]], params, 8)
    err = np.abs(y[[0, 31]] - ref).max()
    assert err <= F32_SDPA_TOL, err


def dense_ref(x, w, b, epilogue, r=None):
    u = x.astype(np.float64) @ w.astype(np.float64) + b
    if epilogue == "bias_gelu":
        return 0.5 * u * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (u + 0.044715 * u ** 3)))
    if epilogue == "bias_residual":
        return r + u
    return u


def dense_args(rng, m, k, n, epilogue):
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((k, n)) / math.sqrt(k)).astype(np.float32)
    b = (0.5 * rng.standard_normal(n)).astype(np.float32)
    return [x, w, b] + ([rng.standard_normal((m, n)).astype(np.float32)] if epilogue == "bias_residual" else [])


@pytest.mark.parametrize("epilogue", ["bias", "bias_gelu", "bias_residual"])
def test_dense_epilogue_fused(client, epilogue):
    """dot_general + its bias / GELU / residual program, planned as one fused
    launch (gemm_ew), against the fp64 dense layer.  Bar 2e-5 max-abs on
    O(1) outputs (fp32 accumulation over K = 256 plus the epilogue's own
    rounding)."""
    rng = np.random.default_rng(31)
    args = dense_args(rng, 512, 256, 384, epilogue)
    (y,) = run(client, M.dense_module(M=512, K=256, N=384, epilogue=epilogue), args, ["f32"] * len(args))
    ref = dense_ref(*args[:3], epilogue, *(args[3:] or [None]))
    assert np.abs(y - ref).max() <= 2e-5


def test_batched_dense_epilogue(client):
    """Batched dense layer + bias + tanh GELU through PJRT (one fused launch),
    against fp64.  Bar 2e-5 max-abs (O(1) outputs)."""
    rng = np.random.default_rng(33)
    x = rng.standard_normal((3, 100, 64)).astype(np.float32)
    w = (rng.standard_normal((3, 64, 96)) / 8.0).astype(np.float32)
    b = (0.5 * rng.standard_normal(96)).astype(np.float32)
    (y,) = run(client, M.batched_dense_module(), [x, w, b], ["f32"] * 3)
    u = np.einsum("bmk,bkn->bmn", x.astype(np.float64), w.astype(np.float64)) + b
    ref = 0.5 * u * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (u + 0.044715 * u ** 3)))
    assert np.abs(y - ref).max() <= 2e-5


def test_dense_epilogue_unaligned_weights_fall_back(client):
    """Weights passed as a device view 4 bytes off 16-byte alignment: the
    fused kernel does not take them, so the step runs the GEMM into its
    output and the program in place there -- the same values within the
    f32 bar, and a result equal to the aligned run's to 1e-5."""
    import torch

    rng = np.random.default_rng(32)
    args = dense_args(rng, 256, 128, 192, "bias_gelu")
    exe = client.compile(M.dense_module(M=256, K=128, N=192, epilogue="bias_gelu"))
    x, w, b = (torch.from_numpy(a).cuda() for a in args)
    flat = torch.zeros(w.numel() + 1, device="cuda")
    flat[1:] = w.flatten()
    w_off = flat[1:].view(w.shape)
    assert w_off.data_ptr() % 16 == 4
    outs = []
    for wv in (w, w_off):
        (o,) = exe.execute([client.buffer_view(x), client.buffer_view(wv), client.buffer_view(b)])
        outs.append(o.to_torch().double().numpy())
        o.destroy()
    exe.destroy()
    ref = dense_ref(*args, "bias_gelu")
    for y in outs:
        assert np.abs(y - ref).max() <= 2e-5
    assert np.abs(outs[0] - outs[1]).max() <= 1e-5


# f16 through the same fused paths.  Bar: ||out - ref||_inf / ||ref||_inf
# <= 5e-3 (f16's 11 significant bits; the kernel tests' f16 bar), against
# the oracle on the f16-rounded inputs.
F16_REL_TOL = 5e-3


def test_f16_norms_through_pjrt(client, oracle):
    rng = np.random.default_rng(91)
    x = f16_round(rng.standard_normal((8, 128, 512)) * 2 + 0.5)
    g = f16_round(1 + 0.1 * rng.standard_normal(512))
    b = f16_round(0.1 * rng.standard_normal(512))
    (y,) = run(client, M.layer_norm_module(dt="f16"), [x, g, b], ["f16"] * 3)
    assert rel_inf(y, oracle.layer_norm(x, g, b, 1e-5)) <= F16_REL_TOL
    (y,) = run(client, M.layer_norm_module(shape=(4, 64, 256), dt="f16", form="flax"),
               [x[:4, :64, :256], g[:256], b[:256]], ["f16"] * 3)
    assert rel_inf(y, oracle.layer_norm(x[:4, :64, :256], g[:256], b[:256], 1e-5)) <= F16_REL_TOL
    xr = x[:2, :4, :128]
    (y,) = run(client, M.rms_norm_module(dt="f16", upcast=True), [xr, g[:128]], ["f16", "f16"])
    assert rel_inf(y, oracle.rms_norm(xr, g[:128], 1e-6)) <= F16_REL_TOL
    xs = f16_round(rng.standard_normal((6, 64)) * 4)
    (y,) = run(client, M.softmax_module(dt="f16"), [xs], ["f16"])
    assert rel_inf(y, oracle.softmax(xs)) <= F16_REL_TOL
    (y,) = run(client, M.log_softmax_module((6, 64), dt="f16"), [xs], ["f16"])
    assert rel_inf(y, oracle.log_softmax(xs)) <= F16_REL_TOL


def test_f16_attention_through_pjrt(client, oracle):
    """Causal BHTD prefill, the jax.nn BTNH form with GQA and a bias, and
    GQA decode with q RMSNorm over a length mask, all f16."""
    rng = np.random.default_rng(92)
    q, k, v = (f16_round(rng.standard_normal((1, 4, 256, 128))) for _ in range(3))
    (o,) = run(client, M.sdpa_bhtd_module(B=1, H=4, T=256, D=128, dt="f16", causal=True), [q, k, v], ["f16"] * 3)
    assert rel_inf(o, oracle.sdpa(q, k, v, 1 / math.sqrt(128), causal=True)) <= F16_REL_TOL
    B, T, N, K, H = 2, 64, 8, 2, 64
    q = f16_round(rng.standard_normal((B, T, N, H)))
    k, v = (f16_round(rng.standard_normal((B, T, K, H))) for _ in range(2))
    bias = rng.standard_normal((B, 1, 1, T)) * 0.5  # the module's [B,1,1,S] f32 bias
    bias[1, ..., 40:] = -np.inf
    (o,) = run(client, M.dot_product_attention_module(B=B, T=T, N=N, K=K, H=H, dt="f16", is_causal=False,
                                                      bias=True), [q, k, v, bias], ["f16"] * 3 + ["f32"])
    tr = lambda a: a.transpose(0, 2, 1, 3)  # noqa: E731
    ref = tr(oracle.sdpa(tr(q), tr(k), tr(v), 1 / math.sqrt(H), mask=bias))
    assert rel_inf(o, ref) <= F16_REL_TOL
    S = 1024
    q = f16_round(rng.standard_normal((2, 32, 1, 128)))
    k, v = (f16_round(rng.standard_normal((2, 8, S, 128))) for _ in range(2))
    lens = np.array([1024, 300])
    mask = np.where(np.arange(S)[None] < lens[:, None], 0.0, -np.inf).reshape(2, 1, 1, S)
    (o,) = run(client, M.gqa_decode_module(B=2, S=S, dt="f16"), [q, k, v, mask], ["f16", "f16", "f16", "f32"])
    qn = f16_round(oracle.rms_norm(q, None, 1e-6))
    assert rel_inf(o, oracle.sdpa(qn, k, v, 1 / math.sqrt(128), mask=mask)) <= F16_REL_TOL


def test_f16_backward_custom_calls_through_pjrt(client, oracle):
    rng = np.random.default_rng(93)
    B, T, N, K, H = 1, 128, 8, 2, 128
    q, g = (f16_round(rng.standard_normal((B, T, N, H))) for _ in range(2))
    k, v = (f16_round(rng.standard_normal((B, T, K, H))) for _ in range(2))
    outs = run(client, M.custom_call_sdpa_bwd_module(B=B, T=T, N=N, K=K, H=H, dt="f16", scale=0.1),
               [q, k, v, g], ["f16"] * 4)
    tr = lambda a: a.transpose(0, 2, 1, 3)  # noqa: E731
    refs = oracle.sdpa_bwd(tr(q), tr(k), tr(v), tr(g), 0.1)
    for o, r in zip(outs, refs):
        assert rel_inf(o, tr(r)) <= F16_REL_TOL
    x, dy = (f16_round(rng.standard_normal((16, 64, 768))) for _ in range(2))
    w = f16_round(1 + 0.1 * rng.standard_normal(768))
    b = f16_round(0.1 * rng.standard_normal(768))
    outs = run(client, M.custom_call_layer_norm_bwd_module(shape=(16, 64, 768), eps=1e-5, dt="f16"),
               [x, w, b, dy], ["f16"] * 4)
    refs = oracle.layer_norm_bwd(x.reshape(-1, 768), w, dy.reshape(-1, 768), 1e-5)
    for o, r in zip(outs, refs):
        assert rel_inf(o.reshape(r.shape), r) <= F16_REL_TOL


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_sdpa_vjp_module_linked(client, dt):
    """jax.vjp of mlx_dot_product_attention as one module: the plan hands the
    forward's output and lse to the backward (no recompute).  Every result
    equals the same module with the backward on a separate (equal) q
    argument, which the planner does not link and which recomputes."""
    rng = np.random.default_rng(41)
    B, T, N, H = 2, 128, 4, 64
    q, k, v, g = (rng.standard_normal((B, T, N, H)).astype(np.float32) for _ in range(4))
    if dt != "f32":
        q, k, v, g = (bf16_round(a) if dt == "bf16" else f16_round(a) for a in (q, k, v, g))
    linked = run(client, M.sdpa_vjp_module(B=B, T=T, N=N, H=H, dt=dt), [q, k, v, g], [dt] * 4)
    plain = run(client, M.sdpa_vjp_module(B=B, T=T, N=N, H=H, dt=dt, same_inputs=False), [q, k, v, g, q],
                [dt] * 5)
    for a, b in zip(linked, plain):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_sdpa_vjp_two_cotangents(client, dt):
    """Two backward steps of one forward (the VJP applied to two
    cotangents): both read the lse the forward writes.  Each (dq, dk, dv)
    equals the single-cotangent module's recomputing path (backward on a
    separate, equal q argument) for that cotangent, bit for bit."""
    rng = np.random.default_rng(43)
    B, T, N, H = 2, 128, 4, 64
    q, k, v, g1, g2 = (rng.standard_normal((B, T, N, H)).astype(np.float32) for _ in range(5))
    if dt == "bf16":
        q, k, v, g1, g2 = (bf16_round(a) for a in (q, k, v, g1, g2))
    both = run(client, M.sdpa_vjp_module(B=B, T=T, N=N, H=H, dt=dt, cotangents=2), [q, k, v, g1, g2], [dt] * 5)
    for g, got in ((g1, both[1:4]), (g2, both[4:7])):
        plain = run(client, M.sdpa_vjp_module(B=B, T=T, N=N, H=H, dt=dt, same_inputs=False), [q, k, v, g, q],
                    [dt] * 5)
        assert np.array_equal(both[0], plain[0])
        for a, b in zip(got, plain[1:]):
            assert np.array_equal(a, b)


def test_executable_serialize_round_trip(client):
    """Executable_Serialize / DeserializeAndLoad (reference
    src/jax_mlx_pjrt.cpp:1585-1601 stubs them): the blob holds the module
    text; the loaded copy runs the same plan, so its outputs are bit-identical
    to the original's.  Blobs this plugin did not write, of another format
    version, or cut short are rejected with INVALID_ARGUMENT."""
    from jax_mlx_amd import pjrt

    rng = np.random.default_rng(44)
    text = M.sdpa_bhtd_module(B=2, H=4, T=96, D=64, causal=True)
    exe = client.compile(text)
    blob = exe.serialize()
    assert blob[:8] == b"MFXPJRT\n" and text.encode() in blob
    again = client.deserialize(blob)
    assert again.num_outputs == exe.num_outputs
    qkv = [rng.standard_normal((2, 4, 96, 64)).astype(np.float32) for _ in range(3)]
    outs = []
    for e in (exe, again):
        bufs = [client.buffer_from_host(host_arg(a, "f32")) for a in qkv]
        o = e.execute(bufs)
        outs.append([t.to_torch().numpy() for t in o])
        for t in o + bufs:
            t.destroy()
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    assert again.serialize() == blob
    for bad in (b"not an executable", blob[:8] + b"\x02\x00\x00\x00" + blob[12:], blob[:-1], blob + b" "):
        with pytest.raises(pjrt.PjrtError) as err:
            client.deserialize(bad)
        assert err.value.code_name == "INVALID_ARGUMENT", err.value.message
    exe.destroy()
    again.destroy()


COMPILE_HOST = r"""
#include <dlfcn.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "pjrt_mi355x.h"
/* argv: plugin, MLIR C-API library (loaded RTLD_GLOBAL first), program file.
 * Prints the error code of Client_Compile, then of the serialize / load
 * round trip, then the stub's live-object count. */
static int code_of(const PJRT_Api* api, PJRT_Error* err) {
  if (!err) return 0;
  PJRT_Error_GetCode_Args g = {sizeof g, NULL, err, 0};
  api->PJRT_Error_GetCode(&g);
  PJRT_Error_Message_Args m = {sizeof m, NULL, err, NULL, 0};
  api->PJRT_Error_Message(&m);
  fprintf(stderr, "%.*s\n", (int)m.message_size, m.message);
  PJRT_Error_Destroy_Args d = {sizeof d, NULL, err};
  api->PJRT_Error_Destroy(&d);
  return g.code;
}
int main(int argc, char** argv) {
  if (argc != 4) return 2;
  void* capi = dlopen(argv[2], RTLD_NOW | RTLD_GLOBAL);
  void* h = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
  if (!capi || !h) return 3;
  const PJRT_Api* api = ((const PJRT_Api* (*)(void))dlsym(h, "GetPjrtApi"))();
  FILE* f = fopen(argv[3], "rb");
  if (!f) return 4;
  fseek(f, 0, SEEK_END);
  long n = ftell(f);
  fseek(f, 0, SEEK_SET);
  char* code = malloc(n);
  if (fread(code, 1, n, f) != (size_t)n) return 5;
  fclose(f);
  PJRT_Client_Create_Args cc = {sizeof cc};
  if (code_of(api, api->PJRT_Client_Create(&cc))) return 6;
  PJRT_Program prog = {sizeof prog, NULL, code, (size_t)n, "mlir", 4};
  PJRT_Client_Compile_Args ca = {sizeof ca, NULL, cc.client, &prog, "", 0, NULL};
  int rc = code_of(api, api->PJRT_Client_Compile(&ca));
  int rc2 = -1;
  if (!rc) {
    PJRT_LoadedExecutable_GetExecutable_Args g = {sizeof g, NULL, ca.executable, NULL};
    api->PJRT_LoadedExecutable_GetExecutable(&g);
    PJRT_Executable_Serialize_Args s = {sizeof s, NULL, g.executable};
    rc2 = code_of(api, api->PJRT_Executable_Serialize(&s));
    if (!rc2) {
      PJRT_Executable_DeserializeAndLoad_Args d = {sizeof d, NULL, cc.client, s.serialized_bytes,
                                                   s.serialized_bytes_size};
      rc2 = code_of(api, api->PJRT_Executable_DeserializeAndLoad(&d));
      s.serialized_executable_deleter(s.serialized_executable);
      if (!rc2) {
        PJRT_LoadedExecutable_Destroy_Args x = {sizeof x, NULL, d.loaded_executable};
        api->PJRT_LoadedExecutable_Destroy(&x);
      }
    }
    PJRT_Executable_Destroy_Args e = {sizeof e, NULL, g.executable};
    api->PJRT_Executable_Destroy(&e);
    PJRT_LoadedExecutable_Destroy_Args x = {sizeof x, NULL, ca.executable};
    api->PJRT_LoadedExecutable_Destroy(&x);
  }
  PJRT_Client_Destroy_Args cd = {sizeof cd, NULL, cc.client};
  api->PJRT_Client_Destroy(&cd);
  printf("%d %d %d\n", rc, rc2, ((int (*)(void))dlsym(capi, "mlir_stub_live"))());
  free(code);
  return 0;
}
"""


def test_client_compile_bytecode_via_mlir_capi_in_c_host(tmp_path):
    """A C host without Python holding an MLIR C API (the test double in
    tests/capi/) compiles portable-artifact bytes with Client_Compile, then
    serializes and reloads the executable."""
    import subprocess

    from jax_mlx_amd import pjrt

    repo = Path(__file__).resolve().parents[1]
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{repo / 'include'}", "-x", "c", "-",
                    "-o", str(tmp_path / "host"), "-ldl"], input=COMPILE_HOST, text=True, check=True)
    subprocess.run(["gcc", "-std=c11", "-shared", "-fPIC", str(repo / "tests" / "capi" / "mlir_capi_stub.c"),
                    "-o", str(tmp_path / "libstub.so")], check=True)
    prog = tmp_path / "prog.bin"
    for tag, want in ((b"VHLO:", "0 0 0"), (b"PARSE:", "0 0 0"), (b"junk", "12 -1 0")):
        prog.write_bytes(b"ML\xefR" + tag + M.layer_norm_module().encode())
        out = subprocess.run([str(tmp_path / "host"), str(pjrt.PLUGIN_LIB), str(tmp_path / "libstub.so"),
                              str(prog)], capture_output=True, text=True, timeout=120)
        assert out.returncode == 0, (out.returncode, out.stderr)
        assert out.stdout.split("\n")[0] == want, (tag, out.stdout, out.stderr)


def test_escaping_intermediates_layer_norm(client, oracle):
    """Escape guard (reference src/jax_mlx_pjrt.cpp:1843-1855): a LayerNorm
    whose mean and variance are also results.  The fusion fires and the
    escaping values keep their own ops; all three results are checked."""
    rng = np.random.default_rng(21)
    x = rng.standard_normal((64, 512)).astype(np.float32) * 2 + 0.5
    g = (1 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    b = (0.1 * rng.standard_normal(512)).astype(np.float32)
    y, mean, var = run(client, M.layer_norm_escape_module((64, 512)), [x, g, b], ["f32"] * 3)
    x64 = x.astype(np.float64)
    assert np.abs(y - oracle.layer_norm(x, g, b, 1e-5)).max() <= F32_NORM_TOL
    assert np.abs(mean[..., 0] - x64.mean(-1)).max() <= F32_NORM_TOL
    assert np.abs(var[..., 0] - x64.var(-1)).max() <= F32_NORM_TOL * max(1.0, x64.var(-1).max())


def test_escaping_intermediates_sdpa_probs(client, oracle):
    """An attention module that also returns its softmax probabilities: the
    SDPA fusion still runs for the output, and the escaping probabilities are
    computed by their own ops.  Both results against the fp64 oracle (the
    probabilities: softmax of the scaled scores)."""
    rng = np.random.default_rng(22)
    B, H, T, D = 2, 2, 64, 64
    q, k, v = (rng.standard_normal((B, H, T, D)).astype(np.float32) for _ in range(3))
    o, p = run(client, M.sdpa_bhtd_module(B=B, H=H, T=T, D=D, return_probs=True), [q, k, v], ["f32"] * 3)
    assert np.abs(o - oracle.sdpa(q, k, v, 0.125)).max() <= F32_SDPA_TOL
    s = np.einsum("bhtd,bhsd->bhts", q.astype(np.float64), k.astype(np.float64)) * 0.125
    assert np.abs(p - oracle.softmax(s)).max() <= F32_NORM_TOL


# ---------------------------------------------------------------- client API

def test_buffers_views_strides_and_reexecution(client, oracle, cuda):
    torch = cuda
    rng = np.random.default_rng(9)
    exe = client.compile(M.layer_norm_module(shape=(64, 256)))
    assert exe.num_outputs == 1 and exe.output_dims == [(64, 256)]
    from jax_mlx_amd import pjrt

    assert exe.output_types == [pjrt.F32]
    g = (1 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    b = (0.1 * rng.standard_normal(256)).astype(np.float32)
    gb, bb = client.buffer_from_host(g), client.buffer_from_host(b)
    for trial in range(2):
        x = rng.standard_normal((64, 256)).astype(np.float32)
        # x from a column-major host array through byte_strides
        xt = torch.from_numpy(np.asfortranarray(x))  # element strides (1, 64)
        assert xt.stride() == (1, 64)
        xb = client.buffer_from_host(xt, byte_strides=[4 * s for s in xt.stride()])
        assert xb.dims == (64, 256) and xb.type == pjrt.F32
        (y,) = exe.execute([xb, gb, bb])
        assert np.abs(y.to_torch().numpy() - oracle.layer_norm(x, g, b, 1e-5)).max() <= F32_NORM_TOL
        # the same through a zero-copy view of a device tensor
        xd = torch.from_numpy(x).cuda()
        (y2,) = exe.execute([client.buffer_view(xd), gb, bb])
        assert np.array_equal(y2.to_torch().numpy(), y.to_torch().numpy())
    cost = exe.cost_analysis()
    assert "flops" in cost
    exe.destroy()


def test_buffers_and_executables_outlive_client(cuda):
    """Destroying the client before its buffers and executables is legal: the
    plugin keeps the client alive until the last of them is destroyed."""
    from jax_mlx_amd import pjrt

    c = pjrt.Client()
    exe = c.compile(M.softmax_module())
    x = np.arange(6 * 64, dtype=np.float32).reshape(6, 64) / 100
    xb = c.buffer_from_host(x)
    (y,) = exe.execute([xb])
    c.destroy()
    out = y.to_torch().numpy()
    np.testing.assert_allclose(out.sum(axis=-1), 1.0, rtol=1e-5)
    for b in (xb, y):
        b.destroy()
    exe.destroy()


def test_wrong_argument_count_and_type(client):
    import torch

    from jax_mlx_amd import pjrt

    exe = client.compile(M.softmax_module())
    with pytest.raises(pjrt.PjrtError) as e:
        exe.execute([])
    assert e.value.code_name == "INVALID_ARGUMENT"
    bad = client.buffer_from_host(torch.zeros((6, 64), dtype=torch.int32))
    with pytest.raises(pjrt.PjrtError) as e:
        exe.execute([bad])
    assert e.value.code_name == "INVALID_ARGUMENT"
    exe.destroy()
