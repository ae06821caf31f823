"""GPU parity of the f16 (IEEE half) paths against the fp64 oracle.

The reference hands f16 tensors to the same MLX fast ops as bf16 (dtype map
src/jax_mlx_pjrt.cpp:317-349; sdpa :4438-4446, :8108-8150; layer_norm :4436;
rms_norm :4428).  Here f16 runs on the bf16 kernels' schedules with the f16
forms of the four type-dependent operations (v_mfma_f32_32x32x16_f16, f16
packing of P, v_dot2_f32_f16 row sums, f16 output rounding).

Bar: ||out - ref||_inf / ||ref||_inf <= 5e-3 (F16_REL_TOL) per output, with
the oracle fed exactly the f16 values the kernel consumed.  f16 keeps 11
significant bits against bf16's 8, so the bar is four times tighter than the
bf16 one (2e-2); a kernel that rounded P or the output to bf16 by mistake
(3 fewer bits, errors ~4e-3 relative per element, more after the sums) or
used the bf16 MFMA on f16 bits (garbage) fails it.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F16_REL_TOL = 5e-3


@pytest.fixture(scope="module")
def nat(cuda):
    from jax_mlx_amd import native

    native.load()
    return native


def dev(torch, a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy().astype(np.float64)


def rel_inf(out, ref):
    return np.abs(out - ref).max() / np.abs(ref).max()


def check(out, ref, tol=F16_REL_TOL):
    out = host(out) if not isinstance(out, np.ndarray) else out
    assert np.isfinite(out).all()
    r = rel_inf(out, ref)
    assert r <= tol, r


def make_qkv(torch, seed, qshape, kshape, vshape=None):
    rng = np.random.default_rng(seed)
    return tuple(dev(torch, rng.standard_normal(s), torch.float16) for s in (qshape, kshape, vshape or kshape))


# ------------------------------------------------------------- prefill

@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("tq,tk,hq,hkv,causal", [(100, 77, 3, 3, False), (100, 77, 4, 2, True),
                                                 (77, 200, 2, 1, True), (129, 129, 3, 3, True),
                                                 (1000, 1000, 2, 2, False), (7, 300, 4, 4, False)])
def test_sdpa_f16_flash_ragged_gqa(cuda, nat, oracle, D, tq, tk, hq, hkv, causal):
    """The pipelined flash kernel on f16: ragged Tq / Tk against the 128-row
    block and 64-key tile, causal, GQA."""
    q, k, v = make_qkv(cuda, 7, (2, hq, tq, D), (2, hkv, tk, D))
    assert nat.sdpa_kernel_name(q, k, v, causal=causal) == f"flash_f16_d{D}"
    out = nat.sdpa(q, k, v, scale=D ** -0.5, causal=causal)
    assert out.dtype == cuda.float16
    check(out, oracle.sdpa(host(q), host(k), host(v), D ** -0.5, causal=causal))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("case", ["spike_15_5", "near_max", "beyond_max", "tile_at_14", "growing"])
@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_f16_rebase_bounds(cuda, nat, oracle, D, case, causal):
    """Scores above the row's exp2 base by amounts placed around f16's
    range.  A probability exp2(s - base) must stay finite in f16 (<= 65504):
    the kernel raises the base of a row whose 32-key lane sum passes 2^15.
    Feature 0 of q is 1 and the scale is 1/log2(e), so a key's score in log2
    units is its feature 0 (the other features are zero for q); keys 0-63
    (the first tile, which sets the base) score in [-1, 0].  Cases: one key
    15.5 above the base (p = 46341, finite, its lane sum past 2^15), one at
    15.95 (p = 63,550, just under f16's maximum), one at 17 (p = 131072,
    which f16 would round to inf), a whole later tile at 14 (each p = 16384,
    lane sums 2^19), and scores growing along the keys by 40 in total."""
    B, H, T = 1, 2, 600
    rng = np.random.default_rng(33)
    q = np.zeros((B, H, T, D))
    q[..., 0] = 1.0
    k = rng.standard_normal((B, H, T, D)) * 0.1
    k[..., 0] = -rng.random((B, H, T))
    key = {"spike_15_5": (15.5, 300), "near_max": (15.95, 450), "beyond_max": (17.0, 200)}
    if case in key:
        val, pos = key[case]
        k[:, :, pos, 0] = val
    elif case == "tile_at_14":
        k[:, :, 256:320, 0] = 14.0
    else:
        k[..., 0] += 40.0 * np.arange(T) / T
    v = rng.standard_normal((B, H, T, D))
    qd, kd, vd = (dev(cuda, a, cuda.float16) for a in (q, k, v))
    scale = 1.0 / np.log2(np.e)
    assert nat.sdpa_kernel_name(qd, kd, vd, causal=causal) == f"flash_f16_d{D}"
    out = nat.sdpa(qd, kd, vd, scale=scale, causal=causal)
    check(out, oracle.sdpa(host(qd), host(kd), host(vd), scale, causal=causal))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("mdt", ["f32", "f16"])
@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_f16_row_shared_mask(cuda, nat, oracle, D, mdt, causal):
    """Padding mask [B,1,1,S] (row-shared, the pipelined kernel's mask
    path): lengths per batch, -inf past them, finite biases before."""
    rng = np.random.default_rng(41)
    B, H, T = 3, 2, 333
    q, k, v = make_qkv(cuda, 42, (B, H, T, D), (B, H, T, D))
    lens = np.array([333, 130, 65])
    m = rng.standard_normal((B, 1, 1, T)) * 0.5
    m[np.arange(T)[None, None, None, :] >= lens[:, None, None, None]] = -np.inf
    td = cuda.float32 if mdt == "f32" else cuda.float16
    maskd = dev(cuda, m, td)
    assert nat.sdpa_kernel_name(q, k, v, mask=maskd, causal=causal) == f"flash_f16_d{D}"
    out = nat.sdpa(q, k, v, scale=D ** -0.5, mask=maskd, causal=causal)
    check(out, oracle.sdpa(host(q), host(k), host(v), D ** -0.5, causal=causal, mask=host(maskd)))


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_f16_per_row_mask(cuda, nat, oracle, D, causal):
    """A mask that varies along query rows ([B,1,T,S], -inf holes): the
    non-pipelined flash kernel's path."""
    rng = np.random.default_rng(43)
    B, H, T, S = 2, 4, 150, 170
    q, k, v = make_qkv(cuda, 44, (B, H, T, D), (B, H, S, D))
    m = rng.standard_normal((B, 1, T, S)) * 0.5
    m[..., ::7] = -np.inf
    m[..., 0] = 0.0
    maskd = dev(cuda, m, cuda.float16)
    assert nat.sdpa_kernel_name(q, k, v, mask=maskd, causal=causal) == f"flash_f16_d{D}"
    out = nat.sdpa(q, k, v, scale=0.11, mask=maskd, causal=causal)
    check(out, oracle.sdpa(host(q), host(k), host(v), 0.11, causal=causal, mask=host(maskd)))


def test_sdpa_f16_btnh_layout(cuda, nat, oracle):
    rng = np.random.default_rng(45)
    B, T, Hq, Hkv, D = 2, 150, 8, 2, 64
    q = dev(cuda, rng.standard_normal((B, T, Hq, D)), cuda.float16)
    k = dev(cuda, rng.standard_normal((B, T, Hkv, D)), cuda.float16)
    v = dev(cuda, rng.standard_normal((B, T, Hkv, D)), cuda.float16)
    out = nat.sdpa(q, k, v, scale=0.2, causal=True, layout="bthd")
    qh, kh, vh = (host(t).transpose(0, 2, 1, 3) for t in (q, k, v))
    ref = oracle.sdpa(qh, kh, vh, 0.2, causal=True).transpose(0, 2, 1, 3)
    check(out, ref)


def test_sdpa_f16_generic_head_size_and_fused_qnorm_prefill(cuda, nat, oracle):
    """Head size 80 with Dv 48 (the shape-general kernel), and a prefill with
    a fused q RMSNorm (the normalised copy of q, rounded to f16)."""
    q, k, v = make_qkv(cuda, 11, (2, 4, 33, 80), (2, 2, 45, 80), (2, 2, 45, 48))
    assert nat.sdpa_kernel_name(q, k, v) == "generic"
    out = nat.sdpa(q, k, v, scale=0.15, causal=True)
    check(out, oracle.sdpa(host(q), host(k), host(v), 0.15, causal=True))
    q, k, v = make_qkv(cuda, 12, (2, 4, 200, 64), (2, 4, 200, 64))
    w = dev(cuda, 1 + 0.1 * np.random.default_rng(13).standard_normal(64), cuda.float16)
    out = nat.sdpa(q, k, v, scale=0.125, causal=True, q_rms_eps=1e-6, q_rms_weight=w)
    qn = oracle.rms_norm(host(q), host(w), 1e-6)
    qn = host(cuda.from_numpy(qn.astype(np.float32)).half())
    check(out, oracle.sdpa(qn, host(k), host(v), 0.125, causal=True))


# -------------------------------------------------------------- decode

@pytest.mark.parametrize("hq,hkv,tq,D,tk", [(32, 1, 1, 128, 64), (16, 2, 4, 64, 1000), (8, 8, 1, 128, 4097),
                                            (32, 4, 4, 128, 777), (4, 2, 1, 64, 1)])
def test_sdpa_f16_decode_mfma(cuda, nat, oracle, hq, hkv, tq, D, tk):
    q, k, v = make_qkv(cuda, 21, (2, hq, tq, D), (2, hkv, tk, D))
    assert nat.sdpa_kernel_name(q, k, v) == "decode_splitkv_mfma"
    out = nat.sdpa(q, k, v, scale=D ** -0.5)
    check(out, oracle.sdpa(host(q), host(k), host(v), D ** -0.5))
    out_c = nat.sdpa(q, k, v, scale=D ** -0.5, causal=True)
    check(out_c, oracle.sdpa(host(q), host(k), host(v), D ** -0.5, causal=True))


@pytest.mark.parametrize("mdt", ["f16", "f32"])
def test_sdpa_f16_decode_mfma_mask_and_qnorm(cuda, nat, oracle, mdt):
    """Config 5's chain on f16: q RMSNorm (weight) then GQA decode over a
    length-masked cache, plus a per-row mask with holes."""
    rng = np.random.default_rng(51)
    B, Hq, Hkv, S, D = 4, 16, 4, 3000, 128
    q, k, v = make_qkv(cuda, 52, (B, Hq, 1, D), (B, Hkv, S, D))
    lens = np.array([3000, 1200, 64, 2047])
    m = np.where(np.arange(S)[None] < lens[:, None], 0.0, -np.inf).reshape(B, 1, 1, S)
    td = cuda.float32 if mdt == "f32" else cuda.float16
    maskd = dev(cuda, m, td)
    w = dev(cuda, 1 + 0.1 * rng.standard_normal(D), cuda.float16)
    assert nat.sdpa_kernel_name(q, k, v, mask=maskd, q_rms_eps=1e-6, q_rms_weight=w) == "decode_splitkv_mfma"
    out = nat.sdpa(q, k, v, scale=D ** -0.5, mask=maskd, q_rms_eps=1e-6, q_rms_weight=w)
    qn = oracle.rms_norm(host(q), host(w), 1e-6)
    qn = host(cuda.from_numpy(qn.astype(np.float32)).half())
    check(out, oracle.sdpa(qn, host(k), host(v), D ** -0.5, mask=m))
    pm = rng.standard_normal((B, Hq, 2, S)) * 0.5
    pm[..., 9::9] = -np.inf  # holes; key 0 stays visible (causal row 0 sees only it)
    q2, _, _ = make_qkv(cuda, 53, (B, Hq, 2, D), (1, 1, 1, D))
    pmd = dev(cuda, pm, td)
    assert nat.sdpa_kernel_name(q2, k, v, mask=pmd) == "decode_splitkv_mfma"
    out2 = nat.sdpa(q2, k, v, scale=0.1, mask=pmd, causal=True)
    check(out2, oracle.sdpa(host(q2), host(k), host(v), 0.1, mask=host(pmd), causal=True))


def test_sdpa_f16_decode_valu_and_broadcast_rows(cuda, nat, oracle):
    """K as a broadcast view (row stride 0): the MFMA decode does not take
    it, the VALU split-KV decode does; a prefill with broadcast V runs on the
    generic kernel, every output row equal to that V row."""
    q, k, v = make_qkv(cuda, 61, (2, 8, 2, 64), (2, 2, 2000, 64))
    kb = k[:, :, :1].expand(2, 2, 2000, 64)
    assert nat.sdpa_kernel_name(q, kb, v) == "decode_splitkv"
    out = nat.sdpa(q, kb, v, scale=0.125)
    check(out, oracle.sdpa(host(q), host(kb), host(v), 0.125))
    q, k, v = make_qkv(cuda, 62, (2, 4, 96, 64), (2, 4, 96, 64))
    vb = v[:, :, :1].expand(2, 4, 96, 64)
    assert nat.sdpa_kernel_name(q, k, vb) == "generic"
    out = nat.sdpa(q, k, vb, scale=0.125)
    check(out, oracle.sdpa(host(q), host(k), host(vb), 0.125))
    assert float(np.abs(host(out) - host(vb)).max()) <= 2e-3


# ------------------------------------------------------------ backward

def bwd_case(cuda, nat, oracle, seed, qshape, kshape, *, causal=False, scale=None, mask=None, vshape=None,
             layout="bhtd"):
    q, k, v = make_qkv(cuda, seed, qshape, kshape, vshape)
    rng = np.random.default_rng(seed + 100)
    oshape = list(qshape)
    oshape[-1] = (vshape or kshape)[-1]
    g = dev(cuda, rng.standard_normal(oshape), cuda.float16)
    grads = nat.sdpa_bwd(q, k, v, g, scale=scale, causal=causal, mask=mask, layout=layout)
    tr = (lambda a: a.transpose(0, 2, 1, 3)) if layout == "bthd" else (lambda a: a)
    sc = scale if scale is not None else 1.0 / np.sqrt(qshape[-1])
    refs = oracle.sdpa_bwd(tr(host(q)), tr(host(k)), tr(host(v)), tr(host(g)), sc, causal=causal,
                           mask=None if mask is None else host(mask))
    for name, o, r in zip(("dq", "dk", "dv"), grads, refs):
        assert o.dtype == cuda.float16
        rr = rel_inf(host(o), tr(r))
        assert rr <= F16_REL_TOL, (name, rr)
    return q, k, v


@pytest.mark.parametrize("D,tq,tk,causal", [(128, 64, 64, True), (64, 256, 256, False), (128, 200, 200, True),
                                            (64, 77, 130, False), (128, 1, 33, False)])
def test_sdpa_f16_bwd_mfma(cuda, nat, oracle, D, tq, tk, causal):
    q, k, v = make_qkv(cuda, 31, (1, 2, tq, D), (1, 2, tk, D))
    assert nat.sdpa_bwd_kernel_name(q, k, v, causal=causal) == f"mfma_f16_d{D}"
    bwd_case(cuda, nat, oracle, 31, (1, 2, tq, D), (1, 2, tk, D), causal=causal)


def test_sdpa_f16_bwd_btnh_gqa_mask(cuda, nat, oracle):
    rng = np.random.default_rng(41)
    m = rng.standard_normal((2, 1, 96, 160)).astype(np.float32)
    m[:, :, :, 5] = -np.inf
    mask = dev(cuda, m, cuda.float16)
    bwd_case(cuda, nat, oracle, 42, (2, 96, 8, 64), (2, 160, 2, 64), mask=mask, layout="bthd", scale=0.2)


@pytest.mark.parametrize("D,tq,tk,causal", [(32, 64, 64, True), (96, 200, 200, True), (96, 77, 130, False),
                                            (32, 1, 33, False)])
def test_sdpa_f16_bwd_padded_head_sizes(cuda, nat, oracle, D, tq, tk, causal):
    """Head sizes 32 / 96 on the matrix-core backward through zero-padded
    64- / 128-feature copies."""
    q, k, v = make_qkv(cuda, 33, (1, 2, tq, D), (1, 2, tk, D))
    assert nat.sdpa_bwd_kernel_name(q, k, v, causal=causal) == f"mfma_f16_d{D}"
    bwd_case(cuda, nat, oracle, 33, (1, 2, tq, D), (1, 2, tk, D), causal=causal)


def test_sdpa_f16_bwd_generic_head_size(cuda, nat, oracle):
    q, k, v = make_qkv(cuda, 43, (1, 3, 50, 80), (1, 3, 70, 80))
    assert nat.sdpa_bwd_kernel_name(q, k, v, causal=True) == "generic"
    bwd_case(cuda, nat, oracle, 43, (1, 3, 50, 80), (1, 3, 70, 80), causal=True, vshape=(1, 3, 70, 48))


# --------------------------------------------------------------- norms

@pytest.mark.parametrize("shape", [(8, 128, 512), (33, 128), (4, 4096), (3, 40), (2, 20000), (3, 77),
                                   (2, 40000)])
@pytest.mark.parametrize("pdt", ["f16", "f32"])
def test_layer_norm_rms_norm_f16(cuda, nat, oracle, shape, pdt):
    """LayerNorm and RMSNorm of f16 rows with f16 or f32 parameters: the
    vector kernels (rows of a multiple of 8 elements, at most 4096 16-byte
    vectors: 16-, 64- and 256-lane row owners) and the looped kernel (77
    elements, not a multiple of 8; 40000, past 4096 vectors)."""
    rng = np.random.default_rng(71)
    x = dev(cuda, rng.standard_normal(shape) * 3 + 1, cuda.float16)
    pt = cuda.float16 if pdt == "f16" else cuda.float32
    g = dev(cuda, 1 + 0.1 * rng.standard_normal(shape[-1]), pt)
    b = dev(cuda, 0.1 * rng.standard_normal(shape[-1]), pt)
    y = nat.layer_norm(x, g, b, eps=1e-5)
    assert y.dtype == cuda.float16
    check(y, oracle.layer_norm(host(x), host(g), host(b), 1e-5))
    yr = nat.rms_norm(x, g, eps=1e-6)
    check(yr, oracle.rms_norm(host(x), host(g), 1e-6))


def test_layer_norm_f16_mixed_param_types_and_strides(cuda, nat, oracle):
    """bf16 rows with f16 parameters, and f16 rows with bf16 parameters: the
    looped kernel (parameter loads of any type); strided f16 rows."""
    rng = np.random.default_rng(72)
    xb = dev(cuda, rng.standard_normal((17, 256)), cuda.bfloat16)
    gh = dev(cuda, 1 + 0.1 * rng.standard_normal(256), cuda.float16)
    y = nat.layer_norm(xb, gh, eps=1e-5)
    assert rel_inf(host(y), oracle.layer_norm(host(xb), host(gh), None, 1e-5)) <= 2e-2
    xh = dev(cuda, rng.standard_normal((17, 256)), cuda.float16)
    gb = dev(cuda, 1 + 0.1 * rng.standard_normal(256), cuda.bfloat16)
    check(nat.layer_norm(xh, gb, eps=1e-5), oracle.layer_norm(host(xh), host(gb), None, 1e-5))
    big = dev(cuda, rng.standard_normal((64, 1024)), cuda.float16)
    xs = big[:, 256:768]
    check(nat.layer_norm(xs, eps=1e-5), oracle.layer_norm(host(xs), None, None, 1e-5))


@pytest.mark.parametrize("shape", [(6, 64), (4, 1000), (3, 2048), (2, 12)])
def test_softmax_log_softmax_f16(cuda, nat, oracle, shape):
    rng = np.random.default_rng(73)
    x = rng.standard_normal(shape) * 4
    x[0, 1] = -np.inf
    xd = dev(cuda, x, cuda.float16)
    check(nat.softmax(xd), oracle.softmax(host(xd)))
    y = host(nat.log_softmax(xd))
    ref = oracle.log_softmax(host(xd))
    assert np.isneginf(y[0, 1]) and np.isneginf(ref[0, 1])
    ok = np.isfinite(ref)
    assert rel_inf(y[ok], ref[ok]) <= F16_REL_TOL


@pytest.mark.parametrize("shape", [(8, 128, 512), (33, 128), (4, 4096), (5, 8200), (9, 30)])
@pytest.mark.parametrize("pdt", ["f16", "f32"])
def test_layer_norm_bwd_f16(cuda, nat, oracle, shape, pdt):
    rng = np.random.default_rng(74)
    n = shape[-1]
    x = dev(cuda, rng.standard_normal(shape) * 2 + 0.5, cuda.float16)
    dy = dev(cuda, rng.standard_normal(shape), cuda.float16)
    pt = cuda.float16 if pdt == "f16" else cuda.float32
    g = dev(cuda, 1 + 0.1 * rng.standard_normal(n), pt)
    dx, dg, db = nat.layer_norm_bwd(x, dy, g, eps=1e-5)
    assert dx.dtype == cuda.float16 and dg.dtype == pt
    refs = oracle.layer_norm_bwd(host(x).reshape(-1, n), host(g), host(dy).reshape(-1, n), 1e-5)
    for o, r in zip((dx, dg, db), refs):
        check(host(o).reshape(r.shape), r)
