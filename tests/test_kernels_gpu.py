"""GPU parity of the libmfx_kernels.so kernels against the fp64 oracle.

Bars: f32 max-abs error <= 1e-5 for the norms and
<= 1e-4 for SDPA; bf16 (fp32 accumulation) ||out - ref||_inf / ||ref||_inf
<= 2e-2.  The oracle sees exactly the values the kernel consumed (bf16 inputs
rounded first).  Inputs come from numpy.random.default_rng(<config#>) in the
order the BASELINE configs list them.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32_NORM_TOL = 1e-5
F32_SDPA_TOL = 1e-4
BF16_REL_TOL = 2e-2


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


# ---------------------------------------------------------------- norms

@pytest.mark.parametrize("shape", [(8, 128, 512), (3, 8), (5, 100), (1025, 512), (7, 1000),
                                   (4, 4096), (3, 6000), (2, 20000), (2, 64)])
def test_layer_norm_f32(cuda, nat, oracle, shape):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(shape).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(shape[-1])).astype(np.float32)
    b = (0.1 * rng.standard_normal(shape[-1])).astype(np.float32)
    xd, gd, bd = (dev(cuda, a, cuda.float32) for a in (x, g, b))
    y = host(nat.layer_norm(xd, gd, bd, eps=1e-5))
    ref = oracle.layer_norm(x, g, b, 1e-5)
    assert np.abs(y - ref).max() <= F32_NORM_TOL
    y0 = host(nat.layer_norm(xd, eps=1e-5))
    assert np.abs(y0 - oracle.layer_norm(x, None, None, 1e-5)).max() <= F32_NORM_TOL


@pytest.mark.parametrize("shape", [(8, 128, 512), (33, 128), (4, 4096), (3, 40)])
def test_layer_norm_bf16(cuda, nat, oracle, shape):
    rng = np.random.default_rng(2)
    x = rng.standard_normal(shape).astype(np.float32) * 3 + 1
    g = (1 + 0.1 * rng.standard_normal(shape[-1])).astype(np.float32)
    b = (0.1 * rng.standard_normal(shape[-1])).astype(np.float32)
    xd = dev(cuda, x, cuda.bfloat16)
    gd, bd = dev(cuda, g, cuda.float32), dev(cuda, b, cuda.float32)
    y = host(nat.layer_norm(xd, gd, bd, eps=1e-5))
    ref = oracle.layer_norm(host(xd), g, b, 1e-5)
    assert rel_inf(y, ref) <= BF16_REL_TOL
    # bf16 parameters too
    y2 = host(nat.layer_norm(xd, gd.bfloat16(), bd.bfloat16(), eps=1e-5))
    ref2 = oracle.layer_norm(host(xd), host(gd.bfloat16()), host(bd.bfloat16()), 1e-5)
    assert rel_inf(y2, ref2) <= BF16_REL_TOL


def test_layer_norm_strided_rows_and_constant_rows(cuda, nat, oracle):
    rng = np.random.default_rng(3)
    big = dev(cuda, rng.standard_normal((64, 1024)), cuda.float32)
    x = big[:, 256:768]  # row stride 1024, 512 elements per row
    y = host(nat.layer_norm(x, eps=1e-5))
    assert np.abs(y - oracle.layer_norm(host(x), None, None, 1e-5)).max() <= F32_NORM_TOL
    beta = dev(cuda, rng.standard_normal(512), cuda.float32)
    c = cuda.full((4, 512), 3.0, device="cuda")
    yc = nat.layer_norm(c, None, beta, eps=1e-5)
    assert cuda.equal(yc, beta.expand(4, 512))



# ------------------------------------------------------- LayerNorm backward
# mfx_layer_norm_bwd against the fp64 oracle (reference closed form
# src/jax_mlx/layer_norm.py:59-76).  f32: ||out - ref||_inf <= 1e-5 *
# max(1, ||ref||_inf) for dx, dgamma and dbeta (the parameter sums add up to
# 65536 rows); bf16 inputs: the bf16 relative bar.

def _ln_bwd_case(cuda, nat, oracle, shape, dtype, pdtype, seed, gamma=True):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float32) * 2 + 0.5
    dy = rng.standard_normal(shape).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(shape[-1])).astype(np.float32)
    xd, dyd = dev(cuda, x, dtype), dev(cuda, dy, dtype)
    gd = dev(cuda, g, pdtype) if gamma else None
    dx, dg, db = nat.layer_norm_bwd(xd, dyd, gd, eps=1e-5, param_dtype=pdtype)
    n = shape[-1]
    ref = oracle.layer_norm_bwd(host(xd).reshape(-1, n), host(gd) if gamma else None,
                                host(dyd).reshape(-1, n), 1e-5)
    return [host(t).reshape(r.shape) for t, r in zip((dx, dg, db), ref)], ref


def _check_f32(outs, refs, tol=F32_NORM_TOL):
    for o, r in zip(outs, refs):
        assert np.abs(o - r).max() <= tol * max(1.0, np.abs(r).max()), np.abs(o - r).max()


@pytest.mark.parametrize("shape", [(8, 128, 512), (3, 8), (5, 100), (1025, 512), (7, 1000),
                                   (4, 4096), (3, 6000), (2, 64), (33, 77), (65536, 64)])
def test_layer_norm_bwd_f32(cuda, nat, oracle, shape):
    outs, refs = _ln_bwd_case(cuda, nat, oracle, shape, cuda.float32, cuda.float32, 11)
    _check_f32(outs, refs)


@pytest.mark.parametrize("shape", [(8, 128, 512), (33, 128), (4, 4096), (3, 40), (5, 8200), (9, 30)])
@pytest.mark.parametrize("pbf16", [False, True])
def test_layer_norm_bwd_bf16(cuda, nat, oracle, shape, pbf16):
    outs, refs = _ln_bwd_case(cuda, nat, oracle, shape, cuda.bfloat16,
                              cuda.bfloat16 if pbf16 else cuda.float32, 12)
    for o, r in zip(outs, refs):
        assert rel_inf(o, r) <= BF16_REL_TOL


def test_layer_norm_bwd_without_gamma_strided_and_empty(cuda, nat, oracle):
    outs, refs = _ln_bwd_case(cuda, nat, oracle, (64, 256), cuda.float32, cuda.float32, 13, gamma=False)
    _check_f32(outs, refs)
    rng = np.random.default_rng(14)
    big = dev(cuda, rng.standard_normal((48, 1024)), cuda.float32)
    gbig = dev(cuda, rng.standard_normal((48, 768)), cuda.float32)
    x, dy = big[:, 256:768], gbig[:, 128:640]  # row strides 1024 and 768
    gam = dev(cuda, 1 + 0.1 * rng.standard_normal(512), cuda.float32)
    dx, dg, db = nat.layer_norm_bwd(x, dy, gam, eps=1e-5)
    ref = oracle.layer_norm_bwd(host(x), host(gam), host(dy), 1e-5)
    _check_f32([host(dx), host(dg), host(db)], ref)
    # dx only: the parameter sums are skipped, dx is unchanged.
    dx2, dg2, db2 = nat.layer_norm_bwd(x, dy, gam, eps=1e-5, param_grads=False)
    assert dg2 is None and db2 is None
    assert np.array_equal(host(dx2), host(dx))
    # No rows: dx is empty and the parameter gradients are zero sums.
    e = cuda.empty((0, 512), device="cuda")
    dx3, dg3, db3 = nat.layer_norm_bwd(e, e, gam, eps=1e-5)
    assert dx3.numel() == 0 and np.all(host(dg3) == 0) and np.all(host(db3) == 0)
    # Caller workspace of the queried size gives identical results.
    ws = cuda.empty(nat.layer_norm_bwd_workspace_size(x, gam), dtype=cuda.uint8, device="cuda")
    dx4, dg4, db4 = nat.layer_norm_bwd(x, dy, gam, eps=1e-5, workspace=ws)
    assert np.array_equal(host(dg4), host(dg)) and np.array_equal(host(db4), host(db))


@pytest.mark.parametrize("dtype,shape", [("f32", (2, 4, 128)), ("f32", (9, 4096)), ("f32", (3, 77)),
                                         ("bf16", (16, 32, 1, 128)), ("bf16", (5, 2048))])
def test_rms_norm(cuda, nat, oracle, dtype, shape):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(shape).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(shape[-1])).astype(np.float32)
    td = cuda.float32 if dtype == "f32" else cuda.bfloat16
    xd, wd = dev(cuda, x, td), dev(cuda, w, td)
    y = host(nat.rms_norm(xd, wd, eps=1e-6))
    ref = oracle.rms_norm(host(xd), host(wd), 1e-6)
    if dtype == "f32":
        assert np.abs(y - ref).max() <= F32_NORM_TOL
    else:
        assert rel_inf(y, ref) <= BF16_REL_TOL
    # x = c * 1 -> c / sqrt(c^2 + eps)
    c = cuda.full((3, shape[-1]), -2.0, device="cuda", dtype=cuda.float32)
    np.testing.assert_allclose(host(nat.rms_norm(c, eps=1e-6)), -2.0 / np.sqrt(4.0 + 1e-6), atol=1e-6)


@pytest.mark.parametrize("shape", [(6, 64), (4, 1000), (3, 2048), (2, 12)])
def test_softmax_f32(cuda, nat, oracle, shape):
    rng = np.random.default_rng(6)
    x = rng.standard_normal(shape).astype(np.float32) * 4
    x[0, 1] = -np.inf
    x[1, :] = -np.inf
    y = host(nat.softmax(dev(cuda, x, cuda.float32)))
    ref = oracle.softmax(x)
    assert np.isnan(y[1]).all()
    ok = np.ones(shape[0], bool)
    ok[1] = False
    assert np.abs(y[ok] - ref[ok]).max() <= F32_NORM_TOL
    np.testing.assert_allclose(host(nat.softmax(cuda.ones(1, 5, device="cuda"))), 0.2, atol=1e-7)


@pytest.mark.parametrize("shape,dtype", [((6, 64), "f32"), ((4, 1000), "f32"), ((3, 2048), "f32"), ((2, 12), "f32"),
                                         ((5, 6000), "f32"), ((33, 77), "f32"), ((8, 512), "bf16"), ((3, 40), "bf16")])
def test_log_softmax(cuda, nat, oracle, shape, dtype):
    """mfx_log_softmax against the fp64 oracle: f32 max-abs <= 1e-5 *
    max(1, |ref|) (log-probabilities reach -40 here); bf16 the relative bar."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal(shape).astype(np.float32) * 4
    x[0, 1] = -np.inf
    td = cuda.float32 if dtype == "f32" else cuda.bfloat16
    xd = dev(cuda, x, td)
    y = host(nat.log_softmax(xd))
    ref = oracle.log_softmax(host(xd))
    assert np.isneginf(y[0, 1]) and np.isneginf(ref[0, 1])
    ok = np.isfinite(ref)
    if dtype == "f32":
        assert np.abs(y[ok] - ref[ok]).max() <= F32_NORM_TOL * max(1.0, np.abs(ref[ok]).max())
    else:
        assert rel_inf(y[ok], ref[ok]) <= BF16_REL_TOL


# ---------------------------------------------------------------- SDPA

def make_qkv(torch, seed, qshape, kshape, dtype, vshape=None):
    rng = np.random.default_rng(seed)
    q = dev(torch, rng.standard_normal(qshape), dtype)
    k = dev(torch, rng.standard_normal(kshape), dtype)
    v = dev(torch, rng.standard_normal(vshape or kshape), dtype)
    return q, k, v


def check_sdpa(out, ref, dtype):
    out = host(out)
    if dtype == "f32":
        err = np.abs(out - ref).max()
        assert err <= F32_SDPA_TOL, err
    else:
        r = rel_inf(out, ref)
        assert r <= BF16_REL_TOL, r


@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_f32_config2(cuda, nat, oracle, causal):
    q, k, v = make_qkv(cuda, 2, (8, 8, 128, 64), (8, 8, 128, 64), cuda.float32)
    assert nat.sdpa_kernel_name(q, k, v) == "flash_f32_split_d64"
    out = nat.sdpa(q, k, v, scale=0.125, causal=causal)
    check_sdpa(out, oracle.sdpa(host(q), host(k), host(v), 0.125, causal=causal), "f32")


@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_f32_d64_in_place_qkv_slices(cuda, nat, oracle, causal):
    """Config 4's attention as the plan runs it: q, k and v are BTNH views of
    one [B*T, 3*512] f32 QKV projection (row stride 1536, element offsets 0,
    512 and 1024), read in place by flash_f32_d64; B32 T256, 8 heads of 64."""
    B, T, N, H = 32, 256, 8, 64
    rng = np.random.default_rng(4)
    qkv = dev(cuda, rng.standard_normal((B * T, 3 * N * H)), cuda.float32)
    q, k, v = (qkv[:, j * N * H:(j + 1) * N * H].view(B, T, N, H) for j in range(3))
    assert q.stride() == (T * 3 * N * H, 3 * N * H, H, 1) and k.storage_offset() == N * H
    assert nat.sdpa_kernel_name(q, k, v, layout="bthd") == "flash_f32_d64"
    out = nat.sdpa(q, k, v, scale=H ** -0.5, causal=causal, layout="bthd")
    t = lambda a: np.ascontiguousarray(host(a).transpose(0, 2, 1, 3))  # noqa: E731
    ref = oracle.sdpa(t(q), t(k), t(v), H ** -0.5, causal=causal)
    check_sdpa(out.permute(0, 2, 1, 3), ref, "f32")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("tq,tk,hq,hkv,causal,masked", [(128, 128, 8, 8, False, False), (100, 77, 4, 2, True, False),
                                                        (33, 300, 4, 1, False, True), (77, 200, 2, 2, True, True),
                                                        (5, 1000, 4, 4, False, False), (31, 31, 4, 2, True, False)])
def test_sdpa_f32_key_split(cuda, nat, oracle, D, tq, tk, hq, hkv, causal, masked):
    """The key-split f32 kernel (four wavefronts per 32 query rows, partials
    merged through LDS): ragged lengths, GQA, causal and an additive mask
    with -inf holes, against the fp64 oracle."""
    q, k, v = make_qkv(cuda, 15, (2, hq, tq, D), (2, hkv, tk, D), cuda.float32)
    mask = None
    if masked:
        m = np.random.default_rng(16).standard_normal((2, 1, tq, tk)) * 0.5
        m[..., ::5] = -np.inf
        m[..., 0] = 0.0
        mask = m
    maskd = None if mask is None else dev(cuda, mask, cuda.float32)
    assert nat.sdpa_kernel_name(q, k, v, causal=causal, mask=maskd) == f"flash_f32_split_d{D}"
    out = nat.sdpa(q, k, v, scale=D ** -0.5, causal=causal, mask=maskd)
    check_sdpa(out, oracle.sdpa(host(q), host(k), host(v), D ** -0.5, causal=causal, mask=mask), "f32")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("tq,tk,causal", [(100, 77, False), (100, 77, True), (77, 200, True),
                                          (129, 129, True), (1000, 1000, False), (7, 300, False)])
def test_sdpa_flash_ragged(cuda, nat, oracle, dtype, D, tq, tk, causal):
    td = cuda.float32 if dtype == "f32" else cuda.bfloat16
    q, k, v = make_qkv(cuda, 7, (2, 3, tq, D), (2, 3, tk, D), td)
    out = nat.sdpa(q, k, v, scale=D ** -0.5, causal=causal)
    check_sdpa(out, oracle.sdpa(host(q), host(k), host(v), D ** -0.5, causal=causal), dtype)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sdpa_btnh_layout_gqa_and_mask(cuda, nat, oracle, dtype):
    td = cuda.float32 if dtype == "f32" else cuda.bfloat16
    rng = np.random.default_rng(8)
    B, T, S, Hq, Hkv, D = 2, 150, 150, 8, 2, 64
    q = dev(cuda, rng.standard_normal((B, T, Hq, D)), td)      # BTNH
    k = dev(cuda, rng.standard_normal((B, S, Hkv, D)), td)
    v = dev(cuda, rng.standard_normal((B, S, Hkv, D)), td)
    lens = np.array([150, 61])
    mask = np.where(np.arange(S)[None] < lens[:, None], 0.0, -np.inf).reshape(B, 1, 1, S)
    maskd = dev(cuda, mask, cuda.float32)
    out = nat.sdpa(q, k, v, scale=0.2, mask=maskd, layout="bthd")
    qh, kh, vh = (host(t).transpose(0, 2, 1, 3) for t in (q, k, v))
    ref = oracle.sdpa(qh, kh, vh, 0.2, mask=mask).transpose(0, 2, 1, 3)
    check_sdpa(out, ref, dtype)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("mdt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("kind", ["padding", "head_bias"])
def test_sdpa_flash_bf16_row_shared_mask(cuda, nat, oracle, D, mdt, causal, kind):
    """Additive masks that do not vary along query rows run on the pipelined
    bf16 kernel (the mask row seeds the S accumulators).  padding: [B,1,1,Tk]
    0 / -inf by sequence length, one batch with whole masked 64-key tiles;
    head_bias: [B,H,1,Tk] N(0,1) biases with -inf holes and a masked run.
    Ragged Tq / Tk, GQA, every mask dtype, causal or not, against the oracle."""
    td = cuda.bfloat16
    rng = np.random.default_rng(40 + D)
    B, Hq, Hkv, Tq, Tk = 2, 4, 2, 200, 333
    q, k, v = make_qkv(cuda, 41, (B, Hq, Tq, D), (B, Hkv, Tk, D), td)
    if kind == "padding":
        lens = np.array([Tk, 150])
        mask = np.where(np.arange(Tk)[None] < lens[:, None], 0.0, -np.inf).reshape(B, 1, 1, Tk)
    else:
        mask = rng.standard_normal((B, Hq, 1, Tk))
        mask[rng.random(mask.shape) < 0.1] = -np.inf
        mask[:, :, :, 64:128] = -np.inf          # a whole masked tile
        mask[:, :, :, 0] = 0.0                   # every row keeps key 0
    mdev = {"f32": cuda.float32, "bf16": cuda.bfloat16, "f16": cuda.float16}[mdt]
    maskd = dev(cuda, mask, cuda.float32).to(mdev)
    assert nat.sdpa_kernel_name(q, k, v, mask=maskd, causal=causal) == f"flash_bf16_d{D}"
    out = nat.sdpa(q, k, v, scale=D ** -0.5, mask=maskd, causal=causal)
    ref = oracle.sdpa(host(q), host(k), host(v), D ** -0.5, causal=causal, mask=host(maskd))
    check_sdpa(out, ref, "bf16")


def test_sdpa_flash_bf16_row_shared_mask_all_inf_is_nan(cuda, nat, oracle):
    """A row-shared mask that is -inf on every key of one batch: that batch's
    rows are 0/0 (NaN, as exp(x - max) / sum gives); the other batch matches
    the oracle."""
    q, k, v = make_qkv(cuda, 42, (2, 4, 130, 128), (2, 4, 200, 128), cuda.bfloat16)
    mask = np.zeros((2, 1, 1, 200))
    mask[1] = -np.inf
    maskd = dev(cuda, mask, cuda.float32)
    assert nat.sdpa_kernel_name(q, k, v, mask=maskd) == "flash_bf16_d128"
    out = nat.sdpa(q, k, v, scale=0.1, mask=maskd).float()
    assert bool(cuda.isnan(out[1]).all())
    ref = oracle.sdpa(host(q[:1]), host(k[:1]), host(v[:1]), 0.1)
    check_sdpa(out[:1], ref, "bf16")


def test_sdpa_flash_bf16_padding_mask_config3_size(cuda, nat, oracle):
    """The bench's masked prefill: [4,32,2048,128] bf16, non-causal, an f32
    padding mask [4,1,1,2048] with lengths from default_rng(3); eight heads
    (one per XCD residue and group slot) against the oracle, every output
    finite, and padded-out keys never reach the output (equal to the same
    heads run on keys cut to the batch's length)."""
    from config3_heads import CONFIG3_HEADS

    q, k, v = make_qkv(cuda, 3, (4, 32, 2048, 128), (4, 32, 2048, 128), cuda.bfloat16)
    lens = np.random.default_rng(3).integers(1024, 2048, size=4, endpoint=True)
    mask = np.where(np.arange(2048)[None] < lens[:, None], 0.0, -np.inf).reshape(4, 1, 1, 2048)
    maskd = dev(cuda, mask, cuda.float32)
    out = nat.sdpa(q, k, v, scale=128 ** -0.5, mask=maskd)
    cuda.cuda.synchronize()
    assert bool(cuda.isfinite(out.float()).all())
    for b, h in CONFIG3_HEADS:
        sl = lambda t: host(t[b:b + 1, h:h + 1])
        ref = oracle.sdpa(sl(q), sl(k)[:, :, :lens[b]], sl(v)[:, :, :lens[b]], 128 ** -0.5)
        check_sdpa(out[b:b + 1, h:h + 1], ref, "bf16")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("case", ["growing", "spike", "shrinking", "wide_scale"])
@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_flash_bf16_rebase(cuda, nat, oracle, D, case, causal):
    """Score ranges that move the mask-free bf16 kernel's exp2 base after the
    first tile: keys whose scale grows along the sequence (later tiles pass
    the first tile's max by far more than the slack), one key with a huge
    score in a late tile, keys that shrink after the first tile (the base
    stays high and later probabilities are small), and a scale four times
    1/sqrt(D).  Every row against the fp64 oracle on the same bf16 inputs."""
    B, H, T = 1, 4, 1000
    rng = np.random.default_rng(31)
    q = rng.standard_normal((B, H, T, D))
    k = rng.standard_normal((B, H, T, D))
    v = rng.standard_normal((B, H, T, D))
    scale = D ** -0.5
    j = np.arange(T)[None, None, :, None]
    if case == "growing":
        k = k * (1 + 4 * j / T)
    elif case == "spike":
        k[:, :, 700] *= 30
    elif case == "shrinking":
        k = k * (5 / (1 + 4 * j / T))
    else:
        scale = 4 * D ** -0.5
    qd, kd, vd = (dev(cuda, a, cuda.bfloat16) for a in (q, k, v))
    assert nat.sdpa_kernel_name(qd, kd, vd, causal=causal) == f"flash_bf16_d{D}"
    out = nat.sdpa(qd, kd, vd, scale=scale, causal=causal)
    ref = oracle.sdpa(host(qd), host(kd), host(vd), scale, causal=causal)
    check_sdpa(out, ref, "bf16")


def test_sdpa_bf16_golden(cuda, nat, golden):
    q, k, v = (dev(cuda, golden[f"sdpa_bf16_{s}"], cuda.bfloat16) for s in "qkv")
    out = nat.sdpa(q, k, v, scale=float(golden["sdpa_bf16_scale"]), causal=True)
    check_sdpa(out, golden["sdpa_bf16_out_causal"], "bf16")


from config3_heads import CONFIG3_BH, CONFIG3_HEADS


def test_config3_heads_cover_every_xcd_and_slot():
    assert sorted(bh % 8 for bh in CONFIG3_BH) == list(range(8))
    assert sorted((bh // 8) % 4 for bh in CONFIG3_BH) == [0, 0, 1, 1, 2, 2, 3, 3]
    assert sorted(bh // 32 for bh in CONFIG3_BH) == [0, 0, 1, 1, 2, 2, 3, 3]


def test_sdpa_bf16_config3_full_size(cuda, nat, oracle):
    """B4/H32/T2048/d128 causal bf16: eight whole heads (one per XCD residue
    and group slot of the kernel's block mapping) against the oracle, plus
    size-independent properties on every head."""
    q, k, v = make_qkv(cuda, 3, (4, 32, 2048, 128), (4, 32, 2048, 128), cuda.bfloat16)
    assert nat.sdpa_kernel_name(q, k, v, causal=True) == "flash_bf16_d128"
    out = nat.sdpa(q, k, v, scale=128 ** -0.5, causal=True)
    cuda.cuda.synchronize()
    for b, h in CONFIG3_HEADS:
        ref = oracle.sdpa(host(q[b:b + 1, h:h + 1]), host(k[b:b + 1, h:h + 1]),
                          host(v[b:b + 1, h:h + 1]), 128 ** -0.5, causal=True)
        check_sdpa(out[b:b + 1, h:h + 1], ref, "bf16")
    # Query 0 sees only key 0: exactly v[..., 0, :].
    assert cuda.equal(out[:, :, 0], v[:, :, 0])
    # Causal row i is a convex combination of v[0..i]: check the running bounds.
    vf = v.float()
    hi = cuda.cummax(vf, dim=2).values
    lo = cuda.cummin(vf, dim=2).values
    of = out.float()
    slack = 1e-2 * vf.abs().max()
    assert bool(((of <= hi + slack) & (of >= lo - slack)).all())
    assert bool(cuda.isfinite(of).all())


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("which", ["k", "v"])
def test_sdpa_broadcast_kv_rows(cuda, nat, oracle, dtype, which):
    """K or V as a broadcast view (row stride 0, torch.expand): the buffer-
    resource kernels do not take it (their extents assume rows of at least
    D elements) and the kernel that does matches the oracle.  With V
    broadcast every output row is that one V row (the weights sum to 1)."""
    td = cuda.float32 if dtype == "f32" else cuda.bfloat16
    q, k, v = make_qkv(cuda, 31, (2, 4, 96, 64), (2, 4, 96, 64), td)
    if which == "v":
        v = v[:, :, :1].expand(2, 4, 96, 64)
    else:
        k = k[:, :, :1].expand(2, 4, 96, 64)
    name = nat.sdpa_kernel_name(q, k, v)
    assert name.startswith("flash_f32") if dtype == "f32" else name == "generic", name
    out = nat.sdpa(q, k, v, scale=0.125)
    ref = oracle.sdpa(host(q), host(k), host(v), 0.125)
    check_sdpa(out, ref, dtype)
    if which == "v":
        err = float(np.abs(host(out) - host(v)).max())
        assert err <= (1e-5 if dtype == "f32" else 1e-2), err


def test_sdpa_decode_library_scratch_per_stream(cuda, nat, oracle):
    """Split-KV decodes without a workspace on two streams at once use the
    library's scratch; each stream gets its own buffer, so the partials of
    one call never overwrite the other's.  Repeated interleaved calls, the
    second stream's problem larger (its buffer grows while the first stream
    still has work queued), every result against the oracle."""
    torch = cuda
    qa, ka, va = make_qkv(cuda, 51, (4, 16, 1, 128), (4, 4, 3000, 128), cuda.bfloat16)
    qb, kb, vb = make_qkv(cuda, 52, (8, 16, 1, 128), (8, 4, 6000, 128), cuda.bfloat16)
    assert nat.sdpa_kernel_name(qa, ka, va) == "decode_splitkv_mfma"
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    outs_a, outs_b = [], []
    for _ in range(4):
        with torch.cuda.stream(sa):
            outs_a.append(nat.sdpa(qa, ka, va, scale=0.1))
        with torch.cuda.stream(sb):
            outs_b.append(nat.sdpa(qb, kb, vb, scale=0.1))
    torch.cuda.synchronize()
    ref_a = oracle.sdpa(host(qa), host(ka), host(va), 0.1)
    ref_b = oracle.sdpa(host(qb), host(kb), host(vb), 0.1)
    for o in outs_a:
        check_sdpa(o, ref_a, "bf16")
    for o in outs_b:
        check_sdpa(o, ref_b, "bf16")


def test_sdpa_gqa_decode_golden(cuda, nat, golden):
    q, k, v = (dev(cuda, golden[f"gqa_{s}"], cuda.bfloat16) for s in "qkv")
    mask = dev(cuda, golden["gqa_mask"], cuda.float32)
    out = nat.sdpa(q, k, v, scale=float(golden["gqa_scale"]), mask=mask)
    check_sdpa(out, golden["gqa_out"], "bf16")


def test_sdpa_config5_decode_rmsnorm_full_size(cuda, nat, oracle):
    """GQA decode: q [16,32,1,128] -> RMSNorm(eps 1e-6) -> SDPA over k/v
    [16,8,8192,128] with a 0/-inf length mask, lengths ~ U{1024..8192}."""
    rng = np.random.default_rng(5)
    q = dev(cuda, rng.standard_normal((16, 32, 1, 128)), cuda.bfloat16)
    k = dev(cuda, rng.standard_normal((16, 8, 8192, 128)), cuda.bfloat16)
    v = dev(cuda, rng.standard_normal((16, 8, 8192, 128)), cuda.bfloat16)
    lens = rng.integers(1024, 8192, size=16, endpoint=True)
    mask = np.where(np.arange(8192)[None] < lens[:, None], 0.0, -np.inf).reshape(16, 1, 1, 8192)
    maskd = dev(cuda, mask, cuda.float32)
    assert nat.sdpa_kernel_name(q, k, v, mask=maskd, q_rms_eps=1e-6) == "decode_splitkv_mfma"
    out = nat.sdpa(q, k, v, scale=128 ** -0.5, mask=maskd, q_rms_eps=1e-6)
    qn = oracle.rms_norm(host(q), None, 1e-6)
    qn = host(cuda.from_numpy(qn.astype(np.float32)).bfloat16())  # the graph's bf16 RMSNorm output
    ref = oracle.sdpa(qn, host(k), host(v), 128 ** -0.5, mask=mask)
    check_sdpa(out, ref, "bf16")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("hq,hkv,tq,D", [(4, 4, 1, 64), (8, 2, 2, 128), (8, 1, 1, 128), (4, 2, 3, 64)])
def test_sdpa_decode_variants(cuda, nat, oracle, dtype, hq, hkv, tq, D):
    td = cuda.float32 if dtype == "f32" else cuda.bfloat16
    q, k, v = make_qkv(cuda, 9, (3, hq, tq, D), (3, hkv, 3000, D), td)
    assert nat.sdpa_kernel_name(q, k, v) == ("decode_splitkv" if dtype == "f32" else "decode_splitkv_mfma")
    w = dev(cuda, 1 + 0.1 * np.random.default_rng(10).standard_normal(D), td)
    out = nat.sdpa(q, k, v, scale=0.1, q_rms_eps=1e-5, q_rms_weight=w)
    qn = oracle.rms_norm(host(q), host(w), 1e-5)
    qn = host(cuda.from_numpy(qn.astype(np.float32)).to(td))
    check_sdpa(out, oracle.sdpa(qn, host(k), host(v), 0.1), dtype)
    out_c = nat.sdpa(q, k, v, scale=0.1, causal=True)
    check_sdpa(out_c, oracle.sdpa(host(q), host(k), host(v), 0.1, causal=True), dtype)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sdpa_generic_head_size_and_fused_qnorm_prefill(cuda, nat, oracle, dtype):
    td = cuda.float32 if dtype == "f32" else cuda.bfloat16
    q, k, v = make_qkv(cuda, 11, (2, 4, 33, 80), (2, 2, 45, 80), td, vshape=(2, 2, 45, 48))
    assert nat.sdpa_kernel_name(q, k, v) == "generic"
    out = nat.sdpa(q, k, v, scale=0.15, causal=True)
    check_sdpa(out, oracle.sdpa(host(q), host(k), host(v), 0.15, causal=True), dtype)
    # Prefill with a fused q RMSNorm goes through the normalised copy of q.
    q, k, v = make_qkv(cuda, 12, (2, 4, 200, 64), (2, 4, 200, 64), td)
    out = nat.sdpa(q, k, v, scale=0.125, causal=True, q_rms_eps=1e-6)
    qn = oracle.rms_norm(host(q), None, 1e-6)
    qn = host(cuda.from_numpy(qn.astype(np.float32)).to(td))
    check_sdpa(out, oracle.sdpa(qn, host(k), host(v), 0.125, causal=True), dtype)


@pytest.mark.parametrize("tq", [1, 64])
def test_sdpa_fully_masked_rows_are_nan(cuda, nat, tq):
    q, k, v = make_qkv(cuda, 13, (1, 2, tq, 64), (1, 2, 300, 64), cuda.bfloat16)
    mask = cuda.zeros(1, 1, tq, 300, device="cuda")
    mask[..., 0, :] = float("-inf")
    out = nat.sdpa(q, k, v, scale=0.125, mask=mask).float()
    assert bool(cuda.isnan(out[:, :, 0]).all())
    if tq > 1:
        assert bool(cuda.isfinite(out[:, :, 1:]).all())


@pytest.mark.parametrize("hq,hkv,tq,D,tk", [(32, 1, 1, 128, 64), (16, 2, 4, 64, 1000), (8, 8, 1, 128, 4097),
                                            (32, 4, 4, 128, 777), (4, 2, 1, 64, 1)])
def test_sdpa_decode_mfma_rows_and_ragged_splits(cuda, nat, oracle, hq, hkv, tq, D, tk):
    """Up to 32 query rows per kv head, Tk not a multiple of the 64-key tile,
    split boundaries, a single key; plus the causal variant (query t sees
    keys 0..t)."""
    q, k, v = make_qkv(cuda, 21, (2, hq, tq, D), (2, hkv, tk, D), cuda.bfloat16)
    assert nat.sdpa_kernel_name(q, k, v) == "decode_splitkv_mfma"
    out = nat.sdpa(q, k, v, scale=D ** -0.5)
    check_sdpa(out, oracle.sdpa(host(q), host(k), host(v), D ** -0.5), "bf16")
    out_c = nat.sdpa(q, k, v, scale=D ** -0.5, causal=True)
    check_sdpa(out_c, oracle.sdpa(host(q), host(k), host(v), D ** -0.5, causal=True), "bf16")


def test_sdpa_decode_mfma_per_row_mask_and_holes(cuda, nat, oracle):
    """An additive mask that differs per head and per query position, with
    holes (-inf runs inside the valid range) and finite biases; one batch has
    a fully masked 64-key tile run that the prepass must skip."""
    rng = np.random.default_rng(22)
    B, Hq, Hkv, Tq, S, D = 2, 8, 2, 2, 900, 128
    q, k, v = make_qkv(cuda, 23, (B, Hq, Tq, D), (B, Hkv, S, D), cuda.bfloat16)
    mask = rng.standard_normal((B, Hq, Tq, S)) * 0.5
    mask[:, :, :, 100:300] = -np.inf                 # whole tiles masked for every row
    mask[0, 3, 1, 500:900] = -np.inf                 # one row sees a shorter prefix
    mask[1, :, 0, ::7] = -np.inf                     # holes
    maskd = dev(cuda, mask, cuda.float32)
    assert nat.sdpa_kernel_name(q, k, v, mask=maskd) == "decode_splitkv_mfma"
    out = nat.sdpa(q, k, v, scale=0.09, mask=maskd)
    check_sdpa(out, oracle.sdpa(host(q), host(k), host(v), 0.09, mask=mask), "bf16")


@pytest.mark.parametrize("mdt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("rows", ["shared", "per_row"])
@pytest.mark.parametrize("D,tk", [(64, 777), (128, 1030)])
def test_sdpa_decode_mfma_mask_dtypes_and_strides(cuda, nat, oracle, mdt, rows, D, tk):
    """Additive masks of every element type on the MFMA decode (the kernel
    gathers them as 2- or 4-byte loads into LDS): one mask row shared by all
    query rows of a kv head, or one per (head, query position); Tk ragged
    against the 32-key tile; keys at stride 2 (a strided view); -inf runs,
    holes and finite biases; the per-row case also causal."""
    rng = np.random.default_rng(31)
    B, Hq, Hkv = 2, 8, 2
    tq = 1 if rows == "shared" else 2
    q, k, v = make_qkv(cuda, 32, (B, Hq, tq, D), (B, Hkv, tk, D), cuda.bfloat16)
    shape = (B, 1, 1, 2 * tk) if rows == "shared" else (B, Hq, tq, 2 * tk)
    base = rng.standard_normal(shape) * 0.5
    base[..., 100:260] = -np.inf                    # keys 50..129 of the strided view
    base[1, ..., 2 * (tk // 2):] = -np.inf          # batch 1 sees half the cache
    base[0, ..., 22::22] = -np.inf                  # holes (every 11th key of the view from 11)
    td = {"bf16": cuda.bfloat16, "f16": cuda.float16, "f32": cuda.float32}[mdt]
    full = dev(cuda, base, td)
    maskd = full[..., ::2]
    assert maskd.stride(-1) == 2
    mask = host(maskd.float())                      # the values the kernel sees
    assert nat.sdpa_kernel_name(q, k, v, mask=maskd) == "decode_splitkv_mfma"
    out = nat.sdpa(q, k, v, scale=D ** -0.5, mask=maskd)
    check_sdpa(out, oracle.sdpa(host(q), host(k), host(v), D ** -0.5, mask=mask), "bf16")
    if rows == "per_row":
        out_c = nat.sdpa(q, k, v, scale=D ** -0.5, mask=maskd, causal=True)
        ref_c = oracle.sdpa(host(q), host(k), host(v), D ** -0.5, causal=True, mask=mask)
        check_sdpa(out_c, ref_c, "bf16")


@pytest.mark.parametrize("D", [64, 128])
def test_sdpa_decode_mfma_ranges_across_many_lists(cuda, nat, oracle, D):
    """More listed tiles than resident wavefronts and (batch, kv head) lists
    shorter than a wavefront's range: ranges start mid-list and span two or
    three lists (several partial segments per wavefront, merged per row by
    the combine); lengths vary per batch, some lists hold a single tile."""
    rng = np.random.default_rng(41)
    B, Hq, Hkv, tk = 64, 8, 8, 517
    q, k, v = make_qkv(cuda, 42, (B, Hq, 1, D), (B, Hkv, tk, D), cuda.bfloat16)
    lens = rng.integers(1, tk, size=B, endpoint=True)
    lens[:4] = [1, 32, 33, tk]
    mask = np.where(np.arange(tk)[None] < lens[:, None], 0.0, -np.inf).reshape(B, 1, 1, tk)
    maskd = dev(cuda, mask, cuda.float32)
    assert nat.sdpa_kernel_name(q, k, v, mask=maskd) == "decode_splitkv_mfma"
    out = nat.sdpa(q, k, v, scale=D ** -0.5, mask=maskd)
    check_sdpa(out, oracle.sdpa(host(q), host(k), host(v), D ** -0.5, mask=mask), "bf16")


def select_semantics_ref(oracle, q, k, v, scale, keep):
    """softmax(where(keep, s, c)) @ v for a very negative finite c, the way
    jax.nn.dot_product_attention masks: rows with a visible key are the
    -inf-masked softmax; a row with none has equal scores, so uniform weights
    and the mean of its kv head's V rows."""
    B, Hq, Tq, _ = q.shape
    Hkv, Tk = k.shape[1], k.shape[2]
    keep = np.broadcast_to(keep, (B, Hq, Tq, Tk))
    ref = oracle.sdpa(q, k, v, scale, mask=np.where(keep, 0.0, -np.inf))
    vmean = np.repeat(v.mean(axis=2), Hq // Hkv, axis=1)            # [B, Hq, Dv]
    full = ~keep.any(-1)                                             # [B, Hq, Tq]
    ref[full] = np.broadcast_to(vmean[:, :, None, :], ref.shape)[full]
    return ref


@pytest.mark.parametrize("case", ["flash_bf16_d128", "flash_bf16_d128_shared", "flash_f32_split_d64",
                                  "flash_f32_split_d128", "flash_f32_d64",
                                  "flash_f32_d128", "generic",
                                  "decode_splitkv_mfma",
                                  "decode_splitkv", "decode_splitkv_mfma_shared"])
@pytest.mark.parametrize("mdt", ["f32", "bf16"])
def test_sdpa_finite_mask_fully_masked_rows(cuda, nat, oracle, case, mdt):
    """A mask value of -0.7 * FLT_MAX (JAX's) or bf16's finfo.min on every key
    of a row returns the mean of V (select semantics), not NaN: the kernels
    keep log2(e) * mask finite."""
    shapes = {"flash_bf16_d128": ((2, 4, 64, 128), (2, 2, 300, 128), "bf16"),
              "flash_bf16_d128_shared": ((2, 4, 150, 128), (2, 2, 500, 128), "bf16"),
              "flash_f32_split_d64": ((2, 4, 64, 64), (2, 2, 200, 64), "f32"),
              "flash_f32_split_d128": ((2, 4, 64, 128), (2, 2, 200, 128), "f32"),
              "flash_f32_d64": ((16, 32, 128, 64), (16, 16, 200, 64), "f32"),  # 512 workgroups
              "flash_f32_d128": ((16, 32, 128, 128), (16, 16, 200, 128), "f32"),
              "generic": ((2, 4, 33, 40), (2, 2, 90, 40), "f32"),
              "decode_splitkv_mfma": ((2, 8, 1, 128), (2, 2, 700, 128), "bf16"),
              "decode_splitkv": ((2, 8, 1, 64), (2, 2, 700, 64), "f32"),
              "decode_splitkv_mfma_shared": ((2, 8, 1, 128), (2, 2, 700, 128), "bf16")}
    qs, ks, dt = shapes[case]
    td = cuda.float32 if dt == "f32" else cuda.bfloat16
    q, k, v = make_qkv(cuda, 31, qs, ks, td)
    rng = np.random.default_rng(32)
    B, Hq, Tq, _ = qs
    Tk = ks[2]
    if case.endswith("shared"):
        keep = np.ones((B, 1, 1, Tk), bool)
        keep[0, :, :, 400:] = False
        keep[1] = False                                # batch 1: every key of every row masked
    else:
        keep = rng.random((B, Hq, Tq, Tk)) > 0.3
        keep[0, 1, Tq - 1] = False                     # fully masked rows
        keep[1, 3, 0] = False
        keep[1, 2, :, :Tk // 2] = False
    neg = -0.7 * np.finfo(np.float32).max if mdt == "f32" else float(cuda.finfo(cuda.bfloat16).min)
    maskd = dev(cuda, np.where(keep, 0.0, neg), cuda.float32).to(cuda.float32 if mdt == "f32" else cuda.bfloat16)
    assert nat.sdpa_kernel_name(q, k, v, mask=maskd) == case.replace("_shared", "")
    out = nat.sdpa(q, k, v, scale=qs[-1] ** -0.5, mask=maskd)
    assert bool(cuda.isfinite(out.float()).all())
    check_sdpa(out, select_semantics_ref(oracle, host(q), host(k), host(v), qs[-1] ** -0.5, keep), dt)


def test_sdpa_decode_mfma_fully_masked_row_is_nan(cuda, nat):
    q, k, v = make_qkv(cuda, 24, (1, 4, 1, 64), (1, 2, 300, 64), cuda.bfloat16)
    mask = cuda.zeros(1, 4, 1, 300, device="cuda")
    mask[:, 1] = float("-inf")
    out = nat.sdpa(q, k, v, scale=0.125, mask=mask).float()
    assert bool(cuda.isnan(out[:, 1]).all())
    assert bool(cuda.isfinite(out[:, [0, 2, 3]]).all())


# ---------------------------------------------------------- SDPA backward
# mfx_sdpa_bwd against the fp64 oracle (reference closed form
# src/jax_mlx/sdpa.py:65-87; masks and GQA as the forward).  f32:
# ||d - ref||_inf <= 1e-4 * max(1, ||ref||_inf) per gradient; bf16: the
# relative bar on each of dq, dk, dv.

def check_grads(outs, refs, dtype):
    for name, o, r in zip(("dq", "dk", "dv"), outs, refs):
        o = host(o)
        if dtype == "f32":
            err = np.abs(o - r).max()
            assert err <= F32_SDPA_TOL * max(1.0, np.abs(r).max()), (name, err)
        else:
            rr = rel_inf(o, r)
            assert rr <= BF16_REL_TOL, (name, rr)


def bwd_case(cuda, nat, oracle, seed, qshape, kshape, dtype, *, causal=False, scale=None, mask=None,
             vshape=None, layout="bhtd"):
    td = cuda.float32 if dtype == "f32" else cuda.bfloat16
    q, k, v = make_qkv(cuda, seed, qshape, kshape, td, vshape)
    rng = np.random.default_rng(seed + 100)
    oshape = list(qshape)
    oshape[-1] = (vshape or kshape)[-1]
    g = dev(cuda, rng.standard_normal(oshape), td)
    grads = nat.sdpa_bwd(q, k, v, g, scale=scale, causal=causal, mask=mask, layout=layout)
    tr = (lambda a: a.transpose(0, 2, 1, 3)) if layout == "bthd" else (lambda a: a)
    D = qshape[-1]
    sc = scale if scale is not None else 1.0 / np.sqrt(D)
    refs = oracle.sdpa_bwd(tr(host(q)), tr(host(k)), tr(host(v)), tr(host(g)), sc, causal=causal,
                           mask=None if mask is None else host(mask))
    return grads, [tr(r) for r in refs]


@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_bwd_f32_config2(cuda, nat, oracle, causal):
    grads, refs = bwd_case(cuda, nat, oracle, 2, (8, 8, 128, 64), (8, 8, 128, 64), "f32", causal=causal,
                           scale=0.125)
    check_grads(grads, refs, "f32")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("D,tq,tk,causal", [(128, 64, 64, True), (64, 256, 256, False), (128, 200, 200, True),
                                            (64, 77, 130, False), (128, 1, 33, False), (64, 130, 130, True)])
def test_sdpa_bwd_shapes(cuda, nat, oracle, dtype, D, tq, tk, causal):
    grads, refs = bwd_case(cuda, nat, oracle, 31, (1, 2, tq, D), (1, 2, tk, D), dtype, causal=causal)
    check_grads(grads, refs, dtype)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sdpa_bwd_btnh_gqa_mask(cuda, nat, oracle, dtype):
    """BTNH layout (the custom_call @mlx_sdpa_bwd operands), Hq 8 over Hkv 2,
    additive mask broadcast over heads, -inf holes."""
    td = cuda.float32 if dtype == "f32" else cuda.bfloat16
    rng = np.random.default_rng(41)
    m = rng.standard_normal((2, 1, 96, 160)).astype(np.float32)
    m[:, :, :, 5] = -np.inf
    mask = dev(cuda, m, td)
    grads, refs = bwd_case(cuda, nat, oracle, 42, (2, 96, 8, 64), (2, 160, 2, 64), dtype, mask=mask,
                           layout="bthd", scale=0.2)
    check_grads(grads, refs, dtype)


@pytest.mark.parametrize("D", [32, 96])
@pytest.mark.parametrize("tq,tk,hq,hkv,causal", [(64, 64, 2, 2, True), (200, 200, 4, 2, True), (77, 130, 2, 1, False),
                                                 (1, 33, 2, 2, False)])
def test_sdpa_bwd_padded_head_sizes(cuda, nat, oracle, D, tq, tk, hq, hkv, causal):
    """bf16 head sizes 32 / 96 on the matrix-core backward: q, k, v, dO and O
    copied into zero-padded 64- / 128-feature rows, the gradients copied out."""
    q, k, v = make_qkv(cuda, 91, (1, hq, tq, D), (1, hkv, tk, D), cuda.bfloat16)
    assert nat.sdpa_bwd_kernel_name(q, k, v, causal=causal) == f"mfma_bf16_d{D}"
    grads, refs = bwd_case(cuda, nat, oracle, 91, (1, hq, tq, D), (1, hkv, tk, D), "bf16", causal=causal)
    check_grads(grads, refs, "bf16")


@pytest.mark.parametrize("D", [32, 96])
def test_sdpa_bwd_padded_btnh_mask_and_residuals(cuda, nat, oracle, D):
    """The padded route on BTNH views with GQA and a per-row mask, and from a
    forward's output and lse: the same gradients as the recomputing call."""
    rng = np.random.default_rng(92)
    m = rng.standard_normal((2, 1, 96, 160)).astype(np.float32)
    m[:, :, :, 5] = -np.inf
    mask = dev(cuda, m, cuda.float32)
    grads, refs = bwd_case(cuda, nat, oracle, 93, (2, 96, 8, D), (2, 160, 2, D), "bf16", mask=mask, layout="bthd",
                           scale=0.2)
    check_grads(grads, refs, "bf16")
    q, k, v = make_qkv(cuda, 94, (2, 4, 130, D), (2, 2, 130, D), cuda.bfloat16)
    g = dev(cuda, rng.standard_normal((2, 4, 130, D)), cuda.bfloat16)
    lse = cuda.empty(2 * 4 * 130, dtype=cuda.float32, device="cuda")
    out = nat.sdpa(q, k, v, causal=True, lse=lse)
    re = nat.sdpa_bwd(q, k, v, g, causal=True)
    fw = nat.sdpa_bwd(q, k, v, g, causal=True, fwd_out=out, fwd_lse=lse)
    for a, b in zip(re, fw):
        assert cuda.equal(a, b)


def test_sdpa_bwd_odd_head_size_generic(cuda, nat, oracle):
    grads, refs = bwd_case(cuda, nat, oracle, 43, (1, 3, 50, 80), (1, 3, 70, 80), "bf16", causal=True,
                           vshape=(1, 3, 70, 48))
    check_grads(grads, refs, "bf16")


def test_sdpa_bwd_known_answers(cuda, nat):
    """Tk = 1: out = v, so dv = sum over query rows of dO and dq = dk = 0.
    Identical keys: P is uniform 1/Tk, so dq = 0 and every dv_j is the sum of
    dO over query rows divided by Tk."""
    q = cuda.randn(1, 1, 8, 64, device="cuda")
    k = cuda.randn(1, 1, 1, 64, device="cuda")
    v = cuda.randn(1, 1, 1, 64, device="cuda")
    g = cuda.randn(1, 1, 8, 64, device="cuda")
    dq, dk, dv = nat.sdpa_bwd(q, k, v, g)
    assert np.abs(host(dq)).max() <= 1e-5 and np.abs(host(dk)).max() <= 1e-5
    np.testing.assert_allclose(host(dv)[0, 0, 0], host(g).sum(axis=2)[0, 0], atol=1e-5)
    k = cuda.randn(1, 1, 1, 64, device="cuda").expand(1, 1, 16, 64).contiguous()
    v = cuda.randn(1, 1, 16, 64, device="cuda")
    dq, dk, dv = nat.sdpa_bwd(q, k, v, g)
    assert np.abs(host(dq)).max() <= 1e-5
    np.testing.assert_allclose(host(dv)[0, 0], np.tile(host(g).sum(axis=2)[0, 0] / 16, (16, 1)), atol=1e-5)


def test_sdpa_bwd_kernel_selection(cuda, nat):
    q, k, v = make_qkv(cuda, 1, (1, 2, 64, 128), (1, 2, 64, 128), cuda.bfloat16)
    assert nat.sdpa_bwd_kernel_name(q, k, v) == "mfma_bf16_d128"
    q, k, v = make_qkv(cuda, 1, (1, 2, 64, 64), (1, 2, 64, 64), cuda.bfloat16)
    assert nat.sdpa_bwd_kernel_name(q, k, v, causal=True) == "mfma_bf16_d64"
    q, k, v = make_qkv(cuda, 1, (1, 2, 64, 64), (1, 2, 64, 64), cuda.float32)
    assert nat.sdpa_bwd_kernel_name(q, k, v) == "generic"


def test_sdpa_bwd_config3_full_size(cuda, nat, oracle):
    """Config 3 shape (bf16 [4,32,2048,128], causal): the gradients of eight
    (batch, head) pairs (one per XCD residue and group slot) against the
    fp64 oracle run on those heads alone (heads are independent), plus
    finiteness everywhere."""
    q, k, v = make_qkv(cuda, 3, (4, 32, 2048, 128), (4, 32, 2048, 128), cuda.bfloat16)
    g = dev(cuda, np.random.default_rng(103).standard_normal((4, 32, 2048, 128)), cuda.bfloat16)
    assert nat.sdpa_bwd_kernel_name(q, k, v, causal=True) == "mfma_bf16_d128"
    dq, dk, dv = nat.sdpa_bwd(q, k, v, g, causal=True)
    cuda.cuda.synchronize()
    for t in (dq, dk, dv):
        assert bool(cuda.isfinite(t).all())
    sc = 1.0 / np.sqrt(128)
    for b, h in CONFIG3_HEADS:
        sl = lambda t: host(t[b:b + 1, h:h + 1])
        refs = oracle.sdpa_bwd(sl(q), sl(k), sl(v), sl(g), sc, causal=True)
        for name, o, r in zip(("dq", "dk", "dv"), (dq, dk, dv), refs):
            rr = rel_inf(sl(o), r)
            assert rr <= BF16_REL_TOL, (b, h, name, rr)


# ---------------------------------------------------------------- elementwise device math

def test_tanh_device_accuracy_and_paths(cuda):
    """stablehlo.tanh as the elementwise kernels compute it (ew_math.h's
    mfx_tanh): the generated kernel and the interpreter give the same bits,
    and every result is within 4 ulp of fp64 tanh on 2^22 points spread over
    the f32 magnitudes (subnormals to 1e4), both signs, the 0.55 switch and
    the specials (+-0, +-inf -> +-1, NaN -> NaN)."""
    import numpy as np

    from jax_mlx_amd import native as nt

    torch = cuda
    rng = np.random.default_rng(7)
    mags = np.exp(rng.uniform(np.log(1e-40), np.log(1e4), 1 << 22)).astype(np.float32)
    x = mags * np.where(rng.random(mags.size) < 0.5, -1, 1).astype(np.float32)
    edge = np.float32(0.55) + np.arange(-64, 64, dtype=np.float32) * np.spacing(np.float32(0.55))
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 44.0, -44.0, 1e-45], dtype=np.float32)
    x = np.concatenate([x, edge, -edge, special]).astype(np.float32)
    n = x.size - x.size % 4
    x = x[:n]
    xd = torch.from_numpy(x).cuda()
    prog = nt.ew_program([n], [(nt.MFX_F32, [1])], [("load", 0, 0), ("tanh", 1, 0)], 1)
    outs = []
    lib = nt.load()
    for jit in (1, 0):
        prev = lib.mfx_ew_jit_enable(jit)
        try:
            y = torch.empty_like(xd)
            nt.elementwise(prog, [xd], y)
            torch.cuda.synchronize()
            outs.append(y.cpu().numpy())
        finally:
            lib.mfx_ew_jit_enable(prev)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    y = outs[0]
    ref = np.tanh(x.astype(np.float64))
    fin = np.isfinite(x)
    ulp = np.abs(y[fin] - ref[fin]) / np.spacing(np.maximum(np.abs(ref[fin]), 1e-38).astype(np.float32)).astype(np.float64)
    assert ulp.max() <= 4.0, (ulp.max(), x[fin][np.argmax(ulp)])
    assert np.isnan(y[np.isnan(x)]).all()
    assert (y[x == np.inf] == 1).all() and (y[x == -np.inf] == -1).all()
    assert np.signbit(y[(x == 0) & np.signbit(x)]).all()


# ---------------------------------------------------------------- backward from forward residuals

@pytest.mark.parametrize("dt,shape,causal,layout,group", [
    ("bf16", (2, 4, 256, 128), True, "bhtd", 1),   # matrix-core backward, causal
    ("bf16", (2, 4, 192, 64), False, "bthd", 2),   # BTNH (strided O), GQA, d = 64
    ("f32", (2, 2, 100, 64), False, "bhtd", 1),    # f32: flash forward, generic backward
])
def test_sdpa_bwd_from_forward_residuals(cuda, dt, shape, causal, layout, group):
    """mfx_sdpa_bwd given the forward call's output and lse (mfx_sdpa_fwd's
    lse output) skips its recompute and returns the recomputing call's
    gradients bit for bit; the lse itself matches fp64 log2-sum-exp2 of the
    scaled, causally limited scores -- within 1e-4 for f32, and for bf16
    within 2^-9 / ln 2 = 0.0028 (the bf16 kernels sum the bf16-rounded
    probabilities that also form O, each within 2^-9 relative)."""
    import numpy as np

    from jax_mlx_amd import native as nt

    torch = cuda
    B, H, T, D = shape
    Hkv = H // group
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    g = torch.Generator(device="cpu").manual_seed(sum(shape) + group)

    def mk(heads):
        t = torch.randn(B, heads, T, D, generator=g)
        if layout == "bthd":
            t = t.transpose(1, 2).contiguous()
        return t.to(tdt).cuda()

    q, k, v, go = mk(H), mk(Hkv), mk(Hkv), mk(H)
    lse = torch.empty(B * H * T, dtype=torch.float32, device="cuda")
    out = nt.sdpa(q, k, v, causal=causal, layout=layout, lse=lse)
    ref = nt.sdpa_bwd(q, k, v, go, causal=causal, layout=layout)
    got = nt.sdpa_bwd(q, k, v, go, causal=causal, layout=layout, fwd_out=out, fwd_lse=lse)
    torch.cuda.synchronize()
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    # lse against fp64 (log2 units, scale 1/sqrt(D))
    qh = (q if layout == "bhtd" else q.transpose(1, 2)).double().cpu().numpy()
    kh = (k if layout == "bhtd" else k.transpose(1, 2)).double().cpu().numpy()
    kh = np.repeat(kh, group, axis=1)
    s = np.einsum("bhtd,bhsd->bhts", qh, kh) / np.sqrt(D)
    if causal:
        s = np.where(np.tril(np.ones((T, T), dtype=bool)), s, -np.inf)
    m = s.max(-1, keepdims=True)
    want = (m[..., 0] + np.log(np.exp(s - m).sum(-1))) / np.log(2.0)
    err = np.abs(lse.cpu().numpy().reshape(B, H, T) - want).max()
    assert err <= (2.0 ** -9 / np.log(2.0) if dt == "bf16" else 1e-4), err


# ------------------------------------------------------ head sizes 32, 96
# The pipelined flash kernel at head sizes 32 (64-wide LDS tiles) and 96
# (128-wide): rows load tile-wide, and only the head's features reach an
# MFMA (DV/16 S k-steps, DV/32 output blocks).  Ragged, causal and GQA
# shapes, plus a row-shared padding mask, against the fp64 oracle; f16 at
# its 5e-3 bar.

@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("D", [32, 96])
@pytest.mark.parametrize("tq,tk,hq,hkv,causal", [(100, 77, 3, 3, False), (100, 77, 4, 2, True),
                                                 (77, 200, 2, 1, True), (129, 129, 3, 3, True),
                                                 (1000, 1000, 2, 2, False), (7, 300, 4, 4, False)])
def test_sdpa_flash_head_sizes_32_96(cuda, nat, oracle, dtype, D, tq, tk, hq, hkv, causal):
    td = cuda.bfloat16 if dtype == "bf16" else cuda.float16
    q, k, v = make_qkv(cuda, 71, (2, hq, tq, D), (2, hkv, tk, D), td)
    assert nat.sdpa_kernel_name(q, k, v, causal=causal) == f"flash_{dtype}_d{D}"
    out = nat.sdpa(q, k, v, scale=D ** -0.5, causal=causal)
    ref = oracle.sdpa(host(q), host(k), host(v), D ** -0.5, causal=causal)
    r = rel_inf(host(out), ref)
    assert r <= (BF16_REL_TOL if dtype == "bf16" else 5e-3), r


@pytest.mark.parametrize("D", [32, 96])
def test_sdpa_flash_head_sizes_32_96_mask_and_layout(cuda, nat, oracle, D):
    """BTNH views of packed rows (row stride above D: the tile-wide loads
    read the next head's features, which no MFMA uses) with a padding mask."""
    rng = np.random.default_rng(72)
    B, T, Hq, Hkv = 2, 150, 8, 2
    q = dev(cuda, rng.standard_normal((B, T, Hq, D)), cuda.bfloat16)
    kv = dev(cuda, rng.standard_normal((B, T, 2 * Hkv, D)), cuda.bfloat16)
    k, v = kv[:, :, :Hkv], kv[:, :, Hkv:]
    lens = np.array([150, 61])
    mask = np.where(np.arange(T)[None] < lens[:, None], 0.0, -np.inf).reshape(B, 1, 1, T)
    maskd = dev(cuda, mask, cuda.float32)
    assert nat.sdpa_kernel_name(q, k, v, mask=maskd, layout="bthd") == f"flash_bf16_d{D}"
    out = nat.sdpa(q, k, v, scale=0.2, mask=maskd, layout="bthd")
    qh, kh, vh = (host(t).transpose(0, 2, 1, 3) for t in (q, k, v))
    ref = oracle.sdpa(qh, kh, vh, 0.2, mask=mask).transpose(0, 2, 1, 3)
    check_sdpa(out, ref, "bf16")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("D", [32, 96])
@pytest.mark.parametrize("hq,hkv,tq,tk", [(32, 1, 1, 64), (16, 2, 4, 1000), (8, 8, 1, 4097), (4, 2, 1, 1)])
def test_sdpa_decode_mfma_head_sizes_32_96(cuda, nat, oracle, dtype, D, hq, hkv, tq, tk):
    """The MFMA split-KV decode at head sizes 32 and 96 (64- / 128-wide LDS
    tiles, the head's features only in the MFMAs; the combine's lanes cover
    the head's features): ragged tiles and splits, GQA, causal, a padding
    mask and a fused q RMSNorm with weight."""
    td = cuda.bfloat16 if dtype == "bf16" else cuda.float16
    tol = BF16_REL_TOL if dtype == "bf16" else 5e-3
    q, k, v = make_qkv(cuda, 73, (2, hq, tq, D), (2, hkv, tk, D), td)
    assert nat.sdpa_kernel_name(q, k, v) == "decode_splitkv_mfma"
    out = nat.sdpa(q, k, v, scale=D ** -0.5)
    assert rel_inf(host(out), oracle.sdpa(host(q), host(k), host(v), D ** -0.5)) <= tol
    out_c = nat.sdpa(q, k, v, scale=D ** -0.5, causal=True)
    assert rel_inf(host(out_c), oracle.sdpa(host(q), host(k), host(v), D ** -0.5, causal=True)) <= tol
    lens = np.array([tk, max(1, tk // 3)])
    mask = np.where(np.arange(tk)[None] < lens[:, None], 0.0, -np.inf).reshape(2, 1, 1, tk)
    maskd = dev(cuda, mask, cuda.float32)
    w = dev(cuda, 1 + 0.1 * np.random.default_rng(74).standard_normal(D), td)
    out_m = nat.sdpa(q, k, v, scale=0.1, mask=maskd, q_rms_eps=1e-6, q_rms_weight=w)
    qn = oracle.rms_norm(host(q), host(w), 1e-6)
    qn = host(cuda.from_numpy(qn.astype(np.float32)).to(td))
    assert rel_inf(host(out_m), oracle.sdpa(qn, host(k), host(v), 0.1, mask=mask)) <= tol


@pytest.mark.parametrize("D", [32, 96])
@pytest.mark.parametrize("tq,tk,hq,hkv,causal,masked", [(128, 128, 8, 8, False, False), (100, 77, 4, 2, True, False),
                                                        (33, 300, 4, 1, False, True), (77, 200, 2, 2, True, True),
                                                        (1000, 1000, 1, 1, True, False)])
def test_sdpa_f32_head_sizes_32_96(cuda, nat, oracle, D, tq, tk, hq, hkv, causal, masked):
    """The f32 flash kernels (row-block and key-split) at head sizes 32 and
    96: ragged, GQA, causal, an additive mask with -inf holes."""
    q, k, v = make_qkv(cuda, 75, (2, hq, tq, D), (2, hkv, tk, D), cuda.float32)
    mask = None
    if masked:
        m = np.random.default_rng(76).standard_normal((2, 1, tq, tk)) * 0.5
        m[..., ::5] = -np.inf
        m[..., 0] = 0.0
        mask = m
    maskd = None if mask is None else dev(cuda, mask, cuda.float32)
    assert nat.sdpa_kernel_name(q, k, v, causal=causal, mask=maskd).startswith("flash_f32")
    assert nat.sdpa_kernel_name(q, k, v, causal=causal, mask=maskd).endswith(f"_d{D}")
    out = nat.sdpa(q, k, v, scale=D ** -0.5, causal=causal, mask=maskd)
    check_sdpa(out, oracle.sdpa(host(q), host(k), host(v), D ** -0.5, causal=causal, mask=mask), "f32")


# ------------------------------------------------------------ head size 256
# bf16 / f16 at head size 256 run on the per-element-mask flash kernel (one
# workgroup per CU: four 32 KB tiles; the pipelined and MFMA decode kernels
# stop at 128) for every mask form, decode (Tq <= 4) included.  Against the
# fp64 oracle at the bf16 / f16 bars.

@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("tq,tk,hq,hkv,causal", [(100, 77, 3, 3, False), (100, 77, 4, 2, True),
                                                 (77, 200, 2, 1, True), (129, 129, 3, 3, True),
                                                 (300, 300, 2, 2, False), (1, 300, 8, 2, False),
                                                 (4, 1000, 4, 4, True)])
def test_sdpa_flash_head_size_256(cuda, nat, oracle, dtype, tq, tk, hq, hkv, causal):
    td = cuda.bfloat16 if dtype == "bf16" else cuda.float16
    q, k, v = make_qkv(cuda, 81, (2, hq, tq, 256), (2, hkv, tk, 256), td)
    assert nat.sdpa_kernel_name(q, k, v, causal=causal) == f"flash_{dtype}_d256"
    out = nat.sdpa(q, k, v, scale=256 ** -0.5, causal=causal)
    ref = oracle.sdpa(host(q), host(k), host(v), 256 ** -0.5, causal=causal)
    r = rel_inf(host(out), ref)
    assert r <= (BF16_REL_TOL if dtype == "bf16" else 5e-3), r


@pytest.mark.parametrize("row_mask", [False, True])
def test_sdpa_flash_head_size_256_masks_layout_qnorm(cuda, nat, oracle, row_mask):
    """Packed BTNH rows (K and V sliced from one buffer), a padding mask or a
    per-row bias with -inf holes, and decode with a fused q RMSNorm."""
    rng = np.random.default_rng(82)
    B, T, Hq, Hkv, D = 2, 150, 4, 2, 256
    q = dev(cuda, rng.standard_normal((B, T, Hq, D)), cuda.bfloat16)
    kv = dev(cuda, rng.standard_normal((B, T, 2 * Hkv, D)), cuda.bfloat16)
    k, v = kv[:, :, :Hkv], kv[:, :, Hkv:]
    if row_mask:
        mask = rng.standard_normal((B, 1, T, T)) * 0.5
        mask[..., ::7] = -np.inf
        mask[..., 0] = 0.0
    else:
        lens = np.array([150, 61])
        mask = np.where(np.arange(T)[None] < lens[:, None], 0.0, -np.inf).reshape(B, 1, 1, T)
    maskd = dev(cuda, mask, cuda.float32)
    assert nat.sdpa_kernel_name(q, k, v, mask=maskd, layout="bthd") == "flash_bf16_d256"
    out = nat.sdpa(q, k, v, scale=0.05, mask=maskd, layout="bthd", causal=True)
    qh, kh, vh = (host(t).transpose(0, 2, 1, 3) for t in (q, k, v))
    ref = oracle.sdpa(qh, kh, vh, 0.05, mask=mask, causal=True).transpose(0, 2, 1, 3)
    check_sdpa(out, ref, "bf16")
    # decode: one query row per head, fused q RMSNorm with a weight
    qd = dev(cuda, rng.standard_normal((B, Hq, 1, D)), cuda.bfloat16)
    kd = dev(cuda, rng.standard_normal((B, Hkv, 700, D)), cuda.bfloat16)
    vd = dev(cuda, rng.standard_normal((B, Hkv, 700, D)), cuda.bfloat16)
    w = dev(cuda, 1 + 0.1 * rng.standard_normal(D), cuda.bfloat16)
    assert nat.sdpa_kernel_name(qd, kd, vd) == "flash_bf16_d256"
    outd = nat.sdpa(qd, kd, vd, scale=0.05, q_rms_eps=1e-6, q_rms_weight=w)
    qn = oracle.rms_norm(host(qd), host(w), 1e-6)
    qn = host(cuda.from_numpy(qn.astype(np.float32)).to(cuda.bfloat16))
    check_sdpa(outd, oracle.sdpa(qn, host(kd), host(vd), 0.05), "bf16")


@pytest.mark.parametrize("tq,tk,hq,hkv,causal,masked", [(128, 128, 4, 4, False, False), (100, 77, 4, 2, True, False),
                                                        (33, 300, 4, 1, False, True), (77, 200, 2, 2, True, True),
                                                        (300, 300, 2, 2, True, False), (1, 500, 4, 2, False, False)])
def test_sdpa_f32_head_size_256(cuda, nat, oracle, tq, tk, hq, hkv, causal, masked):
    """The f32 row-block flash kernel at head size 256 (one workgroup per CU,
    134 KB of LDS; never the key-split kernel): ragged, GQA, causal, an
    additive mask with -inf holes, a single query row."""
    q, k, v = make_qkv(cuda, 83, (2, hq, tq, 256), (2, hkv, tk, 256), cuda.float32)
    mask = None
    if masked:
        m = np.random.default_rng(84).standard_normal((2, 1, tq, tk)) * 0.5
        m[..., ::5] = -np.inf
        m[..., 0] = 0.0
        mask = m
    maskd = None if mask is None else dev(cuda, mask, cuda.float32)
    assert nat.sdpa_kernel_name(q, k, v, causal=causal, mask=maskd) == "flash_f32_d256"
    out = nat.sdpa(q, k, v, scale=256 ** -0.5, causal=causal, mask=maskd)
    check_sdpa(out, oracle.sdpa(host(q), host(k), host(v), 256 ** -0.5, causal=causal, mask=mask), "f32")
