"""mfx_sdpa_fwd_noalloc (the allocation-free variant of mfx_sdpa_fwd, with
its workspace in a static per-device array) against mfx_sdpa_fwd itself.

The two share every kernel, so their outputs must agree bit for bit; each
case runs two calls in a row on the shared scratch, the second on a smaller
problem, and checks both.  Arguments that need more workspace than the
static array holds are rejected before any launch."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nat(cuda):
    from jax_mlx_amd import native

    native.load()
    return native


def _qkv(torch, seed, qshape, kshape, dtype):
    rng = np.random.default_rng(seed)
    return [torch.from_numpy(rng.standard_normal(s).astype(np.float32)).cuda().to(dtype)
            for s in (qshape, kshape, kshape)]


def _length_mask(torch, seed, B, Tk):
    rng = np.random.default_rng(seed)
    lens = rng.integers(max(1, Tk // 8), Tk, size=B, endpoint=True)
    m = np.where(np.arange(Tk)[None] < lens[:, None], 0.0, -np.inf).reshape(B, 1, 1, Tk)
    return torch.from_numpy(m.astype(np.float32)).cuda()


def _both(torch, nat, q, k, v, **kw):
    ref = nat.sdpa(q, k, v, **kw)
    out = torch.full_like(ref, float("nan"))
    nat.sdpa_noalloc(q, k, v, out, **kw)
    torch.cuda.synchronize()
    return out, ref


def test_noalloc_decode_two_calls(cuda, nat):
    """GQA split-KV decode with fused RMSNorm(q) and a length mask (config 5's
    shape, 2 MB of partials and tile lists in the scratch), then a smaller
    decode that reuses the same scratch."""
    q, k, v = _qkv(cuda, 51, (16, 32, 1, 128), (16, 8, 8192, 128), cuda.bfloat16)
    mask = _length_mask(cuda, 52, 16, 8192)
    kw = dict(scale=128 ** -0.5, mask=mask, q_rms_eps=1e-6)
    assert nat.sdpa_kernel_name(q, k, v, **kw) == "decode_splitkv_mfma"
    assert 0 < nat.sdpa_workspace_size(q, k, v, **kw) <= nat.NOALLOC_SCRATCH_BYTES
    out1, ref1 = _both(cuda, nat, q, k, v, **kw)
    assert cuda.equal(out1, ref1)

    q2, k2, v2 = _qkv(cuda, 53, (3, 8, 2, 64), (3, 2, 3000, 64), cuda.bfloat16)
    mask2 = _length_mask(cuda, 54, 3, 3000)
    out2, ref2 = _both(cuda, nat, q2, k2, v2, scale=0.125, mask=mask2)
    assert cuda.equal(out2, ref2)
    assert cuda.equal(out1, ref1)  # the first result is its own buffer, untouched


def test_noalloc_f32_decode_and_prefill_qnorm(cuda, nat):
    """The VALU split-KV decode (f32 partials) and a prefill whose q RMSNorm
    goes through a normalised copy of q in the scratch, each followed by a
    smaller call of the same kind."""
    q, k, v = _qkv(cuda, 55, (4, 8, 1, 64), (4, 4, 5000, 64), cuda.float32)
    assert nat.sdpa_kernel_name(q, k, v) == "decode_splitkv"
    assert nat.sdpa_workspace_size(q, k, v) > 0
    out, ref = _both(cuda, nat, q, k, v, scale=0.125)
    assert cuda.equal(out, ref)
    q, k, v = _qkv(cuda, 56, (2, 4, 1, 64), (2, 2, 1200, 64), cuda.float32)
    out, ref = _both(cuda, nat, q, k, v, scale=0.125)
    assert cuda.equal(out, ref)

    q, k, v = _qkv(cuda, 57, (2, 4, 300, 128), (2, 4, 300, 128), cuda.bfloat16)
    kw = dict(scale=0.09, causal=True, q_rms_eps=1e-6)
    assert nat.sdpa_workspace_size(q, k, v, **kw) > 0
    out, ref = _both(cuda, nat, q, k, v, **kw)
    assert cuda.equal(out, ref)
    q, k, v = _qkv(cuda, 58, (1, 2, 100, 128), (1, 2, 100, 128), cuda.bfloat16)
    out, ref = _both(cuda, nat, q, k, v, **kw)
    assert cuda.equal(out, ref)


def test_noalloc_without_workspace_and_oversize(cuda, nat):
    """A call that needs no workspace (causal flash prefill) runs as well; one
    that needs more than the static scratch is rejected with
    MFX_E_WORKSPACE and launches nothing (its output keeps its contents)."""
    q, k, v = _qkv(cuda, 59, (1, 4, 256, 128), (1, 4, 256, 128), cuda.bfloat16)
    assert nat.sdpa_workspace_size(q, k, v, causal=True) == 0
    out, ref = _both(cuda, nat, q, k, v, scale=0.1, causal=True)
    assert cuda.equal(out, ref)

    q = cuda.zeros(4, 32, 2048, 128, device="cuda", dtype=cuda.bfloat16)
    kw = dict(scale=0.1, causal=True, q_rms_eps=1e-6)
    assert nat.sdpa_workspace_size(q, q, q, **kw) > nat.NOALLOC_SCRATCH_BYTES
    out = cuda.full_like(q, 7.0)
    with pytest.raises(nat.MfxError) as e:
        nat.sdpa_noalloc(q, q, q, out, **kw)
    assert e.value.code == -4 and "static scratch" in str(e.value)
    cuda.cuda.synchronize()
    assert bool((out == 7.0).all())
