"""Pins the fp64 CPU oracle (oracle/oracle.c).

Each oracle function is checked three ways, chosen so a plausible slip (a
dropped term, a wrong sign or index, a transposed operand, the wrong variance
or the wrong causal alignment) fails at least one:
  * the committed golden fixtures (torch float64 library routines);
  * closed forms and special cases;
  * invariants of the mathematics (permutations, GQA == repeated MHA, ...).
The reference's only known-answer test near this path is nn.softmax(ones(5))
== 0.2 (reference tests/test_exhaustive.py:749); it is reproduced here.
"""
import numpy as np
import pytest

TOL = 1e-12


def test_layer_norm_matches_golden(oracle, golden):
    for name in ("ln_a", "ln_b"):
        x, g, b, eps = (golden[f"{name}_{s}"] for s in ("x", "gamma", "beta", "eps"))
        np.testing.assert_allclose(oracle.layer_norm(x, g, b, float(eps)), golden[f"{name}_y"],
                                   rtol=0, atol=TOL)
        np.testing.assert_allclose(oracle.layer_norm(x, None, None, float(eps)),
                                   golden[f"{name}_y_noaffine"], rtol=0, atol=TOL)


def test_layer_norm_closed_forms(oracle):
    rng = np.random.default_rng(0)
    beta = rng.standard_normal(16)
    gamma = rng.standard_normal(16)
    # A constant row has zero deviation: y == beta exactly.
    x = np.full((3, 16), 2.5)
    np.testing.assert_allclose(oracle.layer_norm(x, gamma, beta, 1e-5), np.broadcast_to(beta, x.shape),
                               atol=TOL)
    # Pre-affine output has row mean 0 and row variance var / (var + eps).
    x = rng.standard_normal((5, 64)) * 3.0 + 1.0
    eps = 1e-2
    y = oracle.layer_norm(x, None, None, eps)
    var = x.var(axis=-1)
    np.testing.assert_allclose(y.mean(axis=-1), 0.0, atol=1e-12)
    np.testing.assert_allclose(y.var(axis=-1), var / (var + eps), rtol=1e-12)
    # Invariant to x -> a*x + c (a > 0) once eps is negligible.
    y1 = oracle.layer_norm(x, None, None, 0.0)
    y2 = oracle.layer_norm(4.0 * x - 7.0, None, None, 0.0)
    np.testing.assert_allclose(y1, y2, atol=1e-12)
    # Brute force on n = 2: (x0 - m) / sqrt(((x0-x1)/2)^2 + eps).
    x = np.array([[1.0, 3.0]])
    np.testing.assert_allclose(oracle.layer_norm(x, None, None, 0.5),
                               [[-1.0 / np.sqrt(1.5), 1.0 / np.sqrt(1.5)]], atol=TOL)


def test_rms_norm_matches_golden(oracle, golden):
    x, w, eps = golden["rms_x"], golden["rms_w"], float(golden["rms_eps"])
    np.testing.assert_allclose(oracle.rms_norm(x, w, eps), golden["rms_y"], atol=TOL)
    np.testing.assert_allclose(oracle.rms_norm(x, None, eps), golden["rms_y_noweight"], atol=TOL)


def test_rms_norm_closed_forms(oracle):
    # x = c * 1 gives c / sqrt(c^2 + eps) in every element.
    for c in (0.5, -3.0, 7.25):
        y = oracle.rms_norm(np.full((2, 32), c), None, 1e-3)
        np.testing.assert_allclose(y, c / np.sqrt(c * c + 1e-3), atol=TOL)
    # Unlike LayerNorm, RMSNorm is not shift invariant: a mean-subtracting slip fails here.
    x = np.array([[1.0, 2.0, 3.0]])
    np.testing.assert_allclose(oracle.rms_norm(x, None, 0.0), x / np.sqrt(14.0 / 3.0), atol=TOL)


def test_log_softmax_against_scipy_and_invariants(oracle):
    """log-softmax pins: scipy.special.log_softmax (the routine the reference's
    own tests compare against, tests/test_exhaustive.py:688-689), rows whose
    logsumexp is 0, shift invariance, and the uniform row log(1/n)."""
    import scipy.special

    rng = np.random.default_rng(9)
    x = rng.standard_normal((7, 33)) * 5
    y = oracle.log_softmax(x)
    np.testing.assert_allclose(y, scipy.special.log_softmax(x, axis=-1), atol=1e-12)
    np.testing.assert_allclose(scipy.special.logsumexp(y, axis=-1), 0.0, atol=1e-12)
    np.testing.assert_allclose(oracle.log_softmax(x + 1e3), y, atol=1e-9)
    np.testing.assert_allclose(oracle.log_softmax(np.ones((2, 5))), np.log(0.2), atol=1e-15)
    # exp(log_softmax) is the softmax oracle
    np.testing.assert_allclose(np.exp(y), oracle.softmax(x), atol=1e-12)
    assert np.isnan(oracle.log_softmax(np.full((1, 4), -np.inf))).all()


def test_softmax_matches_golden_and_reference_kat(oracle, golden):
    np.testing.assert_allclose(oracle.softmax(golden["softmax_x"]), golden["softmax_y"], atol=TOL)
    # Reference KAT: nn.softmax(ones(5)) == 0.2 (tests/test_exhaustive.py:749).
    np.testing.assert_allclose(oracle.softmax(np.ones((1, 5))), 0.2, atol=TOL)
    # Shift invariance and an all -inf row giving NaN.
    x = np.random.default_rng(1).standard_normal((4, 9))
    np.testing.assert_allclose(oracle.softmax(x), oracle.softmax(x + 100.0), atol=1e-12)
    assert np.isnan(oracle.softmax(np.full((1, 4), -np.inf))).all()


@pytest.mark.parametrize("case", ["sdpa_f32", "sdpa_x"])
def test_sdpa_matches_golden(oracle, golden, case):
    q, k, v = (golden[f"{case}_{s}"] for s in "qkv")
    sc = float(golden[f"{case}_scale"])
    np.testing.assert_allclose(oracle.sdpa(q, k, v, sc), golden[f"{case}_out"], atol=1e-12)
    np.testing.assert_allclose(oracle.sdpa(q, k, v, sc, causal=True), golden[f"{case}_out_causal"],
                               atol=1e-12)


def test_sdpa_bf16_and_gqa_match_golden(oracle, golden):
    q, k, v = (golden[f"sdpa_bf16_{s}"] for s in "qkv")
    np.testing.assert_allclose(oracle.sdpa(q, k, v, float(golden["sdpa_bf16_scale"]), causal=True),
                               golden["sdpa_bf16_out_causal"], atol=1e-12)
    q, k, v, m = (golden[f"gqa_{s}"] for s in ("q", "k", "v", "mask"))
    np.testing.assert_allclose(oracle.sdpa(q, k, v, float(golden["gqa_scale"]), mask=m),
                               golden["gqa_out"], atol=1e-12)


def _qkv(rng, B=2, H=3, Tq=5, Tk=7, D=4, Dv=None):
    return (rng.standard_normal((B, H, Tq, D)), rng.standard_normal((B, H, Tk, D)),
            rng.standard_normal((B, H, Tk, Dv or D)))


def test_sdpa_closed_forms(oracle):
    rng = np.random.default_rng(2)
    # Tk = 1: every query returns the single value row.
    q, k, v = _qkv(rng, Tk=1)
    np.testing.assert_allclose(oracle.sdpa(q, k, v, 0.7), np.broadcast_to(v, q.shape), atol=TOL)
    # Identical keys: uniform weights, out = mean of the value rows.
    q, k, v = _qkv(rng)
    k[:] = k[:, :, :1, :]
    np.testing.assert_allclose(oracle.sdpa(q, k, v, 0.7),
                               np.broadcast_to(v.mean(axis=2, keepdims=True), q.shape), atol=1e-12)
    # Causal, top-left aligned: query 0 sees only key 0.
    q, k, v = _qkv(rng)
    out = oracle.sdpa(q, k, v, 0.7, causal=True)
    np.testing.assert_allclose(out[:, :, 0], v[:, :, 0], atol=TOL)
    # A row whose keys are all masked except j returns v_j.
    mask = np.full((1, 1, 5, 7), -np.inf)
    for i in range(5):
        mask[0, 0, i, (2 * i + 1) % 7] = 0.0
    out = oracle.sdpa(q, k, v, 0.7, mask=mask)
    for i in range(5):
        np.testing.assert_allclose(out[:, :, i], v[:, :, (2 * i + 1) % 7], atol=TOL)
    # Two keys, brute force: weights sigmoid(scale * q.(k0 - k1)).
    q = np.array([[[[1.0, 2.0]]]])
    k = np.array([[[[0.5, -1.0], [2.0, 0.25]]]])
    v = np.array([[[[1.0, 0.0], [0.0, 1.0]]]])
    s0, s1 = 0.5 * (0.5 - 2.0), 0.5 * (2.0 + 0.5)
    w0 = 1.0 / (1.0 + np.exp(s1 - s0))
    np.testing.assert_allclose(oracle.sdpa(q, k, v, 0.5)[0, 0, 0], [w0, 1 - w0], atol=TOL)


def test_sdpa_invariants(oracle):
    rng = np.random.default_rng(3)
    q, k, v = _qkv(rng, Tq=6, Tk=11, D=8, Dv=5)
    out = oracle.sdpa(q, k, v, 0.4)
    # Permuting keys together with values leaves non-causal attention unchanged.
    perm = rng.permutation(11)
    np.testing.assert_allclose(oracle.sdpa(q, k[:, :, perm], v[:, :, perm], 0.4), out, atol=1e-12)
    # Each output lies in the convex hull of the value rows (per feature bounds).
    assert (out <= v.max(axis=2, keepdims=True) + 1e-12).all()
    assert (out >= v.min(axis=2, keepdims=True) - 1e-12).all()
    # GQA == MHA with K/V repeated per group (repeat_interleave on heads).
    q = rng.standard_normal((2, 6, 4, 8))
    k = rng.standard_normal((2, 2, 9, 8))
    v = rng.standard_normal((2, 2, 9, 8))
    np.testing.assert_allclose(oracle.sdpa(q, k, v, 0.3, causal=True),
                               oracle.sdpa(q, np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1), 0.3,
                                           causal=True), atol=1e-12)
    # An additive mask equal to a constant per row changes nothing.
    mask = np.broadcast_to(rng.standard_normal((1, 1, 4, 1)), (1, 1, 4, 9))
    np.testing.assert_allclose(oracle.sdpa(q, k, v, 0.3, mask=mask), oracle.sdpa(q, k, v, 0.3),
                               atol=1e-12)
    # A fully masked row is NaN (0/0), as in the unfused softmax.
    mask = np.zeros((1, 1, 4, 9))
    mask[..., 2, :] = -np.inf
    out = oracle.sdpa(q, k, v, 0.3, mask=mask)
    assert np.isnan(out[:, :, 2]).all() and np.isfinite(out[:, :, [0, 1, 3]]).all()


def test_sdpa_rejects_bad_head_ratio(oracle):
    rng = np.random.default_rng(4)
    with pytest.raises(ValueError):
        oracle.sdpa(rng.standard_normal((1, 3, 2, 4)), rng.standard_normal((1, 2, 2, 4)),
                    rng.standard_normal((1, 2, 2, 4)), 1.0)


def test_layer_norm_bwd_matches_golden_and_fd(oracle, golden):
    x, w, g, eps = golden["lnb_x"], golden["lnb_w"], golden["lnb_g"], float(golden["lnb_eps"])
    dx, dw, db = oracle.layer_norm_bwd(x, w, g, eps)
    np.testing.assert_allclose(dx, golden["lnb_dx"], atol=1e-10)
    np.testing.assert_allclose(dw, golden["lnb_dw"], atol=1e-10)
    np.testing.assert_allclose(db, golden["lnb_db"], atol=1e-10)
    # Central finite differences of <g, LN(x)> in x.
    h = 1e-6
    fd = np.zeros_like(x)
    for idx in np.ndindex(*x.shape):
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        fd[idx] = ((g * oracle.layer_norm(xp, w, None, eps)).sum()
                   - (g * oracle.layer_norm(xm, w, None, eps)).sum()) / (2 * h)
    np.testing.assert_allclose(dx, fd, atol=1e-6)


def test_sdpa_bwd_matches_golden_and_fd(oracle, golden):
    q, k, v, g = (golden[f"sdpab_{s}"] for s in ("q", "k", "v", "g"))
    sc = float(golden["sdpab_scale"])
    dq, dk, dv = oracle.sdpa_bwd(q, k, v, g, sc)
    np.testing.assert_allclose(dq, golden["sdpab_dq"], atol=1e-10)
    np.testing.assert_allclose(dk, golden["sdpab_dk"], atol=1e-10)
    np.testing.assert_allclose(dv, golden["sdpab_dv"], atol=1e-10)
    # Finite differences for the causal GQA case, which no fixture covers.
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 4, 3, 4))
    k = rng.standard_normal((1, 2, 5, 4))
    v = rng.standard_normal((1, 2, 5, 4))
    g = rng.standard_normal((1, 4, 3, 4))
    dq, dk, dv = oracle.sdpa_bwd(q, k, v, g, 0.6, causal=True)
    h = 1e-6

    def loss(qq, kk, vv):
        return (g * oracle.sdpa(qq, kk, vv, 0.6, causal=True)).sum()

    for arr, grad, which in ((q, dq, 0), (k, dk, 1), (v, dv, 2)):
        fd = np.zeros_like(arr)
        for idx in np.ndindex(*arr.shape):
            ap, am = arr.copy(), arr.copy()
            ap[idx] += h
            am[idx] -= h
            args_p = [q, k, v]
            args_m = [q, k, v]
            args_p[which], args_m[which] = ap, am
            fd[idx] = (loss(*args_p) - loss(*args_m)) / (2 * h)
        np.testing.assert_allclose(grad, fd, atol=1e-6)
