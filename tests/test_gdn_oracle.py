"""The Gated DeltaNet chunked-scan oracle (modal/gdn_fast.py:37-113) against the token-by-token recurrence.

The chunked WY form must reproduce the gated delta rule exactly (float64, no rounding) for any chunk size, for
lengths that need padding and with an initial state; the chunk-local inverse must equal numpy's triangular solve
and the reference's Neumann product (gdn_fast.py:21-34).  With the reference's bf16 rounding points the result
stays within a few bf16 steps of the exact one.  A planted mistake (the decay applied after the delta correction)
fails the recurrence check.
"""
import numpy as np
import pytest

from oracle import gdn_oracle as go


def _inputs(B=2, T=100, H=3, Dk=16, Dv=24, seed=0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, T, H, Dk))
    k = rng.standard_normal((B, T, H, Dk))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)  # the model l2-normalises keys; keeps the delta rule contractive
    v = rng.standard_normal((B, T, H, Dv))
    g = -np.abs(rng.standard_normal((B, T, H))) * 0.1   # log decay <= 0
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H))))
    return q, k, v, g, beta


@pytest.mark.parametrize("chunk,T", [(64, 100), (16, 100), (8, 64), (64, 1), (4, 13)])
def test_chunked_equals_recurrence(chunk, T):
    q, k, v, g, beta = _inputs(T=T, seed=chunk + T)
    o_ref, h_ref = go.gated_delta_recurrence(q, k, v, g, beta)
    o, h = go.gdn_chunked(q, k, v, g, beta, chunk=chunk)
    assert np.allclose(o, o_ref, rtol=1e-9, atol=1e-9)
    assert np.allclose(h, h_ref, rtol=1e-9, atol=1e-9)


def test_initial_state():
    q, k, v, g, beta = _inputs(T=50, seed=3)
    h0 = np.random.default_rng(4).standard_normal((2, 3, 16, 24))
    o_ref, h_ref = go.gated_delta_recurrence(q, k, v, g, beta, h0=h0)
    o, h = go.gdn_chunked(q, k, v, g, beta, chunk=16, h0=h0)
    assert np.allclose(o, o_ref, atol=1e-9) and np.allclose(h, h_ref, atol=1e-9)


def test_inverse_forms():
    rng = np.random.default_rng(5)
    C = 64
    S = np.tril(rng.standard_normal((3, C, C)) * 0.1, k=-1)
    A = go.unit_lower_inverse(S)
    eye = np.broadcast_to(np.eye(C), S.shape)
    assert np.allclose(A, np.linalg.solve(eye + S, eye), atol=1e-10)
    assert np.allclose(go.neumann_inverse(S[0]), A[0], atol=1e-10)


def test_planted_mistake_fails():
    # decay applied after the delta correction instead of before: a different recurrence
    q, k, v, g, beta = _inputs(T=40, seed=6)
    o, _ = go.gdn_chunked(q, k, v, g, beta, chunk=8)
    B, T, H, Dk = k.shape
    S = np.zeros((B, H, Dk, v.shape[-1]))
    bad = np.zeros_like(o)
    for t in range(T):
        pred = np.einsum("bhk,bhkv->bhv", k[:, t], S)
        S = (S + beta[:, t][..., None, None] * np.einsum("bhk,bhv->bhkv", k[:, t], v[:, t] - pred)) \
            * np.exp(g[:, t])[..., None, None]
        bad[:, t] = np.einsum("bhk,bhkv->bhv", q[:, t] / np.sqrt(Dk), S)
    assert not np.allclose(o, bad, atol=1e-6)


def test_bf16_rounding_points_stay_close():
    q, k, v, g, beta = _inputs(T=128, Dk=32, Dv=32, seed=7)
    o, _ = go.gdn_chunked(q, k, v, g, beta, chunk=64)
    o16, _ = go.gdn_chunked(q, k, v, g, beta, chunk=64, rounding="bf16")
    err = np.linalg.norm(o16 - o) / np.linalg.norm(o)
    assert 1e-4 < err < 2e-2, err


def test_correlated_keys_separate_inverse_mistakes(monkeypatch):
    """Keys sharing one direction (k = normalize(dir + 0.5 noise), the case the GPU tests add) make the chunk's
    S = (k beta) k^T large, so the exact inverse matters: the chunked form still equals the recurrence, the bf16
    rounding points stay within 1e-2 of it, and the approximation (I + S)^-1 ~ I - S -- what a blocked inverse that
    drops its diagonal-block factor degenerates to -- is off by far more than the 2e-2 bar (with i.i.d. keys it is
    not, which is why the correlated case is needed)."""
    rng = np.random.default_rng(11)
    B, T, H, D = 1, 128, 2, 128
    q = rng.standard_normal((B, T, H, D))
    v = rng.standard_normal((B, T, H, D))
    g = -np.abs(rng.standard_normal((B, T, H))) * 0.05
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H))))

    def keys(correlated):
        k = rng.standard_normal((B, T, H, D))
        if correlated:
            k = rng.standard_normal((1, 1, H, D)) + 0.5 * k
        return k / np.linalg.norm(k, axis=-1, keepdims=True)

    def rel(a, b):
        return np.linalg.norm(a - b) / np.linalg.norm(b)

    errs = {}
    for correlated in (False, True):
        k = keys(correlated)
        o_ref, _ = go.gated_delta_recurrence(q, k, v, g, beta)
        o, _ = go.gdn_chunked(q, k, v, g, beta, chunk=64)
        assert np.allclose(o, o_ref, rtol=1e-8, atol=1e-8)
        o16, _ = go.gdn_chunked(q, k, v, g, beta, chunk=64, rounding="bf16")
        assert rel(o16, o_ref) < 1e-2
        with monkeypatch.context() as m:
            m.setattr(go, "unit_lower_inverse", lambda S: np.eye(S.shape[-1]) - S)
            bad, _ = go.gdn_chunked(q, k, v, g, beta, chunk=64)
        errs[correlated] = rel(bad, o_ref)
    assert errs[True] > 0.1 and errs[True] > 5 * errs[False], errs


@pytest.mark.parametrize("chunk,T,with_state", [(8, 20, False), (4, 13, True), (16, 16, True)])
def test_backward_finite_differences(chunk, T, with_state):
    """The chunked backward equals central finite differences of the token recurrence (float64) for
    L = <do, o> + <dh_final, h_T>, on every input: q, k, v, g, beta and the initial state."""
    B, H, Dk, Dv = 1, 2, 5, 6
    q, k, v, g, beta = _inputs(B=B, T=T, H=H, Dk=Dk, Dv=Dv, seed=chunk + T)
    rng = np.random.default_rng(99)
    do = rng.standard_normal((B, T, H, Dv))
    h0 = rng.standard_normal((B, H, Dk, Dv)) * 0.3 if with_state else None
    dhf = rng.standard_normal((B, H, Dk, Dv)) if with_state else None
    grads = go.gdn_chunked_bwd(q, k, v, g, beta, do, chunk=chunk, h0=h0, dh_final=dhf)

    def loss(q_, k_, v_, g_, b_, h0_):
        o, hT = go.gated_delta_recurrence(q_, k_, v_, g_, b_, h0=h0_)
        return float((o * do).sum() + ((hT * dhf).sum() if dhf is not None else 0.0))

    args = [q, k, v, g, beta, h0 if h0 is not None else np.zeros((B, H, Dk, Dv))]
    eps = 1e-6
    for ai, name in enumerate(("dq", "dk", "dv", "dg", "dbeta", "dh0")):
        if name == "dh0" and not with_state:
            continue
        flat_idx = rng.choice(args[ai].size, size=min(6, args[ai].size), replace=False)
        for fi in flat_idx:
            idx = np.unravel_index(fi, args[ai].shape)
            plus = [a.copy() for a in args]
            minus = [a.copy() for a in args]
            plus[ai][idx] += eps
            minus[ai][idx] -= eps
            num = (loss(*plus) - loss(*minus)) / (2 * eps)
            got = grads[ai][idx]
            assert abs(num - got) <= 1e-6 * max(1.0, abs(num)), (name, idx, num, got)


def test_backward_planted_mistake_fails(monkeypatch):
    """Dropping the decay's term in the state update's key gradient (a plausible slip) breaks the finite-difference
    agreement the test above checks."""
    q, k, v, g, beta = _inputs(B=1, T=12, H=1, Dk=4, Dv=3, seed=5)
    do = np.random.default_rng(6).standard_normal((1, 12, 1, 3))
    dq, dk, dv, dg, db, _ = go.gdn_chunked_bwd(q, k, v, g, beta, do, chunk=4)
    eps = 1e-6
    kp, km = k.copy(), k.copy()
    kp[0, 2, 0, 1] += eps
    km[0, 2, 0, 1] -= eps
    L = lambda kk: float((go.gated_delta_recurrence(q, kk, v, g, beta)[0] * do).sum())  # noqa: E731
    num = (L(kp) - L(km)) / (2 * eps)
    assert abs(num - dk[0, 2, 0, 1]) < 1e-6
    real_exp = np.exp

    def no_decay_exp(x):  # e^0 = 1 for every decay factor: the gradient of a different function
        return real_exp(np.zeros_like(x))
    monkeypatch.setattr(go.np, "exp", no_decay_exp)
    _, dk_bad, _, _, _, _ = go.gdn_chunked_bwd(q, k, v, g, beta, do, chunk=4)
    monkeypatch.undo()
    assert abs(num - dk_bad[0, 2, 0, 1]) > 1e-3


def test_l2norm_oracle_pins():
    """l2norm_rows against what the formula fixes: each row's norm is sqrt(s / (s + eps)) for s = |x|^2 (so 1 as
    eps -> 0), the result is invariant to scaling a row, a zero row stays zero; l2norm_rows_bwd against central
    finite differences of l2norm_rows (float64), and a planted sign error in the r^3 term fails that check."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((6, 16)) * rng.uniform(0.01, 100, (6, 1))
    x[2] = 0.0
    y, r = go.l2norm_rows(x, 1e-6)
    s = (x * x).sum(-1)
    assert np.allclose(np.linalg.norm(y, axis=-1), np.sqrt(s / (s + 1e-6)), rtol=1e-12)
    y0, _ = go.l2norm_rows(x, 0.0 + 1e-300)
    assert np.allclose(go.l2norm_rows(3.5 * x, 1e-300)[0][[0, 1, 3, 4, 5]], y0[[0, 1, 3, 4, 5]], rtol=1e-12)
    assert not y[2].any() and np.isclose(r[2], 1e3)
    dy = rng.standard_normal(x.shape)
    dx = go.l2norm_rows_bwd(x, dy, 1e-6)
    num = np.zeros_like(x)
    for i in range(x.shape[0]):
        for j in range(x.shape[1]):
            h = 1e-6 * max(1.0, abs(x[i, j]))
            xp, xm = x.copy(), x.copy()
            xp[i, j] += h
            xm[i, j] -= h
            num[i, j] = ((go.l2norm_rows(xp, 1e-6)[0] - go.l2norm_rows(xm, 1e-6)[0]) * dy).sum() / (2 * h)
    assert np.allclose(dx, num, rtol=1e-5, atol=1e-7 * np.abs(num).max())
    xx = np.asarray(x, np.float64)
    rr = 1.0 / np.sqrt((xx * xx).sum(-1, keepdims=True) + 1e-6)
    planted = rr * dy + rr ** 3 * xx * (xx * dy).sum(-1, keepdims=True)
    assert not np.allclose(planted, num, rtol=1e-3)
