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
