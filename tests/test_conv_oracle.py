"""The oracle's causal depthwise Conv1D (modal/fast_conv.py:14-31) on the CPU.

Pinned by numpy's own convolution (y[:, c] is the first T entries of np.convolve(x[:, c], w[::-1, c])), by the
definition written as an explicit loop, and for the backward by the adjoint identities of a bilinear map:
<conv(x; w), dy> = <x, dx> = <w, dw> exactly (up to float64 rounding).  A planted mistake (taps reversed) fails
the convolve check.
"""
import numpy as np

from oracle import moe_oracle as mo


def _inputs(B, T, C, K, seed=0):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((B, T, C)), rng.standard_normal((K, C)), rng.standard_normal((B, T, C))


def test_conv_matches_numpy_convolve():
    x, w, _ = _inputs(2, 37, 5, 4)
    y = mo.causal_conv1d(x, w)
    for b in range(2):
        for c in range(5):
            assert np.allclose(y[b, :, c], np.convolve(x[b, :, c], w[::-1, c])[:37], rtol=1e-12, atol=1e-12)
    # a plausible mistake: taps applied in the opposite order
    bad = mo.causal_conv1d(x, w[::-1])
    assert not np.allclose(bad[0, :, 0], np.convolve(x[0, :, 0], w[::-1, 0])[:37])


def test_conv_explicit_loop_and_edges():
    x, w, _ = _inputs(1, 9, 3, 3, seed=1)
    y = mo.causal_conv1d(x, w)
    for t in range(9):
        want = sum(w[j] * x[0, t - 2 + j] for j in range(3) if t - 2 + j >= 0)
        assert np.allclose(y[0, t], want)
    # K = 1 is a per-channel scale; T < K still works
    assert np.allclose(mo.causal_conv1d(x, w[:1]), x * w[0])
    assert np.allclose(mo.causal_conv1d(x[:, :2], w)[0, 1], w[1] * x[0, 0] + w[2] * x[0, 1])


def test_conv_backward_adjoints():
    x, w, dy = _inputs(3, 50, 7, 4, seed=2)
    y = mo.causal_conv1d(x, w)
    dx, dw = mo.causal_conv1d_bwd(x, w, dy)
    lhs = float((y * dy).sum())
    assert np.isclose(lhs, float((x * dx).sum()), rtol=1e-12)
    assert np.isclose(lhs, float((w * dw).sum()), rtol=1e-12)
    # dx is the same causal convolution run backwards in time: dx[t] = sum_j w[j] dy[t + K-1 - j]
    flip = mo.causal_conv1d(dy[:, ::-1], w)[:, ::-1]
    assert np.allclose(dx, flip)


def test_applies_mirrors_reference_conditions():
    # modal/fast_conv.py:17-22: 1-D kernel, depthwise (groups == in == out), CAUSAL padding, rank-3 input, no bias,
    # dilation and stride 1; anything else goes to the original nnx.Conv
    import fast_conv
    ok = dict(kernel_size=(4,), feature_group_count=64, in_features=64, out_features=64, padding="CAUSAL", ndim=3)
    assert fast_conv.applies(**ok)
    assert fast_conv.applies(**dict(ok, kernel_size=4))
    for bad in (dict(kernel_size=(3, 3)), dict(feature_group_count=1), dict(out_features=128), dict(padding="SAME"),
                dict(ndim=4), dict(has_bias=True), dict(dilation=2), dict(strides=(2,))):
        assert not fast_conv.applies(**dict(ok, **bad)), bad
