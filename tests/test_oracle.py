"""Pins the CPU oracle (oracle/moe_oracle.py, oracle/moe_oracle_c.c) before it is trusted as the checker.

Every function is checked against something independent of its own formula: an independent implementation
(torch's bf16 cast), brute force on tiny inputs, closed forms / invariants, the reference's known-answer case
(modal/te_run.py:72-79), the reference test's case list (modal/test_moe_permute.py:37-92), and central finite
differences for the backward.  A planted mistake test at the end shows the checks catch a wrong oracle.
"""
import itertools

import numpy as np
import pytest
import torch

from oracle import c_oracle as co
from oracle import moe_oracle as mo

# ------------------------------------------------------------------------------------------------ bf16


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    a = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10 ** rng.uniform(-30, 30, 100000),
                        np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 3.3895314e38, 1.0039062, 1.0117188], np.float32)])
    a = a.astype(np.float32)
    want = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(mo.bf16_bits(a), want)
    # ties to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7 -> rounds to 1 (even mantissa)
    assert mo.round_bf16(np.float32(1.0 + 2 ** -8)) == 1.0
    assert mo.round_bf16(np.float32(1.0 + 3 * 2 ** -8)) == np.float32(1.0 + 2 ** -6)


# ------------------------------------------------------------------------------------------------ router


def _brute_logits(x, w):
    T, d = x.shape
    out = np.zeros((T, w.shape[1]), np.float32)
    for t in range(T):
        for e in range(w.shape[1]):
            acc = np.float32(0)
            for i in range(d):
                acc = np.float32(acc + np.float32(x[t, i]) * np.float32(w[i, e]))
            out[t, e] = acc
    return out


def test_router_logits_sequential_order():
    p = mo.make_inputs(T=3, d=37, E=5, k=2, f=8, fs=0, seed=3)
    want = _brute_logits(p["x"], p["w_r"])
    got = mo.router_logits(p["x"], p["w_r"])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # and the value is the matmul up to f32 rounding
    ref = p["x"].astype(np.float64) @ p["w_r"].astype(np.float64)
    assert np.abs(got - ref).max() < 1e-5


def test_router_logits_c_matches_numpy_bitwise():
    p = mo.make_inputs(T=300, d=256, E=64, k=6, f=8, fs=0, seed=1, zipf=True)
    a = mo.router_logits(p["x"], p["w_r"], p["bias"])
    b = co.router_logits(p["x"], p["w_r"], p["bias"])
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_bf16_products_are_exact_in_f32():
    # the reason fused and unfused multiply-add agree in the router's fixed order
    rng = np.random.default_rng(5)
    a = mo.round_bf16(rng.standard_normal(100000).astype(np.float32))
    b = mo.round_bf16(rng.standard_normal(100000).astype(np.float32) * 0.02)
    assert np.array_equal((a * b).astype(np.float64), a.astype(np.float64) * b.astype(np.float64))


def _brute_topk(l, k):
    return np.array([sorted(range(len(r)), key=lambda e: (-float(r[e]), e))[:k] for r in l], np.int32)


@pytest.mark.parametrize("E,k", [(16, 6), (16, 12), (64, 6), (256, 8), (7, 7)])
def test_topk_brute_force_with_ties(E, k):
    rng = np.random.default_rng(E * 31 + k)
    l = rng.integers(-3, 3, size=(200, E)).astype(np.float32)  # many exact ties
    l[0] = 0.0
    l[1, :] = -0.0
    l[1, ::2] = 0.0  # +0 and -0 compare equal -> lower index first
    got = mo.topk_lower_index(l, k)
    assert np.array_equal(got, _brute_topk(l, k))
    assert np.array_equal(co.topk(l, k), got)
    assert np.array_equal(got[0], np.arange(k))  # all-equal row -> 0..k-1


def test_topk_softmax_closed_forms():
    l = np.array([[2.0, 1.0, 0.0, -1.0]], np.float32)
    sel = mo.topk_lower_index(l, 2)
    w = mo.topk_softmax(l, sel)
    assert np.array_equal(sel, [[0, 1]])
    assert np.allclose(w, [[1 / (1 + np.exp(-1.0)), np.exp(-1.0) / (1 + np.exp(-1.0))]], atol=1e-15)
    assert np.allclose(mo.topk_softmax(l, mo.topk_lower_index(l, 1)), 1.0)
    # norm_topk_prob: softmax over all then renormalised over the top-k == softmax over the selected logits
    full = np.exp(l - l.max()) / np.exp(l - l.max()).sum()
    assert np.allclose(w, full[0, :2] / full[0, :2].sum())


# ------------------------------------------------------------------------------------------------ layout


def _brute_sort(flat):
    order = sorted(range(len(flat)), key=lambda i: (flat[i], i))
    pos = [0] * len(flat)
    for p, i in enumerate(order):
        pos[i] = p
    return np.array(order, np.int32), np.array(pos, np.int32)


@pytest.mark.parametrize("n,k,E", [(64, 6, 16), (64, 12, 16), (1, 1, 4), (333, 8, 256), (50, 3, 3)])
def test_sort_indices_brute_force(n, k, E):
    rng = np.random.default_rng(n + k + E)
    sel = np.stack([rng.permutation(E)[:k] for _ in range(n)]).astype(np.int32)
    order, pos = mo.sort_indices(sel.reshape(-1), E)
    bo, bp = _brute_sort(sel.reshape(-1).tolist())
    assert np.array_equal(order, bo) and np.array_equal(pos, bp)


def test_layout_invariants_and_c_oracle():
    rng = np.random.default_rng(7)
    T, k, E = 2000, 6, 64
    logits = rng.standard_normal((T, E)).astype(np.float32) + mo.zipf_bias(E)
    sel = mo.topk_lower_index(logits, k)
    lay = mo.build_layout(sel, E)
    flat = sel.reshape(-1)
    M = flat.shape[0]
    assert np.array_equal(np.sort(lay["order"]), np.arange(M))           # a permutation
    assert np.array_equal(lay["pos"][lay["order"]], np.arange(M))        # pos = order^-1
    assert np.array_equal(lay["group_sizes"], np.bincount(flat, minlength=E))
    assert np.array_equal(lay["offsets"], np.concatenate([[0], np.cumsum(lay["group_sizes"])[:-1]]))
    fs = flat[lay["order"]]
    assert np.all(np.diff(fs) >= 0)                                      # sorted by expert
    same = np.diff(fs) == 0
    assert np.all(np.diff(lay["order"])[same] > 0)                       # stable: slot index ascending in e
    nblk = -(-lay["group_sizes"] // 128)
    assert lay["num_blocks"] == nblk.sum() <= mo.max_blocks(M, E)
    assert np.array_equal(lay["slot"] // 128 - lay["block_off"][flat], (lay["pos"] - lay["offsets"][flat]) // 128)
    assert len(set(lay["slot"].tolist())) == M                            # slots are distinct
    assert np.array_equal(lay["block_expert"][lay["slot"] // 128], flat)  # slot lies in a block of its expert
    c = co.build_layout(sel, E)
    for key in lay:
        assert np.array_equal(np.asarray(lay[key]), np.asarray(c[key])), key


# ------------------------------------------------------------------------------------------------ row movement


def _loops_gather_reduce(y, pos, w):
    n, k = pos.shape
    out = np.zeros((n, y.shape[1]))
    for t in range(n):
        for j in range(k):
            out[t] += (1.0 if w is None else w[t, j]) * y[pos[t, j]]
    return out


def test_gather_ops_against_loops():
    rng = np.random.default_rng(11)
    n, k, d = 9, 3, 5
    y = rng.standard_normal((n * k, d))
    pos = rng.permutation(n * k).reshape(n, k)
    w = rng.random((n, k))
    g = rng.standard_normal((n, d))
    assert np.allclose(mo.gather_reduce(y, pos, w), _loops_gather_reduce(y, pos, w))
    assert np.allclose(mo.gather_reduce(y, pos, None), _loops_gather_reduce(y, pos, None))
    dots = np.array([[sum(g[t, c] * y[pos[t, j], c] for c in range(d)) for j in range(k)] for t in range(n)])
    assert np.allclose(mo.gather_dot(y, pos, g), dots)
    idx = rng.integers(0, n * k, 20)
    assert np.array_equal(mo.gather_rows(y, idx), np.stack([y[i] for i in idx]))


def test_dispatch_combine_identity_expert():
    """Identity expert: combine(dispatch(x)) = sum_j w[t,j] x[t] = x[t] when the weights sum to 1."""
    rng = np.random.default_rng(12)
    n, k, E, d = 64, 6, 16, 32
    x = rng.standard_normal((n, d))
    sel = np.stack([rng.permutation(E)[:k] for _ in range(n)]).astype(np.int32)
    flat = sel.reshape(-1)
    order, pos = mo.sort_indices(flat, E)
    w = rng.random((n, k))
    w /= w.sum(1, keepdims=True)
    assert np.allclose(mo.combine(mo.dispatch(x, order, pos), pos, w), x)
    assert np.allclose(mo.ref_combine(mo.ref_dispatch(x, flat), flat, w), x)
    # one-hot weights pick exactly the chosen expert's row
    oh = np.zeros((n, k))
    oh[:, 2] = 1.0
    ys = mo.dispatch(x, order, pos) * 3.0
    assert np.allclose(mo.combine(ys, pos, oh), 3.0 * x)


def test_combine_bwd_and_permute_rows_vjp():
    rng = np.random.default_rng(13)
    n, k, E, d = 20, 4, 8, 6
    sel = np.stack([rng.permutation(E)[:k] for _ in range(n)]).astype(np.int32)
    order, pos = mo.sort_indices(sel.reshape(-1), E)
    y = rng.standard_normal((n * k, d))
    w = rng.random((n, k))
    g = rng.standard_normal((n, d))
    dy, dw = mo.combine_bwd(y, order, pos, w, g, dtype="f64")
    # finite differences of L = <g, combine(y, w)> (linear, so exact up to rounding)
    L = lambda yy, ww: float((g * mo.combine(yy, pos, ww)).sum())  # noqa: E731
    eps = 1e-6
    for (r, c) in [(0, 0), (5, 3), (n * k - 1, d - 1)]:
        yp = y.copy(); yp[r, c] += eps
        ym = y.copy(); ym[r, c] -= eps
        assert abs((L(yp, w) - L(ym, w)) / (2 * eps) - dy[r, c]) < 1e-6
    for (t, j) in [(0, 0), (7, 3)]:
        wp = w.copy(); wp[t, j] += eps
        wm = w.copy(); wm[t, j] -= eps
        assert abs((L(y, wp) - L(y, wm)) / (2 * eps) - dw[t, j]) < 1e-6
    perm = rng.permutation(n * k)
    gg = rng.standard_normal((n * k, d))
    # <gg, x[perm]> = <permute_rows_bwd(gg), x>
    x = rng.standard_normal((n * k, d))
    assert np.isclose((gg * mo.permute_rows(x, perm)).sum(), (mo.permute_rows_bwd(gg, perm) * x).sum())


def test_invert_permutation_guarded_contract():
    """The inverse of a permutation is its argsort; with out-of-range entries (an index that is not a permutation),
    a scalar loop of the guarded scatter: skipped entries, and m where no index lands."""
    rng = np.random.default_rng(21)
    for m in (1, 2, 37, 1000):
        perm = rng.permutation(m).astype(np.int32)
        assert np.array_equal(mo.invert_permutation(perm), np.argsort(perm, kind="stable"))
        bad = perm.copy()
        hit = rng.choice(m, size=max(1, m // 5), replace=False)
        bad[hit] = rng.choice([-1, -7, m, m + 3, 2**31 - 1], size=hit.size)
        want = [m] * m
        for i, v in enumerate(bad.tolist()):
            if 0 <= v < m:
                want[v] = i
        assert np.array_equal(mo.invert_permutation(bad), np.array(want, np.int32))


# ------------------------------------------------------------------------------------------------ grouped GEMM


def test_ragged_dot_known_answer_case():
    """modal/te_run.py:72-79: gs=[5,0,9,3,7,1,6,4], M = sum(gs)+3 (tail rows), K=64, N=48."""
    gs = np.array([5, 0, 9, 3, 7, 1, 6, 4])
    S = int(gs.sum())
    M, K, N = S + 3, 64, 48
    rng = np.random.default_rng(0)
    a = mo.round_bf16(rng.standard_normal((M, K)).astype(np.float32))
    b = mo.round_bf16(rng.standard_normal((8, K, N)).astype(np.float32))
    out = mo.ragged_dot(a, b, gs)
    assert np.all(out[S:] == 0)
    r = 0
    for e, g in enumerate(gs):
        for i in range(g):  # row by row, no slicing arithmetic shared with the oracle
            assert np.allclose(out[r], a[r].astype(np.float64) @ b[e].astype(np.float64))
            r += 1
    # padded_gmm's capacity layout gives the same result when no group exceeds C ...
    assert padded_ok(a, b, gs, factor=8.0)
    # ... and drops rows past C otherwise (factor 1.0 -> C = 8 < 9)
    cap = mo.padded_ragged_dot_capacity(a, b, gs, 1.0)
    c = mo.padded_capacity(M, 8, 1.0)
    assert c == 8
    assert np.all(cap[5 + 8] == 0) and np.allclose(cap[5:5 + 8], out[5:5 + 8])
    dl, dr = mo.ragged_dot_bwd(a, b, gs, np.ones((M, N)))
    assert np.all(dl[S:] == 0)
    assert np.allclose(dr[1], 0)  # empty group
    assert np.allclose(dr[0], a[:5].astype(np.float64).T @ np.ones((5, N)))


def padded_ok(a, b, gs, factor):
    return np.allclose(mo.padded_ragged_dot_capacity(a, b, gs, factor), mo.ragged_dot(a, b, gs))


# ------------------------------------------------------------------------------------------------ layer


TINY = dict(T=8, d=16, E=8, k=2, f=8, fs=8)


def _loss(p, dy):
    out, _ = mo.moe_layer_fwd(p)
    return float((out * dy).sum())


def test_layer_forward_against_token_loop():
    p = mo.make_inputs(**TINY, seed=4)
    out, cache = mo.moe_layer_fwd(p)
    x = p["x"].astype(np.float64)
    lf = _brute_logits(p["x"], p["w_r"]).astype(np.float64)  # routing runs on the f32 logits
    for t in range(TINY["T"]):
        l = lf[t]
        top = sorted(range(TINY["E"]), key=lambda e: (-l[e], e))[:TINY["k"]]
        l64 = x[t] @ p["w_r"].astype(np.float64)  # weights: softmax of the exact logits at the selection
        z = np.exp(l64[top] - l64[top].max())
        w = z / z.sum()
        acc = np.zeros(TINY["d"])
        for j, e in enumerate(top):
            gg = x[t] @ p["w_gate"][e]
            uu = x[t] @ p["w_up"][e]
            acc += w[j] * ((gg / (1 + np.exp(-gg)) * uu) @ p["w_down"][e])
        gs_ = x[t] @ p["ws_gate"]
        acc += (gs_ / (1 + np.exp(-gs_)) * (x[t] @ p["ws_up"])) @ p["ws_down"]
        assert np.allclose(out[t], acc, rtol=1e-9, atol=1e-12)


def test_layer_backward_finite_differences():
    p = mo.make_inputs(**TINY, seed=5)
    for n in ("w_r", "w_gate", "w_up", "w_down", "ws_gate", "ws_up", "ws_down"):
        p[n] = p[n] * 20.0  # O(1) weights so every term is visible in the differences
    p["x"] = p["x"].astype(np.float64)
    rng = np.random.default_rng(9)
    dy = rng.standard_normal((TINY["T"], TINY["d"]))
    out, cache = mo.moe_layer_fwd(p)
    g = mo.moe_layer_bwd(p, cache, dy)
    eps = 1e-6
    checks = {"x": "dx", "w_r": "dw_r", "w_gate": "dw_gate", "w_up": "dw_up", "w_down": "dw_down",
              "ws_gate": "dws_gate", "ws_up": "dws_up", "ws_down": "dws_down"}
    for name, gname in checks.items():
        arr = np.asarray(p[name], np.float64)
        for _ in range(6):
            idx = tuple(rng.integers(0, s) for s in arr.shape)
            q = dict(p)
            a1 = arr.copy(); a1[idx] += eps
            a2 = arr.copy(); a2[idx] -= eps
            q[name] = a1
            lp = _loss(q, dy)
            q[name] = a2
            lm = _loss(q, dy)
            # the routing must not flip under the perturbation for the difference to be a derivative
            q[name] = a1
            assert np.array_equal(mo.moe_layer_fwd(q)[1]["sel"], cache["sel"])
            fd = (lp - lm) / (2 * eps)
            assert abs(fd - g[gname][idx]) <= 1e-6 * max(1.0, abs(fd)), (name, idx, fd, g[gname][idx])


def test_per_expert_and_shared_slices_match_layer_oracle():
    """expert_grads / shared_grads / router_wgrad (the slices the full-size C5 test uses) equal the whole-layer
    oracle's gradients, which the finite-difference test pins."""
    p = mo.make_inputs(T=300, d=64, E=8, k=3, f=32, fs=48, seed=4)
    out, cache = mo.moe_layer_fwd(p)
    g = mo.moe_layer_bwd(p, cache, p["dy"])
    sel = cache["sel"]
    for e in range(8):
        dwg, dwu, dwd = mo.expert_grads(p, sel, e, p["dy"], np.float64)
        assert np.allclose(dwg, g["dw_gate"][e], rtol=1e-10, atol=1e-12)
        assert np.allclose(dwu, g["dw_up"][e], rtol=1e-10, atol=1e-12)
        assert np.allclose(dwd, g["dw_down"][e], rtol=1e-10, atol=1e-12)
    dsg, dsu, dsd, _ = mo.shared_grads(p, p["dy"], np.float64)
    for a, n in ((dsg, "dws_gate"), (dsu, "dws_up"), (dsd, "dws_down")):
        assert np.allclose(a, g[n], rtol=1e-10, atol=1e-12), n
    assert np.allclose(mo.router_wgrad(p, sel, g["dw"], np.float64), g["dw_r"], rtol=1e-10, atol=1e-12)
    # an expert no token picks has zero gradients
    p2 = dict(p, bias=np.array([9.0] * 3 + [0.0] * 5, np.float32))
    _, c2 = mo.moe_layer_fwd(p2)
    assert not any(a.any() for a in mo.expert_grads(p2, c2["sel"], 7, p2["dy"]))


def test_oracle_catches_planted_mistake(monkeypatch):
    """A wrong oracle (dsilu missing its second term) must fail the finite-difference check."""
    p = mo.make_inputs(**TINY, seed=5)
    for n in ("w_gate", "w_up", "w_down"):
        p[n] = p[n] * 20.0
    p["x"] = p["x"].astype(np.float64)
    rng = np.random.default_rng(9)
    dy = rng.standard_normal((TINY["T"], TINY["d"]))
    monkeypatch.setattr(mo, "dsilu", lambda z: 1.0 / (1.0 + np.exp(-z)))
    out, cache = mo.moe_layer_fwd(p)
    g = mo.moe_layer_bwd(p, cache, dy)
    e = int(cache["sel"][0, 0])
    idx = (e, 3, 2)
    eps = 1e-6
    q = dict(p)
    a1 = p["w_gate"].astype(np.float64).copy(); a1[idx] += eps
    a2 = p["w_gate"].astype(np.float64).copy(); a2[idx] -= eps
    q["w_gate"] = a1
    lp = _loss(q, dy)
    q["w_gate"] = a2
    lm = _loss(q, dy)
    assert abs((lp - lm) / (2 * eps) - g["dw_gate"][idx]) > 1e-6


def test_configs_match_baseline():
    c = mo.CONFIGS
    assert (c["C2"]["T"], c["C2"]["d"], c["C2"]["E"], c["C2"]["k"], c["C2"]["f"], c["C2"]["fs"]) == \
        (16384, 1024, 64, 6, 512, 512)
    assert c["C4"]["zipf"] and c["C5"]["k"] == 8 and c["C5"]["fs"] == 2048
    b = mo.zipf_bias(128)
    assert b[0] == 0 and np.isclose(b[1], -1.5 * np.log(2))


def test_small_case_itertools_topk_exhaustive():
    """All 2-of-4 selections on every tie pattern over {0,1} logits."""
    for bits in itertools.product([0.0, 1.0], repeat=4):
        l = np.array([bits], np.float32)
        assert np.array_equal(mo.topk_lower_index(l, 2), _brute_topk(l, 2))
