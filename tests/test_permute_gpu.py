"""GPU parity of the row-movement kernels and routing indices against the CPU oracle.

Mirrors the reference's own test (modal/test_moe_permute.py:37-92): E=16, n=64, d=256, k in {6, 12},
dtype in {f32, bf16}; gather_rows exact (tol 0), with scale and the reductions at 2e-2 (bf16) / 1e-5 (f32) of the
max-normalised error (29-34, 46); sort_indices bit-exact for both methods (64-68); moe_block forward and gradients
with a tanh expert (70-81); permute_rows gradient (83-87); and the 60-row "untileable" case (89-91).
Plus: larger and ragged shapes, empty inputs, f16, out-of-range sentinels and full-size sorts.
"""
import numpy as np
import pytest
import torch

import moe_permute as mp
from oracle import moe_oracle as mo

pytestmark = pytest.mark.gpu

E = 16
TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _t(a, dtype, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dtype)


def _cast_np(a, name):
    return mo._cast(np.asarray(a, np.float32), name)


def rand_routing(rng, n, k, e=E):
    """Top-k expert ids without repeats per token (modal/test_moe_permute.py:23-26)."""
    logits = rng.standard_normal((n, e)).astype(np.float32)
    return mo.topk_lower_index(logits, k)


def check(got, want, tol):
    got = np.asarray(got.float().cpu() if torch.is_tensor(got) else got, np.float64)
    assert got.shape == np.asarray(want).shape
    err = mo.rel_max(got, want)
    assert err <= tol, err
    return err


@pytest.mark.parametrize("dname,k", [("f32", 6), ("bf16", 6), ("bf16", 12), ("f32", 12), ("f16", 6)])
def test_reference_case(dname, k, dev):
    n, d = 64, 256
    dtype = TORCH_DT[dname]
    rng = np.random.default_rng(k * 7 + (dname == "bf16"))
    x_np = _cast_np(rng.standard_normal((n, d)), dname)
    sel = rand_routing(rng, n, k)
    flat = sel.reshape(-1)
    w_np = rng.standard_normal((n, k))
    w_np = np.exp(w_np) / np.exp(w_np).sum(1, keepdims=True)
    m = n * k
    y_np = _cast_np(rng.standard_normal((m, d)), dname)
    tol = 1e-5 if dname == "f32" else 2e-2
    x, y = _t(x_np, dtype, dev), _t(y_np, dtype, dev)
    w = _t(w_np, torch.float32, dev)

    order_np, pos_np = mo.sort_indices(flat, E)
    pos2 = pos_np.reshape(n, k)
    idx_np = (rng.permutation(m) % n).astype(np.int32)
    scale_np = rng.standard_normal(m).astype(np.float32)
    idx, scale = _t(idx_np, torch.int32, dev), _t(scale_np, torch.float32, dev)
    # 1. kernels vs the oracle
    got = mp.gather_rows(x, idx)
    assert torch.equal(got.cpu(), x.cpu()[idx.cpu().long()])                     # exact copy
    check(mp.gather_rows(x, idx, scale), mo.gather_rows(x_np, idx_np, scale_np, dname), tol)
    pos_t = _t(pos2, torch.int32, dev)
    check(mp.gather_reduce(y, pos_t, None, torch.float32), mo.gather_reduce(y_np, pos2), tol)
    check(mp.gather_reduce(y, pos_t, w, torch.float32), mo.gather_reduce(y_np, pos2, w_np.astype(np.float32)), tol)
    g_np = rng.standard_normal((n, d)).astype(np.float32)
    g = _t(g_np, torch.float32, dev)
    check(mp.gather_dot(y, pos_t, g), mo.gather_dot(y_np, pos2, g_np), tol)
    # 2. sort_indices, both methods, bit-exact
    flat_t = _t(flat, torch.int32, dev)
    for method in ("argsort", "count"):
        o2, p2 = mp.sort_indices(flat_t, E, method)
        assert np.array_equal(o2.cpu().numpy(), order_np)
        assert np.array_equal(p2.cpu().numpy(), pos_np)
    # 3. moe_block forward + gradients (tanh expert) vs the oracle's dispatch/combine and their VJPs
    mp.CFG["num_experts"] = E
    try:
        xg = x.clone().requires_grad_(True)
        wg = w.clone().requires_grad_(True)
        out = mp.moe_block(xg, flat_t, wg, lambda r: torch.tanh(r.float()).to(r.dtype), use_kernels=True)
        loss = (out * g).sum()
        loss.backward()
    finally:
        mp.CFG["num_experts"] = None
    xs = mo.dispatch(x_np, order_np, pos_np)
    ys = _cast_np(np.tanh(xs.astype(np.float64)), dname)
    want_out = mo.combine(ys, pos_np, w_np.astype(np.float32))
    check(out.detach(), want_out, tol)
    # gradients: combine bwd -> tanh' -> dispatch bwd
    dys, dw = mo.combine_bwd(ys, order_np, pos_np, w_np.astype(np.float32), g_np, dname)
    dxs = _cast_np(dys.astype(np.float64) * (1 - np.tanh(xs.astype(np.float64)) ** 2), dname)
    dx = mo.dispatch_bwd(dxs, pos_np, n)
    check(xg.grad, dx, tol)
    check(wg.grad, dw, tol)
    # 4. permute_rows gradient
    perm_np = rng.permutation(m).astype(np.int32)
    yg = y.clone().requires_grad_(True)
    gi = g[idx.long()]
    (mp.permute_rows(yg, _t(perm_np, torch.int32, dev)).float() * gi).sum().backward()
    want = mo.permute_rows_bwd(g_np[idx_np], perm_np)
    check(yg.grad, _cast_np(want, dname), tol)
    # 5. the reference's "untileable" 60-row case: same kernels, no fallback needed
    xs60, ids60 = x[:60], idx[:60] % 60
    assert torch.equal(mp.gather_rows(xs60, ids60).cpu(), xs60.cpu()[ids60.cpu().long()])


def test_ragged_widths_and_sentinels(dev):
    rng = np.random.default_rng(3)
    for d in (1, 3, 7, 100, 1000, 1032):
        x_np = mo.round_bf16(rng.standard_normal((37, d)).astype(np.float32))
        x = _t(x_np, torch.bfloat16, dev)
        idx_np = rng.integers(-2, 40, 50).astype(np.int32)  # out-of-range -> zero rows
        got = mp.gather_rows(x, _t(idx_np, torch.int32, dev)).float().cpu().numpy()
        want = np.where(((idx_np >= 0) & (idx_np < 37))[:, None], x_np[np.clip(idx_np, 0, 36)], 0.0)
        assert np.array_equal(got, want)
        pos = rng.integers(0, 37, (11, 4)).astype(np.int32)
        check(mp.gather_reduce(x, _t(pos, torch.int32, dev), None, torch.float32), mo.gather_reduce(x_np, pos), 1e-6)


@pytest.mark.parametrize("dname,k,d", [("bf16", 3, 256), ("bf16", 9, 1024), ("f32", 17, 264), ("f16", 12, 104),
                                        ("bf16", 8, 7), ("f32", 1, 8)])
def test_gather_reduce_dot_out_of_range_positions(dname, k, d, dev):
    """gather_reduce and gather_dot with a quarter of the positions outside [0, m) (negative or past the end): such
    a position contributes nothing to the reduction and gives the dot product 0.  k below, at and above the
    kernels' batch of 8 choices, and widths on the 16-byte and on the scalar path."""
    rng = np.random.default_rng(k * 100 + d)
    m, n = 50, 40
    dtype = TORCH_DT[dname]
    tol = 1e-5 if dname == "f32" else 2e-2
    y_np = _cast_np(rng.standard_normal((m, d)), dname)
    pos = rng.integers(0, m, (n, k)).astype(np.int32)
    bad = rng.random((n, k)) < 0.25
    pos[bad] = rng.choice(np.array([-1, -7, m, m + 3, 2**31 - 1], np.int32), size=int(bad.sum()))
    w_np = rng.random((n, k)).astype(np.float32)
    g_np = rng.standard_normal((n, d)).astype(np.float32)
    valid = (pos >= 0) & (pos < m)
    rows = np.where(valid[..., None], y_np.astype(np.float64)[np.clip(pos, 0, m - 1)], 0.0)  # (n, k, d)
    want_sum = rows.sum(1)
    want_red = (rows * w_np[..., None]).sum(1)
    want_dot = (rows * g_np[:, None, :]).sum(-1)
    y, pos_t = _t(y_np, dtype, dev), _t(pos, torch.int32, dev)
    check(mp.gather_reduce(y, pos_t, None, torch.float32), want_sum, tol)
    check(mp.gather_reduce(y, pos_t, _t(w_np, torch.float32, dev), torch.float32), want_red, tol)
    got_dot = mp.gather_dot(y, pos_t, _t(g_np, torch.float32, dev))
    check(got_dot, want_dot, tol)
    assert not got_dot.cpu().numpy()[~valid].any()  # exactly 0 where the position is out of range


@pytest.mark.parametrize("dname,k,d", [("bf16", 6, 1024), ("f32", 11, 264), ("bf16", 3, 7)])
def test_combine_bwd_out_of_range_positions(dname, k, d, dev):
    """lsurge_combine_bwd with a quarter of the positions outside [0, m): dy rows are written only at the valid
    positions (w_j g[t], rounded to y's dtype), the others keep what they held, and dw is exactly 0 for the invalid
    choices and <g[t], y[pos]> for the valid ones."""
    import _lib as L
    rng = np.random.default_rng(k + d)
    n = 30
    m = n * k
    dtype = TORCH_DT[dname]
    tol = 1e-5 if dname == "f32" else 2e-2
    y_np = _cast_np(rng.standard_normal((m, d)), dname)
    pos = rng.permutation(m)[: n * k].reshape(n, k).astype(np.int32)
    bad = rng.random((n, k)) < 0.25
    pos[bad] = rng.choice(np.array([-1, -9, m, m + 5], np.int32), size=int(bad.sum()))
    valid = (pos >= 0) & (pos < m)
    w_np = rng.random((n, k)).astype(np.float32)
    g_np = _cast_np(rng.standard_normal((n, d)), dname)
    y, g = _t(y_np, dtype, dev), _t(g_np, dtype, dev)
    pos_t, w = _t(pos, torch.int32, dev), _t(w_np, torch.float32, dev)
    dy = torch.full((m, d), 7.0, dtype=dtype, device=dev)
    dw = torch.empty((n, k), dtype=torch.float32, device=dev)
    L.check(L.lib().lsurge_combine_bwd(L.ptr(y), L.dt(y), L.ptr(pos_t), L.ptr(w), n, k, d, L.ptr(g), L.dt(g),
                                       L.ptr(dy), L.ptr(dw), L.stream(dev)), "combine_bwd")
    got_dy, got_dw = dy.float().cpu().numpy(), dw.cpu().numpy()
    want_dw = np.where(valid, np.einsum("tkd,td->tk", y_np.astype(np.float64)[np.clip(pos, 0, m - 1)],
                                        g_np.astype(np.float64)), 0.0)
    check(got_dw, want_dw, tol)
    assert not got_dw[~valid].any()
    hit = np.zeros(m, bool)
    hit[pos[valid]] = True
    assert np.all(got_dy[~hit] == 7.0)  # rows no valid position names are untouched
    want_rows = w_np[valid][:, None].astype(np.float64) * g_np[np.nonzero(valid)[0]].astype(np.float64)
    check(got_dy[pos[valid]], _cast_np(want_rows, dname), tol)


def test_empty_inputs(dev):
    x = torch.zeros((0, 64), dtype=torch.bfloat16, device=dev)
    idx = torch.zeros((0,), dtype=torch.int32, device=dev)
    assert mp.gather_rows(torch.ones((4, 64), dtype=torch.bfloat16, device=dev), idx).shape == (0, 64)
    o, p = mp.sort_indices(idx, 4)
    assert o.numel() == 0 and p.numel() == 0
    assert mp.gather_reduce(x, torch.zeros((0, 3), dtype=torch.int32, device=dev)).shape == (0, 64)


@pytest.mark.parametrize("name", ["C1", "C2", "C4", "C5"])
def test_sort_indices_full_size(name, dev):
    c = mo.CONFIGS[name]
    rng = np.random.default_rng(c["seed"])
    logits = rng.standard_normal((c["T"], c["E"])).astype(np.float32)
    if c["zipf"]:
        logits += mo.zipf_bias(c["E"])
    flat = mo.topk_lower_index(logits, c["k"]).reshape(-1)
    order_np, pos_np = mo.sort_indices(flat, c["E"])
    o, p = mp.sort_indices(_t(flat, torch.int32, dev), c["E"], "count")
    assert np.array_equal(o.cpu().numpy(), order_np)
    assert np.array_equal(p.cpu().numpy(), pos_np)


def test_full_size_dispatch_combine_round_trip(dev):
    """C2 shape: combine(dispatch(x)) with weights summing to 1 is x (identity expert), f32 accumulate."""
    c = mo.CONFIGS["C2"]
    T, d, k, e = c["T"], c["d"], c["k"], c["E"]
    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((T, d), device=dev, generator=gen).to(torch.bfloat16)
    flat = torch.randint(0, e, (T * k,), device=dev, generator=gen, dtype=torch.int32)
    w = torch.rand((T, k), device=dev, generator=gen)
    w = w / w.sum(1, keepdim=True)
    order, pos = mp.sort_indices(flat, e)
    out = mp.combine(mp.dispatch(x, order, pos), order, pos, w)
    assert (out - x.float()).abs().max().item() < 1e-5 * x.float().abs().max().item() + 1e-6


def test_invert_permutation_out_of_range_entries(dev):
    """The inverse-permutation kernel behind permute_rows' backward skips indices outside [0, m) (no write leaves inv)
    and leaves m where no index lands, so the gather through it gives zero rows there (oracle.invert_permutation)."""
    import _lib as L
    rng = np.random.default_rng(8)
    for m in (1, 300, 70001):
        idx_np = rng.permutation(m).astype(np.int32)
        hit = rng.choice(m, size=max(1, m // 7), replace=False)
        idx_np[hit] = rng.choice(np.array([-1, -5, m, m + 9, 2**31 - 1], np.int32), size=hit.size)
        inv = torch.full((m,), -3, dtype=torch.int32, device=dev)
        idx = _t(idx_np, torch.int32, dev)
        L.check(L.lib().lsurge_invert_permutation(L.ptr(idx), m, L.ptr(inv), L.stream(dev)), "invert_permutation")
        assert np.array_equal(inv.cpu().numpy(), mo.invert_permutation(idx_np))
    # through permute_rows' backward: rows of g whose slot no index names come back as zeros
    m, d = 50, 24
    idx_np = rng.permutation(m).astype(np.int32)
    idx_np[[3, 17]] = [m + 1, -2]
    x = torch.randn((m, d), device=dev).to(torch.bfloat16).requires_grad_(True)
    g = torch.randn((m, d), device=dev).to(torch.bfloat16)
    mp.permute_rows(x, _t(idx_np, torch.int32, dev)).backward(g)
    inv = mo.invert_permutation(idx_np)
    g_np = g.float().cpu().numpy()
    want = np.where((inv < m)[:, None], g_np[np.minimum(inv, m - 1)], 0.0)
    assert np.array_equal(x.grad.float().cpu().numpy(), want)


@pytest.mark.parametrize("k,dname", [(24, "bf16"), (17, "f32"), (40, "f16")])
def test_combine_any_k(k, dname, dev):
    """combine forward and its fused backward for k above 16 (the reference takes any k,
    modal/moe_permute.py:292-312): dy rows, dw and the gather-reduce forward against the oracle."""
    n, d, e = 96, 264, 64
    dtype = TORCH_DT[dname]
    tol = 1e-5 if dname == "f32" else 2e-2
    rng = np.random.default_rng(k)
    sel = rand_routing(rng, n, k, e)
    flat = sel.reshape(-1)
    order_np, pos_np = mo.sort_indices(flat, e)
    w_np = rng.random((n, k)).astype(np.float32)
    y_np = _cast_np(rng.standard_normal((n * k, d)), dname)
    g_np = _cast_np(rng.standard_normal((n, d)), dname)
    yg = _t(y_np, dtype, dev).requires_grad_(True)
    wg = _t(w_np, torch.float32, dev).requires_grad_(True)
    out = mp.combine(yg, _t(order_np, torch.int32, dev), _t(pos_np, torch.int32, dev), wg)
    out.backward(_t(g_np, torch.float32, dev))
    check(out.detach(), mo.combine(y_np, pos_np, w_np), tol)
    dys, dw = mo.combine_bwd(y_np, order_np, pos_np, w_np, g_np, dname)
    check(yg.grad, dys, tol)
    check(wg.grad, dw, tol)
