"""Chunked gated delta rule (modal/gdn_fast.py:37-113) on the GPU against the oracle with the reference's bf16
rounding points (oracle/gdn_oracle.py, itself pinned against the token-by-token recurrence).

Outputs and final states within 5e-3 relative L2 (inside the north star's 2e-2; f32 arithmetic against float64, and
a few bf16 roundings that can fall either way), and the chunk kernel's u and w tiles within 1e-3.  Covers lengths below, at and across chunk boundaries, several heads and
sequences, an initial state, and the reference config's shape (8 value heads x 128, T = 4096;
configs/stage1.yml:49-53).
"""
import numpy as np
import pytest
import torch

import _lib as L
from oracle import gdn_oracle as go
from oracle import moe_oracle as mo

pytestmark = pytest.mark.gpu
D = 128


def _inputs(B, T, H, seed, correlated=False):
    """Synthetic inputs with l2-normalised keys.  correlated: keys share one direction (k = normalize(dir + 0.5 noise)),
    so the strictly lower S = (k beta) k^T of a chunk has entries near beta instead of near 0.05 and (I + S)^-1 is far
    from I - S: a wrong blocked inverse then gives errors of order one, where i.i.d. keys hide it below 2e-2."""
    rng = np.random.default_rng(seed)
    q = mo.round_bf16(rng.standard_normal((B, T, H, D)).astype(np.float32))
    k = rng.standard_normal((B, T, H, D))
    if correlated:
        k = rng.standard_normal((1, 1, H, D)) + 0.5 * k
    k = mo.round_bf16((k / np.linalg.norm(k, axis=-1, keepdims=True)).astype(np.float32))  # l2-normalised keys
    v = mo.round_bf16(rng.standard_normal((B, T, H, D)).astype(np.float32))
    g = (-np.abs(rng.standard_normal((B, T, H))) * 0.05).astype(np.float32)
    beta = mo.round_bf16((1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H))))).astype(np.float32))
    return q, k, v, g, beta


def gpu_gdn(q, k, v, g, beta, dev, h0=None):
    B, T, H, _ = q.shape
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(torch.bfloat16)  # noqa: E731
    qt, kt, vt, bt = bf(q), bf(k), bf(v), bf(beta)
    gt = torch.from_numpy(np.ascontiguousarray(g, np.float32)).to(dev)
    h0t = None if h0 is None else torch.from_numpy(np.ascontiguousarray(h0, np.float32)).to(dev)
    o = torch.empty_like(vt)
    hout = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
    lib = L.lib()
    ws = L.workspace(lib.lsurge_gdn_chunked_workspace_bytes(B, T, H, D, D), dev)
    L.check(lib.lsurge_gdn_chunked_fwd(L.ptr(qt), L.ptr(kt), L.ptr(vt), L.ptr(gt), L.ptr(bt), B, T, H, D, D,
                                       L.ptr(h0t), L.ptr(o), L.ptr(hout), L.ptr(ws), ws.numel(), L.stream(dev)),
            "gdn_chunked_fwd")
    torch.cuda.synchronize()
    # the chunk kernel's u and w tiles, [B, H, N, 64, D] bf16 at the start of the workspace
    N = (T + 63) // 64
    uw = ws[:2 * B * H * N * 64 * D * 2].view(torch.bfloat16).float().cpu().numpy().reshape(2, B, H, N, 64, D)
    return o.float().cpu().numpy(), hout.cpu().numpy(), uw[0], uw[1]


def check_uw(u, w, wu, ww, tol):
    """GPU u / w tiles against the oracle's ([B, N, H, C, D] -> [B, H, N, C, D])."""
    eu = mo.rel_l2(u, wu.transpose(0, 2, 1, 3, 4))
    ew = mo.rel_l2(w, ww.transpose(0, 2, 1, 3, 4))
    assert eu < tol and ew < tol, (eu, ew)
    return eu, ew


# The chunk-local u and w are single bf16 roundings of f32 products: measured at most 6e-5 against the oracle (a
# rounding that falls the other way now and then), so 1e-3 leaves margin while any wrong inverse block (errors of
# order one with correlated keys) fails.  o and the state: measured 1.7e-3 / 5e-5, checked at 5e-3, inside the
# north star's 2e-2.
UW_TOL = 1e-3
OH_TOL = 5e-3


@pytest.mark.parametrize("correlated", [False, True])
@pytest.mark.parametrize("B,T,H", [(1, 1, 1), (1, 63, 2), (2, 64, 1), (2, 100, 3), (1, 333, 2)])
def test_against_oracle(B, T, H, correlated, dev):
    q, k, v, g, beta = _inputs(B, T, H, seed=T + H, correlated=correlated)
    o, h, u, w = gpu_gdn(q, k, v, g, beta, dev)
    wo, wh, wu, ww = go.gdn_chunked(q, k, v, g, beta, chunk=64, rounding="bf16", return_uw=True)
    eo, eh = mo.rel_l2(o, wo), mo.rel_l2(h, wh)
    eu, ew = check_uw(u, w, wu, ww, UW_TOL)
    print(dict(o=eo, h=eh, u=eu, w=ew))
    assert eo < OH_TOL and eh < OH_TOL, (eo, eh)


def test_initial_state(dev):
    q, k, v, g, beta = _inputs(2, 150, 2, seed=7)
    h0 = np.random.default_rng(8).standard_normal((2, 2, D, D)).astype(np.float32) * 0.1
    o, h, _, _ = gpu_gdn(q, k, v, g, beta, dev, h0=h0)
    wo, wh = go.gdn_chunked(q, k, v, g, beta, chunk=64, h0=h0, rounding="bf16")
    assert mo.rel_l2(o, wo) < 2e-2 and mo.rel_l2(h, wh) < 2e-2


@pytest.mark.parametrize("correlated", [False, True])
def test_reference_config_shape(correlated, dev):
    q, k, v, g, beta = _inputs(1, 4096, 8, seed=1, correlated=correlated)
    o, h, u, w = gpu_gdn(q, k, v, g, beta, dev)
    wo, wh, wu, ww = go.gdn_chunked(q, k, v, g, beta, chunk=64, rounding="bf16", return_uw=True)
    eo, eh = mo.rel_l2(o, wo), mo.rel_l2(h, wh)
    eu, ew = check_uw(u, w, wu, ww, UW_TOL)
    print(dict(o=eo, h=eh, u=eu, w=ew))
    assert eo < OH_TOL and eh < OH_TOL, (eo, eh)


def gpu_gdn_bwd(q, k, v, g, beta, do, dev, h0=None, dh_final=None):
    B, T, H, _ = q.shape
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(torch.bfloat16)  # noqa: E731
    f32 = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)  # noqa: E731
    qt, kt, vt, bt, dot = bf(q), bf(k), bf(v), bf(beta), bf(do)
    gt, h0t, dht = f32(g), f32(h0), f32(dh_final)
    dq, dk, dv = torch.empty_like(qt), torch.empty_like(kt), torch.empty_like(vt)
    dg = torch.empty((B, T, H), dtype=torch.float32, device=dev)
    db = torch.empty_like(dg)
    dh0 = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
    lib = L.lib()
    ws = L.workspace(lib.lsurge_gdn_chunked_bwd_workspace_bytes(B, T, H, D, D), dev)
    L.check(lib.lsurge_gdn_chunked_bwd(L.ptr(qt), L.ptr(kt), L.ptr(vt), L.ptr(gt), L.ptr(bt), B, T, H, D, D,
                                       L.ptr(h0t), L.ptr(dot), L.ptr(dht), L.ptr(dq), L.ptr(dk), L.ptr(dv), L.ptr(dg),
                                       L.ptr(db), L.ptr(dh0), L.ptr(ws), ws.numel(), L.stream(dev)), "gdn_chunked_bwd")
    torch.cuda.synchronize()
    return [a.float().cpu().numpy() for a in (dq, dk, dv, dg, db, dh0)]


NAMES = ("dq", "dk", "dv", "dg", "dbeta", "dh0")


def check_bwd(q, k, v, g, beta, dev, seed, h0=None, with_dhf=False, tol=2e-2):
    rng = np.random.default_rng(seed)
    B, T, H, _ = q.shape
    do = mo.round_bf16(rng.standard_normal((B, T, H, D)).astype(np.float32))
    dhf = (rng.standard_normal((B, H, D, D)) * 0.1).astype(np.float32) if with_dhf else None
    got = gpu_gdn_bwd(q, k, v, g, beta, do, dev, h0=h0, dh_final=dhf)
    want = go.gdn_chunked_bwd(q, k, v, g, beta, do, chunk=64, h0=h0, dh_final=dhf, rounding="bf16")
    errs = {n: mo.rel_l2(a, b) for n, a, b in zip(NAMES, got, want)}
    print(errs)
    assert all(e < tol for e in errs.values()), errs
    return errs


@pytest.mark.parametrize("correlated", [False, True])
@pytest.mark.parametrize("B,T,H", [(1, 1, 1), (1, 63, 2), (2, 64, 1), (2, 100, 3), (1, 333, 2)])
def test_backward_against_oracle(B, T, H, correlated, dev):
    """dq, dk, dv, dg, dbeta and dh0 of lsurge_gdn_chunked_bwd against the oracle's reverse-mode gradients (pinned by
    finite differences of the token recurrence), within the north star's 2e-2."""
    q, k, v, g, beta = _inputs(B, T, H, seed=3 * T + H, correlated=correlated)
    check_bwd(q, k, v, g, beta, dev, seed=T)


def test_backward_initial_and_final_state(dev):
    q, k, v, g, beta = _inputs(2, 150, 2, seed=17)
    h0 = np.random.default_rng(18).standard_normal((2, 2, D, D)).astype(np.float32) * 0.1
    check_bwd(q, k, v, g, beta, dev, seed=19, h0=h0, with_dhf=True)


@pytest.mark.parametrize("correlated", [False, True])
def test_backward_reference_config_shape(correlated, dev):
    q, k, v, g, beta = _inputs(1, 4096, 8, seed=2, correlated=correlated)
    check_bwd(q, k, v, g, beta, dev, seed=5)


def test_autograd_surface(dev):
    """gdn_fast.fast_chunk_gated_delta_rule (the reference's signature) forward and backward through torch autograd,
    with an initial state whose final state feeds the loss too."""
    import gdn_fast
    B, T, H = 2, 130, 2
    q, k, v, g, beta = _inputs(B, T, H, seed=31)
    h0 = (np.random.default_rng(32).standard_normal((B, H, D, D)) * 0.1).astype(np.float32)
    rng = np.random.default_rng(33)
    do = mo.round_bf16(rng.standard_normal((B, T, H, D)).astype(np.float32))
    dhf = (rng.standard_normal((B, H, D, D)) * 0.1).astype(np.float32)
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(torch.bfloat16)  # noqa: E731
    ts = [bf(q).requires_grad_(True), bf(k).requires_grad_(True), bf(v).requires_grad_(True),
          torch.from_numpy(g).to(dev).requires_grad_(True), bf(beta).requires_grad_(True),
          torch.from_numpy(h0).to(dev).requires_grad_(True)]
    o, hT = gdn_fast.fast_chunk_gated_delta_rule(*ts[:5], initial_state=ts[5])
    assert o.dtype == torch.bfloat16 and hT.dtype == torch.bfloat16
    (o.float() * torch.from_numpy(do).to(dev)).sum().backward(retain_graph=True)
    # the final state's gradient enters through the second output
    ts2 = [t.detach().clone().requires_grad_(True) for t in ts]
    o2, hT2 = gdn_fast.fast_chunk_gated_delta_rule(*ts2[:5], initial_state=ts2[5])
    ((o2.float() * torch.from_numpy(do).to(dev)).sum() + (hT2.float() * torch.from_numpy(dhf).to(dev)).sum()).backward()
    wo, wh = go.gdn_chunked(q, k, v, g, beta, chunk=64, h0=h0, rounding="bf16")
    assert mo.rel_l2(o.detach().float().cpu().numpy(), wo) < OH_TOL
    for tset, dh in ((ts, None), (ts2, dhf)):
        want = go.gdn_chunked_bwd(q, k, v, g, beta, do, chunk=64, h0=h0, dh_final=dh, rounding="bf16")
        for t, w, n in zip(tset, want, NAMES):
            err = mo.rel_l2(t.grad.float().cpu().numpy(), w)
            assert err < 2e-2, (n, err)
    with pytest.raises(NotImplementedError):
        gdn_fast.fast_chunk_gated_delta_rule(*ts[:5], cp_axis="context")


@pytest.mark.parametrize("B,T,H,states", [(1, 1, 1, False), (2, 100, 3, True), (1, 4096, 8, False)])
def test_saved_residuals_bitwise(B, T, H, states, dev):
    """lsurge_gdn_chunked_fwd_save + lsurge_gdn_chunked_bwd_saved (the training split: residuals kept, no recompute)
    give the bits of lsurge_gdn_chunked_fwd + lsurge_gdn_chunked_bwd; the backward leaves `saved` as it was (a second
    backward from it gives the same bits), and reads nothing of its scratch workspace before writing it (the
    workspace is filled with 0xFF, NaN as floats, first)."""
    q, k, v, g, beta = _inputs(B, T, H, seed=B * T + H, correlated=True)
    rng = np.random.default_rng(T)
    do = mo.round_bf16(rng.standard_normal((B, T, H, D)).astype(np.float32))
    h0 = (rng.standard_normal((B, H, D, D)) * 0.1).astype(np.float32) if states else None
    dhf = (rng.standard_normal((B, H, D, D)) * 0.1).astype(np.float32) if states else None
    o_ref, h_ref, _, _ = gpu_gdn(q, k, v, g, beta, dev, h0=h0)
    grads_ref = gpu_gdn_bwd(q, k, v, g, beta, do, dev, h0=h0, dh_final=dhf)

    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(torch.bfloat16)  # noqa: E731
    f32 = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)  # noqa: E731
    qt, kt, vt, bt, dot = bf(q), bf(k), bf(v), bf(beta), bf(do)
    gt, h0t, dht = f32(g), f32(h0), f32(dhf)
    lib = L.lib()
    o = torch.empty_like(vt)
    hout = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
    saved = L.workspace(lib.lsurge_gdn_chunked_saved_bytes(B, T, H, D, D), dev)
    assert 0 < saved.numel() < lib.lsurge_gdn_chunked_bwd_workspace_bytes(B, T, H, D, D)
    L.check(lib.lsurge_gdn_chunked_fwd_save(L.ptr(qt), L.ptr(kt), L.ptr(vt), L.ptr(gt), L.ptr(bt), B, T, H, D, D,
                                            L.ptr(h0t), L.ptr(o), L.ptr(hout), L.ptr(saved), saved.numel(),
                                            L.stream(dev)), "gdn_chunked_fwd_save")
    torch.cuda.synchronize()
    assert np.array_equal(o.float().cpu().numpy(), o_ref) and np.array_equal(hout.cpu().numpy(), h_ref)
    snap = saved.clone()
    ws = torch.full((lib.lsurge_gdn_chunked_bwd_saved_workspace_bytes(B, T, H, D, D),), 0xFF, dtype=torch.uint8,
                    device=dev)
    for rep in range(2):
        dq, dk, dv = torch.empty_like(qt), torch.empty_like(kt), torch.empty_like(vt)
        dg = torch.empty((B, T, H), dtype=torch.float32, device=dev)
        db = torch.empty_like(dg)
        dh0 = torch.empty((B, H, D, D), dtype=torch.float32, device=dev)
        L.check(lib.lsurge_gdn_chunked_bwd_saved(L.ptr(qt), L.ptr(kt), L.ptr(vt), L.ptr(bt), B, T, H, D, D, L.ptr(dot),
                                                 L.ptr(dht), L.ptr(dq), L.ptr(dk), L.ptr(dv), L.ptr(dg), L.ptr(db),
                                                 L.ptr(dh0), L.ptr(saved), saved.numel(), L.ptr(ws), ws.numel(),
                                                 L.stream(dev)), "gdn_chunked_bwd_saved")
        torch.cuda.synchronize()
        got = [a.float().cpu().numpy() for a in (dq, dk, dv, dg, db, dh0)]
        for n, a, b in zip(NAMES, got, grads_ref):
            assert np.array_equal(a, b), (rep, n)
        assert torch.equal(saved, snap), rep


def test_autograd_saved_vs_recompute_bitwise(dev):
    """gdn_fast with SAVE_RESIDUALS (the default: forward keeps its residuals) and without (the backward recomputes
    them) gives the same output and gradients bit for bit."""
    import gdn_fast
    B, T, H = 2, 200, 2
    q, k, v, g, beta = _inputs(B, T, H, seed=51, correlated=True)
    h0 = (np.random.default_rng(52).standard_normal((B, H, D, D)) * 0.1).astype(np.float32)
    do = torch.from_numpy(mo.round_bf16(np.random.default_rng(53).standard_normal((B, T, H, D)).astype(np.float32)))
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(torch.bfloat16)  # noqa: E731
    outs = []
    prev = gdn_fast.SAVE_RESIDUALS
    try:
        for save in (True, False):
            gdn_fast.SAVE_RESIDUALS = save
            ts = [bf(q).requires_grad_(True), bf(k).requires_grad_(True), bf(v).requires_grad_(True),
                  torch.from_numpy(g).to(dev).requires_grad_(True), bf(beta).requires_grad_(True),
                  torch.from_numpy(h0).to(dev).requires_grad_(True)]
            o, hT = gdn_fast.fast_chunk_gated_delta_rule(*ts[:5], initial_state=ts[5])
            ((o.float() * do.to(dev)).sum() + hT.float().sum()).backward()
            outs.append([o.detach().float().cpu()] + [t.grad.float().cpu() for t in ts])
    finally:
        gdn_fast.SAVE_RESIDUALS = prev
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("rows,dim", [(1, 128), (1000, 128), (77, 64), (300, 96), (33, 512), (5, 8)])
def test_l2norm_rows(rows, dim, dev):
    """lsurge_l2norm_rows / _bwd against the oracle (f64): y within bf16 rounding, r to f32 accuracy, dx within the
    bf16 rounding of its inputs and output; a zero row gives y = 0 and dx = dy / sqrt(eps)."""
    rng = np.random.default_rng(rows + dim)
    x = mo.round_bf16((rng.standard_normal((rows, dim)) * rng.uniform(0.1, 10, (rows, 1))).astype(np.float32))
    x[0] = 0.0
    dy = mo.round_bf16(rng.standard_normal((rows, dim)).astype(np.float32))
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(torch.bfloat16)  # noqa: E731
    xt, dyt = bf(x), bf(dy)
    y = torch.empty_like(xt)
    r = torch.empty(rows, dtype=torch.float32, device=dev)
    dx = torch.empty_like(xt)
    lib = L.lib()
    L.check(lib.lsurge_l2norm_rows(L.ptr(xt), rows, dim, 1e-6, L.ptr(y), L.ptr(r), L.stream(dev)), "l2norm")
    L.check(lib.lsurge_l2norm_rows_bwd(L.ptr(xt), L.ptr(dyt), L.ptr(r), rows, dim, L.ptr(dx), L.stream(dev)), "bwd")
    torch.cuda.synchronize()
    wy, wr = go.l2norm_rows(x, 1e-6)
    wdx = go.l2norm_rows_bwd(x, dy, 1e-6)
    gy, gr, gdx = y.float().cpu().numpy(), r.cpu().numpy(), dx.float().cpu().numpy()
    assert np.abs(gy - wy).max() <= 2.0 ** -8 * np.abs(wy).max() + 1e-7
    assert np.allclose(gr, wr, rtol=2e-6)
    assert not gy[0].any() and np.allclose(gdx[0], mo.round_bf16(dy[0] * wr[0]), rtol=1e-2)
    assert mo.rel_l2(gdx[1:], wdx[1:]) < 1e-2


def test_qk_norm_branch(dev):
    """use_qk_norm_in_gdn (gdn_fast.py:43-46): the forward equals the oracle on l2-normalised query and key, and the
    query / key gradients are the oracle's chunked gradients pulled back through the l2norm."""
    import gdn_fast
    B, T, H = 2, 100, 2
    rng = np.random.default_rng(41)
    q = mo.round_bf16(rng.standard_normal((B, T, H, D)).astype(np.float32))
    k = mo.round_bf16(rng.standard_normal((B, T, H, D)).astype(np.float32))  # not normalised: the branch does it
    _, _, v, g, beta = _inputs(B, T, H, seed=42)
    do = mo.round_bf16(rng.standard_normal((B, T, H, D)).astype(np.float32))
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(torch.bfloat16)  # noqa: E731
    ts = [bf(q).requires_grad_(True), bf(k).requires_grad_(True), bf(v).requires_grad_(True),
          torch.from_numpy(g).to(dev).requires_grad_(True), bf(beta).requires_grad_(True)]
    o, _ = gdn_fast.fast_chunk_gated_delta_rule(*ts, use_qk_norm_in_gdn=True)
    (o.float() * torch.from_numpy(do).to(dev)).sum().backward()
    qn = mo.round_bf16(go.l2norm_rows(q)[0].astype(np.float32))
    kn = mo.round_bf16(go.l2norm_rows(k)[0].astype(np.float32))
    wo, _ = go.gdn_chunked(qn, kn, v, g, beta, chunk=64, rounding="bf16")
    assert mo.rel_l2(o.detach().float().cpu().numpy(), wo) < OH_TOL
    want = go.gdn_chunked_bwd(qn, kn, v, g, beta, do, chunk=64, rounding="bf16")
    dq = go.l2norm_rows_bwd(q, want[0])
    dk = go.l2norm_rows_bwd(k, want[1])
    for t, w, n in zip(ts, [dq, dk] + list(want[2:5]), NAMES):
        err = mo.rel_l2(t.grad.float().cpu().numpy(), w)
        assert err < 2e-2, (n, err)
