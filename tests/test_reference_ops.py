"""The reference surfaces of moe_permute that are plain torch, not HIP kernels: ref_dispatch / ref_combine /
moe_block(use_kernels=False) (modal/moe_permute.py:335-353), every op with CFG["enabled"] = False (the reference's
A/B switch, modal/moe_permute.py:33), and the TPU helpers kept as API (_pick_tile 57-61, _interpret 49-50,
probe_packing 359-362).  They run on the CPU here and on the GPU in the `gpu` run, on the reference test's case list
(modal/test_moe_permute.py:37-92: E=16, n=64, d=256, k in {6, 12}, f32 and bf16) against the CPU oracle.
"""
import numpy as np
import pytest
import torch

import moe_permute as mp
from oracle import moe_oracle as mo

E = 16
TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16}
DEVS = ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)]


def _t(a, dtype, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dtype)


def _cast_np(a, name):
    return mo._cast(np.asarray(a, np.float32), name)


def check(got, want, tol):
    got = np.asarray(got.detach().float().cpu() if torch.is_tensor(got) else got, np.float64)
    assert got.shape == np.asarray(want).shape
    err = mo.rel_max(got, want)
    assert err <= tol, err


@pytest.fixture
def cfg_off():
    old = dict(mp.CFG)
    mp.CFG["enabled"] = False
    yield
    mp.CFG.clear()
    mp.CFG.update(old)


@pytest.mark.parametrize("devname", DEVS)
@pytest.mark.parametrize("dname,k", [("f32", 6), ("bf16", 6), ("bf16", 12), ("f32", 12)])
def test_reference_ops_and_disabled_kernels(dname, k, devname, cfg_off):
    dev = torch.device(devname)
    n, d = 64, 256
    dtype = TORCH_DT[dname]
    tol = 1e-5 if dname == "f32" else 2e-2
    rng = np.random.default_rng(100 + k + (dname == "bf16"))
    x_np = _cast_np(rng.standard_normal((n, d)), dname)
    sel = mo.topk_lower_index(rng.standard_normal((n, E)).astype(np.float32), k)
    flat = sel.reshape(-1).astype(np.int32)
    w_np = rng.standard_normal((n, k))
    w_np = (np.exp(w_np) / np.exp(w_np).sum(1, keepdims=True)).astype(np.float32)
    m = n * k
    y_np = _cast_np(rng.standard_normal((m, d)), dname)
    g_np = rng.standard_normal((n, d)).astype(np.float32)
    x, y, w, g = _t(x_np, dtype, dev), _t(y_np, dtype, dev), _t(w_np, torch.float32, dev), _t(g_np, torch.float32, dev)
    flat_t = _t(flat, torch.int64, dev)
    order_np, pos_np = mo.sort_indices(flat, E)

    # ref_dispatch / ref_combine (modal/moe_permute.py:335-345)
    assert np.array_equal(mp.ref_dispatch(x, flat_t).float().cpu().numpy(), mo.ref_dispatch(x_np, flat))
    check(mp.ref_combine(y, flat_t, w), mo.ref_combine(y_np, flat, w_np), tol)

    # CFG["enabled"] = False: every op takes its plain-torch branch
    order, pos = mp.sort_indices(flat_t, E, "count")
    assert np.array_equal(order.cpu().numpy(), order_np) and np.array_equal(pos.cpu().numpy(), pos_np)
    idx_np = (rng.permutation(m) % n).astype(np.int32)
    scale_np = rng.standard_normal(m).astype(np.float32)
    idx, scale = _t(idx_np, torch.int32, dev), _t(scale_np, torch.float32, dev)
    assert np.array_equal(mp.gather_rows(x, idx).float().cpu().numpy(), x_np[idx_np])
    check(mp.gather_rows(x, idx, scale), mo.gather_rows(x_np, idx_np, scale_np, dname), tol)
    pos2 = pos_np.reshape(n, k)
    pos_t = _t(pos2, torch.int32, dev)
    check(mp.gather_reduce(y, pos_t, None, torch.float32), mo.gather_reduce(y_np, pos2), tol)
    check(mp.gather_reduce(y, pos_t, w, torch.float32), mo.gather_reduce(y_np, pos2, w_np), tol)
    check(mp.gather_dot(y, pos_t, g), mo.gather_dot(y_np, pos2, g_np), tol)

    # moe_block with the reference path (use_kernels=False) and with the kernels' entry points disabled: forward and
    # gradients against the oracle's dispatch / combine and their VJPs (tanh expert, as the reference test)
    xs = mo.dispatch(x_np, order_np, pos_np)
    ys = _cast_np(np.tanh(xs.astype(np.float64)), dname)
    want_out = mo.combine(ys, pos_np, w_np)
    dys, dw = mo.combine_bwd(ys, order_np, pos_np, w_np, g_np, dname)
    dxs = _cast_np(dys.astype(np.float64) * (1 - np.tanh(xs.astype(np.float64)) ** 2), dname)
    dx = mo.dispatch_bwd(dxs, pos_np, n)
    for use_kernels in (False, True):
        xg = x.clone().requires_grad_(True)
        wg = w.clone().requires_grad_(True)
        out = mp.moe_block(xg, flat_t, wg, lambda r: torch.tanh(r.float()).to(r.dtype), use_kernels=use_kernels)
        (out * g).sum().backward()
        check(out, want_out, tol)
        check(xg.grad, dx, tol)
        check(wg.grad, dw, tol)

    # permute_rows and its gradient (argsort of the permutation)
    perm_np = rng.permutation(m).astype(np.int32)
    yg = y.clone().requires_grad_(True)
    gy_np = _cast_np(rng.standard_normal((m, d)), dname)
    (mp.permute_rows(yg, _t(perm_np, torch.int32, dev)).float() * _t(gy_np, torch.float32, dev)).sum().backward()
    assert np.array_equal(yg.grad.float().cpu().numpy(), mo.permute_rows_bwd(gy_np, perm_np))


def test_tpu_helpers_keep_reference_values():
    """_pick_tile is the reference's loop (modal/moe_permute.py:57-61); probe_packing returns CFG["even_low"] as the
    reference does off-TPU (361-362); _interpret is None, the reference's value on the device its kernels target
    (49-50): the HIP kernels always run natively, never interpreted."""
    assert mp.CFG["tile"] == 128
    assert mp._pick_tile(64, 384) == 64        # 128 and 256 do not divide 64
    assert mp._pick_tile(256, 1536) == 128
    assert mp._pick_tile(4096, 24576) == 128
    assert mp._pick_tile(60) is None          # the reference test's "untileable" 60 rows (test_moe_permute.py:89-91)
    assert mp._pick_tile(24) == 8
    old = mp.CFG["tile"]
    try:
        mp.CFG["tile"] = 512
        assert mp._pick_tile(1024) == 512
        mp.CFG["tile"] = None
        assert mp._pick_tile(1024) == 256
    finally:
        mp.CFG["tile"] = old
    assert mp.probe_packing() is True and mp.probe_packing(verbose=False) == mp.CFG["even_low"]
    old = mp.CFG["even_low"]
    try:
        mp.CFG["even_low"] = False
        assert mp.probe_packing() is False
    finally:
        mp.CFG["even_low"] = old
    assert mp._interpret() is None


@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_gdn_qk_norm_rejects_non_bf16(dt):
    """use_qk_norm_in_gdn with f32 / f16 query and key: the reference normalises in the input dtype before its cast
    (modal/gdn_fast.py:43-49); the bf16 l2-norm kernel cannot reproduce that, so the call raises before any device
    work instead of rounding twice."""
    import gdn_fast
    q = torch.zeros((1, 64, 1, 128), dtype=dt)
    v = torch.zeros((1, 64, 1, 128), dtype=dt)
    g = torch.zeros((1, 64, 1), dtype=torch.float32)
    beta = torch.zeros((1, 64, 1), dtype=dt)
    with pytest.raises(ValueError, match="bf16 query and key"):
        gdn_fast.fast_chunk_gated_delta_rule(q, q, v, g, beta, use_qk_norm_in_gdn=True)
