"""Causal depthwise Conv1D (modal/fast_conv.py) on the GPU against the float64 oracle.

bf16 inputs, f32 accumulation, one rounding: y and dx within 1e-2 relative L2 (bf16 output rounding is ~2e-3; the
north-star bar is 2e-2), dw (f32, a sum over B*T products) within 1e-4.  Covers every tap count 1..8, sequences
shorter than the kernel and than one thread's segment, ragged lengths, and the reference config's shape (kernel 4
over 2 * 4 key heads x 128 + 8 value heads x 128 = 2048 channels, T = 4096; configs/stage1.yml:48-52).
"""
import numpy as np
import pytest
import torch

import fast_conv
from oracle import moe_oracle as mo

pytestmark = pytest.mark.gpu


def _bf(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(torch.bfloat16)


def run(B, T, C, K, dev, seed=0):
    rng = np.random.default_rng(seed)
    x = mo.round_bf16(rng.standard_normal((B, T, C)).astype(np.float32))
    w = mo.round_bf16(rng.standard_normal((K, 1, C)).astype(np.float32) * 0.5)
    dy = mo.round_bf16(rng.standard_normal((B, T, C)).astype(np.float32))
    xt = _bf(x, dev).requires_grad_(True)
    wt = _bf(w, dev).requires_grad_(True)
    y = fast_conv.causal_conv1d(xt, wt)
    y.backward(_bf(dy, dev))
    torch.cuda.synchronize()
    want = mo.causal_conv1d(x, w[:, 0])
    dx, dw = mo.causal_conv1d_bwd(x, w[:, 0], dy)
    ey = mo.rel_l2(y.detach().float().cpu().numpy(), want)
    edx = mo.rel_l2(xt.grad.float().cpu().numpy(), dx)
    assert ey < 1e-2 and edx < 1e-2, (ey, edx)
    assert mo.rel_l2(wt.grad.float().cpu().numpy()[:, 0], dw) < 1e-2  # bf16 gradient of a bf16 kernel


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 8])
def test_taps(K, dev):
    run(2, 150, 64, K, dev, seed=K)


@pytest.mark.parametrize("B,T,C,K", [(1, 1, 8, 4), (1, 3, 16, 4), (3, 64, 24, 4), (2, 65, 520, 4), (1, 200, 2056, 3)])
def test_edges(B, T, C, K, dev):
    run(B, T, C, K, dev, seed=T)


def test_dw_exact_order(dev):
    # dw in f32 against float64: a sum over B * T products
    rng = np.random.default_rng(9)
    B, T, C, K = 2, 1000, 128, 4
    x = mo.round_bf16(rng.standard_normal((B, T, C)).astype(np.float32))
    w = mo.round_bf16(rng.standard_normal((K, C)).astype(np.float32))
    dy = mo.round_bf16(rng.standard_normal((B, T, C)).astype(np.float32))
    import _lib as L
    lib = L.lib()
    xt, wt, dyt = _bf(x, dev), _bf(w, dev), _bf(dy, dev)
    dx = torch.empty_like(xt)
    dw = torch.empty((K, C), dtype=torch.float32, device=dev)
    ws = L.workspace(lib.lsurge_causal_conv1d_bwd_workspace_bytes(B, T, C, K), dev)
    L.check(lib.lsurge_causal_conv1d_bwd(L.ptr(xt), L.ptr(wt), L.ptr(dyt), B, T, C, K, L.ptr(dx), L.ptr(dw),
                                         L.ptr(ws), ws.numel(), L.stream(dev)), "causal_conv1d_bwd")
    torch.cuda.synchronize()
    _, want = mo.causal_conv1d_bwd(x, w, dy)
    assert mo.rel_l2(dw.cpu().numpy(), want) < 1e-4


def test_reference_config_shape(dev):
    run(2, 4096, 2048, 4, dev, seed=1)
