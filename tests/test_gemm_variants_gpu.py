"""The two grouped-GEMM kernel families give bitwise identical results.

LSURGE_GEMM_CLASSIC (128 x 256 tiles over 128-row blocks; the 8-wave ping-pong kernel over 256-row tiles) and
LSURGE_GEMM_G256 (the persistent 256 x 256 x 64 kernel, the default) compute every output element with the same
ascending sequence of 16-deep MFMA steps, so every output of ragged_dot (modal/padded_gmm.py:45-69) and of the whole
MoE layer must match bit for bit.  The oracle tests check each family against the reference semantics; this file
checks the identity itself, on shapes that exercise what differs between the two: row, column and K tails (partial
tiles, zero stages past K), empty groups, gathered rows, both B layouts and every epilogue.
"""
import contextlib

import numpy as np
import pytest
import torch

import _lib
import padded_gmm as pg
from moe_layer import MoELayer, MoEShape
from oracle import moe_oracle as mo

pytestmark = pytest.mark.gpu


@contextlib.contextmanager
def variant(v):
    L = _lib.lib()
    old = L.lsurge_get_gemm_variant()
    _lib.check(L.lsurge_set_gemm_variant(v), "set_gemm_variant")
    try:
        yield
    finally:
        L.lsurge_set_gemm_variant(old)


def test_variant_switch_rejects_unknown():
    L = _lib.lib()
    assert L.lsurge_get_gemm_variant() == 1  # the persistent kernel is the default
    assert L.lsurge_set_gemm_variant(7) != 0
    assert L.lsurge_get_gemm_variant() == 1


def _ragged(gs, M, K, N, dt, out_dtype, dev, seed):
    rng = np.random.default_rng(seed)
    E = len(gs)
    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(dev).to(dt)
    b = torch.from_numpy(rng.standard_normal((E, K, N)).astype(np.float32)).to(dev).to(dt)
    g = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(dev).to(out_dtype or dt)
    gst = torch.tensor(gs, dtype=torch.int32, device=dev)
    res = {}
    for v in (0, 1):
        with variant(v):
            at = a.clone().requires_grad_(True)
            bt = b.clone().requires_grad_(True)
            out = pg.padded_ragged_dot(at, bt, gst, preferred_element_type=out_dtype)
            out.backward(g)
            torch.cuda.synchronize()
            res[v] = (out.detach().clone(), at.grad.clone(), bt.grad.clone())
    return res


@pytest.mark.parametrize("gs,M,K,N,dt,out_dtype", [
    ([5, 0, 9, 3, 7, 1, 6, 4], 38, 64, 48, torch.bfloat16, None),       # modal/te_run.py:72-79; one stage + a zero stage
    ([5, 0, 9, 3, 7, 1, 6, 4], 38, 64, 48, torch.bfloat16, torch.float32),
    ([300, 0, 517, 1, 255, 256, 257], 1700, 192, 200, torch.bfloat16, None),  # K of 3 stages, N tail inside a tile
    ([700, 0, 1300, 20, 5000], 7100, 512, 1024, torch.bfloat16, None),
    ([700, 0, 1300, 20, 5000], 7100, 512, 1024, torch.float16, None),
    ([1536] * 16, 24576, 1024, 512, torch.float16, torch.float32),
    ([1000, 3000, 0, 2000], 6001, 1024, 768, torch.bfloat16, torch.float32),
])
def test_ragged_dot_bitwise(gs, M, K, N, dt, out_dtype, dev):
    res = _ragged(gs, M, K, N, dt, out_dtype, dev, seed=M + K)
    for name, x0, x1 in zip(("out", "dlhs", "drhs"), res[0], res[1]):
        assert torch.equal(x0, x1), f"{name}: max |diff| {(x0.float() - x1.float()).abs().max().item()}"


def _layer(p, shape, dev):
    tp = {n: torch.from_numpy(np.ascontiguousarray(p[n])).to(dev).to(torch.bfloat16)
          for n in ("x", "w_r", "w_gate", "w_up", "w_down", "ws_gate", "ws_up", "ws_down") if p.get(n) is not None}
    tp["bias"] = None if p.get("bias") is None else torch.from_numpy(p["bias"]).to(dev)
    dy = torch.from_numpy(np.ascontiguousarray(p["dy"])).to(dev).to(torch.bfloat16)
    res = {}
    for v in (0, 1):
        with variant(v):
            layer = MoELayer(shape, dev)
            out = layer.forward(tp).clone()
            g = layer.backward(tp, dy)
            torch.cuda.synchronize()
            res[v] = {"out": out, **{k: t.clone() for k, t in g.items()}}
    return res


@pytest.mark.parametrize("T,d,E,k,f,fs,zipf", [
    (1000, 512, 64, 6, 256, 256, False),   # shared expert merged as expert E
    (1000, 512, 16, 4, 256, 512, False),   # shared expert on dense GEMMs of its own
    (777, 256, 8, 2, 128, 0, False),       # no shared expert, row tails
    (4096, 1024, 64, 6, 512, 512, False),  # C1's shape, forward and backward
    (4096, 1024, 128, 6, 512, 512, True),  # Zipf loads: empty experts, one hot expert
    (2048, 2048, 256, 8, 512, 2048, False),  # C5's d, E, k and shared width on a token slice
    (1500, 1024, 32, 4, 1024, 1024, False),  # gathered dY rows in the down GEMMs, merged shared expert
])
def test_layer_bitwise(T, d, E, k, f, fs, zipf, dev):
    p = mo.make_inputs(T=T, d=d, E=E, k=k, f=f, fs=fs, seed=T + E, zipf=zipf)
    res = _layer(p, MoEShape(T, d, E, k, f, fs), dev)
    for name in res[0]:
        x0, x1 = res[0][name], res[1][name]
        assert torch.equal(x0, x1), f"{name}: max |diff| {(x0.float() - x1.float()).abs().max().item()}"
