"""Committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

The expected values there come from scalar per-token loops written independently of the vectorised oracle,
so the CPU tests below pin the oracle itself (bit-exact for logits, selection and layout; float64 agreement
for the rest), and the GPU tests check the HIP path against the same vectors (bit-exact indices, values
within the 2e-2 relative-L2 bar of the north star).
"""
import os

import numpy as np
import pytest

from oracle import c_oracle as co
from oracle import moe_oracle as mo

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LAYOUT = ("group_sizes", "offsets", "block_off", "order", "pos", "slot")
TOL = 2e-2


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {n: z[n] for n in z.files}


def bf(a):
    return mo.bf16_to_f32(a)


def layer_params(fx):
    p = {n: bf(fx[n]) for n in ("x", "w_r", "w_gate", "w_up", "w_down", "dy")}
    for n in ("ws_gate", "ws_up", "ws_down"):
        p[n] = bf(fx[n]) if n in fx else None
    p["bias"] = fx.get("bias")
    p["k"] = int(fx["k"])
    return p


# ----------------------------------------------------------------------------------------- oracle (CPU)


def test_router_ties_oracle():
    fx = load("router_ties")
    x, w = bf(fx["x"]), bf(fx["w_r"])
    k = int(fx["k"])
    for lg in (mo.router_logits(x, w), co.router_logits(x, w)):
        assert np.array_equal(lg.view(np.uint32), fx["logits"])
    lg = fx["logits"].view(np.float32)
    sel = mo.topk_lower_index(lg, k)
    assert np.array_equal(sel, fx["sel"])
    assert np.array_equal(co.topk(lg, k), fx["sel"])
    assert np.allclose(mo.topk_softmax(lg, sel), fx["weights"], rtol=0, atol=1e-12)
    for lay in (mo.build_layout(sel, w.shape[1]), co.build_layout(sel, w.shape[1])):
        for n in LAYOUT:
            assert np.array_equal(lay[n], fx[n]), n
        assert lay["num_blocks"] == int(fx["num_blocks"])


def test_ragged_dot_te_oracle():
    fx = load("ragged_dot_te")
    a, b, g = bf(fx["lhs"]), bf(fx["rhs"]), bf(fx["g"])
    gs = fx["group_sizes"]
    assert mo.rel_l2(mo.ragged_dot(a, b, gs), fx["out"]) < 1e-12
    dl, dr = mo.ragged_dot_bwd(a, b, gs, g)
    assert mo.rel_l2(dl, fx["dlhs"]) < 1e-12
    assert mo.rel_l2(dr, fx["drhs"]) < 1e-12


@pytest.mark.parametrize("name", ["layer_small", "layer_zipf"])
def test_layer_oracle(name):
    fx = load(name)
    p = layer_params(fx)
    out, cache = mo.moe_layer_fwd(p, np.float64)
    assert np.array_equal(cache["sel"], fx["sel"])
    for n in LAYOUT:
        assert np.array_equal(cache["lay"][n], fx[n]), n
    assert mo.rel_l2(out, fx["out"]) < 1e-6  # fixture values are stored as float32
    g = mo.moe_layer_bwd(p, cache, p["dy"], np.float64)
    names = {"dx": "dx", "dw_r": "dw_r", "dw_gate": "dw_gate", "dw_up": "dw_up", "dw_down": "dw_down",
             "dweights": "dw"}
    if p["ws_gate"] is not None:
        names.update(dws_gate="dws_gate", dws_up="dws_up", dws_down="dws_down")
    for fn, on in names.items():
        assert mo.rel_l2(g[on], fx["want_" + fn]) < 1e-6, fn


def test_zipf_fixture_has_empty_experts():
    fx = load("layer_zipf")
    assert (fx["group_sizes"] == 0).any() and fx["group_sizes"].max() == fx["x"].shape[0]


# ----------------------------------------------------------------------------------------- HIP path (GPU)


@pytest.mark.gpu
def test_router_ties_gpu(dev):
    from test_router_layout_gpu import gpu_layout, gpu_router
    fx = load("router_ties")
    logits, sel, wts = gpu_router(bf(fx["x"]), bf(fx["w_r"]), int(fx["k"]), None, dev)
    assert np.array_equal(logits.view(np.uint32), fx["logits"])
    assert np.array_equal(sel, fx["sel"])
    assert mo.rel_l2(wts, fx["weights"]) < 1e-6
    got, _ = gpu_layout(sel, bf(fx["w_r"]).shape[1], dev)
    for n in LAYOUT:
        assert np.array_equal(got[n], fx[n]), n
    assert got["num_blocks"][0] == int(fx["num_blocks"])


@pytest.mark.gpu
def test_ragged_dot_te_gpu(dev):
    import torch

    import padded_gmm as pg
    fx = load("ragged_dot_te")
    t = lambda a: torch.from_numpy(bf(a)).to(dev).to(torch.bfloat16)  # noqa: E731
    a = t(fx["lhs"]).requires_grad_(True)
    b = t(fx["rhs"]).requires_grad_(True)
    gs = torch.from_numpy(fx["group_sizes"]).to(dev)
    out = pg.padded_ragged_dot(a, b, gs)
    out.backward(t(fx["g"]))
    S = int(fx["group_sizes"].sum())
    got = out.detach().float().cpu().numpy()
    assert np.all(got[S:] == 0)
    assert mo.rel_l2(got, fx["out"]) < 5e-3
    assert mo.rel_l2(a.grad.float().cpu().numpy(), fx["dlhs"]) < TOL
    assert mo.rel_l2(b.grad.float().cpu().numpy(), fx["drhs"]) < TOL


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["layer_small", "layer_zipf"])
def test_layer_gpu(name, dev):
    from moe_layer import MoEShape
    from test_layer_gpu import run_gpu
    fx = load(name)
    p = layer_params(fx)
    T, d = p["x"].shape
    E, _, f = p["w_gate"].shape
    fs = 0 if p["ws_gate"] is None else p["ws_gate"].shape[1]
    out, views, grads = run_gpu(p, MoEShape(T, d, E, p["k"], f, fs), dev)
    assert np.array_equal(views["sel"], fx["sel"])
    for n in LAYOUT:
        assert np.array_equal(views[n], fx[n]), n
    errs = {"out": mo.rel_l2(out, fx["out"])}
    for n in ("dx", "dw_r", "dw_gate", "dw_up", "dw_down", "dweights") + (("dws_gate", "dws_up", "dws_down")
                                                                           if fs else ()):
        errs[n] = mo.rel_l2(grads[n], fx["want_" + n])
    print({k: f"{v:.2e}" for k, v in errs.items()})
    assert all(v < TOL for v in errs.values()), errs
