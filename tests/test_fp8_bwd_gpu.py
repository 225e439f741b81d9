"""FP8 backward on the GPU, through the C ABI, against the oracle.

- lsurge_fp8_cast_transpose: E4M3 and E5M2 (power-of-two scale) codes and scale_inv bit-exact against
  oracle.fp8_quantize (codecs pinned
  against torch's float8_e4m3fn / float8_e5m2 casts in tests/test_fp8_oracle.py), row-wise and transposed copies,
  ragged row counts (the transposed copy's columns past the rows up to the next multiple of 16 are zeros), ties,
  subnormals and saturation.
- lsurge_moe_bwd_fp8 after lsurge_moe_fwd_fp8: every gradient within the north-star 2e-2 relative L2 of
  oracle.moe_layer_bwd_fp8 (the same quantisation points: E5M2 dY rows and [dG | dU] per tensor, the shared expert's
  on their own; the forward's E4M3 weights, x and h with their scales), at shapes with a merged-width and an
  own-width shared expert, no shared expert, ragged T, and Zipf-skewed routing (hot and empty experts); the FP8
  gradients are a few percent from the bf16 backward's; bitwise equal with and without helper streams; BASELINE
  config C1's shape in full against the float32 oracle.
"""
import numpy as np
import pytest
import torch

import _lib as L
from moe_layer import MoELayer, MoEShape
from oracle import moe_oracle as mo

pytestmark = pytest.mark.gpu

FMT = {"e4m3": 0, "e5m2": 1}


def _bf(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(torch.bfloat16)


def gpu_cast(x, fmt, dev, rows_copy=True, transposed=True):
    R, C = x.shape
    ldq = (R + 63) // 64 * 64
    xt = _bf(x, dev)
    q = torch.full((R, C), 0xAB, dtype=torch.uint8, device=dev) if rows_copy else None
    qt = torch.full((C, ldq), 0xAB, dtype=torch.uint8, device=dev) if transposed else None
    sinv = torch.empty(1, dtype=torch.float32, device=dev)
    lib = L.lib()
    ws = L.workspace(lib.lsurge_fp8_cast_workspace_bytes(), dev)
    L.check(lib.lsurge_fp8_cast_transpose(L.ptr(xt), R, C, FMT[fmt], L.ptr(q) if q is not None else None,
                                          L.ptr(qt) if qt is not None else None, ldq, L.ptr(sinv), L.ptr(ws),
                                          ws.numel(), L.stream(dev)), "fp8_cast_transpose")
    torch.cuda.synchronize()
    return (None if q is None else q.cpu().numpy(), None if qt is None else qt.cpu().numpy(),
            float(sinv.cpu().numpy()[0]))


def _cast_inputs(R, C, fmt, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((R, C)).astype(np.float32) * 3.0
    if fmt == "e5m2":  # amax 57344 (scale 1): ties, subnormals and the largest finite values
        x[0, 0] = 57344.0
        special = [49152.0, -53248.0, 1.125, 1.375, -1.625, 2.0 ** -16, 3 * 2.0 ** -17, 2.0 ** -17, 2.0 ** -15 * 1.5,
                   0.0, -0.0, 2.0 ** -14, 5 * 2.0 ** -17, 24.0, 28.0]
    else:
        x[0, 0] = 448.0
        special = [464.0 - 16, 17.0, -17.0, 1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10, 0.0, -0.0, 2.0 ** -9]
    x.reshape(-1)[1:1 + len(special)] = special
    return mo.round_bf16(x)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("R,C", [(1024, 1024), (777, 96), (64, 16), (130, 272), (5, 32)])
def test_cast_transpose_bit_exact(fmt, R, C, dev):
    x = _cast_inputs(R, C, fmt, seed=R * 7 + C)
    q, qt, sinv = gpu_cast(x, fmt, dev)
    wq, ws = mo.fp8_quantize(x, fmt=fmt)
    assert sinv == ws[0]
    assert np.array_equal(q, wq[0]), np.argwhere(q != wq[0])[:4].tolist()
    assert np.array_equal(qt[:, :R], wq[0].T)
    r16 = (R + 15) // 16 * 16
    assert np.all(qt[:, R:r16] == 0)  # the last 16-column group is padded with zeros


def test_cast_transpose_one_copy_and_scaled_values(dev):
    rng = np.random.default_rng(4)
    x = mo.round_bf16(rng.standard_normal((200, 48)).astype(np.float32) * 1e-3)  # tiny values: a large scale
    q, _, s1 = gpu_cast(x, "e5m2", dev, transposed=False)
    _, qt, s2 = gpu_cast(x, "e5m2", dev, rows_copy=False)
    wq, ws = mo.fp8_quantize(x, fmt="e5m2")
    assert s1 == s2 == ws[0]
    assert np.array_equal(q, wq[0]) and np.array_equal(qt[:, :200], wq[0].T)
    assert mo.E5M2_MAX / 2 < np.abs(mo.e5m2_decode(q)).max() <= mo.E5M2_MAX  # power-of-two scale


LAYER_CASES = [dict(T=1024, d=256, E=16, k=4, f=128, fs=128),  # shared expert of the routed width
               dict(T=777, d=256, E=16, k=3, f=128, fs=256),   # shared expert of its own width; ragged T
               dict(T=512, d=128, E=8, k=2, f=64, fs=0),
               dict(T=2048, d=512, E=64, k=6, f=256, fs=256),
               dict(T=2048, d=256, E=32, k=4, f=128, fs=128, zipf=True)]  # hot and empty experts
GRADS = ("dx", "dw_r", "dw_gate", "dw_up", "dw_down", "dweights")
SHARED = ("dws_gate", "dws_up", "dws_down")


def _run_layer(cfg, p, dev, bf16_too=False):
    s = MoEShape(cfg["T"], cfg["d"], cfg["E"], cfg["k"], cfg["f"], cfg["fs"])
    names = ("x", "w_r", "w_gate", "w_up", "w_down") + (("ws_gate", "ws_up", "ws_down") if cfg["fs"] else ())
    tp = {n: _bf(p[n], dev) for n in names}
    tp["bias"] = torch.from_numpy(p["bias"]).to(dev) if p.get("bias") is not None else None
    dy = _bf(p["dy"], dev)
    layer = MoELayer(s, dev)
    g16 = None
    if bf16_too:
        layer.forward(tp)
        g16 = {n: t.float().cpu().numpy() for n, t in layer.backward(tp, dy).items()}
    layer.quantize_weights_fp8(tp)
    layer.forward_fp8(tp)
    g8 = {n: t.float().cpu().numpy() for n, t in layer.backward_fp8(tp, dy, grads=layer.alloc_grads()).items()}
    sel = layer.views()["sel"].cpu().numpy()
    return g8, g16, sel


@pytest.mark.parametrize("cfg", LAYER_CASES,
                         ids=lambda c: "T{T}_d{d}_E{E}_k{k}_f{f}_fs{fs}".format(**c) + ("_zipf" if c.get("zipf") else ""))
def test_layer_bwd_fp8(cfg, dev):
    p = mo.make_inputs(**cfg, seed=cfg["T"] + 1)
    g8, g16, sel = _run_layer(cfg, p, dev, bf16_too=True)
    _, cache = mo.moe_layer_fwd_fp8(p)
    assert np.array_equal(sel, cache["sel"])
    want = mo.moe_layer_bwd_fp8(p, cache, p["dy"])
    want["dweights"] = want["dw"]
    names = GRADS + (SHARED if cfg["fs"] else ())
    for n in names:
        assert np.all(np.isfinite(g8[n])), n
        err = mo.rel_l2(g8[n], want[n])
        assert err < 2e-2, (n, err)
        e16 = mo.rel_l2(g8[n], g16[n])
        assert e16 < 0.2, (n, e16)  # E5M2 gradients: a few percent from the bf16 backward


def test_layer_bwd_fp8_concurrent_bitwise(dev):
    """The backward's helper-stream schedule (shared expert on one helper, the casts and the down wgrad on the
    other) gives the bits of the serial run."""
    cfg = LAYER_CASES[1]
    p = mo.make_inputs(**cfg, seed=21)
    lib = L.lib()
    prev = lib.lsurge_get_concurrency()
    outs = []
    try:
        for conc in (0, 1, 0, 1):
            lib.lsurge_set_concurrency(conc)
            outs.append(_run_layer(cfg, p, dev)[0])
    finally:
        lib.lsurge_set_concurrency(prev)
    for o in outs[1:]:
        for n in GRADS + SHARED:
            assert np.array_equal(o[n], outs[0][n]), n


def test_layer_bwd_fp8_baseline_c1(dev):
    """BASELINE config C1's shape (T=4096, d=1024, 64 experts x 512, top-6, shared 512) in full, forward + FP8
    backward, against the float32 oracle."""
    cfg = dict(T=4096, d=1024, E=64, k=6, f=512, fs=512)
    p = mo.make_inputs(**cfg, seed=0)
    g8, _, sel = _run_layer(cfg, p, dev)
    _, cache = mo.moe_layer_fwd_fp8(p, dtype=np.float32)
    assert np.array_equal(sel, cache["sel"])
    want = mo.moe_layer_bwd_fp8(p, cache, p["dy"], dtype=np.float32)
    want["dweights"] = want["dw"]
    for n in GRADS + SHARED:
        err = mo.rel_l2(g8[n], want[n])
        assert err < 2e-2, (n, err)
