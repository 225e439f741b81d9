"""FP8 (OCP E4M3, current scaling) kernels on the GPU, through the C ABI, against the oracle.

- Quantisation: codes and scale_inv bit-exact against oracle.fp8_quantize, whose codec is pinned against torch's
  float8_e4m3fn cast (tests/test_fp8_oracle.py); ties, subnormals, an all-zero group and transposed groups.
- lsurge_ragged_dot_fp8: against the oracle's exact product of the dequantised operands.  The products of two E4M3
  values are exact, but the matrix core's FP8 dot-product accumulation does not round like f32 additions (measured
  1.4e-5 relative L2 at K = 64, where one MFMA instruction forms each output), so f32 outputs are held to 1e-4
  relative L2 and bf16 outputs to 5e-3 (one bf16 rounding); rows past the groups are exactly 0.
- lsurge_moe_fwd_fp8: routing bit-exact; output within the north-star 2e-2 relative L2 of oracle.moe_layer_fwd_fp8
  (the same quantisation points: x, each expert's weights, routed h, shared h); saved h within 1e-2.
"""
import ctypes

import numpy as np
import pytest
import torch

import _lib as L
from moe_layer import MoELayer, MoEShape
from oracle import moe_oracle as mo

pytestmark = pytest.mark.gpu


def _bf(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(torch.bfloat16)


def gpu_quantize(x, groups, transpose, dev):
    G = groups
    x = np.asarray(x, np.float32).reshape(G, -1, x.shape[-1])
    R, C = x.shape[1], x.shape[2]
    xt = _bf(x, dev)
    q = torch.empty((G, C, R) if transpose else (G, R, C), dtype=torch.uint8, device=dev)
    sinv = torch.empty(G, dtype=torch.float32, device=dev)
    lib = L.lib()
    ws = L.workspace(lib.lsurge_fp8_quantize_workspace_bytes(G, R, C), dev)
    L.check(lib.lsurge_fp8_quantize(L.ptr(xt), G, R, C, int(transpose), L.ptr(q), L.ptr(sinv), L.ptr(ws), ws.numel(),
                                    L.stream(dev)), "fp8_quantize")
    torch.cuda.synchronize()
    return q, sinv


def _quant_inputs(G, R, C, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((G, R, C)).astype(np.float32) * 3.0
    if G > 1:  # group 1: scale exactly 1 (amax 448) with round-half-even ties and subnormal codes
        x[1] = rng.standard_normal((R, C)).astype(np.float32)
        ties = np.array([448.0, 17.0, -17.0, 1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10, -5 * 2.0 ** -10, 464.0 - 16,
                         0.0, -0.0, 2.0 ** -9, 2.0 ** -12], np.float32)
        x[1].reshape(-1)[:ties.size] = ties
    if G > 2:
        x[2] = 0.0  # amax 0: scale 1, every code +-0
    if G > 3:
        x[3] *= 1e-4  # tiny magnitudes: the scale is large
    return mo.round_bf16(x)


@pytest.mark.parametrize("G,R,C,transpose", [(1, 1024, 1024, False), (4, 512, 96, False), (8, 128, 256, True),
                                             (3, 64, 64, True), (1, 2048, 512, True), (5, 80, 48, True),
                                             (2, 144, 208, True)])
def test_quantize_bit_exact(G, R, C, transpose, dev):
    x = _quant_inputs(G, R, C, seed=G * 1000 + R)
    q, sinv = gpu_quantize(x, G, transpose, dev)
    wq, ws = mo.fp8_quantize(x, groups=G, transpose=transpose)
    assert np.array_equal(sinv.cpu().numpy(), ws)
    got = q.cpu().numpy()
    bad = np.argwhere(got != wq)
    assert bad.size == 0, f"{len(bad)} codes differ, first at {bad[:4].tolist()}: got {got[tuple(bad[0])]:#x} " \
                          f"want {wq[tuple(bad[0])]:#x}"


def _ragged_fp8(gs, K, N, out_dtype, dev, seed=0):
    rng = np.random.default_rng(seed)
    E, S = len(gs), int(sum(gs))
    M = S + 3
    a = mo.round_bf16(rng.standard_normal((M, K)).astype(np.float32))
    b = mo.round_bf16(rng.standard_normal((E, K, N)).astype(np.float32) * 0.05)
    qa, sa = gpu_quantize(a, 1, False, dev)
    qb, sb = gpu_quantize(b, E, True, dev)  # [E, N, K]
    oqa, osa = mo.fp8_quantize(a)
    oqb, osb = mo.fp8_quantize(b, groups=E, transpose=True)
    assert np.array_equal(qa.cpu().numpy(), oqa) and np.array_equal(qb.cpu().numpy(), oqb)
    lib = L.lib()
    gst = torch.tensor(gs, dtype=torch.int32, device=dev)
    out = torch.full((M, N), float("nan"), dtype=out_dtype, device=dev)
    ws = L.workspace(lib.lsurge_ragged_dot_workspace_bytes(M, E), dev)
    L.check(lib.lsurge_ragged_dot_fp8(L.ptr(qa), L.ptr(sa), L.ptr(qb), L.ptr(sb), L.ptr(gst), M, K, N, E, L.ptr(out),
                                      L.dt(out), L.ptr(ws), ws.numel(), L.stream(dev)), "ragged_dot_fp8")
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    want = mo.fp8_ragged_dot(oqa[0], osa, oqb, osb, gs)
    assert np.all(got[S:] == 0)
    return mo.rel_l2(got, want)


@pytest.mark.parametrize("out_dtype,tol", [(torch.bfloat16, 5e-3), (torch.float32, 1e-4)])
def test_ragged_dot_fp8_known_answer_shape(out_dtype, tol, dev):
    gs = [5, 0, 9, 3, 7, 1, 6, 4]  # modal/te_run.py:72-79
    assert _ragged_fp8(gs, 64, 48, out_dtype, dev) < tol


@pytest.mark.parametrize("K,N", [(1024, 512), (512, 1024), (1040, 272)])
def test_ragged_dot_fp8_ragged(K, N, dev):
    rng = np.random.default_rng(K + N)
    gs = rng.integers(0, 700, size=12).tolist()
    gs[3] = 0
    gs[7] = 1
    assert _ragged_fp8(gs, K, N, torch.float32, dev, seed=K) < 1e-4


LAYER_CASES = [dict(T=1024, d=256, E=16, k=4, f=128, fs=128),  # shared expert merged into the grouped GEMMs
               dict(T=777, d=256, E=16, k=3, f=128, fs=256),   # shared expert of its own width; ragged T
               dict(T=512, d=128, E=8, k=2, f=64, fs=0),
               dict(T=2048, d=512, E=64, k=6, f=256, fs=256),
               dict(T=2048, d=256, E=32, k=4, f=128, fs=128, zipf=True)]  # hot and empty experts


@pytest.mark.parametrize("cfg", LAYER_CASES,
                         ids=lambda c: "T{T}_d{d}_E{E}_k{k}_f{f}_fs{fs}".format(**c) + ("_zipf" if c.get("zipf") else ""))
def test_layer_fwd_fp8(cfg, dev):
    p = mo.make_inputs(**cfg, seed=cfg["T"])
    s = MoEShape(cfg["T"], cfg["d"], cfg["E"], cfg["k"], cfg["f"], cfg["fs"])
    names = ("x", "w_r", "w_gate", "w_up", "w_down") + (("ws_gate", "ws_up", "ws_down") if cfg["fs"] else ())
    tp = {n: _bf(p[n], dev) for n in names}
    tp["bias"] = torch.from_numpy(p["bias"]).to(dev) if p.get("bias") is not None else None
    layer = MoELayer(s, dev)
    out16 = layer.forward(tp).float().cpu().numpy()
    layer.quantize_weights_fp8(tp)
    out = layer.forward_fp8(tp, out=torch.empty_like(layer.out)).float().cpu().numpy()
    v = {n: t.cpu().numpy() for n, t in layer.views().items() if t.dtype != torch.bfloat16}
    h_pad = layer.views()["h"].float().cpu().numpy()
    want, cache = mo.moe_layer_fwd_fp8(p)
    assert np.array_equal(v["sel"], cache["sel"])
    err = mo.rel_l2(out, want)
    assert err < 2e-2, err
    h = np.empty_like(cache["h"])
    h[v["pos"]] = h_pad[v["slot"]]  # padded rows -> sorted rows
    assert mo.rel_l2(h, cache["h"]) < 1e-2
    e16 = mo.rel_l2(out, out16)
    assert 1e-3 < e16 < 0.1, e16  # FP8 is a few percent from the bf16 layer


def test_layer_fwd_fp8_concurrent_bitwise(dev):
    """The forward's helper-stream schedule (x quantised beside the router, the shared expert beside the layout)
    gives the bits of the serial run."""
    cfg = LAYER_CASES[0]
    p = mo.make_inputs(**cfg, seed=11)
    s = MoEShape(cfg["T"], cfg["d"], cfg["E"], cfg["k"], cfg["f"], cfg["fs"])
    tp = {n: _bf(p[n], dev) for n in ("x", "w_r", "w_gate", "w_up", "w_down", "ws_gate", "ws_up", "ws_down")}
    lib = L.lib()
    prev = lib.lsurge_get_concurrency()
    outs = []
    try:
        for conc in (0, 1, 0, 1):
            lib.lsurge_set_concurrency(conc)
            layer = MoELayer(s, dev)
            # zeroed, so the buffer's alignment gaps (never written) compare equal too
            layer.wq = torch.zeros(lib.lsurge_moe_fp8_weights_bytes(ctypes.byref(s.c())), dtype=torch.uint8,
                                   device=dev)
            layer._wq_ws = L.workspace(lib.lsurge_moe_fp8_quantize_weights_workspace_bytes(ctypes.byref(s.c())), dev)
            layer.quantize_weights_fp8(tp)
            out = layer.forward_fp8(tp, out=torch.empty_like(layer.out))
            torch.cuda.synchronize()
            v = layer.views()
            outs.append((out.clone(), layer.wq.clone(), v["h"][v["slot"].long()].clone()))  # h of the valid rows
    finally:
        lib.lsurge_set_concurrency(prev)
    for o, w, h in outs[1:]:
        assert torch.equal(o, outs[0][0]) and torch.equal(w, outs[0][1]) and torch.equal(h, outs[0][2])


def test_layer_fwd_fp8_baseline_c1(dev):
    """BASELINE config C1 at full size (T=4096, d=1024, 64 experts x 512, top-6, shared 512) against the float32
    oracle (all tensors: the scales are global)."""
    cfg = dict(T=4096, d=1024, E=64, k=6, f=512, fs=512)
    p = mo.make_inputs(**cfg, seed=0)
    s = MoEShape(cfg["T"], cfg["d"], cfg["E"], cfg["k"], cfg["f"], cfg["fs"])
    tp = {n: _bf(p[n], dev) for n in ("x", "w_r", "w_gate", "w_up", "w_down", "ws_gate", "ws_up", "ws_down")}
    layer = MoELayer(s, dev)
    layer.quantize_weights_fp8(tp)
    out = layer.forward_fp8(tp).float().cpu().numpy()
    sel = layer.views()["sel"].cpu().numpy()
    want, cache = mo.moe_layer_fwd_fp8(p, dtype=np.float32)
    assert np.array_equal(sel, cache["sel"])
    err = mo.rel_l2(out, want)
    assert err < 2e-2, err


def test_layer_fp8_forward_then_bf16_backward(dev):
    cfg = LAYER_CASES[0]
    p = mo.make_inputs(**cfg, seed=5)
    s = MoEShape(cfg["T"], cfg["d"], cfg["E"], cfg["k"], cfg["f"], cfg["fs"])
    tp = {n: _bf(p[n], dev) for n in ("x", "w_r", "w_gate", "w_up", "w_down", "ws_gate", "ws_up", "ws_down")}
    dy = _bf(p["dy"], dev)
    layer = MoELayer(s, dev)
    layer.forward(tp)
    g16 = {n: t.float().cpu().numpy() for n, t in layer.backward(tp, dy).items()}
    layer.quantize_weights_fp8(tp)
    layer.forward_fp8(tp)
    g8 = {n: t.float().cpu().numpy() for n, t in layer.backward(tp, dy).items()}
    for n in ("dx", "dw_gate", "dw_up", "dw_down", "dw_r", "dws_gate", "dweights"):
        assert np.all(np.isfinite(g8[n])), n
        assert mo.rel_l2(g8[n], g16[n]) < 0.1, (n, mo.rel_l2(g8[n], g16[n]))
