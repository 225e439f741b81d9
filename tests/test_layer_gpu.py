"""Whole MoE layer (lsurge_moe_fwd / lsurge_moe_bwd) on the GPU against the oracle.

Bar (north star): routing indices / expert offsets / permutation bit-exact; outputs and gradients within 2e-2
relative L2 of the oracle (float64 on small shapes, float32 on the BASELINE shapes for speed -- either is far
more precise than the bf16 path it checks).  At C5 the oracle runs on a token subset: out[t], dx[t] and
d(weights)[t] depend on token t and the weights only.
"""
import numpy as np
import pytest
import torch

from moe_layer import MoELayer, MoEShape, moe_layer
from oracle import c_oracle as co
from oracle import moe_oracle as mo

pytestmark = pytest.mark.gpu
TOL = 2e-2


def to_dev(p, dev):
    out = {}
    for n in ("x", "w_r", "w_gate", "w_up", "w_down", "ws_gate", "ws_up", "ws_down"):
        if p.get(n) is not None:
            out[n] = torch.from_numpy(np.ascontiguousarray(p[n])).to(dev).to(torch.bfloat16)
    out["bias"] = None if p.get("bias") is None else torch.from_numpy(p["bias"]).to(dev)
    return out


def run_gpu(p, shape, dev, bwd=True):
    layer = MoELayer(shape, dev)
    tp = to_dev(p, dev)
    out = layer.forward(tp).float().cpu().numpy()
    views = {k: v.cpu().numpy() for k, v in layer.views().items()
             if k in ("sel", "group_sizes", "offsets", "block_off", "order", "pos", "slot", "num_blocks")}
    grads = None
    if bwd:
        dy = torch.from_numpy(np.ascontiguousarray(p["dy"])).to(dev).to(torch.bfloat16)
        g = layer.backward(tp, dy)
        grads = {k: v.float().cpu().numpy() for k, v in g.items()}
    return out, views, grads


def check_layer(p, shape, dev, bwd=True, odt=np.float64, fast_route=False):
    route = None
    if fast_route:
        logits, sel, _ = co.router(p["x"], p["w_r"], p["k"], p.get("bias"))
        route = (logits, sel)
    out, views, grads = run_gpu(p, shape, dev, bwd)
    want, cache = mo.moe_layer_fwd(p, odt, route=route)
    lay = cache["lay"]
    assert np.array_equal(views["sel"], cache["sel"])
    for n in ("group_sizes", "offsets", "block_off", "order", "pos", "slot"):
        assert np.array_equal(views[n], lay[n]), n
    errs = {"out": mo.rel_l2(out, want)}
    if bwd:
        g = mo.moe_layer_bwd(p, cache, p["dy"], odt)
        pairs = [("dx", "dx"), ("dw_r", "dw_r"), ("dw_gate", "dw_gate"), ("dw_up", "dw_up"), ("dw_down", "dw_down"),
                 ("dweights", "dw")]
        if shape.fs:
            pairs += [("dws_gate", "dws_gate"), ("dws_up", "dws_up"), ("dws_down", "dws_down")]
        for gn, on in pairs:
            errs[gn] = mo.rel_l2(grads[gn], g[on])
    print({k: f"{v:.2e}" for k, v in errs.items()})
    bad = {k: v for k, v in errs.items() if not v < TOL}
    assert not bad, bad
    return errs


@pytest.mark.parametrize("T,d,E,k,f,fs", [(256, 128, 8, 2, 64, 64), (300, 256, 16, 6, 128, 0),
                                          (1000, 512, 64, 6, 256, 128), (77, 64, 8, 8, 64, 64)])
def test_small_layers_fp64(T, d, E, k, f, fs, dev):
    p = mo.make_inputs(T=T, d=d, E=E, k=k, f=f, fs=fs, seed=T)
    check_layer(p, MoEShape(T, d, E, k, f, fs), dev)


@pytest.mark.parametrize("T,d,E,k,f,fs", [(600, 1024, 16, 4, 1024, 1024), (400, 2048, 16, 6, 512, 0)])
def test_gathered_dy_backward(T, d, E, k, f, fs, dev):
    """Shapes whose down weight gradient has 16+ tiles per chunk: the backward gathers dY rows and applies the
    routing weights inside the down GEMMs instead of writing the padded dY rows (with a merged shared expert, whose
    rows take weight 1, and without one)."""
    p = mo.make_inputs(T=T, d=d, E=E, k=k, f=f, fs=fs, seed=T + 3)
    check_layer(p, MoEShape(T, d, E, k, f, fs), dev)


def test_small_layer_zipf_bias(dev):
    p = mo.make_inputs(T=2048, d=256, E=32, k=4, f=128, fs=128, seed=2, zipf=True)
    check_layer(p, MoEShape(2048, 256, 32, 4, 128, 128), dev)


@pytest.mark.parametrize("E,k,T", [(32, 4, 8192), (64, 6, 8192), (64, 8, 8192), (128, 8, 8192), (128, 1, 8192),
                                   (256, 8, 8192), (256, 3, 4000)])
def test_fused_router_ties(E, k, T, dev):
    """The layer's fused router (one workgroup per 64 tokens: logits, top-k split over several lanes per token and
    merged, softmax, per-chunk histograms for the layout) on planted ties: duplicated router columns give identical
    logits on every token, and all-zero tokens tie every expert.  Logits bitwise those of the C oracle, selection the
    stable descending order (lower expert index first), weights bitwise those of the split router, layout exact."""
    from test_router_layout_gpu import gpu_router
    d, f = 256, 64
    p = mo.make_inputs(T=T, d=d, E=E, k=k, f=f, fs=0, seed=E + k)
    w_r = p["w_r"]
    w_r[:, E // 2:E // 2 + 8] = w_r[:, 0:8]  # experts E/2 .. E/2 + 7 tie with 0..7
    w_r[:, E - 1] = w_r[:, 3]
    p["x"][:5] = 0.0
    p["x"][100] = 0.0                            # a zero token inside the first workgroup and one further on
    layer = MoELayer(MoEShape(T, d, E, k, f, 0), dev)
    layer.forward(to_dev(p, dev))
    v = {n: t.cpu().numpy() for n, t in layer.views().items() if t.dtype != torch.bfloat16}
    logits = co.router_logits(p["x"], w_r)
    sel = co.topk(logits, k)
    assert np.array_equal(v["logits"], logits)
    assert np.array_equal(v["sel"], sel)
    assert np.array_equal(v["sel"][:5], np.tile(np.arange(k), (5, 1)))
    _, sel_s, wts_s = gpu_router(p["x"], w_r, k, None, dev)
    assert np.array_equal(sel_s, sel)
    assert np.array_equal(v["weights"], wts_s)
    lay = co.build_layout(sel, E)
    for n in ("group_sizes", "offsets", "block_off", "order", "pos", "slot"):
        assert np.array_equal(v[n], lay[n]), n


def test_hot_experts_chunked_wgrad(dev):
    """Every token routes to experts 0 and 1 (a large bias), so each holds 5000 rows: the routed weight gradients
    cut them into 4096 + 904-row chunks summed from partials, and the six empty experts get zero gradients."""
    T, d, E, k, f = 5000, 128, 8, 2, 64
    p = mo.make_inputs(T=T, d=d, E=E, k=k, f=f, fs=0, seed=5)
    p["bias"] = np.array([20.0, 19.0] + [0.0] * (E - 2), dtype=np.float32)
    shape = MoEShape(T, d, E, k, f, 0)
    errs = check_layer(p, shape, dev)
    _, views, grads = run_gpu(p, shape, dev)
    assert list(views["group_sizes"]) == [T, T] + [0] * (E - 2)
    for n in ("dw_gate", "dw_up", "dw_down"):
        assert not grads[n][2:].any(), n
    assert errs["dw_gate"] < TOL


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4"])
def test_baseline_configs(name, dev):
    c = mo.CONFIGS[name]
    p = mo.make_inputs(**c)
    shape = MoEShape(c["T"], c["d"], c["E"], c["k"], c["f"], c["fs"])
    check_layer(p, shape, dev, bwd=c["bwd"], odt=np.float32, fast_route=True)


def test_c5_token_subset(dev):
    c = mo.CONFIGS["C5"]
    p = mo.make_inputs(**c)
    shape = MoEShape(c["T"], c["d"], c["E"], c["k"], c["f"], c["fs"])
    out, views, grads = run_gpu(p, shape, dev, bwd=True)
    # the full layout of all 65536 tokens (524288 routed rows over 256 experts) against the C oracle's, from the
    # layer's own selection (itself checked below on a token subset, and in full on an 8192-token slice)
    lay = co.build_layout(views["sel"], c["E"])
    for n in ("group_sizes", "offsets", "block_off", "order", "pos", "slot"):
        assert np.array_equal(views[n], lay[n]), n
    assert int(views["num_blocks"][0]) == lay["num_blocks"]
    toks = np.random.default_rng(0).choice(c["T"], 192, replace=False)
    sub = dict(p)
    sub["x"], sub["dy"] = p["x"][toks], p["dy"][toks]
    logits, sel, _ = co.router(sub["x"], p["w_r"], c["k"])
    assert np.array_equal(views["sel"][toks], sel)
    want, cache = mo.moe_layer_fwd(sub, np.float32, route=(logits, sel))
    g = mo.moe_layer_bwd(sub, cache, sub["dy"], np.float32)
    errs = {"out": mo.rel_l2(out[toks], want), "dx": mo.rel_l2(grads["dx"][toks], g["dx"]),
            "dweights": mo.rel_l2(grads["dweights"][toks], g["dw"])}
    print(errs)
    assert all(v < TOL for v in errs.values()), errs
    assert all(np.isfinite(v).all() for v in grads.values())
    # weight gradients on the full run: the hottest, the coldest and six more routed experts, the shared expert of
    # its own width (fs != f: dense backward GEMMs with split-K partials on a helper stream) and the router
    gs = views["group_sizes"]
    pick = sorted({int(np.argmax(gs)), int(np.argmin(gs))} | set(np.random.default_rng(1).choice(c["E"], 6, replace=False).tolist()))
    werr = {}
    for e in pick:
        dwg, dwu, dwd = mo.expert_grads(p, views["sel"], e, p["dy"])
        werr[f"dw_gate[{e}]"] = mo.rel_l2(grads["dw_gate"][e], dwg)
        werr[f"dw_up[{e}]"] = mo.rel_l2(grads["dw_up"][e], dwu)
        werr[f"dw_down[{e}]"] = mo.rel_l2(grads["dw_down"][e], dwd)
    dsg, dsu, dsd, _ = mo.shared_grads(p, p["dy"])
    werr.update({"dws_gate": mo.rel_l2(grads["dws_gate"], dsg), "dws_up": mo.rel_l2(grads["dws_up"], dsu),
                 "dws_down": mo.rel_l2(grads["dws_down"], dsd)})
    # the router's weight gradient from the layer's own d(weights) (checked on the token subset above)
    werr["dw_r"] = mo.rel_l2(grads["dw_r"], mo.router_wgrad(p, views["sel"], grads["dweights"]))
    print(werr)
    assert all(v < TOL for v in werr.values()), werr


def test_c5_shape_slice_full(dev):
    """C5's layer shape (d = 2048, 256 experts, top-8, shared expert of width 2048) on an 8192-token slice of its input
    stream, where the fused router runs: logits bitwise equal to the C oracle's, the selection and the whole layout
    exact, the softmax weights within 1e-6, and the output and every gradient within 2e-2 of the float32 oracle."""
    c = dict(mo.CONFIGS["C5"], T=8192)
    p = mo.make_inputs(**c)
    shape = MoEShape(c["T"], c["d"], c["E"], c["k"], c["f"], c["fs"])
    layer = MoELayer(shape, dev)
    tp = to_dev(p, dev)
    out = layer.forward(tp).float().cpu().numpy()
    v = {n: t.cpu().numpy() for n, t in layer.views().items()
         if n in ("logits", "sel", "weights", "group_sizes", "offsets", "block_off", "order", "pos", "slot", "num_blocks")}
    dy = torch.from_numpy(np.ascontiguousarray(p["dy"])).to(dev).to(torch.bfloat16)
    grads = {n: t.float().cpu().numpy() for n, t in layer.backward(tp, dy).items()}
    logits = co.router_logits(p["x"], p["w_r"])
    assert np.array_equal(v["logits"].view(np.uint32), logits.view(np.uint32))
    sel = co.topk(logits, c["k"])
    assert np.array_equal(v["sel"], sel)
    assert mo.rel_l2(v["weights"], mo.topk_softmax(logits, sel)) < 1e-6
    lay = co.build_layout(sel, c["E"])
    for n in ("group_sizes", "offsets", "block_off", "order", "pos", "slot"):
        assert np.array_equal(v[n], lay[n]), n
    assert int(v["num_blocks"][0]) == lay["num_blocks"]
    want, cache = mo.moe_layer_fwd(p, np.float32, route=(logits, sel))
    g = mo.moe_layer_bwd(p, cache, p["dy"], np.float32)
    errs = {"out": mo.rel_l2(out, want)}
    for gn, on in [("dx", "dx"), ("dw_r", "dw_r"), ("dw_gate", "dw_gate"), ("dw_up", "dw_up"), ("dw_down", "dw_down"),
                   ("dweights", "dw"), ("dws_gate", "dws_gate"), ("dws_up", "dws_up"), ("dws_down", "dws_down")]:
        errs[gn] = mo.rel_l2(grads[gn], g[on])
    print({k: f"{e:.2e}" for k, e in errs.items()})
    bad = {k: e for k, e in errs.items() if not e < TOL}
    assert not bad, bad


def test_deterministic_bitwise(dev):
    """No atomics: two runs give identical bits for the output and every gradient."""
    c = mo.CONFIGS["C2"]
    p = mo.make_inputs(**c)
    shape = MoEShape(c["T"], c["d"], c["E"], c["k"], c["f"], c["fs"])
    a = run_gpu(p, shape, dev)
    b = run_gpu(p, shape, dev)
    assert np.array_equal(a[0], b[0])
    for k in a[2]:
        assert np.array_equal(a[2][k], b[2][k]), k


def test_concurrent_streams_bitwise(dev):
    """lsurge_set_concurrency(1) runs the independent chains on helper streams: same bits as the serial run."""
    import _lib as L
    c = dict(mo.CONFIGS["C2"], T=4096)
    p = mo.make_inputs(**c)
    shape = MoEShape(c["T"], c["d"], c["E"], c["k"], c["f"], c["fs"])
    lib = L.lib()
    assert lib.lsurge_get_concurrency() == 0
    a = run_gpu(p, shape, dev)
    lib.lsurge_set_concurrency(1)
    try:
        b = run_gpu(p, shape, dev)
        b2 = run_gpu(p, shape, dev)
    finally:
        lib.lsurge_set_concurrency(0)
    assert np.array_equal(a[0], b[0]) and np.array_equal(b[0], b2[0])
    for k in a[2]:
        assert np.array_equal(a[2][k], b[2][k]), k


def test_error_after_fork_keeps_stream_order(dev):
    """A launch that fails after the backward forked its helper streams (forced from the host with
    lsurge_test_fail_launch at the down dgrad, the first launch on the caller's stream after the fork, while the
    helper already holds the down weight gradient): the call returns the error, and the caller's stream still waits
    for the helpers, so once it is idle every helper is idle too.  The next call is unaffected."""
    import _lib as L
    c = mo.CONFIGS["C2"]
    p = mo.make_inputs(**c)
    shape = MoEShape(c["T"], c["d"], c["E"], c["k"], c["f"], c["fs"])
    lib = L.lib()
    names = [lib.lsurge_prof_kernel_name(i).decode() for i in range(lib.lsurge_prof_kernel_count())]
    kid = names.index("gemm_down_dgrad")
    layer = MoELayer(shape, dev)
    tp = to_dev(p, dev)
    dy = torch.from_numpy(np.ascontiguousarray(p["dy"])).to(dev).to(torch.bfloat16)
    layer.forward(tp)
    want = {k: v.clone() for k, v in layer.backward(tp, dy).items()}
    lib.lsurge_set_concurrency(1)
    try:
        layer.backward(tp, dy)  # the helper streams exist
        torch.cuda.synchronize()
        assert lib.lsurge_test_fail_launch(kid, 1) == 0
        with pytest.raises(RuntimeError, match="injected"):
            layer.backward(tp, dy)
        torch.cuda.current_stream(dev).synchronize()
        assert lib.lsurge_test_helpers_idle() == 1
        got = layer.backward(tp, dy)
        torch.cuda.synchronize()
    finally:
        lib.lsurge_test_fail_launch(-1, 0)
        lib.lsurge_set_concurrency(0)
    for k in want:
        assert torch.equal(got[k], want[k]), k


def test_autograd_function(dev):
    T, d, E, k, f, fs = 256, 128, 8, 2, 64, 64
    p = mo.make_inputs(T=T, d=d, E=E, k=k, f=f, fs=fs, seed=1)
    tp = {n: v.requires_grad_(True) if v is not None else None for n, v in to_dev(p, dev).items()}
    out = moe_layer(tp["x"], tp["w_r"], tp["w_gate"], tp["w_up"], tp["w_down"], tp["ws_gate"], tp["ws_up"],
                    tp["ws_down"], k=k)
    dy = torch.from_numpy(p["dy"]).to(dev).to(torch.bfloat16)
    out.backward(dy)
    want, cache = mo.moe_layer_fwd(p)
    g = mo.moe_layer_bwd(p, cache, p["dy"])
    assert mo.rel_l2(out.detach().float().cpu().numpy(), want) < TOL
    assert mo.rel_l2(tp["w_gate"].grad.float().cpu().numpy(), g["dw_gate"]) < TOL
    assert mo.rel_l2(tp["x"].grad.float().cpu().numpy(), g["dx"]) < TOL


def test_graph_capture_replays(dev):
    """A layer step (forward + backward, helper-stream concurrency on) captured in a HIP graph: the library's
    fork/join events join the helper streams into the capture and no memset is recorded.  Several replays, with eager
    steps and synchronisations between them, each bitwise equal to the eager result."""
    import _lib as L
    c = dict(mo.CONFIGS["C2"], T=2048)
    p = mo.make_inputs(**c)
    shape = MoEShape(c["T"], c["d"], c["E"], c["k"], c["f"], c["fs"])
    tp = to_dev(p, dev)
    dy = torch.from_numpy(p["dy"]).to(dev).to(torch.bfloat16)
    lib = L.lib()
    lib.lsurge_set_concurrency(1)
    try:
        layer = MoELayer(shape, dev)

        def step():
            layer.forward(tp)
            layer.backward(tp, dy)

        step()
        torch.cuda.synchronize()
        ref = [layer.out.clone()] + [v.clone() for v in layer.grads.values()]
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            step()
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=s):
                step()
        torch.cuda.synchronize()
        for _ in range(3):
            layer.out.zero_()
            for v in layer.grads.values():
                v.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            got = [layer.out] + list(layer.grads.values())
            assert all(torch.equal(a, b) for a, b in zip(got, ref))
            step()  # eager work between replays
            torch.cuda.synchronize()
    finally:
        lib.lsurge_set_concurrency(0)
