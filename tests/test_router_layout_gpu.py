"""Bit-exact routing on the GPU: router logits / top-k (ties -> lower expert index) and the padded block layout,
against the C oracle, at the BASELINE configs (C5 on a token slice: routing is token-local)."""
import numpy as np
import pytest
import torch

import _lib as L
from oracle import c_oracle as co
from oracle import moe_oracle as mo

pytestmark = pytest.mark.gpu


def _dev(a, dtype, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dtype)


def gpu_router(x_np, w_np, k, bias, dev):
    T, d = x_np.shape
    E = w_np.shape[1]
    x, w = _dev(x_np, torch.bfloat16, dev), _dev(w_np, torch.bfloat16, dev)
    b = None if bias is None else _dev(bias, torch.float32, dev)
    logits = torch.empty((T, E), dtype=torch.float32, device=dev)
    sel = torch.empty((T, k), dtype=torch.int32, device=dev)
    wts = torch.empty((T, k), dtype=torch.float32, device=dev)
    L.check(L.lib().lsurge_router_topk(L.ptr(x), L.ptr(w), L.ptr(b), T, d, E, k, L.ptr(logits), L.ptr(sel),
                                       L.ptr(wts), L.stream(dev)), "router_topk")
    return logits.cpu().numpy(), sel.cpu().numpy(), wts.cpu().numpy()


def gpu_layout(sel_np, E, dev):
    flat = _dev(sel_np.reshape(-1), torch.int32, dev)
    M = flat.numel()
    mb = int(L.lib().lsurge_max_blocks(M, E))
    i32 = lambda n: torch.full((n,), -7, dtype=torch.int32, device=dev)  # noqa: E731
    out = dict(group_sizes=i32(E), offsets=i32(E), block_off=i32(E), order=i32(M), pos=i32(M), slot=i32(M),
               row_src=i32(128 * mb), blk_expert=i32(mb), blk_rows=i32(mb), num_blocks=i32(1))
    ws = L.workspace(L.lib().lsurge_layout_workspace_bytes(M, E), dev)
    names = ("group_sizes", "offsets", "block_off", "order", "pos", "slot", "row_src", "blk_expert", "blk_rows",
             "num_blocks")
    L.check(L.lib().lsurge_build_layout(L.ptr(flat), M, E, *[L.ptr(out[n]) for n in names], L.ptr(ws), ws.numel(),
                                        L.stream(dev)), "build_layout")
    return {n: v.cpu().numpy() for n, v in out.items()}, mb


def check_layout(sel, E, dev):
    got, mb = gpu_layout(sel, E, dev)
    want = co.build_layout(sel, E)
    for n in ("group_sizes", "offsets", "block_off", "order", "pos", "slot"):
        assert np.array_equal(got[n], want[n]), n
    nb = want["num_blocks"]
    assert got["num_blocks"][0] == nb
    assert np.array_equal(got["blk_expert"][:nb], want["block_expert"])
    assert np.all(got["blk_expert"][nb:] == -1) and np.all(got["blk_rows"][nb:] == 0)
    gs = want["group_sizes"]
    rows = np.concatenate([[min(128, g - 128 * j) for j in range(-(-g // 128))] for g in gs if g]).astype(np.int32)
    assert np.array_equal(got["blk_rows"][:nb], rows)
    # row_src: inverse of slot on the used rows, -1 on padding rows of used blocks
    rs = got["row_src"][:128 * nb]
    M = sel.size
    assert np.array_equal(rs[want["slot"]], np.arange(M))
    pad = np.ones(128 * nb, bool)
    pad[want["slot"]] = False
    assert np.all(rs[pad] == -1)
    return want


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5"])
def test_router_and_layout_bit_exact(name, dev):
    c = dict(mo.CONFIGS[name])
    if name == "C5":
        c["T"] = 8192  # token slice of the full input stream: routing of a token depends on that token only
    rng = np.random.default_rng(c["seed"])
    x = mo.round_bf16(rng.standard_normal((c["T"], c["d"]), dtype=np.float32))
    w_r = mo.round_bf16(rng.standard_normal((c["d"], c["E"]), dtype=np.float32) * np.float32(0.02))
    bias = mo.zipf_bias(c["E"]) if c["zipf"] else None
    logits, sel, wts = gpu_router(x, w_r, c["k"], bias, dev)
    want_l = co.router_logits(x, w_r, bias)
    assert np.array_equal(logits.view(np.uint32), want_l.view(np.uint32))
    want_sel = co.topk(want_l, c["k"])
    assert np.array_equal(sel, want_sel)
    assert mo.rel_l2(wts, mo.topk_softmax(want_l, want_sel)) < 1e-6
    lay = check_layout(sel, c["E"], dev)
    if c["zipf"]:  # report the realised load of the Zipf stress config
        gs = lay["group_sizes"]
        print(f"\n{name} load min/mean/max {gs.min()}/{gs.mean():.0f}/{gs.max()} empty={int((gs == 0).sum())}")


@pytest.mark.parametrize("T", [512, 8192])
def test_router_ties_lower_index(T, dev):
    """Planted ties: duplicated router columns give identical logits; the lower expert index must win (both
    selection kernels: one wave per token for small T, one lane per token from 8192 tokens)."""
    rng = np.random.default_rng(5)
    d, E, k = 256, 64, 6
    x = mo.round_bf16(rng.standard_normal((T, d), dtype=np.float32))
    w_r = mo.round_bf16(rng.standard_normal((d, E), dtype=np.float32) * np.float32(0.02))
    w_r[:, 40:48] = w_r[:, 0:8]  # experts 40..47 tie with 0..7 on every token
    w_r[:, 63] = w_r[:, 5]
    x[:7] = 0.0                  # all-zero tokens: every logit is 0 -> experts 0..k-1
    logits, sel, _ = gpu_router(x, w_r, k, None, dev)
    want = co.topk(co.router_logits(x, w_r), k)
    assert np.array_equal(sel, want)
    assert np.array_equal(sel[:7], np.tile(np.arange(k), (7, 1)))


@pytest.mark.parametrize("T,d,E,k,neg_inf", [(1, 8, 8, 1, 0), (65, 100, 20, 3, 0), (130, 64, 37, 16, 0),
                                             (200, 96, 256, 8, 0), (64, 1024, 256, 16, 0), (3000, 256, 64, 6, 0),
                                             (97, 40, 16, 12, 8), (70, 33, 9, 9, 3)])
def test_router_ragged_shapes(T, d, E, k, neg_inf, dev):
    """Router on shapes off every vector width: T not a multiple of 64, d not a multiple of 8 or 32, E not a
    multiple of the expert group, k up to 16 and k = E; `neg_inf` experts carry a -inf bias, so ties at -inf
    are resolved by the lower index and their weights are 0."""
    rng = np.random.default_rng(T * 7 + E)
    x = mo.round_bf16(rng.standard_normal((T, d), dtype=np.float32))
    w_r = mo.round_bf16(rng.standard_normal((d, E), dtype=np.float32) * np.float32(0.05))
    bias = None
    if neg_inf:
        bias = np.zeros(E, np.float32)
        bias[rng.choice(E, neg_inf, replace=False)] = -np.inf
    logits, sel, wts = gpu_router(x, w_r, k, bias, dev)
    want_l = co.router_logits(x, w_r, bias)
    assert np.array_equal(logits.view(np.uint32), want_l.view(np.uint32))
    want_sel = co.topk(want_l, k)
    assert np.array_equal(sel, want_sel)
    assert mo.rel_l2(wts, mo.topk_softmax(want_l, want_sel)) < 1e-6


@pytest.mark.parametrize("T,k,E", [(1, 1, 8), (3, 2, 8), (1000, 6, 16), (4096, 8, 256), (300, 12, 16)])
def test_layout_small_and_ragged(T, k, E, dev):
    rng = np.random.default_rng(T + E)
    sel = mo.topk_lower_index(rng.standard_normal((T, E)).astype(np.float32), k)
    check_layout(sel, E, dev)


def test_layout_all_one_expert(dev):
    """Extreme imbalance: every slot on expert 3 (blocks of one expert back to back, others empty)."""
    sel = np.full((5000, 1), 3, np.int32)
    check_layout(sel, 8, dev)

