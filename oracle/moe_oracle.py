"""CPU oracle for the Lewi Surge MoE-layer hot path (numpy restatement).

TEST INFRASTRUCTURE ONLY.  Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this module, and only as the checker or the timed CPU baseline.  The product
path (the HIP library and the Python surface in `lewi-surge_amd/`) never calls it.

What it restates (reference paths are relative to the reference repository root):

* `modal/moe_permute.py` -- gather_rows (116-158), gather_reduce / gather_dot (161-234),
  sort_indices (240-264), dispatch / combine / permute_rows and their VJPs (270-329),
  ref_dispatch / ref_combine / moe_block (335-353).
* `modal/padded_gmm.py` -- _perm_gather and its gather-only VJP (24-42), padded_ragged_dot with
  the capacity layout (45-69); plus the dropless `jax.lax.ragged_dot` semantics it stands in for.
* The MoE layer around them, whose code is MaxText 0.2.5 (`maxtext.layers.moe.RoutedMoE`, a
  third-party package that is not in the reference tree): router logits, top-k with ties broken
  toward the lower expert index, softmax over the selected logits (`norm_topk_prob: True`,
  configs/stage1.yml:37), SwiGLU experts `silu(x Wg) * (x Wu) -> Wd` (weights `wi_0, wi_1, wo`,
  modal/stage2.py:338), one ungated shared expert (configs/stage1.yml:35), and the backward of all
  of it.  No reference test pins these at the MaxText boundary; they are pinned here by closed
  forms, brute force and finite differences (tests/test_oracle.py).

Numerics contract shared with the HIP path:

* bf16 values are held in float32 arrays whose values are exactly bf16-representable
  (round-to-nearest-even, `round_bf16`).
* Router logits are float32: logits[t, e] = (((0 + x[t,0] w[0,e]) + x[t,1] w[1,e]) + ...) summed
  sequentially over d in float32, then `+ bias[e]` in float32.  Products of two bf16 values are exact
  in float32, so fused and unfused multiply-add give the same bits; this fixed order is what makes
  the routing indices bit-exact between CPU and GPU.
* Everything that is tolerance-checked (weights, layer outputs, gradients) is computed here in
  float64 with no intermediate rounding.
"""
from __future__ import annotations

import math

import numpy as np

BLOCK = 128  # rows per padded expert block

# --------------------------------------------------------------------------------------------- bf16


def bf16_bits(a):
    """float32 -> bf16 bit pattern (uint16), round to nearest even; NaN -> canonical quiet NaN."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    r[np.isnan(a)] = np.uint16(0x7FC0)
    return r


def bf16_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(a):
    return bf16_to_f32(bf16_bits(a))


# --------------------------------------------------------------------------------------------- inputs

CONFIGS = {
    # name: T, d, E, k, f, f_s, seed, zipf, mode
    "C1": dict(T=4096, d=1024, E=64, k=6, f=512, fs=512, seed=0, zipf=False, bwd=False),
    "C2": dict(T=16384, d=1024, E=64, k=6, f=512, fs=512, seed=0, zipf=False, bwd=True),
    "C3": dict(T=16384, d=1024, E=128, k=6, f=512, fs=512, seed=1, zipf=False, bwd=True),
    "C4": dict(T=32768, d=1024, E=128, k=6, f=512, fs=512, seed=1, zipf=True, bwd=True),
    "C5": dict(T=65536, d=2048, E=256, k=8, f=512, fs=2048, seed=0, zipf=False, bwd=True),
}


def zipf_bias(E):
    """Load-imbalance router bias b_e = 1.5 * log(1 / rank_e) with rank_e = e + 1 (expert 0 hottest)."""
    return (1.5 * np.log(1.0 / np.arange(1, E + 1, dtype=np.float64))).astype(np.float32)


def make_inputs(T, d, E, k, f, fs, seed=0, zipf=False, **_):
    """Seeded synthetic layer inputs (numpy PCG64 float32 normals rounded to bf16).

    Draw order: x, w_r, w_gate, w_up, w_down, ws_gate, ws_up, ws_down, dy.
    """
    rng = np.random.default_rng(seed)

    def nrm(shape, std):
        return round_bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))

    p = dict(
        x=nrm((T, d), 1.0),
        w_r=nrm((d, E), 0.02),
        w_gate=nrm((E, d, f), 0.02),
        w_up=nrm((E, d, f), 0.02),
        w_down=nrm((E, f, d), 0.02),
        ws_gate=nrm((d, fs), 0.02) if fs else None,
        ws_up=nrm((d, fs), 0.02) if fs else None,
        ws_down=nrm((fs, d), 0.02) if fs else None,
    )
    p["dy"] = nrm((T, d), 1.0)
    p["bias"] = zipf_bias(E) if zipf else None
    p["k"] = k
    return p


# --------------------------------------------------------------------------------------------- router (A1)


def router_logits(x, w_r, bias=None):
    """float32 logits, summed sequentially over d (see the numerics contract in the module docstring)."""
    x = np.asarray(x, np.float32)
    w_r = np.asarray(w_r, np.float32)
    T, d = x.shape
    acc = np.zeros((T, w_r.shape[1]), np.float32)
    for i in range(d):
        acc += x[:, i:i + 1] * w_r[i][None, :]  # float32 product (exact for bf16 inputs) + float32 add
    if bias is not None:
        acc += np.asarray(bias, np.float32)[None, :]
    return acc


def topk_lower_index(logits, k):
    """Indices of the k largest logits per row, descending; equal logits -> lower expert index first.

    Same as `argsort(-logits)[:, :k]` with a stable sort (modal/test_moe_permute.py:23-26 routes this way).
    """
    return np.argsort(-np.asarray(logits), axis=1, kind="stable")[:, :k].astype(np.int32)


def topk_softmax(logits, sel):
    """Routing weights: softmax over the selected logits (norm_topk_prob=True), float64."""
    l = np.take_along_axis(np.asarray(logits, np.float64), sel.astype(np.int64), axis=1)
    z = np.exp(l - l.max(axis=1, keepdims=True))
    return z / z.sum(axis=1, keepdims=True)


def router(x, w_r, k, bias=None):
    logits = router_logits(x, w_r, bias)
    sel = topk_lower_index(logits, k)
    return logits, sel, topk_softmax(logits, sel)


# --------------------------------------------------------------------------------------------- layout (A2, A3)


def sort_indices(flat_experts, num_experts=None):
    """(order, pos): order = stable argsort of the flat slot experts, pos = its inverse.

    modal/moe_permute.py:240-264 (both the argsort and the counting method give this).
    """
    flat = np.asarray(flat_experts, np.int64).reshape(-1)
    order = np.argsort(flat, kind="stable").astype(np.int32)
    pos = np.empty_like(order)
    pos[order] = np.arange(flat.shape[0], dtype=np.int32)
    return order, pos


def build_layout(sel, E, block=BLOCK):
    """Routing layout for the padded per-expert block format.

    Returns dict with group_sizes [E], offsets [E] (exclusive scan), block_off [E] (exclusive scan of
    ceil(gs/block)), num_blocks, order [M], pos [M], slot [M] (padded row of flat slot i) and
    block_expert [num_blocks].
    """
    flat = np.asarray(sel, np.int64).reshape(-1)
    order, pos = sort_indices(flat, E)
    gs = np.bincount(flat, minlength=E).astype(np.int32)
    offsets = (np.cumsum(gs) - gs).astype(np.int32)
    nblk = (gs + block - 1) // block
    block_off = (np.cumsum(nblk) - nblk).astype(np.int32)
    slot = (block * block_off[flat] + (pos - offsets[flat])).astype(np.int32)
    block_expert = np.repeat(np.arange(E, dtype=np.int32), nblk)
    return dict(group_sizes=gs, offsets=offsets, block_off=block_off, num_blocks=int(nblk.sum()),
                order=order, pos=pos, slot=slot, block_expert=block_expert)


def max_blocks(M, E, block=BLOCK):
    """Static upper bound on the number of padded blocks: sum_e ceil(gs_e/block) <= ceil(M/block) + E."""
    return (M + block - 1) // block + E


# --------------------------------------------------------------------------------------------- row movement (A7-A12)


def gather_rows(x, idx, scale=None, dtype="bf16"):
    """out[i] = x[idx[i]] (* scale[i], then rounded to x's dtype).  modal/moe_permute.py:116-121."""
    out = np.asarray(x)[np.asarray(idx, np.int64)]
    if scale is None:
        return out
    v = out.astype(np.float32) * np.asarray(scale, np.float32)[:, None]
    return _cast(v, dtype)


def gather_reduce(y, pos, w=None):
    """out[t] = sum_j w[t,j] * y[pos[t,j]] (float64 here).  modal/moe_permute.py:214-225."""
    rows = np.asarray(y, np.float64)[np.asarray(pos, np.int64)]  # [N, k, D]
    if w is not None:
        rows = rows * np.asarray(w, np.float64)[:, :, None]
    return rows.sum(axis=1)


def gather_dot(y, pos, g):
    """out[t,j] = <g[t], y[pos[t,j]]> (float64 here).  modal/moe_permute.py:228-234."""
    rows = np.asarray(y, np.float64)[np.asarray(pos, np.int64)]
    return np.einsum("nkd,nd->nk", rows, np.asarray(g, np.float64))


def dispatch(x, order, pos):
    """x[order // k]: tokens to rows grouped by expert.  modal/moe_permute.py:270-275."""
    k = order.shape[0] // x.shape[0]
    return np.asarray(x)[np.asarray(order, np.int64) // k]


def dispatch_bwd(g, pos, n):
    """dx[t] = sum_j g[pos[t,j]].  modal/moe_permute.py:282-286."""
    k = pos.shape[0] // n
    return gather_reduce(g, np.asarray(pos).reshape(n, k))


def combine(y, pos, w):
    """sum_j w[t,j] y[pos[t,j]] in float.  modal/moe_permute.py:292-296."""
    n, k = w.shape
    return gather_reduce(y, np.asarray(pos).reshape(n, k), w)


def combine_bwd(y, order, pos, w, g, dtype="bf16"):
    """(dy, dw): dy[p] = w_sorted[p] * g[order[p]//k] rounded to y's dtype; dw = gather_dot(y, pos, g).

    modal/moe_permute.py:303-309.
    """
    n, k = w.shape
    w_sorted = np.asarray(w, np.float32).reshape(-1)[np.asarray(order, np.int64)]
    dy = gather_rows(_cast(np.asarray(g, np.float32), dtype), np.asarray(order) // k, w_sorted, dtype)
    dw = gather_dot(y, np.asarray(pos).reshape(n, k), g)
    return dy, dw


def permute_rows(x, idx):
    """x[idx]; its VJP is gather_rows(g, argsort(idx)).  modal/moe_permute.py:315-326."""
    return np.asarray(x)[np.asarray(idx, np.int64)]


def permute_rows_bwd(g, idx):
    inv = np.argsort(np.asarray(idx), kind="stable")
    return np.asarray(g)[inv]


def invert_permutation(idx):
    """inv[idx[i]] = i, the argsort of a permutation (modal/moe_permute.py:325-326 takes argsort(idx)).  For an idx that
    is not a permutation this states the guarded kernel's contract: entries outside [0, m) are skipped and entries of
    inv that no index hits hold m (a gather through inv then gives zero rows).  Duplicated in-range entries keep an
    unspecified writer, so callers that test them must not have any."""
    idx = np.asarray(idx, np.int64)
    m = idx.shape[0]
    inv = np.full(m, m, np.int32)
    ok = (idx >= 0) & (idx < m)
    inv[idx[ok]] = np.nonzero(ok)[0].astype(np.int32)
    return inv


def ref_dispatch(x, flat_experts):
    """modal/moe_permute.py:335-338."""
    k = flat_experts.shape[0] // x.shape[0]
    order = np.argsort(flat_experts, kind="stable")
    return np.asarray(x)[order // k]


def ref_combine(y, flat_experts, w):
    """modal/moe_permute.py:341-345 (float64 here)."""
    n, k = w.shape
    pos = np.argsort(np.argsort(flat_experts, kind="stable"), kind="stable")
    rows = np.asarray(y, np.float64)[pos].reshape(n, k, -1)
    return np.einsum("nkd,nk->nd", rows, np.asarray(w, np.float64))


def _cast(v, dtype):
    if dtype == "bf16":
        return round_bf16(v)
    if dtype == "f16":
        return np.asarray(v, np.float32).astype(np.float16).astype(np.float32)
    return np.asarray(v, np.float32)


# --------------------------------------------------------------------------------------------- grouped GEMM (A4, A5)


def ragged_dot(lhs, rhs, group_sizes):
    """Dropless `jax.lax.ragged_dot`: out[r] = lhs[r] @ rhs[e(r)] for r < sum(gs), else 0 (float64)."""
    lhs = np.asarray(lhs, np.float64)
    rhs = np.asarray(rhs, np.float64)
    gs = np.asarray(group_sizes, np.int64)
    out = np.zeros((lhs.shape[0], rhs.shape[2]), np.float64)
    start = 0
    for e, g in enumerate(gs):
        out[start:start + g] = lhs[start:start + g] @ rhs[e]
        start += g
    return out


def padded_capacity(m, e, factor):
    """C = max(8, roundup8(ceil(m / e * factor))).  modal/padded_gmm.py:51-52."""
    c = int(math.ceil(m / e * factor))
    return max(8, (c + 7) // 8 * 8)


def padded_maps(group_sizes, m, factor):
    """(slot, src, C) of padded_gmm's capacity layout.  modal/padded_gmm.py:53-64."""
    gs = np.asarray(group_sizes, np.int64)
    e = gs.shape[0]
    c = padded_capacity(m, e, factor)
    starts = np.cumsum(gs) - gs
    rows = np.arange(m)
    expert = np.minimum(np.searchsorted(np.cumsum(gs), rows, side="right"), e - 1)
    p = rows - starts[expert]
    valid = (rows < gs.sum()) & (p < c)
    slot = np.where(valid, expert * c + p, e * c)
    se = np.arange(e * c) // c
    sc = np.arange(e * c) % c
    src = np.where(sc < np.minimum(gs[se], c), starts[se] + sc, m)
    return slot.astype(np.int32), src.astype(np.int32), c


def padded_ragged_dot_capacity(lhs, rhs, group_sizes, factor):
    """padded_gmm's capacity semantics (rows past C in an expert give 0).  modal/padded_gmm.py:45-69."""
    lhs = np.asarray(lhs, np.float64)
    m, k = lhs.shape
    e, _, n = rhs.shape
    slot, src, c = padded_maps(group_sizes, m, factor)
    lhs_ext = np.concatenate([lhs, np.zeros((1, k))])
    buf = lhs_ext[src].reshape(e, c, k)
    out = np.einsum("eck,ekn->ecn", buf, np.asarray(rhs, np.float64)).reshape(e * c, n)
    out_ext = np.concatenate([out, np.zeros((1, n))])
    return out_ext[slot]


def ragged_dot_bwd(lhs, rhs, group_sizes, g):
    """(dlhs, drhs) of the dropless ragged_dot for upstream g [M, N] (rows past sum(gs) get 0)."""
    lhs = np.asarray(lhs, np.float64)
    rhs = np.asarray(rhs, np.float64)
    g = np.asarray(g, np.float64)
    gs = np.asarray(group_sizes, np.int64)
    dl = np.zeros_like(lhs)
    dr = np.zeros_like(rhs)
    start = 0
    for e, n in enumerate(gs):
        dl[start:start + n] = g[start:start + n] @ rhs[e].T
        dr[e] = lhs[start:start + n].T @ g[start:start + n]
        start += n
    return dl, dr


# --------------------------------------------------------------------------------------------- SwiGLU layer (A6, A13-A16)


def silu(z):
    return z / (1.0 + np.exp(-z))


def dsilu(z):
    s = 1.0 / (1.0 + np.exp(-z))
    return s * (1.0 + z * (1.0 - s))


def swiglu(x, wg, wu, wd):
    g = x @ wg
    u = x @ wu
    h = silu(g) * u
    return h @ wd, (g, u, h)


def swiglu_bwd(x, wg, wu, wd, cache, dy):
    g, u, h = cache
    dh = dy @ wd.T
    dg = dh * u * dsilu(g)
    du = dh * silu(g)
    dx = dg @ wg.T + du @ wu.T
    return dx, x.T @ dg, x.T @ du, h.T @ dy


def moe_layer_fwd(p, dtype=np.float64, route=None):
    """Full MoE layer forward.  Returns (out [T,d], cache).  Routing is integer (bit-exact contract).

    route: optional precomputed (logits, sel) of the same contract (e.g. from the C restatement, for speed).
    """
    x = np.asarray(p["x"], dtype)
    k = p["k"]
    # selection: the bit-exact f32 contract logits; weights: softmax of the same logits computed in `dtype`
    # (the differentiable quantity; it differs from the f32 logits only by f32 rounding)
    if route is None:
        logits, sel, _ = router(p["x"], p["w_r"], k, p.get("bias"))
    else:
        logits, sel = route
    lw = x @ np.asarray(p["w_r"], dtype)
    if p.get("bias") is not None:
        lw = lw + np.asarray(p["bias"], dtype)
    w = topk_softmax(lw, sel)
    E = p["w_gate"].shape[0]
    lay = build_layout(sel, E)
    T, d = x.shape
    flat = sel.reshape(-1)
    order = lay["order"]
    xs = x[order // k]  # dispatched rows, grouped by expert
    gs = lay["group_sizes"]
    wg, wu, wd = (np.asarray(p[n], dtype) for n in ("w_gate", "w_up", "w_down"))
    f = wg.shape[2]
    ys = np.zeros((xs.shape[0], d), dtype)
    gg = np.zeros((xs.shape[0], f), dtype)
    uu = np.zeros_like(gg)
    hh = np.zeros_like(gg)
    start = 0
    for e in range(E):
        n = int(gs[e])
        if n:
            ys[start:start + n], (gg[start:start + n], uu[start:start + n], hh[start:start + n]) = swiglu(
                xs[start:start + n], wg[e], wu[e], wd[e])
        start += n
    w = w.astype(dtype)
    routed = (ys[lay["pos"]].reshape(T, k, d) * w[:, :, None]).sum(axis=1)
    out = routed
    shared = None
    if p.get("ws_gate") is not None:
        ysh, shared = swiglu(x, *(np.asarray(p[n], dtype) for n in ("ws_gate", "ws_up", "ws_down")))
        out = out + ysh
    cache = dict(logits=logits, sel=sel, w=w, lay=lay, xs=xs, ys=ys, g=gg, u=uu, h=hh, shared=shared, flat=flat)
    return out, cache


def moe_layer_bwd(p, cache, dy, dtype=np.float64):
    """Backward of `moe_layer_fwd` for upstream dy [T,d].

    Returns dict dx, dw_r, dw_gate, dw_up, dw_down, dws_gate, dws_up, dws_down, dw (routing weights
    gradient [T,k]) and dlogits [T,E].
    """
    x = np.asarray(p["x"], dtype)
    dy = np.asarray(dy, dtype)
    T, d = x.shape
    k = p["k"]
    lay, w, sel = cache["lay"], cache["w"], cache["sel"]
    order, pos, gs = lay["order"], lay["pos"], lay["group_sizes"]
    E = p["w_gate"].shape[0]
    wg, wu, wd = (np.asarray(p[n], dtype) for n in ("w_gate", "w_up", "w_down"))
    # combine backward: dy_sorted[p] = w_flat[order[p]] * dy[order[p] // k]; dw[t,j] = <dy[t], y[pos[t,j]]>
    w_flat = w.reshape(-1)
    dys = dy[order // k] * w_flat[order][:, None]
    dw = np.einsum("tkd,td->tk", cache["ys"][pos].reshape(T, k, d), dy)
    dxs = np.zeros_like(cache["xs"])
    dwg = np.zeros_like(wg)
    dwu = np.zeros_like(wu)
    dwd = np.zeros_like(wd)
    start = 0
    for e in range(E):
        n = int(gs[e])
        if n:
            sl = slice(start, start + n)
            dxs[sl], dwg[e], dwu[e], dwd[e] = swiglu_bwd(
                cache["xs"][sl], wg[e], wu[e], wd[e], (cache["g"][sl], cache["u"][sl], cache["h"][sl]), dys[sl])
        start += n
    # dispatch backward (gather-only): dx[t] = sum_j dxs[pos[t,j]]
    dx = dxs[pos].reshape(T, k, d).sum(axis=1)
    # router backward: softmax over the selected logits
    dl_sel = w * (dw - (w * dw).sum(axis=1, keepdims=True))
    dlogits = np.zeros((T, E), dtype)
    np.put_along_axis(dlogits, sel.astype(np.int64), dl_sel, axis=1)
    w_r = np.asarray(p["w_r"], dtype)
    dx = dx + dlogits @ w_r.T
    out = dict(dx=dx, dw_r=x.T @ dlogits, dw_gate=dwg, dw_up=dwu, dw_down=dwd, dw=dw, dlogits=dlogits)
    if cache["shared"] is not None:
        ws = [np.asarray(p[n], dtype) for n in ("ws_gate", "ws_up", "ws_down")]
        dxs_, out["dws_gate"], out["dws_up"], out["dws_down"] = swiglu_bwd(x, *ws, cache["shared"], dy)
        out["dx"] = out["dx"] + dxs_
    return out


def expert_grads(p, sel, e, dy, dtype=np.float32):
    """(dw_gate[e], dw_up[e], dw_down[e]) of one routed expert, the per-expert slice of `moe_layer_bwd` computed
    from that expert's tokens only (ascending t, as the stable sort orders them): their routing weights are the
    softmax over the selected logits recomputed in `dtype`, dY rows = w[t,j] dy[t].  For configurations too large
    for the whole-layer oracle."""
    x = np.asarray(p["x"], dtype)
    sel = np.asarray(sel)
    toks, js = np.nonzero(sel == e)
    if toks.size == 0:
        d, f = p["w_gate"].shape[1:]
        return np.zeros((d, f), dtype), np.zeros((d, f), dtype), np.zeros((f, d), dtype)
    xs = x[toks]
    lw = xs @ np.asarray(p["w_r"], dtype)
    if p.get("bias") is not None:
        lw = lw + np.asarray(p["bias"], dtype)
    w = topk_softmax(lw, sel[toks])[np.arange(toks.size), js]
    wg, wu, wd = (np.asarray(p[n][e], dtype) for n in ("w_gate", "w_up", "w_down"))
    _, cache = swiglu(xs, wg, wu, wd)
    dys = np.asarray(dy, dtype)[toks] * w[:, None]
    _, dwg, dwu, dwd = swiglu_bwd(xs, wg, wu, wd, cache, dys)
    return dwg, dwu, dwd


def shared_grads(p, dy, dtype=np.float32):
    """(dws_gate, dws_up, dws_down, dx_shared) of the shared expert over all tokens (its part of `moe_layer_bwd`)."""
    x = np.asarray(p["x"], dtype)
    ws = [np.asarray(p[n], dtype) for n in ("ws_gate", "ws_up", "ws_down")]
    _, cache = swiglu(x, *ws)
    dxs, dwg, dwu, dwd = swiglu_bwd(x, *ws, cache, np.asarray(dy, dtype))
    return dwg, dwu, dwd, dxs


def router_wgrad(p, sel, dweights, dtype=np.float32):
    """dW_r = x^T dlogits, dlogits = the softmax-over-selected Jacobian applied to the routing weights' gradient
    (the router part of `moe_layer_bwd`), for a given d(weights) [T, k]."""
    x = np.asarray(p["x"], dtype)
    lw = x @ np.asarray(p["w_r"], dtype)
    if p.get("bias") is not None:
        lw = lw + np.asarray(p["bias"], dtype)
    w = topk_softmax(lw, sel).astype(dtype)
    dw = np.asarray(dweights, dtype)
    dl_sel = w * (dw - (w * dw).sum(axis=1, keepdims=True))
    dlogits = np.zeros((x.shape[0], p["w_r"].shape[1]), dtype)
    np.put_along_axis(dlogits, np.asarray(sel, np.int64), dl_sel, axis=1)
    return x.T @ dlogits


# --------------------------------------------------------------------------------------------- FP8 variant
#
# FP8 forward GEMMs with current (per-tensor, just-in-time) scaling, the scheme of Transformer Engine's
# Float8CurrentScaling recipe that the reference tries through MaxText's `quantization=te_fp8_currentscaling`
# (modal/te_run.py:99; TE and MaxText are third-party and not in the reference tree, so the recipe is restated
# here from its published definition, and no reference test pins it):
#   amax = max|x| over the tensor (of the bf16 values), scale = 448 / amax in float32 (1 when amax is 0, the
#   largest float32 when the quotient overflows), q = e4m3(float32(x * scale)), scale_inv = 1 / scale (float32)
#   multiplies the GEMM's f32 accumulator back.
# e4m3 is the OCP FP8 E4M3 format ("fn": bias 7, 3 mantissa bits, no infinities, 0x7F / 0xFF NaN, largest 448),
# rounded to nearest even and saturated at +-448.  Weights take one scale per expert and matrix; activations one
# per tensor.  The backward casts gradients to OCP E5M2 (bias 15, 2 mantissa bits, 0x7C infinity, largest 57344),
# the same way with 57344 in place of 448 and the scale rounded down to a power of two (the recipe's hybrid format:
# E4M3 forward, E5M2 backward; TE's power-of-two scale option).

E4M3_MAX = 448.0
E5M2_MAX = 57344.0


def _e4m3_table():
    c = np.arange(128)
    ex, mt = c >> 3, c & 7
    v = np.where(ex == 0, mt * 2.0 ** -9, (1.0 + mt / 8.0) * np.exp2(ex - 7.0))
    v[127] = np.nan
    return v


E4M3_VALUES = _e4m3_table()  # value of codes 0x00..0x7F (sign clear), ascending up to 0x7E


def e4m3_decode(q):
    """E4M3 bit patterns (uint8) -> float64 values."""
    q = np.asarray(q, np.uint8)
    mag = E4M3_VALUES[q & 0x7F]
    return np.where(q & 0x80, -mag, mag)


def e4m3_bits(a):
    """float32 -> E4M3 bit pattern (uint8): round to nearest even, saturate at +-448, sign kept (-0 -> 0x80)."""
    a = np.asarray(a, np.float32)
    m = np.minimum(np.abs(a).astype(np.float64), E4M3_MAX)
    _, ex = np.frexp(m)  # m in [2^(ex-1), 2^ex)
    quantum = np.ldexp(1.0, np.maximum(ex - 4, -9))  # 3 mantissa bits; subnormal spacing 2^-9
    r = np.rint(m / quantum) * quantum  # exact: power-of-two division, ties to even
    code = np.searchsorted(E4M3_VALUES[:127], r).astype(np.uint8)
    return code | np.where(np.signbit(a), np.uint8(0x80), np.uint8(0))


def _e5m2_table():
    c = np.arange(128)
    ex, mt = c >> 2, c & 3
    v = np.where(ex == 0, mt * 2.0 ** -16, (1.0 + mt / 4.0) * np.exp2(ex - 15.0))
    v[124] = np.inf
    v[125:] = np.nan
    return v


E5M2_VALUES = _e5m2_table()  # value of codes 0x00..0x7F (sign clear), ascending up to 0x7C (infinity)


def e5m2_decode(q):
    """E5M2 bit patterns (uint8) -> float64 values."""
    q = np.asarray(q, np.uint8)
    mag = E5M2_VALUES[q & 0x7F]
    return np.where(q & 0x80, -mag, mag)


def e5m2_bits(a):
    """float32 -> E5M2 bit pattern (uint8): round to nearest even, saturate at +-57344, sign kept (-0 -> 0x80)."""
    a = np.asarray(a, np.float32)
    m = np.minimum(np.abs(a).astype(np.float64), E5M2_MAX)
    _, ex = np.frexp(m)  # m in [2^(ex-1), 2^ex)
    quantum = np.ldexp(1.0, np.maximum(ex - 3, -16))  # 2 mantissa bits; subnormal spacing 2^-16
    r = np.rint(m / quantum) * quantum  # exact: power-of-two division, ties to even
    code = np.searchsorted(E5M2_VALUES[:124], r).astype(np.uint8)
    return code | np.where(np.signbit(a), np.uint8(0x80), np.uint8(0))


FP8_FORMATS = {"e4m3": (E4M3_MAX, e4m3_bits, e4m3_decode), "e5m2": (E5M2_MAX, e5m2_bits, e5m2_decode)}


def fp8_scale(amax, fmt="e4m3"):
    """(scale, scale_inv) of current scaling for a float32 amax; E5M2 (gradient) scales are rounded down to a power of
    two (Transformer Engine's power-of-two option: a one-ulp change of a gradient's amax then moves the grid only
    when it crosses a binade)."""
    amax = np.float32(amax)
    if not amax > 0:
        return np.float32(1.0), np.float32(1.0)
    with np.errstate(over="ignore"):
        scale = np.float32(FP8_FORMATS[fmt][0]) / amax
    if not np.isfinite(scale):
        scale = np.float32(np.finfo(np.float32).max)
    if fmt == "e5m2":
        scale = np.float32(np.ldexp(1.0, int(np.frexp(scale)[1]) - 1))
    return scale, np.float32(1.0) / scale


def fp8_quantize(x, groups=1, transpose=False, fmt="e4m3"):
    """Current-scaling quantisation of `groups` equal [R, C] groups of bf16 values to fmt ("e4m3" / "e5m2").

    Returns (q uint8 [groups, R, C], or [groups, C, R] with transpose; scale_inv float32 [groups]).
    """
    x = np.asarray(x, np.float32)
    x = x.reshape(groups, -1, x.shape[-1])
    q = np.empty(x.shape, np.uint8)
    sinv = np.empty(groups, np.float32)
    enc = FP8_FORMATS[fmt][1]
    for g in range(groups):
        scale, sinv[g] = fp8_scale(np.abs(x[g]).max() if x[g].size else 0.0, fmt)
        q[g] = enc(x[g] * scale)
    if transpose:
        q = np.ascontiguousarray(q.transpose(0, 2, 1))
    return q, sinv


def fp8_dequant(q, sinv, fmt="e4m3"):
    """[G, ...] codes times their group's scale_inv, float64."""
    q = np.asarray(q)
    s = np.asarray(sinv, np.float64).reshape((-1,) + (1,) * (q.ndim - 1))
    return FP8_FORMATS[fmt][2](q) * s


def fp8_ragged_dot(lhs_q, lhs_sinv, rhs_q, rhs_sinv, group_sizes):
    """ragged_dot of dequantised FP8 operands: lhs [m, K] (one scale), rhs [e, n, K] (K contiguous, one scale per
    group), exact in float64; rows past sum(group_sizes) are 0."""
    lhs = e4m3_decode(lhs_q) * float(np.asarray(lhs_sinv).reshape(-1)[0])
    rhs = np.transpose(fp8_dequant(rhs_q, rhs_sinv), (0, 2, 1))
    return ragged_dot(lhs, rhs, group_sizes)


def moe_layer_fwd_fp8(p, route=None, dtype=np.float64):
    """`moe_layer_fwd` with every expert GEMM on FP8 operands (current scaling).

    x, each expert's W_gate / W_up / W_down and the shared weights are quantised as above; h = silu(g) * u is
    rounded to bf16 (the saved activation) and quantised over all routed rows (the shared expert's h on its own)
    before the down projection.  Routing, combine and shared-expert sum are those of `moe_layer_fwd`, in float64.
    Returns (out [T, d], cache) with cache["h"] the bf16 routed h in sorted-row order.  dtype: the arithmetic of the
    GEMMs and the combine (float64; float32 for BASELINE-size checks, where float64 would take minutes).
    """
    k = p["k"]
    x = np.asarray(p["x"], np.float32)
    if route is None:
        logits, sel, _ = router(p["x"], p["w_r"], k, p.get("bias"))
    else:
        logits, sel = route
    lw = x.astype(np.float64) @ np.asarray(p["w_r"], np.float64)
    if p.get("bias") is not None:
        lw = lw + np.asarray(p["bias"], np.float64)
    w = topk_softmax(lw, sel)
    E = p["w_gate"].shape[0]
    T, d = x.shape
    xq, sx = fp8_quantize(x)
    xd = fp8_dequant(xq, sx)[0].astype(dtype)

    def deq(name, groups):
        wt = np.asarray(p[name], np.float32)
        q, s = fp8_quantize(wt, groups=groups)
        return fp8_dequant(q, s).astype(dtype)

    wg, wu, wd = deq("w_gate", E), deq("w_up", E), deq("w_down", E)
    lay = build_layout(sel, E)
    gs = lay["group_sizes"]
    xs = xd[lay["order"] // k]
    f = wg.shape[2]
    gg = np.zeros((xs.shape[0], f), dtype)
    uu = np.zeros_like(gg)
    start = 0
    for e in range(E):
        n = int(gs[e])
        gg[start:start + n] = xs[start:start + n] @ wg[e]
        uu[start:start + n] = xs[start:start + n] @ wu[e]
        start += n
    hb = round_bf16(silu(gg) * uu)
    hq, shv = fp8_quantize(hb)
    hd = fp8_dequant(hq, shv)[0].astype(dtype)
    ys = np.zeros((xs.shape[0], d), dtype)
    start = 0
    for e in range(E):
        n = int(gs[e])
        ys[start:start + n] = hd[start:start + n] @ wd[e]
        start += n
    out = (ys[lay["pos"]].reshape(T, k, d) * w.astype(dtype)[:, :, None]).sum(axis=1)
    shared = None
    if p.get("ws_gate") is not None:
        sg_, su_, sd_ = (deq(n, 1)[0] for n in ("ws_gate", "ws_up", "ws_down"))
        sgv, suv = xd @ sg_, xd @ su_
        shb = round_bf16(silu(sgv) * suv)
        sq, ss = fp8_quantize(shb)
        out = out + fp8_dequant(sq, ss)[0].astype(dtype) @ sd_
        shared = dict(h=shb, g=sgv, u=suv, h_sinv=ss[0])
    cache = dict(logits=logits, sel=sel, w=w, lay=lay, g=gg, u=uu, h=hb, y=ys, shared=shared, x_sinv=sx[0],
                 h_sinv=shv[0])
    return out, cache


def _swiglu_bwd_rows(dh, g, u):
    """(dG, dU) of h = silu(g) * u for dH, each rounded to bf16 (the GPU's SwiGLU backward epilogue)."""
    sg = 1.0 / (1.0 + np.exp(-g))
    return round_bf16(dh * u * sg * (1.0 + g * (1.0 - sg))), round_bf16(dh * g * sg)


def moe_layer_bwd_fp8(p, cache, dy, dtype=np.float64, quantize=True):
    """Backward of `moe_layer_fwd_fp8` with every expert GEMM on FP8 operands: the training half of the recipe.

    Gradients are quantised to E5M2 with current scaling just before their GEMMs: the routed dY rows (bf16
    w[t,j] dy[t], all routed rows one tensor) and [dG | dU] (bf16, all routed rows), the shared expert's dY (= dy)
    and [dG | dU] on their own.  dgrads multiply them with the weights' E4M3 values of the forward (one scale per
    expert and matrix, gate and up each their own); wgrads multiply the E4M3 values of the forward's x and h (same
    scales) with the E5M2 gradients.  g and u enter the SwiGLU backward as the bf16 values the forward saved, the
    expert dX rows are rounded to bf16 before the gather-reduce.  Routing-weight, router and dispatch backward are
    those of `moe_layer_bwd` (y rows in bf16).  Returns the dict of `moe_layer_bwd`.
    quantize=False skips every FP8 cast (the operands stay bf16 / exact) and keeps the bf16 roundings: the same data
    flow, for pinning it against `moe_layer_bwd`.
    """
    k = p["k"]
    x = np.asarray(p["x"], np.float32)
    T, d = x.shape
    E = p["w_gate"].shape[0]
    lay, w, sel = cache["lay"], cache["w"], cache["sel"]
    order, pos, gs = lay["order"], lay["pos"], lay["group_sizes"]

    def q4(a, groups=1):  # E4M3 and back, one scale per group
        a = np.asarray(a, np.float32)
        if not quantize:
            return a.astype(dtype).reshape((groups,) + a.shape[-2:])
        q, sc = fp8_quantize(a, groups=groups)
        return fp8_dequant(q, sc).astype(dtype)

    def q5(a):  # one tensor to E5M2 and back
        if not quantize:
            return np.asarray(a, dtype)
        q, sc = fp8_quantize(a, fmt="e5m2")
        return fp8_dequant(q, sc, fmt="e5m2")[0].astype(dtype)

    def deq(name, groups):
        return q4(p[name], groups)

    xd = q4(x)[0]

    wg, wu, wd = deq("w_gate", E), deq("w_up", E), deq("w_down", E)
    f = wg.shape[2]
    xs = xd[order // k]
    gb, ub = round_bf16(cache["g"]), round_bf16(cache["u"])
    hd = q4(cache["h"])[0]
    wf = np.asarray(w, np.float32).reshape(-1)
    dys = q5(round_bf16(np.asarray(dy, np.float32)[order // k] * wf[order][:, None]))
    dh = np.zeros((xs.shape[0], f), dtype)
    start = 0
    for e in range(E):
        n = int(gs[e])
        dh[start:start + n] = dys[start:start + n] @ wd[e].T
        start += n
    dgu = q5(np.concatenate(_swiglu_bwd_rows(dh, gb, ub), axis=1))
    dxs = np.zeros((xs.shape[0], d), dtype)
    dwg, dwu, dwd = np.zeros_like(wg), np.zeros_like(wu), np.zeros_like(wd)
    start = 0
    for e in range(E):
        n = int(gs[e])
        sl = slice(start, start + n)
        dxs[sl] = dgu[sl, :f] @ wg[e].T + dgu[sl, f:] @ wu[e].T
        dwg[e], dwu[e], dwd[e] = xs[sl].T @ dgu[sl, :f], xs[sl].T @ dgu[sl, f:], hd[sl].T @ dys[sl]
        start += n
    dx = round_bf16(dxs)[pos].reshape(T, k, d).sum(axis=1)
    dyf = np.asarray(dy, dtype)
    dw = np.einsum("tkd,td->tk", round_bf16(cache["y"])[pos].reshape(T, k, d), dyf)
    w64 = np.asarray(w, dtype)
    dl_sel = w64 * (dw - (w64 * dw).sum(axis=1, keepdims=True))
    dlogits = np.zeros((T, E), dtype)
    np.put_along_axis(dlogits, sel.astype(np.int64), dl_sel, axis=1)
    x64 = x.astype(dtype)
    dx = dx + dlogits @ np.asarray(p["w_r"], dtype).T
    out = dict(dx=dx, dw_r=x64.T @ dlogits, dw_gate=dwg, dw_up=dwu, dw_down=dwd, dw=dw, dlogits=dlogits)
    if cache["shared"] is not None:
        sh = cache["shared"]
        sgw, suw, sdw = (deq(n, 1)[0] for n in ("ws_gate", "ws_up", "ws_down"))
        fs = sgw.shape[1]
        sdy = q5(np.asarray(dy, np.float32))
        sdgu = q5(np.concatenate(_swiglu_bwd_rows(sdy @ sdw.T, round_bf16(sh["g"]), round_bf16(sh["u"])), axis=1))
        shd = q4(sh["h"])[0]
        out["dx"] = out["dx"] + round_bf16(sdgu[:, :fs] @ sgw.T + sdgu[:, fs:] @ suw.T)
        out["dws_gate"], out["dws_up"], out["dws_down"] = xd.T @ sdgu[:, :fs], xd.T @ sdgu[:, fs:], shd.T @ sdy
    return out


# --------------------------------------------------------------------------------------------- causal depthwise conv
#
# modal/fast_conv.py:14-31 (`_fast_call`, standing in for flax nnx.Conv(padding="CAUSAL",
# feature_group_count=C) on [B, T, C] inputs with a [K, 1, C] kernel): y[b, t, c] = sum_{j<K} w[j, c] x[b, t-(K-1)+j, c],
# zero before t = 0 (fast_conv.py:27-30 pads K-1 rows in front and adds the K shifted products, j ascending).


def causal_conv1d(x, w):
    """x [B, T, C], w [K, C] -> y [B, T, C] in float64."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    K, T = w.shape[0], x.shape[1]
    xp = np.concatenate([np.zeros((x.shape[0], K - 1, x.shape[2])), x], axis=1)
    y = xp[:, 0:T] * w[0]
    for j in range(1, K):
        y = y + xp[:, j:j + T] * w[j]
    return y


def causal_conv1d_bwd(x, w, dy):
    """(dx [B, T, C], dw [K, C]) of causal_conv1d for upstream dy, float64:
    dx[b, t, c] = sum_j w[j, c] dy[b, t+(K-1)-j, c] (zero past T); dw[j, c] = sum_{b,t} dy[b, t, c] x[b, t-(K-1)+j, c]."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    dy = np.asarray(dy, np.float64)
    K, T = w.shape[0], x.shape[1]
    dyp = np.concatenate([dy, np.zeros((dy.shape[0], K - 1, dy.shape[2]))], axis=1)
    dx = np.zeros_like(x)
    for j in range(K):
        dx += w[j] * dyp[:, K - 1 - j:K - 1 - j + T]
    xp = np.concatenate([np.zeros((x.shape[0], K - 1, x.shape[2])), x], axis=1)
    dw = np.stack([(dy * xp[:, j:j + T]).sum(axis=(0, 1)) for j in range(K)])
    return dx, dw


# --------------------------------------------------------------------------------------------- metrics


def rel_l2(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / (np.linalg.norm(want) + 1e-30))


def rel_max(got, want):
    """max|got - want| / (max|want| + 1e-6): modal/test_moe_permute.py:29-34."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / (np.abs(want).max() + 1e-6)) if want.size else 0.0
