"""Write the golden fixtures in this directory (`python tests/golden/make_golden.py`).

The reference repository holds no vectors for this path (its .gitignore excludes .npy/.npz), so these
fixtures are computed here, by scalar per-token loops written independently of the vectorised oracle in
`oracle/moe_oracle.py`: explicit float32 sequential sums for the router logits, a sort key of
(-logit, expert) for the top-k, a stable counting pass for the layout, and float64 per-token / per-choice
loops with the chain rule spelled out for the layer backward.  The oracle and the HIP path are both checked
against them (tests/test_golden.py).

Cases:
* router_ties   -- router + layout with planted exact ties (duplicated router columns, all-zero tokens);
                   semantics of modal/test_moe_permute.py:23-26 (argsort(-logits)[:, :k], stable).
* ragged_dot_te -- the known-answer shape of modal/te_run.py:72-79: gs = [5,0,9,3,7,1,6,4],
                   M = sum(gs) + 3, K = 64, N = 48; rows past sum(gs) are zero; forward and backward.
* layer_small   -- whole MoE layer forward + backward with a shared expert (T=40, d=64, E=8, k=3, f=64).
* layer_zipf    -- whole layer with the Zipf router bias and empty experts, no shared expert
                   (T=24, d=64, E=8, k=2, f=64).
Shapes follow the layer's limits: d, f, f_s multiples of 64, E a multiple of 8.

bf16 tensors are stored as their uint16 bit patterns, float32 logits as uint32 bits.
"""
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BLOCK = 128


def to_bf16_bits(a):
    """float32 -> bf16 bits, round to nearest even (finite inputs only)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def from_bf16_bits(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def draw(rng, shape, std):
    bits = to_bf16_bits(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))
    return bits, from_bf16_bits(bits)


# ------------------------------------------------------------------------------------------------ router, layout


def logits_f32(x, w_r, bias):
    """logits[t, e]: float32 running sum over d in index order, then + bias[e] (one float32 add each)."""
    T, d = x.shape
    E = w_r.shape[1]
    out = np.zeros((T, E), np.float32)
    for t in range(T):
        for e in range(E):
            acc = np.float32(0.0)
            for i in range(d):
                acc = np.float32(acc + np.float32(x[t, i]) * np.float32(w_r[i, e]))
            if bias is not None:
                acc = np.float32(acc + np.float32(bias[e]))
            out[t, e] = acc
    return out


def select(lg, k):
    """k largest logits per token, descending; equal logits -> lower expert index first."""
    return np.array([sorted(range(lg.shape[1]), key=lambda e: (-float(lg[t, e]), e))[:k]
                     for t in range(lg.shape[0])], np.int32)


def layout(sel, E):
    """Counting-sort layout: order (stable by flat slot), pos = order^-1, padded slot of each flat slot."""
    flat = [int(v) for v in sel.reshape(-1)]
    M = len(flat)
    gs = [0] * E
    for e in flat:
        gs[e] += 1
    offsets, block_off = [0] * E, [0] * E
    run, brun = 0, 0
    for e in range(E):
        offsets[e], block_off[e] = run, brun
        run += gs[e]
        brun += -(-gs[e] // BLOCK)
    fill = list(offsets)
    order, pos = [0] * M, [0] * M
    for s, e in enumerate(flat):  # flat slots visited in increasing order -> stable
        order[fill[e]] = s
        pos[s] = fill[e]
        fill[e] += 1
    slot = [BLOCK * block_off[flat[s]] + pos[s] - offsets[flat[s]] for s in range(M)]
    i32 = lambda v: np.array(v, np.int32)  # noqa: E731
    return dict(group_sizes=i32(gs), offsets=i32(offsets), block_off=i32(block_off), order=i32(order),
                pos=i32(pos), slot=i32(slot), num_blocks=np.int32(brun))


def softmax_sel(lg64, sel):
    out = np.zeros(sel.shape, np.float64)
    for t in range(sel.shape[0]):
        v = [lg64[t, e] for e in sel[t]]
        m = max(v)
        z = [math.exp(a - m) for a in v]
        s = sum(z)
        out[t] = [a / s for a in z]
    return out


def make_router_ties():
    rng = np.random.default_rng(11)
    T, d, E, k = 48, 64, 16, 4
    xb, x = draw(rng, (T, d), 1.0)
    wb, w = draw(rng, (d, E), 0.02)
    wb[:, 12:16] = wb[:, 0:4]  # experts 12..15 tie with 0..3 on every token
    wb[:, 9] = wb[:, 6]
    xb[:5] = 0                 # all-zero tokens: every logit is 0 -> experts 0..k-1
    x, w = from_bf16_bits(xb), from_bf16_bits(wb)
    lg = logits_f32(x, w, None)
    sel = select(lg, k)
    assert (sel[:5] == np.arange(k)).all()
    wts = softmax_sel(lg.astype(np.float64), sel)
    return dict(x=xb, w_r=wb, k=np.int32(k), logits=lg.view(np.uint32), sel=sel, weights=wts,
                **layout(sel, E))


# ------------------------------------------------------------------------------------------------ ragged_dot


def make_ragged_dot_te():
    rng = np.random.default_rng(3)
    gs = [5, 0, 9, 3, 7, 1, 6, 4]
    E, K, N = len(gs), 64, 48
    M = sum(gs) + 3
    lb, lhs = draw(rng, (M, K), 1.0)
    rb, rhs = draw(rng, (E, K, N), 1.0)
    gb, g = draw(rng, (M, N), 1.0)
    L, R, G = (a.astype(np.float64) for a in (lhs, rhs, g))
    out = np.zeros((M, N))
    dl = np.zeros((M, K))
    dr = np.zeros((E, K, N))
    r = 0
    for e, n in enumerate(gs):
        for _ in range(n):
            for c in range(N):
                out[r, c] = sum(L[r, i] * R[e, i, c] for i in range(K))
            dl[r] = [sum(G[r, c] * R[e, i, c] for c in range(N)) for i in range(K)]
            dr[e] += np.outer(L[r], G[r])
            r += 1
    return dict(group_sizes=np.array(gs, np.int32), lhs=lb, rhs=rb, g=gb, out=out, dlhs=dl, drhs=dr)


# ------------------------------------------------------------------------------------------------ layer


def sig(z):
    return 1.0 / (1.0 + math.exp(-z))


def swiglu_tok(xt, wg, wu, wd):
    g = xt @ wg
    u = xt @ wu
    s = np.array([sig(v) for v in g])
    h = g * s * u
    return h @ wd, (g, u, s, h)


def swiglu_tok_bwd(xt, wg, wu, wd, cache, dyt):
    """One token through the SwiGLU MLP backward: returns dx_t and adds nothing (callers add weight grads)."""
    g, u, s, h = cache
    dh = wd @ dyt                       # [f]
    dsilu = s * (1.0 + g * (1.0 - s))   # d/dg (g * sigmoid(g))
    dg = dh * u * dsilu
    du = dh * g * s
    dx = wg @ dg + wu @ du
    return dx, np.outer(xt, dg), np.outer(xt, du), np.outer(h, dyt)


def make_layer(T, d, E, k, f, fs, seed, zipf):
    rng = np.random.default_rng(seed)
    names = ["x", "w_r", "w_gate", "w_up", "w_down"] + (["ws_gate", "ws_up", "ws_down"] if fs else []) + ["dy"]
    shapes = dict(x=(T, d), w_r=(d, E), w_gate=(E, d, f), w_up=(E, d, f), w_down=(E, f, d), ws_gate=(d, fs),
                  ws_up=(d, fs), ws_down=(fs, d), dy=(T, d))
    std = dict(x=1.0, dy=1.0)
    bits, val = {}, {}
    for n in names:
        bits[n], val[n] = draw(rng, shapes[n], std.get(n, 0.02))
    bias = (1.5 * np.log(1.0 / np.arange(1, E + 1, dtype=np.float64))).astype(np.float32) if zipf else None
    F = {n: v.astype(np.float64) for n, v in val.items()}

    lg = logits_f32(val["x"], val["w_r"], bias)
    sel = select(lg, k)
    lg64 = F["x"] @ F["w_r"] + (0.0 if bias is None else bias.astype(np.float64))
    w = softmax_sel(lg64, sel)

    out = np.zeros((T, d))
    dx = np.zeros((T, d))
    dwr = np.zeros((d, E))
    dwg, dwu, dwd = (np.zeros_like(F[n]) for n in ("w_gate", "w_up", "w_down"))
    dweights = np.zeros((T, k))
    for t in range(T):
        xt, dyt = F["x"][t], F["dy"][t]
        ys = []
        for j in range(k):
            e = int(sel[t, j])
            y, cache = swiglu_tok(xt, F["w_gate"][e], F["w_up"][e], F["w_down"][e])
            out[t] += w[t, j] * y
            ys.append(y)
            dxt, a, b, c = swiglu_tok_bwd(xt, F["w_gate"][e], F["w_up"][e], F["w_down"][e], cache, w[t, j] * dyt)
            dx[t] += dxt
            dwg[e] += a
            dwu[e] += b
            dwd[e] += c
            dweights[t, j] = float(dyt @ y)
        # softmax over the selected logits: dl_j = w_j (dw_j - sum_i w_i dw_i)
        s = float(w[t] @ dweights[t])
        for j in range(k):
            e = int(sel[t, j])
            dl = w[t, j] * (dweights[t, j] - s)
            dwr[:, e] += xt * dl
            dx[t] += F["w_r"][:, e] * dl
    fx = dict(k=np.int32(k), sel=sel, **{n: bits[n] for n in names})
    if bias is not None:
        fx["bias"] = bias
    grads = dict(dx=dx, dw_r=dwr, dw_gate=dwg, dw_up=dwu, dw_down=dwd, dweights=dweights)
    if fs:
        dsg, dsu, dsd = (np.zeros_like(F[n]) for n in ("ws_gate", "ws_up", "ws_down"))
        for t in range(T):
            y, cache = swiglu_tok(F["x"][t], F["ws_gate"], F["ws_up"], F["ws_down"])
            out[t] += y
            dxt, a, b, c = swiglu_tok_bwd(F["x"][t], F["ws_gate"], F["ws_up"], F["ws_down"], cache, F["dy"][t])
            dx[t] += dxt
            dsg += a
            dsu += b
            dsd += c
        grads.update(dws_gate=dsg, dws_up=dsu, dws_down=dsd)
    fx["out"] = out.astype(np.float32)
    fx.update({"want_" + n: v.astype(np.float32) for n, v in grads.items()})
    fx.update(layout(sel, E))
    return fx


CASES = {
    "router_ties": make_router_ties,
    "ragged_dot_te": make_ragged_dot_te,
    "layer_small": lambda: make_layer(40, 64, 8, 3, 64, 64, seed=7, zipf=False),
    "layer_zipf": lambda: make_layer(24, 64, 8, 2, 64, 0, seed=8, zipf=True),
}


def main():
    for name, fn in CASES.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
