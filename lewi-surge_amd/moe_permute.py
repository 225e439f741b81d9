"""MoE token permute / combine for MI355X: the public surface of the reference's modal/moe_permute.py, with the
row movement done by hand-written gfx950 HIP kernels (liblewi_surge.so) instead of Pallas-TPU DMA kernels.

Same names, arguments, output dtypes and VJP structure as the reference (paths in prostos2162-maker/lewi-surge):

  gather_rows(x, idx[, scale])   out[i] = x[idx[i]] * scale[i]            dispatch fwd, combine bwd (dy)
  gather_reduce(y, pos[, w])     out[t] = sum_j w[t,j] * y[pos[t,j]]      combine fwd, dispatch bwd (dx)
  gather_dot(y, pos, g)          out[t,j] = <g[t], y[pos[t,j]]>           combine bwd (dw)
  sort_indices, dispatch, combine, permute_rows, ref_dispatch, ref_combine, moe_block, probe_packing, install

Arrays are torch tensors on a ROCm device (JAX is not part of this image); differentiable ops are
torch.autograd.Functions with the reference's custom_vjp rules.  The kernels handle every row count and width
(no tiling constraint), so the reference's "untileable shape -> XLA" fallback never triggers; CFG["enabled"] =
False still selects the plain-torch reference ops (the reference's A/B switch, modal/moe_permute.py:33).
"""
from __future__ import annotations

import torch

import _lib as L

CFG = {
    "enabled": True,      # False -> plain torch reference everywhere (A/B switch)
    "tile": 128,          # rows per grid step in the reference's Pallas kernels; kept for API compatibility
    "even_low": True,     # bf16 u32 packing convention on TPU; CDNA moves rows directly, no packing
    "prepack": None,
    "sort": "argsort",    # "argsort" or "count": both map to the same stable counting-sort kernel here
    "num_experts": None,  # needed for sort="count"
    "vmem_mb": None,
}

# ----------------------------------------------------------------------------------------------- helpers


def _interpret():
    """The reference's Pallas interpret mode (CPU tests); HIP kernels always run natively: None."""
    return None


def _pick_tile(*rows):
    """Tile the reference would pick (modal/moe_permute.py:57-61).  Informational: HIP kernels need no tiling."""
    for t in (CFG["tile"], 256, 128, 64, 32, 16, 8):
        if t and all(r % t == 0 for r in rows):
            return t
    return None


def _out_like(shape, dtype, device):
    return torch.empty(shape, dtype=dtype, device=device)


def _i32(t):
    return L.contig(t.to(torch.int32))


# ----------------------------------------------------------------------------------------------- kernels


def gather_rows(x, idx, scale=None):
    """out[i] = x[idx[i]] (* scale[i]).  x: (N, D), idx: (M,) int32, scale: (M,) f32 or None -> (M, D) x.dtype.

    modal/moe_permute.py:116-158.
    """
    if not CFG["enabled"]:
        out = x[idx.long()]
        return out if scale is None else (out.float() * scale.float()[:, None]).to(x.dtype)
    L.require_cuda(x, idx, scale)
    x = L.contig(x)
    idx = _i32(idx)
    scale = None if scale is None else L.contig(scale.to(torch.float32))
    n, d = x.shape
    m = idx.shape[0]
    out = _out_like((m, d), x.dtype, x.device)
    L.check(L.lib().lsurge_gather_rows(L.ptr(x), n, d, L.dt(x), L.ptr(idx), m, L.ptr(scale), L.ptr(out),
                                       L.stream(x.device)), "gather_rows")
    return out


def gather_reduce(y, pos, w=None, out_dtype=None):
    """out[t] = sum_j w[t,j] * y[pos[t,j]] in f32.  y: (M, D), pos: (N, k) int32, w: (N, k) or None -> (N, D).

    modal/moe_permute.py:214-225.
    """
    out_dtype = out_dtype or y.dtype
    n, k = pos.shape
    if w is not None:
        w = w.to(torch.float32)
    if not CFG["enabled"]:
        g = y[pos.reshape(-1).long()].float().reshape(n, k, -1)
        if w is not None:
            g = g * w[:, :, None]
        return g.sum(dim=1).to(out_dtype)
    L.require_cuda(y, pos, w)
    y = L.contig(y)
    pos = _i32(pos)
    w = L.contig(w)
    m, d = y.shape
    out = _out_like((n, d), out_dtype, y.device)
    L.check(L.lib().lsurge_gather_reduce(L.ptr(y), m, d, L.dt(y), L.ptr(pos), n, k, L.ptr(w), L.ptr(out),
                                         L.dt(out), L.stream(y.device)), "gather_reduce")
    return out


def gather_dot(y, pos, g):
    """out[t, j] = <g[t], y[pos[t,j]]> in f32.  y: (M, D), pos: (N, k), g: (N, D) -> (N, k) f32.

    modal/moe_permute.py:228-234.
    """
    n, k = pos.shape
    if not CFG["enabled"]:
        rows = y[pos.reshape(-1).long()].float().reshape(n, k, -1)
        return torch.einsum("nkd,nd->nk", rows, g.float())
    L.require_cuda(y, pos, g)
    y, g = L.contig(y), L.contig(g)
    pos = _i32(pos)
    m, d = y.shape
    out = _out_like((n, k), torch.float32, y.device)
    L.check(L.lib().lsurge_gather_dot(L.ptr(y), m, d, L.dt(y), L.ptr(pos), n, k, L.ptr(g), L.dt(g), L.ptr(out),
                                      L.stream(y.device)), "gather_dot")
    return out


# ----------------------------------------------------------------------------------------------- routing indices


def sort_indices(flat_experts, num_experts=None, method=None):
    """Stable sort of the N*k expert slots by expert id.  modal/moe_permute.py:240-264.

    Returns (order, pos): order[p] = slot at sorted position p (what argsort gives), pos[i] = sorted position of
    slot i (its inverse).  Both methods use the same deterministic counting-sort kernel (per-wave LDS histograms,
    an exclusive scan over chunks, and ballot/popcount ranks), which is exactly a stable argsort.
    """
    method = method or CFG["sort"]
    flat = _i32(flat_experts.reshape(-1))
    m = flat.shape[0]
    if not CFG["enabled"]:
        order = torch.argsort(flat, stable=True).to(torch.int32)
        return order, torch.argsort(order, stable=True).to(torch.int32)
    L.require_cuda(flat)
    e = num_experts
    if e is None:  # the argsort path needs no expert count; take it from the data (one host sync)
        e = int(flat.max().item()) + 1 if m else 1
    order = torch.empty(m, dtype=torch.int32, device=flat.device)
    pos = torch.empty_like(order)
    ws = L.workspace(L.lib().lsurge_sort_indices_workspace_bytes(m, e), flat.device)
    L.check(L.lib().lsurge_sort_indices(L.ptr(flat), m, e, L.ptr(order), L.ptr(pos), None, L.ptr(ws), ws.numel(),
                                        L.stream(flat.device)), "sort_indices")
    return order, pos


def _invert(idx):
    inv = torch.empty_like(idx)
    L.check(L.lib().lsurge_invert_permutation(L.ptr(idx), idx.shape[0], L.ptr(inv), L.stream(idx.device)),
            "invert_permutation")
    return inv


# ----------------------------------------------------------------------------------------------- differentiable ops


class _Dispatch(torch.autograd.Function):
    """x: (N, D) tokens -> (N*k, D) rows grouped by expert (row p = x[order[p] // k]).  moe_permute.py:270-289."""

    @staticmethod
    def forward(ctx, x, order, pos):
        k = order.shape[0] // x.shape[0]
        ctx.save_for_backward(order, pos)
        ctx.n, ctx.xdtype = x.shape[0], x.dtype
        return gather_rows(x, torch.div(order, k, rounding_mode="floor"))

    @staticmethod
    def backward(ctx, g):
        order, pos = ctx.saved_tensors
        n = ctx.n
        k = order.shape[0] // n
        return gather_reduce(g, pos.reshape(n, k), None, ctx.xdtype), None, None


class _Combine(torch.autograd.Function):
    """y: (N*k, D) expert outputs in sorted order, w: (N, k) -> (N, D) f32.  moe_permute.py:292-312."""

    @staticmethod
    def forward(ctx, y, order, pos, w):
        n, k = w.shape
        ctx.save_for_backward(y, order, pos, w)
        return gather_reduce(y, pos.reshape(n, k), w, torch.float32)

    @staticmethod
    def backward(ctx, g):
        y, order, pos, w = ctx.saved_tensors
        n, k = w.shape
        if not CFG["enabled"]:
            w_sorted = w.reshape(-1).float()[order.long()]
            dy = gather_rows(g.to(y.dtype), torch.div(order, k, rounding_mode="floor"), w_sorted)
            dw = gather_dot(y, pos.reshape(n, k), g).to(w.dtype)
            return dy, None, None, dw
        # one fused pass: dy[pos[t,j]] = w[t,j] g[t] and dw[t,j] = <g[t], y[pos[t,j]]>
        y = L.contig(y)
        g = L.contig(g)
        pos = _i32(pos)
        wf = L.contig(w.to(torch.float32))
        d = y.shape[1]
        dy = torch.empty_like(y)
        dw = torch.empty((n, k), dtype=torch.float32, device=y.device)
        L.check(L.lib().lsurge_combine_bwd(L.ptr(y), L.dt(y), L.ptr(pos), L.ptr(wf), n, k, d, L.ptr(g), L.dt(g),
                                           L.ptr(dy), L.ptr(dw), L.stream(y.device)), "combine_bwd")
        return dy, None, None, dw.to(w.dtype)


class _PermuteRows(torch.autograd.Function):
    """x[idx] for a permutation idx; backward un-permutes.  moe_permute.py:315-329."""

    @staticmethod
    def forward(ctx, x, idx):
        ctx.save_for_backward(idx)
        return gather_rows(x, idx)

    @staticmethod
    def backward(ctx, g):
        (idx,) = ctx.saved_tensors
        if not CFG["enabled"]:
            return gather_rows(g, torch.argsort(idx)), None
        return gather_rows(g, _invert(_i32(idx))), None


def dispatch(x, order, pos):
    return _Dispatch.apply(x, _i32(order), _i32(pos))


def combine(y, order, pos, w):
    return _Combine.apply(y, _i32(order), _i32(pos), w)


def permute_rows(x, idx):
    return _PermuteRows.apply(x, _i32(idx))


# ----------------------------------------------------------------------------------------------- reference (plain torch)


def ref_dispatch(x, flat_experts):
    """modal/moe_permute.py:335-338."""
    k = flat_experts.shape[0] // x.shape[0]
    order = torch.argsort(flat_experts, stable=True)
    return x[torch.div(order, k, rounding_mode="floor")]


def ref_combine(y, flat_experts, w):
    """modal/moe_permute.py:341-345."""
    n, k = w.shape
    pos = torch.argsort(torch.argsort(flat_experts, stable=True), stable=True)
    rows = y[pos].float().reshape(n, k, -1)
    return torch.einsum("nkd,nk->nd", rows, w.float())


def moe_block(x, flat_experts, w, expert_fn, use_kernels=True):
    """dispatch -> expert_fn(rows) -> combine, with kernels or the reference.  modal/moe_permute.py:348-353."""
    if use_kernels:
        order, pos = sort_indices(flat_experts, CFG["num_experts"])
        return combine(expert_fn(dispatch(x, order, pos)), order, pos, w)
    return ref_combine(expert_fn(ref_dispatch(x, flat_experts)), flat_experts, w)


# ----------------------------------------------------------------------------------------------- device probe


def probe_packing(d=256, n=64, verbose=True):
    """The reference probes the TPU's bf16 u32 packing (modal/moe_permute.py:359-380); rows are moved unpacked on
    CDNA, so like the reference off-TPU (361-362) this returns CFG["even_low"]."""
    return CFG["even_low"]


# ----------------------------------------------------------------------------------------------- MaxText patch


def install(mode="gather", tile=None, sort=None, num_experts=None, probe=True):
    """Patch maxtext.layers.moe (0.2.5 dropless path).  modal/moe_permute.py:386-436.

    MaxText is a JAX package: it is imported first, as in the reference, so without it this raises ImportError.
    JAX callers reach the same kernels through the XLA FFI binding of the C ABI.
    """
    import maxtext.layers.moe as moe  # noqa: F401  pylint: disable=import-outside-toplevel,import-error

    if tile:
        CFG["tile"] = tile
    if sort:
        CFG["sort"] = sort
    if num_experts:
        CFG["num_experts"] = num_experts
    if probe:
        probe_packing()
    raise NotImplementedError("moe_permute.install: patching JAX MaxText needs the XLA FFI binding of liblewi_surge")


def abi_version():
    return int(L.lib().lsurge_abi_version())


__all__ = ["CFG", "gather_rows", "gather_reduce", "gather_dot", "sort_indices", "dispatch", "combine", "permute_rows",
           "ref_dispatch", "ref_combine", "moe_block", "probe_packing", "install"]

