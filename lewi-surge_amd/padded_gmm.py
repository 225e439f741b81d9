"""Grouped GEMM in place of jax.lax.ragged_dot -- the public surface of the reference's modal/padded_gmm.py,
computed by hand-written gfx950 MFMA kernels (liblewi_surge.so) on bf16, f16 or f32 operands.

Input as for ragged_dot: lhs [M, K] sorted by group, rhs [E, K, N], group_sizes [E] -> [M, N].  float32 operands
run on the same bf16 kernels, each value split into three bf16 terms (see padded_ragged_dot).

Layout.  The reference copies the rows into a capacity buffer [E, C, K] (C = roundup8(ceil(M/E * FACTOR))), runs
one batched einsum and gathers back, silently dropping rows past C (modal/padded_gmm.py:8, 51-69).  Here the
rows stay where they are: the kernel walks 128-row blocks that start at each group's first row, so there is no
capacity, no copy and no drop -- the result is dropless ragged_dot semantics, which equal the reference's
whenever max(group_sizes) <= C.  FACTOR is kept and set by install() for API compatibility only.

Backward (gather-only in the reference, 10-11, 35-39): dlhs = g @ rhs[e]^T per block and drhs[e] = lhs_e^T g_e
with the reduction over the group's rows; no scatter, no atomics.
"""
from __future__ import annotations

import math

import torch

import _lib as L


def _orig_ragged_dot(lhs, rhs, group_sizes, precision=None, preferred_element_type=None, **kw):
    """Stands in for the saved jax.lax.ragged_dot (modal/padded_gmm.py:20), which the reference calls for inputs
    outside the padded kernel (lhs not 2-D, rhs not 3-D, or group_offset given, 46-48).  There is no other
    ragged_dot implementation on this stack, so those inputs are rejected."""
    raise NotImplementedError(f"ragged_dot: unsupported inputs lhs.ndim={lhs.ndim} rhs.ndim={rhs.ndim} "
                              f"group_offset={kw.get('group_offset')!r}")


FACTOR = 2.0


def capacity(m, e, factor=None):
    """The reference's per-expert capacity C (modal/padded_gmm.py:51-52); informational here."""
    c = int(math.ceil(m / e * (FACTOR if factor is None else factor)))
    return max(8, (c + 7) // 8 * 8)


class _PermGather(torch.autograd.Function):
    """y[i] = x_ext[idx[i]], x_ext = x plus a zero row (idx == len(x) -> 0); backward dx = gather(g, inv_idx).

    modal/padded_gmm.py:24-42 (gather-only VJP).
    """

    @staticmethod
    def forward(ctx, x, idx, inv_idx):
        ctx.save_for_backward(idx, inv_idx)
        ctx.n = x.shape[0]
        return _gather_ext(x, idx)

    @staticmethod
    def backward(ctx, g):
        idx, inv_idx = ctx.saved_tensors
        dx = _gather_ext(g, inv_idx)
        return (dx[:ctx.n] if dx.shape[0] != ctx.n else dx), None, None


def _gather_ext(x, idx):
    x = L.contig(x)
    idx = L.contig(idx.to(torch.int32))
    n, d = x.shape
    out = torch.empty((idx.shape[0], d), dtype=x.dtype, device=x.device)
    # the kernel writes a zero row for every index outside [0, n), which covers the sentinel n
    L.check(L.lib().lsurge_gather_rows(L.ptr(x), n, d, L.dt(x), L.ptr(idx), idx.shape[0], None, L.ptr(out),
                                       L.stream(x.device)), "perm_gather")
    return out


def _perm_gather(x, idx, inv_idx):
    L.require_cuda(x, idx, inv_idx)
    return _PermGather.apply(x, idx, inv_idx)


def _aligned(t):
    """t, or a copy of it when its data does not start on a 16-byte boundary (the f32 split kernels' float4 loads)."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


class _RaggedDot(torch.autograd.Function):

    @staticmethod
    def forward(ctx, lhs, rhs, group_sizes, out_dtype):
        m, k = lhs.shape
        e, _, n = rhs.shape
        out = torch.empty((m, n), dtype=out_dtype, device=lhs.device)
        if lhs.dtype == torch.float32:
            lhs, rhs = _aligned(lhs), _aligned(rhs)
            wsb = L.lib().lsurge_ragged_dot_f32_workspace_bytes(m, k, n, e)
        else:
            wsb = L.lib().lsurge_ragged_dot_workspace_bytes(m, e)
        ws = L.workspace(wsb, lhs.device)
        L.check(L.lib().lsurge_ragged_dot(L.ptr(lhs), L.ptr(rhs), L.ptr(group_sizes), m, k, n, e, L.dt(lhs),
                                          L.ptr(out), L.dt(out), L.ptr(ws), ws.numel(), L.stream(lhs.device)),
                "ragged_dot")
        ctx.save_for_backward(lhs, rhs, group_sizes)
        return out

    @staticmethod
    def backward(ctx, g):
        lhs, rhs, gs = ctx.saved_tensors
        m, k = lhs.shape
        e, _, n = rhs.shape
        g = L.contig(g.to(lhs.dtype))
        dlhs = torch.empty_like(lhs)
        drhs = torch.empty((e, k, n), dtype=torch.float32, device=lhs.device)
        if lhs.dtype == torch.float32:
            g = _aligned(g)
            wsb = L.lib().lsurge_ragged_dot_bwd_f32_workspace_bytes(m, k, n, e)
        else:
            wsb = L.lib().lsurge_ragged_dot_bwd_workspace_bytes(m, k, n, e)
        ws = L.workspace(wsb, lhs.device)
        L.check(L.lib().lsurge_ragged_dot_bwd(L.ptr(lhs), L.ptr(rhs), L.ptr(gs), L.ptr(g), m, k, n, e, L.dt(lhs),
                                              L.ptr(dlhs), L.ptr(drhs), L.ptr(ws), ws.numel(), L.stream(lhs.device)),
                "ragged_dot_bwd")
        return dlhs, drhs.to(rhs.dtype), None, None


def padded_ragged_dot(lhs, rhs, group_sizes, precision=None, preferred_element_type=None, **kw):
    """Dropless grouped GEMM with ragged_dot's signature.  modal/padded_gmm.py:45-69.

    lhs [M, K] bf16, f16 or float32 (rows sorted by group), rhs [E, K, N] (cast to lhs.dtype as in the reference,
    67), group_sizes [E] int -> [M, N] in preferred_element_type (default lhs.dtype); rows past sum(gs) are 0.
    float32 operands run on the bf16 matrix cores as three bf16 terms per value, summing the six term products of
    order <= 2 in f32 (about 2^-24 relative error per product: the einsum's f32 result at its highest precision,
    whatever `precision` asks); their output is float32 or bfloat16.
    """
    if lhs.ndim != 2 or rhs.ndim != 3 or kw.get("group_offset") is not None:
        return _orig_ragged_dot(lhs, rhs, group_sizes, precision=precision,
                                preferred_element_type=preferred_element_type, **kw)
    L.require_cuda(lhs, rhs, group_sizes)
    if lhs.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"padded_ragged_dot: lhs must be bfloat16, float16 or float32, got {lhs.dtype}")
    out_dtype = preferred_element_type or lhs.dtype
    allowed = (torch.float32, torch.bfloat16) if lhs.dtype == torch.float32 else (lhs.dtype, torch.float32)
    if out_dtype not in allowed:
        raise TypeError(f"padded_ragged_dot: preferred_element_type {out_dtype} not supported for {lhs.dtype} "
                        f"operands ({' or '.join(str(a) for a in allowed)})")
    m, k = lhs.shape
    e, k2, n = rhs.shape
    if k2 != k or group_sizes.shape != (e,):
        raise ValueError(f"padded_ragged_dot: shapes lhs {tuple(lhs.shape)} rhs {tuple(rhs.shape)} "
                         f"group_sizes {tuple(group_sizes.shape)} do not match")
    return _RaggedDot.apply(L.contig(lhs), L.contig(rhs.to(lhs.dtype)), L.contig(group_sizes.to(torch.int32)),
                            out_dtype)


def install(factor=2.0):
    """Set FACTOR and announce the kernel (modal/padded_gmm.py:72-76).  The reference rebinds jax.lax.ragged_dot;
    with JAX absent, callers use padded_ragged_dot directly (JAX callers bind the C ABI through XLA FFI)."""
    global FACTOR
    FACTOR = float(factor)
    try:
        import jax  # noqa: F401  pylint: disable=import-outside-toplevel
        raise NotImplementedError("padded_gmm.install: rebinding jax.lax.ragged_dot needs the XLA FFI binding")
    except ImportError:
        pass
    print(f"[padded_gmm] ragged_dot -> gfx950 grouped GEMM, dropless 128-row blocks (factor={FACTOR} kept for "
          "API compatibility)", flush=True)
