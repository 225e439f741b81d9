"""Chunked gated delta rule of the Gated DeltaNet block on the HIP library (mirrors modal/gdn_fast.py).

The reference swaps MaxText's `jax_chunk_gated_delta_rule` for `fast_chunk_gated_delta_rule` (gdn_fast.py:37-113) and
trains through it with XLA autodiff, which keeps the forward's residuals for the backward.  Here, when a gradient is
needed, the forward is lsurge_gdn_chunked_fwd_save (the chunk products and the state entering every chunk kept, about
2.25 KiB per token and head) and the backward lsurge_gdn_chunked_bwd_saved.  With SAVE_RESIDUALS = False the forward
keeps only its inputs and the backward lsurge_gdn_chunked_bwd recomputes the rest (less memory, one more forward's
work); the results are bitwise the same.  Without gradients the forward is lsurge_gdn_chunked_fwd.

  fast_chunk_gated_delta_rule(query, key, value, g, beta, chunk_size=64, initial_state=None, ...)
      differentiable op with the reference's signature: query, key [B, T, H, 128], value [B, T, H, 128], g [B, T, H]
      (log decay, float32), beta [B, T, H]; returns (o [B, T, H, 128] in query's dtype, the final state in the compute
      dtype when initial_state is given, else None)
  install(prec, inv, unroll)   the reference's switches (gdn_fast.py:116-125): recorded, the kernels always compute in
      f32 with the exact inverse
With use_qk_norm_in_gdn the query and key heads are l2-normalised first (gdn_fast.py:43-46) by lsurge_l2norm_rows,
whose backward is lsurge_l2norm_rows_bwd.
"""
from __future__ import annotations

import torch

import _lib as L

SAVE_RESIDUALS = True
PREC = "highest"
INV = "solve"
UNROLL = 1
D = 128


class _GdnFn(torch.autograd.Function):

    @staticmethod
    def forward(ctx, q, k, v, g, beta, h0, want_state):
        B, T, H, _ = q.shape
        o = torch.empty_like(v)
        h_out = torch.empty((B, H, D, D), dtype=torch.float32, device=q.device) if want_state else None
        lib = L.lib()
        ctx.saved = None
        if SAVE_RESIDUALS and any(ctx.needs_input_grad[:6]):
            ctx.saved = L.workspace(lib.lsurge_gdn_chunked_saved_bytes(B, T, H, D, D), q.device)
            L.check(lib.lsurge_gdn_chunked_fwd_save(L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(g), L.ptr(beta), B, T, H, D,
                                                    D, L.ptr(h0), L.ptr(o), L.ptr(h_out), L.ptr(ctx.saved),
                                                    ctx.saved.numel(), L.stream(q.device)), "gdn_chunked_fwd_save")
        else:
            ws = L.workspace(lib.lsurge_gdn_chunked_workspace_bytes(B, T, H, D, D), q.device)
            L.check(lib.lsurge_gdn_chunked_fwd(L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(g), L.ptr(beta), B, T, H, D, D,
                                               L.ptr(h0), L.ptr(o), L.ptr(h_out), L.ptr(ws), ws.numel(),
                                               L.stream(q.device)), "gdn_chunked_fwd")
        ctx.save_for_backward(q, k, v, g, beta, h0)
        ctx.has_h0 = h0 is not None
        return (o, h_out) if want_state else (o,)

    @staticmethod
    def backward(ctx, do, dh_final=None):
        q, k, v, g, beta, h0 = ctx.saved_tensors
        B, T, H, _ = q.shape
        do = L.contig(do.to(torch.bfloat16))
        dhf = None if dh_final is None else L.contig(dh_final.to(torch.float32))
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        dg = torch.empty((B, T, H), dtype=torch.float32, device=q.device)
        db = torch.empty_like(dg)
        dh0 = torch.empty((B, H, D, D), dtype=torch.float32, device=q.device) if ctx.has_h0 else None
        lib = L.lib()
        if ctx.saved is not None:
            ws = L.workspace(lib.lsurge_gdn_chunked_bwd_saved_workspace_bytes(B, T, H, D, D), q.device)
            L.check(lib.lsurge_gdn_chunked_bwd_saved(L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(beta), B, T, H, D, D,
                                                     L.ptr(do), L.ptr(dhf), L.ptr(dq), L.ptr(dk), L.ptr(dv), L.ptr(dg),
                                                     L.ptr(db), L.ptr(dh0), L.ptr(ctx.saved), ctx.saved.numel(),
                                                     L.ptr(ws), ws.numel(), L.stream(q.device)), "gdn_chunked_bwd_saved")
            ctx.saved = None
        else:
            ws = L.workspace(lib.lsurge_gdn_chunked_bwd_workspace_bytes(B, T, H, D, D), q.device)
            L.check(lib.lsurge_gdn_chunked_bwd(L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(g), L.ptr(beta), B, T, H, D, D,
                                               L.ptr(h0), L.ptr(do), L.ptr(dhf), L.ptr(dq), L.ptr(dk), L.ptr(dv),
                                               L.ptr(dg), L.ptr(db), L.ptr(dh0), L.ptr(ws), ws.numel(),
                                               L.stream(q.device)), "gdn_chunked_bwd")
        return dq, dk, dv, dg, db, dh0, None


class _L2NormFn(torch.autograd.Function):
    """Row-wise l2 normalisation over the last axis (MaxText l2norm, eps as given), bf16 in and out."""

    @staticmethod
    def forward(ctx, x, eps):
        rows = x.numel() // x.shape[-1]
        y = torch.empty_like(x)
        r = torch.empty(rows, dtype=torch.float32, device=x.device)
        L.check(L.lib().lsurge_l2norm_rows(L.ptr(x), rows, x.shape[-1], float(eps), L.ptr(y), L.ptr(r),
                                           L.stream(x.device)), "l2norm_rows")
        ctx.save_for_backward(x, r)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, r = ctx.saved_tensors
        dy = L.contig(dy.to(torch.bfloat16))
        dx = torch.empty_like(x)
        L.check(L.lib().lsurge_l2norm_rows_bwd(L.ptr(x), L.ptr(dy), L.ptr(r), r.numel(), x.shape[-1], L.ptr(dx),
                                               L.stream(x.device)), "l2norm_rows_bwd")
        return dx, None


def fast_chunk_gated_delta_rule(query, key, value, g, beta, chunk_size=64, initial_state=None,
                                use_qk_norm_in_gdn=False, cp_axis=None, compute_dtype=torch.bfloat16):
    """modal/gdn_fast.py:37-113.  The kernels take chunks of 64, head dims of 128 and the bf16 compute dtype.  With
    use_qk_norm_in_gdn, query and key are l2-normalised over the head dim first (43-46).  The reference normalises in
    the input dtype and casts afterwards; the l2-norm kernel takes bf16, so qk-norm requires bf16 query and key (for
    them the two orders agree) and other dtypes raise ValueError rather than round twice.  The context-parallel
    branch (39-42) is not built and raises NotImplementedError."""
    if cp_axis is not None:
        raise NotImplementedError("fast_chunk_gated_delta_rule: context parallelism (cp_axis) is not built")
    if use_qk_norm_in_gdn and (query.dtype != torch.bfloat16 or key.dtype != torch.bfloat16):
        raise ValueError("fast_chunk_gated_delta_rule: use_qk_norm_in_gdn takes bf16 query and key (got "
                         f"{query.dtype}, {key.dtype}); the reference normalises before its cast, which the bf16 "
                         "l2-norm kernel reproduces only for bf16 inputs")
    if chunk_size != 64 or compute_dtype != torch.bfloat16:
        raise ValueError("fast_chunk_gated_delta_rule: the kernels take chunk_size=64 and a bf16 compute dtype")
    if query.shape[-1] != D or value.shape[-1] != D or key.shape != query.shape:
        raise ValueError(f"fast_chunk_gated_delta_rule: head dims must be {D} (query {tuple(query.shape)}, "
                         f"value {tuple(value.shape)})")
    L.require_cuda(query, key, value, g, beta, initial_state)
    out_dtype = query.dtype
    q, k, v = (L.contig(t.to(torch.bfloat16)) for t in (query, key, value))
    if use_qk_norm_in_gdn:
        q, k = _L2NormFn.apply(q, 1e-6), _L2NormFn.apply(k, 1e-6)
    bt = L.contig(beta.to(torch.bfloat16))
    gf = L.contig(g.to(torch.float32))
    h0 = None if initial_state is None else L.contig(initial_state.to(torch.float32))
    res = _GdnFn.apply(q, k, v, gf, bt, h0, initial_state is not None)
    o = res[0].to(out_dtype)
    return o, (res[1].to(compute_dtype) if initial_state is not None else None)


def install(prec="high", inv="neumann", unroll=1):
    """Record the reference's switches (gdn_fast.py:116-125).  The reference then rebinds MaxText's
    qwen3.jax_chunk_gated_delta_rule; MaxText is a JAX package and absent here, so JAX callers bind the C ABI through
    XLA FFI instead."""
    global PREC, INV, UNROLL
    PREC, INV, UNROLL = prec, inv, int(unroll)
    print(f"[gdn_fast] chunked gated delta rule -> gfx950 kernels (precision={prec} and inverse={inv} recorded; "
          "f32 arithmetic, exact inverse)", flush=True)
