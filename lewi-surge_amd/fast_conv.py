"""Causal depthwise Conv1D of the Gated DeltaNet block on the HIP library (mirrors modal/fast_conv.py).

The reference replaces flax `nnx.Conv(padding="CAUSAL", feature_group_count=C)` on [B, T, C] inputs by K shifted
multiply-adds (fast_conv.py:14-31):  y[b, t, c] = sum_{j<K} w[j, 0, c] x[b, t-(K-1)+j, c].  Here the same operator is
one memory-bound kernel each way (lsurge_causal_conv1d / lsurge_causal_conv1d_bwd): x read once, y written once,
products accumulated in f32 with one rounding.

  applies(...)                 the reference's eligibility test (fast_conv.py:17-22)
  causal_conv1d(inputs, kernel) differentiable op: inputs [B, T, C] bf16, kernel [K, 1, C] (or [K, C]) bf16
"""
from __future__ import annotations


import torch

import _lib as L


def applies(kernel_size, feature_group_count, in_features, out_features, padding, ndim, has_bias=False,
            dilation=1, strides=1):
    """Shapes the reference's fast path takes (modal/fast_conv.py:17-22); the others go to the original Conv."""
    k = kernel_size if isinstance(kernel_size, (tuple, list)) else (kernel_size,)
    depthwise = feature_group_count == in_features == out_features
    return (len(k) == 1 and depthwise and padding == "CAUSAL" and ndim == 3 and not has_bias
            and dilation in (1, (1,), None) and strides in (1, (1,), None))


def _check(x, w):
    if x.dim() != 3 or x.dtype != torch.bfloat16 or not x.is_cuda:
        raise ValueError("causal_conv1d: inputs must be a [B, T, C] bf16 ROCm tensor")
    if w.dim() == 3:
        w = w.reshape(w.shape[0], w.shape[2])
    if w.dim() != 2 or w.shape[1] != x.shape[2]:
        raise ValueError("causal_conv1d: kernel must be [K, 1, C] or [K, C] with C = inputs.shape[-1]")
    return L.contig(x), L.contig(w.to(torch.bfloat16))


class _ConvFn(torch.autograd.Function):

    @staticmethod
    def forward(ctx, x, w):
        B, T, C = x.shape
        y = torch.empty_like(x)
        L.check(L.lib().lsurge_causal_conv1d(L.ptr(x), L.ptr(w), B, T, C, w.shape[0], L.ptr(y), L.stream(x.device)),
                "causal_conv1d")
        ctx.save_for_backward(x, w)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        B, T, C = x.shape
        K = w.shape[0]
        dy = L.contig(dy.to(torch.bfloat16))
        dx = torch.empty_like(x)
        dw = torch.empty((K, C), dtype=torch.float32, device=x.device)
        lib = L.lib()
        ws = L.workspace(lib.lsurge_causal_conv1d_bwd_workspace_bytes(B, T, C, K), x.device)
        L.check(lib.lsurge_causal_conv1d_bwd(L.ptr(x), L.ptr(w), L.ptr(dy), B, T, C, K, L.ptr(dx), L.ptr(dw),
                                             L.ptr(ws), ws.numel(), L.stream(x.device)), "causal_conv1d_bwd")
        return dx, dw.to(w.dtype)


def causal_conv1d(inputs, kernel):
    """y = causal depthwise conv of inputs [B, T, C] with kernel [K, 1, C] (modal/fast_conv.py:24-31)."""
    x, w = _check(inputs, kernel)
    y = _ConvFn.apply(x, w)
    return y
