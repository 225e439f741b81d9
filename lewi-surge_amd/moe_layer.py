"""The whole MoE layer (router top-k -> permute into 128-row expert blocks -> SwiGLU grouped GEMMs -> weighted
combine + shared expert), forward and gather-only backward, as two C-ABI calls into liblewi_surge.so.

This is the fused entry the north-star path needs: the reference composes it from MaxText RoutedMoE (third-party,
not vendored) patched by modal/moe_permute.py (dispatch/combine) and modal/padded_gmm.py (ragged_dot); MaxText
calls ragged_dot once per weight, so SiLU*mul can only be fused into the gate/up GEMM at this level.

Weights follow MaxText's layout: w_gate/w_up = wi_0/wi_1 [E, d, f], w_down = wo [E, f, d] (modal/stage2.py:338),
router w_r [d, E]; shared expert ws_gate/ws_up [d, fs], ws_down [fs, d].

  MoELayer(shape)           buffers sized once; .forward(params) / .backward(params, dy) call the C ABI
  moe_layer(x, ...)         autograd function over the same calls
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

import _lib as L


@dataclass
class MoEShape:
    t: int
    d: int
    e: int
    k: int
    f: int
    fs: int = 0

    def c(self):
        return L.MoeShape(self.t, self.d, self.e, self.k, self.f, self.fs)

    @property
    def m(self):
        return self.t * self.k

    @property
    def max_blocks(self):
        return int(L.lib().lsurge_max_blocks(self.m, self.e))


PARAM_NAMES = ("x", "w_r", "bias", "w_gate", "w_up", "w_down", "ws_gate", "ws_up", "ws_down")
GRAD_NAMES = ("dx", "dw_r", "dw_gate", "dw_up", "dw_down", "dws_gate", "dws_up", "dws_down", "dweights")


def _check_params(s: MoEShape, p: dict):
    want = {"x": (s.t, s.d), "w_r": (s.d, s.e), "w_gate": (s.e, s.d, s.f), "w_up": (s.e, s.d, s.f),
            "w_down": (s.e, s.f, s.d)}
    if s.fs:
        want.update(ws_gate=(s.d, s.fs), ws_up=(s.d, s.fs), ws_down=(s.fs, s.d))
    for n, shp in want.items():
        t = p.get(n)
        if t is None or tuple(t.shape) != shp or t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous():
            got = None if t is None else (tuple(t.shape), t.dtype, t.device)
            raise ValueError(f"moe_layer: {n} must be a contiguous bf16 ROCm tensor of shape {shp}, got {got}")
    b = p.get("bias")
    if b is not None and (tuple(b.shape) != (s.e,) or b.dtype != torch.float32 or not b.is_cuda):
        raise ValueError("moe_layer: bias must be a float32 ROCm tensor of shape (e,)")


def _params_struct(p: dict):
    return L.MoeParams(*[None if p.get(n) is None else p[n].data_ptr() for n in PARAM_NAMES])


class MoELayer:
    """Preallocated buffers for one layer shape on one device; no allocation per call."""

    def __init__(self, shape: MoEShape, device="cuda"):
        self.shape = shape
        self.device = torch.device(device)
        lib = L.lib()
        cs = shape.c()
        self._cs = cs
        nbytes = lib.lsurge_moe_saved_bytes(ctypes.byref(cs))
        if nbytes == 0:
            L.check(-1, "moe_saved_bytes")
        self.saved = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        self.fwd_ws = L.workspace(lib.lsurge_moe_fwd_workspace_bytes(ctypes.byref(cs)), self.device)
        self._bwd_ws = None
        self.out = torch.empty((shape.t, shape.d), dtype=torch.bfloat16, device=self.device)
        self.grads = None

    # -- forward / backward ---------------------------------------------------------------------------------
    def forward(self, p: dict, out=None):
        s = self.shape
        _check_params(s, p)
        out = self.out if out is None else out
        ps = _params_struct(p)
        L.check(L.lib().lsurge_moe_fwd(ctypes.byref(self._cs), ctypes.byref(ps), L.ptr(out), L.ptr(self.saved),
                                       self.saved.numel(), L.ptr(self.fwd_ws), self.fwd_ws.numel(),
                                       L.stream(self.device)), "moe_fwd")
        return out

    # -- FP8 forward (E4M3 expert GEMMs, current scaling) ------------------------------------------------------
    def quantize_weights_fp8(self, p: dict):
        """Quantise the expert and shared weights of p into this layer's FP8 weight buffer (one scale per expert
        and matrix).  Call again whenever the weights change."""
        _check_params(self.shape, p)
        lib = L.lib()
        if getattr(self, "wq", None) is None:
            self.wq = torch.empty(lib.lsurge_moe_fp8_weights_bytes(ctypes.byref(self._cs)), dtype=torch.uint8,
                                  device=self.device)
            self._wq_ws = L.workspace(lib.lsurge_moe_fp8_quantize_weights_workspace_bytes(ctypes.byref(self._cs)),
                                      self.device)
        ps = _params_struct(p)
        L.check(lib.lsurge_moe_fp8_quantize_weights(ctypes.byref(self._cs), ctypes.byref(ps), L.ptr(self.wq),
                                                    self.wq.numel(), L.ptr(self._wq_ws), self._wq_ws.numel(),
                                                    L.stream(self.device)), "moe_fp8_quantize_weights")
        return self.wq

    def forward_fp8(self, p: dict, out=None):
        """forward() with the expert GEMMs in FP8 on the weights of the last quantize_weights_fp8(); the saved
        activations start with the bf16 layout, so backward() (bf16) or backward_fp8() runs after it."""
        s = self.shape
        _check_params(s, p)
        if getattr(self, "wq", None) is None:
            raise RuntimeError("moe_layer: call quantize_weights_fp8() before forward_fp8()")
        lib = L.lib()
        if getattr(self, "_fwd8_ws", None) is None:
            self._fwd8_ws = L.workspace(lib.lsurge_moe_fwd_fp8_workspace_bytes(ctypes.byref(self._cs)), self.device)
            # the FP8 forward also keeps its E4M3 x and h in `saved`, after the bf16 layout
            n8 = lib.lsurge_moe_saved_bytes_fp8(ctypes.byref(self._cs))
            if n8 > self.saved.numel():
                self.saved = torch.empty(n8, dtype=torch.uint8, device=self.device)
        out = self.out if out is None else out
        ps = _params_struct(p)
        L.check(lib.lsurge_moe_fwd_fp8(ctypes.byref(self._cs), ctypes.byref(ps), L.ptr(self.wq), self.wq.numel(),
                                       L.ptr(out), L.ptr(self.saved), self.saved.numel(), L.ptr(self._fwd8_ws),
                                       self._fwd8_ws.numel(), L.stream(self.device)), "moe_fwd_fp8")
        return out

    def alloc_grads(self):
        s = self.shape
        z = lambda *shape: torch.empty(shape, dtype=torch.float32, device=self.device)  # noqa: E731
        g = dict(dx=torch.empty((s.t, s.d), dtype=torch.bfloat16, device=self.device), dw_r=z(s.d, s.e),
                 dw_gate=z(s.e, s.d, s.f), dw_up=z(s.e, s.d, s.f), dw_down=z(s.e, s.f, s.d), dweights=z(s.t, s.k))
        if s.fs:
            g.update(dws_gate=z(s.d, s.fs), dws_up=z(s.d, s.fs), dws_down=z(s.fs, s.d))
        return g

    def backward(self, p: dict, dy, grads=None):
        s = self.shape
        _check_params(s, p)
        if tuple(dy.shape) != (s.t, s.d) or dy.dtype != torch.bfloat16 or not dy.is_contiguous():
            raise ValueError("moe_layer: dy must be a contiguous bf16 [t, d] tensor")
        if grads is None:
            if self.grads is None:
                self.grads = self.alloc_grads()
            grads = self.grads
        if self._bwd_ws is None:
            self._bwd_ws = L.workspace(L.lib().lsurge_moe_bwd_workspace_bytes(ctypes.byref(self._cs)), self.device)
        gs = L.MoeGrads(*[None if grads.get(n) is None else grads[n].data_ptr() for n in GRAD_NAMES])
        ps = _params_struct(p)
        L.check(L.lib().lsurge_moe_bwd(ctypes.byref(self._cs), ctypes.byref(ps), L.ptr(dy), L.ptr(self.saved),
                                       ctypes.byref(gs), L.ptr(self._bwd_ws), self._bwd_ws.numel(),
                                       L.stream(self.device)), "moe_bwd")
        return grads

    def backward_fp8(self, p: dict, dy, grads=None):
        """backward() with the expert GEMMs in FP8 (E5M2 gradients x the E4M3 weights / activations of the forward),
        after forward_fp8() on the same weights; same gradient buffers and dtypes as backward()."""
        s = self.shape
        _check_params(s, p)
        if getattr(self, "wq", None) is None:
            raise RuntimeError("moe_layer: call quantize_weights_fp8() and forward_fp8() before backward_fp8()")
        if tuple(dy.shape) != (s.t, s.d) or dy.dtype != torch.bfloat16 or not dy.is_contiguous():
            raise ValueError("moe_layer: dy must be a contiguous bf16 [t, d] tensor")
        if grads is None:
            if self.grads is None:
                self.grads = self.alloc_grads()
            grads = self.grads
        lib = L.lib()
        if getattr(self, "_bwd8_ws", None) is None:
            self._bwd8_ws = L.workspace(lib.lsurge_moe_bwd_fp8_workspace_bytes(ctypes.byref(self._cs)), self.device)
        gs = L.MoeGrads(*[None if grads.get(n) is None else grads[n].data_ptr() for n in GRAD_NAMES])
        ps = _params_struct(p)
        L.check(lib.lsurge_moe_bwd_fp8(ctypes.byref(self._cs), ctypes.byref(ps), L.ptr(self.wq), self.wq.numel(),
                                       L.ptr(dy), L.ptr(self.saved), ctypes.byref(gs), L.ptr(self._bwd8_ws),
                                       self._bwd8_ws.numel(), L.stream(self.device)), "moe_bwd_fp8")
        return grads

    # -- views of the saved routing data / activations (device tensors) ----------------------------------------
    def views(self):
        s = self.shape
        v = L.MoeSavedViews()
        L.check(L.lib().lsurge_moe_saved_layout(ctypes.byref(self._cs), L.ptr(self.saved), ctypes.byref(v)),
                "moe_saved_layout")
        base = self.saved.data_ptr()
        mb = s.max_blocks
        p_rows = 128 * mb

        def view(name, dtype, shape):
            off = getattr(v, name) - base
            n = 1
            for x in shape:
                n *= x
            nbytes = n * torch.tensor([], dtype=dtype).element_size()
            return self.saved[off:off + nbytes].view(dtype).view(*shape)

        i32, f32, b16 = torch.int32, torch.float32, torch.bfloat16
        return dict(
            logits=view("logits", f32, (s.t, s.e)), sel=view("sel", i32, (s.t, s.k)),
            weights=view("weights", f32, (s.t, s.k)), group_sizes=view("group_sizes", i32, (s.e,)),
            offsets=view("offsets", i32, (s.e,)), block_off=view("block_off", i32, (s.e,)),
            order=view("order", i32, (s.m,)), pos=view("pos", i32, (s.m,)), slot=view("slot", i32, (s.m,)),
            row_src=view("row_src", i32, (p_rows,)), blk_expert=view("blk_expert", i32, (mb,)),
            blk_rows=view("blk_rows", i32, (mb,)), num_blocks=view("num_blocks", i32, (1,)),
            h_gate=view("h_gate", b16, (p_rows, s.f)),
            h_up=view("h_up", b16, (p_rows, s.f)), h=view("h", b16, (p_rows, s.f)),
            y_pad=view("y_pad", b16, (p_rows, s.d)))


class _MoEFn(torch.autograd.Function):

    @staticmethod
    def forward(ctx, k, bias, x, w_r, w_gate, w_up, w_down, ws_gate, ws_up, ws_down):
        e, d, f = w_gate.shape
        fs = 0 if ws_gate is None else ws_gate.shape[1]
        layer = MoELayer(MoEShape(x.shape[0], d, e, k, f, fs), x.device)
        p = dict(x=x, w_r=w_r, bias=bias, w_gate=w_gate, w_up=w_up, w_down=w_down, ws_gate=ws_gate, ws_up=ws_up,
                 ws_down=ws_down)
        out = layer.forward(p, out=torch.empty_like(x))
        ctx.layer, ctx.p = layer, p
        return out

    @staticmethod
    def backward(ctx, dy):
        g = ctx.layer.backward(ctx.p, L.contig(dy.to(torch.bfloat16)))
        p = ctx.p
        cast = lambda name, ref: None if ref is None else g[name].to(ref.dtype)  # noqa: E731
        return (None, None, g["dx"], cast("dw_r", p["w_r"]), cast("dw_gate", p["w_gate"]), cast("dw_up", p["w_up"]),
                cast("dw_down", p["w_down"]), cast("dws_gate", p["ws_gate"]), cast("dws_up", p["ws_up"]),
                cast("dws_down", p["ws_down"]))


def moe_layer(x, w_r, w_gate, w_up, w_down, ws_gate=None, ws_up=None, ws_down=None, bias=None, k=6):
    """Differentiable MoE layer: out [T, d] bf16 (see module docstring)."""
    return _MoEFn.apply(k, bias, x, w_r, w_gate, w_up, w_down, ws_gate, ws_up, ws_down)
