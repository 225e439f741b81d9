"""ctypes wrapper of the C restatement in moe_oracle_c.c (test infrastructure only).

Used by tests and the smoke checker at sizes where the numpy restatement in moe_oracle.py is slow.
Build with `make -C oracle` (done by __graft_entry__.build()).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from . import moe_oracle as mo

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        p, i64 = ctypes.c_void_p, ctypes.c_int64
        L.oracle_router_logits.argtypes = [p, p, p, i64, i64, i64, p]
        L.oracle_topk.argtypes = [p, i64, i64, i64, p]
        L.oracle_layout.argtypes = [p, i64, i64, i64, p, p, p, p, p, p]
        L.oracle_layout.restype = i64
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def router_logits(x, w_r, bias=None):
    """Same values as moe_oracle.router_logits; x, w_r hold bf16 values."""
    xb = np.ascontiguousarray(mo.bf16_bits(x))
    wb = np.ascontiguousarray(mo.bf16_bits(w_r))
    T, d = xb.shape
    E = wb.shape[1]
    out = np.empty((T, E), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().oracle_router_logits(_ptr(xb), _ptr(wb), None if b is None else _ptr(b), T, d, E, _ptr(out))
    return out


def topk(logits, k):
    l = np.ascontiguousarray(logits, np.float32)
    T, E = l.shape
    sel = np.empty((T, k), np.int32)
    lib().oracle_topk(_ptr(l), T, E, k, _ptr(sel))
    return sel


def router(x, w_r, k, bias=None):
    logits = router_logits(x, w_r, bias)
    sel = topk(logits, k)
    return logits, sel, mo.topk_softmax(logits, sel)


def build_layout(sel, E, block=mo.BLOCK):
    flat = np.ascontiguousarray(np.asarray(sel, np.int32).reshape(-1))
    M = flat.shape[0]
    gs, off, boff = (np.empty(E, np.int32) for _ in range(3))
    order, pos, slot = (np.empty(M, np.int32) for _ in range(3))
    nb = lib().oracle_layout(_ptr(flat), M, E, block, _ptr(gs), _ptr(off), _ptr(boff), _ptr(order), _ptr(pos),
                             _ptr(slot))
    nblk = (gs + block - 1) // block
    return dict(group_sizes=gs, offsets=off, block_off=boff, num_blocks=int(nb), order=order, pos=pos, slot=slot,
                block_expert=np.repeat(np.arange(E, dtype=np.int32), nblk))
