"""lsurge_ragged_dot_noalloc (the grouped GEMM with its block table in the library's static device array) against
lsurge_ragged_dot with a caller workspace: bitwise equal outputs on two calls in a row, the second smaller (the
array keeps the first call's table, which the second must fully overwrite where it reads), plus the size limit."""
import ctypes

import numpy as np
import pytest
import torch

import _lib as L
from oracle import moe_oracle as mo

pytestmark = pytest.mark.gpu


def _case(gs, K, N, dt, dev, seed):
    rng = np.random.default_rng(seed)
    M = int(sum(gs)) + 5  # tail rows past the groups: zeros
    E = len(gs)
    rnd = mo.round_bf16 if dt == torch.bfloat16 else (lambda v: v.astype(np.float16).astype(np.float32))
    a = torch.from_numpy(rnd(rng.standard_normal((M, K)).astype(np.float32))).to(dev).to(dt)
    b = torch.from_numpy(rnd(rng.standard_normal((E, K, N)).astype(np.float32))).to(dev).to(dt)
    return a, b, torch.tensor(gs, dtype=torch.int32, device=dev), M, E


def _both(a, b, gst, M, K, N, E, out_dt, dev):
    lib = L.lib()
    st = L.stream(dev)
    want = torch.full((M, N), 7, dtype=out_dt, device=dev)
    got = torch.full((M, N), 3, dtype=out_dt, device=dev)
    ws = L.workspace(lib.lsurge_ragged_dot_workspace_bytes(M, E), dev)
    L.check(lib.lsurge_ragged_dot(L.ptr(a), L.ptr(b), L.ptr(gst), M, K, N, E, L.dt(a), L.ptr(want), L.dt(want),
                                  L.ptr(ws), ws.numel(), st), "ragged_dot")
    L.check(lib.lsurge_ragged_dot_noalloc(L.ptr(a), L.ptr(b), L.ptr(gst), M, K, N, E, L.dt(a), L.ptr(got), L.dt(got),
                                          st), "ragged_dot_noalloc")
    torch.cuda.synchronize()
    return got, want


@pytest.mark.parametrize("dt,out_f32", [(torch.bfloat16, False), (torch.float16, False), (torch.bfloat16, True)])
def test_noalloc_matches_workspace_entry_point(dt, out_f32, dev):
    # first call: 300 groups with a hot one (many blocks); second call: 5 groups, fewer rows and blocks
    rng = np.random.default_rng(2)
    gs1 = [int(v) for v in rng.integers(0, 300, 300)]
    gs1[7] = 9000
    calls = [(gs1, 256, 192), ([40, 0, 260, 1, 128], 128, 64)]
    for i, (gs, K, N) in enumerate(calls):
        a, b, gst, M, E = _case(gs, K, N, dt, dev, seed=i)
        out_dt = torch.float32 if out_f32 else dt
        got, want = _both(a, b, gst, M, K, N, E, out_dt, dev)
        assert torch.equal(got, want), i
        S = sum(gs)
        assert not got[S:].any()
        ref = mo.ragged_dot(a.float().cpu().numpy(), b.float().cpu().numpy(), gs)
        assert mo.rel_l2(got.float().cpu().numpy(), ref) < 5e-3


def test_noalloc_limits(dev):
    lib = L.lib()
    assert lib.lsurge_ragged_dot_noalloc_max_rows() == 1 << 21
    assert lib.lsurge_ragged_dot_noalloc_max_groups() == 1024
    p = ctypes.c_void_p(16)  # never dereferenced: the size check returns first
    rc = lib.lsurge_ragged_dot_noalloc(p, p, p, (1 << 21) + 1, 64, 64, 8, L.BF16, p, L.BF16, L.stream(dev))
    assert rc == -1 and b"static scratch" in lib.lsurge_last_error()
    rc = lib.lsurge_ragged_dot_noalloc(p, p, p, 1024, 64, 64, 1025, L.BF16, p, L.BF16, L.stream(dev))
    assert rc == -1 and b"static scratch" in lib.lsurge_last_error()
