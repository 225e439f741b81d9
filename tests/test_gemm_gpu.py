"""Grouped GEMM (padded_gmm.padded_ragged_dot surface) on the GPU against the oracle's dropless ragged_dot.

The reference's known-answer case is modal/te_run.py:72-79: gs=[5,0,9,3,7,1,6,4], M = sum(gs)+3 (tail rows past
the groups), K=64, N=48, bf16, forward + dlhs + drhs.  Tolerance: 2e-2 relative L2 against the fp64 oracle
(north-star tolerance); in practice bf16 inputs with f32 accumulation land near 1e-3.
"""
import numpy as np
import pytest
import torch

import padded_gmm as pg
from oracle import moe_oracle as mo

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _bf(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(torch.bfloat16)


def run_case(gs, M, K, N, dev, seed=0, out_dtype=None, dt=torch.bfloat16):
    """Forward and backward of padded_ragged_dot on operands of dtype dt (bf16 or f16) against the fp64 oracle."""
    rng = np.random.default_rng(seed)
    E = len(gs)
    rnd = mo.round_bf16 if dt == torch.bfloat16 else (lambda v: v.astype(np.float16).astype(np.float32))
    a = rnd(rng.standard_normal((M, K)).astype(np.float32))
    b = rnd(rng.standard_normal((E, K, N)).astype(np.float32))
    g = rnd(rng.standard_normal((M, N)).astype(np.float32))
    tdev = lambda v: torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(dev).to(dt)  # noqa: E731
    at = tdev(a).requires_grad_(True)
    bt = tdev(b).requires_grad_(True)
    gst = torch.tensor(gs, dtype=torch.int32, device=dev)
    out = pg.padded_ragged_dot(at, bt, gst, preferred_element_type=out_dtype)
    assert out.dtype == (out_dtype or dt)
    out.backward(tdev(g).to(out.dtype))
    want = mo.ragged_dot(a, b, gs)
    S = int(np.sum(gs))
    got = out.detach().float().cpu().numpy()
    assert np.all(got[S:] == 0)
    assert mo.rel_l2(got, want) < TOL
    dl, dr = mo.ragged_dot_bwd(a, b, gs, g)
    gl = at.grad.float().cpu().numpy()
    assert np.all(gl[S:] == 0)
    assert mo.rel_l2(gl, dl) < TOL
    gr = bt.grad.float().cpu().numpy()
    for e in range(E):
        if gs[e] == 0:
            assert np.all(gr[e] == 0)
    assert mo.rel_l2(gr, dr) < TOL
    return mo.rel_l2(got, want)


def test_te_known_answer_case(dev):
    gs = [5, 0, 9, 3, 7, 1, 6, 4]
    err = run_case(gs, sum(gs) + 3, 64, 48, dev)
    assert err < 5e-3


def test_f32_output(dev):
    gs = [5, 0, 9, 3, 7, 1, 6, 4]
    run_case(gs, sum(gs) + 3, 64, 48, dev, out_dtype=torch.float32)


@pytest.mark.parametrize("gs,M,K,N,out_dtype", [([5, 0, 9, 3, 7, 1, 6, 4], 38, 64, 48, None),
                                                ([5, 0, 9, 3, 7, 1, 6, 4], 38, 64, 48, torch.float32),
                                                ([700, 0, 1300, 20, 5000], 7100, 512, 1024, None),
                                                ([1536] * 16, 24576, 1024, 512, None)])
def test_f16_operands(gs, M, K, N, out_dtype, dev):
    """f16 lhs / rhs (the reference's einsum runs in lhs.dtype, modal/padded_gmm.py:67): v_mfma_f32_32x32x16_f16,
    f16 or f32 output, dlhs in f16, drhs f32 -- including a group big enough for the chunked weight gradient."""
    err = run_case(gs, M, K, N, dev, seed=3, out_dtype=out_dtype, dt=torch.float16)
    assert err < 5e-3


F32_TOL = 1e-5  # the reference's f32 tolerance, max-normalised (modal/test_moe_permute.py:27-31, 44)


def max_err(got, want):
    """max |got - want| / (max |want| + 1e-6), the reference's check (modal/test_moe_permute.py:27-31)."""
    return float(np.abs(got - want).max() / (np.abs(want).max() + 1e-6)) if want.size else 0.0


def run_case_f32(gs, M, K, N, dev, seed=0, out_dtype=None, offset=0):
    """float32 operands (split into bf16 terms on the device) against the fp64 oracle, forward and backward.
    offset > 0 starts lhs and rhs `offset` floats into their storage (not 16-byte aligned)."""
    rng = np.random.default_rng(seed)
    E = len(gs)
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((E, K, N)).astype(np.float32)
    g = rng.standard_normal((M, N)).astype(np.float32)

    def tdev(v):
        flat = torch.zeros(v.size + offset, dtype=torch.float32, device=dev)
        t = flat[offset:].view(v.shape)
        t.copy_(torch.from_numpy(v))
        return t

    at = tdev(a).requires_grad_(True)
    bt = tdev(b).requires_grad_(True)
    gst = torch.tensor(gs, dtype=torch.int32, device=dev)
    out = pg.padded_ragged_dot(at, bt, gst, preferred_element_type=out_dtype)
    assert out.dtype == (out_dtype or torch.float32)
    out.backward(tdev(g).to(out.dtype))
    S = int(np.sum(gs))
    got = out.detach().float().cpu().numpy()
    gl = at.grad.cpu().numpy()
    gr = bt.grad.cpu().numpy()
    assert at.grad.dtype == torch.float32 and bt.grad.dtype == torch.float32
    assert np.all(got[S:] == 0) and np.all(gl[S:] == 0)
    for e in range(E):
        if gs[e] == 0:
            assert np.all(gr[e] == 0)
    want = mo.ragged_dot(a, b, gs)
    gw = mo.round_bf16(g) if out_dtype == torch.bfloat16 else g
    dl, dr = mo.ragged_dot_bwd(a, b, gs, gw)
    return max_err(got, want), max_err(gl, dl), max_err(gr, dr)


@pytest.mark.parametrize("gs,M,K,N", [
    ([5, 0, 9, 3, 7, 1, 6, 4], 38, 64, 48),              # modal/te_run.py:72-79's case list, f32
    ([300, 0, 517, 1, 255, 256, 257], 1700, 192, 200),   # K of 3 stages (x6 = 18), N tail inside a tile
    ([1536] * 16, 24576, 1024, 512),                     # the dense shape of modal/gemm_bench.py:25-41
    ([0, 8000, 0, 995], 9000, 128, 64),                  # hot group: the chunked weight gradient over 6 m rows
    ([0, 0], 3, 64, 32),                                 # no rows in any group
])
def test_f32_operands(gs, M, K, N, dev):
    """f32 lhs / rhs (the reference's einsum runs in lhs.dtype, modal/padded_gmm.py:67-68) against the fp64 oracle
    at the reference's f32 tolerance, forward, dlhs and drhs."""
    errs = run_case_f32(gs, M, K, N, dev, seed=M + K)
    assert max(errs) <= F32_TOL, errs


def test_f32_operands_many_groups(dev):
    """E > 256: the f32 weight gradient without the chunk table (one slice per group)."""
    rng = np.random.default_rng(5)
    gs = rng.integers(0, 20, 300).tolist()
    errs = run_case_f32(gs, int(np.sum(gs)) + 7, 64, 32, dev, seed=9)
    assert max(errs) <= F32_TOL, errs


def test_f32_operands_unaligned_and_bf16_out(dev):
    """lhs / rhs starting 4 bytes into their storage (copied to aligned memory first), and bf16 output of f32
    operands (the output rounding bounds the forward; the gradients stay f32)."""
    gs = [100, 0, 57, 230]
    errs = run_case_f32(gs, 400, 128, 96, dev, seed=2, offset=1)
    assert max(errs) <= F32_TOL, errs
    errs = run_case_f32(gs, 400, 128, 96, dev, seed=2, out_dtype=torch.bfloat16)
    assert errs[0] <= 8e-3 and max(errs[1:]) <= F32_TOL, errs


def test_f32_operands_reject_f16_output(dev):
    a = torch.zeros((16, 64), dtype=torch.float32, device=dev)
    b = torch.zeros((2, 64, 32), dtype=torch.float32, device=dev)
    with pytest.raises(TypeError, match="preferred_element_type"):
        pg.padded_ragged_dot(a, b, torch.tensor([8, 8], dtype=torch.int32, device=dev),
                             preferred_element_type=torch.float16)


@pytest.mark.parametrize("E,M,K,N", [(8, 1000, 256, 192), (4, 777, 128, 1024), (64, 6000, 1024, 512),
                                     (3, 129, 520, 136),
                                     # fewer weight-gradient chunks than XCDs: the tiles of one chunk are dealt over
                                     # every XCD, the shares cut inside a row of tiles
                                     (1, 3000, 768, 1024), (2, 2500, 1280, 768)])
def test_random_groups(E, M, K, N, dev):
    rng = np.random.default_rng(M)
    cuts = np.sort(rng.integers(0, M - 5, E - 1))
    gs = np.diff(np.concatenate([[0], cuts, [M - 5]])).astype(int).tolist()  # 5 tail rows, some empty groups
    run_case(gs, M, K, N, dev, seed=E)


def test_all_rows_one_group_and_capacity_semantics(dev):
    """One hot group past padded_gmm's capacity: the reference would drop rows, the kernel is dropless."""
    gs = [0, 700, 0, 20]
    M = 720
    c = pg.capacity(M, 4, 1.5)
    assert c < 700
    run_case(gs, M, 128, 64, dev, seed=3)


def test_perm_gather_sentinel(dev):
    """_perm_gather: y[i] = x_ext[idx[i]] with a zero row at index len(x); backward is the inverse gather."""
    x = torch.randn(6, 16, device=dev).to(torch.bfloat16).requires_grad_(True)
    idx = torch.tensor([3, 6, 0, 6, 5, 1, 2, 4], dtype=torch.int32, device=dev)
    inv = torch.tensor([2, 5, 6, 0, 7, 4], dtype=torch.int32, device=dev)
    y = pg._perm_gather(x, idx, inv)
    xe = torch.cat([x.detach(), torch.zeros(1, 16, device=dev, dtype=x.dtype)])
    assert torch.equal(y.detach(), xe[idx.long()])
    g = torch.randn(8, 16, device=dev).to(torch.bfloat16)
    y.backward(g)
    assert torch.equal(x.grad, g[inv.long()])


def test_hot_group_chunked_weight_gradient(dev):
    """A group far above the mean (8000 of 9000 rows): drhs cuts it into row chunks summed from partials."""
    gs = [0, 8000, 0, 995]
    run_case(gs, 9000, 128, 64, dev, seed=11)


def test_many_groups_block_table(dev):
    """1500 groups: the block-table scan takes two passes of 1024 groups; drhs takes one slice per group (E > 256)."""
    rng = np.random.default_rng(7)
    gs = rng.integers(0, 5, 1500).tolist()
    run_case(gs, int(np.sum(gs)) + 7, 64, 64, dev, seed=12)


def test_ragged_bwd_forward_sized_workspace(dev):
    """lsurge_ragged_dot_bwd also accepts the forward's workspace size (one slice per group, no chunk partials)."""
    import _lib as L
    gs = [0, 8000, 0, 995]
    M, K, N, E = 9000, 128, 64, 4
    rng = np.random.default_rng(13)
    a = mo.round_bf16(rng.standard_normal((M, K)).astype(np.float32))
    b = mo.round_bf16(rng.standard_normal((E, K, N)).astype(np.float32))
    g = mo.round_bf16(rng.standard_normal((M, N)).astype(np.float32))
    at, bt, gt = _bf(a, dev), _bf(b, dev), _bf(g, dev)
    gst = torch.tensor(gs, dtype=torch.int32, device=dev)
    lib = L.lib()
    outs = []
    for nbytes in (lib.lsurge_ragged_dot_workspace_bytes(M, E), lib.lsurge_ragged_dot_bwd_workspace_bytes(M, K, N, E)):
        ws = L.workspace(nbytes, dev)
        dl = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
        dr = torch.empty((E, K, N), dtype=torch.float32, device=dev)
        L.check(lib.lsurge_ragged_dot_bwd(L.ptr(at), L.ptr(bt), L.ptr(gst), L.ptr(gt), M, K, N, E, L.BF16, L.ptr(dl), L.ptr(dr),
                                          L.ptr(ws), ws.numel(), L.stream(dev)), "ragged_dot_bwd")
        outs.append((dl.float().cpu().numpy(), dr.cpu().numpy()))
    want_l, want_r = mo.ragged_dot_bwd(a, b, gs, g)
    for dl, dr in outs:
        assert mo.rel_l2(dl, want_l) < TOL and mo.rel_l2(dr, want_r) < TOL
    assert np.array_equal(outs[0][0], outs[1][0])  # dlhs does not depend on the workspace


def test_large_table_grid_fill(dev):
    """m past 2^22 rows: the block table (over 32768 entries) is filled by the grid kernel instead of the group
    workgroup; forward against the fp64 oracle on every row, and the rows past the groups are zero."""
    gs = [3 << 20, 7, 0, (1 << 21) + 999, 12345]
    M, K, N = int(np.sum(gs)) + 300, 16, 8
    rng = np.random.default_rng(21)
    a = mo.round_bf16(rng.standard_normal((M, K)).astype(np.float32))
    b = mo.round_bf16(rng.standard_normal((len(gs), K, N)).astype(np.float32))
    out = pg.padded_ragged_dot(_bf(a, dev), _bf(b, dev), torch.tensor(gs, dtype=torch.int32, device=dev),
                               preferred_element_type=torch.float32)
    got = out.cpu().numpy()
    S = int(np.sum(gs))
    assert np.all(got[S:] == 0)
    want = mo.ragged_dot(a, b, gs)
    assert mo.rel_l2(got, want) < 5e-3


def test_mfma_rate_probe(dev):
    """The calibration kernel of the bench: zero operands leave every accumulator 0; pseudo-random ones give finite,
    nonzero per-lane sums that do not depend on the run (the operands are a hash of the element index)."""
    import _lib as L
    out = torch.empty(L.lib().lsurge_mfma_rate_probe_out_floats(), dtype=torch.float32, device=dev)
    L.check(L.lib().lsurge_mfma_rate_probe(1, 3, L.ptr(out), L.stream(dev)), "mfma_rate_probe")
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0
    runs = []
    for _ in range(2):
        L.check(L.lib().lsurge_mfma_rate_probe(0, 3, L.ptr(out), L.stream(dev)), "mfma_rate_probe")
        torch.cuda.synchronize()
        runs.append(out.clone())
    assert torch.isfinite(runs[0]).all() and torch.count_nonzero(runs[0]).item() == out.numel()
    assert torch.equal(runs[0], runs[1])
    assert L.lib().lsurge_mfma_rate_probe(0, 0, L.ptr(out), L.stream(dev)) == -1  # iters out of range
