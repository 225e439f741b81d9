"""The C-ABI library loads and exports every entry point include/lewi_surge.h declares; host-side argument
checks work without a GPU (they return an error code before any launch)."""
import ctypes
import os
import re

import pytest

import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lewi_surge.h")


def declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(lsurge_[a-z0-9_]+)\s*\(", txt)))


def test_library_built_and_loads():
    assert os.path.exists(L.LIB_PATH), "run __graft_entry__.build() first"
    assert L.lib().lsurge_abi_version() == 3


def test_every_declared_symbol_is_exported_and_bound():
    lib = ctypes.CDLL(L.LIB_PATH)
    names = declared()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(L.exported_symbols())


def test_argument_errors_without_gpu():
    lib = L.lib()
    rc = lib.lsurge_gather_rows(None, -1, 8, L.BF16, None, 4, None, None, None)
    assert rc == -1 and b"negative" in lib.lsurge_last_error()
    rc = lib.lsurge_router_topk(ctypes.c_void_p(16), ctypes.c_void_p(16), None, 4, 8, 300, 6, None,
                                ctypes.c_void_p(16), ctypes.c_void_p(16), None)
    assert rc == -1 and b"bad shape" in lib.lsurge_last_error()
    rc = lib.lsurge_gather_reduce(ctypes.c_void_p(16), 4, 8, 7, ctypes.c_void_p(16), 2, 2, None,
                                  ctypes.c_void_p(16), L.F32, None)
    assert rc == -2  # dtype 7 unknown
    with pytest.raises(RuntimeError, match="unsupported dtype"):
        L.check(rc, "gather_reduce")


def test_sizes():
    lib = L.lib()
    assert lib.lsurge_max_blocks(98304, 64) == 768 + 64
    s = L.MoeShape(16384, 1024, 64, 6, 512, 512)
    saved = lib.lsurge_moe_saved_bytes(ctypes.byref(s))
    # 3 f-wide activations + y_pad over the padded rows dominate (the dispatched rows are gathered from x, not
    # saved)
    p_rows = 128 * (768 + 64)
    assert saved >= p_rows * (1024 + 3 * 512) * 2
    assert saved < p_rows * (2 * 1024 + 3 * 512) * 2
    assert lib.lsurge_moe_bwd_workspace_bytes(ctypes.byref(s)) > 0
    # the FP8 forward adds its E4M3 x [T, d], routed h [P, f] and shared h [T, fs] (and 4 scales) after the bf16
    # layout; the bf16 size does not pay for them
    saved8 = lib.lsurge_moe_saved_bytes_fp8(ctypes.byref(s))
    fp8_tail = 16384 * 1024 + p_rows * 512 + 16384 * 512 + 16  # xq, hq over the routed padded rows, shq, scales
    assert fp8_tail <= saved8 - saved < fp8_tail + 4 * 256
    bad = L.MoeShape(16, 100, 64, 6, 512, 512)  # d not a multiple of 64
    assert lib.lsurge_moe_saved_bytes(ctypes.byref(bad)) == 0
    assert lib.lsurge_moe_saved_bytes_fp8(ctypes.byref(bad)) == 0


def test_fp8_backward_argument_errors_without_gpu():
    lib = L.lib()
    s = L.MoeShape(512, 128, 8, 2, 64, 0)
    fake = ctypes.c_void_p(256)
    p = L.MoeParams(x=fake, w_r=fake)
    g = L.MoeGrads(dx=fake, dw_r=fake, dw_gate=fake, dw_up=fake, dw_down=fake)
    need_w = lib.lsurge_moe_fp8_weights_bytes(ctypes.byref(s))
    assert need_w >= 3 * 8 * 64 * 128 * 2  # forward and backward copies of every expert matrix
    need_ws = lib.lsurge_moe_bwd_fp8_workspace_bytes(ctypes.byref(s))
    assert need_ws > lib.lsurge_moe_bwd_workspace_bytes(ctypes.byref(s))
    rc = lib.lsurge_moe_bwd_fp8(ctypes.byref(s), ctypes.byref(p), fake, need_w - 1, fake, fake, ctypes.byref(g), fake,
                                need_ws, None)
    assert rc != 0 and b"weight buffer" in lib.lsurge_last_error()
    rc = lib.lsurge_moe_bwd_fp8(ctypes.byref(s), ctypes.byref(p), fake, need_w, fake, fake, ctypes.byref(g), fake,
                                need_ws - 1, None)
    assert rc != 0 and b"workspace" in lib.lsurge_last_error()
    rc = lib.lsurge_fp8_cast_transpose(fake, 64, 24, 1, fake, None, 64, fake, fake, 1 << 20, None)
    assert rc != 0 and b"multiple of 16" in lib.lsurge_last_error()
    rc = lib.lsurge_fp8_cast_transpose(fake, 64, 32, 2, fake, None, 64, fake, fake, 1 << 20, None)
    assert rc != 0 and b"format" in lib.lsurge_last_error()


def test_l2norm_argument_errors_without_gpu():
    """lsurge_l2norm_rows / _bwd reject bad shapes and alignment before touching the device."""
    lib = L.lib()
    fake = ctypes.c_void_p(256)
    for rows, dim, eps, msg in ((10, 12, 1e-6, b"multiple of 8"), (10, 520, 1e-6, b"multiple of 8"),
                                (1 << 31, 128, 1e-6, b"rows < 2^31"), (10, 128, -1.0, b"eps >= 0"),
                                (10, 128, float("nan"), b"eps >= 0")):
        assert lib.lsurge_l2norm_rows(fake, rows, dim, eps, fake, None, None) != 0
        assert msg in lib.lsurge_last_error(), lib.lsurge_last_error()
    assert lib.lsurge_l2norm_rows(ctypes.c_void_p(264), 10, 128, 1e-6, fake, None, None) != 0
    assert b"16-byte aligned" in lib.lsurge_last_error()
    assert lib.lsurge_l2norm_rows_bwd(fake, fake, fake, 1 << 31, 128, fake, None) != 0
    assert b"rows < 2^31" in lib.lsurge_last_error()
    assert lib.lsurge_l2norm_rows_bwd(fake, fake, None, 10, 128, fake, None) != 0
    assert b"null pointer" in lib.lsurge_last_error()
    assert lib.lsurge_l2norm_rows(fake, 0, 128, 1e-6, fake, None, None) == 0  # empty: nothing launched


def test_gdn_saved_split_argument_errors_without_gpu():
    """lsurge_gdn_chunked_fwd_save / lsurge_gdn_chunked_bwd_saved check their buffers and shapes before touching the
    device; the saved buffer is smaller than the recomputing backward's workspace, and the two parts add up to it."""
    lib = L.lib()
    fake = ctypes.c_void_p(256)
    B, T, H, D = 2, 200, 3, 128
    saved = lib.lsurge_gdn_chunked_saved_bytes(B, T, H, D, D)
    scratch = lib.lsurge_gdn_chunked_bwd_saved_workspace_bytes(B, T, H, D, D)
    full = lib.lsurge_gdn_chunked_bwd_workspace_bytes(B, T, H, D, D)
    assert 0 < saved < full and saved + scratch == full
    assert lib.lsurge_gdn_chunked_saved_bytes(B, T, H, 64, D) == 0
    rc = lib.lsurge_gdn_chunked_fwd_save(fake, fake, fake, fake, fake, B, T, H, D, D, None, fake, None, fake, saved - 1,
                                         None)
    assert rc != 0 and b"saved buffer" in lib.lsurge_last_error()
    rc = lib.lsurge_gdn_chunked_fwd_save(fake, fake, fake, fake, fake, B, T, H, D, D, None, None, None, fake, saved,
                                         None)
    assert rc != 0 and b"null pointer" in lib.lsurge_last_error()
    rc = lib.lsurge_gdn_chunked_fwd_save(fake, fake, fake, fake, fake, B, T, H, 64, D, None, fake, None, fake, saved,
                                         None)
    assert rc != 0 and b"head dims" in lib.lsurge_last_error()
    args = [fake] * 4 + [B, T, H, D, D, fake, None, fake, fake, fake, fake, fake, None]
    rc = lib.lsurge_gdn_chunked_bwd_saved(*args, fake, saved, fake, scratch - 1, None)
    assert rc != 0 and b"workspace" in lib.lsurge_last_error()
    rc = lib.lsurge_gdn_chunked_bwd_saved(*args, fake, saved - 1, fake, scratch, None)
    assert rc != 0 and b"saved buffer" in lib.lsurge_last_error()
    rc = lib.lsurge_gdn_chunked_bwd_saved(*args, ctypes.c_void_p(264), saved, fake, scratch, None)
    assert rc != 0 and b"16-byte aligned" in lib.lsurge_last_error()
