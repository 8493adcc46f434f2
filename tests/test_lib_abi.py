"""The C-ABI library loads and exports every symbol include/nsw.h declares;
host-side argument validation works without a GPU (no kernel is launched:
every call below fails validation before any HIP call)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "nsw.h")


def declared_functions():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(nsw_[a-z0-9_]+)\s*\(", txt)))


@pytest.fixture(scope="module")
def L():
    from nsw import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libnsw.so is not built: run python neural-scaling-weather_amd/build.py")
    return _lib.lib()


def test_header_declares_the_abi():
    fns = declared_functions()
    for f in ["nsw_swin_block_forward", "nsw_window_attention", "nsw_linear", "nsw_qkv_projection",
              "nsw_rmsnorm_roll_partition", "nsw_proj_reverse_residual", "nsw_weighted_metrics",
              "nsw_last_error", "nsw_block_workspace_size", "nsw_swin_blocks_forward",
              "nsw_blocks_workspace_size", "nsw_window_partition_sumsq"]:
        assert f in fns


def test_every_declared_symbol_is_exported(L):
    from nsw import _lib
    for f in declared_functions():
        assert hasattr(L, f), f"{f} missing from libnsw.so"
        assert f in _lib.SIGNATURES, f"{f} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(declared_functions())


def test_version_and_error_string(L):
    assert L.nsw_version() >= 1
    assert isinstance(L.nsw_last_error(), bytes)


def test_workspace_sizes_are_host_only(L):
    from nsw import _lib
    s = _lib.BlockShape(1, 1, 180, 360, 1024, 16, 9, 18, 4, 9, 4096, 1e-7, _lib.NSW_DTYPE_BF16)
    M = 180 * 360
    n = L.nsw_block_workspace_size(s)
    parts = 1024 * 2 // 512                      # row sums of squares: one float per 512 B of h1 row
    assert L.nsw_row_sumsq_parts(1024, _lib.NSW_DTYPE_BF16) == parts
    assert L.nsw_row_sumsq_parts(1024, _lib.NSW_DTYPE_F32) == 8
    # the larger of the two block forms: the one-block window-order chain
    # (two row buffers, qkv / u, o, h1, two sums arrays) when both norms are folded
    assert n == L.nsw_blocks_workspace_size(ctypes.byref(s), 1)
    assert n >= M * (4 * 1024 + 4096) * 2 + 2 * M * parts * 4
    assert n < M * (4 * 1024 + 4096) * 2 + 2 * M * parts * 4 + 8 * 256
    assert L.nsw_weighted_metrics_workspace_size(70, 720, 1440) > 0
    bad = _lib.BlockShape(0, 1, 180, 360, 1024, 16, 9, 18, 4, 9, 4096, 1e-7, 1)
    assert L.nsw_block_workspace_size(bad) == 0


def test_validation_errors_without_gpu(L):
    from nsw import _lib
    # K not a multiple of the k tile
    rc = L.nsw_linear(16, 16, None, None, 16, 10, 8, 3, 0, _lib.NSW_DTYPE_BF16, None)
    assert rc == _lib.NSW_ERR_INVALID and b"multiple" in L.nsw_last_error()
    # unknown epilogue
    rc = L.nsw_linear(16, 16, 16, None, 16, 10, 8, 64, 99, _lib.NSW_DTYPE_BF16, None)
    assert rc == _lib.NSW_ERR_INVALID
    # window does not divide the image
    rc = L.nsw_window_partition(16, 16, 1, 1, 10, 10, 8, 3, 3, _lib.NSW_DTYPE_F32, None)
    assert rc == _lib.NSW_ERR_INVALID and b"divisible" in L.nsw_last_error()
    # unsupported head dim for the fused q/k norm
    rc = L.nsw_qkv_projection(16, 16, 16, 16, 16, 1e-7, 16, 10, 192, 2, _lib.NSW_DTYPE_BF16, None)
    assert rc == _lib.NSW_ERR_INVALID and b"head_dim" in L.nsw_last_error()
    # weighted metrics: bad weight shape
    rc = L.nsw_weighted_metrics(16, 16, 16, 7, None, 70, 8, 16, 70, 16, None, 16, 1 << 20, None)
    assert rc == _lib.NSW_ERR_INVALID
    # block: aliasing input and output
    shp = _lib.BlockShape(1, 1, 18, 36, 64, 2, 9, 18, 4, 9, 256, 1e-7, _lib.NSW_DTYPE_F32)
    prm = _lib.BlockParams()
    rc = L.nsw_swin_block_forward(16, 16, ctypes.byref(prm), ctypes.byref(shp), 16, 1 << 30, None)
    assert rc == _lib.NSW_ERR_INVALID and b"alias" in L.nsw_last_error()
    # block: norm1 folded without norm2 (the window-order chain needs both)
    prm = _lib.BlockParams()
    prm.wqkv_n1 = 16
    rc = L.nsw_swin_block_forward(16, 32, ctypes.byref(prm), ctypes.byref(shp), 16, 1 << 40, None)
    assert rc == _lib.NSW_ERR_INVALID and b"w1_n2" in L.nsw_last_error()


def test_blocks_chain_validation_without_gpu(L):
    """nsw_swin_blocks_forward refuses malformed stacks before any launch."""
    from nsw import _lib
    shapes = (_lib.BlockShape * 2)(_lib.BlockShape(1, 1, 18, 36, 128, 2, 9, 18, 0, 0, 512, 1e-7, 1),
                                   _lib.BlockShape(1, 1, 18, 36, 128, 2, 9, 18, 4, 9, 512, 1e-7, 1))
    params = (_lib.BlockParams * 2)()
    for i in range(2):
        params[i].wqkv_n1 = params[i].w1_n2 = 16
    ws = 1 << 30
    # depth 0
    rc = L.nsw_swin_blocks_forward(16, 32, params, shapes, 0, 16, ws, None)
    assert rc == _lib.NSW_ERR_INVALID and b"depth" in L.nsw_last_error()
    # the folded weights are required
    params[1].w1_n2 = None
    rc = L.nsw_swin_blocks_forward(16, 32, params, shapes, 2, 16, ws, None)
    assert rc == _lib.NSW_ERR_INVALID and b"norm-folded" in L.nsw_last_error()
    params[1].w1_n2 = 16
    # all blocks share one geometry (shift aside)
    shapes[1].C = 256
    rc = L.nsw_swin_blocks_forward(16, 32, params, shapes, 2, 16, ws, None)
    assert rc == _lib.NSW_ERR_INVALID and b"differs" in L.nsw_last_error()
    shapes[1].C = 128
    # workspace too small
    need = L.nsw_blocks_workspace_size(shapes, 2)
    rc = L.nsw_swin_blocks_forward(16, 32, params, shapes, 2, 16, need - 1, None)
    assert rc == _lib.NSW_ERR_INVALID and b"workspace" in L.nsw_last_error()
    # two window-order row buffers, qkv/u, o, h1 and two sums-of-squares arrays
    M, C, Hm, parts = 18 * 36, 128, 512, 1        # qkv and u share one buffer of max(3C, Hm) columns
    assert need >= M * C * 2 * 4 + M * Hm * 2 + 2 * M * parts * 4
    assert need < M * C * 2 * 4 + M * Hm * 2 + 2 * M * parts * 4 + 8 * 256
    assert L.nsw_blocks_workspace_size(shapes, 0) == 0


def test_fastdiv_selftest(L):
    """The exact division by launch constants used by every window <-> token
    row map matches '/' (host-side check, no GPU)."""
    assert L.nsw_selftest_fastdiv() == 0


def test_gemm_stamps_only_in_the_stamps_build(L):
    """The default library has no phase stamps: the reader refuses (no HIP
    call is made)."""
    from nsw import _lib
    buf = (ctypes.c_uint64 * 8)()
    assert L.nsw_gemm_read_stamps(ctypes.addressof(buf), ctypes.sizeof(buf)) == _lib.NSW_ERR_UNSUPPORTED
    assert b"--stamps" in L.nsw_last_error()


def test_token_count_limit(L):
    from nsw import _lib
    # the row maps index tokens in 32 bits: 2^31 tokens and more are refused
    rc = L.nsw_window_partition(16, 16, 1 << 15, 1, 256, 256, 8, 8, 8, _lib.NSW_DTYPE_BF16, None)
    assert rc == _lib.NSW_ERR_INVALID and b"2^31" in L.nsw_last_error()


def test_ops_refuse_cpu_tensors():
    import torch
    from nsw import ops
    x = torch.zeros(1, 1, 18, 36, 8)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.window_partition(x, (9, 18))
