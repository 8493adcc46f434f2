"""ctypes binding of libnsw.so (the C ABI declared in include/nsw.h).

The library is loaded lazily on first use.  There is no fallback: if
``libnsw.so`` is missing every op raises, naming the build command.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnsw.so")

NSW_OK = 0
NSW_ERR_INVALID = 1
NSW_ERR_UNSUPPORTED = 2
NSW_ERR_HIP = 3

NSW_DTYPE_F32 = 0
NSW_DTYPE_BF16 = 1

NSW_EPI_NONE = 0
NSW_EPI_BIAS = 1
NSW_EPI_BIAS_GELU = 2
NSW_EPI_BIAS_RESIDUAL = 3
NSW_EPI_BIAS_GELU_TANH = 4
NSW_METRICS_SCRATCH_BYTES = 1 << 20   # scratch of nsw_weighted_metrics_unnorm_noalloc (per GPU)

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_int = ctypes.c_int


class BlockParams(ctypes.Structure):
    _fields_ = [(n, _vp) for n in (
        "norm1_w", "wqkv", "bqkv", "qn_w", "kn_w", "wproj", "bproj",
        "norm2_w", "w1", "b1", "w2", "b2", "wqkv_n1", "w1_n2")]


class BlockShape(ctypes.Structure):
    _fields_ = [("B", _i64), ("T", _i64), ("H", _i64), ("W", _i64), ("C", _i64),
                ("num_heads", _i64), ("ws0", _i64), ("ws1", _i64), ("s0", _i64), ("s1", _i64),
                ("hidden", _i64), ("eps", _f32), ("dtype", _int), ("gelu_tanh", _int)]


# name -> (restype, argtypes); must match include/nsw.h
SIGNATURES = {
    "nsw_last_error": (ctypes.c_char_p, []),
    "nsw_version": (_int, []),
    "nsw_roll_hw": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp]),
    "nsw_window_partition": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp]),
    "nsw_window_reverse": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp]),
    "nsw_roll_window_partition": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                         _int, _vp]),
    "nsw_window_reverse_roll": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                       _int, _vp]),
    "nsw_make_attention_mask": (_int, [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp]),
    "nsw_selftest_fastdiv": (_int, []),
    "nsw_gemm_read_stamps": (_int, [_vp, ctypes.c_size_t]),
    "nsw_rmsnorm": (_int, [_vp, _vp, _f32, _vp, _i64, _i64, _int, _vp]),
    "nsw_layernorm": (_int, [_vp, _vp, _vp, _f32, _vp, _i64, _i64, _int, _vp]),
    "nsw_rmsnorm_roll_partition": (_int, [_vp, _vp, _f32, _vp, _i64, _i64, _i64, _i64, _i64,
                                          _i64, _i64, _i64, _i64, _int, _vp]),
    "nsw_linear": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _vp]),
    "nsw_qkv_projection": (_int, [_vp, _vp, _vp, _vp, _vp, _f32, _vp, _i64, _i64, _i64, _int, _vp]),
    "nsw_window_attention": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32, _i64, _i64,
                                    _i64, _i64, _i64, _i64, _i64, _int, _vp]),
    "nsw_proj_reverse_residual": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                         _i64, _i64, _i64, _i64, _int, _vp]),
    "nsw_block_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(BlockShape)]),
    "nsw_swin_block_forward": (_int, [_vp, _vp, ctypes.POINTER(BlockParams), ctypes.POINTER(BlockShape),
                                      _vp, ctypes.c_size_t, _vp]),
    "nsw_blocks_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(BlockShape), _i64]),
    "nsw_swin_blocks_forward": (_int, [_vp, _vp, ctypes.POINTER(BlockParams), ctypes.POINTER(BlockShape), _i64,
                                       _vp, ctypes.c_size_t, _vp]),
    "nsw_swin_blocks_forward_windowed": (_int, [_vp, _vp, _vp, ctypes.POINTER(BlockParams),
                                                ctypes.POINTER(BlockShape), _i64, _vp, ctypes.c_size_t, _vp]),
    "nsw_window_partition_sumsq": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                          _int, _vp]),
    "nsw_weighted_metrics_workspace_size": (ctypes.c_size_t, [_i64, _i64, _i64]),
    "nsw_weighted_metrics": (_int, [_vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp,
                                    ctypes.c_size_t, _vp]),
    "nsw_weighted_metrics_unnorm": (_int, [_vp, _int, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64,
                                           _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "nsw_weighted_metrics_unnorm_f64stats": (_int, [_vp, _int, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64,
                                                    _i64, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "nsw_weighted_metrics_unnorm_noalloc": (_int, [_vp, _int, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64,
                                                   _i64, _vp, _vp, _vp]),
    "nsw_hbm_stream": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "nsw_linear_rowscale": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _f32, _int,
                                   _vp]),
    "nsw_row_sumsq_parts": (_i64, [_i64, _int]),
    "nsw_qkv_projection_rowscale": (_int, [_vp, _vp, _vp, _vp, _vp, _f32, _vp, _vp, _i64, _i64, _i64, _i64, _int,
                                           _vp]),
    "nsw_linear_remap_residual": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _i64, _i64, _i64,
                                         _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp]),
    "nsw_proj_reverse_residual_sumsq": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                               _i64, _i64, _i64, _i64, _int, _vp]),
    "nsw_patch_im2col": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _int,
                                _int, _vp]),
    "nsw_unpatchify": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _vp]),
    "nsw_head_unpatchify": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _vp]),
    "nsw_skip_conv_accumulate": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                        _int, _int, _int, _vp]),
}

_lib = None
_lock = threading.Lock()


class NswError(RuntimeError):
    """A libnsw entry point returned an error code."""


def load(path: str) -> ctypes.CDLL:
    """Open a build of the library at `path` with the signatures above."""
    h = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(h, name)
        fn.restype = res
        fn.argtypes = args
    return h


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise NswError(
                        f"{LIB_PATH} is not built; run `python neural-scaling-weather_amd/build.py` "
                        "(the Swin block has no non-HIP implementation)")
                _lib = load(LIB_PATH)
    return _lib


def use(path: str) -> None:
    """Route every op through the build at `path` (a measurement build such
    as nsw/libnsw_stamps.so) for the rest of the process."""
    global _lib
    with _lock:
        _lib = load(path)


def check(rc: int, what: str = "") -> None:
    if rc != NSW_OK:
        msg = lib().nsw_last_error().decode(errors="replace")
        if rc == NSW_ERR_INVALID:
            raise ValueError(f"libnsw{(' ' + what) if what else ''}: {msg}")
        raise NswError(f"libnsw{(' ' + what) if what else ''} (code {rc}): {msg}")
