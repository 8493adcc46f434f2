"""The library's functional ops as PyTorch custom operators, ``torch.ops.nsw.*``.

Each op is registered with ``torch.library.custom_op`` and a shape function
(``register_fake``), so the modules built on them (``nsw.Block``,
``WindowMultiHeadAttention``, ``MLP``, ``NormLayer``, ``LinearLayer``,
``SwinTransformer``, ``WeightedRMSE`` ...) trace under ``torch.compile``
without graph breaks: the op bodies call the ctypes layer (``nsw/ops.py``),
which stays opaque to the tracer.  The ops allocate their outputs with torch
and enqueue HIP kernels on the current stream, so they also run under CUDA
graph capture.  Ops that write into a caller's tensor (``out=``) are not
registered; their callers keep the ``nsw.ops`` functions.

The block parameters travel as one list in the field order of
``nsw_block_params`` (``BLOCK_PARAMS``), None for absent fields; shapes,
windows and shifts as int lists.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from . import _lib, ops

BLOCK_PARAMS = [n for n, _ in _lib.BlockParams._fields_]


def block_param_list(packed: dict) -> List[Optional[torch.Tensor]]:
    return [packed.get(n) for n in BLOCK_PARAMS]


def _unpack_block(params: List[Optional[torch.Tensor]]) -> dict:
    if len(params) != len(BLOCK_PARAMS):
        raise ValueError(f"a block takes {len(BLOCK_PARAMS)} parameter slots, got {len(params)}")
    return {n: t for n, t in zip(BLOCK_PARAMS, params) if t is not None}


# ----------------------------------------------------------------- blocks ---

@torch.library.custom_op("nsw::swin_block", mutates_args=())
def swin_block(x: torch.Tensor, params: List[Optional[torch.Tensor]], num_heads: int, window_size: List[int],
               shift_size: List[int], eps: float, gelu_tanh: bool) -> torch.Tensor:
    """Block.forward (models/swin_helpers.py:435-459) through nsw_swin_block_forward."""
    return ops.swin_block_forward(x.contiguous(), _unpack_block(params), num_heads, tuple(window_size),
                                  tuple(shift_size), eps=eps, gelu_tanh=gelu_tanh)


@swin_block.register_fake
def _(x, params, num_heads, window_size, shift_size, eps, gelu_tanh):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


@torch.library.custom_op("nsw::swin_blocks", mutates_args=())
def swin_blocks(x: torch.Tensor, params: List[Optional[torch.Tensor]], num_heads: int, window_size: List[int],
                shifts: List[int], eps: float, gelu_tanh: bool) -> torch.Tensor:
    """``for blk in blocks: x = blk(x)`` (models/swin.py:307-308) as one window-order chain;
    params = the blocks' parameter lists concatenated, shifts = [s0, s1] per block."""
    nb = len(BLOCK_PARAMS)
    depth = len(shifts) // 2
    if depth == 0 or len(shifts) != 2 * depth or len(params) != nb * depth:
        raise ValueError("swin_blocks: one parameter list and one shift pair per block")
    packs = [_unpack_block(params[i * nb:(i + 1) * nb]) for i in range(depth)]
    sh = [(shifts[2 * i], shifts[2 * i + 1]) for i in range(depth)]
    return ops.swin_blocks_forward(x.contiguous(), packs, num_heads, tuple(window_size), sh, eps=eps,
                                   gelu_tanh=gelu_tanh)


@swin_blocks.register_fake
def _(x, params, num_heads, window_size, shifts, eps, gelu_tanh):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


@torch.library.custom_op("nsw::swin_blocks_windowed", mutates_args=())
def swin_blocks_windowed(xw: torch.Tensor, row_sumsq: torch.Tensor, params: List[Optional[torch.Tensor]],
                         num_heads: int, window_size: List[int], shifts: List[int], eps: float,
                         gelu_tanh: bool) -> torch.Tensor:
    """swin_blocks from block 0's window order: xw [B, T, H, W, C] holding the
    rows in block 0's window order, row_sumsq their norm1 partial sums."""
    nb = len(BLOCK_PARAMS)
    depth = len(shifts) // 2
    if depth == 0 or len(shifts) != 2 * depth or len(params) != nb * depth:
        raise ValueError("swin_blocks_windowed: one parameter list and one shift pair per block")
    packs = [_unpack_block(params[i * nb:(i + 1) * nb]) for i in range(depth)]
    sh = [(shifts[2 * i], shifts[2 * i + 1]) for i in range(depth)]
    return ops.swin_blocks_forward(xw.contiguous(), packs, num_heads, tuple(window_size), sh, eps=eps,
                                   gelu_tanh=gelu_tanh, row_sumsq=row_sumsq.contiguous())


@swin_blocks_windowed.register_fake
def _(xw, row_sumsq, params, num_heads, window_size, shifts, eps, gelu_tanh):
    return torch.empty_like(xw, memory_format=torch.contiguous_format)


# ------------------------------------------------------------ linear / norm ---

@torch.library.custom_op("nsw::linear", mutates_args=())
def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], residual: Optional[torch.Tensor],
           epilogue: int) -> torch.Tensor:
    """y = epi(x . weight^T) (F.linear with a fused bias / GELU / residual epilogue)."""
    return ops.linear(x.contiguous(), weight.contiguous(), bias, None if residual is None else residual.contiguous(),
                      epilogue=epilogue)


@linear.register_fake
def _(x, weight, bias, residual, epilogue):
    return x.new_empty(tuple(x.shape[:-1]) + (weight.shape[0],))


@torch.library.custom_op("nsw::linear_to_window", mutates_args=())
def linear_to_window(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, residual: torch.Tensor,
                     image: List[int], window_size: List[int], shift_size: List[int]) -> Tuple[torch.Tensor,
                                                                                               torch.Tensor]:
    """(y, row_sumsq): token-ordered rows x . weight^T + bias + residual stored
    in the window order of image (B, T, H, W) rolled by -shift, with the
    stored rows' partial sums of squares (nsw_linear_remap_residual mode 3)."""
    return ops.linear_remap_residual(x.contiguous(), weight.contiguous(), bias.contiguous(), residual.contiguous(),
                                     3, image=tuple(image), window_size=tuple(window_size),
                                     shift_size=tuple(shift_size))


@linear_to_window.register_fake
def _(x, weight, bias, residual, image, window_size, shift_size):
    M, N = x.numel() // x.shape[-1], weight.shape[0]
    P = (N * x.element_size() + 511) // 512
    return x.new_empty((M, N)), x.new_empty((M, P), dtype=torch.float32)


def linear_epi(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
               residual: Optional[torch.Tensor] = None, epilogue: Optional[int] = None) -> torch.Tensor:
    """torch.ops.nsw.linear with ops.linear's default epilogue (none / bias / bias + residual)."""
    if epilogue is None:
        epilogue = _lib.NSW_EPI_NONE if bias is None else (
            _lib.NSW_EPI_BIAS if residual is None else _lib.NSW_EPI_BIAS_RESIDUAL)
    return torch.ops.nsw.linear(x, weight, bias, residual, int(epilogue))


@torch.library.custom_op("nsw::rms_norm", mutates_args=())
def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    return ops.rms_norm(x.contiguous(), weight.contiguous(), eps)


@rms_norm.register_fake
def _(x, weight, eps):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


@torch.library.custom_op("nsw::layer_norm", mutates_args=())
def layer_norm(x: torch.Tensor, weight: Optional[torch.Tensor], bias: Optional[torch.Tensor],
               eps: float) -> torch.Tensor:
    return ops.layer_norm(x.contiguous(), weight, bias, eps)


@layer_norm.register_fake
def _(x, weight, bias, eps):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


# -------------------------------------------------------------- attention ---

@torch.library.custom_op("nsw::qkv_projection", mutates_args=())
def qkv_projection(x: torch.Tensor, wqkv: torch.Tensor, bqkv: torch.Tensor, qn_w: torch.Tensor,
                   kn_w: torch.Tensor, num_heads: int, eps: float) -> torch.Tensor:
    return ops.qkv_projection(x.contiguous(), wqkv, bqkv, qn_w, kn_w, num_heads, eps)


@qkv_projection.register_fake
def _(x, wqkv, bqkv, qn_w, kn_w, num_heads, eps):
    return x.new_empty(tuple(x.shape[:-1]) + (3 * x.shape[-1],))


@torch.library.custom_op("nsw::window_attention", mutates_args=())
def window_attention(qkv: torch.Tensor, num_heads: int, scale: float, mask: Optional[torch.Tensor],
                     geometry: List[int]) -> torch.Tensor:
    """geometry = [H, W, ws0, ws1, s0, s1, T] (shift mask from indices) or []."""
    geo = None
    if len(geometry) == 7:
        H, W, ws0, ws1, s0, s1, T = geometry
        geo = (H, W, (ws0, ws1), (s0, s1), T)
    elif len(geometry) != 0:
        raise ValueError("window_attention: geometry is [H, W, ws0, ws1, s0, s1, T] or empty")
    return ops.window_attention(qkv.contiguous(), num_heads, scale,
                                mask=None if mask is None else mask.contiguous(), geometry=geo)


@window_attention.register_fake
def _(qkv, num_heads, scale, mask, geometry):
    Bw, L, C3 = qkv.shape
    return qkv.new_empty((Bw, L, C3 // 3))


# ------------------------------------------------------------ window maps ---

@torch.library.custom_op("nsw::window_partition", mutates_args=())
def window_partition(x: torch.Tensor, window_size: List[int]) -> torch.Tensor:
    return ops.window_partition(x.contiguous(), tuple(window_size))


@window_partition.register_fake
def _(x, window_size):
    B, T, H, W, C = x.shape
    return x.new_empty((B * (H // window_size[0]) * (W // window_size[1]), T, window_size[0], window_size[1], C))


@torch.library.custom_op("nsw::window_reverse", mutates_args=())
def window_reverse(windows: torch.Tensor, window_size: List[int], img_size: List[int]) -> torch.Tensor:
    return ops.window_reverse(windows.contiguous(), tuple(window_size), tuple(img_size))


@window_reverse.register_fake
def _(windows, window_size, img_size):
    T, C = windows.shape[1], windows.shape[-1]
    H, W = img_size
    B = windows.shape[0] // ((H // window_size[0]) * (W // window_size[1]))
    return windows.new_empty((B, T, H, W, C))


@torch.library.custom_op("nsw::roll_hw", mutates_args=())
def roll_hw(x: torch.Tensor, shifts: List[int]) -> torch.Tensor:
    return ops.roll_hw(x.contiguous(), tuple(shifts))


@roll_hw.register_fake
def _(x, shifts):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


@torch.library.custom_op("nsw::roll_window_partition", mutates_args=())
def roll_window_partition(x: torch.Tensor, window_size: List[int], shift_size: List[int]) -> torch.Tensor:
    return ops.roll_window_partition(x.contiguous(), tuple(window_size), tuple(shift_size))


@roll_window_partition.register_fake
def _(x, window_size, shift_size):
    B, T, H, W, C = x.shape
    return x.new_empty((B * (H // window_size[0]) * (W // window_size[1]), T, window_size[0], window_size[1], C))


@torch.library.custom_op("nsw::window_reverse_roll", mutates_args=())
def window_reverse_roll(windows: torch.Tensor, window_size: List[int], img_size: List[int],
                        shift_size: List[int]) -> torch.Tensor:
    return ops.window_reverse_roll(windows.contiguous(), tuple(window_size), tuple(img_size), tuple(shift_size))


@window_reverse_roll.register_fake
def _(windows, window_size, img_size, shift_size):
    T, C = windows.shape[1], windows.shape[-1]
    H, W = img_size
    B = windows.shape[0] // ((H // window_size[0]) * (W // window_size[1]))
    return windows.new_empty((B, T, H, W, C))


# ----------------------------------------------------------- model layout ---

@torch.library.custom_op("nsw::patch_im2col", mutates_args=())
def patch_im2col(x: torch.Tensor, p: int, Kp: int, dtype: torch.dtype, invariants: Optional[torch.Tensor],
                 frame0: int) -> torch.Tensor:
    return ops.patch_im2col(x.contiguous(), p, Kp, dtype,
                            invariants=None if invariants is None else invariants.contiguous(), frame0=frame0)


@patch_im2col.register_fake
def _(x, p, Kp, dtype, invariants, frame0):
    B, T, _, H, W = x.shape
    return x.new_empty((B * T * (H // p) * (W // p), Kp), dtype=dtype)


@torch.library.custom_op("nsw::unpatchify", mutates_args=())
def unpatchify(y: torch.Tensor, B: int, C_out: int, H: int, W: int, p: int,
               dtype: Optional[torch.dtype]) -> torch.Tensor:
    return ops.unpatchify(y.contiguous(), B, C_out, H, W, p, dtype=dtype)


@unpatchify.register_fake
def _(y, B, C_out, H, W, p, dtype):
    return y.new_empty((B, 1, C_out, H, W), dtype=dtype if dtype is not None else y.dtype)


@torch.library.custom_op("nsw::head_unpatchify", mutates_args=())
def head_unpatchify(x: torch.Tensor, w_perm: torch.Tensor, B: int, C_out: int, H: int, W: int, p: int,
                    dtype: Optional[torch.dtype]) -> torch.Tensor:
    """The head GEMM with the head layout in its write-out (w_perm from ops.head_weight_perm)."""
    return ops.head_unpatchify(x.contiguous(), w_perm.contiguous(), B, C_out, H, W, p, dtype=dtype)


@head_unpatchify.register_fake
def _(x, w_perm, B, C_out, H, W, p, dtype):
    return x.new_empty((B, 1, C_out, H, W), dtype=dtype if dtype is not None else x.dtype)


@torch.library.custom_op("nsw::skip_conv_accumulate", mutates_args=("out",))
def skip_conv_accumulate(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, invariants: Optional[torch.Tensor],
                         frame0: int) -> None:
    """The model's big skip added in place to its predicted frame."""
    ops.skip_conv_accumulate(x, weight, out, invariants=invariants, frame0=frame0)


@skip_conv_accumulate.register_fake
def _(x, weight, out, invariants, frame0):
    return None


# ---------------------------------------------------------------- metrics ---

@torch.library.custom_op("nsw::weighted_metrics", mutates_args=())
def weighted_metrics(pred: torch.Tensor, target: torch.Tensor, weights: torch.Tensor,
                     clim: Optional[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
    """(rmse, acc) float64 [B, T, C]; acc is empty ([0]) without a climatology."""
    rmse, acc = ops.weighted_metrics(pred.contiguous(), target.contiguous(), weights, clim)
    if acc is None:
        acc = rmse.new_empty((0,))
    return rmse, acc


@weighted_metrics.register_fake
def _(pred, target, weights, clim):
    B, T, C = pred.shape[:3]
    rmse = pred.new_empty((B, T, C), dtype=torch.float64)
    acc = pred.new_empty((B, T, C) if clim is not None else (0,), dtype=torch.float64)
    return rmse, acc
