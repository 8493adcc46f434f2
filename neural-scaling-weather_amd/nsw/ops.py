"""Tensor-level wrappers of the libnsw C ABI.

Every op takes / returns torch tensors on the GPU, enqueues HIP kernels on
torch's current stream and allocates its outputs with torch (plumbing only:
all arithmetic runs in libnsw's kernels).  Inputs must be contiguous,
16-byte aligned, fp32 or bf16, on a HIP device; anything else raises.
"""
from __future__ import annotations

import threading
from typing import Optional, Sequence, Tuple

import torch

from . import _lib
from ._lib import check, lib

_DTYPES = {torch.float32: _lib.NSW_DTYPE_F32, torch.bfloat16: _lib.NSW_DTYPE_BF16}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"libnsw supports float32 and bfloat16 tensors, got {t.dtype}") from None


def _dev(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("libnsw ops run on the GPU only; got a tensor on " + str(t.device))
        if not t.is_contiguous():
            raise RuntimeError("libnsw ops need contiguous tensors")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError("libnsw op arguments are on different devices")
    return dev


def _same_dtype(ref: torch.Tensor, *ts: Optional[torch.Tensor]) -> None:
    for t in ts:
        if t is not None and t.dtype != ref.dtype:
            raise TypeError(f"dtype mismatch: {t.dtype} vs {ref.dtype}")


def _p(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device):
    return torch.cuda.current_stream(dev).cuda_stream


def default_eps(dtype: torch.dtype) -> float:
    """nn.RMSNorm(eps=None) uses finfo(input dtype).eps."""
    return float(torch.finfo(dtype).eps)


# ------------------------------------------------------------------ index ---

def roll_hw(x: torch.Tensor, shifts: Tuple[int, int]) -> torch.Tensor:
    """torch.roll(x, shifts, dims=(-3, -2)) of a [B,T,H,W,C] tensor."""
    B, T, H, W, C = x.shape
    dev = _dev(x)
    y = torch.empty_like(x)
    check(lib().nsw_roll_hw(x.data_ptr(), y.data_ptr(), B, T, H, W, C, int(shifts[0]), int(shifts[1]),
                            dtype_code(x), _stream(dev)), "roll_hw")
    return y


def window_partition(x: torch.Tensor, window_size: Tuple[int, int]) -> torch.Tensor:
    B, T, H, W, C = x.shape
    ws0, ws1 = window_size
    if H % ws0 or W % ws1:
        raise ValueError(f"image {H}x{W} is not divisible by window {window_size}")
    dev = _dev(x)
    out = torch.empty((B * (H // ws0) * (W // ws1), T, ws0, ws1, C), dtype=x.dtype, device=dev)
    check(lib().nsw_window_partition(x.data_ptr(), out.data_ptr(), B, T, H, W, C, ws0, ws1,
                                     dtype_code(x), _stream(dev)), "window_partition")
    return out


def window_reverse(windows: torch.Tensor, window_size: Tuple[int, int],
                   img_size: Tuple[int, int]) -> torch.Tensor:
    H, W = img_size
    ws0, ws1 = window_size
    T, C = windows.shape[1], windows.shape[-1]
    nw = (H // ws0) * (W // ws1)
    if windows.shape[0] % nw:
        raise ValueError("number of windows is not a multiple of the image's windows")
    B = windows.shape[0] // nw
    dev = _dev(windows)
    out = torch.empty((B, T, H, W, C), dtype=windows.dtype, device=dev)
    check(lib().nsw_window_reverse(windows.data_ptr(), out.data_ptr(), B, T, H, W, C, ws0, ws1,
                                   dtype_code(windows), _stream(dev)), "window_reverse")
    return out


def roll_window_partition(x: torch.Tensor, window_size, shift_size) -> torch.Tensor:
    """window_partition(torch.roll(x, -shift, (H, W)), window_size) in one pass."""
    B, T, H, W, C = x.shape
    ws0, ws1 = window_size
    dev = _dev(x)
    out = torch.empty((B * (H // ws0) * (W // ws1), T, ws0, ws1, C), dtype=x.dtype, device=dev)
    check(lib().nsw_roll_window_partition(x.data_ptr(), out.data_ptr(), B, T, H, W, C, ws0, ws1,
                                          int(shift_size[0]), int(shift_size[1]), dtype_code(x),
                                          _stream(dev)), "roll_window_partition")
    return out


def window_reverse_roll(windows: torch.Tensor, window_size, img_size, shift_size) -> torch.Tensor:
    """torch.roll(window_reverse(windows), +shift, (H, W)) in one pass."""
    H, W = img_size
    ws0, ws1 = window_size
    T, C = windows.shape[1], windows.shape[-1]
    B = windows.shape[0] // ((H // ws0) * (W // ws1))
    dev = _dev(windows)
    out = torch.empty((B, T, H, W, C), dtype=windows.dtype, device=dev)
    check(lib().nsw_window_reverse_roll(windows.data_ptr(), out.data_ptr(), B, T, H, W, C, ws0, ws1,
                                        int(shift_size[0]), int(shift_size[1]), dtype_code(windows),
                                        _stream(dev)), "window_reverse_roll")
    return out


def make_attention_mask(H: int, W: int, window_size: Tuple[int, int], shift_size: Tuple[int, int],
                        T: int, device) -> torch.Tensor:
    ws0, ws1 = window_size
    nW = (H // ws0) * (W // ws1)
    L = T * ws0 * ws1
    m = torch.empty((nW, L, L), dtype=torch.float32, device=device)
    check(lib().nsw_make_attention_mask(m.data_ptr(), H, W, ws0, ws1, int(shift_size[0]),
                                        int(shift_size[1]), T, _stream(m.device)), "make_attention_mask")
    return m


# ------------------------------------------------------------------- norms ---

def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: Optional[float] = None) -> torch.Tensor:
    dev = _dev(x, weight)
    _same_dtype(x, weight)
    C = x.shape[-1]
    if weight.numel() != C:
        raise ValueError(f"norm weight has {weight.numel()} elements, input has {C} features")
    eps = default_eps(x.dtype) if eps is None else float(eps)
    y = torch.empty_like(x)
    check(lib().nsw_rmsnorm(x.data_ptr(), weight.data_ptr(), eps, y.data_ptr(), x.numel() // C, C,
                            dtype_code(x), _stream(dev)), "rms_norm")
    return y


def layer_norm(x: torch.Tensor, weight: Optional[torch.Tensor], bias: Optional[torch.Tensor],
               eps: float = 1e-5) -> torch.Tensor:
    """nn.LayerNorm over the last dim (biased variance); weight / bias may be
    None (elementwise_affine=False)."""
    dev = _dev(x, weight, bias)
    _same_dtype(x, weight, bias)
    C = x.shape[-1]
    for t in (weight, bias):
        if t is not None and t.numel() != C:
            raise ValueError(f"layer-norm parameter has {t.numel()} elements, input has {C} features")
    y = torch.empty_like(x)
    check(lib().nsw_layernorm(x.data_ptr(), _p(weight), _p(bias), float(eps), y.data_ptr(), x.numel() // C, C,
                              dtype_code(x), _stream(dev)), "layer_norm")
    return y


def rmsnorm_roll_partition(x: torch.Tensor, weight: torch.Tensor, window_size, shift_size,
                           eps: Optional[float] = None) -> torch.Tensor:
    """norm1 + roll by -shift + window_partition, as [B*nW, T*wa, C]."""
    B, T, H, W, C = x.shape
    dev = _dev(x, weight)
    _same_dtype(x, weight)
    eps = default_eps(x.dtype) if eps is None else float(eps)
    ws0, ws1 = window_size
    out = torch.empty((B * (H // ws0) * (W // ws1), T * ws0 * ws1, C), dtype=x.dtype, device=dev)
    check(lib().nsw_rmsnorm_roll_partition(x.data_ptr(), weight.data_ptr(), eps, out.data_ptr(), B, T, H, W,
                                           C, ws0, ws1, int(shift_size[0]), int(shift_size[1]),
                                           dtype_code(x), _stream(dev)), "rmsnorm_roll_partition")
    return out


# -------------------------------------------------------------------- GEMM ---

def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
           residual: Optional[torch.Tensor] = None, epilogue: Optional[int] = None,
           out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = epi(x . weight^T): F.linear with an optional fused bias / GELU / residual.
    ``out`` (contiguous, x.shape[:-1] + (N,), x's dtype) receives y if given."""
    dev = _dev(x, weight, bias, residual, out)
    _same_dtype(x, weight, bias, residual, out)
    K = x.shape[-1]
    N, Kw = weight.shape
    if Kw != K:
        raise ValueError(f"linear: x has {K} features, weight expects {Kw}")
    M = x.numel() // K
    if epilogue is None:
        epilogue = _lib.NSW_EPI_NONE if bias is None else (
            _lib.NSW_EPI_BIAS if residual is None else _lib.NSW_EPI_BIAS_RESIDUAL)
    if out is not None:
        if out.numel() != M * N:
            raise ValueError(f"linear: out has {out.numel()} elements, expected {M * N}")
        y = out.view(x.shape[:-1] + (N,))
    else:
        y = torch.empty(x.shape[:-1] + (N,), dtype=x.dtype, device=dev)
    if residual is not None and residual.shape != y.shape:
        raise ValueError(f"residual shape {tuple(residual.shape)} != output {tuple(y.shape)}")
    check(lib().nsw_linear(x.data_ptr(), weight.data_ptr(), _p(bias), _p(residual), y.data_ptr(), M, N, K,
                           int(epilogue), dtype_code(x), _stream(dev)), "linear")
    return y


def qkv_projection(x: torch.Tensor, wqkv: torch.Tensor, bqkv: torch.Tensor, qn_w: torch.Tensor,
                   kn_w: torch.Tensor, num_heads: int, eps: Optional[float] = None) -> torch.Tensor:
    """[.., C] -> [.., 3C]: q|k|v = x W^T + b with per-head RMSNorm on q and k."""
    dev = _dev(x, wqkv, bqkv, qn_w, kn_w)
    _same_dtype(x, wqkv, bqkv, qn_w, kn_w)
    C = x.shape[-1]
    M = x.numel() // C
    eps = default_eps(x.dtype) if eps is None else float(eps)
    y = torch.empty(x.shape[:-1] + (3 * C,), dtype=x.dtype, device=dev)
    check(lib().nsw_qkv_projection(x.data_ptr(), wqkv.data_ptr(), bqkv.data_ptr(), qn_w.data_ptr(),
                                   kn_w.data_ptr(), eps, y.data_ptr(), M, C, num_heads, dtype_code(x),
                                   _stream(dev)), "qkv_projection")
    return y


# --------------------------------------------------------------- attention ---

def window_attention(qkv: torch.Tensor, num_heads: int, scale: float, mask: Optional[torch.Tensor] = None,
                     geometry: Optional[Tuple[int, int, Tuple[int, int], Tuple[int, int], int]] = None
                     ) -> torch.Tensor:
    """qkv [Bw, L, 3C] -> o [Bw, L, C].  ``mask`` [nW, L, L] or None, with
    F.scaled_dot_product_attention's meaning (models/swin_helpers.py:247): a
    float mask is added to the scaled logits, a boolean mask marks the keys
    that take part (True) and is applied as 0 / -inf.  ``geometry`` = (H, W,
    window_size, shift_size, T) computes the reference's shift mask from
    indices instead (ignored when mask is given)."""
    Bw, L, C3 = qkv.shape
    C = C3 // 3
    dev = _dev(qkv, mask)
    if mask is not None:
        if mask.dtype == torch.bool:
            mask = torch.zeros(mask.shape, dtype=torch.float32, device=mask.device).masked_fill_(
                ~mask, float("-inf"))
        elif mask.dtype != torch.float32:
            mask = mask.float().contiguous()
        if mask.shape[-2:] != (L, L):
            raise ValueError(f"mask shape {tuple(mask.shape)} does not match L={L}")
        nWm = mask.shape[0]
    else:
        nWm = 0
    H = W = ws0 = ws1 = 1
    s0 = s1 = 0
    T = 1
    if geometry is not None and mask is None:
        H, W, (ws0, ws1), (s0, s1), T = geometry
    o = torch.empty((Bw, L, C), dtype=qkv.dtype, device=dev)
    check(lib().nsw_window_attention(qkv.data_ptr(), o.data_ptr(), _p(mask), nWm, Bw, L, C, num_heads,
                                     float(scale), H, W, ws0, ws1, s0, s1, T, dtype_code(qkv),
                                     _stream(dev)), "window_attention")
    return o


def proj_reverse_residual(o: torch.Tensor, wproj: torch.Tensor, bproj: torch.Tensor, skip: torch.Tensor,
                          window_size, shift_size) -> torch.Tensor:
    """skip + roll(window_reverse(o W^T + b), +shift) with skip [B,T,H,W,C]."""
    B, T, H, W, C = skip.shape
    dev = _dev(o, wproj, bproj, skip)
    _same_dtype(o, wproj, bproj, skip)
    y = torch.empty_like(skip)
    check(lib().nsw_proj_reverse_residual(o.data_ptr(), wproj.data_ptr(), bproj.data_ptr(), skip.data_ptr(),
                                          y.data_ptr(), B, T, H, W, C, window_size[0], window_size[1],
                                          int(shift_size[0]), int(shift_size[1]), dtype_code(o),
                                          _stream(dev)), "proj_reverse_residual")
    return y


def proj_reverse_residual_sumsq(o: torch.Tensor, wproj: torch.Tensor, bproj: torch.Tensor, skip: torch.Tensor,
                                window_size, shift_size):
    """proj_reverse_residual that also returns the partial sums of squares of
    each output row [B*T*H*W, P] (fp32, one per 512 bytes of row), the
    statistics of the RMSNorm that follows."""
    B, T, H, W, C = skip.shape
    dev = _dev(o, wproj, bproj, skip)
    _same_dtype(o, wproj, bproj, skip)
    y = torch.empty_like(skip)
    P = int(lib().nsw_row_sumsq_parts(C, dtype_code(skip)))
    ss = torch.empty(B * T * H * W, P, dtype=torch.float32, device=dev)
    check(lib().nsw_proj_reverse_residual_sumsq(o.data_ptr(), wproj.data_ptr(), bproj.data_ptr(),
                                                skip.data_ptr(), y.data_ptr(), ss.data_ptr(), B, T, H, W, C,
                                                window_size[0], window_size[1], int(shift_size[0]),
                                                int(shift_size[1]), dtype_code(o), _stream(dev)),
          "proj_reverse_residual_sumsq")
    return y, ss


def linear_rowscale(x: torch.Tensor, w_n: torch.Tensor, row_sumsq: torch.Tensor, bias: Optional[torch.Tensor] = None,
                    residual: Optional[torch.Tensor] = None, epilogue: Optional[int] = None,
                    eps: Optional[float] = None) -> torch.Tensor:
    """y = epi(RMSNorm(x) . W^T) with w_n = W * norm_w and the rows' sums of
    squares given as partials row_sumsq [M, P] (from proj_reverse_residual_sumsq)."""
    dev = _dev(x, w_n, bias, residual, row_sumsq)
    _same_dtype(x, w_n, bias, residual)
    K = x.shape[-1]
    N, Kw = w_n.shape
    if Kw != K:
        raise ValueError(f"linear_rowscale: x has {K} features, weight expects {Kw}")
    M = x.numel() // K
    if row_sumsq.dtype != torch.float32 or row_sumsq.dim() != 2 or row_sumsq.shape[0] != M \
            or not row_sumsq.is_contiguous():
        raise ValueError("linear_rowscale: row_sumsq must be a contiguous fp32 [M, P] tensor")
    if epilogue is None:
        epilogue = _lib.NSW_EPI_NONE if bias is None else (
            _lib.NSW_EPI_BIAS if residual is None else _lib.NSW_EPI_BIAS_RESIDUAL)
    eps = default_eps(x.dtype) if eps is None else float(eps)
    y = torch.empty(x.shape[:-1] + (N,), dtype=x.dtype, device=dev)
    check(lib().nsw_linear_rowscale(x.data_ptr(), w_n.data_ptr(), _p(bias), _p(residual), y.data_ptr(),
                                    row_sumsq.data_ptr(), row_sumsq.shape[1], M, N, K, int(epilogue), eps,
                                    dtype_code(x), _stream(dev)), "linear_rowscale")
    return y


def qkv_projection_rowscale(x: torch.Tensor, wqkv_n: torch.Tensor, bqkv: torch.Tensor, qn_w: torch.Tensor,
                            kn_w: torch.Tensor, row_sumsq: torch.Tensor, num_heads: int,
                            eps: Optional[float] = None) -> torch.Tensor:
    """[M, C] -> [M, 3C]: q|k|v of RMSNorm(x) (norm1's weight folded into
    wqkv_n) with the row statistics given as partial sums of squares
    row_sumsq [M, P] (from window_partition_sumsq or linear_remap_residual)."""
    dev = _dev(x, wqkv_n, bqkv, qn_w, kn_w, row_sumsq)
    _same_dtype(x, wqkv_n, bqkv, qn_w, kn_w)
    C = x.shape[-1]
    M = x.numel() // C
    if row_sumsq.dtype != torch.float32 or row_sumsq.dim() != 2 or row_sumsq.shape[0] != M:
        raise ValueError("qkv_projection_rowscale: row_sumsq must be a contiguous fp32 [M, P] tensor")
    eps = default_eps(x.dtype) if eps is None else float(eps)
    y = torch.empty(x.shape[:-1] + (3 * C,), dtype=x.dtype, device=dev)
    check(lib().nsw_qkv_projection_rowscale(x.data_ptr(), wqkv_n.data_ptr(), bqkv.data_ptr(), qn_w.data_ptr(),
                                            kn_w.data_ptr(), eps, y.data_ptr(), row_sumsq.data_ptr(),
                                            row_sumsq.shape[1], M, C, num_heads, dtype_code(x), _stream(dev)),
          "qkv_projection_rowscale")
    return y


def linear_remap_residual(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor, residual: torch.Tensor,
                          map_mode: int, image=None, window_size=(1, 1), shift_size=(0, 0), next_shift=(0, 0)):
    """(y, row_sumsq): y[map(m)] = x[m] . w^T + bias + residual[m] for window
    rows of ``image`` = (B, T, H, W) with ``window_size`` / ``shift_size``:
    map_mode 0 identity, 1 to token order, 2 to the window order of the
    same image rolled by ``next_shift``, 3 from token-ordered rows into the
    window order with ``shift_size``; row_sumsq [M, P] fp32 (the stored
    rows' partial sums of squares, at the stored rows) for modes 0, 2 and 3,
    None for mode 1."""
    dev = _dev(x, w, bias, residual)
    _same_dtype(x, w, bias, residual)
    K = x.shape[-1]
    N = w.shape[0]
    M = x.numel() // K
    B, T, H, W = image if image is not None else (1, 1, 1, M)
    y = torch.empty(M, N, dtype=x.dtype, device=dev)
    ss = None
    if map_mode != 1:
        ss = torch.empty(M, lib().nsw_row_sumsq_parts(N, dtype_code(x)), dtype=torch.float32, device=dev)
    check(lib().nsw_linear_remap_residual(x.data_ptr(), w.data_ptr(), bias.data_ptr(), residual.data_ptr(),
                                          y.data_ptr(), _p(ss), M, N, K, int(map_mode), B, T, H, W,
                                          window_size[0], window_size[1], int(shift_size[0]), int(shift_size[1]),
                                          int(next_shift[0]), int(next_shift[1]), dtype_code(x), _stream(dev)),
          "linear_remap_residual")
    return y, ss


# ------------------------------------------------------------------- block ---

_ws_lock = threading.Lock()
_workspaces = {}      # (device index, stream) -> [buffer, handed out under graph capture]
_ws_retired = []      # replaced buffers that a captured graph may still address


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Grow-only scratch buffer per (device, stream), reused by every block
    launched on that stream (kernels on one stream run in order).  A buffer
    handed out while the stream was being captured into a CUDA graph is
    never freed: when a later, larger call replaces it, it moves to a list
    kept for the life of the process, so that replays of the graph keep
    writing memory they own."""
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    capturing = torch.cuda.is_current_stream_capturing()
    with _ws_lock:
        ent = _workspaces.get(key)
        if ent is None or ent[0].numel() < nbytes:
            if ent is not None and ent[1]:
                _ws_retired.append(ent[0])
            ent = [torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device), False]
            _workspaces[key] = ent
        if capturing:
            ent[1] = True
        return ent[0]


def block_shape(x: torch.Tensor, num_heads: int, window_size, shift_size, hidden: int,
                eps: Optional[float], gelu_tanh: bool = False) -> _lib.BlockShape:
    B, T, H, W, C = x.shape
    eps = default_eps(x.dtype) if eps is None else float(eps)
    return _lib.BlockShape(B, T, H, W, C, num_heads, window_size[0], window_size[1],
                           int(shift_size[0]), int(shift_size[1]), hidden, eps, dtype_code(x),
                           1 if gelu_tanh else 0)


def swin_block_forward(x: torch.Tensor, packed: dict, num_heads: int, window_size, shift_size,
                       eps: Optional[float] = None, out: Optional[torch.Tensor] = None,
                       gelu_tanh: bool = False) -> torch.Tensor:
    """Whole Block.forward through one C-ABI call.  ``packed`` holds the
    tensors named like the fields of nsw_block_params; ``gelu_tanh`` selects
    the tanh-form GELU (the reference's TE block) instead of the erf form."""
    dev = _dev(x, *packed.values())
    _same_dtype(x, *packed.values())
    hidden = packed["w1"].shape[0]
    shp = block_shape(x, num_heads, window_size, shift_size, hidden, eps, gelu_tanh)
    params = _lib.BlockParams(*[_p(packed.get(n)) for n, _ in _lib.BlockParams._fields_])
    nbytes = lib().nsw_block_workspace_size(shp)
    ws = workspace(nbytes, dev)
    y = torch.empty_like(x) if out is None else out
    check(lib().nsw_swin_block_forward(x.data_ptr(), y.data_ptr(), params, shp, ws.data_ptr(), ws.numel(),
                                       _stream(dev)), "swin_block_forward")
    return y


def swin_blocks_forward(x: torch.Tensor, packs, num_heads: int, window_size, shifts, eps: Optional[float] = None,
                        out: Optional[torch.Tensor] = None, gelu_tanh: bool = False,
                        row_sumsq: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The blocks loop ``for blk in blocks: x = blk(x)`` through one C-ABI
    call that keeps the residual stream in window order between blocks.
    ``packs[i]`` is block i's dict of nsw_block_params tensors and must hold
    the norm-folded ``wqkv_n1`` and ``w1_n2``; ``shifts[i]`` its shift.  With
    ``row_sumsq`` ([rows, P] fp32, as window_partition_sumsq returns), x holds
    block 0's input already in block 0's window order (same [B, T, H, W, C]
    shape, rows in window order) and those are its norm1 sums of squares;
    the result is in token order either way."""
    packs = list(packs)
    if not packs or len(packs) != len(shifts):
        raise ValueError("swin_blocks_forward: one pack and one shift per block")
    tensors = [t for pk in packs for t in pk.values()]
    dev = _dev(x, *tensors)
    _same_dtype(x, *tensors)
    if x.dim() != 5 or not x.is_contiguous():
        raise ValueError("swin_blocks_forward: x must be a contiguous [B, T, H, W, C] tensor")
    depth = len(packs)
    hidden = packs[0]["w1"].shape[0]
    shapes = (_lib.BlockShape * depth)(*[block_shape(x, num_heads, window_size, shifts[i], hidden, eps, gelu_tanh)
                                         for i in range(depth)])
    params = (_lib.BlockParams * depth)(*[_lib.BlockParams(*[_p(pk.get(n)) for n, _ in _lib.BlockParams._fields_])
                                          for pk in packs])
    nbytes = lib().nsw_blocks_workspace_size(shapes, depth)
    if nbytes == 0:
        raise ValueError("swin_blocks_forward: malformed block shape")
    ws = workspace(nbytes, dev)
    y = torch.empty_like(x) if out is None else out
    if row_sumsq is None:
        check(lib().nsw_swin_blocks_forward(x.data_ptr(), y.data_ptr(), params, shapes, depth, ws.data_ptr(),
                                            ws.numel(), _stream(dev)), "swin_blocks_forward")
    else:
        if row_sumsq.dtype != torch.float32 or not row_sumsq.is_contiguous() or row_sumsq.device != dev:
            raise ValueError("swin_blocks_forward: row_sumsq must be a contiguous float32 tensor on x's device")
        if row_sumsq.numel() != (x.numel() // x.shape[-1]) * lib().nsw_row_sumsq_parts(x.shape[-1], dtype_code(x)):
            raise ValueError("swin_blocks_forward: row_sumsq must be [rows, nsw_row_sumsq_parts(C)]")
        check(lib().nsw_swin_blocks_forward_windowed(x.data_ptr(), row_sumsq.data_ptr(), y.data_ptr(), params,
                                                     shapes, depth, ws.data_ptr(), ws.numel(), _stream(dev)),
              "swin_blocks_forward")
    return y


def window_partition_sumsq(x: torch.Tensor, window_size, shift_size):
    """(windows, row_sumsq): x [B,T,H,W,C] rolled by -shift and split into
    windows [B*nW, T, ws0, ws1, C], and fp32 [rows, nparts] partial sums of
    squares of each stored row (512-byte parts)."""
    dev = _dev(x)
    if x.dim() != 5 or not x.is_contiguous():
        raise ValueError("window_partition_sumsq: x must be a contiguous [B, T, H, W, C] tensor")
    B, T, H, W, C = x.shape
    ws0, ws1 = window_size
    nW = (H // ws0) * (W // ws1)
    xw = torch.empty((B * nW, T, ws0, ws1, C), dtype=x.dtype, device=dev)
    nparts = lib().nsw_row_sumsq_parts(C, dtype_code(x))
    ss = torch.empty((x.numel() // C, nparts), dtype=torch.float32, device=dev)
    check(lib().nsw_window_partition_sumsq(x.data_ptr(), xw.data_ptr(), ss.data_ptr(), B, T, H, W, C, ws0, ws1,
                                           int(shift_size[0]), int(shift_size[1]), dtype_code(x), _stream(dev)),
          "window_partition_sumsq")
    return xw, ss


# ----------------------------------------------------------------- metrics ---

def weighted_metrics(pred: torch.Tensor, target: torch.Tensor, weights: torch.Tensor,
                     clim: Optional[torch.Tensor] = None):
    """Per-(b,t,c) weighted RMSE and (if clim is given) ACC, float64 [B,T,C].
    ``weights``: [H], [H, 1] (cos-lat) or [H, W] (a full map)."""
    if pred.shape != target.shape or pred.dim() != 5:
        raise ValueError("pred and target must be [B, T, C, H, W] of the same shape")
    if pred.dtype != torch.float32 or target.dtype != torch.float32:
        raise TypeError("weighted metrics take float32 fields")
    B, T, C, H, W = pred.shape
    dev = _dev(pred, target, clim)
    w = weights.to(device=dev, dtype=torch.float64).contiguous()
    if w.numel() == H:
        w_cols = 1
    elif w.numel() == H * W and (w.dim() < 2 or tuple(w.shape[-2:]) == (H, W)):
        w_cols = W
    else:
        raise ValueError(f"weights of shape {tuple(weights.shape)} do not match a {H}x{W} field")
    if clim is not None:
        clim = clim.reshape(-1).to(torch.float32).contiguous()
        if clim.numel() != C:
            raise ValueError("climatology must have one value per channel")
    P = B * T * C
    rmse = torch.empty(P, dtype=torch.float64, device=dev)
    acc = torch.empty(P, dtype=torch.float64, device=dev) if clim is not None else None
    nbytes = lib().nsw_weighted_metrics_workspace_size(P, H, W)
    ws = torch.empty(max(nbytes, 8), dtype=torch.uint8, device=dev)
    check(lib().nsw_weighted_metrics(pred.data_ptr(), target.data_ptr(), w.data_ptr(), w_cols, _p(clim), P,
                                     H, W, C,
                                     rmse.data_ptr(), _p(acc), ws.data_ptr(), ws.numel(), _stream(dev)),
          "weighted_metrics")
    rmse = rmse.view(B, T, C)
    return rmse, (acc.view(B, T, C) if acc is not None else None)


# ------------------------------------------------------------ model layout ---

def k_granule(dtype: torch.dtype) -> int:
    """K padding of the patch matrix: one 128-byte operand stage of the GEMM,
    64 (bf16) / 32 (f32) elements, so that its rows start on whole cache
    lines (the GEMM itself takes K a multiple of 32 / 16)."""
    return 64 if dtype == torch.bfloat16 else 32


def patch_im2col(x: torch.Tensor, p: int, Kp: int, dtype: torch.dtype,
                 invariants: Optional[torch.Tensor] = None, frame0: int = 0) -> torch.Tensor:
    """Patch matrix of the stride-p patch convolution: x [B, T, C_x, H, W]
    (+ invariants [C_inv, H, W] as extra channels; frame t read from slot
    (t + frame0) mod T) -> [B*T*(H/p)*(W/p), Kp] in ``dtype``."""
    if x.dim() != 5:
        raise ValueError("patch_im2col: x must be [B, T, C, H, W]")
    B, T, Cx, H, W = x.shape
    if invariants is not None:
        if invariants.dtype != x.dtype:
            raise TypeError("patch_im2col: invariants must have x's dtype")
        if invariants.dim() != 3 or tuple(invariants.shape[1:]) != (H, W):
            raise ValueError("patch_im2col: invariants must be [C_inv, H, W]")
    dev = _dev(x, invariants)
    Cinv = 0 if invariants is None else invariants.shape[0]
    M = B * T * (H // p) * (W // p)
    out = torch.empty(M, Kp, dtype=dtype, device=dev)
    check(lib().nsw_patch_im2col(x.data_ptr(), _p(invariants), B, T, Cx, Cinv, H, W, p, int(frame0), Kp,
                                 out.data_ptr(), dtype_code(x), _DTYPES[dtype], _stream(dev)), "patch_im2col")
    return out


def unpatchify(y: torch.Tensor, B: int, C_out: int, H: int, W: int, p: int,
               dtype: Optional[torch.dtype] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Head layout: y [B*(H/p)*(W/p), p*p*C_out] -> [B, 1, C_out, H, W].  With
    ``out`` (a [B, 1, C_out, H, W] tensor whose frames are contiguous, e.g.
    one slot of a [B, T, C, H, W] ring buffer) the result is written there in
    out's dtype."""
    if out is not None:
        if tuple(out.shape) != (B, 1, C_out, H, W):
            raise ValueError(f"unpatchify: out must be [{B}, 1, {C_out}, {H}, {W}]")
        if out.stride()[2:] != (H * W, W, 1) or out.stride(0) < C_out * H * W:
            raise ValueError("unpatchify: every frame of out must be contiguous")
        if not out.is_cuda:
            raise RuntimeError("libnsw ops run on the GPU only")
        bstride = out.stride(0)
        dst = out
    else:
        dst = torch.empty(B, 1, C_out, H, W, dtype=dtype or y.dtype, device=y.device)
        bstride = C_out * H * W
    dev = _dev(y)
    if dst.device != dev:
        raise RuntimeError("libnsw op arguments are on different devices")
    check(lib().nsw_unpatchify(y.data_ptr(), dst.data_ptr(), B, C_out, H, W, p, bstride, dtype_code(y),
                               dtype_code(dst), _stream(dev)), "unpatchify")
    return dst


def head_weight_perm(weight: torch.Tensor, C_out: int, p: int) -> torch.Tensor:
    """The head weight [p*p*C_out, E] (reference row (u*p + v)*C_out + c,
    models/swin.py:201-209,293-299) with its rows reordered to c*p*p + u*p + v,
    the order nsw_head_unpatchify takes."""
    E = weight.shape[-1]
    if weight.shape[0] != p * p * C_out:
        raise ValueError(f"head weight has {weight.shape[0]} rows, expected p*p*C_out = {p * p * C_out}")
    return weight.view(p * p, C_out, E).transpose(0, 1).reshape(C_out * p * p, E).contiguous()


def head_unpatchify(x: torch.Tensor, w_perm: torch.Tensor, B: int, C_out: int, H: int, W: int, p: int,
                    dtype: Optional[torch.dtype] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """unpatchify(x . W^T) in one launch: x [B*(H/p)*(W/p), E] tokens, w_perm
    from head_weight_perm -> [B, 1, C_out, H, W] in ``dtype`` (x's dtype or
    float32), or into ``out`` (frames contiguous, e.g. one slot of a ring
    buffer) in out's dtype."""
    if x.dim() != 2 or x.shape[0] != B * (H // p) * (W // p):
        raise ValueError("head_unpatchify: x must be [B*(H/p)*(W/p), E]")
    if w_perm.shape != (C_out * p * p, x.shape[1]):
        raise ValueError(f"head_unpatchify: w_perm must be [{C_out * p * p}, {x.shape[1]}]")
    if out is not None:
        if tuple(out.shape) != (B, 1, C_out, H, W):
            raise ValueError(f"head_unpatchify: out must be [{B}, 1, {C_out}, {H}, {W}]")
        if out.stride()[2:] != (H * W, W, 1) or out.stride(0) < C_out * H * W:
            raise ValueError("head_unpatchify: every frame of out must be contiguous")
        bstride = out.stride(0)
        dst = out
    else:
        dst = torch.empty(B, 1, C_out, H, W, dtype=dtype or x.dtype, device=x.device)
        bstride = C_out * H * W
    dev = _dev(x, w_perm)
    if dst.device != dev:
        raise RuntimeError("libnsw op arguments are on different devices")
    _same_dtype(x, w_perm)
    check(lib().nsw_head_unpatchify(x.data_ptr(), w_perm.data_ptr(), dst.data_ptr(), B, C_out, H, W, p,
                                    x.shape[1], bstride, dtype_code(x), dtype_code(dst), _stream(dev)),
          "head_unpatchify")
    return dst


def skip_conv_accumulate(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor,
                         invariants: Optional[torch.Tensor] = None, frame0: int = 0,
                         model_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """The big skip of SwinTransformer.forward (models/swin.py:310-319) in
    place: out [B, 1, C_out, H, W] += Conv2d 1x1 (``weight`` [C_out, C_in]
    or [C_out, C_in, 1, 1], no bias) of x's last frame (ring slot (T - 1 +
    frame0) mod T of x [B, T, C_x, H, W]) with the invariant planes
    [C_inv, H, W] appended; values rounded to ``model_dtype`` (weight's
    dtype by default) as the reference's model-dtype conv and add."""
    if x.dim() != 5 or out.dim() != 5:
        raise ValueError("skip_conv_accumulate: x and out must be [B, T, C, H, W] / [B, 1, C_out, H, W]")
    B, T, C_x, H, W = x.shape
    C_inv = 0 if invariants is None else invariants.shape[0]
    w2 = weight.reshape(weight.shape[0], -1)
    C_out = w2.shape[0]
    if w2.shape[1] != C_x + C_inv:
        raise ValueError(f"skip_conv_accumulate: weight has {w2.shape[1]} input channels, x + invariants "
                         f"{C_x + C_inv}")
    if tuple(out.shape) != (B, 1, C_out, H, W) or out.stride()[2:] != (H * W, W, 1):
        raise ValueError(f"skip_conv_accumulate: out must be [{B}, 1, {C_out}, {H}, {W}] with contiguous frames")
    if invariants is not None and (tuple(invariants.shape) != (C_inv, H, W) or invariants.dtype != x.dtype):
        raise ValueError("skip_conv_accumulate: invariants must be [C_inv, H, W] in x's dtype")
    xc = x.contiguous()
    inv = None if invariants is None else invariants.contiguous()
    wf = w2.detach().to(torch.float32).contiguous()
    dev = _dev(xc, wf, inv)
    if out.device != dev:                      # out may be a strided ring slot (frames contiguous)
        raise RuntimeError("libnsw op arguments are on different devices")
    md = model_dtype or weight.dtype
    check(lib().nsw_skip_conv_accumulate(xc.data_ptr(), _p(inv), wf.data_ptr(), out.data_ptr(), B, T, C_x, C_inv,
                                         C_out, H, W, int(frame0), out.stride(0), dtype_code(xc),
                                         _lib.NSW_DTYPE_BF16 if md == torch.bfloat16 else _lib.NSW_DTYPE_F32,
                                         dtype_code(out), _stream(dev)), "skip_conv_accumulate")
    return out


def weighted_metrics_unnorm(pred: torch.Tensor, target: torch.Tensor, std: torch.Tensor, mean: torch.Tensor,
                            weights: torch.Tensor, clim: Optional[torch.Tensor] = None):
    """Weighted RMSE (and ACC with ``clim``) of pred * std + mean against
    target * std + mean, per (b, t, c), float64 [B, T, C].  pred fp32 or
    bf16, target fp32, std / mean per channel; float64 std or mean (stats
    read from a float64 file) make the unnormalised fields float64, as the
    reference's type promotion does, otherwise they are fp32."""
    if pred.shape != target.shape or pred.dim() != 5:
        raise ValueError("pred and target must be [B, T, C, H, W] of the same shape")
    if target.dtype != torch.float32:
        raise TypeError("target must be float32")
    B, T, C, H, W = pred.shape
    dev = _dev(pred, target)
    w = weights.to(device=dev, dtype=torch.float64).contiguous()
    if w.numel() == H:
        w_cols = 1
    elif w.numel() == H * W and (w.dim() < 2 or tuple(w.shape[-2:]) == (H, W)):
        w_cols = W
    else:
        raise ValueError(f"weights of shape {tuple(weights.shape)} do not match a {H}x{W} field")
    f64 = torch.float64 in (torch.as_tensor(std).dtype, torch.as_tensor(mean).dtype)
    sdt = torch.float64 if f64 else torch.float32
    sc = torch.as_tensor(std).reshape(-1).to(device=dev, dtype=sdt).contiguous()
    of = torch.as_tensor(mean).reshape(-1).to(device=dev, dtype=sdt).contiguous()
    if sc.numel() != C or of.numel() != C:
        raise ValueError("std and mean must have one value per channel")
    if clim is not None:
        clim = clim.reshape(-1).to(device=dev, dtype=torch.float32).contiguous()
        if clim.numel() != C:
            raise ValueError("climatology must have one value per channel")
    P = B * T * C
    rmse = torch.empty(P, dtype=torch.float64, device=dev)
    acc = torch.empty(P, dtype=torch.float64, device=dev) if clim is not None else None
    nbytes = lib().nsw_weighted_metrics_workspace_size(P, H, W)
    ws = workspace(max(nbytes, 8), dev)
    fn = lib().nsw_weighted_metrics_unnorm_f64stats if f64 else lib().nsw_weighted_metrics_unnorm
    check(fn(pred.data_ptr(), dtype_code(pred), target.data_ptr(), sc.data_ptr(), of.data_ptr(), w.data_ptr(),
             w_cols, _p(clim), P, H, W, C, rmse.data_ptr(), _p(acc), ws.data_ptr(), ws.numel(), _stream(dev)),
          "weighted_metrics_unnorm")
    rmse = rmse.view(B, T, C)
    return rmse, (acc.view(B, T, C) if acc is not None else None)
