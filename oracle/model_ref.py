"""fp32 CPU restatement of the reference SwinTransformer forward and its
rollout (test oracle only: imported by tests/, smoke() and bench.py's CPU
baseline, never by the product path).

Reference routines (ShashankSubramanian/neural-scaling-weather):
  * get_spatial_coords            utils/misc_utils.py:14-26
  * SwinTransformer._init_coords  models/swin.py:227-244
  * PatchEmbedLayer / Conv2DLayer models/layer_helpers.py:120-172
  * SwinTransformer.prepare_tokens models/swin.py:269-284
  * SwinTransformer.forward_head  models/swin.py:286-299
  * SwinTransformer.forward       models/swin.py:301-323 (blocks built at
                                  :179-199: shift (0, 0) for even i, (ws0//2,
                                  ws1//2) for odd i)
  * TimeStepper.forward           models/helpers.py:18-37
  * inference step                utils/inferencer.py:393-449 with the
                                  preprocessor of utils/data_utils.py:175-197

Pinning (tests/test_oracle_model.py): the patch embedding is checked against
an im2col matrix product built by brute-force loops (two independent
formulations of the strided convolution); unpatchify against a per-element
loop; the coordinates against closed-form values (poles, equator, prime
meridian); the model composition against special cases (zero blocks ->
head(embed(x)) in closed form, T = 1 -> last-frame selection is the
identity); the rollout against a hand-unrolled two-step loop.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from . import swin_ref


def spatial_coords(lat_deg: torch.Tensor, lon_deg: torch.Tensor) -> torch.Tensor:
    """``get_spatial_coords`` (utils/misc_utils.py:14-26): unit-sphere (x, y, z)
    of every (lat, lon) grid point, [nlat, nlon, 3]."""
    lat, lon = torch.meshgrid(lat_deg.double(), lon_deg.double(), indexing="ij")
    la, lo = torch.deg2rad(lat), torch.deg2rad(lon)
    return torch.stack((torch.cos(la) * torch.cos(lo), torch.cos(la) * torch.sin(lo), torch.sin(la)),
                       dim=-1).float()


def model_coords(spatial: torch.Tensor, T: int) -> torch.Tensor:
    """``_init_coords`` (models/swin.py:227-244): [T, H, W, 4] = spatial
    coordinates with t = linspace(0, 1, T) appended."""
    H, W, _ = spatial.shape
    t = torch.linspace(0, 1, T).view(T, 1, 1, 1).expand(-1, H, W, 1)
    return torch.cat([spatial.unsqueeze(0).expand(T, -1, -1, -1), t], dim=-1)


def patch_conv(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], p: int) -> torch.Tensor:
    """``PatchEmbedLayer.forward`` = ``Conv2d(k=p, stride=p)``
    (models/layer_helpers.py:138-172): [N, C, H, W] -> [N, E, H/p, W/p].
    On a GPU device the same convolution is evaluated by
    :func:`patch_conv_unfold` (no run-time convolution kernel compilation)."""
    if x.device.type == "cpu":
        return F.conv2d(x, weight, bias, stride=p)
    return patch_conv_unfold(x, weight, bias, p)


def patch_conv_unfold(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], p: int) -> torch.Tensor:
    """The stride-p convolution as ``F.unfold`` (the patch matrix, columns in
    the (c, u, v) order of the flattened Conv2d weight) times the weight
    (tests check it against ``F.conv2d`` and a brute-force im2col)."""
    N, C, H, W = x.shape
    E = weight.shape[0]
    cols = F.unfold(x, kernel_size=p, stride=p)                     # [N, C*p*p, h*w]
    y = torch.matmul(weight.reshape(E, -1), cols)                   # [N, E, h*w]
    if bias is not None:
        y = y + bias.view(1, E, 1)
    return y.view(N, E, H // p, W // p)


def prepare_tokens(x: torch.Tensor, pe_w: torch.Tensor, pe_b: torch.Tensor, p: int,
                   pos: torch.Tensor) -> torch.Tensor:
    """``prepare_tokens`` (models/swin.py:269-284).  ``pos`` is either the
    coordinate embedding [T, h, w, E] (``pos_tokens``) or the learned
    parameter [1, T, h, w, E]; both broadcast over the batch."""
    b, t, c, h, w = x.shape
    y = patch_conv(x.reshape(-1, c, h, w), pe_w, pe_b, p)
    E = y.shape[1]
    y = y.view(b, t, E, h // p, w // p)
    y = torch.einsum("btchw->bthwc", y)
    return y + pos


def pos_tokens(coords: torch.Tensor, pos_w: torch.Tensor, pos_b: torch.Tensor, p: int) -> torch.Tensor:
    """Coordinate positional embedding (models/swin.py:278-282): the patch
    convolution of the [T, H, W, 4] coordinates, as [T, h, w, E]."""
    pos = torch.einsum("thwc->tchw", coords)
    pos = patch_conv(pos, pos_w, pos_b, p)
    return torch.einsum("tchw->thwc", pos)


def forward_head(x: torch.Tensor, head_w: torch.Tensor, p: int, out_chans: int) -> torch.Tensor:
    """``forward_head`` (models/swin.py:286-299): Linear E -> C_out*p*p (no
    bias), then [b,t,h,w,p,p,c] -> [b,t,c,h*p,w*p]."""
    b, t, h, w, c = x.shape
    y = F.linear(x.contiguous(), head_w)
    y = y.reshape(b, t, h, w, p, p, out_chans)
    y = torch.einsum("nthwpqc->ntchpwq", y)
    return y.reshape(b, t, out_chans, h * p, w * p)


def block_shift(i: int, window_size: Tuple[int, int]) -> Tuple[int, int]:
    """Shift schedule of the block list (models/swin.py:187-189)."""
    return (0, 0) if i % 2 == 0 else tuple(wv // 2 for wv in window_size)


def model_forward(x: torch.Tensor, params: Dict[str, torch.Tensor], *, patch_size: int,
                  window_size: Tuple[int, int], depth: int, num_heads: int, out_chans: int,
                  coords: Optional[torch.Tensor] = None, eps: Optional[float] = None,
                  gelu: str = "none") -> torch.Tensor:
    """``SwinTransformer.forward`` (models/swin.py:301-323); with a
    ``skip_conv.conv.weight`` in ``params`` the big skip convolution
    (``use_big_skip_conv=True``, :305-319) is applied to every frame of the
    input and added to the head's image before the last frame is taken.  ``params``
    uses the reference's state-dict names; ``coords`` is [T, H, W, 4] for the
    coordinate embedding, None for a learned ``pos_embed`` parameter.  ``eps``
    is the blocks' RMSNorm eps: nn.RMSNorm(eps=None) takes finfo(dtype).eps
    of the tensors it runs on, so a model run in bf16 uses 2**-7 (None: the
    fp32 value)."""
    p = patch_size
    if coords is not None:
        pos = pos_tokens(coords, params["pos_embed.proj.conv.weight"], params["pos_embed.proj.conv.bias"], p)
    else:
        pos = params["pos_embed"]
    y = prepare_tokens(x, params["patch_embed.proj.conv.weight"], params["patch_embed.proj.conv.bias"], p, pos)
    for i in range(depth):
        bp = {k[len(f"blocks.{i}."):]: v for k, v in params.items() if k.startswith(f"blocks.{i}.")}
        y = swin_ref.block_forward(y, bp, num_heads, window_size, block_shift(i, window_size), eps=eps,
                                   gelu=gelu)
    y = forward_head(y, params["head.weight"], p, out_chans)
    if "skip_conv.conv.weight" in params:
        b, t, c, h, w = x.shape
        skip = F.conv2d(x.reshape(b * t, c, h, w), params["skip_conv.conv.weight"])
        y = y + skip.view(b, t, out_chans, h, w)
    return y[:, -1:]


def stepper_forward(model, inp: torch.Tensor, num_rollout_steps: int, num_invariants: int) -> torch.Tensor:
    """``TimeStepper.forward`` (models/helpers.py:18-37): feed each
    prediction back with the invariant channels re-appended; predictions
    concatenated along time."""
    result: List[torch.Tensor] = []
    inpt = inp
    c_in = inp.shape[2]
    for _ in range(num_rollout_steps):
        pred = model(inpt)
        c_out = pred.shape[2]
        result.append(pred)
        n_inv = c_in - c_out
        assert n_inv == num_invariants, "number of invariants does not match"
        inpt = torch.cat([pred, inp[:, :, c_in - n_inv:]], dim=2) if n_inv > 0 else pred
    return torch.cat(result, dim=1)


def rollout(model, input_window: torch.Tensor, invariants: Optional[torch.Tensor], targets: torch.Tensor,
            mean: torch.Tensor, std: torch.Tensor, w_lat, clim: Optional[torch.Tensor] = None):
    """One initial condition of the inference loop (utils/inferencer.py:393-449):
    per lead step i, inputs = window with invariants appended (data_utils.py:
    185-197, mode "inference"); gen = model(inputs); pred = gen*std + mean;
    target_i*std + mean; RMSE (and, with ``clim``, ACC) per channel; the
    window rolls by one frame and takes gen.  ``targets`` [S, C, H, W] are
    normalised fields, ``mean`` / ``std`` [C], ``w_lat`` the area weights.
    Returns (rmse [S, C], acc [S, C] or None, gens [S, C, H, W])."""
    import numpy as np

    from . import metrics_ref

    win = input_window.clone()
    S = targets.shape[0]
    rm, ac, gens = [], [], []
    dev = input_window.device
    ms, ss = mean.view(1, 1, -1, 1, 1).to(dev), std.view(1, 1, -1, 1, 1).to(dev)
    for i in range(S):
        inp = win
        if invariants is not None:
            B, T, _, H, W = win.shape
            inv = invariants.to(dev).view(1, 1, -1, H, W).expand(B, T, -1, H, W)
            inp = torch.cat([win, inv], dim=2)
        gen = model(inp)
        pred = gen.float() * ss + ms
        targ = targets[i].view(1, 1, *targets.shape[1:]).to(dev).float() * ss + ms
        pn, tn = pred.double().cpu().numpy(), targ.double().cpu().numpy()
        rm.append(metrics_ref.weighted_rmse(pn, tn, np.asarray(w_lat)))
        if clim is not None:
            ac.append(metrics_ref.weighted_acc(pn, tn, np.asarray(w_lat), clim.double().cpu().numpy()))
        gens.append(gen[0, 0].float())
        win = torch.roll(win, shifts=-1, dims=1)
        win[:, -1] = gen[:, 0].to(win.dtype)
    rmse = torch.from_numpy(np.stack(rm))
    acc = torch.from_numpy(np.stack(ac)) if clim is not None else None
    return rmse, acc, torch.stack(gens)


# ----------------------------------------------------------------------------
# brute-force index formulations (pins for the strided convolution and the
# head's unpatchify)
# ----------------------------------------------------------------------------


def im2col_bruteforce(x: torch.Tensor, p: int) -> torch.Tensor:
    """Patch matrix of ``x`` [N, C, H, W]: row (n, i, j) holds the C*p*p
    values x[n, c, i*p + u, j*p + v] in (c, u, v) order (the flattening
    order of a Conv2d weight [E, C, p, p])."""
    N, C, H, W = x.shape
    h, w = H // p, W // p
    out = torch.empty(N * h * w, C * p * p, dtype=x.dtype)
    for n in range(N):
        for i in range(h):
            for j in range(w):
                r = (n * h + i) * w + j
                k = 0
                for c in range(C):
                    for u in range(p):
                        for v in range(p):
                            out[r, k] = x[n, c, i * p + u, j * p + v]
                            k += 1
    return out


def unpatchify_bruteforce(y: torch.Tensor, b: int, t: int, h: int, w: int, p: int, c_out: int) -> torch.Tensor:
    """Inverse layout of the head: y [(b, t, i, j), (u, v, c)] ->
    out [b, t, c, i*p + u, j*p + v], element by element."""
    out = torch.empty(b, t, c_out, h * p, w * p, dtype=y.dtype)
    for bb in range(b):
        for tt in range(t):
            for i in range(h):
                for j in range(w):
                    r = ((bb * t + tt) * h + i) * w + j
                    for u in range(p):
                        for v in range(p):
                            for c in range(c_out):
                                out[bb, tt, c, i * p + u, j * p + v] = y[r, (u * p + v) * c_out + c]
    return out
