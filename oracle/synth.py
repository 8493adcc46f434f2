"""Seeded synthetic inputs and reference-style weights (test oracle only).

Weights follow the reference init: Linear weights ``trunc_normal_(std=0.02)``
with absolute bounds [-2, 2] (models/timm_helpers.py:46-98, called from
models/layer_helpers.py:36-37), biases zero (layer_helpers.py:68), RMSNorm
weights one (models/swin.py:263-266).  The truncated normal uses the inverse
CDF method the reference uses (uniform on [2l-1, 2u-1] -> erfinv -> scale ->
clamp).  Everything is drawn in fp32 from a CPU ``torch.Generator``; seeds are
1000*k + {1: weights, 2: activations, 3: target, 4: climatology}.
"""
from __future__ import annotations

import math
from typing import Dict

import torch

from .swin_ref import BLOCK_PARAM_SHAPES


def trunc_normal(shape, std: float, gen: torch.Generator, mean: float = 0.0,
                 a: float = -2.0, b: float = 2.0) -> torch.Tensor:
    def cdf(v):
        return (1.0 + math.erf(v / math.sqrt(2.0))) / 2.0
    lo, hi = cdf((a - mean) / std), cdf((b - mean) / std)
    t = torch.empty(shape, dtype=torch.float32)
    t.uniform_(2 * lo - 1, 2 * hi - 1, generator=gen)
    t.erfinv_()
    t.mul_(std * math.sqrt(2.0)).add_(mean)
    return t.clamp_(min=a, max=b)


def block_params(C: int, num_heads: int, mlp_ratio: float = 4.0, seed: int = 1,
                 random_bias: bool = False, random_norm: bool = False) -> Dict[str, torch.Tensor]:
    """Reference-initialised parameters of one block (vanilla key names).
    ``random_bias`` / ``random_norm`` replace the zero biases / unit norm
    weights with random values so that tests exercise those terms."""
    g = torch.Generator().manual_seed(seed)
    hd = C // num_heads
    Hm = int(C * mlp_ratio)
    p = {}
    for name, shp in BLOCK_PARAM_SHAPES.items():
        shape = shp(C, hd, Hm)
        if name.endswith(".weight") and len(shape) == 2:
            p[name] = trunc_normal(shape, 0.02, g)
        elif name.endswith(".bias"):
            p[name] = (torch.randn(shape, generator=g) * 0.1) if random_bias else torch.zeros(shape)
        else:  # norm weights
            p[name] = (1.0 + 0.2 * torch.randn(shape, generator=g)) if random_norm else torch.ones(shape)
    return p


def activations(shape, seed: int = 2) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32)


def model_params(in_chans: int, out_chans: int, embed_dim: int, depth: int, num_heads: int,
                 patch_size: int, mlp_ratio: float = 4.0, seed: int = 1, coord_pos_embed: bool = True,
                 pos_shape=None, random_bias: bool = False, random_norm: bool = False,
                 big_skip: bool = False) -> Dict[str, torch.Tensor]:
    """Reference-initialised SwinTransformer parameters (state-dict names of
    models/swin.py:120-209): conv weights trunc_normal(0.02) with zero biases
    (models/swin.py:246-256), the learned ``pos_embed`` trunc_normal(0.02)
    when ``coord_pos_embed`` is False (``pos_shape`` = [1, T, h, w, E]), and
    with ``big_skip`` the 1x1 skip convolution's weight."""
    g = torch.Generator().manual_seed(seed)
    p = patch_size
    out: Dict[str, torch.Tensor] = {}

    def bias(n):
        return (torch.randn(n, generator=g) * 0.1) if random_bias else torch.zeros(n)

    out["patch_embed.proj.conv.weight"] = trunc_normal((embed_dim, in_chans, p, p), 0.02, g)
    out["patch_embed.proj.conv.bias"] = bias(embed_dim)
    if coord_pos_embed:
        out["pos_embed.proj.conv.weight"] = trunc_normal((embed_dim, 4, p, p), 0.02, g)
        out["pos_embed.proj.conv.bias"] = bias(embed_dim)
    else:
        out["pos_embed"] = trunc_normal(tuple(pos_shape), 0.02, g)
    for i in range(depth):
        bp = block_params(embed_dim, num_heads, mlp_ratio, seed=seed * 7919 + i, random_bias=random_bias,
                          random_norm=random_norm)
        out.update({f"blocks.{i}.{k}": v for k, v in bp.items()})
    out["head.weight"] = trunc_normal((out_chans * p * p, embed_dim), 0.02, g)
    if big_skip:   # models/swin.py:212-223: Conv2d 1x1, no bias, trunc_normal(0.02) like every conv
        out["skip_conv.conv.weight"] = trunc_normal((out_chans, in_chans, 1, 1), 0.02, g)
    return out


def smooth_field(shape, sigma: float, seed: int) -> torch.Tensor:
    """Per-channel standardised Gaussian-filtered noise [..., H, W]: a seeded
    N(0, 1) field convolved with a Gaussian of ``sigma`` pixels (FFT,
    periodic in both directions), then standardised to zero mean and unit
    variance per leading index.  Stands in for ERA5 fields."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g, dtype=torch.float64)
    H, W = shape[-2], shape[-1]
    ky = torch.fft.fftfreq(H, dtype=torch.float64).view(H, 1)
    kx = torch.fft.rfftfreq(W, dtype=torch.float64).view(1, -1)
    filt = torch.exp(-2.0 * (math.pi * sigma) ** 2 * (ky ** 2 + kx ** 2))
    y = torch.fft.irfft2(torch.fft.rfft2(x) * filt, s=(H, W))
    y = y - y.mean(dim=(-2, -1), keepdim=True)
    y = y / y.std(dim=(-2, -1), keepdim=True)
    return y.float()
