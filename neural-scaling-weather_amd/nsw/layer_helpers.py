"""Parameter wrappers with the reference's names (models/layer_helpers.py:8-119).

Same attributes and state-dict keys as the reference (``weight`` of
``LinearLayer``, ``bias`` of ``BiasLayer``, ``norm.weight`` of ``NormLayer``)
and the same init (trunc-normal std 0.02, zero bias, unit norm weight); the
forward passes run libnsw kernels.  ``comm_metadata`` is kept as an attribute
for API compatibility (every communicator has size 1 here).
"""
from __future__ import annotations

import math

import torch
from torch import nn

from . import ops, torch_ops

_DEFAULT_META = {"sharded": [None, None], "shared": [], "reduce": []}


def trunc_normal_(tensor: torch.Tensor, mean: float = 0.0, std: float = 1.0, a: float = -2.0,
                  b: float = 2.0) -> torch.Tensor:
    """Truncated normal by the inverse-CDF method with absolute bounds [a, b]
    (models/timm_helpers.py:46-98)."""
    def cdf(v):
        return (1.0 + math.erf(v / math.sqrt(2.0))) / 2.0
    lo, hi = cdf((a - mean) / std), cdf((b - mean) / std)
    with torch.no_grad():
        tensor.uniform_(2 * lo - 1, 2 * hi - 1)
        tensor.erfinv_()
        tensor.mul_(std * math.sqrt(2.0)).add_(mean)
        tensor.clamp_(min=a, max=b)
    return tensor


class LinearLayer(nn.Module):
    """Bias-free ``F.linear`` (models/layer_helpers.py:8-42)."""

    def __init__(self, in_features, out_features, comm_metadata=None):
        super().__init__()
        self.weight = nn.Parameter(torch.empty((out_features, in_features)))
        self.weight.comm_metadata = comm_metadata or dict(_DEFAULT_META)
        trunc_normal_(self.weight, std=0.02)

    def forward(self, x):
        return torch_ops.linear_epi(x, self.weight)


class BiasLayer(nn.Module):
    """Separate bias add (models/layer_helpers.py:45-72)."""

    def __init__(self, dim, comm_metadata=None):
        super().__init__()
        self.bias = nn.Parameter(torch.zeros(dim))
        self.bias.comm_metadata = comm_metadata or {"sharded": [None], "shared": [], "reduce": []}

    def forward(self, x):
        # y = x . I^T + b would waste a GEMM; the blocks fuse the bias into the
        # producing GEMM's epilogue instead.  Stand-alone use is a broadcast add.
        return x + self.bias


class NormLayer(nn.Module):
    """``NormLayer`` (models/layer_helpers.py:75-119): ``rms_norm`` runs the
    libnsw RMSNorm kernel, ``layer_norm`` the libnsw LayerNorm kernel (same
    parameters and eps as the wrapped nn.RMSNorm / nn.LayerNorm)."""

    def __init__(self, normalized_shape, elementwise_affine=True, norm_type="layer_norm",
                 comm_metadata=None):
        super().__init__()
        self.norm_type = norm_type
        if norm_type == "layer_norm":
            self.norm = nn.LayerNorm(normalized_shape, elementwise_affine=elementwise_affine, bias=True)
        elif norm_type == "rms_norm":
            self.norm = nn.RMSNorm(normalized_shape, elementwise_affine=elementwise_affine)
        else:
            raise ValueError(f"Invalid norm type: {norm_type}")
        if elementwise_affine:
            meta = comm_metadata or {"sharded": [None], "shared": [], "reduce": []}
            self.norm.weight.comm_metadata = meta
            if norm_type == "layer_norm":
                self.norm.bias.comm_metadata = meta

    def forward(self, x):
        if self.norm_type == "layer_norm":
            n = self.norm
            if len(n.normalized_shape) != 1:
                raise NotImplementedError("libnsw normalises over the last dim only")
            return torch.ops.nsw.layer_norm(x, n.weight, n.bias, float(n.eps))
        w = self.norm.weight
        if w is None:
            w = torch.ones(x.shape[-1], dtype=x.dtype, device=x.device)
        eps = self.norm.eps
        return torch.ops.nsw.rms_norm(x, w, ops.default_eps(x.dtype) if eps is None else float(eps))
