"""``MLP`` (models/mlp.py:14-95): fc1 -> +bias1 -> GELU -> fc2 -> +bias2.

Two libnsw GEMM launches: fc1 with the bias + GELU epilogue, fc2 with the
bias epilogue.  The GELU is ``act_layer``'s: nn.GELU() (exact erf, the
reference's default) or nn.GELU(approximate="tanh") (the form of the
reference's Transformer-Engine block, models/swin_helpers_te.py:318-323).
Dropout is the identity in eval (p = 0 in every config); a training-mode
dropout with p > 0 is not implemented and raises.
"""
from __future__ import annotations

import torch
from torch import nn

from . import _lib, torch_ops
from .layer_helpers import BiasLayer, LinearLayer
from .profiler_utils import profile


class MLP(nn.Module):
    def __init__(self, in_features, hidden_features=None, out_features=None, act_layer=nn.GELU, drop=0.0):
        super().__init__()
        out_features = out_features or in_features
        hidden_features = hidden_features or in_features
        self.fc1 = LinearLayer(in_features, hidden_features,
                               comm_metadata={"sharded": ["tp", None], "shared": ["sp1-sp2"], "reduce": ["sp1-sp2"]})
        self.bias1 = BiasLayer(hidden_features,
                               comm_metadata={"sharded": ["tp"], "shared": ["sp1-sp2"], "reduce": ["sp1-sp2"]})
        self.act = act_layer()
        self.fc2 = LinearLayer(hidden_features, out_features,
                               comm_metadata={"sharded": [None, "tp"], "shared": ["sp1-sp2"], "reduce": ["sp1-sp2"]})
        self.bias2 = BiasLayer(out_features,
                               comm_metadata={"sharded": [], "shared": ["tp-sp1-sp2"], "reduce": ["sp1-sp2"]})
        self.drop = nn.Dropout(drop)

    def _check_fusable(self):
        if not (isinstance(self.act, nn.GELU) and self.act.approximate in ("none", "tanh")):
            raise NotImplementedError("libnsw fuses nn.GELU (approximate 'none' or 'tanh') only")
        if self.training and self.drop.p > 0:
            raise NotImplementedError("dropout with p > 0 in training mode is not implemented")

    @property
    def gelu_tanh(self) -> bool:
        return self.act.approximate == "tanh"

    @property
    def gelu_epilogue(self) -> int:
        return _lib.NSW_EPI_BIAS_GELU_TANH if self.gelu_tanh else _lib.NSW_EPI_BIAS_GELU

    @profile("mlp")
    def forward(self, x, residual=None):
        """``residual`` (same shape as the output) is added in fc2's epilogue;
        the reference adds the block's skip right after the MLP
        (models/swin_helpers.py:456)."""
        self._check_fusable()
        x = x.contiguous()
        h = torch_ops.linear_epi(x, self.fc1.weight, self.bias1.bias, epilogue=self.gelu_epilogue)
        if residual is None:
            return torch_ops.linear_epi(h, self.fc2.weight, self.bias2.bias, epilogue=_lib.NSW_EPI_BIAS)
        return torch_ops.linear_epi(h, self.fc2.weight, self.bias2.bias, residual=residual,
                                    epilogue=_lib.NSW_EPI_BIAS_RESIDUAL)
