"""nsw — MI355X-native shifted-window Swin block of neural-scaling-weather.

Drop-in replacements for the reference's hot-path modules, running HIP
kernels for gfx950 from ``libnsw.so`` through its C ABI (include/nsw.h):

    from nsw import Block, WindowMultiHeadAttention, window_partition, window_reverse
    from nsw import WeightedRMSE, WeightedACC, build_spherical_area_weights
    from nsw import SwinTransformer, TimeStepper, Rollout

Build the library first: ``python neural-scaling-weather_amd/build.py``.
"""
from .layer_helpers import BiasLayer, LinearLayer, NormLayer, trunc_normal_
from .losses import WeightedACC, WeightedRMSE, weighted_rmse_acc
from .misc_utils import build_spherical_area_weights, create_dummy_metadata, get_spatial_coords
from .mlp import MLP
from .swin_helpers import (Block, SwinTransformerBlock, WindowAttention, WindowMultiHeadAttention,
                           roll_forward_reverseroll_backward, window_partition, window_reverse)
from .swin import Conv2DLayer, PatchEmbedLayer, SwinTransformer, TimeStepper, get_model
from .inference import Rollout
from . import checkpoint, ops, profiler_utils, torch_ops   # torch_ops registers torch.ops.nsw.*

__all__ = [
    "Block", "SwinTransformerBlock", "WindowMultiHeadAttention", "WindowAttention", "MLP",
    "LinearLayer", "BiasLayer", "NormLayer", "trunc_normal_", "window_partition", "window_reverse",
    "roll_forward_reverseroll_backward", "WeightedRMSE", "WeightedACC", "weighted_rmse_acc",
    "build_spherical_area_weights", "get_spatial_coords", "create_dummy_metadata", "checkpoint", "ops",
    "SwinTransformer", "PatchEmbedLayer", "Conv2DLayer", "TimeStepper", "get_model", "Rollout", "torch_ops",
    "profiler_utils",
]
