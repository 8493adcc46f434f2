"""Named profiler ranges around the forward passes (utils/profiler_utils.py).

The reference wraps `SwinTransformer.prepare_tokens` / `forward_head` /
`forward`, `Block._shifted_window_attn` and `MLP.forward` in NVTX ranges
(`@profile`, utils/profiler_utils.py:82-89; used at models/swin.py:269,286,
301, models/swin_helpers.py:399, models/mlp.py:75) that a global profiler
turns on for chosen ranks and an epoch (:9-53).  Here the ranges go through
`torch.cuda.nvtx`, which on ROCm records roctx ranges (`rocprofv3
--marker-trace` shows them around the kernels each forward launches).

Same interface: `init_profiler(cfg)` with `cfg.profiler.enabled`,
`.profile_ranks`, `.profile_epoch` (attribute or dict access), `get_profiler()`
(a no-op profiler until initialised), `profile(name)` and `profile_range(name)`.
The rank is `RANK` from the environment (one process per GPU; 0 alone).
While no profiler is enabled the decorator calls the function directly, so
the decorated modules still trace under `torch.compile(fullgraph=True)`.
"""
from __future__ import annotations

import functools
import os
from contextlib import contextmanager

import torch


def _get(cfg, key, default=None):
    if cfg is None:
        return default
    if isinstance(cfg, dict):
        return cfg.get(key, default)
    return getattr(cfg, key, default)


class Profiler:
    """utils/profiler_utils.py:9-53: ranges on the ranks in profile_ranks;
    the device profiler (roctracer's start/stop through torch.cuda.profiler)
    around the epoch profile_epoch."""

    def __init__(self, cfg):
        pc = _get(cfg, "profiler", cfg)
        self.enabled = bool(_get(pc, "enabled", False))
        self.profile_ranks = list(_get(pc, "profile_ranks", [0]) or [])
        self.profile_epoch = int(_get(pc, "profile_epoch", 0))
        self.current_rank = int(os.environ.get("RANK", "0"))
        self.current_epoch = 0
        self.is_profiling = False

    def should_profile(self) -> bool:
        return self.enabled and self.current_rank in self.profile_ranks

    def should_start_cuda_profiler(self) -> bool:
        return self.should_profile() and self.current_epoch == self.profile_epoch

    def set_epoch(self, epoch: int) -> None:
        if self.is_profiling:
            torch.cuda.profiler.stop()
            self.is_profiling = False
        self.current_epoch = epoch
        if self.should_start_cuda_profiler():
            torch.cuda.profiler.start()
            self.is_profiling = True

    @contextmanager
    def profile_range(self, name: str):
        if not self.should_profile():
            yield
            return
        torch.cuda.nvtx.range_push(name)
        try:
            yield
        finally:
            torch.cuda.nvtx.range_pop()


class NoOpProfiler:
    enabled = False

    def should_profile(self) -> bool:
        return False

    def set_epoch(self, _epoch: int) -> None:
        pass

    @contextmanager
    def profile_range(self, _name: str):
        yield


_profiler = None


def init_profiler(cfg) -> Profiler:
    """Set the global profiler (utils/profiler_utils.py:68-72)."""
    global _profiler
    _profiler = Profiler(cfg)
    return _profiler


def get_profiler():
    return _profiler if _profiler is not None else NoOpProfiler()


def profile(name: str | None = None):
    """Decorator: run the function inside a named range when profiling."""
    def decorator(func):
        label = name or func.__name__

        @functools.wraps(func)
        def wrapper(*args, **kwargs):
            prof = get_profiler()
            if not prof.should_profile():
                return func(*args, **kwargs)
            with prof.profile_range(label):
                return func(*args, **kwargs)
        return wrapper
    return decorator


@contextmanager
def profile_range(name: str):
    with get_profiler().profile_range(name):
        yield
