"""Profiler ranges (utils/profiler_utils.py): the decorator is a plain call
until a profiler is enabled for this rank, then pushes / pops one named range
around the call; the reference's range names sit on the same functions
(models/swin.py:269,286,301, models/swin_helpers.py:399, models/mlp.py:75)."""
import pytest
import torch

from nsw import profiler_utils as pu


@pytest.fixture(autouse=True)
def reset_profiler(monkeypatch):
    monkeypatch.setattr(pu, "_profiler", None)
    calls = []
    monkeypatch.setattr(torch.cuda.nvtx, "range_push", lambda name: calls.append(("push", name)))
    monkeypatch.setattr(torch.cuda.nvtx, "range_pop", lambda: calls.append(("pop",)))
    yield calls


def test_noop_by_default(reset_profiler):
    @pu.profile("x")
    def f(a, b=2):
        return a + b
    assert f(1, b=3) == 4
    assert isinstance(pu.get_profiler(), pu.NoOpProfiler)
    with pu.profile_range("y"):
        pass
    assert reset_profiler == []


def test_ranges_when_enabled(reset_profiler, monkeypatch):
    monkeypatch.setenv("RANK", "0")
    pu.init_profiler({"profiler": {"enabled": True, "profile_ranks": [0], "profile_epoch": 3}})

    @pu.profile()
    def g():
        return 7
    assert g() == 7
    with pu.profile_range("blk"):
        pass
    assert reset_profiler == [("push", "g"), ("pop",), ("push", "blk"), ("pop",)]


def test_range_popped_on_error(reset_profiler):
    pu.init_profiler({"profiler": {"enabled": True, "profile_ranks": [0]}})

    @pu.profile("boom")
    def h():
        raise ValueError("x")
    with pytest.raises(ValueError):
        h()
    assert reset_profiler == [("push", "boom"), ("pop",)]


def test_other_rank_and_attribute_config(reset_profiler, monkeypatch):
    class C:
        class profiler:
            enabled = True
            profile_ranks = [1]
            profile_epoch = 0
    monkeypatch.setenv("RANK", "0")
    p = pu.init_profiler(C)
    assert not p.should_profile()
    pu.profile("z")(lambda: None)()
    assert reset_profiler == []


def test_reference_range_names():
    import nsw
    assert nsw.SwinTransformer.forward.__wrapped__ is not None
    for fn in (nsw.SwinTransformer.prepare_tokens, nsw.SwinTransformer.forward_head, nsw.SwinTransformer.forward,
               nsw.Block._shifted_window_attn, nsw.MLP.forward):
        assert hasattr(fn, "__wrapped__"), fn
