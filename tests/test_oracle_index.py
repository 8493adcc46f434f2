"""Pins the oracle's index work (roll, partition, reverse, fused gather/scatter,
shift mask) bit-exactly: closed forms vs brute-force loops vs the
torch.roll + view/permute composition of the reference."""
import numpy as np
import pytest
import torch

from oracle import index_maps as im
from oracle import swin_ref as ref

SHAPES = [
    # B, T, H, W, ws0, ws1, s0, s1
    (1, 1, 18, 36, 9, 18, 4, 9),
    (2, 1, 18, 36, 9, 18, 0, 0),
    (1, 2, 18, 36, 9, 18, 4, 9),
    (2, 2, 8, 16, 4, 8, 2, 4),
    (1, 1, 12, 12, 3, 4, 1, 2),
    (1, 3, 6, 10, 3, 5, 1, 2),
]


@pytest.mark.parametrize("B,T,H,W,ws0,ws1,s0,s1", SHAPES)
def test_gather_closed_form_vs_bruteforce(B, T, H, W, ws0, ws1, s0, s1):
    a = im.gather_rows(B, T, H, W, ws0, ws1, s0, s1)
    b = im.gather_rows_bruteforce(B, T, H, W, ws0, ws1, s0, s1)
    assert np.array_equal(a, b)
    # a permutation of all tokens (bijection -> scatter is its inverse)
    assert np.array_equal(np.sort(a), np.arange(B * T * H * W))


@pytest.mark.parametrize("B,T,H,W,ws0,ws1,s0,s1", SHAPES)
def test_gather_matches_roll_partition(B, T, H, W, ws0, ws1, s0, s1):
    C = 3
    x = torch.arange(B * T * H * W * C, dtype=torch.float64).reshape(B, T, H, W, C)
    xr = ref.roll(x, (-s0, -s1), (-3, -2))
    xw = ref.window_partition(xr, (ws0, ws1)).reshape(-1, C)
    idx = im.gather_rows(B, T, H, W, ws0, ws1, s0, s1)
    assert torch.equal(xw, x.reshape(-1, C)[torch.from_numpy(idx)])


@pytest.mark.parametrize("B,T,H,W,ws0,ws1,s0,s1", SHAPES)
def test_scatter_is_reverse_unroll(B, T, H, W, ws0, ws1, s0, s1):
    C = 2
    nW = B * (H // ws0) * (W // ws1)
    o = torch.randn(nW, T, ws0, ws1, C, dtype=torch.float64)
    y = ref.roll(ref.window_reverse(o, (ws0, ws1), (H, W)), (s0, s1), (-3, -2))
    idx = torch.from_numpy(im.gather_rows(B, T, H, W, ws0, ws1, s0, s1))
    y2 = torch.empty(B * T * H * W, C, dtype=torch.float64)
    y2[idx] = o.reshape(-1, C)
    assert torch.equal(y.reshape(-1, C), y2)


@pytest.mark.parametrize("B,T,H,W,ws0,ws1,s0,s1", SHAPES)
def test_partition_reverse_roundtrip(B, T, H, W, ws0, ws1, s0, s1):
    # reference test: tests/test_windows.py:67-76 (serial half)
    x = torch.randn(B, T, H, W, 5)
    assert torch.equal(ref.window_reverse(ref.window_partition(x, (ws0, ws1)), (ws0, ws1), (H, W)), x)


def test_roll_index_matches_torch_roll():
    H, W = 7, 11
    x = torch.arange(H * W).reshape(H, W)
    for s0, s1 in [(0, 0), (3, -4), (-2, 5), (7, 11)]:
        idx = im.roll_index(H, W, s0, s1)
        assert torch.equal(torch.roll(x, (s0, s1), (0, 1)).reshape(-1), x.reshape(-1)[torch.from_numpy(idx)])


def test_roll_skips_zero_shift_and_composes():
    x = torch.randn(1, 1, 6, 8, 2)
    assert torch.equal(ref.roll(x, (0, 0), (-3, -2)), x)
    assert torch.equal(ref.roll(ref.roll(x, (-2, -3), (-3, -2)), (2, 3), (-3, -2)), x)


@pytest.mark.parametrize("T", [1, 2])
@pytest.mark.parametrize("H,W,ws0,ws1,s0,s1", [
    (18, 36, 9, 18, 4, 9), (18, 36, 9, 18, 0, 0), (12, 8, 4, 4, 2, 2), (9, 10, 3, 5, 1, 2)])
def test_mask_closed_form_vs_bruteforce_vs_restatement(T, H, W, ws0, ws1, s0, s1):
    a = im.mask_closed_form(H, W, ws0, ws1, s0, s1, T)
    b = im.mask_bruteforce(H, W, ws0, ws1, s0, s1, T)
    c = ref.make_attention_mask(H, W, (ws0, ws1), (s0, s1), T).numpy()
    assert np.array_equal(a, b)
    assert np.array_equal(a, c)


def test_mask_special_cases():
    H, W, ws0, ws1, s0, s1 = 180, 360, 9, 18, 4, 9
    m = im.mask_closed_form(H, W, ws0, ws1, s0, s1)
    assert m.shape == (400, 162, 162)
    assert set(np.unique(m).tolist()) <= {0.0, -100.0}
    nz = np.nonzero(m.reshape(400, -1).any(axis=1))[0]
    assert nz.tolist() == list(range(380, 400))   # only the last latitude band
    assert np.array_equal(m, m.transpose(0, 2, 1))  # symmetric
    # unshifted block: all zero
    assert not im.mask_closed_form(H, W, ws0, ws1, 0, 0).any()
    # in the last band, rows r >= ws0 - s0 (= 5) form one group: 4 rows x 18 = 72 tokens
    lab = (np.arange(162) // 18) >= 5
    assert lab.sum() == 72
    assert (m[399][lab][:, ~lab] == -100.0).all() and (m[399][lab][:, lab] == 0).all()
