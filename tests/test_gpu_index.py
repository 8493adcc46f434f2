"""GPU parity of the index kernels (bit-exact): roll, window partition /
reverse, fused roll+partition and reverse+roll, the shift mask."""
import numpy as np
import pytest
import torch

from oracle import index_maps as im
from oracle import swin_ref as ref

pytestmark = pytest.mark.gpu

CASES = [
    # B, T, H, W, C, ws, shift
    (1, 1, 180, 360, 1024, (9, 18), (4, 9)),   # config 2 geometry
    (1, 1, 90, 180, 192, (9, 18), (4, 9)),     # config 1 geometry
    (2, 2, 18, 36, 64, (9, 18), (4, 9)),
    (1, 1, 18, 36, 8, (9, 18), (0, 0)),
    (4, 8, 16, 32, 8, (4, 8), (2, 4)),         # reference tests/test_windows.py shape
    (1, 3, 12, 20, 24, (3, 5), (1, 2)),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,H,W,C,ws,shift", CASES)
def test_partition_reverse_roll_bitexact(device, dtype, B, T, H, W, C, ws, shift):
    import nsw
    from nsw import ops
    x = torch.randn(B, T, H, W, C, generator=torch.Generator().manual_seed(1)).to(dtype)
    xd = x.to(device)
    # window_partition / window_reverse
    got = nsw.window_partition(xd, ws).cpu()
    want = ref.window_partition(x, ws)
    assert torch.equal(got, want)
    assert torch.equal(nsw.window_reverse(nsw.window_partition(xd, ws), ws, (H, W)).cpu(), x)
    # torch.roll by (-s0, -s1) and (+s0, +s1)
    for s in [(-shift[0], -shift[1]), shift, (H + 1, -W - 3)]:
        assert torch.equal(ops.roll_hw(xd, s).cpu(), torch.roll(x, s, (-3, -2)))
    # fused roll + partition and reverse + roll
    xw = ops.roll_window_partition(xd, ws, shift)
    assert torch.equal(xw.cpu(), ref.window_partition(ref.roll(x, (-shift[0], -shift[1]), (-3, -2)), ws))
    back = ops.window_reverse_roll(xw, ws, (H, W), shift)
    assert torch.equal(back.cpu(), x)


@pytest.mark.parametrize("T", [1, 2])
@pytest.mark.parametrize("H,W,ws,shift", [(180, 360, (9, 18), (4, 9)), (18, 36, (9, 18), (0, 0)),
                                          (12, 8, (4, 4), (2, 2)), (90, 180, (9, 18), (4, 9))])
def test_mask_bitexact(device, T, H, W, ws, shift):
    from nsw import ops
    m = ops.make_attention_mask(H, W, ws, shift, T, device).cpu().numpy()
    want = im.mask_closed_form(H, W, ws[0], ws[1], shift[0], shift[1], T)
    assert np.array_equal(m, want)
    if H * W <= 400:
        assert np.array_equal(m, ref.make_attention_mask(H, W, ws, shift, T).numpy())


def test_block_attn_mask_property(device):
    import nsw
    blk = nsw.Block(64, 2, (18, 36), (9, 18), 1, shift_size=(4, 9)).to(device)
    assert torch.equal(blk.attn_mask.cpu(), ref.make_attention_mask(18, 36, (9, 18), (4, 9), 1))
