"""torch.ops.nsw.*: the custom operators the modules call (no GPU needed).

* every op is registered and its shape function gives the output shapes and
  dtypes of the C-ABI entry point it wraps (meta tensors);
* nsw.Block, a small nsw.SwinTransformer and WeightedRMSE trace under
  torch.compile(fullgraph=True) into one graph each (no graph breaks), with
  the libnsw ops as single nodes; the capturing backend never runs the graph,
  so no kernel is launched.
"""
import pytest
import torch

import nsw
from nsw import torch_ops

OPS = ["swin_block", "swin_blocks", "swin_blocks_windowed", "linear_to_window", "linear", "rms_norm", "layer_norm", "qkv_projection", "window_attention",
       "window_partition", "window_reverse", "roll_hw", "roll_window_partition", "window_reverse_roll",
       "patch_im2col", "unpatchify", "head_unpatchify", "weighted_metrics"]


def meta(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, device="meta", dtype=dtype)


def test_ops_registered():
    for name in OPS:
        assert hasattr(torch.ops.nsw, name), name


def test_shape_functions():
    n = torch.ops.nsw
    P = [None] * len(torch_ops.BLOCK_PARAMS)
    x = meta(2, 1, 18, 36, 128)
    assert n.swin_block(x, P, 2, [9, 18], [4, 9], 1e-7, False).shape == x.shape
    assert n.swin_blocks(x, P * 3, 2, [9, 18], [0, 0, 4, 9, 0, 0], 1e-7, False).shape == x.shape
    assert n.swin_blocks_windowed(x, meta(648 * 2, 1, dtype=torch.float32), P * 2, 2, [9, 18], [0, 0, 4, 9],
                                  1e-7, False).shape == x.shape
    yw, ss = n.linear_to_window(meta(648, 1152), meta(1024, 1152), meta(1024), meta(648, 1024), [1, 1, 18, 36],
                                [9, 18], [0, 0])
    assert yw.shape == (648, 1024) and ss.shape == (648, 4) and ss.dtype == torch.float32
    y = n.linear(meta(7, 5, 64), meta(96, 64), meta(96), None, 1)
    assert y.shape == (7, 5, 96) and y.dtype == torch.bfloat16
    assert n.rms_norm(meta(3, 64), meta(64), 1e-7).shape == (3, 64)
    assert n.layer_norm(meta(3, 64), None, None, 1e-5).shape == (3, 64)
    assert n.qkv_projection(meta(4, 162, 128), meta(384, 128), meta(384), meta(64), meta(64), 2, 1e-7).shape \
        == (4, 162, 384)
    assert n.window_attention(meta(4, 162, 384), 2, 0.125, None, [18, 36, 9, 18, 4, 9, 1]).shape == (4, 162, 128)
    assert n.window_partition(x, [9, 18]).shape == (8, 1, 9, 18, 128)
    assert n.roll_window_partition(x, [9, 18], [4, 9]).shape == (8, 1, 9, 18, 128)
    assert n.window_reverse(meta(8, 1, 9, 18, 128), [9, 18], [18, 36]).shape == x.shape
    assert n.window_reverse_roll(meta(8, 1, 9, 18, 128), [9, 18], [18, 36], [4, 9]).shape == x.shape
    assert n.roll_hw(x, [4, 9]).shape == x.shape
    pm = n.patch_im2col(meta(2, 3, 70, 72, 144, dtype=torch.float32), 4, 1152, torch.bfloat16, None, 0)
    assert pm.shape == (2 * 3 * 18 * 36, 1152) and pm.dtype == torch.bfloat16
    out = n.unpatchify(meta(2 * 18 * 36, 1120), 2, 70, 72, 144, 4, torch.float32)
    assert out.shape == (2, 1, 70, 72, 144) and out.dtype == torch.float32
    out = n.head_unpatchify(meta(2 * 18 * 36, 1024), meta(1120, 1024), 2, 70, 72, 144, 4, torch.float32)
    assert out.shape == (2, 1, 70, 72, 144) and out.dtype == torch.float32
    f = meta(2, 3, 70, 8, 16, dtype=torch.float32)
    r, a = n.weighted_metrics(f, f, meta(8, dtype=torch.float64), None)
    assert r.shape == (2, 3, 70) and r.dtype == torch.float64 and a.numel() == 0
    r, a = n.weighted_metrics(f, f, meta(8, dtype=torch.float64), meta(70, dtype=torch.float32))
    assert a.shape == (2, 3, 70)


class Capture:
    """torch.compile backend that records the traced graphs and never runs them."""

    def __init__(self):
        self.graphs = []

    def __call__(self, gm, example_inputs):
        self.graphs.append(gm)
        outs = [n for n in gm.graph.nodes if n.op == "output"][0].args[0]
        vals = [o.meta.get("example_value") if hasattr(o, "meta") else None for o in outs]

        def run(*args):   # empty tensors of the traced output shapes: nothing is launched
            return [None if v is None else torch.empty(v.shape, dtype=v.dtype) for v in vals]
        return run


def targets(gm):
    return [str(nd.target) for nd in gm.graph.nodes if nd.op == "call_function"]


def count(ts, op):
    return sum(t in (f"nsw.{op}", f"nsw.{op}.default") for t in ts)


@pytest.fixture(autouse=True)
def fresh_dynamo():
    torch._dynamo.reset()
    yield
    torch._dynamo.reset()


def test_block_traces_into_one_graph():
    blk = nsw.Block(128, 2, (18, 36), (9, 18), 1, shift_size=(4, 9)).eval()
    cap = Capture()
    torch.compile(blk, backend=cap, fullgraph=True)(torch.randn(1, 1, 18, 36, 128))
    assert len(cap.graphs) == 1
    t = targets(cap.graphs[0])
    assert count(t, "swin_block") == 1


def test_model_traces_into_one_graph():
    H, W, C = 72, 144, 5
    meta_d = {"coords": torch.randn(H, W, 3), "sp_shapes": [[H], [W]], "n_channels": C}
    model = nsw.SwinTransformer(window_size=(9, 18), patch_size=4, in_chans=C, out_chans=C, embed_dim=128,
                                depth=4, num_heads=2, domain_metadata=meta_d).eval()
    cap = Capture()
    torch.compile(model, backend=cap, fullgraph=True)(torch.randn(1, 1, C, H, W))
    assert len(cap.graphs) == 1
    t = targets(cap.graphs[0])
    assert count(t, "swin_blocks_windowed") == 1  # the blocks as one window-order chain
    assert count(t, "linear_to_window") == 1      # fed by the embedding in block 0's window order
    assert count(t, "patch_im2col") == 2         # the image and the coordinate embedding
    assert count(t, "head_unpatchify") == 1       # the head GEMM with the head layout fused
    model.chain_blocks = False
    cap = Capture()
    torch._dynamo.reset()
    torch.compile(model, backend=cap, fullgraph=True)(torch.randn(1, 1, C, H, W))
    assert count(targets(cap.graphs[0]), "swin_block") == 4


def test_head_weight_perm_matches_the_head_layout():
    """Row c*p*p + u*p + v of the permuted weight is the reference's head row
    (u*p + v)*C_out + c (models/swin.py:201-209,293-299)."""
    from nsw import ops
    Co, p, E = 5, 3, 4
    Wt = torch.randn(p * p * Co, E)
    Wp = ops.head_weight_perm(Wt, Co, p)
    for c in range(Co):
        for u in range(p):
            for v in range(p):
                assert torch.equal(Wp[c * p * p + u * p + v], Wt[(u * p + v) * Co + c])


def test_metric_traces_into_one_graph():
    lat = torch.linspace(-80, 80, 8)
    m = nsw.WeightedRMSE(nsw.build_spherical_area_weights(lat)[:, None])
    cap = Capture()
    torch.compile(m, backend=cap, fullgraph=True)(torch.randn(2, 1, 3, 8, 16), torch.randn(2, 1, 3, 8, 16))
    assert len(cap.graphs) == 1
    assert count(targets(cap.graphs[0]), "weighted_metrics") == 1


def test_model_with_big_skip_traces_into_one_graph():
    """use_big_skip_conv: the skip is one in-place op on the head's output."""
    H, W, C = 72, 144, 5
    meta_d = {"coords": torch.randn(H, W, 3), "sp_shapes": [[H], [W]], "n_channels": C}
    model = nsw.SwinTransformer(window_size=(9, 18), patch_size=4, in_chans=C, out_chans=C, embed_dim=128,
                                depth=2, num_heads=2, use_big_skip_conv=True, domain_metadata=meta_d).eval()
    cap = Capture()
    torch._dynamo.reset()
    torch.compile(model, backend=cap, fullgraph=True)(torch.randn(1, 1, C, H, W))
    assert len(cap.graphs) == 1
    t = targets(cap.graphs[0])
    assert count(t, "skip_conv_accumulate") == 1
    assert count(t, "head_unpatchify") == 1
