"""GPU parity of the drop-in surface around the block: NormLayer's LayerNorm
branch (models/layer_helpers.py:94-100,118-119), Conv2DLayer.forward
(:171-172), boolean attention masks with F.scaled_dot_product_attention's
meaning (models/swin_helpers.py:247), and the TE block's arithmetic (tanh
GELU, eps 1e-5; models/swin_helpers_te.py:302,318-323) for checkpoints in
the TE layout.  Library routines (F.layer_norm, F.conv2d, F.gelu) and the
oracle are the references; fp32 within 1e-5 relative L2, bf16 within 1e-2."""
import pytest
import torch
import torch.nn.functional as F

from oracle import model_ref as mr, swin_ref as ref, synth

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm()).item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,C,affine", [(5000, 1024, True), (37, 192, True), (300, 64, False), (3, 4096, True)])
def test_layer_norm(device, dtype, rows, C, affine):
    from nsw.layer_helpers import NormLayer
    g = torch.Generator().manual_seed(rows + C)
    x = (torch.randn(rows, C, generator=g) * 2 + 0.5).to(dtype)
    n = NormLayer(C, elementwise_affine=affine, norm_type="layer_norm")
    if affine:
        with torch.no_grad():
            n.norm.weight.copy_(1 + 0.2 * torch.randn(C, generator=g))
            n.norm.bias.copy_(0.1 * torch.randn(C, generator=g))
    n = n.to(device=device, dtype=dtype)
    got = n(x.to(device))
    w = n.norm.weight.float().cpu() if affine else None
    b = n.norm.bias.float().cpu() if affine else None
    want = F.layer_norm(x.float(), (C,), w, b, n.norm.eps)
    assert got.dtype == dtype
    assert rel_l2(got, want) < (1e-6 if dtype == torch.float32 else 5e-3)


@pytest.mark.parametrize("N,C,E,H,W,p", [(2, 5, 64, 16, 32, 4), (1, 70, 128, 36, 72, 2), (3, 4, 32, 18, 21, 3)])
def test_conv2d_layer_is_conv2d(device, N, C, E, H, W, p):
    """Conv2DLayer(kernel = stride = p) runs the patch GEMM; an extent that
    is not a multiple of p drops the remainder as Conv2d does."""
    from nsw.swin import Conv2DLayer
    layer = Conv2DLayer(C, E, kernel_size=p, stride=p)
    with torch.no_grad():
        layer.conv.bias.normal_()
    x = torch.randn(N, C, H, W, generator=torch.Generator().manual_seed(C))
    want = F.conv2d(x, layer.conv.weight, layer.conv.bias, stride=p)
    got = layer.to(device)(x.to(device))
    assert got.shape == want.shape and got.is_contiguous()
    assert rel_l2(got, want) < 1e-6


def test_conv2d_layer_rejects_overlapping_kernels():
    from nsw.swin import Conv2DLayer
    with pytest.raises(NotImplementedError):
        Conv2DLayer(3, 8, kernel_size=3, stride=1).patch


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_window_attention_bool_mask(device, dtype):
    """A boolean mask marks the keys that take part (True), as in SDPA."""
    from nsw import ops
    Bw, L, C, heads = 12, 162, 128, 2
    g = torch.Generator().manual_seed(21)
    qkv = torch.randn(Bw, L, 3 * C, generator=g).to(dtype)
    keep = torch.rand(6, L, L, generator=g) > 0.3
    keep[:, torch.arange(L), torch.arange(L)] = True                 # no fully masked row
    scale = 0.125
    got = ops.window_attention(qkv.to(device), heads, scale, mask=keep.to(device))
    hd = C // heads
    q, k, v = [t.reshape(Bw, L, heads, hd).permute(0, 2, 1, 3) for t in qkv.float().split(C, -1)]
    m = keep[None].expand(Bw // 6, 6, L, L).reshape(Bw, 1, L, L)
    want = F.scaled_dot_product_attention(q, k, v, attn_mask=m, scale=scale).transpose(1, 2).reshape(Bw, L, C)
    assert rel_l2(got, want) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", [(64800, 4096, 1024), (1000, 576, 192), (257, 4096, 256)])
def test_linear_gelu_tanh(device, dtype, M, N, K):
    from nsw import _lib, ops
    g = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = synth.trunc_normal((N, K), 0.02, g).to(dtype)
    b = (0.1 * torch.randn(N, generator=g)).to(dtype)
    got = ops.linear(x.to(device), w.to(device), b.to(device), epilogue=_lib.NSW_EPI_BIAS_GELU_TANH)
    lin = F.linear(x.to(device).float(), w.to(device).float()).cpu()
    want = F.gelu(lin + b.float(), approximate="tanh")
    assert rel_l2(got, want) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_te_semantics(device, dtype):
    """A block switched to the TE arithmetic (eps 1e-5, tanh GELU) matches the
    oracle evaluated with the same choices, through the fused block call."""
    import nsw
    from nsw import checkpoint
    B, T, H, W, C, heads, ws, shift = 1, 1, 90, 180, 192, 6, (9, 18), (4, 9)
    p = synth.block_params(C, heads, seed=41, random_bias=True, random_norm=True)
    p = {k: v.to(dtype).float() for k, v in p.items()}
    x = synth.activations((B, T, H, W, C), seed=42).to(dtype).float()
    blk = nsw.Block(C, heads, (H, W), ws, T, shift_size=shift)
    blk.load_state_dict(p)
    assert checkpoint.apply_te_semantics(blk) == 1
    blk = blk.to(device=device, dtype=dtype)
    with torch.inference_mode():
        y = blk(x.to(device=device, dtype=dtype))
    want = ref.block_forward(x, p, heads, ws, shift, eps=1e-5, gelu="tanh")
    assert rel_l2(y, want) < TOL[dtype]
    if dtype == torch.float32:
        # the erf / finfo-eps oracle is measurably different (the switch
        # matters; in bf16 the difference is below the bf16 rounding error)
        other = ref.block_forward(x, p, heads, ws, shift, eps=torch.finfo(dtype).eps)
        assert rel_l2(want, other) > 10 * rel_l2(y, want)


def test_model_from_te_checkpoint_runs_te_arithmetic(device, tmp_path):
    """A whole model saved in the TE layout and read back with
    load_model_checkpoint computes the TE block's arithmetic (fp32)."""
    import nsw
    from nsw import checkpoint
    B, T, C, H, W, p, E, heads, ws, depth = 1, 1, 6, 36, 72, 2, 64, 4, (9, 18), 2
    lat = torch.linspace(90, -90, H + 1)[:-1]
    lon = torch.linspace(0, 360, W + 1)[:-1]
    sp = mr.spatial_coords(lat, lon)
    meta = {"coords": sp, "sp_shapes": [[H], [W]], "n_channels": C}
    model = nsw.SwinTransformer(temporal_context_window_size=T, window_size=ws, patch_size=p, in_chans=C,
                                out_chans=C, embed_dim=E, depth=depth, num_heads=heads, domain_metadata=meta)
    prm = synth.model_params(C, C, E, depth, heads, p, seed=31, random_bias=True, random_norm=True)
    torch.save({"model_state": {"module.model." + k: v for k, v in checkpoint.vanilla_to_te(prm).items()}},
               tmp_path / "ckpt_best.tar")
    _, _, te = checkpoint.load_model_checkpoint(model, str(tmp_path / "ckpt_best.tar"))
    assert te
    x = synth.activations((B, T, C, H, W), seed=33)
    got = model.to(device)(x.to(device))
    want = mr.model_forward(x, prm, patch_size=p, window_size=ws, depth=depth, num_heads=heads, out_chans=C,
                            coords=mr.model_coords(sp, T), eps=1e-5, gelu="tanh")
    assert rel_l2(got, want) < 1e-5
