"""SwinTransformer's big skip convolution (use_big_skip_conv=True,
models/swin.py:212-223,305-319): the 1x1 convolution of the input added to
the head's image.  The op against a float64 restatement of its rounding
contract, and whole models (fp32 <= 1e-5, bf16 <= 1e-2 relative L2 per
output, the block tolerances) against the oracle's model forward, which
applies the reference's F.conv2d skip to every frame before taking the last
one."""
import pytest
import torch

from oracle import model_ref as mr, synth

pytestmark = pytest.mark.gpu

BF16_EPS = torch.finfo(torch.bfloat16).eps


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm()).item()


def rnd(v, dt):
    return v.to(dt).double()


@pytest.mark.parametrize("xd,md,od", [(torch.float32, torch.float32, torch.float32),
                                      (torch.float32, torch.bfloat16, torch.bfloat16),
                                      (torch.float32, torch.bfloat16, torch.float32),
                                      (torch.bfloat16, torch.bfloat16, torch.bfloat16)])
@pytest.mark.parametrize("B,T,Cx,Ci,Co,H,W,frame0", [(2, 2, 5, 2, 5, 8, 12, 1), (1, 1, 70, 0, 70, 16, 36, 0),
                                                      (1, 3, 3, 1, 17, 4, 6, 2)])
def test_skip_conv_accumulate(device, xd, md, od, B, T, Cx, Ci, Co, H, W, frame0):
    import nsw
    g = torch.Generator().manual_seed(B * 131 + Cx * 7 + Co)
    x = torch.randn(B, T, Cx, H, W, generator=g).to(xd)
    inv = torch.randn(Ci, H, W, generator=g).to(xd) if Ci else None
    w = (torch.randn(Co, Cx + Ci, 1, 1, generator=g) * 0.1).to(md)
    base = torch.randn(B, 1, Co, H, W, generator=g).to(od)
    out = base.to(device)
    nsw.ops.skip_conv_accumulate(x.to(device), w.to(device), out, invariants=None if inv is None else inv.to(device),
                                 frame0=frame0)
    # restatement: model-dtype input, float64 sum rounded to the model dtype, then out's dtype
    xin = x[:, (T - 1 + frame0) % T].double()
    if inv is not None:
        xin = torch.cat([xin, inv.double().unsqueeze(0).expand(B, -1, -1, -1)], dim=1)
    s = torch.einsum("oc,bchw->bohw", w.reshape(Co, -1).double(), rnd(xin, md))
    want = rnd(base.double() + rnd(s, md).unsqueeze(1), od)
    err = rel_l2(out, want)
    assert err < (1e-6 if od == torch.float32 and md == torch.float32 else 4e-3), err


def make(device, dtype, B, T, C, Ci, H, W, p, E, heads, depth, seed):
    import nsw
    lat = torch.linspace(90, -90, H + 1)[:-1]
    lon = torch.linspace(0, 360, W + 1)[:-1]
    sp = mr.spatial_coords(lat, lon)
    model = nsw.SwinTransformer(temporal_context_window_size=T, window_size=(9, 18), patch_size=p,
                                in_chans=C + Ci, out_chans=C, embed_dim=E, depth=depth, num_heads=heads,
                                use_big_skip_conv=True,
                                domain_metadata={"coords": sp, "sp_shapes": [[H], [W]], "n_channels": C})
    prm = synth.model_params(C + Ci, C, E, depth, heads, p, seed=seed, random_bias=True, random_norm=True,
                             big_skip=True)
    prm["skip_conv.conv.weight"] = prm["skip_conv.conv.weight"] * 10   # a skip well above rounding noise
    missing, unexpected = model.load_state_dict(prm, strict=False)
    assert not unexpected and not [k for k in missing if not k.endswith("attn_mask")], (missing, unexpected)
    return model.to(device=device, dtype=dtype), prm, mr.model_coords(sp, T)


@pytest.mark.parametrize("B,T,Ci,frame0", [(1, 1, 0, 0), (2, 2, 1, 1)])
def test_model_big_skip_fp32(device, B, T, Ci, frame0):
    C, H, W, p, E, heads, depth = 6, 36, 72, 2, 64, 4, 2
    model, prm, coords = make(device, torch.float32, B, T, C, Ci, H, W, p, E, heads, depth, seed=41)
    x = synth.activations((B, T, C, H, W), seed=43)
    inv = synth.activations((Ci, H, W), seed=44) if Ci else None
    got = model(x.to(device), invariants=None if inv is None else inv.to(device), frame0=frame0)
    # oracle input: frames in model order, invariants appended to every frame
    xo = x[:, [(t + frame0) % T for t in range(T)]]
    if inv is not None:
        xo = torch.cat([xo, inv.unsqueeze(0).unsqueeze(0).expand(B, T, -1, -1, -1)], dim=2)
    want = mr.model_forward(xo, prm, patch_size=p, window_size=(9, 18), depth=depth, num_heads=heads,
                            out_chans=C, coords=coords)
    assert got.shape == (B, 1, C, H, W)
    assert rel_l2(got, want) < 1e-5
    # the skip matters: without it the output is far off
    noskip = {k: v for k, v in prm.items() if not k.startswith("skip_conv")}
    base = mr.model_forward(xo, noskip, patch_size=p, window_size=(9, 18), depth=depth, num_heads=heads,
                            out_chans=C, coords=coords)
    assert rel_l2(got, base) > 0.1


def test_model_big_skip_bf16(device):
    B, T, C, Ci, H, W, p, E, heads, depth = 1, 2, 6, 0, 36, 72, 2, 128, 4, 2
    model, prm, coords = make(device, torch.bfloat16, B, T, C, Ci, H, W, p, E, heads, depth, seed=47)
    x = synth.activations((B, T, C, H, W), seed=48)
    rp = {k: v.bfloat16().float() for k, v in prm.items()}
    want = mr.model_forward(x.bfloat16().float(), rp, patch_size=p, window_size=(9, 18), depth=depth,
                            num_heads=heads, out_chans=C, coords=coords.bfloat16().float(), eps=BF16_EPS)
    got = model(x.to(device))
    assert got.dtype == torch.bfloat16
    assert rel_l2(got, want) < 1e-2 * (depth + 2)
    # into an fp32 ring slot (the rollout's form): same values up to the bf16 output rounding
    out = torch.zeros(B, 1, C, H, W, device=device)
    model(x.to(device), out=out)
    assert rel_l2(out, got.float()) < 4e-3
