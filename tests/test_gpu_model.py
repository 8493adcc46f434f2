"""GPU parity of the model-level path (SwinTransformer.forward, its patch
embedding / positional embedding / head, and the rollout with fused
unnormalised metrics) against the CPU oracle (oracle/model_ref.py).

Layout kernels (patch gather, unpatchify) are pure copies / conversions and
must match bit for bit.  Whole-model outputs: fp32 within 1e-5 relative L2,
bf16 within 1e-2 relative L2 (the block tolerances)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import metrics_ref, model_ref as mr, synth

pytestmark = pytest.mark.gpu


# nn.RMSNorm(eps=None) on bf16 tensors (models/layer_helpers.py:101-106)
BF16_EPS = torch.finfo(torch.bfloat16).eps


def bf16_round(v):
    """Round weights / inputs to bf16 (kept as fp32) for the oracle of a bf16 model."""
    if v is None:
        return None
    if isinstance(v, dict):
        return {k: t.bfloat16().float() for k, t in v.items()}
    return v.bfloat16().float()


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).norm() / b.norm()).item()


@pytest.mark.parametrize("xd,od", [(torch.float32, torch.float32), (torch.float32, torch.bfloat16),
                                   (torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("B,T,Cx,Ci,H,W,p,frame0", [(2, 2, 3, 0, 8, 12, 4, 0), (1, 3, 5, 2, 12, 16, 2, 1),
                                                    (1, 1, 70, 0, 32, 64, 4, 0), (2, 2, 4, 1, 6, 9, 3, 1),
                                                    (1, 1, 5, 0, 8, 16, 2, 0),      # a chunk straddles C*p*p
                                                    (1, 1, 3, 1, 4, 1440, 4, 0),    # 6 patch groups, last partial
                                                    (1, 2, 5, 0, 2, 1440, 2, 1)])   # p = 2, 128-patch groups
def test_patch_im2col_bit_exact(device, xd, od, B, T, Cx, Ci, H, W, p, frame0):
    import nsw
    g = torch.Generator().manual_seed(B * 7 + Cx)
    x = torch.randn(B, T, Cx, H, W, generator=g).to(xd)
    inv = torch.randn(Ci, H, W, generator=g).to(xd) if Ci else None
    K = (Cx + Ci) * p * p
    Kp = (K + 63) // 64 * 64
    got = nsw.ops.patch_im2col(x.to(device), p, Kp, od, invariants=None if inv is None else inv.to(device),
                               frame0=frame0).cpu()
    # oracle: frames in model order, invariants appended, brute-force im2col
    order = [(t + frame0) % T for t in range(T)]
    src = x[:, order]
    if inv is not None:
        src = torch.cat([src, inv.view(1, 1, Ci, H, W).expand(B, T, Ci, H, W)], dim=2)
    want = mr.im2col_bruteforce(src.reshape(B * T, Cx + Ci, H, W).float(), p).to(od)
    assert got.shape == (B * T * (H // p) * (W // p), Kp)
    assert torch.equal(got[:, :K], want)
    assert torch.all(got[:, K:] == 0)


@pytest.mark.parametrize("p,od", [(4, torch.bfloat16), (2, torch.bfloat16), (4, torch.float32)])
def test_patch_im2col_full_size(device, p, od):
    """The patch matrix of a [1, 1, 70, 720, 1440] float image (configs 3-5)
    against the view / permute form of the same layout (the brute-force
    oracle's order, checked on small shapes above)."""
    import nsw
    C, H, W = 70, 720, 1440
    x = torch.randn(1, 1, C, H, W, generator=torch.Generator().manual_seed(p))
    K = C * p * p
    Kp = (K + 63) // 64 * 64
    got = nsw.ops.patch_im2col(x.to(device), p, Kp, od).cpu()
    h, w = H // p, W // p
    want = x.view(C, h, p, w, p).permute(1, 3, 0, 2, 4).reshape(h * w, K).to(od)
    assert torch.equal(got[:, :K], want)
    assert torch.all(got[:, K:] == 0)


@pytest.mark.parametrize("idt,odt", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                     (torch.float32, torch.float32)])
@pytest.mark.parametrize("B,Co,H,W,p", [(1, 70, 32, 64, 4), (2, 6, 12, 16, 2), (3, 4, 9, 6, 3),
                                         (1, 8, 8, 20, 4),      # odd patches per row: one patch per lane
                                         (2, 70, 36, 40, 4)])   # two patches per lane, many workgroups
def test_unpatchify_bit_exact(device, idt, odt, B, Co, H, W, p):
    import nsw
    h, w = H // p, W // p
    N = p * p * Co
    y = torch.randn(B * h * w, N, generator=torch.Generator().manual_seed(Co)).to(idt)
    if N % (8 if idt == torch.bfloat16 else 4):
        # rows not a whole number of 16-byte vectors: refused, not computed
        with pytest.raises(ValueError, match="multiple of"):
            nsw.ops.unpatchify(y.to(device), B, Co, H, W, p, dtype=odt)
        return
    got = nsw.ops.unpatchify(y.to(device), B, Co, H, W, p, dtype=odt).cpu()
    want = mr.unpatchify_bruteforce(y, B, 1, h, w, p, Co).to(odt)
    assert torch.equal(got, want)
    # into one slot of a [B, T, C, H, W] ring buffer
    ring = torch.full((B, 3, Co, H, W), 7.0, dtype=odt, device=device)
    nsw.ops.unpatchify(y.to(device), B, Co, H, W, p, out=ring[:, 1:2])
    ring = ring.cpu()
    assert torch.equal(ring[:, 1:2], want)
    assert torch.all(ring[:, 0] == 7) and torch.all(ring[:, 2] == 7)


@pytest.mark.parametrize("dt,odt", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                    (torch.float32, torch.float32)])
@pytest.mark.parametrize("B,Co,H,W,p,E", [(1, 70, 32, 64, 4, 128), (2, 6, 12, 16, 2, 64),
                                           (1, 70, 72, 144, 4, 64),    # 648 tokens, 5 column tiles
                                           (2, 5, 36, 40, 4, 64),      # N = 80 < one tile
                                           (1, 3, 16, 32, 8, 64), (1, 296, 4, 8, 1, 64), (1, 2, 32, 32, 16, 64)])
def test_head_unpatchify_matches_two_launches(device, dt, odt, B, Co, H, W, p, E):
    """nsw_head_unpatchify = nsw_linear (no bias) + nsw_unpatchify bit for bit
    (both paths round the GEMM result to the GEMM dtype first)."""
    import nsw
    h, w = H // p, W // p
    g = torch.Generator().manual_seed(Co * 31 + p)
    x = torch.randn(B * h * w, E, generator=g).to(dt).to(device)
    Wt = (torch.randn(p * p * Co, E, generator=g) * 0.1).to(dt).to(device)
    y = nsw.ops.linear(x, Wt)
    want = nsw.ops.unpatchify(y, B, Co, H, W, p, dtype=odt).cpu()
    got = nsw.ops.head_unpatchify(x, nsw.ops.head_weight_perm(Wt, Co, p), B, Co, H, W, p, dtype=odt).cpu()
    assert torch.equal(got, want)
    # into one slot of a [B, T, C, H, W] ring buffer
    ring = torch.full((B, 3, Co, H, W), 7.0, dtype=odt, device=device)
    nsw.ops.head_unpatchify(x, nsw.ops.head_weight_perm(Wt, Co, p), B, Co, H, W, p, out=ring[:, 1:2])
    ring = ring.cpu()
    assert torch.equal(ring[:, 1:2], want)
    assert torch.all(ring[:, 0] == 7) and torch.all(ring[:, 2] == 7)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_head_unpatchify_exact_against_bruteforce(device, dt):
    """Small-integer operands make every product and sum exact in both dtypes,
    so the fused head must equal the element-by-element head layout of the
    exact product (oracle/model_ref.unpatchify_bruteforce)."""
    import nsw
    B, Co, H, W, p, E = 2, 6, 12, 20, 2, 64
    h, w = H // p, W // p
    g = torch.Generator().manual_seed(3)
    x = torch.randint(-2, 3, (B * h * w, E), generator=g).float()
    Wt = torch.randint(-2, 3, (p * p * Co, E), generator=g).float()
    want = mr.unpatchify_bruteforce(x @ Wt.T, B, 1, h, w, p, Co)
    got = nsw.ops.head_unpatchify(x.to(dt).to(device), nsw.ops.head_weight_perm(Wt.to(dt).to(device), Co, p),
                                  B, Co, H, W, p, dtype=torch.float32).cpu()
    assert torch.equal(got, want)


def test_patch_embed_layer_is_conv2d(device):
    import nsw
    layer = nsw.PatchEmbedLayer(patch_size=4, in_chans=5, embed_dim=64, sp1_shapes=[16], sp2_shapes=[32])
    with torch.no_grad():
        layer.proj.conv.bias.normal_()
    x = torch.randn(3, 5, 16, 32)
    want = F.conv2d(x, layer.proj.conv.weight, layer.proj.conv.bias, stride=4)
    got = layer.to(device)(x.to(device)).cpu()
    assert rel_l2(got, want) < 1e-6


def make_model(device, dtype, *, B, T, C_in, C_out, H, W, p, E, heads, ws, depth, coord, seed=1):
    import nsw
    lat = torch.linspace(90, -90, H + 1)[:-1]
    lon = torch.linspace(0, 360, W + 1)[:-1]
    sp = mr.spatial_coords(lat, lon)
    meta = {"coords": sp, "sp_shapes": [[H], [W]], "n_channels": C_out}
    model = nsw.SwinTransformer(temporal_context_window_size=T, window_size=ws, patch_size=p, in_chans=C_in,
                                out_chans=C_out, embed_dim=E, depth=depth, num_heads=heads, coord_pos_embed=coord,
                                domain_metadata=meta)
    prm = synth.model_params(C_in, C_out, E, depth, heads, p, seed=seed, coord_pos_embed=coord,
                             pos_shape=(1, T, H // p, W // p, E), random_bias=True, random_norm=True)
    missing, unexpected = model.load_state_dict(prm, strict=False)
    assert not unexpected and not [k for k in missing if not k.endswith("attn_mask")], (missing, unexpected)
    coords = mr.model_coords(sp, T) if coord else None
    return model.to(device=device, dtype=dtype), prm, coords


MODEL_CASES = [
    # B, T, C_in, C_out, H, W, p, E, heads, ws, depth, coord
    (2, 2, 6, 6, 36, 72, 2, 64, 4, (9, 18), 2, True),
    (1, 1, 8, 6, 36, 72, 4, 128, 2, (3, 6), 3, False),
    (1, 2, 8, 8, 18, 36, 1, 64, 2, (9, 18), 2, True),
    # the reference's model test (tests/test_all.py:165-171): batch 4, T = 2,
    # 720 x 1440, p4, window 9 x 18, 20 channels, e32 with 8 heads (head dim
    # 4), depth 2, learned and coordinate positional embeddings
    (4, 2, 20, 20, 720, 1440, 4, 32, 8, (9, 18), 2, False),
    (4, 2, 20, 20, 720, 1440, 4, 32, 8, (9, 18), 2, True),
]


@pytest.mark.parametrize("B,T,C_in,C_out,H,W,p,E,heads,ws,depth,coord", MODEL_CASES)
def test_model_fp32(device, B, T, C_in, C_out, H, W, p, E, heads, ws, depth, coord):
    model, prm, coords = make_model(device, torch.float32, B=B, T=T, C_in=C_in, C_out=C_out, H=H, W=W, p=p,
                                    E=E, heads=heads, ws=ws, depth=depth, coord=coord)
    x = synth.activations((B, T, C_in, H, W), seed=17)
    want = mr.model_forward(x, prm, patch_size=p, window_size=ws, depth=depth, num_heads=heads,
                            out_chans=C_out, coords=coords)
    got = model(x.to(device))
    assert got.shape == (B, 1, C_out, H, W) and got.dtype == torch.float32
    assert rel_l2(got, want) < 1e-5
    # forward_head on all frames against the oracle's
    tok = model.prepare_tokens(x.to(device))
    pos = mr.pos_tokens(coords, prm["pos_embed.proj.conv.weight"], prm["pos_embed.proj.conv.bias"], p) \
        if coord else prm["pos_embed"]
    tw = mr.prepare_tokens(x, prm["patch_embed.proj.conv.weight"], prm["patch_embed.proj.conv.bias"], p, pos)
    assert rel_l2(tok, tw) < 1e-6
    assert rel_l2(model.forward_head(tok), mr.forward_head(tw, prm["head.weight"], p, C_out)) < 1e-6


def test_model_from_te_checkpoint_fp32(device, tmp_path):
    """A whole-model checkpoint in the production layout (TE block names, DDP
    and TimeStepper prefixes, a TE _extra_state entry; models/helpers.py:53-70,
    tests/test_te.py:34-71) written to disk, read back with the safe loader
    into a freshly initialised model and run on the GPU matches the oracle
    forward of the parameters that were saved."""
    import nsw
    from nsw import checkpoint
    B, T, C_in, C_out, H, W, p, E, heads, ws, depth, coord = MODEL_CASES[0]
    lat = torch.linspace(90, -90, H + 1)[:-1]
    lon = torch.linspace(0, 360, W + 1)[:-1]
    sp = mr.spatial_coords(lat, lon)
    meta = {"coords": sp, "sp_shapes": [[H], [W]], "n_channels": C_out}
    model = nsw.SwinTransformer(temporal_context_window_size=T, window_size=ws, patch_size=p, in_chans=C_in,
                                out_chans=C_out, embed_dim=E, depth=depth, num_heads=heads, coord_pos_embed=coord,
                                domain_metadata=meta)
    prm = synth.model_params(C_in, C_out, E, depth, heads, p, seed=23, coord_pos_embed=coord,
                             pos_shape=(1, T, H // p, W // p, E), random_bias=True, random_norm=True)
    state = {"module.model." + k: v for k, v in checkpoint.vanilla_to_te(prm).items()}
    state["module.model.blocks.1.rms_norm_mlp._extra_state"] = torch.zeros(4)
    path = tmp_path / "ckpt_best.tar"
    torch.save({"model_state": state, "epoch": 7}, path)
    missing, unexpected = model.load_state_dict(checkpoint.load_checkpoint_model_state(str(path)), strict=False)
    assert not unexpected and not [k for k in missing if not k.endswith("attn_mask")], (missing, unexpected)
    model = model.to(device)
    x = synth.activations((B, T, C_in, H, W), seed=29)
    want = mr.model_forward(x, prm, patch_size=p, window_size=ws, depth=depth, num_heads=heads,
                            out_chans=C_out, coords=mr.model_coords(sp, T) if coord else None)
    got = model(x.to(device))
    assert got.shape == (B, 1, C_out, H, W)
    assert rel_l2(got, want) < 1e-5


BF16_CASES = [
    # bf16 MFMA attention head dims (32, 64)
    (2, 2, 6, 6, 36, 72, 2, 128, 4, (9, 18), 2, True),
    (1, 1, 8, 6, 36, 72, 4, 128, 2, (3, 6), 3, False),
    # the reference's model test model (tests/test_all.py:168-169) in bf16:
    # e32 (a GEMM k of one 32-element MFMA step), head dim 4
    (1, 2, 20, 20, 720, 1440, 4, 32, 8, (9, 18), 2, False),
]


@pytest.mark.parametrize("B,T,C_in,C_out,H,W,p,E,heads,ws,depth,coord", BF16_CASES)
def test_model_bf16(device, B, T, C_in, C_out, H, W, p, E, heads, ws, depth, coord):
    """The bf16 bound is 1e-2 relative L2 per block: every block is checked
    against the oracle block applied to the GPU's own block input, the
    embedding against the oracle embedding; the end-to-end output (drift over
    embed + depth blocks + head) is bounded by 1e-2 per stage and printed."""
    model, prm, coords = make_model(device, torch.bfloat16, B=B, T=T, C_in=C_in, C_out=C_out, H=H, W=W, p=p,
                                    E=E, heads=heads, ws=ws, depth=depth, coord=coord)
    x = synth.activations((B, T, C_in, H, W), seed=18)
    prm_r, x_r, coords_r = bf16_round(prm), bf16_round(x), bf16_round(coords)
    want = mr.model_forward(x_r, prm_r, patch_size=p, window_size=ws, depth=depth, num_heads=heads,
                            out_chans=C_out, coords=coords_r, eps=BF16_EPS)
    got = model(x.to(device))            # fp32 input, bf16 model: converted in the patch gather
    assert got.dtype == torch.bfloat16
    e2e = rel_l2(got, want)
    print(f"bf16 end-to-end relative L2 after {depth} blocks: {e2e:.3e}")
    assert e2e < 1e-2 * (depth + 2)
    # stage by stage
    tok = model.prepare_tokens(x.to(device))
    pos = mr.pos_tokens(coords_r, prm_r["pos_embed.proj.conv.weight"], prm_r["pos_embed.proj.conv.bias"], p) \
        if coord else prm_r["pos_embed"]
    tw = mr.prepare_tokens(x_r, prm_r["patch_embed.proj.conv.weight"], prm_r["patch_embed.proj.conv.bias"], p, pos)
    assert rel_l2(tok, tw) < 1e-2
    for i, blk in enumerate(model.blocks):
        bp = {k[len(f"blocks.{i}."):]: v for k, v in prm_r.items() if k.startswith(f"blocks.{i}.")}
        ref = mr.swin_ref.block_forward(tok.float().cpu(), bp, heads, ws, mr.block_shift(i, ws), eps=BF16_EPS)
        tok = blk(tok)
        err = rel_l2(tok, ref)
        print(f"block {i}: relative L2 {err:.3e}")
        assert err < 1e-2, f"block {i}"


def test_model_config3_channels_bf16(device):
    """70 channels, p = 4, hd 64 on a 180x360 grid (the config-3 layer shapes
    at a quarter of the extent), two blocks."""
    B, T, C, H, W, p, E, heads, ws, depth = 1, 1, 70, 180, 360, 4, 256, 4, (9, 18), 2
    model, prm, coords = make_model(device, torch.bfloat16, B=B, T=T, C_in=C, C_out=C, H=H, W=W, p=p, E=E,
                                    heads=heads, ws=ws, depth=depth, coord=True, seed=3)
    x = synth.smooth_field((B, T, C, H, W), 4.0, 19)
    want = mr.model_forward(bf16_round(x), bf16_round(prm), patch_size=p, window_size=ws, depth=depth,
                            num_heads=heads, out_chans=C, coords=bf16_round(coords), eps=BF16_EPS)
    got = model(x.to(device))
    assert rel_l2(got, want) < 1e-2


@pytest.mark.parametrize("sd", [torch.float32, torch.float64])
@pytest.mark.parametrize("pd", [torch.float32, torch.bfloat16])
def test_metrics_unnorm_vs_oracle(device, pd, sd):
    import nsw
    B, T, C, H, W = 1, 1, 5, 90, 180
    g = torch.Generator().manual_seed(23)
    gen = torch.randn(B, T, C, H, W, generator=g).to(pd)
    tgt = torch.randn(B, T, C, H, W, generator=g)
    std = (torch.rand(C, generator=g, dtype=torch.float64) + 0.5).to(sd)
    mean = (torch.randn(C, generator=g, dtype=torch.float64) * 10).to(sd)
    clim = torch.randn(C, generator=g) * 10
    w = torch.from_numpy(metrics_ref.area_weights(metrics_ref.era5_latitudes(H)))
    r, a = nsw.ops.weighted_metrics_unnorm(gen.to(device), tgt.to(device), std, mean, w[:, None], clim)
    # reference: separate product and sum with torch's type promotion (fp32
    # fields with fp32 stats stay fp32, float64 stats promote them), then the
    # metrics in float64
    pred = (gen.float() * std.view(1, 1, C, 1, 1)) + mean.view(1, 1, C, 1, 1)
    targ = (tgt * std.view(1, 1, C, 1, 1)) + mean.view(1, 1, C, 1, 1)
    assert pred.dtype == sd
    fd = np.float64 if sd == torch.float64 else np.float32
    wr = metrics_ref.weighted_rmse(pred.double().numpy(), targ.double().numpy(), w.numpy(), True, field_dtype=fd)
    wa = metrics_ref.weighted_acc(pred.double().numpy(), targ.double().numpy(), w.numpy(), clim.double().numpy(),
                                  True, field_dtype=fd)
    np.testing.assert_allclose(r.cpu().numpy()[0, 0], wr, rtol=1e-10)
    np.testing.assert_allclose(a.cpu().numpy()[0, 0], wa, rtol=1e-9, atol=1e-12)


def test_rollout_vs_oracle(device):
    import nsw
    T, C, Ci, H, W, p, E, heads, ws, depth, S = 2, 4, 2, 36, 72, 2, 64, 4, (9, 18), 2, 3
    model, prm, coords = make_model(device, torch.float32, B=1, T=T, C_in=C + Ci, C_out=C, H=H, W=W, p=p, E=E,
                                    heads=heads, ws=ws, depth=depth, coord=True, seed=5)
    win = synth.smooth_field((1, T, C, H, W), 2.0, 29)
    inv = synth.smooth_field((Ci, H, W), 3.0, 31)
    targets = synth.smooth_field((S, C, H, W), 2.0, 37)
    g = torch.Generator().manual_seed(41)
    mean, std = torch.randn(C, generator=g) * 5, torch.rand(C, generator=g) + 0.5
    clim = torch.randn(C, generator=g)
    w = metrics_ref.area_weights(metrics_ref.era5_latitudes(H))

    def oracle_model(inp):
        return mr.model_forward(inp, prm, patch_size=p, window_size=ws, depth=depth, num_heads=heads,
                                out_chans=C, coords=coords)

    r0, a0, f0 = mr.rollout(oracle_model, win, inv, targets, mean, std, w, clim)
    ro = nsw.Rollout(model, mean, std, torch.from_numpy(w)[:, None], invariants=inv.to(device), clim=clim)
    r1, a1, f1 = ro.run(win.to(device), targets.to(device), keep_fields=True)
    assert rel_l2(f1, f0) < 1e-5
    np.testing.assert_allclose(r1.cpu().numpy(), r0.numpy(), rtol=1e-4)
    np.testing.assert_allclose(a1.cpu().numpy(), a0.numpy(), rtol=1e-4, atol=1e-6)


def test_time_stepper(device):
    import types
    import nsw
    T, C, Ci, H, W, p, E, heads, ws = 1, 4, 1, 36, 72, 2, 64, 2, (9, 18)
    model, prm, coords = make_model(device, torch.float32, B=1, T=T, C_in=C + Ci, C_out=C, H=H, W=W, p=p, E=E,
                                    heads=heads, ws=ws, depth=1, coord=True, seed=7)
    cfg = types.SimpleNamespace(train=types.SimpleNamespace(num_rollout_steps=2),
                                data=types.SimpleNamespace(invariants=["lsm"]))
    stepper = nsw.TimeStepper(cfg, model)
    x = synth.activations((1, T, C + Ci, H, W), seed=43)
    got = stepper(x.to(device)).cpu()

    def oracle_model(inp):
        return mr.model_forward(inp, prm, patch_size=p, window_size=ws, depth=1, num_heads=heads, out_chans=C,
                                coords=coords)

    want = mr.stepper_forward(oracle_model, x, 2, 1)
    assert got.shape == (1, 2, C, H, W)
    assert rel_l2(got, want) < 1e-5
