"""Pins of the model-level oracle (oracle/model_ref.py) on the CPU: two
independent formulations of the patch convolution and of the head's
unpatchify, closed-form coordinates, a zero-block model in closed form, and
hand-unrolled rollout loops."""
import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import metrics_ref, model_ref as mr, synth


def test_patch_conv_is_im2col_product():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 5, 8, 12, generator=g)
    w = torch.randn(7, 5, 4, 4, generator=g)
    b = torch.randn(7, generator=g)
    y = mr.patch_conv(x, w, b, 4)                                   # [3, 7, 2, 3]
    cols = mr.im2col_bruteforce(x, 4)                               # [(n, i, j), (c, u, v)]
    want = cols @ w.reshape(7, -1).T + b                            # [(n, i, j), 7]
    got = y.permute(0, 2, 3, 1).reshape(-1, 7)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_patch_conv_unfold_form():
    """The device form of the patch convolution (unfold x weight) against
    F.conv2d and against the brute-force im2col product."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 6, 12, 20, generator=g)
    w = torch.randn(9, 6, 4, 4, generator=g)
    b = torch.randn(9, generator=g)
    got = mr.patch_conv_unfold(x, w, b, 4)
    torch.testing.assert_close(got, F.conv2d(x, w, b, stride=4), rtol=1e-5, atol=1e-5)
    cols = mr.im2col_bruteforce(x, 4)
    want = (cols @ w.reshape(9, -1).T + b).view(2, 3, 5, 9).permute(0, 3, 1, 2)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


def test_head_unpatchify_matches_elementwise_loop():
    g = torch.Generator().manual_seed(1)
    b, t, h, w, E, p, c = 2, 2, 3, 4, 8, 2, 3
    x = torch.randn(b, t, h, w, E, generator=g)
    hw = torch.randn(c * p * p, E, generator=g)
    got = mr.forward_head(x, hw, p, c)
    lin = F.linear(x.reshape(-1, E), hw)
    want = mr.unpatchify_bruteforce(lin, b, t, h, w, p, c)
    torch.testing.assert_close(got, want, rtol=0, atol=0)


def test_spatial_coords_closed_form():
    lat = torch.tensor([90.0, 0.0, -90.0, 45.0])
    lon = torch.tensor([0.0, 90.0, 180.0])
    xyz = mr.spatial_coords(lat, lon)
    assert xyz.shape == (4, 3, 3)
    torch.testing.assert_close(xyz[1, 0], torch.tensor([1.0, 0.0, 0.0]), atol=1e-7, rtol=0)
    torch.testing.assert_close(xyz[1, 1], torch.tensor([0.0, 1.0, 0.0]), atol=1e-7, rtol=0)
    torch.testing.assert_close(xyz[1, 2], torch.tensor([-1.0, 0.0, 0.0]), atol=1e-7, rtol=0)
    for j in range(3):
        torch.testing.assert_close(xyz[0, j], torch.tensor([0.0, 0.0, 1.0]), atol=1e-7, rtol=0)
        torch.testing.assert_close(xyz[2, j], torch.tensor([0.0, 0.0, -1.0]), atol=1e-7, rtol=0)
    s = math.sqrt(0.5)
    torch.testing.assert_close(xyz[3, 0], torch.tensor([s, 0.0, s]), atol=1e-7, rtol=0)
    torch.testing.assert_close(xyz.norm(dim=-1), torch.ones(4, 3), atol=1e-6, rtol=0)


def test_model_coords_time_channel():
    sp = torch.rand(5, 6, 3)
    c = mr.model_coords(sp, 3)
    assert c.shape == (3, 5, 6, 4)
    torch.testing.assert_close(c[..., 3], torch.tensor([0.0, 0.5, 1.0]).view(3, 1, 1).expand(3, 5, 6))
    for t in range(3):
        torch.testing.assert_close(c[t, ..., :3], sp)
    assert torch.all(mr.model_coords(sp, 1)[..., 3] == 0)


def test_zero_block_model_closed_form():
    """depth 0: out = unpatchify(im2col(x) W_e^T + b_e + pos) W_h^T at the
    last frame, built from the brute-force formulations."""
    B, T, C, H, W, p, E, c_out = 2, 2, 3, 8, 12, 4, 16, 2
    prm = synth.model_params(C, c_out, E, 0, 2, p, seed=4, random_bias=True)
    x = synth.activations((B, T, C, H, W), seed=5)
    coords = mr.model_coords(torch.rand(H, W, 3, generator=torch.Generator().manual_seed(6)), T)
    got = mr.model_forward(x, prm, patch_size=p, window_size=(1, 1), depth=0, num_heads=2,
                           out_chans=c_out, coords=coords)
    we = prm["patch_embed.proj.conv.weight"].reshape(E, -1)
    wp = prm["pos_embed.proj.conv.weight"].reshape(E, -1)
    tok = mr.im2col_bruteforce(x.reshape(B * T, C, H, W), p) @ we.T + prm["patch_embed.proj.conv.bias"]
    pos = mr.im2col_bruteforce(coords.permute(0, 3, 1, 2), p) @ wp.T + prm["pos_embed.proj.conv.bias"]
    h, w = H // p, W // p
    tok = tok.view(B, T * h * w, E) + pos.view(1, T * h * w, E)
    lin = tok.reshape(-1, E) @ prm["head.weight"].T
    full = mr.unpatchify_bruteforce(lin, B, T, h, w, p, c_out)
    torch.testing.assert_close(got, full[:, -1:], rtol=1e-5, atol=1e-6)


def test_learned_pos_embed_path():
    B, T, C, H, W, p, E = 1, 2, 2, 8, 8, 2, 8
    prm = synth.model_params(C, C, E, 0, 2, p, seed=7, coord_pos_embed=False, pos_shape=(1, T, H // p, W // p, E))
    x = synth.activations((B, T, C, H, W), seed=8)
    tok = mr.prepare_tokens(x, prm["patch_embed.proj.conv.weight"], prm["patch_embed.proj.conv.bias"], p,
                            prm["pos_embed"])
    base = mr.prepare_tokens(x, prm["patch_embed.proj.conv.weight"], prm["patch_embed.proj.conv.bias"], p,
                             torch.zeros(1))
    torch.testing.assert_close(tok - base, prm["pos_embed"].expand_as(tok), rtol=0, atol=1e-6)


def test_head_is_per_token():
    """The build applies the head to the last frame only; the reference
    applies it to every frame and slices (models/swin.py:318-323)."""
    x = torch.randn(2, 3, 2, 3, 8)
    hw = torch.randn(12, 8)
    torch.testing.assert_close(mr.forward_head(x, hw, 2, 3)[:, -1:], mr.forward_head(x[:, -1:], hw, 2, 3))


def test_stepper_two_steps_by_hand():
    lin = torch.randn(4, 5)

    def model(inp):                      # [B, T, 5, H, W] -> [B, 1, 4, H, W]
        return torch.einsum("oc,btchw->bthw o".replace(" ", ""), lin, inp[:, -1:]).permute(0, 1, 4, 2, 3)

    inp = torch.randn(2, 1, 5, 3, 3)
    got = mr.stepper_forward(model, inp, 2, 1)
    p1 = model(inp)
    p2 = model(torch.cat([p1, inp[:, :, 4:]], dim=2))
    torch.testing.assert_close(got, torch.cat([p1, p2], dim=1))


def test_rollout_matches_unrolled_loop():
    H, W, C = 6, 8, 2
    g = torch.Generator().manual_seed(9)

    def model(inp):                      # deterministic toy: mean over the window, one invariant channel dropped
        return (0.5 * inp[:, :, :C].mean(dim=1, keepdim=True) + 0.1 * inp[:, -1:, C:].sum(2, keepdim=True))

    win = torch.randn(1, 2, C, H, W, generator=g)
    inv = torch.randn(1, H, W, generator=g)
    targets = torch.randn(3, C, H, W, generator=g)
    mean, std = torch.tensor([1.0, -2.0]), torch.tensor([2.0, 0.5])
    w = metrics_ref.area_weights(metrics_ref.era5_latitudes(H))
    clim = torch.tensor([0.3, -0.7])
    rmse, acc, gens = mr.rollout(model, win, inv, targets, mean, std, w, clim)
    # by hand
    cur = win.clone()
    for i in range(3):
        inp = torch.cat([cur, inv.view(1, 1, 1, H, W).expand(1, 2, 1, H, W)], dim=2)
        gen = model(inp)
        pred = (gen * std.view(1, 1, C, 1, 1) + mean.view(1, 1, C, 1, 1)).double().numpy()
        targ = (targets[i].view(1, 1, C, H, W) * std.view(1, 1, C, 1, 1) + mean.view(1, 1, C, 1, 1)).double().numpy()
        np.testing.assert_allclose(rmse[i].numpy(), metrics_ref.weighted_rmse(pred, targ, w), rtol=1e-12)
        np.testing.assert_allclose(acc[i].numpy(), metrics_ref.weighted_acc(pred, targ, w, clim.double().numpy()),
                                   rtol=1e-12)
        torch.testing.assert_close(gens[i], gen[0, 0])
        cur = torch.cat([cur[:, 1:], gen], dim=1)


def test_smooth_field_is_standardised_and_smooth():
    f = synth.smooth_field((2, 32, 64), 3.0, 11)
    assert torch.allclose(f.mean(dim=(-2, -1)), torch.zeros(2), atol=1e-5)
    assert torch.allclose(f.std(dim=(-2, -1)), torch.ones(2), atol=1e-4)
    # neighbouring pixels are strongly correlated (white noise would give ~0)
    corr = (f[:, :, 1:] * f[:, :, :-1]).mean()
    assert corr > 0.8


def test_big_skip_is_the_last_frames_channel_mix():
    """models/swin.py:305-319: with a zero head the model returns exactly the
    1x1 skip convolution of the input's last frame (the skip is per frame and
    the model keeps x[:, -1:]); brute-force channel sums."""
    B, T, C_in, C_out, H, W, p, E = 2, 3, 4, 3, 18, 36, 2, 16
    prm = synth.model_params(C_in, C_out, E, 0, 2, p, seed=5, big_skip=True)
    prm["head.weight"] = torch.zeros_like(prm["head.weight"])
    x = synth.activations((B, T, C_in, H, W), seed=6)
    lat = torch.linspace(90, -90, H + 1)[:-1]
    lon = torch.linspace(0, 360, W + 1)[:-1]
    coords = mr.model_coords(mr.spatial_coords(lat, lon), T)
    got = mr.model_forward(x, prm, patch_size=p, window_size=(9, 18), depth=0, num_heads=2, out_chans=C_out,
                           coords=coords)
    w = prm["skip_conv.conv.weight"][:, :, 0, 0].double()
    want = torch.zeros(B, 1, C_out, H, W, dtype=torch.float64)
    for o in range(C_out):
        for c in range(C_in):
            want[:, 0, o] += w[o, c] * x[:, T - 1, c].double()
    assert torch.allclose(got.double(), want, atol=1e-6, rtol=1e-5)
