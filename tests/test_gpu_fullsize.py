"""Parity at the BASELINE workloads' own sizes: the config-3 and config-4
models (720x1440, 70 channels, depth 16 / 8) in bf16 and the config-5
8-step rollout, against the oracle (oracle/model_ref.py, oracle/swin_ref.py).

At these sizes the oracle runs with fp32 library kernels on the GPU device
(torch matmul / softmax, TF32 off, the patch convolution as unfold x weight);
it is the same code the CPU tests pin.  Bounds:

* config 3 / 4: embedding, every block (on the GPU's own block input) and
  the head within 1e-2 relative L2 (bf16, north_star), every block's branch
  y - x within 2e-2; the forward (the window-order block chain), end to
  end, within 3e-2 of the oracle model (compounded bf16 rounding over depth
  + 2 stages) and no more than 1.25x the error of the per-block path (the
  values are printed).
* config 5: the bf16 rollout against the fp32 oracle rollout of the same
  (bf16-rounded) weights: per-step forecast fields within 3e-2 relative L2,
  per-channel RMSE within 1% relative, ACC within 1e-2 absolute; the drift
  table is printed as one JSON line.
"""
import json

import numpy as np
import pytest
import torch

from oracle import metrics_ref, model_ref as mr, swin_ref, synth

pytestmark = pytest.mark.gpu

BF16_EPS = torch.finfo(torch.bfloat16).eps

# name: (C_in = C_out, H, W, p, E, heads, ws, depth)
CONFIGS = {
    "config3": (70, 720, 1440, 4, 1024, 16, (9, 18), 16),
    "config4": (70, 720, 1440, 2, 512, 8, (9, 18), 8),
}


def rel_l2(a, b):
    a, b = a.double(), b.double().to(a.device)
    return ((a - b).norm() / b.norm()).item()


def era5_grid(H, W):
    lat = torch.linspace(90, -90, H + 1)[:-1]
    lon = torch.linspace(0, 360, W + 1)[:-1]
    return mr.spatial_coords(lat, lon)


def build(device, name, seed):
    """The nsw model in bf16 and its parameters rounded to bf16 (fp32 values,
    on the device) for the oracle."""
    import nsw
    C, H, W, p, E, heads, ws, depth = CONFIGS[name]
    sp = era5_grid(H, W)
    meta = {"coords": sp, "sp_shapes": [[H], [W]], "n_channels": C}
    model = nsw.SwinTransformer(temporal_context_window_size=1, window_size=ws, patch_size=p, in_chans=C,
                                out_chans=C, embed_dim=E, depth=depth, num_heads=heads, coord_pos_embed=True,
                                domain_metadata=meta)
    prm = synth.model_params(C, C, E, depth, heads, p, seed=seed, random_bias=True, random_norm=True)
    missing, unexpected = model.load_state_dict(prm, strict=False)
    assert not unexpected and not [k for k in missing if not k.endswith("attn_mask")], (missing, unexpected)
    model = model.to(device=device, dtype=torch.bfloat16).eval()
    prm_r = {k: v.bfloat16().float().to(device) for k, v in prm.items()}
    del prm
    coords_r = mr.model_coords(sp, 1).bfloat16().float().to(device)
    return model, prm_r, coords_r


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_model_fullsize_bf16(device, name):
    C, H, W, p, E, heads, ws, depth = CONFIGS[name]
    print(f"{name}: p{p} e{E} d{depth} {C}x{H}x{W} bf16", flush=True)
    model, prm, coords = build(device, name, seed=11 if name == "config3" else 13)
    x = synth.smooth_field((1, 1, C, H, W), 8.0, 3002).to(device)
    xr = x.bfloat16().float()
    with torch.inference_mode():
        got = model(x)                                  # fp32 input, converted in the patch gather
        assert got.shape == (1, 1, C, H, W) and got.dtype == torch.bfloat16
        assert model.chain_blocks                       # the forward ran the window-order block chain
        model.chain_blocks = False
        got_calls = model(x)                            # one fused call per block
        model.chain_blocks = True
        # embedding
        tok = model.prepare_tokens(x)
        pos = mr.pos_tokens(coords, prm["pos_embed.proj.conv.weight"], prm["pos_embed.proj.conv.bias"], p)
        tw = mr.prepare_tokens(xr, prm["patch_embed.proj.conv.weight"], prm["patch_embed.proj.conv.bias"], p,
                               pos)
        e = rel_l2(tok, tw)
        print(f"  embed: {e:.3e}", flush=True)
        assert e < 1e-2
        del tw, pos
        # every block on the GPU's own input
        worst = 0.0
        for i, blk in enumerate(model.blocks):
            bp = {k[len(f"blocks.{i}."):]: v for k, v in prm.items() if k.startswith(f"blocks.{i}.")}
            xin = tok.float()
            ref = swin_ref.block_forward(xin, bp, heads, ws, mr.block_shift(i, ws), eps=BF16_EPS)
            tok = blk(tok)
            e, eb = rel_l2(tok, ref), rel_l2(tok.float() - xin, ref - xin)
            worst = max(worst, e)
            print(f"  block {i:2d} shift {mr.block_shift(i, ws)}: {e:.3e} (branch {eb:.3e})", flush=True)
            assert e < 1e-2, f"block {i}"
            assert eb < 2e-2, f"block {i} branch"
            del ref, xin
        # head on the last frame
        hw = model._head_last(tok)
        want_h = mr.forward_head(tok.float(), prm["head.weight"], p, C)[:, -1:]
        e = rel_l2(hw, want_h)
        print(f"  head: {e:.3e}", flush=True)
        assert e < 1e-2
        assert torch.equal(hw, got_calls)               # the staged path is the per-block forward
        ec = rel_l2(got, got_calls)
        print(f"  window-order chain vs per-block calls: {ec:.3e}", flush=True)
        del want_h, tok
        # end to end, against the whole oracle model
        want = mr.model_forward(xr, prm, patch_size=p, window_size=ws, depth=depth, num_heads=heads,
                                out_chans=C, coords=coords, eps=BF16_EPS)
        e2e = rel_l2(got, want)
        e2e_calls = rel_l2(got_calls, want)
    print(f"  end-to-end after {depth} blocks: {e2e:.3e} (per-block calls {e2e_calls:.3e}, worst block "
          f"{worst:.3e})", flush=True)
    assert e2e < 3e-2
    assert e2e < 1.25 * e2e_calls
    del model, prm
    torch.cuda.empty_cache()


def test_model_config3_fp32(device):
    """Config 3's model (p4, e1024, depth 16, 16 heads, 70 channels,
    720x1440) in fp32, the reference's inference precision
    (utils/inferencer.py:337-449 runs without autocast): the forward (patch
    embedding into block 0's window order, the window-order block chain,
    the fused head) against the fp32 oracle model on the device, within
    1e-5 relative L2 per stage (embedding, 16 blocks, head)."""
    C, H, W, p, E, heads, ws, depth = CONFIGS["config3"]
    print(f"config3 fp32: p{p} e{E} d{depth} {C}x{H}x{W}", flush=True)
    model, prm, coords = build(device, "config3", seed=11)
    model = model.float()                               # the bf16-rounded weights, in fp32
    x = synth.smooth_field((1, 1, C, H, W), 8.0, 3002).to(device)
    with torch.inference_mode():
        got = model(x)
        assert got.dtype == torch.float32 and model.chain_blocks
        want = mr.model_forward(x, prm, patch_size=p, window_size=ws, depth=depth, num_heads=heads,
                                out_chans=C, coords=coords)
        e2e = rel_l2(got, want)
    print(f"  end-to-end after {depth} blocks: {e2e:.3e}", flush=True)
    assert e2e < 1e-5 * (depth + 2)
    del model, prm, got, want
    torch.cuda.empty_cache()


def test_rollout_config5(device):
    """Config 5: 8 autoregressive steps of the config-3 model (bf16, nsw.Rollout
    with the fused unnormalising RMSE/ACC) against the oracle rollout of the
    same weights in fp32 (utils/inferencer.py:393-449 restated)."""
    import nsw
    C, H, W, p, E, heads, ws, depth = CONFIGS["config3"]
    S = 8
    model, prm, coords = build(device, "config3", seed=17)
    win = synth.smooth_field((1, 1, C, H, W), 8.0, 5002)
    targets = torch.stack([synth.smooth_field((C, H, W), 8.0, 5010 + i) for i in range(S)])
    g = torch.Generator().manual_seed(5003)
    mean = torch.randn(C, generator=g) * 10.0
    std = torch.rand(C, generator=g) * 1.5 + 0.5
    clim = mean + std * torch.randn(C, generator=g) * 0.01
    w = metrics_ref.area_weights(metrics_ref.era5_latitudes(H))
    print(f"config5: {S} steps of the config-3 model, bf16 vs the fp32 oracle", flush=True)
    with torch.inference_mode():
        ro = nsw.Rollout(model, mean, std, torch.from_numpy(w)[:, None], clim=clim)
        r1, a1, f1 = ro.run(win.to(device), targets.to(device), keep_fields=True)
        torch.cuda.synchronize()
        print("  bf16 rollout done", flush=True)

        def oracle_model(inp):
            return mr.model_forward(inp, prm, patch_size=p, window_size=ws, depth=depth, num_heads=heads,
                                    out_chans=C, coords=coords)

        r0, a0, f0 = mr.rollout(oracle_model, win.to(device), None, targets.to(device), mean, std, w, clim)
        print("  fp32 oracle rollout done", flush=True)
    r1, a1 = r1.cpu().numpy(), a1.cpu().numpy()
    r0, a0 = r0.numpy(), a0.numpy()
    fld = [rel_l2(f1[i], f0[i]) for i in range(S)]
    rdrift = (np.abs(r1 - r0) / r0).max(axis=1)
    adrift = np.abs(a1 - a0).max(axis=1)
    print(json.dumps({"config5_drift_vs_fp32_oracle": {
        "field_rel_l2": [round(v, 6) for v in fld],
        "rmse_rel_drift_max": [round(float(v), 6) for v in rdrift],
        "acc_abs_drift_max": [round(float(v), 6) for v in adrift],
        "rmse_mean_bf16": [round(float(v), 6) for v in r1.mean(1)],
        "rmse_mean_fp32_oracle": [round(float(v), 6) for v in r0.mean(1)],
        "acc_mean_bf16": [round(float(v), 6) for v in a1.mean(1)]}}), flush=True)
    assert max(fld) < 3e-2
    assert rdrift.max() < 1e-2
    assert adrift.max() < 1e-2
    del model, prm, f0, f1
    torch.cuda.empty_cache()


def test_rollout_config5_bench_setup(device):
    """Config 5 on bench.py's own model and inputs (bench.config3_model,
    bench.rollout_setup): the bf16 rollout (nsw.Rollout) against the fp32
    oracle rollout of the same weights (bf16 values in fp32) and inputs.
    The oracle's per-step RMSE / ACC are what bench.py's rollout drift is
    measured against: they are kept in tests/golden/rollout_c5_fp32_oracle.json
    (written to $NSW_GOLDEN_OUT when set) and must be reproduced here."""
    import os
    import sys
    import nsw
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    if root not in sys.path:
        sys.path.insert(0, root)
    import bench
    C, H, W, p, E, depth, heads, ws, T = bench.C3
    S = bench.ROLLOUT_STEPS
    model, x = bench.config3_model(device)
    mean, std, clim, w, targets = bench.rollout_setup(device)
    print(f"config5 (bench setup): {S} steps, bf16 vs the fp32 oracle", flush=True)
    with torch.inference_mode():
        r1, a1, _ = nsw.Rollout(model, mean, std, w, clim=clim).run(x, targets)
        torch.cuda.synchronize()
        prm = {k: v.float() for k, v in model.state_dict().items()}
        coords = model.coords.float()

        def oracle_model(inp):
            return mr.model_forward(inp, prm, patch_size=p, window_size=ws, depth=depth, num_heads=heads,
                                    out_chans=C, coords=coords)

        r0, a0, _ = mr.rollout(oracle_model, x, None, targets, mean, std, w[:, 0].double().numpy(), clim)
    r1, a1, r0, a0 = r1.cpu().numpy(), a1.cpu().numpy(), r0.numpy(), a0.numpy()
    rdrift = (np.abs(r1 - r0) / r0).max(axis=1)
    adrift = np.abs(a1 - a0).max(axis=1)
    rec = {"steps": S, "channels": C,
           "setup": "bench.config3_model (seeds 3001 / 3002) + bench.rollout_setup (seeds 3003 / 3004); "
                    "oracle/model_ref.rollout in fp32 on the GPU, TF32 off",
           "rmse": [[float(v) for v in row] for row in r0], "acc": [[float(v) for v in row] for row in a0]}
    out = os.environ.get("NSW_GOLDEN_OUT")
    if out:
        with open(out, "w") as fh:
            json.dump(rec, fh)
    print(json.dumps({"config5_bench_setup_drift_vs_fp32_oracle": {
        "rmse_rel_drift_max": [round(float(v), 6) for v in rdrift],
        "acc_abs_drift_max": [round(float(v), 6) for v in adrift]}}), flush=True)
    assert rdrift.max() < 1e-2
    assert adrift.max() < 1e-2
    golden = os.path.join(root, "tests", "golden", "rollout_c5_fp32_oracle.json")
    if os.path.exists(golden):
        with open(golden) as fh:
            g = json.load(fh)
        np.testing.assert_allclose(r0, np.asarray(g["rmse"]), rtol=1e-4)
        np.testing.assert_allclose(a0, np.asarray(g["acc"]), rtol=0, atol=1e-5)
    del model
    torch.cuda.empty_cache()

