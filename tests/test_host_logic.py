"""Host-side logic of the drop-in modules (no GPU): parameter names, shapes
and init match the reference; checkpoint layouts map both ways."""
import numpy as np
import pytest
import torch

from oracle import metrics_ref
from oracle.swin_ref import BLOCK_PARAM_SHAPES


def make_block(C=64, heads=2, shift=(4, 9), T=1):
    import nsw
    return nsw.Block(dim=C, num_heads=heads, feat_size=(18, 36), window_size=(9, 18),
                     temporal_context_window_size=T, shift_size=shift)


def test_block_state_dict_keys_and_shapes_match_reference():
    blk = make_block()
    sd = blk.state_dict()
    C, hd, Hm = 64, 32, 256
    assert set(sd) == set(BLOCK_PARAM_SHAPES)
    for k, shp in BLOCK_PARAM_SHAPES.items():
        assert tuple(sd[k].shape) == shp(C, hd, Hm), k


def test_block_init_matches_reference_distribution():
    torch.manual_seed(0)
    blk = make_block(C=256, heads=4)
    w = blk.attn.q.weight.detach()
    assert abs(w.std().item() - 0.02) < 0.002 and w.abs().max().item() < 0.2
    assert torch.all(blk.attn.biasq.bias == 0) and torch.all(blk.norm1.norm.weight == 1)
    assert blk.attn.q_norm.norm.weight.shape == (64,)


def test_block_loads_oracle_params_and_packs():
    from oracle import synth
    blk = make_block()
    p = synth.block_params(64, 2, seed=1, random_bias=True)
    blk.load_state_dict(p)
    pk = blk.packed()
    assert torch.equal(pk["wqkv"], torch.cat([p["attn.q.weight"], p["attn.k.weight"], p["attn.v.weight"]]))
    assert torch.equal(pk["bqkv"], torch.cat([p["attn.biasq.bias"], p["attn.biask.bias"], p["attn.biasv.bias"]]))
    # cache invalidates when a parameter changes in place
    with torch.no_grad():
        blk.attn.k.weight.add_(1.0)
    assert torch.equal(blk.packed()["wqkv"][64:128], p["attn.k.weight"] + 1.0)


def test_constructor_checks_mirror_reference():
    import nsw
    with pytest.raises(AssertionError):
        nsw.WindowMultiHeadAttention(dim=30, num_heads=4, window_size=(9, 18))
    with pytest.raises(ValueError):
        nsw.Block(dim=64, num_heads=2, feat_size=(10, 36), window_size=(9, 18), temporal_context_window_size=1)


def test_checkpoint_te_vanilla_roundtrip():
    from nsw import checkpoint as ck
    blk = make_block()
    sd = {f"module.model.blocks.3.{k}": v for k, v in blk.state_dict().items()}
    sd["module.model.head.weight"] = torch.zeros(3)
    te = ck.vanilla_to_te(ck.strip_prefixes(sd))
    assert "blocks.3.rms_norm_mlp.fc1_weight" in te and "blocks.3.attn.q.bias" in te
    te["blocks.3.attn.q._extra_state"] = None
    back = ck.to_vanilla({"module.model." + k: v for k, v in te.items()})
    assert set(back) == set(ck.strip_prefixes(sd))
    blk2 = make_block()
    blk2.load_state_dict(ck.block_state(back, 3))
    for k, v in blk.state_dict().items():
        assert torch.equal(blk2.state_dict()[k], v)


def test_te_map_covers_every_vanilla_block_key():
    from nsw import checkpoint as ck
    assert set(ck.BLOCK_KEYS) == set(BLOCK_PARAM_SHAPES)


def test_area_weights_match_oracle():
    from nsw.misc_utils import build_spherical_area_weights, era5_latitudes
    w = build_spherical_area_weights(era5_latitudes(720))
    assert w.dtype == torch.float64
    assert np.allclose(w.numpy(), metrics_ref.area_weights(metrics_ref.era5_latitudes(720)), rtol=0, atol=0)


def test_mlp_rejects_unfusable_activation():
    from nsw.mlp import MLP
    m = MLP(16, 32, act_layer=torch.nn.ReLU)
    with pytest.raises(NotImplementedError):
        m._check_fusable()


def test_full_model_te_checkpoint_loads_into_swin_transformer(tmp_path):
    """A reference checkpoint of the whole model in production layout (TE block
    names, DDP + TimeStepper prefixes, TE _extra_state entries) saved as
    {"model_state": ...} loads through the safe loader into nsw.SwinTransformer
    with every tensor in place (models/helpers.py:53-70, tests/test_te.py:34-71)."""
    import torch
    import nsw
    from nsw import checkpoint
    from oracle import synth
    C, E, depth, heads, p, H, W = 6, 64, 2, 4, 2, 36, 72
    prm = synth.model_params(C, C, E, depth, heads, p, seed=11, random_bias=True, random_norm=True)
    te = checkpoint.vanilla_to_te(prm)
    state = {"module.model." + k: v for k, v in te.items()}
    state["module.model.blocks.0.rms_norm_mlp._extra_state"] = torch.zeros(3)
    state["module.model.blocks.1.attn.q._extra_state"] = torch.zeros(2)
    path = tmp_path / "ckpt_best.tar"
    torch.save({"model_state": state, "epoch": 3}, path)
    loaded = checkpoint.load_checkpoint_model_state(str(path))
    meta = {"coords": torch.rand(H, W, 3), "sp_shapes": [[H], [W]], "n_channels": C}
    model = nsw.SwinTransformer(temporal_context_window_size=1, window_size=(9, 18), patch_size=p, in_chans=C,
                                out_chans=C, embed_dim=E, depth=depth, num_heads=heads, domain_metadata=meta)
    model.load_state_dict(loaded, strict=True)
    sd = model.state_dict()
    assert set(sd) == set(prm)
    for k, v in prm.items():
        assert torch.equal(sd[k], v), k


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N with N > 1 exits (status 2) with one JSON line that
    says the build runs on one GPU, before it initialises any device."""
    import json
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], cwd=root,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2, r.stderr
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]
