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
    t = MLP(16, 32, act_layer=lambda: torch.nn.GELU(approximate="tanh"))
    t._check_fusable()
    assert t.gelu_tanh


@pytest.mark.parametrize("H,W,ws,shift,T", [(18, 36, (9, 18), (4, 9), 1), (18, 36, (9, 18), (4, 9), 2),
                                            (18, 36, (9, 18), (0, 0), 1), (18, 36, (9, 18), (0, 9), 1),
                                            (16, 32, (4, 8), (2, 4), 1), (24, 16, (4, 8), (6, 4), 1)])
def test_block_attn_mask_buffer_at_construction(H, W, ws, shift, T):
    """The reference registers attn_mask as a non-persistent buffer when the
    block is built (models/swin_helpers.py:320,397): available on the CPU,
    equal to the oracle's mask, absent from the state dict, moved and cast
    with the module."""
    import nsw
    from oracle import swin_ref
    blk = nsw.Block(dim=64, num_heads=2, feat_size=(H, W), window_size=ws, temporal_context_window_size=T,
                    shift_size=shift)
    assert blk.attn_mask.device.type == "cpu" and blk.attn_mask.dtype == torch.float32
    assert torch.equal(blk.attn_mask, swin_ref.make_attention_mask(H, W, ws, shift, T))
    assert "attn_mask" not in blk.state_dict()
    assert torch.equal(blk.to(torch.bfloat16).attn_mask.float(), swin_ref.make_attention_mask(H, W, ws, shift, T))


def test_apply_te_semantics():
    """TE-layout checkpoints switch the blocks to the TE arithmetic: eps 1e-5
    on all four RMSNorms and the tanh-form GELU (models/swin_helpers_te.py)."""
    import nsw
    from nsw import checkpoint
    meta = {"coords": torch.rand(36, 72, 3), "sp_shapes": [[36], [72]], "n_channels": 4}
    model = nsw.SwinTransformer(temporal_context_window_size=1, window_size=(9, 18), patch_size=2, in_chans=4,
                                out_chans=4, embed_dim=64, depth=2, num_heads=2, domain_metadata=meta)
    assert checkpoint.apply_te_semantics(model) == 2
    for blk in model.blocks:
        assert blk._eps(torch.bfloat16) == 1e-5 and blk._eps(torch.float32) == 1e-5
        assert blk.mlp.gelu_tanh


def test_load_model_checkpoint_te_and_vanilla(tmp_path):
    import nsw
    from nsw import checkpoint
    from oracle import synth
    C, E, depth, heads, p, H, W = 4, 64, 2, 2, 2, 36, 72
    meta = {"coords": torch.rand(H, W, 3), "sp_shapes": [[H], [W]], "n_channels": C}

    def mk():
        return nsw.SwinTransformer(temporal_context_window_size=1, window_size=(9, 18), patch_size=p, in_chans=C,
                                   out_chans=C, embed_dim=E, depth=depth, num_heads=heads, domain_metadata=meta)
    prm = synth.model_params(C, C, E, depth, heads, p, seed=5)
    torch.save({"model_state": {"module.model." + k: v for k, v in checkpoint.vanilla_to_te(prm).items()}},
               tmp_path / "te.tar")
    torch.save({"model_state": {"module." + k: v for k, v in prm.items()}}, tmp_path / "van.tar")
    m = mk()
    _, _, te = checkpoint.load_model_checkpoint(m, str(tmp_path / "te.tar"))
    assert te and all(b.mlp.gelu_tanh for b in m.blocks)
    m2 = mk()
    _, _, te2 = checkpoint.load_model_checkpoint(m2, str(tmp_path / "van.tar"))
    assert not te2 and not any(b.mlp.gelu_tanh for b in m2.blocks)
    for k, v in prm.items():
        assert torch.equal(m.state_dict()[k], v) and torch.equal(m2.state_dict()[k], v), k


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


def test_workspace_cache_keeps_buffers_a_capture_has_seen(monkeypatch):
    """The per-stream workspace grows by replacement; a buffer handed out
    while the stream was being captured into a graph stays alive after it is
    replaced (replays still write it), any other one is released."""
    import gc
    import weakref
    from nsw import ops

    class _Stream:
        cuda_stream = 12345

    capturing = [False]
    monkeypatch.setattr(torch.cuda, "current_stream", lambda device=None: _Stream())
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: capturing[0])
    monkeypatch.setattr(ops, "_workspaces", {})
    monkeypatch.setattr(ops, "_ws_retired", [])
    dev = torch.device("cpu")

    a = ops.workspace(100, dev)
    assert ops.workspace(64, dev) is a                 # smaller: same buffer
    ra = weakref.ref(a)
    del a
    b = ops.workspace(200, dev)                        # grows: the uncaptured buffer goes
    gc.collect()
    assert ra() is None and b.numel() >= 200

    capturing[0] = True
    assert ops.workspace(150, dev) is b                # handed out under capture
    capturing[0] = False
    rb = weakref.ref(b)
    del b
    c = ops.workspace(400, dev)                        # grows: the captured one is retired, kept
    gc.collect()
    assert rb() is not None and any(t is rb() for t in ops._ws_retired)
    assert c.numel() >= 400 and ops.workspace(400, dev) is c


def test_big_skip_conv_parameters():
    """use_big_skip_conv=True (models/swin.py:212-223): a bias-free 1x1
    Conv2DLayer skip_conv [out_chans, in_chans, 1, 1], trunc_normal(0.02)
    initialised, in the state dict under the reference's key; the oracle's
    parameter set for the same model loads strictly."""
    import nsw
    from oracle import synth
    C_in, C_out, H, W, p, E, heads, depth = 5, 4, 36, 72, 2, 64, 2, 2
    meta = {"coords": torch.rand(H, W, 3), "sp_shapes": [[H], [W]], "n_channels": C_out}
    torch.manual_seed(0)
    m = nsw.SwinTransformer(temporal_context_window_size=1, window_size=(9, 18), patch_size=p, in_chans=C_in,
                            out_chans=C_out, embed_dim=E, depth=depth, num_heads=heads, use_big_skip_conv=True,
                            domain_metadata=meta)
    w = m.skip_conv.conv.weight
    assert tuple(w.shape) == (C_out, C_in, 1, 1) and m.skip_conv.conv.bias is None
    assert w.abs().max() <= 0.04 + 1e-6 and 0.005 < w.std().item() < 0.04
    prm = synth.model_params(C_in, C_out, E, depth, heads, p, seed=5, big_skip=True)
    m.load_state_dict(prm, strict=True)
    assert "skip_conv.conv.weight" in m.state_dict()
    m2 = nsw.SwinTransformer(temporal_context_window_size=1, window_size=(9, 18), patch_size=p, in_chans=C_in,
                             out_chans=C_out, embed_dim=E, depth=depth, num_heads=heads, domain_metadata=meta)
    assert not hasattr(m2, "skip_conv")
