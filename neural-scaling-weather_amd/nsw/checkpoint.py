"""Checkpoint state-dict layouts of the Swin block.

The reference writes ``model_state`` with DDP's ``module.`` and TimeStepper's
``model.`` prefixes (models/helpers.py:14,53-70) and, in production, with
Transformer-Engine parameter names (config/parallelism/hybrid.yaml:9).  The
vanilla <-> TE correspondence is the one the reference's own test spells out
(tests/test_te.py:34-71):

    vanilla                              TE
    norm1.norm.weight                    norm1.weight
    attn.{q,k,v,proj}.weight             attn.{q,k,v,proj}.weight
    attn.bias{q,k,v,proj}.bias           attn.{q,k,v,proj}.bias
    attn.{q,k}_norm.norm.weight          attn.{q,k}_norm.weight
    norm2.norm.weight                    rms_norm_mlp.layer_norm_weight
    mlp.fc1.weight / mlp.bias1.bias      rms_norm_mlp.fc1_weight / fc1_bias
    mlp.fc2.weight / mlp.bias2.bias      rms_norm_mlp.fc2_weight / fc2_bias

TE's ``*_extra_state`` entries carry FP8 metadata and are dropped.

The TE block also computes differently from the vanilla one: its norms are
te.RMSNorm / te.LayerNormMLP at their default eps = 1e-5 (the vanilla
nn.RMSNorm(eps=None) takes finfo(dtype).eps) and its MLP activation "gelu" is
the tanh form (the vanilla block uses the exact erf).  ``apply_te_semantics``
switches a model's blocks to that arithmetic; ``load_model_checkpoint`` does
it whenever the file holds TE-layout weights.
"""
from __future__ import annotations

import re
from collections import OrderedDict
from typing import Dict, Mapping

# TE suffix -> vanilla suffix, relative to a block prefix "blocks.{i}."
_TE_TO_VANILLA = {
    "norm1.weight": "norm1.norm.weight",
    "attn.q.weight": "attn.q.weight",
    "attn.q.bias": "attn.biasq.bias",
    "attn.k.weight": "attn.k.weight",
    "attn.k.bias": "attn.biask.bias",
    "attn.v.weight": "attn.v.weight",
    "attn.v.bias": "attn.biasv.bias",
    "attn.q_norm.weight": "attn.q_norm.norm.weight",
    "attn.k_norm.weight": "attn.k_norm.norm.weight",
    "attn.proj.weight": "attn.proj.weight",
    "attn.proj.bias": "attn.biasproj.bias",
    "rms_norm_mlp.layer_norm_weight": "norm2.norm.weight",
    "rms_norm_mlp.fc1_weight": "mlp.fc1.weight",
    "rms_norm_mlp.fc1_bias": "mlp.bias1.bias",
    "rms_norm_mlp.fc2_weight": "mlp.fc2.weight",
    "rms_norm_mlp.fc2_bias": "mlp.bias2.bias",
}
_VANILLA_TO_TE = {v: k for k, v in _TE_TO_VANILLA.items()}

BLOCK_KEYS = tuple(_VANILLA_TO_TE.keys())

_BLOCK_RE = re.compile(r"^(?P<pre>(?:.*\.)?blocks\.\d+\.)(?P<rest>.+)$")


def strip_prefixes(sd: Mapping[str, object], prefixes=("module.", "model.")) -> "OrderedDict[str, object]":
    """Remove DDP / TimeStepper prefixes (models/helpers.py:53-70 strips
    ``module.``; TimeStepper adds ``model.``)."""
    out = OrderedDict()
    for k, v in sd.items():
        changed = True
        while changed:
            changed = False
            for p in prefixes:
                if k.startswith(p):
                    k = k[len(p):]
                    changed = True
        out[k] = v
    return out


def te_to_vanilla(sd: Mapping[str, object]) -> "OrderedDict[str, object]":
    """Rename TE block keys to the vanilla layout; drop ``_extra_state``."""
    out = OrderedDict()
    for k, v in sd.items():
        if k.endswith("_extra_state"):
            continue
        m = _BLOCK_RE.match(k)
        if m and m.group("rest") in _TE_TO_VANILLA:
            k = m.group("pre") + _TE_TO_VANILLA[m.group("rest")]
        out[k] = v
    return out


def vanilla_to_te(sd: Mapping[str, object]) -> "OrderedDict[str, object]":
    out = OrderedDict()
    for k, v in sd.items():
        m = _BLOCK_RE.match(k)
        if m and m.group("rest") in _VANILLA_TO_TE:
            k = m.group("pre") + _VANILLA_TO_TE[m.group("rest")]
        out[k] = v
    return out


def is_te_layout(sd: Mapping[str, object]) -> bool:
    return any(k.endswith("rms_norm_mlp.fc1_weight") or k.endswith("_extra_state") for k in sd)


def to_vanilla(sd: Mapping[str, object]) -> "OrderedDict[str, object]":
    """Any reference checkpoint layout -> vanilla keys without prefixes."""
    sd = strip_prefixes(sd)
    return te_to_vanilla(sd) if is_te_layout(sd) else OrderedDict(sd)


def block_state(sd: Mapping[str, object], index: int) -> Dict[str, object]:
    """The vanilla state dict of block ``index`` (keys relative to the block)."""
    sd = to_vanilla(sd)
    pre = f"blocks.{index}."
    return {k[len(pre):]: v for k, v in sd.items() if k.startswith(pre)}


def load_checkpoint_model_state(path: str) -> "OrderedDict[str, object]":
    """Read ``model_state`` of a reference checkpoint file with the safe loader
    (tensors only; nothing in the file is executed)."""
    import torch
    ck = torch.load(path, map_location="cpu", weights_only=True)
    return to_vanilla(ck["model_state"] if "model_state" in ck else ck)


TE_EPS = 1e-5


def apply_te_semantics(model) -> int:
    """Give every nsw.Block of ``model`` the TE block's arithmetic: eps = 1e-5
    on norm1, norm2, q_norm and k_norm (te.RMSNorm / te.LayerNormMLP defaults,
    models/swin_helpers_te.py:132-137, 302, 318) and the tanh-form GELU (TE's
    "gelu", :318-323).  Returns the number of blocks changed."""
    from torch import nn

    from .swin_helpers import Block
    n = 0
    for m in model.modules():
        if isinstance(m, Block):
            for norm in (m.norm1, m.norm2, m.attn.q_norm, m.attn.k_norm):
                norm.norm.eps = TE_EPS
            m.mlp.act = nn.GELU(approximate="tanh")
            n += 1
    return n


def load_model_checkpoint(model, path: str, strict: bool = True, te_semantics: bool = True):
    """Load a reference checkpoint file (any prefix / TE or vanilla layout)
    into ``model`` with the safe loader.  When the file holds TE-layout block
    weights and ``te_semantics`` is set, the blocks are switched to the TE
    arithmetic (``apply_te_semantics``) so that they compute what the
    checkpoint was trained with.  Returns (missing, unexpected, te_layout)."""
    import torch
    ck = torch.load(path, map_location="cpu", weights_only=True)
    raw = ck["model_state"] if "model_state" in ck else ck
    te = is_te_layout(strip_prefixes(raw))
    sd = to_vanilla(raw)
    missing, unexpected = model.load_state_dict(sd, strict=False)
    missing = [k for k in missing if not k.endswith("attn_mask")]
    if strict and (missing or unexpected):
        raise RuntimeError(f"checkpoint does not match the model: missing {missing}, unexpected {unexpected}")
    if te and te_semantics:
        apply_te_semantics(model)
    return missing, unexpected, te
