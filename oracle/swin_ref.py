"""fp32 CPU restatement of the reference Swin block forward (test oracle only).

Every function follows one reference routine, cited by file:line of
ShashankSubramanian/neural-scaling-weather.  The op sequence (including where
the residuals, norms, biases and the additive mask enter) is the reference's;
the code is an independent eager-mode restatement in plain PyTorch, run on
the CPU, or (for the full-size checks) with fp32 library kernels on a GPU
device, whichever device its inputs are on.

Single-GPU semantics: every communicator has size 1, so the reference's
distributed wrappers (``identity_forward_allreduce_backward``,
``allreduce_forward_identity_backward``, ``split_forward_allgather_backward``)
are identities and ``_distributed_roll`` is ``torch.roll``
(``distributed/helpers.py:210-212``).

Pinning (see ``tests/test_oracle_block.py``):
  * roll / partition / reverse / mask: bit-exact against the numpy closed forms
    and brute-force loops of ``oracle.index_maps``;
  * rms_norm: ``torch.nn.RMSNorm`` (eps=None) library routine;
  * attention core: ``F.scaled_dot_product_attention`` math path and a
    hand-rolled softmax, plus special cases (uniform keys -> mean of values,
    -100 mask -> blocked keys);
  * mlp: ``F.linear`` + ``nn.GELU()`` (erf) library routines;
  * block composition (residual / norm placement, QK-norm before the scale):
    special-case constructions that reduce the block to a closed form
    (zero weights -> identity plus biases; single-window brute force loop).
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

# ----------------------------------------------------------------------------
# index work
# ----------------------------------------------------------------------------


def roll(x: torch.Tensor, shifts: Sequence[int], dims: Sequence[int]) -> torch.Tensor:
    """``RollForwardReverseRollBackward.forward`` (distributed/mappings.py:121-132):
    one ``torch.roll`` per dim, skipped when the shift is 0; on one GPU
    ``_distributed_roll`` is ``torch.roll`` (distributed/helpers.py:204-212)."""
    for s, d in zip(shifts, dims):
        if s != 0:
            x = torch.roll(x, shifts=(s,), dims=(d,))
    return x


def window_partition(x: torch.Tensor, window_size: Tuple[int, int]) -> torch.Tensor:
    """models/swin_helpers.py:26-51: [B,T,H,W,C] -> [B*nW, T, ws0, ws1, C],
    window index = b*nW + i*(W/ws1) + j."""
    B, T, H, W, C = x.shape
    a, b = window_size
    v = x.reshape(B, T, H // a, a, W // b, b, C)
    v = v.permute(0, 2, 4, 1, 3, 5, 6).contiguous()
    return v.reshape(-1, T, a, b, C)


def window_reverse(windows: torch.Tensor, window_size: Tuple[int, int],
                   img_size: Tuple[int, int]) -> torch.Tensor:
    """models/swin_helpers.py:54-77: inverse of :func:`window_partition`."""
    H, W = img_size
    a, b = window_size
    T, C = windows.shape[1], windows.shape[-1]
    nh, nw = H // a, W // b
    B = windows.shape[0] // (nh * nw)
    v = windows.reshape(B, nh, nw, T, a, b, C)
    v = v.permute(0, 3, 1, 4, 2, 5, 6).contiguous()
    return v.reshape(B, T, H, W, C)


def make_attention_mask(H: int, W: int, window_size: Tuple[int, int],
                        shift_size: Tuple[int, int], T: int = 1,
                        causal: bool = False, device=None) -> torch.Tensor:
    """``Block._make_attention_mask`` (models/swin_helpers.py:322-397), one GPU
    (sp shapes [H], [W]).  Returns the additive fp32 mask [nW, T*wa, T*wa].

    Latitude labels only: rows [0, H-ws0) get 0, rows [H-s0, H) get 1, rows
    [H-ws0, H-s0) keep the initial 0 (:353-356).  Pairs with different labels
    get -100.0 (:376-378).  The temporal part is zero (or -100 upper triangular
    when causal, :333-345) and is added per (t_q, t_k) block (:383-395)."""
    a, b = window_size
    wa = a * b
    if causal:
        temporal = torch.triu(torch.ones(T, T), diagonal=1)
        temporal = torch.where(temporal == 1, torch.tensor(-100.0), torch.tensor(0.0))
    else:
        temporal = torch.zeros(T, T)
    # [1, T, T, wa, wa]
    temporal = temporal[:, :, None, None].expand(T, T, wa, wa)[None]
    if any(shift_size):
        img = torch.zeros(1, 1, H, W, 1)
        img[:, :, 0:H - a] = 0.0
        img[:, :, H - shift_size[0]:H] = 1.0
        lab = window_partition(img, window_size).reshape(-1, wa)  # [nW, wa]
        diff = lab[:, None, :] - lab[:, :, None]                   # [nW, wa(q), wa(k)]
        spatial = torch.where(diff != 0, torch.tensor(-100.0), torch.tensor(0.0))
        combined = spatial[:, None, None].expand(-1, T, T, wa, wa) + temporal
    else:
        nW = (H // a) * (W // b)
        combined = temporal.expand(nW, T, T, wa, wa)
    # [nW, Tq, Tk, wa, wa] -> [nW, Tq, wa, Tk, wa] -> [nW, T*wa, T*wa]
    m = combined.permute(0, 1, 3, 2, 4).reshape(-1, T * wa, T * wa).contiguous()
    return m if device is None else m.to(device)


# ----------------------------------------------------------------------------
# floating-point pieces
# ----------------------------------------------------------------------------


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: Optional[float] = None) -> torch.Tensor:
    """``NormLayer(norm_type="rms_norm")`` -> ``nn.RMSNorm`` with eps=None
    (models/layer_helpers.py:101-119): y = x * rsqrt(mean(x^2) + eps) * w,
    eps = finfo(x.dtype).eps."""
    if eps is None:
        eps = torch.finfo(x.dtype).eps
    ms = x.pow(2).mean(dim=-1, keepdim=True)
    return x * torch.rsqrt(ms + eps) * weight


def gelu_erf(x: torch.Tensor, approximate: str = "none") -> torch.Tensor:
    """``nn.GELU()`` default (approximate='none'), models/mlp.py:55,82: the
    library routine the reference calls, x * Phi(x) with the exact erf.
    ``approximate="tanh"``: the tanh form, the "gelu" activation of the TE
    block's te.LayerNormMLP (models/swin_helpers_te.py:318-323)."""
    return F.gelu(x, approximate=approximate)


def window_attention(x: torch.Tensor, p: Dict[str, torch.Tensor], num_heads: int,
                     mask: Optional[torch.Tensor] = None,
                     eps: Optional[float] = None) -> torch.Tensor:
    """``WindowMultiHeadAttention.forward`` (models/swin_helpers.py:203-256).

    x: [Bw, L, C].  q/k/v = F.linear (no bias, layer_helpers.py:41-42) then a
    separate bias add (layer_helpers.py:71-72); per-head RMSNorm on q and k
    (:233-234); SDPA with scale hd^-1/2 and the additive mask broadcast over
    heads and over the batch of windows (:236-247); heads merged (:249); proj
    then its bias after the (identity) all-reduce (:250-254)."""
    Bw, L, C = x.shape
    hd = C // num_heads

    def heads(t):
        return t.reshape(Bw, L, num_heads, hd).permute(0, 2, 1, 3)

    q = heads(F.linear(x, p["attn.q.weight"]) + p["attn.biasq.bias"])
    k = heads(F.linear(x, p["attn.k.weight"]) + p["attn.biask.bias"])
    v = heads(F.linear(x, p["attn.v.weight"]) + p["attn.biasv.bias"])
    q = rms_norm(q, p["attn.q_norm.norm.weight"], eps)
    k = rms_norm(k, p["attn.k_norm.norm.weight"], eps)
    # k^T materialised: the same product, and no transposed-view operand in
    # batched GPU matmuls when the oracle runs on a device
    scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) * (hd ** -0.5)
    if mask is not None:
        nW = mask.shape[0]
        m = mask[None].expand(Bw // nW, nW, L, L).reshape(Bw, 1, L, L)
        scores = scores + m
    probs = torch.softmax(scores, dim=-1)
    o = torch.matmul(probs, v)
    o = o.transpose(1, 2).reshape(Bw, L, C)
    o = F.linear(o, p["attn.proj.weight"])
    return o + p["attn.biasproj.bias"]


def mlp(x: torch.Tensor, p: Dict[str, torch.Tensor], gelu: str = "none") -> torch.Tensor:
    """``MLP.forward`` (models/mlp.py:75-95): fc1 -> +bias1 -> GELU(erf) ->
    dropout(identity) -> fc2 -> +bias2 (after the identity all-reduce)."""
    h = F.linear(x, p["mlp.fc1.weight"]) + p["mlp.bias1.bias"]
    h = gelu_erf(h, gelu)
    y = F.linear(h, p["mlp.fc2.weight"])
    return y + p["mlp.bias2.bias"]


def shifted_window_attn(x: torch.Tensor, p: Dict[str, torch.Tensor], num_heads: int,
                        window_size: Tuple[int, int], shift_size: Tuple[int, int],
                        mask: torch.Tensor, eps: Optional[float] = None) -> torch.Tensor:
    """``Block._shifted_window_attn`` (models/swin_helpers.py:399-433)."""
    B, T, H, W, C = x.shape
    x = roll(x, tuple(-s for s in shift_size), (-3, -2))
    xw = window_partition(x, window_size)
    xw = xw.reshape(-1, T * window_size[0] * window_size[1], C)
    o = window_attention(xw, p, num_heads, mask=mask, eps=eps)
    o = o.reshape(-1, T, window_size[0], window_size[1], C)
    y = window_reverse(o, window_size, (H, W))
    return roll(y, tuple(shift_size), (-3, -2))


def block_forward(x: torch.Tensor, p: Dict[str, torch.Tensor], num_heads: int,
                  window_size: Tuple[int, int], shift_size: Tuple[int, int],
                  mask: Optional[torch.Tensor] = None,
                  eps: Optional[float] = None, gelu: str = "none") -> torch.Tensor:
    """``Block.forward`` (models/swin_helpers.py:435-459): pre-norm residual
    attention, then pre-norm residual MLP over [B, T*H*W, C].  ``gelu`` and
    ``eps`` = ("tanh", 1e-5) give the TE block's arithmetic
    (models/swin_helpers_te.py:302, 318-323: te.RMSNorm / te.LayerNormMLP at
    their default eps and TE's tanh-form "gelu")."""
    B, T, H, W, C = x.shape
    if mask is None:
        mask = make_attention_mask(H, W, window_size, shift_size, T, device=x.device)
    skip = x
    h = rms_norm(x, p["norm1.norm.weight"], eps)
    h = shifted_window_attn(h, p, num_heads, window_size, shift_size, mask, eps)
    x = h + skip
    x = x.reshape(B, -1, C)
    y = mlp(rms_norm(x, p["norm2.norm.weight"], eps), p, gelu) + x
    return y.reshape(B, T, H, W, C)


# ----------------------------------------------------------------------------
# parameters (names = the reference's vanilla state-dict keys of one block)
# ----------------------------------------------------------------------------

BLOCK_PARAM_SHAPES = {
    "norm1.norm.weight": lambda C, hd, Hm: (C,),
    "attn.q.weight": lambda C, hd, Hm: (C, C),
    "attn.biasq.bias": lambda C, hd, Hm: (C,),
    "attn.k.weight": lambda C, hd, Hm: (C, C),
    "attn.biask.bias": lambda C, hd, Hm: (C,),
    "attn.q_norm.norm.weight": lambda C, hd, Hm: (hd,),
    "attn.k_norm.norm.weight": lambda C, hd, Hm: (hd,),
    "attn.v.weight": lambda C, hd, Hm: (C, C),
    "attn.biasv.bias": lambda C, hd, Hm: (C,),
    "attn.proj.weight": lambda C, hd, Hm: (C, C),
    "attn.biasproj.bias": lambda C, hd, Hm: (C,),
    "norm2.norm.weight": lambda C, hd, Hm: (C,),
    "mlp.fc1.weight": lambda C, hd, Hm: (Hm, C),
    "mlp.bias1.bias": lambda C, hd, Hm: (Hm,),
    "mlp.fc2.weight": lambda C, hd, Hm: (C, Hm),
    "mlp.bias2.bias": lambda C, hd, Hm: (C,),
}
