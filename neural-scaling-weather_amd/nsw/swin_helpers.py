"""Drop-in Swin block for neural-scaling-weather on MI355X.

Same classes, constructor signatures, attribute names and state-dict keys as
the reference's non-TE block (models/swin_helpers.py), so ``SwinTransformer``
can select it as its block class (models/swin.py:173-177) and load existing
checkpoints.  Every forward runs libnsw HIP kernels:

* ``Block.forward`` is one C-ABI call (``nsw_swin_block_forward``): fused
  norm1 + roll + partition gather, QKV GEMM with bias and per-head q/k
  RMSNorm epilogue, window attention with the shift mask computed from
  indices, proj GEMM with bias + reverse/unroll scatter + residual epilogue,
  RMSNorm, fc1 GEMM with bias + erf-GELU, fc2 GEMM with bias + residual.
* ``WindowMultiHeadAttention.forward`` and the module-level helpers call the
  individual kernels (a materialised mask tensor is honoured).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib, ops, torch_ops
from .layer_helpers import BiasLayer, LinearLayer, NormLayer
from .mlp import MLP
from .profiler_utils import profile


def window_partition(x: torch.Tensor, window_size: Tuple[int, int]) -> torch.Tensor:
    """models/swin_helpers.py:26-51: [B,T,H,W,C] -> [B*nW, T, ws0, ws1, C]."""
    return torch.ops.nsw.window_partition(x, [int(w) for w in window_size])


def window_reverse(windows: torch.Tensor, window_size: Tuple[int, int],
                   img_size: Tuple[int, int]) -> torch.Tensor:
    """models/swin_helpers.py:54-77: [B*nW, T, ws0, ws1, C] -> [B,T,H,W,C]."""
    return torch.ops.nsw.window_reverse(windows, [int(w) for w in window_size], [int(v) for v in img_size])


def roll_forward_reverseroll_backward(x, shifts, dims, comm_names=None):
    """distributed/mappings.py:207-209 on one GPU: torch.roll over (H, W)."""
    dims = tuple(d % x.dim() for d in dims)
    if dims != (x.dim() - 3, x.dim() - 2) or x.dim() != 5:
        raise NotImplementedError("libnsw rolls the (H, W) dims of a [B,T,H,W,C] tensor")
    if not any(shifts):
        return x
    return torch.ops.nsw.roll_hw(x, [int(v) for v in shifts])


def attention_mask_closed_form(H: int, W: int, window_size: Tuple[int, int], shift_size: Tuple[int, int],
                               T: int = 1) -> torch.Tensor:
    """``Block._make_attention_mask`` (models/swin_helpers.py:322-397, one GPU,
    causal=False) on the host: the additive fp32 mask [nW, T*wa, T*wa].

    With a shift, the reference labels the image rows with the slices
    ``[0:-ws0] = 0`` then ``[-s0:] = 1`` (:353-356) and blocks (-100) the
    query/key pairs of a window whose rows carry different labels (:371-378);
    the temporal part is 0 and a token's label does not depend on its frame.
    Without a shift the mask is 0."""
    a, b = window_size
    wa = a * b
    nhb, nwb = H // a, W // b
    L = T * wa
    if not any(shift_size):
        return torch.zeros(nhb * nwb, L, L)
    rows = torch.zeros(H)
    rows[0:H - a] = 0.0
    rows[-int(shift_size[0]):] = 1.0
    band = torch.arange(nhb * nwb) // nwb                          # window -> band i
    r = (torch.arange(L) % wa) // b                                # token -> row in the window
    lab = rows[band[:, None] * a + r[None, :]]                     # [nW, L]
    return torch.where(lab[:, :, None] != lab[:, None, :], torch.tensor(-100.0), torch.tensor(0.0))


def _eps_of(norm: NormLayer, dtype: torch.dtype) -> float:
    e = norm.norm.eps
    return float(torch.finfo(dtype).eps) if e is None else float(e)


class WindowMultiHeadAttention(nn.Module):
    """models/swin_helpers.py:80-256 (parameter names :117-201)."""

    def __init__(self, dim: int, num_heads: int, window_size: Tuple[int, int]) -> None:
        super().__init__()
        assert dim % num_heads == 0, \
            "The number of input features (dim) are not divisible by the number of heads (num_heads)."
        self.dim = dim
        self.window_size = window_size
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.scale = self.head_dim ** -0.5
        self.num_heads_local = num_heads
        meta_col = {"sharded": ["tp", None], "shared": ["sp1-sp2"], "reduce": ["sp1-sp2"]}
        meta_bias = {"sharded": ["tp"], "shared": ["sp1-sp2"], "reduce": ["sp1-sp2"]}
        qk_meta = {"sharded": [None], "shared": ["tp-sp1-sp2"], "reduce": ["tp-sp1-sp2"]}
        self.q = LinearLayer(dim, dim, comm_metadata=meta_col)
        self.biasq = BiasLayer(dim, comm_metadata=meta_bias)
        self.k = LinearLayer(dim, dim, comm_metadata=meta_col)
        self.biask = BiasLayer(dim, comm_metadata=meta_bias)
        self.q_norm = NormLayer(self.head_dim, norm_type="rms_norm", comm_metadata=qk_meta)
        self.k_norm = NormLayer(self.head_dim, norm_type="rms_norm", comm_metadata=qk_meta)
        self.v = LinearLayer(dim, dim, comm_metadata=meta_col)
        self.biasv = BiasLayer(dim, comm_metadata=meta_bias)
        self.proj = LinearLayer(dim, dim, comm_metadata={"sharded": [None, "tp"], "shared": ["sp1-sp2"],
                                                         "reduce": ["sp1-sp2"]})
        self.biasproj = BiasLayer(dim, comm_metadata={"sharded": [], "shared": ["tp-sp1-sp2"],
                                                      "reduce": ["sp1-sp2"]})
        self._pack_key = None
        self._pack = None

    def packed_qkv(self):
        """[Wq;Wk;Wv] and [bq;bk;bv], rebuilt when a parameter changes (not
        cached while torch.compile traces: the cache key reads data_ptr)."""
        ps = (self.q.weight, self.k.weight, self.v.weight, self.biasq.bias, self.biask.bias, self.biasv.bias)
        if torch.compiler.is_compiling():
            return (torch.cat([p.detach() for p in ps[:3]], 0).contiguous(),
                    torch.cat([p.detach() for p in ps[3:]], 0).contiguous())
        key = tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in ps)
        if key != self._pack_key:
            with torch.no_grad():
                w = torch.cat([p.detach() for p in ps[:3]], 0).contiguous()
                b = torch.cat([p.detach() for p in ps[3:]], 0).contiguous()
            self._pack = (w, b)
            self._pack_key = key
        return self._pack

    def qk_norm_weights(self, dtype, device):
        out = []
        for n in (self.q_norm, self.k_norm):
            w = n.norm.weight
            out.append(torch.ones(self.head_dim, dtype=dtype, device=device) if w is None else w.detach())
        return out

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None,
                geometry=None) -> torch.Tensor:
        """x [Bw, L, C]; mask [nW, L, L] additive or None.  ``geometry`` =
        (H, W, window_size, shift_size, T) lets the kernel compute the shift
        mask from indices instead of reading a mask tensor."""
        Bw, L, C = x.shape
        wqkv, bqkv = self.packed_qkv()
        qn, kn = self.qk_norm_weights(x.dtype, x.device)
        eps = _eps_of(self.q_norm, x.dtype)
        if eps != _eps_of(self.k_norm, x.dtype):
            raise NotImplementedError("q_norm and k_norm must share eps")
        qkv = torch.ops.nsw.qkv_projection(x, wqkv, bqkv, qn, kn, self.num_heads, float(eps))
        geo = []
        if mask is None and geometry is not None:
            H, W, ws, sh, T = geometry
            geo = [int(H), int(W), int(ws[0]), int(ws[1]), int(sh[0]), int(sh[1]), int(T)]
        o = torch.ops.nsw.window_attention(qkv, self.num_heads, float(self.scale), mask, geo)
        return torch_ops.linear_epi(o, self.proj.weight, self.biasproj.bias)


class Block(nn.Module):
    """models/swin_helpers.py:259-459 (pre-norm residual window attention +
    pre-norm residual MLP)."""

    def __init__(self, dim, num_heads, feat_size, window_size, temporal_context_window_size,
                 shift_size=(0, 0), mlp_ratio=4.0, drop=0.0, act_layer=nn.GELU, sp1_shapes=None,
                 sp2_shapes=None):
        super().__init__()
        mlp_hidden_dim = int(dim * mlp_ratio)
        self.sp1_shapes = sp1_shapes if sp1_shapes is not None else [feat_size[0]]
        self.sp2_shapes = sp2_shapes if sp2_shapes is not None else [feat_size[1]]
        if len(self.sp1_shapes) != 1 or len(self.sp2_shapes) != 1:
            raise NotImplementedError("libnsw runs the single-GPU (unsharded) block")
        self.feat_size = tuple(feat_size)
        self.window_size = tuple(window_size)
        self.window_area = self.window_size[0] * self.window_size[1]
        self.temporal_context_window_size = temporal_context_window_size
        self.shift_size = tuple(shift_size)
        self.num_heads = num_heads
        norm_meta = {"sharded": [None], "shared": ["tp-sp1-sp2"], "reduce": ["sp1-sp2"]}
        self.norm1 = NormLayer(dim, norm_type="rms_norm", comm_metadata=norm_meta)
        self.attn = WindowMultiHeadAttention(dim, num_heads=num_heads, window_size=window_size)
        self.norm2 = NormLayer(dim, norm_type="rms_norm", comm_metadata=norm_meta)
        self.mlp = MLP(in_features=dim, hidden_features=mlp_hidden_dim, act_layer=act_layer, drop=drop)
        H, W = self.feat_size
        if H % self.window_size[0] or W % self.window_size[1]:
            raise ValueError(f"feat_size {self.feat_size} is not divisible by window {self.window_size}")
        # the reference registers the additive mask as a non-persistent buffer
        # at construction (models/swin_helpers.py:320,397); Block.forward never
        # reads it (the attention kernel evaluates the same closed form)
        self.register_buffer("attn_mask", attention_mask_closed_form(
            H, W, self.window_size, self.shift_size, temporal_context_window_size), persistent=False)
        self._pack_key = None
        self._pack = None
        # fold_norm2 (default): fc1 applies norm2 as a row scale (norm2's
        # weight folded into W1) from row sums of squares written by the
        # proj GEMM (no norm2 pass; 6 launches).  fold_norm1 as well: the
        # block runs as a one-block window-order chain -- a partition pass
        # that also writes the norm1 row sums, the QKV GEMM with norm1 as a
        # row scale, h1 kept in window order, fc2 scattering to tokens (6
        # launches, the same time at config 2).  fold_norm1 implies
        # fold_norm2 (the chain needs both folded weights).
        self.fold_norm1 = False
        self.fold_norm2 = True

    def attention_mask(self, device) -> torch.Tensor:
        """The additive mask on ``device`` as fp32 (the buffer's values)."""
        return self.attn_mask.to(device=device, dtype=torch.float32)

    def _eps(self, dtype) -> float:
        es = {_eps_of(n, dtype) for n in (self.norm1, self.norm2, self.attn.q_norm, self.attn.k_norm)}
        if len(es) != 1:
            raise NotImplementedError("the fused block needs one eps for all four RMSNorms")
        return es.pop()

    def packed(self, fold_all: bool = False):
        """Tensors named like the fields of nsw_block_params.  The norm-folded
        weights are included as fold_norm1 / fold_norm2 ask, or both when
        ``fold_all`` (the window-order chain of SwinTransformer.forward)."""
        a = self.attn
        fold1 = self.fold_norm1 or fold_all
        fold2 = self.fold_norm2 or fold1
        if torch.compiler.is_compiling():
            # traced: built from the parameters each call (the cache key reads data_ptr)
            return self._build_pack(fold1, fold2)
        ps = [self.norm1.norm.weight, a.q.weight, a.k.weight, a.v.weight, a.biasq.bias, a.biask.bias,
              a.biasv.bias, a.q_norm.norm.weight, a.k_norm.norm.weight, a.proj.weight, a.biasproj.bias,
              self.norm2.norm.weight, self.mlp.fc1.weight, self.mlp.bias1.bias, self.mlp.fc2.weight,
              self.mlp.bias2.bias]
        key = tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in ps)
        if key != self._pack_key:
            self._pack = self._build_pack(False, False)
            self._pack_key = key
        pk = self._pack
        with torch.no_grad():
            if fold1 and "wqkv_n1" not in pk:
                pk["wqkv_n1"] = self._fold(pk["wqkv"], pk["norm1_w"])
            if fold2 and "w1_n2" not in pk:
                pk["w1_n2"] = self._fold(pk["w1"], pk["norm2_w"])
        return self._pack

    @staticmethod
    def _fold(w: torch.Tensor, norm_w: torch.Tensor) -> torch.Tensor:
        """Norm weight folded into the GEMM weight that consumes the normalised
        rows: RMSNorm(x) . W^T = rs(x) * (x . (W * norm_w)^T), per input column."""
        return (w.float() * norm_w.float()[None, :]).to(w.dtype).contiguous()

    def _build_pack(self, fold1: bool, fold2: bool) -> dict:
        a = self.attn
        wqkv, bqkv = a.packed_qkv()
        d = lambda t: t.detach().contiguous()
        pk = {
            "norm1_w": d(self.norm1.norm.weight), "wqkv": wqkv, "bqkv": bqkv,
            "qn_w": d(a.q_norm.norm.weight), "kn_w": d(a.k_norm.norm.weight),
            "wproj": d(a.proj.weight), "bproj": d(a.biasproj.bias),
            "norm2_w": d(self.norm2.norm.weight), "w1": d(self.mlp.fc1.weight),
            "b1": d(self.mlp.bias1.bias), "w2": d(self.mlp.fc2.weight), "b2": d(self.mlp.bias2.bias),
        }
        if fold1:
            pk["wqkv_n1"] = self._fold(pk["wqkv"], pk["norm1_w"])
        if fold2:
            pk["w1_n2"] = self._fold(pk["w1"], pk["norm2_w"])
        return pk

    def check_input(self, x: torch.Tensor) -> None:
        if x.dim() != 5 or tuple(x.shape[2:4]) != self.feat_size:
            raise ValueError(f"expected [B, T, {self.feat_size[0]}, {self.feat_size[1]}, C], got {tuple(x.shape)}")
        if x.shape[1] != self.temporal_context_window_size:
            raise ValueError("temporal dim does not match temporal_context_window_size")
        self.mlp._check_fusable()

    @profile(name="shifted_wmha")
    def _shifted_window_attn(self, x: torch.Tensor) -> torch.Tensor:
        """models/swin_helpers.py:399-433 on an already-normalised x."""
        B, T, H, W, C = x.shape
        ws, sh = [int(v) for v in self.window_size], [int(v) for v in self.shift_size]
        xw = torch.ops.nsw.roll_window_partition(x, ws, sh)
        xw = xw.view(-1, T * self.window_area, C)
        o = self.attn(xw, geometry=(H, W, self.window_size, self.shift_size, T))
        return torch.ops.nsw.window_reverse_roll(o.view(-1, T, self.window_size[0], self.window_size[1], C),
                                                 ws, [H, W], sh)

    def forward(self, x: torch.Tensor, condition: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x [B, T, H, W, C] -> [B, T, H, W, C] (models/swin_helpers.py:435-459)."""
        self.check_input(x)
        pk = self.packed()
        drop = ([] if self.fold_norm1 else ["wqkv_n1"]) + ([] if self.fold_norm2 or self.fold_norm1 else ["w1_n2"])
        if drop:
            pk = {k: v for k, v in pk.items() if k not in drop}
        return torch.ops.nsw.swin_block(x, torch_ops.block_param_list(pk), self.num_heads,
                                        [int(v) for v in self.window_size], [int(v) for v in self.shift_size],
                                        self._eps(x.dtype), self.mlp.gelu_tanh)


# Names used by north_star / other Swin code bases.
SwinTransformerBlock = Block
WindowAttention = WindowMultiHeadAttention
