"""SwinTransformer and its patch-embedding layers (models/swin.py:44-323,
models/layer_helpers.py:120-172), with the reference's constructor
signatures, attribute names and state-dict keys, running libnsw kernels.

Forward path on the GPU (models/swin.py:301-323):
  prepare_tokens  patch matrix of the input (nsw_patch_im2col) -> one GEMM
                  with the conv bias and the positional embedding fused in its
                  epilogue (bias + residual) -> tokens [B, T, h, w, E];
                  the coordinate embedding is the same patch GEMM over the
                  constant coordinate fields, computed once and cached until
                  its weights change.
  blocks          nsw.Block (the fused shifted-window block).
  forward_head    GEMM E -> C_out*p*p (no bias) with the head layout in its
                  write-out (nsw_head_unpatchify).  forward()
                  applies the head to the last frame only, which equals the
                  reference's all-frame head followed by ``x[:, -1:]`` because
                  the head is per token.
  big skip        with ``use_big_skip_conv=True`` (off by default and in every
                  configuration of the reference's experiments), the 1x1
                  convolution of the input's predicted frame added to the
                  head's image in place (nsw_skip_conv_accumulate).
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from . import ops, torch_ops
from .layer_helpers import LinearLayer, trunc_normal_
from .profiler_utils import profile
from .swin_helpers import Block as BlockDefault

_EMBED_META = {"sharded": [], "shared": ["tp-sp1-sp2"], "reduce": ["sp1-sp2"]}


class Conv2DLayer(nn.Module):
    """``Conv2DLayer`` (models/layer_helpers.py:152-172): holds ``conv`` (an
    nn.Conv2d, for the parameter names and init).  The forward runs the
    non-overlapping case the model uses (stride = kernel size, no padding,
    dilation or groups) as a patch-matrix GEMM: ``nsw_patch_im2col`` then
    ``nsw_linear`` with the conv bias in the epilogue.  Other convolutions
    are not on the Swin path and raise."""

    def __init__(self, in_chans, out_chans, kernel_size, stride=1, bias=True, comm_metadata=None):
        super().__init__()
        self.conv = nn.Conv2d(in_chans, out_chans, kernel_size=kernel_size, stride=stride, bias=bias)
        meta = comm_metadata or dict(_EMBED_META)
        self.conv.weight.comm_metadata = meta
        if bias:
            self.conv.bias.comm_metadata = meta
        self._pack_key = None
        self._pack = None

    @property
    def patch(self) -> int:
        c = self.conv
        k, st = tuple(c.kernel_size), tuple(c.stride)
        if (k[0] != k[1] or st != k or tuple(c.padding) != (0, 0) or tuple(c.dilation) != (1, 1)
                or c.groups != 1 or c.padding_mode != "zeros"):
            raise NotImplementedError("libnsw runs the non-overlapping patch convolution (stride = square "
                                      f"kernel, no padding / dilation / groups); got kernel {k}, stride {st}")
        return k[0]

    def packed(self):
        """Weight as a [E, Kp] GEMM operand (rows of the Conv2d weight in
        (c, u, v) order, zero columns up to the GEMM k granularity), cached
        until the parameters change."""
        w, b = self.conv.weight, self.conv.bias
        if torch.compiler.is_compiling():     # traced: built each call (the cache key reads data_ptr)
            return self._build_pack()
        key = (w.data_ptr(), w._version, w.dtype, w.device,
               None if b is None else (b.data_ptr(), b._version))
        if self._pack_key != key:
            with torch.no_grad():
                self._pack = self._build_pack()
            self._pack_key = key
        return self._pack

    def _build_pack(self):
        w, b = self.conv.weight, self.conv.bias
        E = w.shape[0]
        K = w[0].numel()
        g = ops.k_granule(w.dtype)
        Kp = (K + g - 1) // g * g
        wp = torch.nn.functional.pad(w.detach().reshape(E, K), (0, Kp - K)).contiguous()
        return wp, None if b is None else b.detach().contiguous(), Kp

    def tokens(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None,
               invariants: Optional[torch.Tensor] = None, frame0: int = 0) -> torch.Tensor:
        """[B, T, C, H, W] (p | H, p | W) -> conv output in token layout
        [B, T, H/p, W/p, E], plus ``residual`` [B*T*(H/p)*(W/p), E] if given."""
        B, T, C, H, W = x.shape
        p = self.patch
        wp, b, Kp = self.packed()
        pm = torch.ops.nsw.patch_im2col(x, p, Kp, wp.dtype, invariants, int(frame0))
        if b is None:
            if residual is not None:
                raise NotImplementedError("a residual without a conv bias is not fused")
            y = torch_ops.linear_epi(pm, wp)
        else:
            y = torch_ops.linear_epi(pm, wp, b, residual=residual)
        return y.view(B, T, H // p, W // p, wp.shape[0])

    def tokens_windowed(self, x: torch.Tensor, residual: torch.Tensor, window_size, shift_size,
                        invariants: Optional[torch.Tensor] = None, frame0: int = 0):
        """tokens() with the rows stored straight in the window order of the
        token image rolled by -shift (the first block's order), together with
        their partial sums of squares: (y [B, T, H/p, W/p, E] holding the
        window-ordered rows, row_sumsq [rows, P] fp32)."""
        B, T, C, H, W = x.shape
        p = self.patch
        wp, b, Kp = self.packed()
        if b is None:
            raise NotImplementedError("the window-order embedding fuses the conv bias and a residual")
        pm = torch.ops.nsw.patch_im2col(x, p, Kp, wp.dtype, invariants, int(frame0))
        y, ss = torch.ops.nsw.linear_to_window(pm, wp, b, residual, [B, T, H // p, W // p],
                                               [int(v) for v in window_size], [int(v) for v in shift_size])
        return y.view(B, T, H // p, W // p, wp.shape[0]), ss

    def forward(self, x):
        """Conv2d semantics: [N, C, H, W] -> [N, E, H // p, W // p] (rows and
        columns beyond the last whole patch are ignored, as Conv2d does)."""
        p = self.patch
        N, C, H, W = x.shape
        h, w = H // p, W // p
        if (H, W) != (h * p, w * p):
            x = x[:, :, :h * p, :w * p]
        return self.tokens(x.unsqueeze(1))[:, 0].permute(0, 3, 1, 2).contiguous()


class PatchEmbedLayer(nn.Module):
    """``PatchEmbedLayer`` (models/layer_helpers.py:120-150): Conv2d with
    kernel = stride = patch_size as a patch-matrix GEMM."""

    def __init__(self, patch_size=16, in_chans=3, embed_dim=768, sp1_shapes=None, sp2_shapes=None,
                 comm_metadata=None):
        super().__init__()
        if sp1_shapes is None or sp2_shapes is None:
            raise ValueError("PatchEmbedLayer needs the image extent (sp1_shapes=[H], sp2_shapes=[W])")
        if len(sp1_shapes) != 1 or len(sp2_shapes) != 1:
            raise NotImplementedError("libnsw runs the single-GPU (unsharded) model")
        self.proj = Conv2DLayer(in_chans, embed_dim, kernel_size=patch_size, stride=patch_size,
                                comm_metadata=comm_metadata)
        self.patch_size = patch_size
        self.in_chans = in_chans
        self.embed_dim = embed_dim
        self.sp1_patch_shapes = [s // patch_size for s in sp1_shapes]
        self.h = self.sp1_patch_shapes[0]
        self.sp2_patch_shapes = [s // patch_size for s in sp2_shapes]
        self.w = self.sp2_patch_shapes[0]
        self.num_patches = self.h * self.w

    def packed(self):
        return self.proj.packed()

    def tokens(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None,
               invariants: Optional[torch.Tensor] = None, frame0: int = 0) -> torch.Tensor:
        """[B, T, C, H, W] -> conv output in token layout [B, T, h, w, E],
        plus ``residual`` [B*T*h*w, E] if given."""
        B, T, C, H, W = x.shape
        p = self.patch_size
        if H != self.h * p or W != self.w * p:
            raise ValueError(f"input extent {(H, W)} does not match the layer's {(self.h * p, self.w * p)}")
        return self.proj.tokens(x, residual=residual, invariants=invariants, frame0=frame0)

    def tokens_windowed(self, x: torch.Tensor, residual: torch.Tensor, window_size, shift_size,
                        invariants: Optional[torch.Tensor] = None, frame0: int = 0):
        """tokens() stored in the window order of the first block, with the rows'
        partial sums of squares (Conv2DLayer.tokens_windowed)."""
        B, T, C, H, W = x.shape
        p = self.patch_size
        if H != self.h * p or W != self.w * p:
            raise ValueError(f"input extent {(H, W)} does not match the layer's {(self.h * p, self.w * p)}")
        return self.proj.tokens_windowed(x, residual, window_size, shift_size, invariants=invariants,
                                         frame0=frame0)

    def forward(self, x):
        """Conv2d semantics: [N, C, H, W] -> [N, E, H/p, W/p]."""
        return self.proj(x)


class SwinTransformer(nn.Module):
    """``SwinTransformer`` (models/swin.py:44-323) for one GPU."""

    @classmethod
    def instantiate_from_cfg(cls, cfg, domain_metadata):
        """models/swin.py:61-85 (cfg with attribute access: cfg.model.*,
        cfg.train.temporal_context_window, cfg.data.invariants,
        cfg.parallelism.use_transformer_engine)."""
        ws = cfg.model.window_size
        window_size = tuple(ws) if isinstance(ws, (list, tuple)) else (ws, ws)
        invariants = getattr(cfg.data, "invariants", None)
        extra_inputs = len(invariants) if invariants else 0
        return cls(
            patch_size=cfg.model.patch_size,
            window_size=window_size,
            depth=cfg.model.depth,
            num_heads=cfg.model.num_heads,
            temporal_context_window_size=cfg.train.temporal_context_window,
            in_chans=domain_metadata["n_channels"] + extra_inputs,
            out_chans=domain_metadata["n_channels"],
            embed_dim=cfg.model.embed_dim,
            mlp_ratio=cfg.model.mlp_ratio,
            drop_rate=cfg.model.dropout,
            coord_pos_embed=getattr(cfg.model, "coord_pos_embed", True),
            use_transformer_engine=getattr(getattr(cfg, "parallelism", None), "use_transformer_engine", True),
            domain_metadata=domain_metadata,
        )

    def __init__(self, temporal_context_window_size=1, window_size=(9, 9), patch_size=16, in_chans=3,
                 out_chans=3, embed_dim=768, depth=12, num_heads=12, mlp_ratio=4.0, drop_rate=0.0,
                 coord_pos_embed=True, domain_metadata=None, use_transformer_engine=True,
                 use_big_skip_conv=False, **kwargs):
        super().__init__()
        if domain_metadata is None:
            raise ValueError("data loader must provide domain metadata")
        self.num_features = self.embed_dim = embed_dim
        self.patch_size = patch_size
        self.temporal_context_window_size = temporal_context_window_size
        self.window_size = tuple(window_size)
        self.in_chans = in_chans
        self.out_chans = out_chans
        self.drop_rate = drop_rate
        self.coord_pos_embed = coord_pos_embed
        self.domain_metadata = domain_metadata
        self.use_transformer_engine = use_transformer_engine
        self.use_big_skip_conv = use_big_skip_conv
        sp1, sp2 = domain_metadata["sp_shapes"]

        self.patch_embed = PatchEmbedLayer(patch_size=patch_size, in_chans=in_chans, embed_dim=embed_dim,
                                           sp1_shapes=sp1, sp2_shapes=sp2, comm_metadata=dict(_EMBED_META))
        if coord_pos_embed:
            self._init_coords()
            self.pos_embed = PatchEmbedLayer(patch_size=patch_size, in_chans=self.coords.shape[-1],
                                             embed_dim=embed_dim, sp1_shapes=sp1, sp2_shapes=sp2,
                                             comm_metadata=dict(_EMBED_META))
        else:
            self.pos_embed = nn.Parameter(torch.zeros(1, temporal_context_window_size, self.patch_embed.h,
                                                      self.patch_embed.w, embed_dim))
            trunc_normal_(self.pos_embed, std=0.02)
            self.pos_embed.comm_metadata = {"sharded": [None, None, "sp1", "sp2", None], "shared": ["tp"],
                                            "reduce": []}

        self.blocks = nn.ModuleList([
            BlockDefault(dim=embed_dim, num_heads=num_heads, feat_size=(self.patch_embed.h, self.patch_embed.w),
                         window_size=self.window_size, temporal_context_window_size=temporal_context_window_size,
                         shift_size=tuple(0 if (i % 2) == 0 else w // 2 for w in self.window_size),
                         mlp_ratio=mlp_ratio, drop=drop_rate, sp1_shapes=self.patch_embed.sp1_patch_shapes,
                         sp2_shapes=self.patch_embed.sp2_patch_shapes)
            for i in range(depth)])
        self.out_size = out_chans * patch_size * patch_size
        self.head = LinearLayer(embed_dim, self.out_size, comm_metadata=dict(_EMBED_META))
        # modulate the skip with a conv (models/swin.py:211-223): added to
        # the head's image in forward by nsw_skip_conv_accumulate
        if use_big_skip_conv:
            self.skip_conv = Conv2DLayer(in_chans, out_chans, kernel_size=1, bias=False,
                                         comm_metadata=dict(_EMBED_META))
        self.apply(self._init_weights)
        # chain_blocks: run the blocks loop as one C-ABI call that keeps the
        # residual stream in window order between blocks (each block's fc2
        # stores its rows in the next block's window order with their norm1
        # statistics: no per-block gather / scatter / norm passes, 1 + 5 *
        # depth launches).  False: one fused call per block.
        self.chain_blocks = True
        self._pos_key = None
        self._pos = None
        self._head_key = None
        self._head_w = None

    def _init_coords(self):
        """models/swin.py:227-244: coords [T, H, W, 4] = spatial (x, y, z) with
        t = linspace(0, 1, T) appended (non-persistent buffer)."""
        T = self.temporal_context_window_size
        spatial = torch.as_tensor(self.domain_metadata["coords"]).float()
        H, W, _ = spatial.shape
        t = torch.linspace(0, 1, T).view(T, 1, 1, 1).expand(-1, H, W, 1)
        coords = torch.cat([spatial.unsqueeze(0).expand(T, -1, -1, -1), t], dim=-1)
        self.register_buffer("coords", coords, persistent=False)

    def _init_weights(self, m):
        """models/swin.py:246-267."""
        if isinstance(m, (nn.Linear, nn.Conv2d)):
            trunc_normal_(m.weight, std=0.02)
            if m.bias is not None:
                nn.init.constant_(m.bias, 0)
        elif isinstance(m, nn.LayerNorm):
            nn.init.constant_(m.bias, 0)
            nn.init.constant_(m.weight, 1.0)
        elif isinstance(m, nn.RMSNorm):
            nn.init.constant_(m.weight, 1.0)

    # ------------------------------------------------------------ embedding --
    def _pos_tokens(self, B: int, dtype: torch.dtype, device) -> torch.Tensor:
        """Positional embedding in token layout, repeated over the batch:
        [B*T*h*w, E] (the GEMM epilogue's residual operand); cached until the
        parameters change, rebuilt each call while torch.compile traces."""
        if torch.compiler.is_compiling():
            return self._build_pos(B, dtype, device)
        if self.coord_pos_embed:
            w, b = self.pos_embed.proj.conv.weight, self.pos_embed.proj.conv.bias
            key = ("coord", w.data_ptr(), w._version, b.data_ptr(), b._version, self.coords.data_ptr(),
                   self.coords._version, dtype, torch.device(device), B)
        else:
            key = ("param", self.pos_embed.data_ptr(), self.pos_embed._version, dtype, torch.device(device), B)
        if self._pos_key != key:
            with torch.no_grad():
                self._pos = self._build_pos(B, dtype, device)
            self._pos_key = key
        return self._pos

    def _build_pos(self, B: int, dtype: torch.dtype, device) -> torch.Tensor:
        if self.coord_pos_embed:
            c = self.coords.to(device=device, dtype=self.pos_embed.proj.conv.weight.dtype)
            c = c.permute(0, 3, 1, 2).contiguous().unsqueeze(0)       # [1, T, 4, H, W]
            pos = self.pos_embed.tokens(c)                             # [1, T, h, w, E]
        else:
            pos = self.pos_embed.detach()
        pos = pos.to(device=device, dtype=dtype).expand(B, -1, -1, -1, -1)
        return pos.reshape(-1, self.embed_dim).contiguous()

    @profile("embed")
    def prepare_tokens(self, x: torch.Tensor, invariants: Optional[torch.Tensor] = None,
                       frame0: int = 0) -> torch.Tensor:
        """models/swin.py:269-284: [B, T, C, H, W] -> [B, T, h, w, E]."""
        w = self.patch_embed.proj.conv.weight
        pos = self._pos_tokens(x.shape[0], w.dtype, w.device)
        return self.patch_embed.tokens(x, residual=pos, invariants=invariants, frame0=frame0)

    # ----------------------------------------------------------------- head --
    def _head_weight(self) -> torch.Tensor:
        """head.weight with its rows in the order of the fused head
        (ops.head_weight_perm), cached until the weight changes; rebuilt each
        call while torch.compile traces."""
        W = self.head.weight
        if torch.compiler.is_compiling():
            return ops.head_weight_perm(W.detach(), self.out_chans, self.patch_size)
        key = (W.data_ptr(), W._version, W.dtype, W.device)
        if self._head_key != key:
            with torch.no_grad():
                self._head_w = ops.head_weight_perm(W.detach(), self.out_chans, self.patch_size)
            self._head_key = key
        return self._head_w

    @profile("head")
    def forward_head(self, x: torch.Tensor) -> torch.Tensor:
        """models/swin.py:286-299: [B, T, h, w, E] -> [B, T, C_out, H, W]: the
        head GEMM with the reshape + einsum layout in its write-out."""
        b, t, h, w, c = x.shape
        p = self.patch_size
        out = torch.ops.nsw.head_unpatchify(x.reshape(-1, c), self._head_weight(), b * t, self.out_chans, h * p,
                                            w * p, p, None)
        return out.view(b, t, self.out_chans, h * p, w * p)

    def _head_last(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Head of the last frame only: [B, T, h, w, E] -> [B, 1, C_out, H, W]
        (into ``out`` when given, in out's dtype: the fused head writes bf16
        or float32 images, other dtypes go through a bf16/f32 result)."""
        b, t, h, w, c = x.shape
        p = self.patch_size
        Wp = self._head_weight()
        H, W = h * p, w * p
        if out is None:
            return torch.ops.nsw.head_unpatchify(x[:, t - 1].reshape(b * h * w, c), Wp, b, self.out_chans, H, W, p,
                                                 None)
        if out.dtype not in (x.dtype, torch.float32):
            out.copy_(self._head_last(x))
            return out
        for bi in range(b):
            ops.head_unpatchify(x[bi, t - 1].view(h * w, c), Wp, 1, self.out_chans, H, W, p, out=out[bi:bi + 1])
        return out

    # -------------------------------------------------------------- forward --
    @profile("forward")
    def forward(self, x: torch.Tensor, invariants: Optional[torch.Tensor] = None, frame0: int = 0,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """models/swin.py:301-323: [B, T, C_in, H, W] -> [B, 1, C_out, H, W].

        Beyond the reference's signature (all optional): ``invariants``
        [C_inv, H, W] are appended as input channels inside the patch gather,
        frame t is read from slot (t + frame0) mod T of x, and ``out`` receives
        the prediction (any float dtype; e.g. a slot of the input ring)."""
        if self._embed_into_chain():
            # the embedding GEMM stores its rows in block 0's window order with
            # their norm1 statistics, the chain's own first pass
            b0 = self.blocks[0]
            w = self.patch_embed.proj.conv.weight
            pos = self._pos_tokens(x.shape[0], w.dtype, w.device)
            yw, ss = self.patch_embed.tokens_windowed(x, pos, b0.window_size, b0.shift_size, invariants=invariants,
                                                      frame0=frame0)
            params, shifts, eps, tanh = self._chain_args(yw)
            y = torch.ops.nsw.swin_blocks_windowed(yw, ss, params, b0.num_heads, [int(v) for v in b0.window_size],
                                                   shifts, eps, tanh)
        else:
            y = self.prepare_tokens(x, invariants=invariants, frame0=frame0)
            y = self.forward_blocks(y)
        res = self._head_last(y, out=out)
        if self.use_big_skip_conv:
            # x + skip_conv(x) of models/swin.py:310-317, on the frame returned
            torch.ops.nsw.skip_conv_accumulate(x, self.skip_conv.conv.weight, res, invariants, int(frame0))
        return res

    def _embed_into_chain(self) -> bool:
        """The embedding writes the chain's window-ordered input when the blocks
        run as the chain and the patch convolution has the bias that the
        fused write-out needs."""
        return (self.chain_blocks and len(self.blocks) > 0 and self.patch_embed.proj.conv.bias is not None)

    def _chain_args(self, y: torch.Tensor):
        """(params, shifts, eps, gelu_tanh) of the blocks as one chain."""
        for blk in self.blocks:
            blk.check_input(y)
        eps = {blk._eps(y.dtype) for blk in self.blocks}
        tanh = {blk.mlp.gelu_tanh for blk in self.blocks}
        if len(eps) != 1 or len(tanh) != 1:
            raise NotImplementedError("the block chain needs one eps and one GELU form for all blocks")
        params, shifts = [], []
        for blk in self.blocks:
            params += torch_ops.block_param_list(blk.packed(fold_all=True))
            shifts += [int(blk.shift_size[0]), int(blk.shift_size[1])]
        return params, shifts, eps.pop(), tanh.pop()

    def forward_blocks(self, y: torch.Tensor) -> torch.Tensor:
        """``for blk in self.blocks: y = blk(y)`` (models/swin.py:307-308),
        through the window-order chain when ``chain_blocks`` is set."""
        if not self.chain_blocks or len(self.blocks) == 0:
            for blk in self.blocks:
                y = blk(y)
            return y
        b0 = self.blocks[0]
        params, shifts, eps, tanh = self._chain_args(y)
        return torch.ops.nsw.swin_blocks(y, params, b0.num_heads, [int(v) for v in b0.window_size], shifts, eps,
                                         tanh)


class TimeStepper(nn.Module):
    """``TimeStepper`` (models/helpers.py:9-37): autoregressive steps with the
    invariant channels re-appended to every prediction."""

    def __init__(self, cfg, model_handle):
        super().__init__()
        self.model = model_handle
        self.num_rollout_steps = cfg.train.num_rollout_steps
        invariants = getattr(cfg.data, "invariants", None)
        self.num_invariants = len(invariants) if invariants else 0

    def forward(self, inp):
        result = []
        inpt = inp
        c_in = inp.shape[2]
        for step in range(self.num_rollout_steps):
            pred = self.model(inpt)
            c_out = pred.shape[2]
            result.append(pred)
            n_invariants = c_in - c_out
            assert n_invariants == self.num_invariants, "number of invariants does not match"
            if n_invariants > 0:
                inpt = torch.cat([pred.to(inp.dtype), inp[:, :, c_in - n_invariants:]], dim=2)
            else:
                inpt = pred
        return torch.cat(result, dim=1)


def get_model(cfg, domain_metadata=None):
    """models/helpers.py:40-50."""
    if cfg.model.arch != "swin":
        raise NotImplementedError(f"model type {cfg.model.arch} not implemented")
    return TimeStepper(cfg, SwinTransformer.instantiate_from_cfg(cfg, domain_metadata=domain_metadata))
