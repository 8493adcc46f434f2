"""GPU parity of the blocks loop of SwinTransformer.forward (models/swin.py:
307-308, ``for blk in self.blocks: x = blk(x)``) run as one window-order
chain (nsw_swin_blocks_forward): the fp32 CPU oracle applies the reference
block (models/swin_helpers.py:435-459) depth times in token order.

Tolerances: fp32 relative L2 <= 1e-5 per block of depth (the block's bar,
north_star's fp32 parity mode); bf16 relative L2 <= 1e-2 of the output
(north_star's bf16 bar, the same as one block) and the chain's error no
more than 1.25x that of depth separate fused block calls on the same
inputs.  The chain equals the separate calls up to rounding (same
arithmetic, norms applied as row scales), checked in fp32 at 2e-6."""
import pytest
import torch

from oracle import swin_ref as ref
from oracle import synth

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return (torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b)).item()


def make_stack(device, dtype, T, H, W, C, heads, ws, shifts, seed):
    import nsw
    blocks, params = [], []
    for i, sh in enumerate(shifts):
        p = synth.block_params(C, heads, seed=100 * seed + i, random_bias=True, random_norm=True)
        p = {k: v.to(dtype).float() for k, v in p.items()}
        blk = nsw.Block(C, heads, (H, W), ws, T, shift_size=sh)
        blk.load_state_dict(p)
        blocks.append(blk.to(device=device, dtype=dtype))
        params.append(p)
    return blocks, params


def run_chain(blocks, x):
    from nsw import ops
    b0 = blocks[0]
    packs = [b.packed(fold_all=True) for b in blocks]
    return ops.swin_blocks_forward(x, packs, b0.num_heads, b0.window_size, [b.shift_size for b in blocks],
                                   eps=b0._eps(x.dtype), gelu_tanh=b0.mlp.gelu_tanh)


def oracle_stack(x, params, heads, ws, shifts, eps, device=None):
    y = x
    for p, sh in zip(params, shifts):
        if device is not None:
            p = {k: v.to(device) for k, v in p.items()}
        y = ref.block_forward(y, p, heads, ws, sh, eps=eps)
    return y


ALT = [(0, 0), (4, 9)]

FP32_CASES = [
    # B, T, H, W, C, heads, ws, shifts
    (1, 1, 90, 180, 192, 6, (9, 18), ALT * 2),
    (2, 1, 18, 36, 128, 2, (9, 18), ALT * 2 + [(0, 0)]),
    (1, 2, 18, 36, 128, 4, (9, 18), [(4, 9), (4, 9), (2, 5), (0, 0)]),   # equal and arbitrary shifts
    (1, 1, 16, 32, 64, 4, (4, 8), [(2, 4)]),                             # depth 1
]


@pytest.mark.parametrize("B,T,H,W,C,heads,ws,shifts", FP32_CASES)
def test_chain_fp32(device, B, T, H, W, C, heads, ws, shifts):
    blocks, params = make_stack(device, torch.float32, T, H, W, C, heads, ws, shifts, seed=B * 7 + T)
    x = synth.activations((B, T, H, W, C), seed=11 * B + T)
    with torch.inference_mode():
        xd = x.to(device)
        y = run_chain(blocks, xd)
        y_sep = xd
        for blk in blocks:
            y_sep = blk(y_sep)
    torch.cuda.synchronize()
    want = oracle_stack(x, params, heads, ws, shifts, torch.finfo(torch.float32).eps)
    assert rel_l2(y, want) < 1e-5 * len(shifts)
    assert rel_l2(y - x.to(device), want - x) < 1e-4 * len(shifts)
    assert rel_l2(y, y_sep) < 2e-6


def test_chain_fp32_production_width(device):
    """fp32 (the reference's inference precision) at config 2's geometry and
    width: 180x360 tokens, C=1024, 16 heads (hd 64), window 9x18, four
    blocks with alternating shift.  The chain of the first d + 1 blocks is
    checked against the oracle block d applied to the chain's own output
    after d blocks (every block within 1e-5, north_star's fp32 bar), and the
    whole stack against the oracle stack; oracle in fp32 on the device."""
    T, H, W, C, heads, ws = 1, 180, 360, 1024, 16, (9, 18)
    shifts = ALT * 2
    eps = torch.finfo(torch.float32).eps
    blocks, params = make_stack(device, torch.float32, T, H, W, C, heads, ws, shifts, seed=6)
    x = synth.activations((1, T, H, W, C), seed=66).to(device)
    errs = []
    with torch.inference_mode():
        prev = x
        for d in range(len(shifts)):
            y = run_chain(blocks[:d + 1], x)
            pd = {k: v.to(device) for k, v in params[d].items()}
            want = ref.block_forward(prev, pd, heads, ws, shifts[d], eps=eps)
            errs.append(rel_l2(y, want))
            prev = y
        want_all = oracle_stack(x, params, heads, ws, shifts, eps, device=device)
        e_all = rel_l2(prev, want_all)
    torch.cuda.synchronize()
    print(f"fp32 chain at C=1024: per block {[f'{e:.2e}' for e in errs]}, stack {e_all:.2e}", flush=True)
    assert max(errs) < 1e-5
    assert e_all < 1e-5 * len(shifts)


def test_chain_bf16_config2(device):
    """Four blocks at config 2's geometry (180x360, C=1024, 16 heads, window
    9x18, alternating shift), bf16; oracle in fp32 on the device."""
    T, H, W, C, heads, ws = 1, 180, 360, 1024, 16, (9, 18)
    shifts = ALT * 2
    blocks, params = make_stack(device, torch.bfloat16, T, H, W, C, heads, ws, shifts, seed=5)
    x = synth.activations((1, T, H, W, C), seed=55).to(torch.bfloat16).float()
    with torch.inference_mode():
        xd = x.to(device, torch.bfloat16)
        y = run_chain(blocks, xd).float()
        y_sep = xd
        for blk in blocks:
            y_sep = blk(y_sep)
        y_sep = y_sep.float()
        want = oracle_stack(x.to(device), params, heads, ws, shifts, torch.finfo(torch.bfloat16).eps,
                            device=device)
    torch.cuda.synchronize()
    e_chain, e_sep = rel_l2(y, want), rel_l2(y_sep, want)
    assert e_chain < 1e-2
    assert e_chain < 1.25 * e_sep


def test_chain_input_untouched_and_repeatable(device):
    """x is read only; two calls give identical results (no state kept in
    the shared workspace between calls)."""
    shifts = ALT * 2
    blocks, _ = make_stack(device, torch.bfloat16, 1, 18, 36, 128, 2, (9, 18), shifts, seed=9)
    x = synth.activations((1, 1, 18, 36, 128), seed=99).to(device, torch.bfloat16)
    x0 = x.clone()
    with torch.inference_mode():
        y1 = run_chain(blocks, x)
        y2 = run_chain(blocks, x)
    torch.cuda.synchronize()
    assert torch.equal(x, x0)
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shift", [(0, 0), (4, 9)])
def test_window_partition_sumsq(device, dtype, shift):
    """Rows equal the fused roll + partition bit for bit; each 512-byte part's
    sum of squares equals the float64 sum of the stored values' squares."""
    from nsw import ops
    B, T, H, W, C, ws = 2, 1, 18, 36, 320, (9, 18)
    x = synth.activations((B, T, H, W, C), seed=3).to(device, dtype)
    with torch.inference_mode():
        xw, ss = ops.window_partition_sumsq(x, ws, shift)
        want_w = ops.roll_window_partition(x, ws, shift)
    torch.cuda.synchronize()
    assert torch.equal(xw, want_w)
    per = 512 // x.element_size()
    rows = xw.reshape(-1, C).double().cpu()
    nparts = -(-C // per)
    assert ss.shape == (rows.shape[0], nparts)
    want = torch.stack([(rows[:, p * per:(p + 1) * per] ** 2).sum(1) for p in range(nparts)], 1)
    torch.testing.assert_close(ss.double().cpu(), want, rtol=2e-6, atol=1e-6)


def test_model_chain_matches_block_calls(device):
    """SwinTransformer.forward with chain_blocks on and off (small model,
    fp32): the same prediction up to rounding."""
    import nsw
    H, W, p, C = 72, 144, 4, 5
    meta = {"coords": torch.randn(H, W, 3), "sp_shapes": [[H], [W]], "n_channels": C}
    torch.manual_seed(4)
    model = nsw.SwinTransformer(window_size=(9, 18), patch_size=p, in_chans=C, out_chans=C, embed_dim=128,
                                depth=4, num_heads=2, domain_metadata=meta).to(device).eval()
    x = torch.randn(1, 1, C, H, W, device=device)
    with torch.inference_mode():
        y_chain = model(x)
        model.chain_blocks = False
        y_sep = model(x)
    torch.cuda.synchronize()
    assert rel_l2(y_chain, y_sep) < 2e-6


def test_chain_argument_errors(device):
    from nsw import ops
    blocks, _ = make_stack(device, torch.float32, 1, 18, 36, 128, 2, (9, 18), ALT, seed=3)
    x = torch.zeros(1, 1, 18, 36, 128, device=device)
    packs = [b.packed(fold_all=True) for b in blocks]
    with pytest.raises(ValueError):
        ops.swin_blocks_forward(x, packs, 2, (9, 18), [(0, 0)])            # one shift for two blocks
    bad = [dict(packs[0]), packs[1]]
    del bad[0]["w1_n2"]
    with pytest.raises(ValueError, match="norm-folded"):
        ops.swin_blocks_forward(x, bad, 2, (9, 18), [(0, 0), (4, 9)])
    with pytest.raises(ValueError, match="alias"):
        ops.swin_blocks_forward(x, packs, 2, (9, 18), [(0, 0), (4, 9)], out=x)


def _partial_sumsq(rows: torch.Tensor, es: int) -> torch.Tensor:
    """float32 [M, P] sums of squares per 512-byte part (float64 sums)."""
    per = 512 // es
    r = rows.double()
    C = r.shape[1]
    return torch.stack([(r[:, p * per:(p + 1) * per] ** 2).sum(1) for p in range(-(-C // per))], 1).float()


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
def test_qkv_projection_rowscale(device, dtype, tol):
    """nsw_qkv_projection_rowscale against the oracle: per-head q/k RMSNorm of
    RMSNorm(x; norm1) . [Wq;Wk;Wv]^T + b (models/swin_helpers.py:446, 212-241),
    the row statistics given as 512-byte partial sums of x's squares."""
    from nsw import ops
    C, heads, M = 256, 4, 1000
    p = synth.block_params(C, heads, seed=61, random_bias=True, random_norm=True)
    p = {k: v.to(dtype).float() for k, v in p.items()}
    x = synth.activations((M, C), seed=62).to(dtype).float()
    eps = torch.finfo(dtype).eps
    wqkv = torch.cat([p["attn.q.weight"], p["attn.k.weight"], p["attn.v.weight"]], 0)
    bqkv = torch.cat([p["attn.biasq.bias"], p["attn.biask.bias"], p["attn.biasv.bias"]], 0)
    n1 = p["norm1.norm.weight"]
    wqkv_n = (wqkv * n1[None, :]).to(dtype)
    ss = _partial_sumsq(x.to(dtype), torch.finfo(dtype).bits // 8)
    d = lambda t: t.to(device, dtype).contiguous()
    with torch.inference_mode():
        got = ops.qkv_projection_rowscale(d(x), d(wqkv_n), d(bqkv), d(p["attn.q_norm.norm.weight"]),
                                          d(p["attn.k_norm.norm.weight"]), ss.to(device), heads, eps)
    torch.cuda.synchronize()
    xn = ref.rms_norm(x, n1, eps)
    lin = xn @ wqkv.T + bqkv
    q, k, v = lin.split(C, dim=1)
    hd = C // heads
    q = ref.rms_norm(q.reshape(M, heads, hd), p["attn.q_norm.norm.weight"], eps).reshape(M, C)
    k = ref.rms_norm(k.reshape(M, heads, hd), p["attn.k_norm.norm.weight"], eps).reshape(M, C)
    want = torch.cat([q, k, v], 1)
    assert rel_l2(got, want) < tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_linear_remap_residual(device, dtype, mode):
    """nsw_linear_remap_residual: rows of x . w^T + b + residual stored at
    the identity (0), the token of each window row (1), that token's row in
    the window order of another shift (2), or, for token-ordered rows, each
    token's row in the window order (3), with the stored rows' partial sums
    of squares for modes 0, 2 and 3 (index maps from oracle/index_maps.py)."""
    from nsw import ops
    from oracle import index_maps
    B, T, H, W, ws, sh, sh2, K, N = 2, 1, 18, 36, (9, 18), (4, 9), (0, 0), 128, 256
    M = B * T * H * W
    g = torch.Generator().manual_seed(71)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (torch.randn(N, K, generator=g) * 0.05).to(dtype)
    b = torch.randn(N, generator=g).to(dtype)
    r = torch.randn(M, N, generator=g).to(dtype)
    with torch.inference_mode():
        y, ss = ops.linear_remap_residual(x.to(device), w.to(device), b.to(device), r.to(device), mode,
                                          image=(B, T, H, W), window_size=ws, shift_size=sh, next_shift=sh2)
    torch.cuda.synchronize()
    rows = x.double() @ w.double().T + b.double() + r.double()
    tok = torch.from_numpy(index_maps.gather_rows(B, T, H, W, ws[0], ws[1], sh[0], sh[1]))
    if mode == 0:
        dest = torch.arange(M)
    elif mode == 3:
        dest = torch.empty(M, dtype=torch.int64)
        dest[tok] = torch.arange(M)                  # token m -> its window row
    else:
        dest = tok
        if mode == 2:
            tok2 = torch.from_numpy(index_maps.gather_rows(B, T, H, W, ws[0], ws[1], sh2[0], sh2[1]))
            row_of_tok = torch.empty(M, dtype=torch.int64)
            row_of_tok[tok2] = torch.arange(M)
            dest = row_of_tok[tok]
    want = torch.empty(M, N, dtype=torch.float64)
    want[dest] = rows
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert rel_l2(y, want) < tol
    if mode == 1:
        assert ss is None
    else:
        es = 4 if dtype == torch.float32 else 2
        torch.testing.assert_close(ss.cpu(), _partial_sumsq(y.cpu(), es), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_chain_from_window_order(device, dtype):
    """nsw_swin_blocks_forward_windowed on block 0's window order and norm1
    sums (as the partition pre-pass writes them) equals the chain from
    token order bit for bit, and leaves its inputs untouched."""
    from nsw import ops
    shifts = [(4, 9), (0, 0), (4, 9)]
    blocks, _ = make_stack(device, dtype, 1, 18, 36, 128, 2, (9, 18), shifts, seed=12)
    x = synth.activations((2, 1, 18, 36, 128), seed=13).to(device, dtype)
    b0 = blocks[0]
    packs = [b.packed(fold_all=True) for b in blocks]
    with torch.inference_mode():
        want = run_chain(blocks, x)
        xw, ss = ops.window_partition_sumsq(x, b0.window_size, b0.shift_size)
        xw, ss0 = xw.reshape(x.shape), ss.clone()
        xw0 = xw.clone()
        got = ops.swin_blocks_forward(xw, packs, b0.num_heads, b0.window_size, shifts, eps=b0._eps(dtype),
                                      gelu_tanh=b0.mlp.gelu_tanh, row_sumsq=ss)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(xw, xw0) and torch.equal(ss, ss0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_embedding_into_window_order(device, dtype):
    """The embedding GEMM's window-order write-out (map mode 3) stores the
    rows the partition pre-pass makes of its token-order output, and their
    sums of squares up to summation order."""
    from nsw import ops, torch_ops
    B, T, H, W, ws, sh, K, N = 1, 1, 18, 36, (9, 18), (0, 0), 128, 256
    M = B * T * H * W
    g = torch.Generator().manual_seed(5)
    x = torch.randn(M, K, generator=g).to(dtype).to(device)
    w = (torch.randn(N, K, generator=g) * 0.05).to(dtype).to(device)
    b = torch.randn(N, generator=g).to(dtype).to(device)
    r = torch.randn(M, N, generator=g).to(dtype).to(device)
    with torch.inference_mode():
        tok = torch_ops.linear_epi(x, w, b, residual=r)
        want_w, want_ss = ops.window_partition_sumsq(tok.view(B, T, H, W, N), ws, sh)
        got_w, got_ss = torch.ops.nsw.linear_to_window(x, w, b, r, [B, T, H, W], list(ws), list(sh))
    torch.cuda.synchronize()
    assert torch.equal(got_w.reshape(-1), want_w.reshape(-1))
    torch.testing.assert_close(got_ss, want_ss, rtol=2e-6, atol=1e-6)
