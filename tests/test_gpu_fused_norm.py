"""GPU parity of the GEMMs with a fused input RMSNorm: the proj scatter that
also writes its rows' partial sums of squares
(nsw_proj_reverse_residual_sumsq) and the linear layer that takes them
(nsw_linear_rowscale), against the fp32 oracle (RMSNorm -> fc1,
models/swin_helpers.py:457 + models/mlp.py:80-85).  Tolerances: fp32
1e-5, bf16 1e-2 relative L2, as for the unfused kernels."""
import pytest
import torch
import torch.nn.functional as F

from oracle import swin_ref as ref, synth

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return (torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b)).item()


def fold(w, nw, dtype):
    return (w.float() * nw.float()[None, :]).to(dtype)


CASES = [
    # B, T, H, W, C, heads, ws, shift
    (1, 1, 180, 360, 1024, 16, (9, 18), (4, 9)),
    (1, 1, 90, 180, 192, 6, (9, 18), (4, 9)),
    (1, 1, 90, 180, 192, 6, (9, 18), (0, 0)),
    (2, 2, 18, 36, 128, 2, (9, 18), (4, 9)),
    (1, 1, 16, 32, 64, 2, (4, 8), (2, 4)),
]


def segment_sumsq(y, seg):
    """float64 sums of squares of each row of y [M, C] over consecutive
    segments of `seg` elements (the oracle of the partials layout)."""
    y = y.double().cpu()
    M, C = y.shape
    P = (C + seg - 1) // seg
    pad = torch.zeros(M, P * seg, dtype=torch.float64)
    pad[:, :C] = y
    return (pad * pad).view(M, P, seg).sum(-1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,H,W,C,ws,shift", [(1, 1, 180, 360, 1024, (9, 18), (4, 9)),
                                                (1, 1, 90, 180, 192, (9, 18), (0, 0)),
                                                (2, 2, 18, 36, 320, (9, 18), (4, 9)),
                                                (1, 1, 16, 32, 64, (4, 8), (2, 4))])
def test_proj_reverse_residual_sumsq(device, dtype, B, T, H, W, C, ws, shift):
    """The output equals nsw_proj_reverse_residual's bit for bit, and the
    partials are the sums of squares of the stored rows over 256-byte
    segments, in token order."""
    from nsw import _lib, ops
    g = torch.Generator().manual_seed(C + W)
    nW = B * (H // ws[0]) * (W // ws[1])
    L = T * ws[0] * ws[1]
    o = torch.randn(nW, L, C, generator=g).to(dtype)
    wp = synth.trunc_normal((C, C), 0.02, g).to(dtype)
    bp = (0.1 * torch.randn(C, generator=g)).to(dtype)
    skip = torch.randn(B, T, H, W, C, generator=g).to(dtype)
    d = lambda t: t.to(device)
    y0 = ops.proj_reverse_residual(d(o), d(wp), d(bp), d(skip), ws, shift)
    y, ss = ops.proj_reverse_residual_sumsq(d(o), d(wp), d(bp), d(skip), ws, shift)
    assert torch.equal(y, y0)
    es = 2 if dtype == torch.bfloat16 else 4
    P = (C * es + 511) // 512
    assert ss.shape == (B * T * H * W, P) and ss.dtype == torch.float32
    assert _lib.lib().nsw_row_sumsq_parts(C, ops.dtype_code(y)) == P
    want = segment_sumsq(y.reshape(-1, C), 512 // es)
    assert rel_l2(ss, want) < 1e-6
    assert (ss.double().cpu() - want).abs().max().item() <= 1e-5 * want.abs().max().item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", [(64800, 4096, 1024), (1000, 576, 192), (257, 4096, 256), (16, 64, 64)])
@pytest.mark.parametrize("epi", ["none", "gelu", "residual"])
def test_linear_rowscale(device, dtype, M, N, K, epi):
    from nsw import _lib, ops
    g = torch.Generator().manual_seed(M + N + K + 7)
    x = (2.0 * torch.randn(M, K, generator=g) - 0.3).to(dtype)
    nw = (1 + 0.2 * torch.randn(K, generator=g)).to(dtype)
    w = synth.trunc_normal((N, K), 0.02, g).to(dtype)
    b = (0.1 * torch.randn(N, generator=g)).to(dtype)
    r = torch.randn(M, N, generator=g).to(dtype)
    eps = torch.finfo(dtype).eps
    es = 2 if dtype == torch.bfloat16 else 4
    ss = segment_sumsq(x.float(), 512 // es).float().contiguous()
    code = {"none": _lib.NSW_EPI_NONE, "gelu": _lib.NSW_EPI_BIAS_GELU, "residual": _lib.NSW_EPI_BIAS_RESIDUAL}[epi]
    d = lambda t: t.to(device)
    got = ops.linear_rowscale(d(x), d(fold(w, nw, dtype)), d(ss), None if epi == "none" else d(b),
                              d(r) if epi == "residual" else None, epilogue=code, eps=eps)
    # the fp32 reference runs where it finishes in seconds: on the host for
    # the small shapes, on the GPU (torch fp32, full-precision matmul) for
    # the production shape (64800 x 4096 x 1024)
    rd = device if M * N * K > 3e11 else torch.device("cpu")
    y = F.linear(ref.rms_norm(x.to(rd).float(), nw.to(rd).float(), eps), w.to(rd).float())
    if epi != "none":
        y = y + b.to(rd).float()
    if epi == "gelu":
        y = ref.gelu_erf(y)
    if epi == "residual":
        y = y + r.to(rd).float()
    assert got.dtype == dtype
    assert rel_l2(got.to(rd), y) < TOL[dtype]


def test_linear_rowscale_rejects_bad_partials(device):
    from nsw import ops
    x = torch.randn(16, 64, device=device)
    w = torch.randn(64, 64, device=device)
    with pytest.raises(ValueError, match="row_sumsq"):
        ops.linear_rowscale(x, w, torch.ones(15, 1, device=device))
    with pytest.raises(ValueError, match="row_sumsq"):
        ops.linear_rowscale(x, w, torch.ones(16, 1, device=device, dtype=torch.float64))


@pytest.mark.parametrize("dtype,case", [(torch.float32, (1, 1, 90, 180, 192, 6, (9, 18), (4, 9))),
                                        (torch.bfloat16, (1, 1, 180, 360, 1024, 16, (9, 18), (4, 9))),
                                        (torch.bfloat16, (2, 2, 18, 36, 128, 2, (9, 18), (4, 9)))])
def test_block_norm_folds(device, dtype, case):
    """Block.forward with norm2 folded (6 launches: norm1 gather, proj
    scatter; the default), both norms folded (the one-block window-order
    chain, 6; fold_norm1 alone selects it too) and neither (7) matches the
    oracle."""
    import nsw
    B, T, H, W, C, heads, ws, shift = case
    p = synth.block_params(C, heads, seed=41, random_bias=True, random_norm=True)
    p = {k: v.to(dtype).float() for k, v in p.items()}
    x = (2.0 * synth.activations((B, T, H, W, C), seed=42)).to(dtype).float()
    blk = nsw.Block(C, heads, (H, W), ws, T, shift_size=shift)
    blk.load_state_dict(p)
    blk = blk.to(device=device, dtype=dtype)
    assert blk.fold_norm2 and not blk.fold_norm1
    want = ref.block_forward(x, p, heads, ws, shift, eps=torch.finfo(dtype).eps)
    outs = {}
    with torch.inference_mode():
        xd = x.to(device=device, dtype=dtype)
        for f1, f2 in [(True, True), (False, True), (True, False), (False, False)]:
            blk.fold_norm1, blk.fold_norm2 = f1, f2
            outs[(f1, f2)] = blk(xd)
    # the residual increment y - x is checked too; its error floor is what
    # rounding the exact result to the output dtype alone costs (large when
    # the increment is small against x, as at C = 128)
    floor = rel_l2(want.to(dtype).float() - x, want - x)
    for k, y in outs.items():
        assert rel_l2(y, want) < TOL[dtype], k
        assert rel_l2(y - xd, want - x) < 2 * TOL[dtype] + floor, k
