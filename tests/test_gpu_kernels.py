"""GPU parity of the floating-point kernels against the fp32 CPU oracle:
RMSNorm, the fused norm+gather, the MFMA GEMM with every epilogue, the
QKV projection with per-head QK-RMSNorm, window attention (shift mask from
indices, a mask tensor, no mask).

Tolerances (relative L2 error, float64 norms): fp32 mode <= 1e-5; bf16 mode
<= 1e-2 against the oracle evaluated on the same bf16-rounded inputs."""
import pytest
import torch
import torch.nn.functional as F

from oracle import swin_ref as ref
from oracle import synth

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def rel_l2(a, b):
    a = a.double().cpu()
    b = b.double().cpu()
    return (torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b)).item()


def rnd(t, dtype):
    """Round to the kernel dtype and back to fp32 (the oracle's input)."""
    return t.to(dtype).float()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,C", [(64800, 1024), (1000, 192), (37, 4096), (5, 8)])
def test_rmsnorm(device, dtype, rows, C):
    from nsw import ops
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(rows, C, generator=g) * 3).to(dtype)
    w = (1 + 0.3 * torch.randn(C, generator=g)).to(dtype)
    eps = torch.finfo(dtype).eps
    got = ops.rms_norm(x.to(device), w.to(device), eps)
    want = ref.rms_norm(x.float(), w.float(), eps)
    assert rel_l2(got, want) < (1e-6 if dtype == torch.float32 else 5e-3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rmsnorm_roll_partition(device, dtype):
    from nsw import ops
    B, T, H, W, C, ws, s = 1, 2, 18, 36, 256, (9, 18), (4, 9)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, T, H, W, C, generator=g).to(dtype)
    w = (1 + 0.3 * torch.randn(C, generator=g)).to(dtype)
    eps = torch.finfo(dtype).eps
    got = ops.rmsnorm_roll_partition(x.to(device), w.to(device), ws, s, eps)
    xr = ref.roll(ref.rms_norm(x.float(), w.float(), eps), (-s[0], -s[1]), (-3, -2))
    want = ref.window_partition(xr, ws).reshape(-1, T * 162, C)
    assert rel_l2(got, want) < (1e-6 if dtype == torch.float32 else 5e-3)


GEMM_SHAPES = [
    # M, N, K
    (64800, 1024, 1024),
    (64800, 1024, 4096),  # fc2 at config 2 (128 stages)
    (1000, 576, 192),     # N not a multiple of the 128 tile, M tail
    (300, 192, 768),
    (257, 4096, 256),
    (16, 64, 64),
    # stage counts around the main loop's 12-step iterations (the operand
    # copies past the last stage land in unused LDS slots): 2, 7 and 5 stages
    (96, 128, 128),
    (513, 320, 448),
    (64, 256, 320),
]


def ref_linear(x, w, device):
    """F.linear in fp32 (the library routine the reference calls), on the CPU
    for small products and with the fp32 device GEMM (TF32 off) for large
    ones, returned on the CPU."""
    if x.shape[0] * w.shape[0] * x.shape[1] <= 2e10:
        return F.linear(x.float(), w.float())
    return F.linear(x.to(device).float(), w.to(device).float()).cpu()


# K an odd number of MFMA steps (32 bf16 / 16 fp32 elements each): the last
# operand stage holds one step's k and its second half is never consumed
ODD_K_SHAPES = [
    (torch.bfloat16, 777, 96, 32), (torch.bfloat16, 513, 128, 96), (torch.bfloat16, 300, 64, 160),
    (torch.bfloat16, 1000, 256, 2080), (torch.bfloat16, 64800, 128, 32),
    (torch.float32, 777, 96, 16), (torch.float32, 513, 128, 48), (torch.float32, 300, 64, 80),
]


@pytest.mark.parametrize("dtype,M,N,K", ODD_K_SHAPES)
@pytest.mark.parametrize("epi", ["none", "bias", "gelu", "residual"])
def test_linear_odd_k_steps(device, dtype, M, N, K, epi):
    test_linear_epilogues(device, dtype, M, N, K, epi)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
@pytest.mark.parametrize("epi", ["none", "bias", "gelu", "residual"])
def test_linear_epilogues(device, dtype, M, N, K, epi):
    from nsw import _lib, ops
    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = synth.trunc_normal((N, K), 0.02, g).to(dtype)
    b = (0.1 * torch.randn(N, generator=g)).to(dtype)
    r = torch.randn(M, N, generator=g).to(dtype)
    lin = ref_linear(x, w, device)
    if epi == "none":
        got = ops.linear(x.to(device), w.to(device))
        want = lin
    elif epi == "bias":
        got = ops.linear(x.to(device), w.to(device), b.to(device))
        want = lin + b.float()
    elif epi == "gelu":
        got = ops.linear(x.to(device), w.to(device), b.to(device), epilogue=_lib.NSW_EPI_BIAS_GELU)
        want = F.gelu(lin + b.float())
    else:
        got = ops.linear(x.to(device), w.to(device), b.to(device), residual=r.to(device))
        want = lin + b.float() + r.float()
        # the residual dominates: also check the GEMM part alone
        assert rel_l2(got.float().cpu() - r.float(), want - r.float()) < 3 * TOL[dtype]
    assert got.dtype == dtype
    assert rel_l2(got, want) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,C,heads", [(64800, 1024, 16), (16200, 192, 6), (500, 128, 8), (100, 64, 1),
                                      (500, 64, 16), (700, 128, 16)])   # head dims 4 and 8
def test_qkv_projection_headnorm(device, dtype, M, C, heads):
    from nsw import ops
    hd = C // heads
    g = torch.Generator().manual_seed(7)
    x = torch.randn(M, C, generator=g).to(dtype)
    w = synth.trunc_normal((3 * C, C), 0.02, g).to(dtype)
    b = (0.1 * torch.randn(3 * C, generator=g)).to(dtype)
    qn = (1 + 0.2 * torch.randn(hd, generator=g)).to(dtype)
    kn = (1 + 0.2 * torch.randn(hd, generator=g)).to(dtype)
    eps = torch.finfo(dtype).eps
    got = ops.qkv_projection(x.to(device), w.to(device), b.to(device), qn.to(device), kn.to(device), heads, eps)
    y = ref_linear(x, w, device) + b.float()
    q, k, v = y.split(C, dim=-1)
    q = ref.rms_norm(q.reshape(M, heads, hd), qn.float(), eps).reshape(M, C)
    k = ref.rms_norm(k.reshape(M, heads, hd), kn.float(), eps).reshape(M, C)
    want = torch.cat([q, k, v], -1)
    assert rel_l2(got, want) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_qkv_projection_headnorm_c32(device, dtype):
    """C = 32 with 8 heads (head dim 4), the width of the reference's model
    test (tests/test_all.py:168-169); in bf16 the GEMM's k is one MFMA step."""
    from nsw import ops
    M, C, heads, hd = 777, 32, 8, 4
    g = torch.Generator().manual_seed(9)
    x = torch.randn(M, C, generator=g).to(dtype)
    w = synth.trunc_normal((3 * C, C), 0.02, g).to(dtype)
    b = (0.1 * torch.randn(3 * C, generator=g)).to(dtype)
    qn = (1 + 0.2 * torch.randn(hd, generator=g)).to(dtype)
    kn = (1 + 0.2 * torch.randn(hd, generator=g)).to(dtype)
    eps = torch.finfo(dtype).eps
    got = ops.qkv_projection(x.to(device), w.to(device), b.to(device), qn.to(device), kn.to(device), heads, eps)
    y = ref_linear(x, w, device) + b.float()
    q, k, v = y.split(C, dim=-1)
    q = ref.rms_norm(q.reshape(M, heads, hd), qn.float(), eps).reshape(M, C)
    k = ref.rms_norm(k.reshape(M, heads, hd), kn.float(), eps).reshape(M, C)
    assert rel_l2(got, torch.cat([q, k, v], -1)) < TOL[dtype]


def attention_oracle(qkv, heads, scale, mask):
    Bw, L, C3 = qkv.shape
    C = C3 // 3
    hd = C // heads
    q, k, v = [t.reshape(Bw, L, heads, hd).permute(0, 2, 1, 3) for t in qkv.float().split(C, -1)]
    s = torch.matmul(q, k.transpose(-1, -2)) * scale
    if mask is not None:
        nW = mask.shape[0]
        s = s + mask[None].expand(Bw // nW, nW, L, L).reshape(Bw, 1, L, L)
    o = torch.matmul(torch.softmax(s, -1), v)
    return o.transpose(1, 2).reshape(Bw, L, C)


ATTN_CASES = [
    # B, T, H, W, C, heads, ws, shift
    (1, 1, 180, 360, 1024, 16, (9, 18), (4, 9)),
    (1, 1, 90, 180, 192, 6, (9, 18), (4, 9)),
    (1, 1, 18, 36, 128, 2, (9, 18), (0, 0)),
    (2, 2, 18, 36, 128, 2, (9, 18), (4, 9)),
    (1, 1, 16, 32, 64, 2, (4, 8), (2, 4)),
    (1, 1, 9, 18, 128, 2, (9, 18), (0, 0)),
    (3, 1, 18, 36, 320, 5, (9, 18), (4, 9)),
    (1, 2, 18, 36, 64, 16, (9, 18), (4, 9)),       # head dim 4 (the reference's test model: e32 / 8 heads)
    (2, 1, 18, 36, 64, 8, (9, 18), (4, 9)),        # head dim 8
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,H,W,C,heads,ws,shift", ATTN_CASES)
@pytest.mark.parametrize("mode", ["index", "tensor"])
def test_window_attention(device, dtype, B, T, H, W, C, heads, ws, shift, mode):
    from nsw import ops
    L = T * ws[0] * ws[1]
    nW = (H // ws[0]) * (W // ws[1])
    Bw = B * nW
    g = torch.Generator().manual_seed(11)
    qkv = torch.randn(Bw, L, 3 * C, generator=g)
    hd = C // heads
    # QK-normed inputs as the block produces them (|q| = |k| = sqrt(hd))
    qkv[..., :2 * C] = ref.rms_norm(qkv[..., :2 * C].reshape(Bw, L, 2 * heads, hd), torch.ones(hd)).reshape(Bw, L, 2 * C)
    qkv = qkv.to(dtype)
    mask = ref.make_attention_mask(H, W, ws, shift, T)
    scale = hd ** -0.5
    if mode == "index":
        got = ops.window_attention(qkv.to(device), heads, scale, geometry=(H, W, ws, shift, T))
    else:
        got = ops.window_attention(qkv.to(device), heads, scale, mask=mask.to(device))
    want = attention_oracle(qkv, heads, scale, mask)
    assert rel_l2(got, want) < TOL[dtype]


@pytest.mark.parametrize("H,W,C,heads", [(180, 360, 1024, 16), (9, 18, 128, 2), (18, 36, 320, 5)])
def test_window_attention_kernels_agree(device, H, W, C, heads):
    """bf16, head dim 64, 9 x 18 windows: the persistent kernel (index mode,
    no mask) and the staged one (an all-zero mask tensor) do the same
    arithmetic in the same order, so their outputs are bit-identical."""
    from nsw import ops
    ws = (9, 18)
    L = ws[0] * ws[1]
    nW = (H // ws[0]) * (W // ws[1])
    g = torch.Generator().manual_seed(13)
    qkv = (torch.randn(nW, L, 3 * C, generator=g) * 2).to(torch.bfloat16).to(device)
    scale = (C // heads) ** -0.5
    a = ops.window_attention(qkv, heads, scale, geometry=(H, W, ws, (0, 0), 1))
    b = ops.window_attention(qkv, heads, scale, mask=torch.zeros(nW, L, L, device=device))
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shift", [(0, 0), (4, 9)])
def test_window_attention_windows_isolated(device, shift, dtype):
    """Head dim 64: a window's output depends on its own rows only.
    Every third window holds NaN; the others (including the last, whose
    padding rows lie past the end of qkv) must match the oracle.  512 windows
    x 2 heads, so that each CU runs several items and reuses its LDS after
    NaN windows."""
    from nsw import ops
    H, W, C, heads, ws = 144, 576, 128, 2, (9, 18)
    L = ws[0] * ws[1]
    nW = (H // ws[0]) * (W // ws[1])
    g = torch.Generator().manual_seed(14)
    qkv = torch.randn(nW, L, 3 * C, generator=g).to(dtype)
    bad = torch.arange(nW) % 3 == 1
    qkv[bad] = float("nan")
    scale = (C // heads) ** -0.5
    got = ops.window_attention(qkv.to(device), heads, scale, geometry=(H, W, ws, shift, 1)).cpu()
    want = attention_oracle(qkv, heads, scale, ref.make_attention_mask(H, W, ws, shift, 1))
    assert torch.isfinite(got[~bad]).all()
    assert rel_l2(got[~bad], want[~bad]) < TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_window_attention_no_mask_and_random_mask(device, dtype):
    from nsw import ops
    Bw, L, C, heads = 24, 162, 128, 2
    g = torch.Generator().manual_seed(12)
    qkv = torch.randn(Bw, L, 3 * C, generator=g).to(dtype)
    scale = 0.125
    got = ops.window_attention(qkv.to(device), heads, scale)
    assert rel_l2(got, attention_oracle(qkv, heads, scale, None)) < TOL[dtype]
    mask = torch.randn(6, L, L, generator=g) * 3
    got = ops.window_attention(qkv.to(device), heads, scale, mask=mask.to(device))
    assert rel_l2(got, attention_oracle(qkv, heads, scale, mask)) < TOL[dtype]
