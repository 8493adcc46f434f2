"""GPU checks of the torch.ops.nsw.* surface: modules compiled with
torch.compile(fullgraph=True) (eager backend: the traced graph runs the same
libnsw kernels) give the eager outputs bit for bit, and a CUDA graph of the
model forward, replayed several times with eager work between the replays,
reproduces the eager output every time."""
import pytest
import torch

from oracle import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def fresh_dynamo():
    torch._dynamo.reset()
    yield
    torch._dynamo.reset()


def small_model(device, dtype):
    import nsw
    H, W, C = 72, 144, 5
    meta = {"coords": torch.randn(H, W, 3, generator=torch.Generator().manual_seed(5)), "sp_shapes": [[H], [W]],
            "n_channels": C}
    torch.manual_seed(6)
    model = nsw.SwinTransformer(window_size=(9, 18), patch_size=4, in_chans=C, out_chans=C, embed_dim=128,
                                depth=4, num_heads=2, domain_metadata=meta).to(device=device, dtype=dtype).eval()
    x = torch.randn(1, 1, C, H, W, generator=torch.Generator().manual_seed(7)).to(device)
    return model, x


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_compiled_block_matches_eager(device, dtype):
    import nsw
    C, heads = 128, 2
    blk = nsw.Block(C, heads, (18, 36), (9, 18), 1, shift_size=(4, 9))
    blk.load_state_dict(synth.block_params(C, heads, seed=41, random_bias=True, random_norm=True))
    blk = blk.to(device=device, dtype=dtype).eval()
    x = synth.activations((2, 1, 18, 36, C), seed=42).to(device, dtype)
    with torch.inference_mode():
        want = blk(x)
        got = torch.compile(blk, backend="eager", fullgraph=True)(x)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("chain", [True, False])
def test_compiled_model_matches_eager(device, chain):
    model, x = small_model(device, torch.float32)
    model.chain_blocks = chain
    with torch.inference_mode():
        want = model(x)
        got = torch.compile(model, backend="eager", fullgraph=True)(x)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_cuda_graph_of_model_forward(device):
    model, x = small_model(device, torch.bfloat16)
    other = torch.randn_like(x)
    with torch.inference_mode():
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):                 # warm-up: packed weights, workspaces
            for _ in range(2):
                model(x)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y_static = model(x)
        want = model(x)
        torch.cuda.synchronize()
        for _ in range(3):
            model(other)                              # eager work between the replays
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(y_static, want)
