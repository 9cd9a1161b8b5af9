"""A decode step captured once as a HIP graph and replayed (the way bench.py runs its 40 layers): every replay,
with new inputs copied into the captured buffers and eager layer calls in between, gives exactly the eager result.
Covers the plans: fused (1 token), GEMV (2..8 tokens) and split (more than 8: at 40 tokens over 64 experts the
GEMV experts run on the library's second stream, forked and joined by events, which capture turns into graph
edges). The layers record no memset nodes (their counters and flags are cleared by kernels)."""
import pytest
import torch

from gguf import synth
from gguf.hip.moe import MoELayer, new_workspace

pytestmark = pytest.mark.gpu
N_LAYERS = 3


@pytest.fixture(scope="module")
def layers():
    return [MoELayer.from_host(synth.moe_layer(90 + i, experts=64, top_k=8)) for i in range(N_LAYERS)]


@pytest.mark.parametrize("tokens", [1, 5, 40])
def test_graph_replays_match_eager(layers, tokens):
    ws = new_workspace(max(layer.workspace_bytes(tokens) for layer in layers), "cuda")
    x_in = torch.zeros(N_LAYERS, tokens, 2048, device="cuda")
    y_out = torch.zeros(N_LAYERS, tokens, 2048, device="cuda")
    for l, layer in enumerate(layers):  # load the kernels before capture
        layer(x_in[l], out=y_out[l], workspace=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=torch.cuda.Stream()):
        for l, layer in enumerate(layers):
            layer(x_in[l], out=y_out[l], workspace=ws)
    torch.cuda.synchronize()
    for rep in range(4):
        xs = torch.stack([torch.from_numpy(synth.tokens(1000 * rep + 10 * tokens + l, tokens))
                          for l in range(N_LAYERS)]).cuda()
        x_in.copy_(xs)
        graph.replay()
        eager = torch.stack([layer(xs[l]) for l, layer in enumerate(layers)])
        torch.cuda.synchronize()
        assert torch.isfinite(eager).all()
        assert torch.equal(y_out, eager), f"replay {rep}: max diff {(y_out - eager).abs().max().item()}"
