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


def test_split_fork_from_two_threads(layers):
    """Split-plan calls from two host threads at once, each on its own stream: their GEMV experts share the
    library's second stream (fork and join under one lock), and every result equals the same call made alone."""
    import threading
    tokens = 40
    xs = [torch.from_numpy(synth.tokens(500 + i, tokens)).cuda() for i in range(2)]
    want = [layers[i](xs[i]) for i in range(2)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(2)]
    outs = [[None] * 6 for _ in range(2)]
    errors = []

    def worker(i):
        try:
            with torch.cuda.stream(streams[i]):
                ws = new_workspace(layers[i].workspace_bytes(tokens), "cuda")
                for r in range(6):
                    outs[i][r] = layers[i](xs[i], workspace=ws)
            streams[i].synchronize()
        except Exception as e:  # reported below, in the test's thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not errors, errors
    torch.cuda.synchronize()
    for i in range(2):
        for r in range(6):
            assert torch.equal(outs[i][r], want[i]), f"thread {i}, call {r}"
