"""Fork scopes (wl_moe_fork_begin / wl_moe_fork_end): split-plan layer calls inside a scope hand their MFMA experts to
the library's second stream and back through words of their workspace instead of a fork and a join event each.
They run the same kernels in the same order of arithmetic, so every result equals the same call outside a scope bit
for bit: eagerly, captured in a graph and replayed with eager work in between, with one workspace shared by the
layers or one each, at prefill sizes (where a call takes no second stream), on the full-shape Zipf batched-decode
layer, and through a chained decoder step (pre-norm and residual, each layer reading the previous one's output). Misuse of the scope is an error, and a
hand-off that gives up (forced from the host: the grouping withholds its flag, the wait gives up after a short
bounded spin and the MFMA kernels are skipped, so every kernel exits) is reported once by wl_moe_workspace_status,
after which the next call is correct again."""
import contextlib

import pytest
import torch

from gguf import hip, synth
from gguf.hip.moe import MoELayer, new_workspace

pytestmark = pytest.mark.gpu
N_LAYERS = 3
TOKENS = 40  # 64 experts, top-8: 320 pairs, both expert classes, the second stream used


@pytest.fixture(scope="module")
def layers():
    return [MoELayer.from_host(synth.moe_layer(190 + i, experts=64, top_k=8)) for i in range(N_LAYERS)]


def inputs(seed, tokens=TOKENS, n=N_LAYERS):
    return torch.stack([torch.from_numpy(synth.tokens(seed + l, tokens)) for l in range(n)]).cuda()


def per_call(layers, xs):
    out = torch.stack([layer(xs[l]) for l, layer in enumerate(layers)])
    torch.cuda.synchronize()
    return out


def test_scope_eager_matches_per_call(layers):
    assert all(layer.plan(TOKENS) == "split" for layer in layers)
    shared_ws = new_workspace(max(layer.workspace_bytes(TOKENS) for layer in layers), "cuda")
    own_ws = [new_workspace(layer.workspace_bytes(TOKENS), "cuda") for layer in layers]
    for rep in range(3):
        xs = inputs(300 + 10 * rep)
        want = per_call(layers, xs)
        with hip.fork_scope():
            got_shared = torch.stack([layer(xs[l], workspace=shared_ws) for l, layer in enumerate(layers)])
            got_own = torch.stack([layer(xs[l], workspace=own_ws[l]) for l, layer in enumerate(layers)])
        torch.cuda.synchronize()
        assert torch.isfinite(want).all()
        assert torch.equal(got_shared, want), f"rep {rep}: max diff {(got_shared - want).abs().max().item()}"
        assert torch.equal(got_own, want), f"rep {rep}: max diff {(got_own - want).abs().max().item()}"
    assert layers[0].status(shared_ws) == 0
    assert all(layer.status(own_ws[l]) == 0 for l, layer in enumerate(layers))


def test_scope_graph_replays_match_eager(layers):
    ws = new_workspace(max(layer.workspace_bytes(TOKENS) for layer in layers), "cuda")
    x_in = torch.zeros(N_LAYERS, TOKENS, 2048, device="cuda")
    y_out = torch.zeros(N_LAYERS, TOKENS, 2048, device="cuda")

    def step():
        with hip.fork_scope():
            for l, layer in enumerate(layers):
                layer(x_in[l], out=y_out[l], workspace=ws)

    step()  # load the kernels before capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=torch.cuda.Stream()):
        step()
    torch.cuda.synchronize()
    for rep in range(4):
        xs = inputs(700 + 10 * rep)
        x_in.copy_(xs)
        graph.replay()
        eager = per_call(layers, xs)  # outside the scope, on the per-call fork and join
        assert torch.isfinite(eager).all()
        assert torch.equal(y_out, eager), f"replay {rep}: max diff {(y_out - eager).abs().max().item()}"
    assert layers[0].status(ws) == 0


@pytest.mark.parametrize("graph", [False, True])
def test_scope_prefill_size_matches_per_call(layers, graph):
    """At prefill sizes (experts averaging 32 tokens or more) a split call takes no second stream, in a scope or
    not: the same results, eagerly and replayed."""
    tokens = 300
    ws = new_workspace(max(layer.workspace_bytes(tokens) for layer in layers), "cuda")
    xs = inputs(1100, tokens=tokens)
    want = per_call(layers, xs)
    y = torch.zeros_like(want)

    def step():
        with hip.fork_scope():
            for l, layer in enumerate(layers):
                layer(xs[l], out=y[l], workspace=ws)

    step()
    torch.cuda.synchronize()
    assert torch.equal(y, want), f"max diff {(y - want).abs().max().item()}"
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=torch.cuda.Stream()):
            step()
        for rep in range(3):
            y.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, want), f"replay {rep}: max diff {(y - want).abs().max().item()}"
    assert layers[0].status(ws) == 0


@pytest.fixture(scope="module")
def zipf_layer():
    return MoELayer.from_host(synth.moe_layer(3, zipf_alpha=1.1))


@pytest.mark.parametrize("tokens", [64, 128, 512])
def test_scope_zipf_matches_per_call(zipf_layer, tokens):
    """The batched-decode workload's layer (256 experts, Zipf(1.1) routing) at 64 tokens, as the benchmark runs
    it, and at 128 and 512 tokens (single-workgroup and multi-chunk grouping), where the MFMA experts dominate and
    the scope still takes the second stream: scoped calls equal per-call ones bit for bit, and no wait gave up."""
    layer = zipf_layer
    assert layer.plan(tokens) == "split"
    ws = new_workspace(layer.workspace_bytes(tokens), "cuda")
    xs = inputs(33 + tokens, tokens=tokens, n=4)
    print(f"[fork] zipf layer, T={tokens}", flush=True)
    want = torch.stack([layer(x) for x in xs])
    with hip.fork_scope():
        got = torch.stack([layer(x, workspace=ws) for x in xs])
    torch.cuda.synchronize()
    assert layer.status(ws) == 0
    assert torch.isfinite(want).all()
    assert torch.equal(got, want), f"max diff {(got - want).abs().max().item()}"


def test_scope_chained_decoder_step(layers):
    """A decoder step's MoE half chained through the layers, x <- x + MoE(rms_norm(x)) (WL_MOE_PRE_NORM and
    WL_MOE_RESIDUAL, each layer reading the previous one's output), in one scope and per call: the same bits."""
    chained = [layer.with_norm(torch.from_numpy(synth.tokens(40 + l, 1)[0] * 0.1).cuda()) for l, layer in
               enumerate(layers)]
    ws = new_workspace(max(layer.workspace_bytes(TOKENS) for layer in chained), "cuda")
    x0 = inputs(1300, n=1)[0]

    def run(scoped):
        xs = [x0]
        with hip.fork_scope() if scoped else contextlib.nullcontext():
            for layer in chained:
                xs.append(layer(xs[-1], workspace=ws))
        torch.cuda.synchronize()
        return torch.stack(xs[1:])

    want = run(False)
    got = run(True)
    assert torch.isfinite(want).all()
    assert torch.equal(got, want), f"max diff {(got - want).abs().max().item()}"
    assert chained[0].status(ws) == 0


def test_scope_misuse_is_an_error():
    lib = hip.library()
    s = torch.cuda.current_stream().cuda_stream
    other = torch.cuda.Stream()
    assert lib.wl_moe_fork_end(s) == hip.EINVAL_SCOPE  # none open
    assert lib.wl_moe_fork_begin(s) == 0
    try:
        assert lib.wl_moe_fork_begin(s) == hip.EINVAL_SCOPE  # one per device
        assert lib.wl_moe_fork_end(other.cuda_stream) == hip.EINVAL_SCOPE  # not this scope's stream
    finally:
        assert lib.wl_moe_fork_end(s) == 0
    assert lib.wl_moe_fork_end(s) == hip.EINVAL_SCOPE
    torch.cuda.synchronize()


def test_scope_give_up_is_reported(layers):
    layer = layers[0]
    starved = MoELayer.from_host(synth.moe_layer(190, experts=64, top_k=8))
    starved.struct.flags |= hip.MOE_TEST_STARVE
    ws = new_workspace(layer.workspace_bytes(TOKENS), "cuda")
    x = inputs(900, n=1)[0]
    want = layer(x)
    torch.cuda.synchronize()
    with hip.fork_scope():
        y = starved(x, workspace=ws)  # the MFMA experts are skipped
    torch.cuda.synchronize()
    assert torch.isnan(y).all()  # a hand-off that gave up shows in the outputs, not only in the status word
    assert layer.status(ws) == hip.ESYNC
    assert layer.status(ws) == 0  # reported once, then cleared
    with hip.fork_scope():
        got = layer(x, workspace=ws)
    torch.cuda.synchronize()
    assert layer.status(ws) == 0
    assert torch.equal(got, want)
