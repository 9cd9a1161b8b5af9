"""The single-expert workload (one SwiGLU expert at batch 1: gate/up Q4_K 512 x 2048, down Q6_K 2048 x 512) through
exactly the layer instance the benchmark times for it: a one-expert, top-1 MoELayer without a shared expert on the
fused plan, each copy a row view of one [copies, bytes] tensor, called eagerly and replayed from one graph. Its
output is the expert's FFN (engines/base.py:99-102, 566-571; its routing weight is softmax over one logit = 1),
checked against the oracle's fp32 expert chain within 2e-3."""
import numpy as np
import pytest
import torch

from gguf import synth
from gguf.hip.moe import MoELayer, new_workspace
from oracle import moe_ref
from oracle import quants_ref as q

pytestmark = pytest.mark.gpu
COPIES = 4


@pytest.fixture(scope="module")
def experts():
    cases = [synth.expert_case(seed) for seed in range(COPIES)]
    gate_up = np.stack([np.concatenate((c["gate"], c["up"])).reshape(-1) for c in cases])
    down = np.stack([c["down"].reshape(-1) for c in cases])
    return cases, torch.from_numpy(gate_up).cuda(), torch.from_numpy(down).cuda()


def one_expert_layers(gate_up, down):
    router = torch.from_numpy(np.random.default_rng(11).standard_normal((1, 2048)).astype(np.float32) * 0.02).cuda()
    return [MoELayer(gate_up=gate_up[i:i + 1], down=down[i:i + 1], router=router, hidden=2048, inter=512,
                     n_experts=1, top_k=1) for i in range(gate_up.shape[0])]


def oracle_expert(case):
    gu = q.dequantize_matrix(np.concatenate((case["gate"], case["up"])), "Q4_K", 1024, 2048)
    dn = q.dequantize_matrix(case["down"], "Q6_K", 2048, 512)
    return moe_ref.expert_ffn(case["x"], gu, dn, 512)


@pytest.mark.parametrize("graph", [False, True])
def test_config1_expert_as_benchmarked(hip, experts, graph):
    cases, gate_up, down = experts
    layers = one_expert_layers(gate_up, down)
    assert all(layer.plan(1) == "fused" for layer in layers)
    xs = [torch.from_numpy(c["x"]).cuda() for c in cases]
    ys = torch.full((COPIES, 1, 2048), float("nan"), device="cuda")
    ids = torch.full((COPIES, 1, 1), -1, dtype=torch.int32, device="cuda")
    wts = torch.zeros(COPIES, 1, 1, device="cuda")
    ws = new_workspace(layers[0].workspace_bytes(1), "cuda")

    def calls():
        for i, layer in enumerate(layers):
            layer(xs[i], out=ys[i], ids=ids[i], weights=wts[i], workspace=ws)

    print(f"[config1] {COPIES} one-expert layers, graph={graph}", flush=True)
    calls()
    torch.cuda.synchronize()
    if graph:
        ys.fill_(float("nan"))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            calls()
        for _ in range(2):
            ys.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
    assert layers[0].status(ws) == 0
    assert bool((ids == 0).all()) and bool((wts == 1.0).all())
    for i, case in enumerate(cases):
        y = ys[i].cpu().numpy()
        err = moe_ref.rel_err(y, oracle_expert(case))
        assert err < 2e-3, f"copy {i}: rel err {err:.2e}"
