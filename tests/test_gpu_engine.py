"""The drop-in: Engine.moe through the HipMoE mixin on an HBM-resident expert store, against the CPU oracle, with
the engine attributes and weight names the reference's Engine uses (engines/base.py:285-286,445-490)."""
import contextlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gguf import synth
from gguf.hbm_store import HBMExpertStore
from gguf.hip import GGMLWeight
from engines.qwen36 import HipMoE
from oracle import moe_ref
from oracle import quants_ref as q

pytestmark = pytest.mark.gpu
PREFIX = "model.language_model."


class TinyEngine(HipMoE):
    """The attributes Engine.moe reads, nothing else."""
    prefix = PREFIX

    def __init__(self, store, weights, top_k, norm=True):
        self.experts, self.weights, self.top_k, self.norm_topk_prob = store, weights, top_k, norm


def engine_weights(lw, layer=0, quantized_shared=True):
    p = f"{PREFIX}layers.{layer}.mlp"
    H, I = lw["hidden"], lw["shared_inter"]
    w = {p + ".gate.weight": torch.from_numpy(lw["router"]).cuda(),
         p + ".shared_expert_gate.weight": torch.from_numpy(lw["shared_gate"][None]).cuda()}
    gu = lw["shared_gate_up"]
    if quantized_shared:
        rb = q.row_bytes("Q4_K", H)
        w[p + ".shared_expert.gate_proj.weight"] = GGMLWeight(torch.from_numpy(gu[:I].reshape(-1)).cuda(), "Q4_K", (I, H))
        w[p + ".shared_expert.up_proj.weight"] = GGMLWeight(torch.from_numpy(gu[I:].reshape(-1)).cuda(), "Q4_K", (I, H))
        w[p + ".shared_expert.down_proj.weight"] = GGMLWeight(
            torch.from_numpy(lw["shared_down"].reshape(-1)).cuda(), lw["shared_down_type"], (H, I))
        assert gu.shape[1] == rb
    else:
        dq = q.dequantize_matrix(gu, "Q4_K", 2 * I, H)
        w[p + ".shared_expert.gate_proj.weight"] = torch.from_numpy(dq[:I]).cuda()
        w[p + ".shared_expert.up_proj.weight"] = torch.from_numpy(dq[I:]).cuda()
        w[p + ".shared_expert.down_proj.weight"] = torch.from_numpy(
            q.dequantize_matrix(lw["shared_down"], lw["shared_down_type"], H, I)).cuda()
    return w


@pytest.fixture(scope="module")
def small_layer():
    return synth.moe_layer(61, hidden=2048, inter=512, shared_inter=512, experts=64, top_k=8)


@pytest.mark.parametrize("quantized_shared", [True, False])
@pytest.mark.parametrize("tokens", [1, 9])
def test_engine_moe_matches_oracle(small_layer, quantized_shared, tokens):
    lw = small_layer
    store = HBMExpertStore.from_host([lw])
    eng = TinyEngine(store, engine_weights(lw, quantized_shared=quantized_shared), lw["top_k"])
    x = synth.tokens(62 + tokens, tokens)
    y = eng.moe(torch.from_numpy(x).cuda(), 0, residual=None)
    assert y.shape == (tokens, 2048) and y.dtype == torch.float32
    # each expert by its own token count; a dense shared expert runs in torch on its fp32 weights
    ref = moe_ref.layer(x, lw, chain="split", shared_chain=None if quantized_shared else "fp32", dtype=np.float64)
    assert moe_ref.rel_err(y.cpu().numpy(), ref) < 2e-3
    yb = eng.moe(torch.from_numpy(x).cuda().to(torch.bfloat16), 0)
    assert yb.dtype == torch.bfloat16


def test_store_surface(small_layer):
    """load_many / load_batches hand out GGMLWeight views that F.linear runs (engines/base.py:552-571)."""
    lw = small_layer
    store = HBMExpertStore.from_host([lw])
    assert store.runs_batched(0)
    assert store.nbytes() == lw["gate_up"].nbytes + lw["down"].nbytes
    x = torch.from_numpy(synth.tokens(5, 1)).cuda()
    (batch,) = list(store.load_batches(0, [3, 17]))
    assert [e for e, _ in batch] == [3, 17]
    for e, (gate_up, down) in store.load_many(0, [3, 17]):
        gu = F.linear(x, gate_up)
        h = F.silu(gu[:, :512]) * gu[:, 512:]
        y = F.linear(h, down).cpu().numpy()
        ref = moe_ref.expert_ffn(x.cpu().numpy(), q.dequantize_matrix(lw["gate_up"][e], "Q4_K", 1024, 2048),
                                 q.dequantize_matrix(lw["down"][e], "Q6_K", 2048, 512), 512)
        assert moe_ref.rel_err(y, ref) < 2e-3
        base, off = gate_up.location()
        assert off == e * lw["gate_up"][0].nbytes
    store.record_usage(0, torch.tensor([[3, 17], [3, 5]]))
    assert int(store.usage[0][3]) == 2


def rms_norm_zero_centered(x, w, eps=1e-6):
    """engines/base.py:27-31 with zero_centered (Qwen3.5's norm, engines/qwen36/model.py:37), in torch fp32."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * (1 + w)


@pytest.mark.parametrize("tokens", [1, 9, 40])  # 40: experts of more than 8 tokens, the second stream
def test_engine_model_loop(tokens):
    """The MoE half of the decoder loop as engines/qwen36/model.py:22 runs it, x = x + moe(rms_norm(x), layer,
    residual=x), over three layers of one HBMExpertStore through HipMoE.moe: each layer names the next (the
    next-layer overlap), and the layer cache is built once. Each layer's output is checked against the oracle on
    the same normalized input the engine got (so the check cannot depend on how torch orders the norm's sums)."""
    lws = [synth.moe_layer(81 + l, hidden=2048, inter=512, shared_inter=512, experts=64, top_k=8) for l in range(3)]
    store = HBMExpertStore.from_host(lws)
    weights = {}
    for l, lw in enumerate(lws):
        weights.update(engine_weights(lw, layer=l))
    eng = TinyEngine(store, weights, 8)
    rng = np.random.default_rng(90)
    norm_w = [torch.from_numpy(rng.normal(0, 0.1, 2048).astype(np.float32)).cuda() for _ in lws]
    x = torch.from_numpy(synth.tokens(91 + tokens, tokens)).cuda()
    for l, lw in enumerate(lws):
        print(f"[engine] model loop T={tokens} layer {l}", flush=True)
        xn = rms_norm_zero_centered(x, norm_w[l])
        y = eng.moe(xn, l, residual=x)
        ref = moe_ref.layer(xn.cpu().numpy(), lw, chain="split", dtype=np.float64)
        assert moe_ref.rel_err(y.cpu().numpy(), ref) < 2e-3
        x = x + y
    views = eng.__dict__["_hip_moe_layers"]
    assert sorted(views) == [0, 1, 2]
    assert views[0][0]._next is views[1][0] and views[1][0]._next is views[2][0]
    assert torch.isfinite(x).all()
    # the same loop as one decode step in the engine's fork scope: the same bits
    x1 = torch.from_numpy(synth.tokens(91 + tokens, tokens)).cuda()
    outs = []
    for scoped in (False, True):
        xs = x1
        with eng.moe_step() if scoped else contextlib.nullcontext():
            for l in range(len(lws)):
                xs = xs + eng.moe(rms_norm_zero_centered(xs, norm_w[l]), l, residual=xs)
        torch.cuda.synchronize()
        outs.append(xs)
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("tokens", [1, 40])  # 1: the fused kernel's exchange; 40: a fork-scope hand-off
def test_engine_step_raises_on_give_up(small_layer, tokens):
    """A bounded wait that gives up inside a decode step (forced from the host with WL_MOE_TEST_STARVE: a fused
    workgroup or the grouping withholds its flag, and the waits give up after a short spin, so every kernel
    exits) raises HipError when the step's scope ends, and the debug check after each layer raises too; once the
    flag is cleared the next step is clean."""
    from gguf import hip
    lw = small_layer
    store = HBMExpertStore.from_host([lw])
    eng = TinyEngine(store, engine_weights(lw), lw["top_k"])
    x = torch.from_numpy(synth.tokens(95 + tokens, tokens)).cuda()
    view = eng.hip_layer(0)[0]
    good = eng.moe(x, 0)
    view.struct.flags |= hip.MOE_TEST_STARVE
    print(f"[engine] forced give-up, T={tokens}", flush=True)
    with pytest.raises(hip.HipError):
        with eng.moe_step():
            eng.moe(x, 0)
    eng.moe_check_status = True  # now the check after the layer itself raises, inside the step
    with pytest.raises(hip.HipError):
        with eng.moe_step():
            eng.moe(x, 0)
    eng.moe_check_status = False
    view.struct.flags &= ~hip.MOE_TEST_STARVE
    with eng.moe_step():
        again = eng.moe(x, 0)
    torch.cuda.synchronize()
    assert torch.equal(again, good)
