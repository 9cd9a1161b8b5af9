"""A GGUF model's MoE blocks loaded straight into HBM (gguf/loader.py) and run through Engine.moe's HIP backend:
the device bytes equal the file's, and the layer's output matches the oracle on the weights written to the file.
Two layers with different down types, as Q4_K_M files have (gguf/compiler.py:42-44)."""
import numpy as np
import pytest
import torch

from engines.qwen36 import HipMoE
from gguf import loader, synth
from gguf.hip import GGMLWeight
from oracle import moe_ref

pytestmark = pytest.mark.gpu


class TinyEngine(HipMoE):
    prefix = loader.PREFIX

    def __init__(self, store, weights, cfg):
        self.experts, self.weights = store, weights
        self.top_k, self.norm_topk_prob = cfg["num_experts_per_tok"], cfg["norm_topk_prob"]


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    layers = [synth.moe_layer(70 + i, hidden=2048, inter=512, shared_inter=512, experts=32, top_k=8, down_type=dt)
              for i, dt in enumerate(("Q6_K", "Q4_K"))]
    path = str(tmp_path_factory.mktemp("gguf") / "synthetic-moe.gguf")
    synth.write_moe_gguf(path, layers)
    # a small staging buffer, so that each tensor crosses several chunks
    header = loader.read_gguf(path)
    store = loader.load_experts(header, "cuda", chunk_bytes=3 << 20)
    weights = loader.load_moe_weights(header, "cuda")
    return layers, loader.moe_config(header), store, weights


def test_loaded_bytes_match_the_file(model):
    layers, cfg, store, weights = model
    assert cfg["num_experts"] == 32 and cfg["num_experts_per_tok"] == 8 and cfg["num_hidden_layers"] == 2
    assert store.loaded_bytes == store.nbytes()
    for n, lw in enumerate(layers):
        l = store.layers[n]
        assert (l.gate_up_type, l.down_type, l.hidden, l.inter) == ("Q4_K", lw["down_type"], 2048, 512)
        assert np.array_equal(l.gate_up.cpu().numpy(), lw["gate_up"].reshape(32, -1))
        assert np.array_equal(l.down.cpu().numpy(), lw["down"].reshape(32, -1))
        p = f"{loader.PREFIX}layers.{n}.mlp"
        assert torch.equal(weights[p + ".gate.weight"].cpu(), torch.from_numpy(lw["router"]))
        assert weights[p + ".shared_expert_gate.weight"].shape == (1, 2048)
        gp = weights[p + ".shared_expert.gate_proj.weight"]
        assert isinstance(gp, GGMLWeight) and gp.type_name == "Q4_K" and tuple(gp.shape) == (512, 2048)
        assert np.array_equal(gp.raw.cpu().numpy(), lw["shared_gate_up"][:512].reshape(-1))
        dp = weights[p + ".shared_expert.down_proj.weight"]
        assert dp.type_name == lw["shared_down_type"]


@pytest.mark.parametrize("layer", [0, 1])
@pytest.mark.parametrize("tokens", [1, 9])
def test_loaded_model_runs(model, layer, tokens):
    layers, cfg, store, weights = model
    eng = TinyEngine(store, weights, cfg)
    x = synth.tokens(80 + tokens, tokens)
    y = eng.moe(torch.from_numpy(x).cuda(), layer).cpu().numpy()
    ref = moe_ref.layer(x, layers[layer], chain="split", dtype=np.float64)  # each expert by its own count
    assert moe_ref.rel_err(y, ref) < 2e-3
