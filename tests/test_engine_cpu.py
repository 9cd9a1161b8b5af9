"""The HIP engine mixin's host-side behaviour that needs no GPU."""
import torch

from engines.qwen36 import HipMoE


class SkippingEngine(HipMoE):
    """An engine run with --min-expert-weight (engines/base.py:240; main.py:108)."""
    min_expert_weight = 0.05


def test_min_expert_weight_reaches_the_layer():
    """Engine.min_expert_weight (engines/base.py:240, main.py:108) is handed to the layer each call, as
    skip_small_experts runs inside Engine.moe (:463-464); a view records what it was given."""
    eng = SkippingEngine()

    class View:
        device = torch.device("cpu")
        _next = None

        def __init__(self):
            self.set_to = []
            self.min_expert_weight = 0.0

        def set_min_expert_weight(self, w):
            self.set_to.append(w)
            self.min_expert_weight = w

        def __call__(self, x):
            return x

    view = View()
    eng.__dict__["_hip_moe_layers"] = {0: (view, None)}
    eng.experts = type("Store", (), {"layers": [None]})()
    x = torch.zeros(1, 2048)
    eng.moe(x, 0)
    eng.moe(x, 0)
    assert view.set_to == [0.05]  # set once, kept while the engine's value does not change
    eng.min_expert_weight = 0.0
    eng.moe(x, 0)
    assert view.set_to == [0.05, 0.0]
