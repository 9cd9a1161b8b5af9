"""The HIP engine mixin's host-side behaviour that needs no GPU."""
import pytest
import torch

from engines.qwen36 import HipMoE


class SkippingEngine(HipMoE):
    """An engine run with --min-expert-weight (engines/base.py:240; main.py:108)."""
    min_expert_weight = 0.05


def test_min_expert_weight_is_refused():
    """skip_small_experts (engines/base.py:413-430) is not run by the HIP layer: a nonzero threshold raises instead
    of silently computing every routed expert."""
    with pytest.raises(NotImplementedError):
        SkippingEngine().moe(torch.zeros(1, 2048), 0)
