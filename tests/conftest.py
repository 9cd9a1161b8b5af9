import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "willow-v2_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built libwillow_hip.so")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def hip():
    """The HIP backend, loaded; a GPU test fails (not skips) if the library is missing."""
    import torch
    from gguf import hip as hip_mod
    assert torch.cuda.is_available()
    hip_mod.library()
    return hip_mod


@pytest.fixture(scope="session")
def layer_c2():
    """The full Qwen3.6-35B-A3B-shaped layer (256 experts, top-8, shared expert), seed 1, as numpy."""
    from gguf import synth
    return synth.moe_layer(1)
