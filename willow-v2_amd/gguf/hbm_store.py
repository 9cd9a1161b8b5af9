"""Every routed expert of every layer resident in device memory (288 GB of HBM holds the ~21 GB of Qwen3.6-35B-A3B
experts many times over), in place of gguf/store.py's ExpertStore, which streams experts from an SSD pack into
slab slots with an LRU (gguf/store.py:41-536). The SSD reads, slabs, LRU, hot set, prefetch and usage table have
no role here; the store keeps ExpertStore's calling surface (load_many / load_batches / runs_batched / prefetch /
record_usage / save_usage, gguf/store.py:132-219,482-492) so engines/base.py's call sites keep working, and adds
layer_view(), the per-layer device view the fused MoE kernel takes.

Layout per layer (one allocation each, so an expert is a fixed stride away from the next):
    gate_up  uint8 [n_experts, 2*inter * row_bytes(gate_up_type, hidden)]   gate rows, then up rows
    down     uint8 [n_experts, hidden * row_bytes(down_type, inter)]
Expert strides are 1,179,648 B (Q4_K gate_up) and 860,160 B (Q6_K down) at Qwen3.6's shape, both multiples of 16.
"""
from dataclasses import dataclass

import torch

from .hip import GGMLWeight, MoELayer, row_bytes


@dataclass
class LayerExperts:
    gate_up: torch.Tensor
    down: torch.Tensor
    gate_up_type: str
    down_type: str
    hidden: int
    inter: int

    @property
    def n_experts(self) -> int:
        return self.gate_up.shape[0]


class HBMExpertStore:
    """All layers' experts on one GPU. `layers` is a list of LayerExperts (device tensors)."""

    def __init__(self, layers: list, device="cuda"):
        self.layers = layers
        self.device = torch.device(device)
        self.usage = None  # per-layer expert use counts, kept only when record_usage is called

    @classmethod
    def from_host(cls, host_layers: list, device="cuda"):
        """From per-layer dicts of numpy arrays (gguf.synth.moe_layer's layout), copied to the device once."""
        layers = []
        for lw in host_layers:
            E = lw["experts"]
            layers.append(LayerExperts(
                gate_up=torch.from_numpy(lw["gate_up"].reshape(E, -1)).to(device),
                down=torch.from_numpy(lw["down"].reshape(E, -1)).to(device),
                gate_up_type=lw["gate_up_type"], down_type=lw["down_type"], hidden=lw["hidden"], inter=lw["inter"]))
        return cls(layers, device)

    def nbytes(self) -> int:
        return sum(l.gate_up.numel() + l.down.numel() for l in self.layers)

    # -- ExpertStore's surface ----------------------------------------------------------------------------------

    def weights(self, layer: int, expert: int):
        """(gate_up, down) of one expert as GGMLWeight views into the layer's tensors (no copy)."""
        l = self.layers[layer]
        return (GGMLWeight(l.gate_up[expert], l.gate_up_type, (2 * l.inter, l.hidden)),
                GGMLWeight(l.down[expert], l.down_type, (l.hidden, l.inter)))

    def load_many(self, layer: int, experts: list):
        """Iterator of (expert, (gate_up, down)): every expert is a hit (gguf/store.py:132-137)."""
        return ((e, self.weights(layer, e)) for e in experts)

    def load_batches(self, layer: int, experts: list):
        """One batch holding every expert (gguf/store.py:139-175)."""
        yield [(e, self.weights(layer, e)) for e in experts]

    def runs_batched(self, layer: int) -> bool:
        """Fused gate_up + down of types the kernels run (gguf/store.py:197-202)."""
        l = self.layers[layer]
        return l.gate_up_type in ("Q4_K", "Q6_K") and l.down_type in ("Q4_K", "Q6_K")

    def prefetch(self, layer: int, experts):
        """Nothing to prefetch: everything is resident."""

    def record_usage(self, layer: int, used: torch.Tensor):
        if self.usage is None:
            self.usage = [torch.zeros(l.n_experts, dtype=torch.int64) for l in self.layers]
        self.usage[layer] += torch.bincount(used.reshape(-1).cpu().long(), minlength=self.layers[layer].n_experts)

    def save_usage(self):
        """Usage is not persisted: it steered SSD caching, which an HBM-resident store does not do."""

    # -- the fused kernel's view ----------------------------------------------------------------------------------

    def layer_view(self, layer: int, router: torch.Tensor, top_k: int, norm_topk_prob: bool = True,
                   router_bias=None, shared_gate_up=None, shared_down=None, shared_gate=None, shared_inter=None,
                   shared_gate_up_type=None, shared_down_type=None) -> MoELayer:
        """The MoELayer of one layer: its experts from the store plus the non-expert weights given here (router
        fp32 [n_experts, hidden]; the shared expert's quantized matrices as uint8 tensors)."""
        l = self.layers[layer]
        return MoELayer(gate_up=l.gate_up, down=l.down, router=router, router_bias=router_bias, hidden=l.hidden,
                        inter=l.inter, n_experts=l.n_experts, top_k=top_k, norm_topk_prob=norm_topk_prob,
                        gate_up_type=l.gate_up_type, down_type=l.down_type, shared_gate_up=shared_gate_up,
                        shared_down=shared_down, shared_gate=shared_gate, shared_inter=shared_inter,
                        shared_gate_up_type=shared_gate_up_type, shared_down_type=shared_down_type)


def expert_row_bytes(layer: LayerExperts):
    """(gate_up, down) bytes of one expert."""
    return (2 * layer.inter * row_bytes(layer.gate_up_type, layer.hidden),
            layer.hidden * row_bytes(layer.down_type, layer.inter))
