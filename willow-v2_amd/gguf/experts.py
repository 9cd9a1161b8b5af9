"""Where each MoE layer's routed experts are in a GGUF model, worked out from the header alone.

llama.cpp stores all of one layer's experts in one stacked tensor per projection, PyTorch shape
[n_experts, out_features, in_features], quantized along in_features:

    blk.<layer>.ffn_gate_exps.weight, blk.<layer>.ffn_up_exps.weight   (or one blk.<layer>.ffn_gate_up_exps.weight)
    blk.<layer>.ffn_down_exps.weight

Expert e of a stacked tensor is its e-th equal byte slice. The kernels take each expert's gate and up projections
as one [2 * inter, hidden] matrix, gate rows first (the reference's expert pack fuses them the same way,
gguf/compiler.py:69-88), so index_experts requires gate and up to agree in type and shape and hands the loader the
two slices to place back to back. Quant types may change from layer to layer (Q4_K_M files store some layers'
down projections as Q6_K and others as Q4_K), so every layer carries its own types.

Replaces, for this path, the expert scan the reference runs before packing experts for SSD streaming
(gguf/compiler.py:24-88); here the loader copies the slices straight into HBM.
"""
import re
from dataclasses import dataclass

_PROJECTION = re.compile(r"blk\.(?P<layer>\d+)\.ffn_(?P<proj>gate_up|gate|up|down)_exps\.weight")


class ExpertLayoutError(ValueError):
    """The model's expert tensors do not form the layout the MoE kernels run."""


def decoder_layer_count(metadata: dict) -> int:
    """Layers a forward pass runs: the block count less the multi-token-prediction blocks that some models store
    after the decoder layers (`<arch>.nextn_predict_layers`)."""
    arch = metadata["general.architecture"]
    return int(metadata[f"{arch}.block_count"]) - int(metadata.get(f"{arch}.nextn_predict_layers", 0))


@dataclass
class ExpertTensors:
    """One layer's stacked expert tensors. gate_up_parts is [gate, up] or [gate_up] (GGUFTensor each); down the
    stacked down projection."""
    layer: int
    n_experts: int
    gate_up_parts: list
    down: object

    @property
    def gate_up_type(self) -> str:
        return self.gate_up_parts[0].type

    @property
    def down_type(self) -> str:
        return self.down.type

    @property
    def hidden(self) -> int:
        return self.gate_up_parts[0].shape[2]

    @property
    def inter(self) -> int:
        return sum(t.shape[1] for t in self.gate_up_parts) // 2

    @property
    def gate_up_bytes(self) -> int:
        """Bytes of one expert's fused gate_up matrix."""
        return sum(t.nbytes for t in self.gate_up_parts) // self.n_experts

    @property
    def down_bytes(self) -> int:
        return self.down.nbytes // self.n_experts

    def gate_up_ranges(self, e: int) -> list:
        """[(file, offset, size), ...] whose concatenation is expert e's gate_up matrix, gate rows first."""
        return [t.slice(e, self.n_experts) for t in self.gate_up_parts]

    def down_range(self, e: int) -> tuple:
        return self.down.slice(e, self.n_experts)


def index_experts(metadata: dict, tensors: dict) -> list:
    """[ExpertTensors] for layers 0 .. decoder_layer_count - 1, checked to be a layout the kernels run: every
    decoder layer has routed experts, the same expert count in all its projections, gate and up of one type and
    shape, and a down projection of shape [hidden, inter]."""
    n_layers = decoder_layer_count(metadata)
    found = {}
    for name, t in tensors.items():
        m = _PROJECTION.fullmatch(name)
        if m and int(m["layer"]) < n_layers:
            found.setdefault(int(m["layer"]), {})[m["proj"]] = t
    missing = [n for n in range(n_layers) if n not in found]
    if missing:
        raise ExpertLayoutError(f"{len(missing)} of {n_layers} decoder layers have no routed-expert tensors "
                                f"(first: layer {missing[0]}); only all-MoE models are handled")
    out = []
    for n in range(n_layers):
        proj = found[n]
        if "gate_up" in proj:
            parts = [proj["gate_up"]]
        elif "gate" in proj and "up" in proj:
            gate, up = proj["gate"], proj["up"]
            if (gate.type, gate.shape) != (up.type, up.shape):
                raise ExpertLayoutError(f"layer {n}: gate is {gate.type} {gate.shape} but up is {up.type} "
                                        f"{up.shape}; the kernels need them as one fused matrix")
            parts = [gate, up]
        else:
            raise ExpertLayoutError(f"layer {n}: expert projections {sorted(proj)} lack gate/up")
        if "down" not in proj:
            raise ExpertLayoutError(f"layer {n}: no stacked down projection")
        down = proj["down"]
        counts = {t.shape[0] for t in parts + [down]}
        if len(counts) != 1 or any(len(t.shape) != 3 for t in parts + [down]):
            raise ExpertLayoutError(f"layer {n}: stacked expert tensors disagree on the expert count "
                                    f"({[t.shape for t in parts + [down]]})")
        lay = ExpertTensors(n, counts.pop(), parts, down)
        if tuple(down.shape[1:]) != (lay.hidden, lay.inter):
            raise ExpertLayoutError(f"layer {n}: down is {tuple(down.shape[1:])}, expected "
                                    f"({lay.hidden}, {lay.inter}) for a gate_up of "
                                    f"{2 * lay.inter} x {lay.hidden}")
        out.append(lay)
    if len({lay.n_experts for lay in out}) != 1:
        raise ExpertLayoutError("layers differ in their expert count")
    return out
