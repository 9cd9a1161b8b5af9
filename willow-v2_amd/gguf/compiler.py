"""Where every routed expert's bytes live in a GGUF model, from the header alone: the expert scan and the gate/up
fusion of gguf/compiler.py (EXPERT_RE, PART_ORDER, num_decoder_layers, scan_experts, fuse_gate_up;
gguf/compiler.py:13-88), with the same return values. The reference then copies the experts into an SSD pack
(compile_pack, build_converted_pack); here gguf/loader.py copies them straight into HBM instead, so nothing of the
pack format is kept.
"""
import re

from .reader import read_gguf  # noqa: F401  (the reference's module exposes it too)

PART_ORDER = ["gate", "up", "gate_up", "down"]

# llama.cpp stacks one layer's experts in one tensor, PyTorch shape [n_experts, out, in], quantized along `in`:
# blk.N.ffn_{gate,up,down}_exps.weight, or a fused blk.N.ffn_gate_up_exps.weight
EXPERT_RE = re.compile(r"^blk\.(\d+)\.ffn_(gate|up|down|gate_up)_exps\.weight$")


def num_decoder_layers(metadata: dict) -> int:
    """The layers the model runs: block_count less any multi-token-prediction layers stored after them
    (gguf/compiler.py:24-27)."""
    arch = metadata["general.architecture"]
    return metadata[f"{arch}.block_count"] - metadata.get(f"{arch}.nextn_predict_layers", 0)


def scan_experts(metadata: dict, tensors: dict):
    """(num_layers, num_experts, largest expert payload in bytes, plan, part_info) (gguf/compiler.py:29-67).
    plan[(layer, expert)] = [(part, path, offset, size), ...] in PART_ORDER; part_info["<layer>.<part>"] =
    {"shape": [out, in], "dtype": ggml type name}, per layer because quant types differ between layers.
    Expert e of a stacked tensor is its e-th equal slice (quant blocks never cross rows)."""
    num_layers = num_decoder_layers(metadata)
    plan, part_info = {}, {}
    for name, t in tensors.items():
        m = EXPERT_RE.match(name)
        if m is None:
            continue
        layer, part = int(m.group(1)), m.group(2)
        if layer >= num_layers:
            continue
        part_info[f"{layer}.{part}"] = {"shape": list(t.shape[1:]), "dtype": t.type}
        n = t.shape[0]
        size = t.nbytes // n
        for e in range(n):
            plan.setdefault((layer, e), []).append((part, t.path, t.offset + e * size, size))
    if not plan:
        raise SystemExit("No MoE expert tensors found (expected names like blk.N.ffn_gate_exps.weight)")
    layers = sorted({layer for layer, _ in plan})
    num_experts = 1 + max(e for _, e in plan)
    if layers != list(range(num_layers)):
        raise SystemExit(f"Expected experts in layers 0..{num_layers - 1}, found {layers[0]}..{layers[-1]} "
                         f"({len(layers)} layers); models with dense layers are not supported yet")
    for layer in layers:
        for e in range(num_experts):
            parts = sorted(plan.get((layer, e), []), key=lambda p: PART_ORDER.index(p[0]))
            names = [p[0] for p in parts]
            if names not in (["gate", "up", "down"], ["gate_up", "down"]):
                raise SystemExit(f"Expert {layer}_{e} has parts {names}, expected gate, up and down "
                                 "(or gate_up and down)")
            plan[(layer, e)] = parts
    max_payload = max(sum(p[3] for p in parts) for parts in plan.values())
    return num_layers, num_experts, max_payload, plan, part_info


def fuse_gate_up(plan: dict, part_info: dict):
    """Each layer's gate and up parts as one gate_up part, gate rows then up rows, where the two agree in shape
    and type (gguf/compiler.py:69-88); appending up's bytes to gate's is a valid [2 rows, k] tensor because quant
    blocks never cross rows. Returns (plan, part_info) with parts as (part, [(path, offset, size), ...])."""
    fused = set()
    for layer in {layer for layer, _ in plan}:
        gate, up = part_info.get(f"{layer}.gate"), part_info.get(f"{layer}.up")
        if gate and up and gate == up:
            fused.add(layer)
            part_info[f"{layer}.gate_up"] = {"shape": [2 * gate["shape"][0], gate["shape"][1]],
                                             "dtype": gate["dtype"]}
            del part_info[f"{layer}.gate"], part_info[f"{layer}.up"]
    out = {}
    for (layer, e), parts in plan.items():
        src = {part: (path, offset, size) for part, path, offset, size in parts}
        if layer in fused:
            out[(layer, e)] = [("gate_up", [src["gate"], src["up"]]), ("down", [src["down"]])]
        else:
            out[(layer, e)] = [(part, [s]) for part, s in src.items()]
    return out, part_info
