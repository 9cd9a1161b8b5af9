"""A Qwen3.6 GGUF model's MoE weights straight into HBM, still quantized.

The reference reads the header (gguf/reader.py), locates every expert (scan_experts / fuse_gate_up,
gguf/compiler.py:29-88), copies the experts into an SSD pack for streaming (compile_pack, gguf/compiler.py:90-197),
and dequantizes the other weights to bf16 in RAM (load_weights, engines/qwen36/loader.py:195-234). Here the experts
of every layer go from the file into one device tensor per layer and part (the HBMExpertStore layout: gate_up
[E, gate rows then up rows], down [E, rows]) with no pack in between, and the MoE block's other weights (router,
shared-expert gate, shared expert) are loaded under the Hugging Face names Engine.moe reads
(engines/qwen36/loader.py:37-41), the shared expert's quantized matrices as GGMLWeight views that stay quantized on
the GPU. Each layer keeps its own down type (Q4_K_M mixes Q6_K and Q4_K down layers, gguf/compiler.py:42-44).

File bytes are read with preadv into pinned staging buffers and copied to the device asynchronously, two buffers
in flight, so reading the file overlaps the host-to-device copies.
"""
import os

import numpy as np
import torch

from . import hip
from .compiler import fuse_gate_up, num_decoder_layers, scan_experts
from .hbm_store import HBMExpertStore, LayerExperts
from .reader import read_gguf

PREFIX = "model.language_model."  # Qwen35MoEEngine's weight-name prefix
# llama.cpp names of the MoE block's non-routed tensors -> Hugging Face names (engines/qwen36/loader.py:37-41)
MOE_LAYER_NAMES = {
    "ffn_gate_inp.weight": "mlp.gate.weight",
    "ffn_gate_inp_shexp.weight": "mlp.shared_expert_gate.weight",
    "ffn_gate_shexp.weight": "mlp.shared_expert.gate_proj.weight",
    "ffn_up_shexp.weight": "mlp.shared_expert.up_proj.weight",
    "ffn_down_shexp.weight": "mlp.shared_expert.down_proj.weight",
}
FP32_NAMES = ("mlp.gate.weight", "mlp.shared_expert_gate.weight")  # kept fp32 for the router matmul


def _header(model):
    """(metadata, tensors) from a path or from read_gguf's result."""
    return read_gguf(model) if isinstance(model, (str, os.PathLike)) else model


def moe_config(model) -> dict:
    """The MoE fields of the engine config, from the GGUF metadata (engines/qwen36/loader.py:58-77)."""
    metadata, _ = _header(model)
    arch = metadata["general.architecture"]

    def get(key, default=None):
        return metadata.get(f"{arch}.{key}", default)

    return {"num_hidden_layers": num_decoder_layers(metadata), "hidden_size": get("embedding_length"),
            "num_experts": get("expert_count"), "num_experts_per_tok": get("expert_used_count"),
            "norm_topk_prob": get("expert_weights_norm", True),
            "moe_intermediate_size": get("expert_feed_forward_length"),
            "shared_expert_intermediate_size": get("expert_shared_feed_forward_length")}


class _Stager:
    """File ranges -> device tensors through two pinned buffers of `chunk` bytes."""

    def __init__(self, device, chunk: int):
        self.device = torch.device(device)
        self.chunk = chunk
        self.bufs = [torch.empty(chunk, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        self.views = [memoryview(b.numpy()) for b in self.bufs]
        self.events = [None, None]
        self.turn = 0
        self.fds = {}
        self.bytes = 0

    def _fd(self, path):
        if path not in self.fds:
            self.fds[path] = os.open(path, os.O_RDONLY)
        return self.fds[path]

    def copy(self, path: str, offset: int, dst: torch.Tensor, row_bytes: int):
        """dst ([n, row_bytes] uint8 device view, rows may be strided) <- the n * row_bytes bytes at offset."""
        n = dst.shape[0]
        per = max(1, self.chunk // row_bytes)
        if row_bytes > self.chunk:
            raise ValueError(f"a {row_bytes}-byte row does not fit the {self.chunk}-byte staging buffer")
        fd = self._fd(path)
        for r0 in range(0, n, per):
            r1 = min(n, r0 + per)
            nbytes = (r1 - r0) * row_bytes
            i = self.turn
            self.turn ^= 1
            if self.events[i] is not None:
                self.events[i].synchronize()  # the buffer's previous copy has left it
            got = os.preadv(fd, [self.views[i][:nbytes]], offset + r0 * row_bytes)
            if got != nbytes:
                raise IOError(f"short read in {path}: {got} of {nbytes} bytes at {offset + r0 * row_bytes}")
            dst[r0:r1].copy_(self.bufs[i][:nbytes].view(r1 - r0, row_bytes), non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            self.events[i] = ev
            self.bytes += nbytes

    def close(self):
        for ev in self.events:
            if ev is not None:
                ev.synchronize()
        for fd in self.fds.values():
            os.close(fd)
        self.fds = {}


def _runs(sources_by_expert, part_index):
    """Split experts 0..E-1 into runs whose part_index source ranges are back to back in one file:
    [(e0, e1, path, offset, size)]. A stacked ffn_*_exps tensor is one run."""
    runs = []
    for e, sources in enumerate(sources_by_expert):
        path, offset, size = sources[part_index]
        if runs:
            e0, e1, p, o, s = runs[-1]
            if p == path and s == size and e == e1 and offset == o + (e1 - e0) * s:
                runs[-1] = (e0, e + 1, p, o, s)
                continue
        runs.append((e, e + 1, path, offset, size))
    return runs


def load_experts(model, device="cuda", chunk_bytes: int = 64 << 20) -> HBMExpertStore:
    """Every layer's routed experts in HBM: an HBMExpertStore whose layer l holds gate_up [E, gate rows then up
    rows] and down [E, rows] exactly as the file's blocks (gate and up fused per expert as fuse_gate_up plans it)."""
    metadata, tensors = _header(model)
    num_layers, num_experts, _, plan, part_info = scan_experts(metadata, tensors)
    plan, part_info = fuse_gate_up(plan, part_info)
    stager = _Stager(device, chunk_bytes)
    layers = []
    try:
        for layer in range(num_layers):
            gu, dn = part_info.get(f"{layer}.gate_up"), part_info[f"{layer}.down"]
            if gu is None:
                raise ValueError(f"layer {layer}: gate and up differ in shape or type "
                                 f"({part_info.get(f'{layer}.gate')} vs {part_info.get(f'{layer}.up')}); "
                                 "the expert kernels need them fused")
            parts = [dict(plan[(layer, e)]) for e in range(num_experts)]
            gu_src = [p["gate_up"] for p in parts]
            dn_src = [p["down"] for p in parts]
            gu_bytes = sum(s[2] for s in gu_src[0])
            dn_bytes = dn_src[0][0][2]
            gate_up = torch.empty(num_experts, gu_bytes, dtype=torch.uint8, device=device)
            down = torch.empty(num_experts, dn_bytes, dtype=torch.uint8, device=device)
            col = 0
            for j in range(len(gu_src[0])):  # gate, then up (or the one fused source)
                width = gu_src[0][j][2]
                for e0, e1, path, offset, size in _runs(gu_src, j):
                    stager.copy(path, offset, gate_up[e0:e1, col:col + width], size)
                col += width
            for e0, e1, path, offset, size in _runs(dn_src, 0):
                stager.copy(path, offset, down[e0:e1], size)
            inter, hidden = gu["shape"][0] // 2, gu["shape"][1]
            if dn["shape"] != [hidden, inter]:
                raise ValueError(f"layer {layer}: down has shape {dn['shape']}, expected {[hidden, inter]}")
            layers.append(LayerExperts(gate_up=gate_up, down=down, gate_up_type=gu["dtype"], down_type=dn["dtype"],
                                       hidden=hidden, inter=inter))
    finally:
        stager.close()
    store = HBMExpertStore(layers, device)
    store.loaded_bytes = stager.bytes
    return store


def _read(t) -> np.ndarray:
    return np.fromfile(t.path, dtype=np.uint8, count=t.nbytes, offset=t.offset)


def _dense(t) -> np.ndarray:
    """A float tensor's values as fp32 numpy, in its PyTorch shape."""
    raw = _read(t)
    if t.type == "F32":
        v = raw.view(np.float32)
    elif t.type == "F16":
        v = raw.view(np.float16).astype(np.float32)
    elif t.type == "BF16":
        v = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    else:
        raise ValueError(f"{t.name}: {t.type} is not a float type")
    return v.reshape(t.shape)


def load_moe_weights(model, device="cuda", prefix: str = PREFIX) -> dict:
    """The MoE blocks' non-routed weights under Engine.moe's names: router [E, hidden] and shared-expert gate
    [1, hidden] in fp32 (the engine keeps its routers out of lower precision, engines/qwen36/loader.py:50-52), the
    shared expert's gate/up/down as GGMLWeight when their type runs on the kernels (Q4_K, Q6_K), else dense bf16."""
    metadata, tensors = _header(model)
    weights = {}
    for layer in range(num_decoder_layers(metadata)):
        for gguf_name, hf_name in MOE_LAYER_NAMES.items():
            t = tensors.get(f"blk.{layer}.{gguf_name}")
            if t is None:
                continue
            name = f"{prefix}layers.{layer}.{hf_name}"
            if hf_name in FP32_NAMES:
                if t.type in hip.TYPES:  # a quantized router: its values, for the fp32 matmul
                    raw = torch.from_numpy(_read(t)).to(device)
                    v = hip.dequantize_gpu(raw, t.type, tuple(t.shape), torch.float32)
                else:
                    v = torch.from_numpy(np.ascontiguousarray(_dense(t))).to(device)
                # the shared-expert gate is stored as [hidden]; the engine's matmul takes [1, hidden]
                # (engines/qwen36/loader.py:128-129)
                weights[name] = v.reshape(1, -1) if v.dim() == 1 else v
            elif t.type in hip.TYPES:
                weights[name] = hip.GGMLWeight(torch.from_numpy(_read(t)).to(device), t.type, tuple(t.shape))
            else:
                weights[name] = torch.from_numpy(np.ascontiguousarray(_dense(t))).to(device=device,
                                                                                     dtype=torch.bfloat16)
    return weights


def load_moe(path: str, device="cuda"):
    """(config, expert store, non-routed weights) of a GGUF model's MoE blocks, read from one header parse."""
    header = read_gguf(path)
    return moe_config(header), load_experts(header, device), load_moe_weights(header, device)
