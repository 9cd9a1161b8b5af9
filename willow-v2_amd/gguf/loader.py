"""A Qwen3.6 GGUF model's MoE weights straight into HBM, still quantized.

The reference reads the header (gguf/reader.py), locates every expert (gguf/compiler.py:29-88), copies the
experts into an SSD pack for streaming (compile_pack, gguf/compiler.py:90-197),
and dequantizes the other weights to bf16 in RAM (load_weights, engines/qwen36/loader.py:195-234). Here the experts
of every layer go from the file into one device tensor per layer and part (the HBMExpertStore layout: gate_up
[E, gate rows then up rows], down [E, rows]) with no pack in between, and the MoE block's other weights (router,
shared-expert gate, shared expert) are loaded under the Hugging Face names Engine.moe reads
(engines/qwen36/loader.py:37-41), the shared expert's quantized matrices as GGMLWeight views that stay quantized on
the GPU. Each layer keeps its own down type (Q4_K_M mixes Q6_K and Q4_K down layers, gguf/compiler.py:42-44).

File bytes are read with preadv by several threads into a ring of pinned staging buffers and copied to the device
asynchronously, so reading the file overlaps the host-to-device copies.
"""
import os

import numpy as np
import torch

from . import hip
from .experts import decoder_layer_count, index_experts
from .hbm_store import HBMExpertStore, LayerExperts
from .reader import GGUFHeader, read_gguf

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
    """(metadata, tensors) from a path, a GGUFHeader or a (metadata, tensors) pair."""
    if isinstance(model, (str, os.PathLike)):
        model = read_gguf(os.fspath(model))
    if isinstance(model, GGUFHeader):
        return model.metadata, model.tensors
    return model


def moe_config(model) -> dict:
    """The MoE fields of the engine config, from the GGUF metadata (engines/qwen36/loader.py:58-77)."""
    metadata, _ = _header(model)
    arch = metadata["general.architecture"]

    def get(key, default=None):
        return metadata.get(f"{arch}.{key}", default)

    return {"num_hidden_layers": decoder_layer_count(metadata), "hidden_size": get("embedding_length"),
            "num_experts": get("expert_count"), "num_experts_per_tok": get("expert_used_count"),
            "norm_topk_prob": get("expert_weights_norm", True),
            "moe_intermediate_size": get("expert_feed_forward_length"),
            "shared_expert_intermediate_size": get("expert_shared_feed_forward_length")}


class _Stager:
    """File ranges -> device tensors through `depth` pinned buffers of `chunk` bytes: `threads` reader threads
    fill buffers with preadv (which runs without the GIL) while the main thread issues the host-to-device copies of
    the buffers already read, in order. A buffer is read into again only after its last copy has completed."""

    def __init__(self, device, chunk: int, depth: int = 8, threads: int = 8):
        self.device = torch.device(device)
        self.chunk = chunk
        self.bufs = [torch.empty(chunk, dtype=torch.uint8, pin_memory=True) for _ in range(depth)]
        self.views = [memoryview(b.numpy()) for b in self.bufs]
        self.events = [None] * depth
        self.threads = threads
        self.jobs = []
        self.fds = {}
        self.bytes = 0

    def _fd(self, path):
        if path not in self.fds:
            self.fds[path] = os.open(path, os.O_RDONLY)
        return self.fds[path]

    def add(self, dst: torch.Tensor, sources: list):
        """Queue dst ([n, W] contiguous uint8 device tensor) <- row i = the concatenation of the file ranges
        sources[i] = [(path, offset, size), ...] (sizes summing to W). Rows are staged a chunk of whole rows at a
        time; within a chunk, each column piece is read with one preadv per run of rows whose ranges lie back to
        back in the file, scattered straight into the rows' places in the staging buffer."""
        n, width = dst.shape
        if width > self.chunk:
            raise ValueError(f"a {width}-byte row does not fit the {self.chunk}-byte staging buffer")
        if sum(size for _, _, size in sources[0]) != width:
            raise ValueError(f"the pieces of a row do not add up to its {width} bytes")
        per = min(self.chunk // width, 512)  # 512 rows: within the kernel's limit on preadv buffers (IOV_MAX)
        for r0 in range(0, n, per):
            r1 = min(n, r0 + per)
            reads, col = [], 0
            for j, (_, _, size) in enumerate(sources[r0]):
                run = None
                for r in range(r0, r1):
                    path, offset, sz = sources[r][j]
                    if sz != size:
                        raise ValueError(f"row {r} piece {j} has {sz} bytes, row {r0} has {size}")
                    if run is not None and run[1] == path and run[2] + run[3] == offset:
                        run[3] += size
                        run[4].append((r - r0) * width + col)
                    else:
                        run = [self._fd(path), path, offset, size, [(r - r0) * width + col]]
                        reads.append(run)
                col += size
            self.jobs.append((reads, dst[r0:r1]))

    def _read(self, slot, reads):
        view = self.views[slot]
        for fd, path, offset, nbytes, places in reads:
            size = nbytes // len(places)
            got = os.preadv(fd, [view[p:p + size] for p in places], offset)
            if got != nbytes:
                raise IOError(f"short read in {path}: {got} of {nbytes} bytes at {offset}")

    def run(self):
        from collections import deque
        from concurrent.futures import ThreadPoolExecutor

        depth = len(self.bufs)
        pending = deque()

        def finish():
            slot, fut, dst = pending.popleft()
            fut.result()
            dst.copy_(self.bufs[slot][:dst.numel()].view(dst.shape), non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            self.events[slot] = ev
            self.bytes += dst.numel()

        with ThreadPoolExecutor(self.threads) as pool:
            for i, (reads, dst) in enumerate(self.jobs):
                slot = i % depth
                if len(pending) == depth:
                    finish()
                if self.events[slot] is not None:
                    self.events[slot].synchronize()  # the slot's previous copy has left it
                pending.append((slot, pool.submit(self._read, slot, reads), dst))
            while pending:
                finish()
        self.jobs = []

    def close(self):
        for ev in self.events:
            if ev is not None:
                ev.synchronize()
        for fd in self.fds.values():
            os.close(fd)
        self.fds = {}


def load_experts(model, device="cuda", chunk_bytes: int = 32 << 20, threads: int = 8) -> HBMExpertStore:
    """Every layer's routed experts in HBM: an HBMExpertStore whose layer l holds gate_up [E, gate rows then up
    rows] and down [E, rows], byte for byte the file's blocks."""
    metadata, tensors = _header(model)
    stager = _Stager(device, chunk_bytes, threads=threads)
    layers = []
    try:
        for lay in index_experts(metadata, tensors):
            E = lay.n_experts
            gate_up = torch.empty(E, lay.gate_up_bytes, dtype=torch.uint8, device=device)
            down = torch.empty(E, lay.down_bytes, dtype=torch.uint8, device=device)
            stager.add(gate_up, [lay.gate_up_ranges(e) for e in range(E)])
            stager.add(down, [[lay.down_range(e)] for e in range(E)])
            layers.append(LayerExperts(gate_up=gate_up, down=down, gate_up_type=lay.gate_up_type,
                                       down_type=lay.down_type, hidden=lay.hidden, inter=lay.inter))
        stager.run()
    finally:
        stager.close()
    store = HBMExpertStore(layers, device)
    store.loaded_bytes = stager.bytes
    return store


def _read(t) -> np.ndarray:
    return np.fromfile(t.file, dtype=np.uint8, count=t.nbytes, offset=t.offset)


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
    for layer in range(decoder_layer_count(metadata)):
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
