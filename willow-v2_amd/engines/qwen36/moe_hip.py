"""Engine.moe on the HIP backend, as a mixin for willow's engines (engines/base.py:445-490).

Put HipMoE ahead of the reference's Engine in an engine's bases and give the engine an HBMExpertStore as its
`experts`:

    class Qwen35MoEEngineHip(HipMoE, Qwen35MoEEngine): ...

moe(x, layer, residual) keeps the layer API called at engines/qwen36/model.py:22: x [T, hidden] on the engine's
device in, the same shape and dtype out. It reads the same attributes and weight names as the reference
(self.prefix, self.top_k, self.norm_topk_prob; <prefix>layers.N.mlp.{gate, shared_expert.{gate,up,down}_proj,
shared_expert_gate}.weight; engines/base.py:285-286,446,481-485) and runs the router, top-k, grouping, experts and
combine on the GPU in one call: no `selected.cpu()` wait per layer (engines/base.py:456-460) and no per-expert
launches. In place of guess_next_layer (engines/base.py:392-406), which guesses the next layer's experts to start
their SSD reads, each layer's view names the next layer, and a batch-1 call pulls the next layer's router and
shared-expert rows (read before its routing is known) into the GPU's caches while it waits on its own exchanges.

Batched decode: a runner may wrap one decode step's layers (attention included) in `with engine.moe_step():`, a
fork scope of the library (gguf.hip.fork_scope): the layers' experts given more than 8 tokens then meet the rest
through the workspace instead of a fork and a join per layer (64 tokens, Zipf routing: ~10 us per layer). The
step's calls must come from one thread, in order, on the current stream.

Shared expert: when its three matrices are GGMLWeight (kept quantized), they run inside the fused kernel; when
they are dense tensors (the reference's loader dequantizes them to bf16, engines/qwen36/loader.py:224), the
routed part runs fused and the shared expert is added with the reference's own formula (engines/base.py:104-107).
Arithmetic is fp32 inside the kernel; the result is cast back to x's dtype.
"""
import contextlib

import torch
import torch.nn.functional as F

from gguf.hip import ESYNC, GGMLWeight, HipError, fork_scope, library


def dense_shared_expert(x, gate_w, up_w, down_w, shared_gate_w):
    """engines/base.py:104-107."""
    h = F.linear(F.silu(F.linear(x, gate_w)) * F.linear(x, up_w), down_w)
    return torch.sigmoid(F.linear(x, shared_gate_w)) * h


class HipMoE:
    """Mixin replacing Engine.moe with the fused device-side MoE layer."""

    def hip_layer(self, layer: int):
        """(MoELayer, dense shared-expert weights or None), built once per layer from the engine's weights."""
        cache = self.__dict__.setdefault("_hip_moe_layers", {})
        if layer in cache:
            return cache[layer]
        p = f"{self.prefix}layers.{layer}.mlp"
        device = self.experts.device
        router = self.weights[p + ".gate.weight"].to(device=device, dtype=torch.float32).contiguous()
        bias = self.weights.get(p + ".gate.bias")
        if bias is not None:
            bias = bias.to(device=device, dtype=torch.float32).contiguous()
        sp = p + ".shared_expert"
        names = (sp + ".gate_proj.weight", sp + ".up_proj.weight", sp + ".down_proj.weight")
        shared = {}
        dense = None
        if all(n in self.weights for n in names):
            gate_w, up_w, down_w = (self.weights[n] for n in names)
            gate_g = self.weights.get(p + ".shared_expert_gate.weight")
            quantized = (isinstance(gate_w, GGMLWeight) and isinstance(up_w, GGMLWeight)
                         and isinstance(down_w, GGMLWeight) and gate_w.type_name == up_w.type_name)
            if quantized:
                for w in (gate_w, up_w, down_w):
                    w.to_gpu()
                # fused [gate | up] bytes, as the expert pack fuses them (gguf/compiler.py:69-88)
                shared = dict(shared_gate_up=torch.cat((gate_w.raw.reshape(-1), up_w.raw.reshape(-1))).to(device),
                              shared_down=down_w.raw.reshape(-1).to(device), shared_inter=gate_w.shape[0],
                              shared_gate_up_type=gate_w.type_name, shared_down_type=down_w.type_name,
                              shared_gate=None if gate_g is None else
                              gate_g.to(device=device, dtype=torch.float32).reshape(-1).contiguous())
            else:
                dense = (gate_w, up_w, down_w, gate_g)
        view = self.experts.layer_view(layer, router, self.top_k, self.norm_topk_prob, router_bias=bias, **shared)
        cache[layer] = (view, dense)
        return cache[layer]

    @contextlib.contextmanager
    def moe_step(self):
        """A context for one decode step's layers: the library's fork scope on the experts' device. On leaving it,
        every layer's workspace status is read (one stream synchronization), and a bounded wait that gave up inside
        the step (the MFMA experts of a hand-off skipped, or a fused-kernel exchange: outputs NaN) raises HipError,
        so such outputs never pass into the residual stream unnoticed."""
        with fork_scope(self.experts.device):
            yield
        self.check_moe_status()

    def check_moe_status(self):
        """Raises HipError (code ESYNC) when a bounded wait of any built layer gave up since the last check."""
        for layer, (view, _) in sorted(self.__dict__.get("_hip_moe_layers", {}).items()):
            if view.status() == ESYNC:
                raise HipError(ESYNC, f"layer {layer}: " + library().wl_error_string(ESYNC).decode())

    def moe(self, x: torch.Tensor, layer: int, residual: torch.Tensor = None) -> torch.Tensor:
        view, dense = self.hip_layer(layer)
        min_w = float(getattr(self, "min_expert_weight", 0.0) or 0.0)
        if view.min_expert_weight != min_w:
            # Engine.skip_small_experts (engines/base.py:413-430), applied in the layer as Engine.moe does (:463-464)
            view.set_min_expert_weight(min_w)
        nxt = layer + 1
        if getattr(view, "_next", None) is None and nxt < len(getattr(self.experts, "layers", ())):
            # the next layer's router and shared-expert rows are pulled into the caches during this layer
            # (the overlap guess_next_layer gives the reference's SSD reads, engines/base.py:392-406)
            view.set_next(self.hip_layer(nxt)[0])
        flat = x.reshape(-1, x.shape[-1])
        out = view(flat.to(view.device))
        if dense is not None:
            gate_w, up_w, down_w, gate_g = dense
            out = out + dense_shared_expert(flat.to(gate_w.dtype), gate_w, up_w, down_w, gate_g).float()
        if getattr(self, "moe_check_status", False):  # debug: read the status after every layer (a sync each)
            self.check_moe_status()
        return out.to(device=x.device, dtype=x.dtype).view_as(x)
