"""The fused MoE layer (wl_moe_layer): one call runs the router, top-k, token->expert grouping, the SwiGLU experts
and the weighted combine with the shared expert, all on the GPU with no host synchronization. This is
Engine.moe (engines/base.py:445-490) without its `.cpu()` dispatch (:456-460).
"""
import copy
import ctypes

import torch

from . import (MOE_FORCE_MFMA, MOE_GUESS_NEXT, MOE_NO_FUSED, MOE_NO_MFMA, MOE_PRE_NORM, MOE_RESIDUAL, TYPE_IDS,
               WlMoeLayer, _on_gpu, _stream, _type_id, check, library, row_bytes)


def _ptr(t):
    return None if t is None else t.data_ptr()


class MoELayer:
    """One MoE layer's weights in device memory and the call that runs it.

    gate_up: uint8 [n_experts, 2*inter * row_bytes(gate_up_type, hidden)], each expert's fused [gate | up] matrix
             (gate rows first, gguf/compiler.py:69-88); down: uint8 [n_experts, hidden * row_bytes(down_type,
             inter)]; router: fp32 [n_experts, hidden]; router_bias: fp32 [n_experts] or None; shared_gate_up,
             shared_down: the shared expert's matrices (or None); shared_gate: fp32 [hidden] or None.
    Tensors may be views into a larger store; each expert's bytes must be contiguous (a row of a 2-D tensor).
    pre_norm: run on the zero-centered RMSNorm of x (norm_weight fp32 [hidden] or None for 0, norm_eps), as the
    model calls the layer on rms_norm(x) (engines/qwen36/model.py:22, engines/base.py:27-31); residual: return
    x + MoE(...), the residual add of the same line. min_expert_weight: Engine.skip_small_experts
    (engines/base.py:413-430): routed experts below this routing weight are skipped (each token keeps its top one;
    the kept weights are scaled back to the sum of the k), 0 = off."""

    def __init__(self, *, gate_up, down, router, hidden: int, inter: int, n_experts: int, top_k: int,
                 norm_topk_prob: bool = True, gate_up_type: str = "Q4_K", down_type: str = "Q6_K",
                 router_bias=None, shared_gate_up=None, shared_down=None, shared_gate=None, shared_inter=None,
                 shared_gate_up_type=None, shared_down_type=None, fused: bool = True, mfma: str = "auto",
                 pre_norm: bool = False, norm_weight=None, norm_eps: float = 1e-6, residual: bool = False,
                 min_expert_weight: float = 0.0):
        for name, t in (("gate_up", gate_up), ("down", down), ("router", router)):
            _on_gpu(t, name)
        if router.dtype != torch.float32:
            raise ValueError("router weights must be fp32 [n_experts, hidden]")
        self.hidden, self.inter, self.n_experts, self.top_k = hidden, inter, n_experts, top_k
        self.norm_topk_prob = bool(norm_topk_prob)
        self.gate_up_type, self.down_type = gate_up_type, down_type
        self.shared_inter = shared_inter if shared_inter is not None else inter
        self.shared_gate_up_type = shared_gate_up_type or gate_up_type
        self.shared_down_type = shared_down_type or down_type
        gu_bytes = 2 * inter * row_bytes(gate_up_type, hidden)
        dn_bytes = hidden * row_bytes(down_type, inter)
        self.gate_up = gate_up.reshape(n_experts, -1)
        self.down = down.reshape(n_experts, -1)
        if self.gate_up.shape[1] < gu_bytes or self.down.shape[1] < dn_bytes:
            raise ValueError("expert tensors are smaller than their shapes need")
        self.router = router.contiguous()
        self.router_bias = None if router_bias is None else router_bias.to(torch.float32).contiguous()
        self.shared_gate_up = shared_gate_up
        self.shared_down = shared_down
        self.shared_gate = None if shared_gate is None else shared_gate.to(torch.float32).reshape(-1).contiguous()
        self.device = router.device
        self._ws = None
        s = WlMoeLayer()
        s.gate_up, s.down, s.router = self.gate_up.data_ptr(), self.down.data_ptr(), self.router.data_ptr()
        s.router_bias = _ptr(self.router_bias)
        s.shared_gate_up, s.shared_down = _ptr(shared_gate_up), _ptr(shared_down)
        s.shared_gate = _ptr(self.shared_gate)
        s.gate_up_stride = self.gate_up.stride(0) * self.gate_up.element_size()
        s.down_stride = self.down.stride(0) * self.down.element_size()
        s.gate_up_type, s.down_type = _type_id(gate_up_type), _type_id(down_type)
        s.shared_gate_up_type = TYPE_IDS.get(self.shared_gate_up_type, -1)
        s.shared_down_type = TYPE_IDS.get(self.shared_down_type, -1)
        s.hidden, s.inter, s.shared_inter = hidden, inter, self.shared_inter
        s.n_experts, s.top_k, s.norm_topk_prob = n_experts, top_k, int(self.norm_topk_prob)
        if mfma not in ("auto", "never", "always"):
            raise ValueError("mfma must be 'auto', 'never' or 'always'")
        s.flags = (0 if fused else MOE_NO_FUSED) | {"auto": 0, "never": MOE_NO_MFMA, "always": MOE_FORCE_MFMA}[mfma]
        self.norm_weight = None
        if pre_norm:
            s.flags |= MOE_PRE_NORM
            if norm_weight is not None:
                self.norm_weight = torch.as_tensor(norm_weight).to(device=self.device,
                                                                   dtype=torch.float32).reshape(-1).contiguous()
            s.norm_weight = _ptr(self.norm_weight)
            s.norm_eps = float(norm_eps)
        if residual:
            s.flags |= MOE_RESIDUAL
        s.min_expert_weight = float(min_expert_weight)
        self.min_expert_weight = float(min_expert_weight)
        self.struct = s
        check(library().wl_moe_check(ctypes.byref(s)))

    @classmethod
    def from_host(cls, lw: dict, device="cuda", fused: bool = True, mfma: str = "auto", **kw):
        """From a layer dict of numpy arrays (gguf.synth.moe_layer's layout), copied to the GPU; kw: pre_norm,
        norm_weight, norm_eps, residual."""
        def dev(a):
            return None if a is None else torch.from_numpy(a).to(device)
        return cls(gate_up=dev(lw["gate_up"].reshape(lw["experts"], -1)),
                   down=dev(lw["down"].reshape(lw["experts"], -1)), router=dev(lw["router"]),
                   router_bias=dev(lw.get("router_bias")), hidden=lw["hidden"], inter=lw["inter"],
                   n_experts=lw["experts"], top_k=lw["top_k"], norm_topk_prob=lw["norm_topk_prob"],
                   gate_up_type=lw["gate_up_type"], down_type=lw["down_type"],
                   shared_gate_up=dev(lw.get("shared_gate_up")), shared_down=dev(lw.get("shared_down")),
                   shared_gate=dev(lw.get("shared_gate")), shared_inter=lw.get("shared_inter"),
                   shared_gate_up_type=lw.get("shared_gate_up_type"), shared_down_type=lw.get("shared_down_type"),
                   fused=fused, mfma=mfma, **kw)

    def with_norm(self, norm_weight=None, norm_eps: float = 1e-6, residual: bool = True) -> "MoELayer":
        """The same weights as one decoder step's MoE half, x + MoE(rms_norm(x)) (engines/qwen36/model.py:22):
        a new layer object sharing this one's device tensors, with pre_norm set (and residual unless told not
        to). Its next layer is unset."""
        other = copy.copy(self)
        other._ws, other._next = None, None
        s = WlMoeLayer.from_buffer_copy(self.struct)
        s.next = None
        s.flags |= MOE_PRE_NORM | (MOE_RESIDUAL if residual else 0)
        other.norm_weight = None
        if norm_weight is not None:
            other.norm_weight = torch.as_tensor(norm_weight).to(device=self.device,
                                                                dtype=torch.float32).reshape(-1).contiguous()
        s.norm_weight = _ptr(other.norm_weight)
        s.norm_eps = float(norm_eps)
        other.struct = s
        check(library().wl_moe_check(ctypes.byref(s)))
        return other

    def set_min_expert_weight(self, w: float):
        """Engine.min_expert_weight for this layer's calls (0 = off); see the class docstring."""
        self.struct.min_expert_weight = float(w)
        check(library().wl_moe_check(ctypes.byref(self.struct)))
        self.min_expert_weight = float(w)

    def set_next(self, layer: "MoELayer" = None, guess: bool = False):
        """The layer the caller runs after this one (or None). With the same shapes, a batch-1 call pulls the rows
        that layer reads before its routing is known (router, shared expert) into the GPU's caches while this
        layer waits on its exchanges (WlMoeLayer.next). `layer` is kept alive by this one.
        guess: the caller runs `layer` on an input derived from this call's (the decoder loop, both layers with
        pre_norm): a batch-1 call then also guesses that layer's experts, the top-k of its router on its RMSNorm
        of this call's x, and pulls their gate_up rows into the caches (guess_next_layer's early read,
        engines/base.py:392-406,472-474). Results are the same either way."""
        self._next = layer
        self.struct.next = None if layer is None else ctypes.addressof(layer.struct)
        if guess and layer is not None:
            self.struct.flags |= MOE_GUESS_NEXT
        else:
            self.struct.flags &= ~MOE_GUESS_NEXT
        check(library().wl_moe_check(ctypes.byref(self.struct)))

    def workspace_bytes(self, tokens: int) -> int:
        return int(library().wl_moe_workspace_bytes(ctypes.byref(self.struct), tokens))

    def plan(self, tokens: int) -> str:
        """How a call with this many tokens runs: 'fused' (one persistent kernel, 1 token); 'gemv' (every expert on
        the fp32 GEMV kernels); 'split' (each expert by its own token count, as the reference's each_expert hands
        F.linear only that expert's tokens, engines/base.py:566-571, and GGMLWeight.linear switches at
        MAX_TOKENS = 8, gguf/metal.py:20,404-407: an expert with more than 8 tokens, and the shared expert, on the
        bf16 MFMA GEMMs, the rest on GEMV); 'mfma' (every expert on the MFMA GEMMs). mfma='never' / 'always' at
        construction pins 'gemv' / 'mfma'."""
        return {1: "fused", 0: "gemv", 2: "split", 3: "mfma"}[library().wl_moe_plan(ctypes.byref(self.struct),
                                                                                    tokens)]

    def workspace(self, tokens: int) -> torch.Tensor:
        need = self.workspace_bytes(tokens)
        if self._ws is None or self._ws.numel() < need:
            self._ws = new_workspace(need, self.device)
        return self._ws

    def _check_out(self, t, name, dtype, shape):
        if t is None:
            return
        if t.dtype != dtype or tuple(t.shape) != shape or not t.is_contiguous() or t.device != self.device:
            raise ValueError(f"{name} must be a contiguous {dtype} tensor of shape {list(shape)} on {self.device} "
                             f"(got {t.dtype} {list(t.shape)} on {t.device}"
                             f"{'' if t.is_contiguous() else ', not contiguous'})")

    def __call__(self, x: torch.Tensor, out: torch.Tensor = None, ids: torch.Tensor = None,
                 weights: torch.Tensor = None, workspace: torch.Tensor = None) -> torch.Tensor:
        """x [T, hidden] -> fp32 [T, hidden] (written into `out` when given). ids int32 / weights fp32 [T, top_k]
        receive the routing when given. Every given output must be contiguous, of its dtype and shape, on the
        layer's device; a workspace must be a uint8 device tensor of at least workspace_bytes(T) bytes prepared
        by new_workspace."""
        _on_gpu(x, "x")
        xf = x.reshape(-1, self.hidden).to(device=self.device, dtype=torch.float32).contiguous()
        tokens = xf.shape[0]
        self._check_out(out, "out", torch.float32, (tokens, self.hidden))
        self._check_out(ids, "ids", torch.int32, (tokens, self.top_k))
        self._check_out(weights, "weights", torch.float32, (tokens, self.top_k))
        y = out if out is not None else torch.empty(tokens, self.hidden, dtype=torch.float32, device=self.device)
        if workspace is not None and (workspace.dtype != torch.uint8 or workspace.device != self.device
                                      or not workspace.is_contiguous()):
            raise ValueError("workspace must be a contiguous uint8 tensor on the layer's device")
        ws = workspace if workspace is not None else self.workspace(tokens)
        check(library().wl_moe_layer(ctypes.byref(self.struct), xf.data_ptr(), tokens, y.data_ptr(), _ptr(ids),
                                     _ptr(weights), ws.data_ptr(), ws.numel(), _stream(self.device)))
        return y

    def call_noalloc(self, x: torch.Tensor, out: torch.Tensor, ids: torch.Tensor = None,
                     weights: torch.Tensor = None) -> torch.Tensor:
        """The layer through wl_moe_layer_noalloc: no workspace, nothing allocated by the library (its scratch is a
        device array of NOALLOC_SCRATCH_BYTES per GPU, shared by every such call on that GPU). x must already be a
        contiguous fp32 [T, hidden] device tensor and out is required, so this call allocates nothing either."""
        if x.dtype != torch.float32 or not x.is_contiguous() or x.device != self.device or x.dim() != 2:
            raise ValueError("x must be a contiguous fp32 [T, hidden] tensor on the layer's device")
        tokens = x.shape[0]
        self._check_out(out, "out", torch.float32, (tokens, self.hidden))
        self._check_out(ids, "ids", torch.int32, (tokens, self.top_k))
        self._check_out(weights, "weights", torch.float32, (tokens, self.top_k))
        check(library().wl_moe_layer_noalloc(ctypes.byref(self.struct), x.data_ptr(), tokens, out.data_ptr(),
                                             _ptr(ids), _ptr(weights), _stream(self.device)))
        return out

    def status(self, workspace: torch.Tensor = None) -> int:
        """wl_moe_workspace_status on `workspace` (default: this layer's own). Synchronizes the stream; returns 0,
        or -10 (ESYNC) when a bounded wait gave up since the previous query (a fused-kernel wait: those outputs
        hold NaN; a fork-scope hand-off: the scope's MFMA experts were skipped since)."""
        ws = workspace if workspace is not None else self._ws
        if ws is None:
            return 0
        return int(library().wl_moe_workspace_status(ws.data_ptr(), ws.numel(), _stream(self.device)))

    def status_noalloc(self) -> int:
        """wl_moe_workspace_status on the no-allocation entry point's scratch of this device."""
        return int(library().wl_moe_workspace_status(None, 0, _stream(self.device)))

    def route(self, x: torch.Tensor, return_logits: bool = False):
        """-> (weights fp32 [T, top_k], ids int32 [T, top_k], shared gate fp32 [T] or None): engines/base.py:91-97
        on the router logits, plus sigmoid(x . shared_gate); with return_logits also the logits fp32 [T, E]
        (bias included)."""
        xf = x.reshape(-1, self.hidden).to(torch.float32).contiguous()
        tokens = xf.shape[0]
        logits = torch.empty(tokens, self.n_experts, dtype=torch.float32, device=self.device)
        ids = torch.empty(tokens, self.top_k, dtype=torch.int32, device=self.device)
        weights = torch.empty(tokens, self.top_k, dtype=torch.float32, device=self.device)
        sg = None
        if self.shared_gate_up is not None and self.shared_gate is not None:
            sg = torch.empty(tokens, dtype=torch.float32, device=self.device)
        check(library().wl_moe_route(ctypes.byref(self.struct), xf.data_ptr(), tokens, logits.data_ptr(),
                                     ids.data_ptr(), weights.data_ptr(), _ptr(sg), _stream(self.device)))
        if return_logits:
            return weights, ids, sg, logits
        return weights, ids, sg


def new_workspace(nbytes: int, device) -> torch.Tensor:
    """A device workspace with its synchronization words zeroed (wl_moe_workspace_init), ready for any layer."""
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
    check(library().wl_moe_workspace_init(ws.data_ptr(), ws.numel(), _stream(ws.device)))
    return ws


def moe_layer(x: torch.Tensor, layer: MoELayer) -> torch.Tensor:
    """The whole layer in one call: y = MoE(x) as fp32."""
    return layer(x)
