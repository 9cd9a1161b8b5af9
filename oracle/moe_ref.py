"""Oracle (test infrastructure): the MoE layer on the CPU, restating the reference's dequantize-then-matmul path.

layer(): engines/base.py:445-490 (Engine.moe) with its general expert path (each_expert, :534-591: per expert,
the tokens that picked it, gate_up -> silu(gate) * up -> down, scaled by the routing weight and summed in
ascending expert order with index_add_) and the shared expert (:104-107, :481-489). Weights are dequantized with
quants_ref (gguf/quants.py) and multiplied in fp32 (numpy BLAS), or in float64 for high-precision checks.
Router logits come from cref.router_logits, the C replay of the GPU's fixed FMA order, so expert selection can be
compared exactly.
"""
import numpy as np

from . import cref
from .quants_ref import dequantize_matrix, round_bf16


def softmax_f32(logits: np.ndarray) -> np.ndarray:
    """F.softmax(logits, dim=-1, dtype=torch.float32) (engines/base.py:93)."""
    z = logits.astype(np.float32)
    e = np.exp(z - z.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def select_topk(logits: np.ndarray, top_k: int) -> np.ndarray:
    """Top-k expert ids per token, largest logit first, ties to the lower id. Softmax is monotone, so this is the
    same choice torch.topk makes on the probabilities (engines/base.py:94) wherever those are distinct."""
    order = np.argsort(-logits, axis=-1, kind="stable")
    return order[:, :top_k].astype(np.int32)


def route(logits: np.ndarray, top_k: int, normalize: bool):
    """engines/base.py:91-97 -> (weights fp32 [T, top_k], ids int32 [T, top_k])."""
    probs = softmax_f32(logits)
    ids = select_topk(logits, top_k)
    weights = np.take_along_axis(probs, ids.astype(np.int64), axis=-1)
    if normalize:
        weights = (weights / weights.sum(axis=-1, keepdims=True)).astype(np.float32)
    return weights.astype(np.float32), ids


def skip_small(weights: np.ndarray, ids: np.ndarray, min_weight: float):
    """engines/base.py:413-430 (Engine.skip_small_experts) on route()'s output, columns in pick order (largest weight
    first): keep = weight >= min_weight, and column 0 always; kept weights are scaled by S / K (S the sum of the k
    weights, K of the kept ones, each added left to right in pick order in float32; torch's .sum order is not
    specified, this is the order the kernels use); dropped columns get weight 0 and id -1. Returns (weights, ids)."""
    w = np.asarray(weights, dtype=np.float32)
    keep = w >= np.float32(min_weight)
    keep[:, 0] = True
    kept = np.where(keep, w, np.float32(0.0)).astype(np.float32)
    S = w[:, 0].copy()
    K = kept[:, 0].copy()
    for i in range(1, w.shape[1]):
        S = (S + w[:, i]).astype(np.float32)
        K = (K + kept[:, i]).astype(np.float32)
    scale = (S / K).astype(np.float32)
    out = np.where(keep, (kept * scale[:, None]).astype(np.float32), np.float32(0.0)).astype(np.float32)
    return out, np.where(keep, ids, -1).astype(np.int32)


def silu(v: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):  # exp(-v) -> inf for very negative v gives silu = -0, as on the GPU
        return v / (1 + np.exp(-v))


def sigmoid(v: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return 1 / (1 + np.exp(-v))


# Up to this many tokens F.linear on a quantized weight runs the exact-weight GEMV; above it, a bf16 matmul of the
# weight dequantized to bf16 (gguf/metal.py:20,404-407).
MAX_TOKENS = 8
CHAINS = ("fp32", "bf16", "split")


def expert_ffn(x: np.ndarray, gate_up_w: np.ndarray, down_w: np.ndarray, inter: int, dtype=np.float32,
               chain: str = "fp32") -> np.ndarray:
    """down(silu(gate x) * (up x)) for x [n, hidden], with dequantized fused gate_up [2*inter, hidden] (gate rows
    first) and down [hidden, inter] (engines/base.py:99-102, :567-571).

    chain "fp32": exact weights and fp32 activations throughout (the GEMV numerics at fp32 inputs).
    chain "bf16": the reference's prefill chain on bf16 tensors. x and the dequantized weights are rounded to bf16
    (gguf/metal.py:407; gguf/quants.py:223); each F.linear accumulates in fp32 and returns bf16 (the gate and up
    halves of gate_up's output, and down's output); F.silu(gate) returns bf16, and so does silu(gate) * up
    (engines/base.py:568-570)."""
    h = swiglu_hidden(x, gate_up_w, inter, dtype, chain)
    if chain == "fp32":
        return h @ down_w.astype(dtype).T
    return round_bf16(h.astype(dtype) @ round_bf16(down_w).astype(dtype).T).astype(dtype)


def swiglu_hidden(x: np.ndarray, gate_up_w: np.ndarray, inter: int, dtype=np.float32,
                  chain: str = "fp32") -> np.ndarray:
    """silu(gate x) * (up x), the input of an expert's down projection, in expert_ffn's chain."""
    if chain == "fp32":
        gu = x.astype(dtype) @ gate_up_w.astype(dtype).T
        return silu(gu[:, :inter]) * gu[:, inter:]
    if chain != "bf16":
        raise ValueError(f"chain must be 'fp32' or 'bf16', not {chain!r}")
    gu = round_bf16(round_bf16(x).astype(dtype) @ round_bf16(gate_up_w).astype(dtype).T)
    gate, up = gu[:, :inter], gu[:, inter:]
    return round_bf16(round_bf16(silu(gate)) * up)


def layer(x: np.ndarray, lw: dict, dtype=np.float32, chain: str = "fp32", return_routing: bool = False,
          shared_chain: str = None, counts=None, layer_tokens: int = None, min_expert_weight: float = 0.0):
    """The whole MoE layer for x fp32 [T, hidden]; lw is a layer dict as synth.moe_layer builds it. Returns
    y [T, hidden] (in dtype), and with return_routing also (ids, weights, shared gate values).

    chain picks each expert's numerics (expert_ffn): "fp32" or "bf16" for every expert, or "split", the
    reference's own rule: in each_expert an expert's F.linear receives only the tokens routed to it
    (engines/base.py:566-571), so an expert given more than MAX_TOKENS tokens takes the bf16 chain and the others
    the exact-weight fp32 one (gguf/metal.py:404-407); the shared expert sees all T tokens. shared_chain overrides
    the shared expert's (e.g. "fp32" for dense fp32 shared weights run by torch). The weighted sum over experts is
    fp32, in ascending expert order. For x a sample of a larger call's tokens, counts ([n_experts], each expert's
    tokens in the whole call) and layer_tokens (the call's token count) let "split" place the experts as that
    call does. min_expert_weight > 0: skip_small on the routing first, as Engine.moe applies it
    (engines/base.py:463-464); dropped picks (id -1) run no expert, and an expert's token count is its kept pairs."""
    if chain not in CHAINS:
        raise ValueError(f"chain must be one of {CHAINS}, not {chain!r}")

    def pick(n_tokens: int) -> str:
        if chain != "split":
            return chain
        return "bf16" if n_tokens > MAX_TOKENS else "fp32"

    hidden, inter, experts = lw["hidden"], lw["inter"], lw["experts"]
    x = np.ascontiguousarray(x, dtype=np.float32)
    logits = cref.router_logits(x, lw["router"], lw.get("router_bias"))
    weights, ids = route(logits, lw["top_k"], lw["norm_topk_prob"])
    if min_expert_weight > 0:
        weights, ids = skip_small(weights, ids, min_expert_weight)
    y = np.zeros((x.shape[0], hidden), dtype=dtype)
    for expert in np.unique(ids[ids >= 0]):  # ascending, like each_expert's sorted combine (engines/base.py:580-589)
        token_idx, slot = np.nonzero(ids == expert)
        gate_up_w = dequantize_matrix(lw["gate_up"][expert], lw["gate_up_type"], 2 * inter, hidden)
        down_w = dequantize_matrix(lw["down"][expert], lw["down_type"], hidden, inter)
        n_tok = len(token_idx) if counts is None else int(counts[expert])
        h = expert_ffn(x[token_idx], gate_up_w, down_w, inter, dtype, pick(n_tok))
        np.add.at(y, token_idx, h * weights[token_idx, slot, None].astype(dtype))
    shared_gate = None
    if lw.get("shared_gate_up") is not None:
        s_inter = lw["shared_inter"]
        gate_up_w = dequantize_matrix(lw["shared_gate_up"], lw["shared_gate_up_type"], 2 * s_inter, hidden)
        down_w = dequantize_matrix(lw["shared_down"], lw["shared_down_type"], hidden, s_inter)
        h = expert_ffn(x, gate_up_w, down_w, s_inter, dtype,
                       shared_chain or pick(x.shape[0] if layer_tokens is None else layer_tokens))
        if lw.get("shared_gate") is not None:
            z = cref.router_logits(x, lw["shared_gate"][None, :])[:, 0]
            shared_gate = sigmoid(z.astype(np.float32)).astype(np.float32)
            h = h * shared_gate[:, None].astype(dtype)
        y = y + h
    if return_routing:
        return y, ids, weights, shared_gate
    return y


def rms_norm(x: np.ndarray, weight=None, eps: float = 1e-6) -> np.ndarray:
    """engines/base.py:27-31 with zero_centered (x * rsqrt(mean(x^2) + eps) * (1 + w); Qwen3.5's norm,
    engines/qwen36/model.py:37) in the layer's fixed fp32 order: the sum of squares in the router's order
    (cref.router_logits of x with itself), then mean = s / H, inv = 1 / sqrt(mean + eps), x * inv * (1 + w), every
    step a correctly rounded float32 operation."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, H = x.shape
    ss = np.array([cref.router_logits(x[t:t + 1], x[t:t + 1])[0, 0] for t in range(T)], dtype=np.float32)
    mean = ss / np.float32(H)
    inv = np.float32(1.0) / np.sqrt(mean + np.float32(eps))
    out = x * inv[:, None]
    if weight is not None:
        out = out * (np.float32(1.0) + np.asarray(weight, dtype=np.float32))
    return out.astype(np.float32)


def topk_margins(logits: np.ndarray, top_k: int) -> np.ndarray:
    """Per token, the gap between its top_k-th and (top_k + 1)-th largest logit: how far the selection is from a
    tie (a gap of 0 is a tie, broken toward the lower expert id)."""
    part = -np.sort(-logits, axis=-1)
    return (part[:, top_k - 1] - part[:, top_k]).astype(np.float32)


def rel_err(y: np.ndarray, y_ref: np.ndarray) -> float:
    """Normwise error max|y - y_ref| / max|y_ref| (outputs of random weights cross zero, so elementwise relative
    error is not meaningful)."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    return float(np.max(np.abs(y - y_ref)) / max(np.max(np.abs(y_ref)), 1e-30))
