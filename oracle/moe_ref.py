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


def silu(v: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):  # exp(-v) -> inf for very negative v gives silu = -0, as on the GPU
        return v / (1 + np.exp(-v))


def sigmoid(v: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return 1 / (1 + np.exp(-v))


def expert_ffn(x: np.ndarray, gate_up_w: np.ndarray, down_w: np.ndarray, inter: int, dtype=np.float32,
               bf16_operands: bool = False, bf16_output: bool = False) -> np.ndarray:
    """down(silu(gate x) * (up x)) for x [n, hidden], with dequantized fused gate_up [2*inter, hidden] (gate rows
    first) and down [hidden, inter] (engines/base.py:99-102, :567-571). bf16_operands rounds x, the weights and
    the SwiGLU output to bf16 before each product, as a bf16 matmul of dequantized weights does
    (gguf/metal.py:407); bf16_output rounds the result to bf16 too, as that F.linear returns it."""
    if bf16_operands:
        x, gate_up_w, down_w = round_bf16(x), round_bf16(gate_up_w), round_bf16(down_w)
    gu = x.astype(dtype) @ gate_up_w.astype(dtype).T
    h = silu(gu[:, :inter]) * gu[:, inter:]
    if bf16_operands:
        h = round_bf16(h.astype(np.float32)).astype(dtype)
    out = h @ down_w.astype(dtype).T
    if bf16_output:
        out = round_bf16(out.astype(np.float32)).astype(dtype)
    return out


def layer(x: np.ndarray, lw: dict, dtype=np.float32, bf16_operands: bool = False, return_routing: bool = False,
          bf16_shared: bool = None, bf16_outputs: bool = False):
    """The whole MoE layer for x fp32 [T, hidden]; lw is a layer dict as synth.moe_layer builds it. Returns
    y [T, hidden] (in dtype), and with return_routing also (ids, weights, shared gate values). bf16_operands
    rounds the routed experts' operands to bf16 (expert_ffn); bf16_shared does the same for the shared expert
    (default: as bf16_operands). bf16_outputs also rounds each expert's output to bf16 (the shared expert's only
    with bf16_shared); the weighted sum stays fp32."""
    if bf16_shared is None:
        bf16_shared = bf16_operands
    hidden, inter, experts = lw["hidden"], lw["inter"], lw["experts"]
    x = np.ascontiguousarray(x, dtype=np.float32)
    logits = cref.router_logits(x, lw["router"], lw.get("router_bias"))
    weights, ids = route(logits, lw["top_k"], lw["norm_topk_prob"])
    y = np.zeros((x.shape[0], hidden), dtype=dtype)
    for expert in np.unique(ids):  # ascending, like each_expert's sorted combine (engines/base.py:580-589)
        token_idx, slot = np.nonzero(ids == expert)
        gate_up_w = dequantize_matrix(lw["gate_up"][expert], lw["gate_up_type"], 2 * inter, hidden)
        down_w = dequantize_matrix(lw["down"][expert], lw["down_type"], hidden, inter)
        h = expert_ffn(x[token_idx], gate_up_w, down_w, inter, dtype, bf16_operands, bf16_outputs)
        np.add.at(y, token_idx, h * weights[token_idx, slot, None].astype(dtype))
    shared_gate = None
    if lw.get("shared_gate_up") is not None:
        s_inter = lw["shared_inter"]
        gate_up_w = dequantize_matrix(lw["shared_gate_up"], lw["shared_gate_up_type"], 2 * s_inter, hidden)
        down_w = dequantize_matrix(lw["shared_down"], lw["shared_down_type"], hidden, s_inter)
        h = expert_ffn(x, gate_up_w, down_w, s_inter, dtype, bf16_shared, bf16_outputs and bf16_shared)
        if lw.get("shared_gate") is not None:
            z = cref.router_logits(x, lw["shared_gate"][None, :])[:, 0]
            shared_gate = sigmoid(z.astype(np.float32)).astype(np.float32)
            h = h * shared_gate[:, None].astype(dtype)
        y = y + h
    if return_routing:
        return y, ids, weights, shared_gate
    return y


def rel_err(y: np.ndarray, y_ref: np.ndarray) -> float:
    """Normwise error max|y - y_ref| / max|y_ref| (outputs of random weights cross zero, so elementwise relative
    error is not meaningful)."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    return float(np.max(np.abs(y - y_ref)) / max(np.max(np.abs(y_ref)), 1e-30))
