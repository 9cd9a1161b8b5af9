"""Seeded synthetic GGUF weights and inputs for the Qwen3.6-35B-A3B MoE-layer workloads (no real checkpoint is
available offline). Everything is drawn from numpy.random.default_rng(seed) in the field order written in each
docstring, so a given seed always gives the same bytes.

Block recipes (one block = 256 values):
  Q4_K (144 B): d, dmin = fp16(|N(0,1)| * 0.01); then 12 scale bytes, then 128 qs bytes, uniform 0..255.
  Q6_K (210 B): ql 128 B and qh 64 B uniform 0..255; 16 int8 scales uniform in [-32, 31]; d = fp16(|N(0,1)|*0.01).
Each recipe draws a field for all n blocks before the next field (d for every block, then dmin, ...).
"""
import numpy as np

BLOCK_BYTES = {"Q4_K": 144, "Q6_K": 210}
TYPE_IDS = {"Q4_K": 12, "Q6_K": 14}


def _f16_bytes(values: np.ndarray) -> np.ndarray:
    return values.astype(np.float16).view(np.uint8).reshape(-1, 2)


def q4_k_blocks(rng: np.random.Generator, n: int) -> np.ndarray:
    """[n, 144] uint8. Draw order: d [n], dmin [n], scales [n, 12], qs [n, 128]."""
    d = _f16_bytes(np.abs(rng.standard_normal(n)) * 0.01)
    dmin = _f16_bytes(np.abs(rng.standard_normal(n)) * 0.01)
    scales = rng.integers(0, 256, (n, 12), dtype=np.uint8)
    qs = rng.integers(0, 256, (n, 128), dtype=np.uint8)
    return np.concatenate((d, dmin, scales, qs), axis=1)


def q6_k_blocks(rng: np.random.Generator, n: int) -> np.ndarray:
    """[n, 210] uint8. Draw order: ql [n, 128], qh [n, 64], scales [n, 16], d [n]."""
    ql = rng.integers(0, 256, (n, 128), dtype=np.uint8)
    qh = rng.integers(0, 256, (n, 64), dtype=np.uint8)
    scales = rng.integers(-32, 32, (n, 16), dtype=np.int8).view(np.uint8)
    d = _f16_bytes(np.abs(rng.standard_normal(n)) * 0.01)
    return np.concatenate((ql, qh, scales, d), axis=1)


BLOCKS = {"Q4_K": q4_k_blocks, "Q6_K": q6_k_blocks}


def row_bytes(type_name: str, k: int) -> int:
    return k // 256 * BLOCK_BYTES[type_name]


def matrix(rng: np.random.Generator, type_name: str, rows: int, k: int, count: int = 1) -> np.ndarray:
    """`count` matrices [rows x k] of type_name as bytes: [count, rows, row_bytes] (or [rows, row_bytes] when
    count == 1), drawn as one run of count*rows*k/256 blocks."""
    blocks = BLOCKS[type_name](rng, count * rows * (k // 256))
    out = blocks.reshape(count, rows, row_bytes(type_name, k))
    return out[0] if count == 1 else out


def gemv_case(seed: int = 0, rows: int = 512, k: int = 2048, type_name: str = "Q4_K", tokens: int = 1):
    """One quantized GEMV (the 512x2048 Q4_K case is the reference's CPU-runnable single-matrix workload).
    Draw order: W, then x ~ N(0,1) fp32 [tokens, k]."""
    rng = np.random.default_rng(seed)
    w = matrix(rng, type_name, rows, k)
    x = rng.standard_normal((tokens, k)).astype(np.float32)
    return {"w": w, "x": x, "type": type_name, "rows": rows, "k": k}


def expert_case(seed: int = 0, hidden: int = 2048, inter: int = 512, tokens: int = 1):
    """One SwiGLU expert at batch `tokens`: gate, up Q4_K [inter x hidden], down Q6_K [hidden x inter].
    Draw order: gate, up, down, x ~ N(0,1) fp32 [tokens, hidden]."""
    rng = np.random.default_rng(seed)
    gate = matrix(rng, "Q4_K", inter, hidden)
    up = matrix(rng, "Q4_K", inter, hidden)
    down = matrix(rng, "Q6_K", hidden, inter)
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    return {"gate": gate, "up": up, "down": down, "x": x, "hidden": hidden, "inter": inter}


def zipf_bias(rng: np.random.Generator, experts: int, alpha: float = 1.1) -> np.ndarray:
    """Router bias making expert popularity Zipf(alpha)-shaped: expert perm[r] gets -alpha*log(r+1). The router
    product x.W (std ~0.9 for x ~ N(0,1), W ~ N(0, 0.02), hidden 2048) supplies the per-token noise."""
    perm = rng.permutation(experts)
    bias = np.empty(experts, dtype=np.float32)
    bias[perm] = (-alpha * np.log(np.arange(1, experts + 1))).astype(np.float32)
    return bias


def moe_layer(seed: int, hidden: int = 2048, inter: int = 512, shared_inter: int = 512, experts: int = 256,
              top_k: int = 8, gate_up_type: str = "Q4_K", down_type: str = "Q6_K", zipf_alpha: float = None):
    """One Qwen3.6-35B-A3B-shaped MoE layer. Draw order:
      router fp32 [experts, hidden] ~ N(0, 0.02);
      gate [experts x inter x hidden], up [experts x inter x hidden] (gate_up_type), each one run of blocks;
      down [experts x hidden x inter] (down_type);
      shared gate_proj [shared_inter x hidden], shared up_proj, shared down_proj [hidden x shared_inter];
      shared_expert_gate fp32 [hidden] ~ N(0, 0.02);
      then, with zipf_alpha, the router bias (zipf_bias).
    gate_up is stored fused per expert, gate rows then up rows (gguf/compiler.py:69-88)."""
    rng = np.random.default_rng(seed)
    router = (rng.standard_normal((experts, hidden)) * 0.02).astype(np.float32)
    gate = matrix(rng, gate_up_type, inter, hidden, count=experts).reshape(experts, inter, -1)
    up = matrix(rng, gate_up_type, inter, hidden, count=experts).reshape(experts, inter, -1)
    gate_up = np.concatenate((gate, up), axis=1)  # [E, 2*inter, row_bytes]
    del gate, up
    down = matrix(rng, down_type, hidden, inter, count=experts).reshape(experts, hidden, -1)
    s_gate = matrix(rng, gate_up_type, shared_inter, hidden)
    s_up = matrix(rng, gate_up_type, shared_inter, hidden)
    s_down = matrix(rng, down_type, hidden, shared_inter)
    shared_gate = (rng.standard_normal(hidden) * 0.02).astype(np.float32)
    bias = zipf_bias(rng, experts, zipf_alpha) if zipf_alpha else None
    return {
        "hidden": hidden, "inter": inter, "shared_inter": shared_inter, "experts": experts, "top_k": top_k,
        "norm_topk_prob": True, "gate_up_type": gate_up_type, "down_type": down_type,
        "shared_gate_up_type": gate_up_type, "shared_down_type": down_type,
        "router": router, "router_bias": bias, "gate_up": np.ascontiguousarray(gate_up),
        "down": np.ascontiguousarray(down), "shared_gate_up": np.concatenate((s_gate, s_up), axis=0),
        "shared_down": s_down, "shared_gate": shared_gate,
    }


def tokens(seed: int, count: int, hidden: int = 2048) -> np.ndarray:
    """x ~ N(0,1) fp32 [count, hidden] from its own generator."""
    return np.random.default_rng(seed).standard_normal((count, hidden)).astype(np.float32)


def write_moe_gguf(path: str, layers: list, arch: str = "qwen35moe", extra_metadata: dict = None,
                   alignment: int = 32):
    """A GGUF file holding the MoE blocks of `layers` (moe_layer dicts; every layer the same shape) under
    llama.cpp's tensor names: blk.N.ffn_{gate,up,down}_exps.weight stacked [experts, out, in], ffn_gate_inp.weight
    (router, F32 [experts, hidden]), ffn_gate_inp_shexp.weight (F32 [hidden]) and ffn_{gate,up,down}_shexp.weight,
    with the metadata keys the loader reads. Layers may differ in down type."""
    from .writer import write_gguf

    lw0 = layers[0]
    H, I, SI, E = lw0["hidden"], lw0["inter"], lw0["shared_inter"], lw0["experts"]
    metadata = {"general.architecture": arch, "general.alignment": alignment, f"{arch}.block_count": len(layers),
                f"{arch}.embedding_length": H, f"{arch}.expert_count": E, f"{arch}.expert_used_count": lw0["top_k"],
                f"{arch}.expert_feed_forward_length": I, f"{arch}.expert_shared_feed_forward_length": SI}
    metadata.update(extra_metadata or {})
    tensors = []
    for n, lw in enumerate(layers):
        gu, dt = lw["gate_up_type"], lw["down_type"]
        p = f"blk.{n}."
        tensors += [
            (p + "ffn_gate_inp.weight", "F32", (E, H), lw["router"]),
            (p + "ffn_gate_exps.weight", gu, (E, I, H), np.ascontiguousarray(lw["gate_up"][:, :I])),
            (p + "ffn_up_exps.weight", gu, (E, I, H), np.ascontiguousarray(lw["gate_up"][:, I:])),
            (p + "ffn_down_exps.weight", dt, (E, H, I), lw["down"]),
            (p + "ffn_gate_inp_shexp.weight", "F32", (H,), lw["shared_gate"]),
            (p + "ffn_gate_shexp.weight", lw["shared_gate_up_type"], (SI, H), lw["shared_gate_up"][:SI]),
            (p + "ffn_up_shexp.weight", lw["shared_gate_up_type"], (SI, H), lw["shared_gate_up"][SI:]),
            (p + "ffn_down_shexp.weight", lw["shared_down_type"], (H, SI), lw["shared_down"]),
        ]
    write_gguf(path, metadata, tensors, alignment=alignment)
