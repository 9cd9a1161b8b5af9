"""Oracle (test infrastructure): GGUF Q4_K / Q6_K block dequantization on the CPU, in numpy.

Two formulations of each type, which must agree bit for bit:
  dequant_q4_k / dequant_q6_k                 vectorized over whole blocks, following gguf/quants.py:73-116
  dequant_q4_k_chunks / dequant_q6_k_chunks   one 32-value chunk at a time, following gguf/metal.py:133-168
Every product in both is exact in fp32 (an fp16 scale times a 6-bit integer times a 4/6-bit integer fits in 24
bits), so the only rounding is Q4_K's final subtraction: results cannot depend on evaluation order or on fused
multiply-add, and a GPU dequantizer must reproduce them exactly.
"""
import numpy as np

QK_K = 256
# ggml type id -> (name, values per block, bytes per block), as gguf/reader.py:25,27 (Q4_K = 2+2+12+128,
# Q6_K = 128+64+16+2)
TYPE_IDS = {"Q4_K": 12, "Q6_K": 14}
BLOCK_SIZES = {"Q4_K": (QK_K, 144), "Q6_K": (QK_K, 210)}


def f16(raw2: np.ndarray) -> np.ndarray:
    """[n, 2] little-endian bytes -> [n, 1] float32 (gguf/quants.py:12-14)."""
    return np.ascontiguousarray(raw2).view(np.float16).astype(np.float32)


def k_scale_min(scales: np.ndarray):
    """[n, 12] packed bytes -> (scales [n, 8], mins [n, 8]) as float32: the 6-bit fields of Q4_K
    (gguf/quants.py:73-80). Bytes 0..3 hold sub-blocks 0..3's scales (low 6 bits) and the top 2 bits of 4..7's,
    bytes 4..7 the same for the mins, bytes 8..11 the low 4 bits of sub-blocks 4..7's scale (low nibble) and min
    (high nibble)."""
    s = scales.reshape(-1, 3, 4)
    d, m, m_d = s[:, 0], s[:, 1], s[:, 2]
    sc = np.concatenate((d & 0x3F, (m_d & 0x0F) | ((d >> 2) & 0x30)), axis=-1)
    mn = np.concatenate((m & 0x3F, (m_d >> 4) | ((m >> 2) & 0x30)), axis=-1)
    return sc.astype(np.float32), mn.astype(np.float32)


def q4_k_parts(b: np.ndarray):
    """Q4_K blocks [n, 144] -> (d*scale [n, 8], dmin*min [n, 8], nibbles [n, 8, 32]) (gguf/quants.py:82-88).
    qs byte 32g + l holds value 64g + l in its low nibble and 64g + 32 + l in its high nibble."""
    n = b.shape[0]
    d, dmin = f16(b[:, 0:2]), f16(b[:, 2:4])
    sc, mn = k_scale_min(b[:, 4:16])
    qs = b[:, 16:].reshape(n, 4, 1, 32)
    q = ((qs >> np.array([0, 4], dtype=np.uint8).reshape(1, 1, 2, 1)) & 0x0F).reshape(n, 8, 32)
    return d * sc, dmin * mn, q


def dequant_q4_k(b: np.ndarray) -> np.ndarray:
    """[n, 144] uint8 -> [n, 256] float32: value = (d*sc_j)*q - dmin*m_j (gguf/quants.py:90-92)."""
    scale, mn, q = q4_k_parts(b)
    return (scale[..., None] * q.astype(np.float32) - mn[..., None]).reshape(b.shape[0], QK_K)


def q6_k_parts(b: np.ndarray):
    """Q6_K blocks [n, 210] -> (d*scale [n, 16], signed 6-bit values [n, 16, 16]) (gguf/quants.py:104-112).
    Value 128h + 32t + c: low 4 bits from ql[64h + 32(t%2) + c] (shifted by 4 when t >= 2), high 2 bits from
    bits 2t..2t+1 of qh[32h + c], minus 32; scale = d * int8 scales[(128h + 32t + c) // 16]."""
    n = b.shape[0]
    ql, qh = b[:, :128], b[:, 128:192]
    scales = f16(b[:, 208:210]) * np.ascontiguousarray(b[:, 192:208]).view(np.int8).astype(np.float32)
    lo = ((ql.reshape(n, 2, 1, 64) >> np.array([0, 4], dtype=np.uint8).reshape(1, 1, 2, 1)) & 0x0F)
    lo = lo.reshape(n, 8, 32)
    hi = ((qh.reshape(n, 2, 1, 32) >> np.array([0, 2, 4, 6], dtype=np.uint8).reshape(1, 1, 4, 1)) & 3)
    hi = hi.reshape(n, 8, 32)
    q = (lo | (hi << 4)).astype(np.int8) - np.int8(32)
    return scales, q.reshape(n, 16, 16)


def dequant_q6_k(b: np.ndarray) -> np.ndarray:
    """[n, 210] uint8 -> [n, 256] float32 (gguf/quants.py:114-116)."""
    scales, q = q6_k_parts(b)
    return (scales[..., None] * q.astype(np.float32)).reshape(b.shape[0], QK_K)


def dequant_q4_k_chunks(b: np.ndarray) -> np.ndarray:
    """The same values as dequant_q4_k, computed one 32-value chunk (sub-block j) at a time with the scale/min
    unpacking written per sub-block, as gguf/metal.py:133-152 does (vectorized over blocks only)."""
    n = b.shape[0]
    out = np.empty((n, QK_K), dtype=np.float32)
    d, dmin = f16(b[:, 0:2])[:, 0], f16(b[:, 2:4])[:, 0]
    s = b[:, 4:16].astype(np.uint32)
    for j in range(8):
        if j < 4:
            sc, mn = s[:, j] & 63, s[:, j + 4] & 63
        else:
            sc = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 2) & 0x30)
            mn = (s[:, j + 4] >> 4) | ((s[:, j] >> 2) & 0x30)
        scale, m = d * sc.astype(np.float32), dmin * mn.astype(np.float32)
        qs = b[:, 16 + 32 * (j // 2):16 + 32 * (j // 2) + 32]
        q = ((qs >> (4 * (j % 2))) & 0xF).astype(np.float32)
        out[:, 32 * j:32 * j + 32] = scale[:, None] * q - m[:, None]
    return out


def dequant_q6_k_chunks(b: np.ndarray) -> np.ndarray:
    """The same values as dequant_q6_k, one 32-value chunk at a time as gguf/metal.py:154-168 does: chunk `sub`
    is half h = sub // 4, quarter s = sub % 4."""
    n = b.shape[0]
    out = np.empty((n, QK_K), dtype=np.float32)
    d = f16(b[:, 208:210])[:, 0]
    sc8 = np.ascontiguousarray(b[:, 192:208]).view(np.int8).astype(np.float32)
    for sub in range(8):
        h, s = sub // 4, sub % 4
        ql = b[:, 64 * h + 32 * (s % 2):64 * h + 32 * (s % 2) + 32].astype(np.int32)
        qh = b[:, 128 + 32 * h:128 + 32 * h + 32].astype(np.int32)
        q = (((ql >> (4 * (s // 2))) & 0xF) | (((qh >> (2 * s)) & 3) << 4)) - 32
        scale0, scale1 = d * sc8[:, 2 * sub], d * sc8[:, 2 * sub + 1]
        scale = np.concatenate((np.repeat(scale0[:, None], 16, 1), np.repeat(scale1[:, None], 16, 1)), axis=1)
        out[:, 32 * sub:32 * sub + 32] = scale * q.astype(np.float32)
    return out


DEQUANTIZERS = {"Q4_K": dequant_q4_k, "Q6_K": dequant_q6_k}
CHUNK_DEQUANTIZERS = {"Q4_K": dequant_q4_k_chunks, "Q6_K": dequant_q6_k_chunks}


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even, as torch's Tensor.to(torch.bfloat16)
    (used by gguf/quants.py:223). NaN becomes the quiet NaN 0x7FC0."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, np.uint16(0x7FC0), rounded)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(a: np.ndarray) -> np.ndarray:
    """float32 values rounded to bf16 and widened back to float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


def row_bytes(type_name: str, k: int) -> int:
    """gguf/metal.py:323-325."""
    elements, block_bytes = BLOCK_SIZES[type_name]
    return k // elements * block_bytes


def dequantize(raw, type_name: str, shape: tuple, dtype: str = "bf16") -> np.ndarray:
    """raw bytes of one [rows, k] tensor -> float32 values, or bf16 bit patterns (uint16) when dtype == "bf16"
    (the reference's default dtype, gguf/quants.py:207-227). Unsupported types raise NotImplementedError like
    gguf/quants.py:214-216."""
    if type_name not in DEQUANTIZERS:
        raise NotImplementedError(f"ggml type {type_name} is not supported (supported: Q4_K, Q6_K)")
    raw = np.frombuffer(raw, dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw.reshape(-1)
    elements, block_bytes = BLOCK_SIZES[type_name]
    blocks = raw.reshape(-1, block_bytes)
    assert blocks.shape[0] * elements == int(np.prod(shape)), (type_name, shape, raw.shape)
    values = DEQUANTIZERS[type_name](blocks).reshape(shape)
    return f32_to_bf16_bits(values) if dtype == "bf16" else values


def dequantize_matrix(raw: np.ndarray, type_name: str, rows: int, k: int) -> np.ndarray:
    """[rows, row_bytes] (or flat) bytes -> float32 [rows, k]."""
    return dequantize(np.ascontiguousarray(raw).reshape(-1), type_name, (rows, k), dtype="f32")
