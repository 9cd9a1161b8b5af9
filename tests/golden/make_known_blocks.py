"""Writes known_blocks.npz: hand-built Q4_K / Q6_K blocks and their values, computed from the block format's
definition written out per value (not by any dequantizer), so the oracle and the GPU kernels are checked against
an independent statement of the format.

Q4_K value i of a block (sub-block j = i // 32, l = i % 32):
    q = (qs[32*(j//2) + l] >> (4*(j%2))) & 15;   value = d*sc_j*q - dmin*m_j
  where the 6-bit (sc_j, m_j) are packed ggml-style into 12 bytes:
    j < 4:  s[j] low 6 bits = sc_j, s[j+4] low 6 bits = m_j
    j >= 4: s[j+4] = (sc_j & 15) | ((m_j & 15) << 4); the top 2 bits of sc_j sit in bits 6-7 of s[j-4], of m_j in
            bits 6-7 of s[j]
Q6_K value i (h = i // 128, t = (i % 128) // 32, c = i % 32):
    q = ((ql[64h + 32(t%2) + c] >> (4*(t//2))) & 15) | (((qh[32h + c] >> (2t)) & 3) << 4);  value = d*sc[i//16]*(q-32)
All chosen scales are small integers and d, dmin powers of two, so every value is exact in float32.

    python tests/golden/make_known_blocks.py
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f16_bytes(v: float) -> list:
    return list(np.array([v], dtype=np.float16).view(np.uint8))


def pack_q4_k_scales(sc, mn) -> list:
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return s


def q4_k_block(d, dmin, sc, mn, qs):
    raw = bytes(f16_bytes(d) + f16_bytes(dmin) + pack_q4_k_scales(sc, mn) + list(qs))
    values = []
    for i in range(256):
        j, l = divmod(i, 32)
        q = (qs[32 * (j // 2) + l] >> (4 * (j % 2))) & 15
        values.append(d * sc[j] * q - dmin * mn[j])
    return np.frombuffer(raw, dtype=np.uint8), np.array(values, dtype=np.float64)


def q6_k_block(d, scales, ql, qh):
    raw = bytes(list(ql) + list(qh) + list(np.array(scales, dtype=np.int8).view(np.uint8)) + f16_bytes(d))
    values = []
    for i in range(256):
        h, rem = divmod(i, 128)
        t, c = divmod(rem, 32)
        q = ((ql[64 * h + 32 * (t % 2) + c] >> (4 * (t // 2))) & 15) | (((qh[32 * h + c] >> (2 * t)) & 3) << 4)
        values.append(d * scales[i // 16] * (q - 32))
    return np.frombuffer(raw, dtype=np.uint8), np.array(values, dtype=np.float64)


def main():
    sc = [63, 1, 32, 17, 48, 5, 33, 60]  # values >= 16 in sub-blocks 4..7 exercise the split high bits
    mn = [0, 63, 15, 40, 21, 62, 7, 44]
    pattern = [(7 * b + 3) & 255 for b in range(128)]
    q4 = [
        q4_k_block(0.0, 0.0, [0] * 8, [0] * 8, [0] * 128),          # all zero
        q4_k_block(1.0, 0.5, sc, mn, [0] * 128),                    # q = 0: -dmin*m_j
        q4_k_block(0.25, 0.125, sc, mn, [255] * 128),               # q = 15: 15*d*sc_j - dmin*m_j
        q4_k_block(2.0 ** -6, 2.0 ** -9, sc, mn, pattern),          # every nibble position distinct
        q4_k_block(2.0 ** -24, 2.0 ** -20, sc[::-1], mn[::-1], pattern[::-1]),  # fp16 subnormal d
    ]
    s6 = [-32, -1, 0, 1, 31, 7, -8, 15, -17, 2, 30, -31, 5, -5, 12, -12]
    ql_pat = [(5 * i + 1) & 255 for i in range(128)]
    qh_pat = [(3 * i + 2) & 255 for i in range(64)]
    q6 = [
        q6_k_block(0.25, s6, [0] * 128, [0] * 64),                  # q = -32: -32*d*sc
        q6_k_block(0.5, s6, [255] * 128, [255] * 64),               # q = 31: 31*d*sc
        q6_k_block(2.0 ** -7, s6, ql_pat, qh_pat),                  # every field position distinct
        q6_k_block(-2.0 ** -5, s6[::-1], ql_pat[::-1], qh_pat[::-1]),  # negative d
    ]
    out = {
        "q4_k_blocks": np.stack([b for b, _ in q4]), "q4_k_values": np.stack([v for _, v in q4]).astype(np.float32),
        "q6_k_blocks": np.stack([b for b, _ in q6]), "q6_k_values": np.stack([v for _, v in q6]).astype(np.float32),
    }
    for name in ("q4_k", "q6_k"):  # every value is exact in float32
        assert np.array_equal(out[name + "_values"].astype(np.float64), np.stack([v for _, v in (q4 if name == "q4_k" else q6)]))
    np.savez(os.path.join(HERE, "known_blocks.npz"), **out)
    print("wrote", os.path.join(HERE, "known_blocks.npz"))


if __name__ == "__main__":
    main()
