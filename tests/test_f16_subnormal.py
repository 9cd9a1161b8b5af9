"""The arithmetic behind the kernels' f16-subnormal products (CPU; no GPU needed).

The dequantizing kernels hand a quantized value q to `v_fma_mix_f32` as the f16 half whose exponent bits are zero
and whose mantissa holds q where it sits: a Q4_K low nibble (bits 0..3 of the half) is q * 2^-24, a high nibble
(bits 4..7) q * 2^-20, a Q6_K 6-bit value (bits 0..5) q * 2^-24. The block scale is multiplied by the inverse power
of two, so scale * value is the same exact product as before and every rounding that follows is the same. These
tests pin those facts on the CPU: the half values, the exactness of the scale products, and that a dot product in
fp32 scaled by a power of two rounds to the unscaled one scaled (for normal results).
"""
import numpy as np


def half(bits):
    return np.array(bits, dtype=np.uint16).view(np.float16).astype(np.float64)


def test_nibble_halves_are_exact_subnormals():
    q = np.arange(16)
    np.testing.assert_array_equal(half(q), q * 2.0 ** -24)          # low nibble in place
    np.testing.assert_array_equal(half(q << 4), q * 2.0 ** -20)     # high nibble in place
    q6 = np.arange(64)
    np.testing.assert_array_equal(half(q6), q6 * 2.0 ** -24)        # a Q6_K byte (6 bits)
    # the masks the kernels use pick exactly those fields out of a dword of four qs bytes
    rng = np.random.default_rng(0)
    w = rng.integers(0, 2 ** 32, 1000, dtype=np.uint64).astype(np.uint32)
    lo = (w & 0x000F000F).view(np.uint16).reshape(-1, 2)
    np.testing.assert_array_equal(lo[:, 0], w & 0xF)
    np.testing.assert_array_equal(lo[:, 1], (w >> 16) & 0xF)
    hi = (w & 0x00F000F0).view(np.uint16).reshape(-1, 2)
    np.testing.assert_array_equal(hi[:, 0] >> 4, (w >> 4) & 0xF)
    np.testing.assert_array_equal(hi[:, 1] >> 4, (w >> 20) & 0xF)
    assert ((hi & 0x7C00) == 0).all() and ((lo & 0x7C00) == 0).all()  # exponent bits zero: subnormal or zero


def test_scaled_scale_products_are_exact():
    """(d * 2^k) * sc and d * sc times 2^k agree bit for bit, d any finite f16 and sc a 6-bit (Q4_K) or signed
    8-bit (Q6_K) scale: the products have at most 19 significant bits and stay normal."""
    d = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)  # every non-negative finite f16
    for sc in (0, 1, 7, 33, 63, -128, 127):
        for k in (20, 24):
            a = (d * np.float32(2.0 ** k)) * np.float32(sc)
            b = (d * np.float32(sc)) * np.float32(2.0 ** k)
            np.testing.assert_array_equal(a, b)


def test_power_of_two_scaled_dot_rounds_the_same():
    """The per-lane dot in the kernels' order (two interleaved fp32 chains) on q 2^-24 equals the one on q, times
    2^-24, bit for bit, and the scale times 2^24 multiplies it back to the same float."""
    rng = np.random.default_rng(1)
    f32 = np.float32
    for _ in range(200):
        q = rng.integers(0, 16, 16).astype(np.float32)
        x = rng.standard_normal(16).astype(np.float32)
        a = f32(rng.integers(1, 64)) * f32(np.float16(rng.uniform(1e-3, 1e-1)))

        def chains(qv):
            s0, s1 = f32(0), f32(0)
            for i in range(0, 16, 4):
                # fma(q, x, s) with an exact product: q x has at most 4 + 24 bits, so f64 holds it exactly and one
                # rounding to f32 is the fused multiply-add's
                s0 = f32(np.float64(qv[i]) * np.float64(x[i]) + np.float64(s0))
                s1 = f32(np.float64(qv[i + 1]) * np.float64(x[i + 1]) + np.float64(s1))
                s0 = f32(np.float64(qv[i + 2]) * np.float64(x[i + 2]) + np.float64(s0))
                s1 = f32(np.float64(qv[i + 3]) * np.float64(x[i + 3]) + np.float64(s1))
            return f32(s0 + s1)

        plain = chains(q)
        scaled = chains((q * f32(2.0 ** -24)).astype(np.float32))
        assert scaled == f32(plain * f32(2.0 ** -24))
        assert f32(a * f32(2.0 ** 24)) * scaled == a * plain
