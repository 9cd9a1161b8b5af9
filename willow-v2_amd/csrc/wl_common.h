// Device-side building blocks shared by the MoE-layer kernels (gfx950, wave64).
//
// Lane decomposition of a GGML K-quant block (256 values). Every kernel here gives one block to 8 consecutive
// lanes of a wavefront. Lane c (0..7) of the group owns 32 values as two runs of 16 consecutive values ("lo" and
// "hi"), so each lane reads one 16-byte slice of the packed values and its x operands are two 64-byte runs:
//   Q4_K (144 B: d f16 | dmin f16 | scales[12] | qs[128]), gguf/quants.py:73-92, gguf/metal.py:133-152:
//     lane c reads qs[16c .. 16c+15]. qs byte 32g + l holds value 64g + l (low nibble, sub-block 2g) and
//     64g + 32 + l (high nibble, sub-block 2g+1), so lo = values 64(c/2) + 16(c%2) + i, hi = lo + 32.
//     value = (d * sc_j) * q - dmin * m_j, with (sc_j, m_j) the 6-bit fields unpacked from scales[12].
//   Q6_K (210 B: ql[128] | qh[64] | int8 scales[16] | d f16), gguf/quants.py:104-116, gguf/metal.py:154-168:
//     value 128h + 32t + c' has its low 4 bits in ql[64h + 32(t%2) + c'] (high nibble when t >= 2) and its high
//     2 bits at bit 2t of qh[32h + c'], minus 32; scale = d * scales[value / 16].
//     Lane c reads ql[16c .. 16c+15] (h = c/4, t%2 = (c/2)%2, c' = 16(c%2) + i) and the matching 16 qh bytes, so
//     lo = values 128h + 32((c/2)%2) + 16(c%2) + i (low nibbles, t = (c/2)%2), hi = lo + 64 (high nibbles).
// Each run has one scale (Q6_K's scale covers 16 values), so a lane's dot product with x is
//     a_lo * sum(v_lo * x_lo) + b_lo * sum(x_lo) + a_hi * sum(v_hi * x_hi) + b_hi * sum(x_hi)
// with v the raw unsigned field (Q4_K nibble; Q6_K 6-bit value + 32), a the run's scale and b its offset
// (Q4_K: -dmin*m; Q6_K: -32*a).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/willow_hip.h"

namespace wl {

constexpr int kQK = 256;
constexpr int kWave = 64;
constexpr int kQ4KBytes = 144;
constexpr int kQ6KBytes = 210;

template <int TYPE>
struct BlockInfo;
template <>
struct BlockInfo<WL_TYPE_Q4_K> {
    static constexpr int bytes = kQ4KBytes;
    static constexpr int hi_offset = 32;  // hi run starts this many values after lo
    __device__ static constexpr int lo_start(int c) { return 64 * (c >> 1) + 16 * (c & 1); }
};
template <>
struct BlockInfo<WL_TYPE_Q6_K> {
    static constexpr int bytes = kQ6KBytes;
    static constexpr int hi_offset = 64;
    __device__ static constexpr int lo_start(int c) { return 128 * (c >> 2) + 32 * ((c >> 1) & 1) + 16 * (c & 1); }
};

__device__ __forceinline__ float half_to_float(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits & 0xFFFFu)));
}

// byte n of w as a float (v_cvt_f32_ubyteN)
__device__ __forceinline__ float ubyte(uint32_t w, int n) { return static_cast<float>((w >> (8 * n)) & 0xFFu); }

// Hides w's bits from the optimizer. Run words masked to one field per byte (w & 0x0F0F0F0F) through it, or the
// mask is folded into each byte's extraction (a v_bfe_u32 per value before v_cvt_f32_ubyte0) instead of staying
// one instruction per 4 values, with v_cvt_f32_ubyteN reading the bytes in place.
__device__ __forceinline__ uint32_t opaque(uint32_t w) {
    __asm__("" : "+v"(w));
    return w;
}

// 16 bytes from a 2-byte-aligned address, read as 5 aligned dwords and realigned with v_alignbyte. Every caller
// stays inside its 210-byte Q6_K block: the extra bytes read lie at most 2 before and 4 after the 16 wanted ones,
// and the ranges used (ql: block offsets 0..131, qh: 126..195) are inside the block.
// The aligned address is formed by subtracting from the byte pointer (not rebuilt from an integer), so the compiler
// keeps the pointer's global address space and emits global loads, not flat ones.
__device__ __forceinline__ const uint32_t* align_down4(const uint8_t* p, uint32_t& sh) {
    sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
    return reinterpret_cast<const uint32_t*>(p - sh);
}

__device__ __forceinline__ uint4 load16_a2(const uint8_t* p) {
    uint32_t sh;
    const uint32_t* q = align_down4(p, sh);
    const uint32_t w0 = q[0], w1 = q[1], w2 = q[2], w3 = q[3], w4 = q[4];
    uint4 r;
    r.x = __builtin_amdgcn_alignbyte(w1, w0, sh);
    r.y = __builtin_amdgcn_alignbyte(w2, w1, sh);
    r.z = __builtin_amdgcn_alignbyte(w3, w2, sh);
    r.w = __builtin_amdgcn_alignbyte(w4, w3, sh);
    return r;
}

// A lane's 32 values of one block: raw fields packed one per byte, and the per-run affine constants.
struct Lane32 {
    uint32_t lo[4], hi[4];
    float a_lo, a_hi, b_lo, b_hi;
};

// Q4_K's 6-bit scale and min of sub-block j, from the 12 scale bytes held as 3 dwords (s0 = bytes 0..3,
// s1 = 4..7, s2 = 8..11), as gguf/quants.py:73-80.
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t& sc,
                                              uint32_t& m) {
    if (j < 4) {
        const uint32_t sh = 8 * j;
        sc = (s0 >> sh) & 63u;
        m = (s1 >> sh) & 63u;
    } else {
        const uint32_t sh = 8 * (j - 4);
        const uint32_t lowbits = (s2 >> sh) & 0xFFu;
        sc = (lowbits & 0xFu) | (((s0 >> sh) >> 2) & 0x30u);
        m = (lowbits >> 4) | (((s1 >> sh) >> 2) & 0x30u);
    }
}

// Q4_K's scales and mins of the two sub-blocks j0 and j0 + 1 (j0 even) as bytes 0 and 1 of sc2 and m2: the 6-bit
// fields of gguf/quants.py:73-80 for both at once, with per-lane shifts instead of a branch on j0 < 4.
__device__ __forceinline__ void q4k_scale_min2(int j0, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t& sc2,
                                               uint32_t& m2) {
    const uint32_t sh = 8 * (j0 & 3);
    const bool upper = j0 >= 4;
    const uint32_t a = s0 >> sh, b = s1 >> sh, c = s2 >> sh;
    const uint32_t t = upper ? 2u : 0u;
    sc2 = ((upper ? c : a) & 0x0F0Fu) | ((a >> t) & 0x3030u);
    m2 = ((upper ? c >> 4 : b) & 0x0F0Fu) | ((b >> t) & 0x3030u);
}

// blk: 16-byte-aligned Q4_K block.
__device__ __forceinline__ void decode_q4k(const uint8_t* __restrict__ blk, int c, Lane32& o) {
    const uint4 hd = *reinterpret_cast<const uint4*>(blk);
    const uint4 qv = *reinterpret_cast<const uint4*>(blk + 16 + 16 * c);
    const float d = half_to_float(hd.x), dmin = half_to_float(hd.x >> 16);
    const int j0 = 2 * (c >> 1);
    uint32_t sc0, m0, sc1, m1;
    q4k_scale_min(j0, hd.y, hd.z, hd.w, sc0, m0);
    q4k_scale_min(j0 + 1, hd.y, hd.z, hd.w, sc1, m1);
    o.a_lo = d * static_cast<float>(sc0);
    o.b_lo = -(dmin * static_cast<float>(m0));
    o.a_hi = d * static_cast<float>(sc1);
    o.b_hi = -(dmin * static_cast<float>(m1));
    const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        o.lo[i] = opaque(q[i] & 0x0F0F0F0Fu);
        o.hi[i] = opaque((q[i] >> 4) & 0x0F0F0F0Fu);
    }
}

// blk: 2-byte-aligned Q6_K block (odd blocks of a row of 210-byte blocks start 2 bytes past a dword).
__device__ __forceinline__ void decode_q6k(const uint8_t* __restrict__ blk, int c, Lane32& o) {
    const int h = c >> 2, t0 = (c >> 1) & 1, half = c & 1;
    const uint4 ql = load16_a2(blk + 16 * c);
    const uint4 qh = load16_a2(blk + 128 + 32 * h + 16 * half);
    const float d = half_to_float(*reinterpret_cast<const uint16_t*>(blk + 208));
    const int lo_idx = 8 * h + 2 * t0 + half;
    const float s_lo = static_cast<float>(static_cast<int8_t>(blk[192 + lo_idx]));
    const float s_hi = static_cast<float>(static_cast<int8_t>(blk[192 + lo_idx + 4]));
    o.a_lo = d * s_lo;
    o.a_hi = d * s_hi;
    o.b_lo = -32.0f * o.a_lo;
    o.b_hi = -32.0f * o.a_hi;
    const uint32_t l4[4] = {ql.x, ql.y, ql.z, ql.w};
    const uint32_t h2[4] = {qh.x, qh.y, qh.z, qh.w};
    const uint32_t sh = 2 * t0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        o.lo[i] = opaque((l4[i] & 0x0F0F0F0Fu) | (((h2[i] >> sh) & 0x03030303u) << 4));
        o.hi[i] = opaque(((l4[i] >> 4) & 0x0F0F0F0Fu) | (((h2[i] >> (sh + 4)) & 0x03030303u) << 4));
    }
}

template <int TYPE>
__device__ __forceinline__ void decode(const uint8_t* __restrict__ blk, int c, Lane32& o) {
    if constexpr (TYPE == WL_TYPE_Q4_K)
        decode_q4k(blk, c, o);
    else
        decode_q6k(blk, c, o);
}

// decode() split in two: fetch() only issues the lane's loads (raw words kept as loaded), unpack() does the
// arithmetic later, so code placed between them does not wait for the loads. unpack(fetch(b)) == decode(b).
typedef _Float16 wl_f16x2 __attribute__((ext_vector_type(2)));

// dot16 of a Q4_K lane's run from its raw qs dwords q[4], scaled: each nibble is read in place as the mantissa of an
// f16 subnormal (exponent bits zero) and each product is a v_fma_mix_f32, which takes the f16 half directly, so no
// conversion instruction is spent per value. The low nibbles (bits 0..3 of a half: value q 2^-24) give the low
// run times 2^-24, the high nibbles (bits 4..7: q 2^-20) the high run times 2^-20. Every partial sum is dot16's
// times that power of two exactly (normal floats; power-of-two scaling rounds the same), so with the scale
// multiplied back (exact) the lane's sum is dot16's bit for bit.
template <bool HIGH>
__device__ __forceinline__ float dot16_q4mix(const uint32_t q[4], const float4 x[4]) {
    constexpr uint32_t m = HIGH ? 0x00F000F0u : 0x000F000Fu;
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const wl_f16x2 e = __builtin_bit_cast(wl_f16x2, q[i] & m);         // bytes 0, 2
        const wl_f16x2 o = __builtin_bit_cast(wl_f16x2, (q[i] >> 8) & m);  // bytes 1, 3
        s0 = __builtin_fmaf(static_cast<float>(e.x), x[i].x, s0);
        s1 = __builtin_fmaf(static_cast<float>(o.x), x[i].y, s1);
        s0 = __builtin_fmaf(static_cast<float>(e.y), x[i].z, s0);
        s1 = __builtin_fmaf(static_cast<float>(o.y), x[i].w, s1);
    }
    return s0 + s1;
}

template <int TYPE>
struct RawLane;
template <>
struct RawLane<WL_TYPE_Q4_K> {
    uint4 hd, qv;
    __device__ __forceinline__ void fetch(const uint8_t* __restrict__ blk, int c) {
        hd = *reinterpret_cast<const uint4*>(blk);
        qv = *reinterpret_cast<const uint4*>(blk + 16 + 16 * c);
    }
    __device__ __forceinline__ void unpack(int c, Lane32& o) const {
        const float d = half_to_float(hd.x), dmin = half_to_float(hd.x >> 16);
        uint32_t sc2, m2;
        q4k_scale_min2(2 * (c >> 1), hd.y, hd.z, hd.w, sc2, m2);
        o.a_lo = d * ubyte(sc2, 0);
        o.b_lo = -(dmin * ubyte(m2, 0));
        o.a_hi = d * ubyte(sc2, 1);
        o.b_hi = -(dmin * ubyte(m2, 1));
        const uint32_t q[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o.lo[i] = opaque(q[i] & 0x0F0F0F0Fu);
            o.hi[i] = opaque((q[i] >> 4) & 0x0F0F0F0Fu);
        }
    }
    // for lane_dot_q4mix: the raw qs dwords in lo, the low run's scale times 2^24, the high run's times 2^20
    __device__ __forceinline__ void unpack_mix(int c, Lane32& o) const {
        const float d = half_to_float(hd.x), dmin = half_to_float(hd.x >> 16);
        uint32_t sc2, m2;
        q4k_scale_min2(2 * (c >> 1), hd.y, hd.z, hd.w, sc2, m2);
        o.a_lo = (d * 16777216.0f) * ubyte(sc2, 0);
        o.b_lo = -(dmin * ubyte(m2, 0));
        o.a_hi = (d * 1048576.0f) * ubyte(sc2, 1);
        o.b_hi = -(dmin * ubyte(m2, 1));
        o.lo[0] = qv.x;
        o.lo[1] = qv.y;
        o.lo[2] = qv.z;
        o.lo[3] = qv.w;
    }
};

// lane_dot_s for a Q4_K lane unpacked by unpack_mix (the same bits)
__device__ __forceinline__ float lane_dot_q4mix(const Lane32& w, const float4 xl[4], const float4 xh[4], float sxl,
                                                float sxh) {
    return w.a_lo * dot16_q4mix<false>(w.lo, xl) + w.b_lo * sxl + w.a_hi * dot16_q4mix<true>(w.lo, xh) +
           w.b_hi * sxh;
}
template <>
struct RawLane<WL_TYPE_Q6_K> {
    uint32_t l[5], h[5];  // the aligned dwords around the lane's 16 ql and 16 qh bytes
    uint32_t lsh, hsh;    // their misalignment (0 or 2)
    uint32_t d16, s_lo, s_hi;
    __device__ __forceinline__ void fetch(const uint8_t* __restrict__ blk, int c) {
        const int hh = c >> 2, t0 = (c >> 1) & 1, half = c & 1;
        const uint32_t* ql = align_down4(blk + 16 * c, lsh);
        const uint32_t* qh = align_down4(blk + 128 + 32 * hh + 16 * half, hsh);
#pragma unroll
        for (int i = 0; i < 5; i++) {
            l[i] = ql[i];
            h[i] = qh[i];
        }
        d16 = *reinterpret_cast<const uint16_t*>(blk + 208);
        const int lo_idx = 8 * hh + 2 * t0 + half;
        s_lo = blk[192 + lo_idx];
        s_hi = blk[192 + lo_idx + 4];
    }
    __device__ __forceinline__ void unpack(int c, Lane32& o) const {
        const int t0 = (c >> 1) & 1;
        const float d = half_to_float(d16);
        o.a_lo = d * static_cast<float>(static_cast<int8_t>(s_lo));
        o.a_hi = d * static_cast<float>(static_cast<int8_t>(s_hi));
        o.b_lo = -32.0f * o.a_lo;
        o.b_hi = -32.0f * o.a_hi;
        const uint32_t sh = 2 * t0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t l4 = __builtin_amdgcn_alignbyte(l[i + 1], l[i], lsh);
            const uint32_t h2 = __builtin_amdgcn_alignbyte(h[i + 1], h[i], hsh);
            o.lo[i] = opaque((l4 & 0x0F0F0F0Fu) | (((h2 >> sh) & 0x03030303u) << 4));
            o.hi[i] = opaque(((l4 >> 4) & 0x0F0F0F0Fu) | (((h2 >> (sh + 4)) & 0x03030303u) << 4));
        }
    }
};

// The dequantized value of byte n of a run word: bit-exact with the CPU dequantizers (every product is exact,
// so the fused multiply-add rounds once, as the CPU's separate multiply and subtract do).
template <int TYPE>
__device__ __forceinline__ float dequant_value(uint32_t w, int n, float a, float b) {
    if constexpr (TYPE == WL_TYPE_Q4_K)
        return __builtin_fmaf(a, ubyte(w, n), b);
    else
        return a * static_cast<float>(static_cast<int>((w >> (8 * n)) & 0xFFu) - 32);
}

__device__ __forceinline__ float dot16(const uint32_t q[4], const float4 x[4]) {
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        s0 = __builtin_fmaf(ubyte(q[i], 0), x[i].x, s0);
        s1 = __builtin_fmaf(ubyte(q[i], 1), x[i].y, s1);
        s0 = __builtin_fmaf(ubyte(q[i], 2), x[i].z, s0);
        s1 = __builtin_fmaf(ubyte(q[i], 3), x[i].w, s1);
    }
    return s0 + s1;
}

__device__ __forceinline__ float sum16(const float4 x[4]) {
    float s0 = (x[0].x + x[0].y) + (x[0].z + x[0].w);
    float s1 = (x[1].x + x[1].y) + (x[1].z + x[1].w);
    float s2 = (x[2].x + x[2].y) + (x[2].z + x[2].w);
    float s3 = (x[3].x + x[3].y) + (x[3].z + x[3].w);
    return (s0 + s1) + (s2 + s3);
}

__device__ __forceinline__ void load_run(const float* __restrict__ p, float4 x[4]) {
    const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int i = 0; i < 4; i++) x[i] = q[i];
}

// One lane's share of a block's dot product with x (x_lo / x_hi: the lane's two 16-value runs of x).
__device__ __forceinline__ float lane_dot(const Lane32& w, const float4 xl[4], const float4 xh[4]) {
    return w.a_lo * dot16(w.lo, xl) + w.b_lo * sum16(xl) + w.a_hi * dot16(w.hi, xh) + w.b_hi * sum16(xh);
}

// Same with the run sums of x already known.
__device__ __forceinline__ float lane_dot_s(const Lane32& w, const float4 xl[4], const float4 xh[4], float sxl,
                                            float sxh) {
    return w.a_lo * dot16(w.lo, xl) + w.b_lo * sxl + w.a_hi * dot16(w.hi, xh) + w.b_hi * sxh;
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// v plus its partner's v across 16-lane rows (XOR 16: ROWS = 16) or wavefront halves (XOR 32: ROWS = 32), in one
// VALU swap: v_permlane16_swap / v_permlane32_swap with both operands v give every lane its own v and its
// partner's, one in each result, and their sum (addition commutes exactly) is v + v[lane ^ ROWS] bit for bit, with
// no trip through the LDS crossbar that a shuffle takes.
template <int ROWS>
__device__ __forceinline__ float swap_add(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = ROWS == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                              : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, static_cast<uint32_t>(r[0])) +
           __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
}

// Sum over aligned groups of WIDTH lanes (2..64); every lane of a group gets the same bits. Must be called with
// the whole wavefront active.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp<0xB1>(v);                      // quad_perm [1,0,3,2]: lane ^ 1
    if constexpr (WIDTH >= 4) v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
    if constexpr (WIDTH >= 8) v += dpp<0x141>(v);  // row_half_mirror: the other quad of the 8
    if constexpr (WIDTH >= 16) v += dpp<0x140>(v); // row_mirror: the other 8 of the 16
    if constexpr (WIDTH >= 32) v = swap_add<16>(v);
    if constexpr (WIDTH >= 64) v = swap_add<32>(v);
    return v;
}

// GEMV geometry: a wavefront's 8 lane groups take 8 blocks. With nb = k/256 blocks per row:
//   nb in {1, 2, 4}: the wave covers R = 8/nb whole rows at once (group g: row g/nb, block g%nb), and each row's
//                    partial sums are reduced over its `width` = 8*nb lanes;
//   otherwise:       one row per wave, group g takes blocks g, g+8, ...; reduction over all 64 lanes.
struct RowGeom {
    int R, width;
};
__host__ __device__ inline RowGeom row_geom(int nb) {
    if (nb < 8 && (nb & (nb - 1)) == 0) return {8 / nb, 8 * nb};
    return {1, 64};
}
__host__ __device__ inline int row_geom_width(int nb) { return row_geom(nb).width; }

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }
__device__ __forceinline__ float sigmoid(float z) { return 1.0f / (1.0f + expf(-z)); }

// bf16 bits of f, round to nearest even (torch's conversion); NaN -> 0x7FC0.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

}  // namespace wl
