/*
 * Oracle (test infrastructure, never the product): plain-C restatements used to check the GPU kernels.
 *
 *  - oracle_router_logits: the router's x . W_r^T in the exact floating-point order the GPU router kernels use,
 *    so expert selection can be compared bit for bit (engines/base.py:448 computes these logits with F.linear,
 *    whose summation order is unspecified; the order fixed here is the library's documented one):
 *        for each (token t, expert e):
 *            for each segment s of 64 consecutive k (s = 0 .. H/64-1):
 *                p_s = 0; for k in segment, ascending: p_s = fmaf(x[t,k], W[e,k], p_s)
 *            total = p_0 + p_1 + ... + p_{S-1}   (left to right)
 *            logit = total + bias[e]             (when a bias is given)
 *  - oracle_dequant_q4_k_scalar / oracle_dequant_q6_k_scalar: one value at a time, restating the scalar
 *    per-chunk Metal decoders (gguf/metal.py:24-28 f16_at, :133-152 deq_Q4_K, :154-168 deq_Q6_K) with the fp16
 *    decode written out by hand, a third formulation beside the two numpy ones.
 *
 * Build: gcc -O2 -fPIC -shared -ffp-contract=off oracle_ref.c -o build/liboracle_ref.so -lm
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define ORACLE_ROUTER_SEGMENT 64

static float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t man = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalize */
            int e = -1;
            do {
                e++;
                man <<= 1;
            } while ((man & 0x400) == 0);
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3FF) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float f16_at(const uint8_t* p) { return half_to_float((uint16_t)(p[0] | (p[1] << 8))); }

void oracle_router_logits(const float* x, const float* w, const float* bias, int64_t tokens, int64_t hidden,
                          int64_t experts, float* out) {
    const int64_t segments = hidden / ORACLE_ROUTER_SEGMENT;
    for (int64_t t = 0; t < tokens; t++) {
        const float* xt = x + t * hidden;
        for (int64_t e = 0; e < experts; e++) {
            const float* we = w + e * hidden;
            float total = 0.0f;
            for (int64_t s = 0; s < segments; s++) {
                float p = 0.0f;
                for (int64_t k = ORACLE_ROUTER_SEGMENT * s; k < ORACLE_ROUTER_SEGMENT * (s + 1); k++)
                    p = fmaf(xt[k], we[k], p);
                total = s == 0 ? p : total + p;
            }
            if (bias) total = total + bias[e];
            out[t * experts + e] = total;
        }
    }
}

void oracle_dequant_q4_k_scalar(const uint8_t* blocks, int64_t n, float* out) {
    for (int64_t i = 0; i < n; i++) {
        const uint8_t* b = blocks + i * 144;
        const float d = f16_at(b), dmin = f16_at(b + 2);
        const uint8_t* s = b + 4;
        for (int j = 0; j < 8; j++) {
            uint32_t sc, mn;
            if (j < 4) {
                sc = s[j] & 63;
                mn = s[j + 4] & 63;
            } else {
                sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 2) & 0x30);
                mn = (s[j + 4] >> 4) | ((s[j] >> 2) & 0x30);
            }
            const float scale = d * (float)sc, m = dmin * (float)mn;
            const uint8_t* qs = b + 16 + 32 * (j / 2);
            const int shift = 4 * (j % 2);
            for (int l = 0; l < 32; l++) out[i * 256 + 32 * j + l] = scale * (float)((qs[l] >> shift) & 0xF) - m;
        }
    }
}

void oracle_dequant_q6_k_scalar(const uint8_t* blocks, int64_t n, float* out) {
    for (int64_t i = 0; i < n; i++) {
        const uint8_t* b = blocks + i * 210;
        const float d = f16_at(b + 208);
        for (int sub = 0; sub < 8; sub++) {
            const int h = sub / 4, s = sub % 4;
            const uint8_t* ql = b + 64 * h + 32 * (s % 2);
            const uint8_t* qh = b + 128 + 32 * h;
            const int shift = 4 * (s / 2);
            const float scale0 = d * (float)(int8_t)b[192 + 2 * sub];
            const float scale1 = d * (float)(int8_t)b[193 + 2 * sub];
            for (int l = 0; l < 32; l++) {
                const int q = (int)(((ql[l] >> shift) & 0xF) | (((qh[l] >> (2 * s)) & 3) << 4)) - 32;
                out[i * 256 + 32 * sub + l] = (l < 16 ? scale0 : scale1) * (float)q;
            }
        }
    }
}
