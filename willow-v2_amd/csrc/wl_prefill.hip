// Prefill (many tokens per expert): the expert products as grouped bf16 MFMA GEMMs.
//
// Replaces the reference's prefill branch: GGMLWeight.linear dequantizes the whole weight to bf16 and multiplies
// with torch (gguf/metal.py:401-408), once per expert (engines/base.py:534-591). Here no dequantized weight is
// ever written: each wavefront decodes its Q4_K / Q6_K rows straight into v_mfma_f32_16x16x32_bf16 A-operands in
// registers (fp32 value, rounded to bf16 like Tensor.to(torch.bfloat16)), while the tokens' activations (bf16) are
// staged in LDS as the B-operand. Accumulation is fp32.
//
//   k_router_mfma    logits for many tokens in the router's fixed order (64-value FMA segments, added left to
//                    right); also writes x as bf16 (the small-batch router in wl_moe.hip does the same)
//   (sort)           the sort's single-workgroup stage writes the tile lists (tile_list): per-expert tiles of
//                    sorted positions, then the shared expert's, of at most 144 (gate_up) and 128 (down) tokens
//   k_gemm_gate_up   per (tile, 128 intermediate rows): gate and up rows together, epilogue h = silu(g) * u -> bf16
//   k_gemm_down      per (tile, 256 output rows): o = down h, fp32, by sorted position (combined by k_combine)
//
// MFMA 16x16x32 bf16 operand layout (wave64): lane l holds A[l % 16][8 (l / 16) + i], B[8 (l / 16) + i][l % 16],
// and C[4 (l / 16) + i][l % 16], i < 8 (A, B) or < 4 (C). A wavefront covers kRT row tiles x up to 9 token tiles.
#include <hip/hip_runtime.h>

#include "wl_common.h"
#include "wl_host.h"
#include "wl_moe.h"
#include "wl_moe_dev.h"

namespace wl {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kBK = 256;              // k per staged chunk: one K-quant block per row
constexpr int kTileRowBytes = kBK * 2;                     // one token's chunk in LDS: 512 bytes, 32 slots of 16
template <int TILE>
constexpr int tile_bytes() { return TILE * kTileRowBytes; }  // one LDS buffer: 72 KiB for 144 tokens
// A GEMM workgroup covers 16 row tiles of 16 rows against one token tile: kGemmWaves wavefronts of kRT row tiles
// each. Two row tiles per wavefront keep a wavefront within 256 registers, so the 8 wavefronts of a workgroup run
// two per SIMD and one's dequantization overlaps the other's waits.
constexpr int kRT = 2;
constexpr int kGemmWaves = 16 / kRT;
constexpr int kGemmThreads = 64 * kGemmWaves;

// 8 bytes from a 2-byte-aligned address: 3 aligned dwords, realigned. Reads [p & ~3, (p & ~3) + 12), within
// [p - 2, p + 12); all three loads are unconditional so that no branch splits the wavefront.
__device__ __forceinline__ uint2 load8_a2(const uint8_t* p) {
    uint32_t sh;
    const uint32_t* q = align_down4(p, sh);
    const uint32_t w0 = q[0], w1 = q[1], w2 = q[2];
    return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh));
}

// ---------------------------------------------------------------------------------------------------------------
// Router for many tokens on the matrix core. v_mfma_f32_16x16x4_f32 computes each output as four fused multiply-adds
// onto the accumulator in k order (c = fma(a[k], b[k], c), k = 0..3, bit for bit the same), so a chain of 16 of them
// from a zero accumulator over k = 4 s + j (s = 0..15, j = 0..3) is a 64-value segment's fused multiply-add chain in
// ascending k; each segment partial is then added to the running total: the order of router_row and of the CPU
// replay. A workgroup computes 32 TM tokens x 64 rows (rows: experts, then the shared gate as row E); wavefront w
// the TM x 2 tiles of 16 x 16 at tokens 16 TM (w & 1) + 16 m and rows 32 (w >> 1) + 16 n. Per segment the operands
// are staged in LDS as [j][token or row][s] with 20-float rows: lane (l % 16, j = l / 16) reads its 16 values of the
// segment as four 16-byte loads, and the 8 lanes of one LDS cycle fall in 8 different bank groups. The staging is
// double-buffered: while segment s is computed, segment s + 1 is written to the other buffer and segment s + 3 is
// loaded into the register set segment s + 1 leaves (two sets, so each segment's loads have two segments' time to
// land), one barrier per segment.
constexpr int kRmRow = 20;
constexpr int kRouterMfmaTM = 1;  // token tiles of 16 per wavefront

template <int TM>
__global__ __launch_bounds__(256) void k_router_mfma(const float* __restrict__ x, const float* __restrict__ w,
                                                     const float* __restrict__ bias,
                                                     const float* __restrict__ shared_gate, int T, int H, int E,
                                                     float* __restrict__ logits, float* __restrict__ sg,
                                                     uint16_t* __restrict__ xb, const float* __restrict__ gate_row) {
    constexpr int kTok = 32 * TM;              // tokens per workgroup
    constexpr int kXq = kTok * 16 / 256;       // float4 loads per thread per segment (tokens)
    __shared__ __attribute__((aligned(16))) float xs[2][4 * kTok * kRmRow];
    __shared__ __attribute__((aligned(16))) float ws[2][4 * 64 * kRmRow];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int t0 = blockIdx.x * kTok, r0 = blockIdx.y * 64;
    const int rows = E + (shared_gate ? 1 : 0);
    const int nseg = H / kRouterSeg;
    // staging: float4 f = tid + 256 q holds values 4 s4 .. 4 s4 + 3 (s4 = f % 16) of token / row f / 16
    const int s4 = tid & 15;
    const float* xrow[kXq];
    const float* wrow[4];
#pragma unroll
    for (int q = 0; q < kXq; q++) {
        const int t = t0 + ((tid + 256 * q) >> 4);
        xrow[q] = x + static_cast<int64_t>(t < T ? t : T - 1) * H + 4 * s4;
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int r = r0 + ((tid + 256 * q) >> 4);
        wrow[q] = r < rows ? (r < E ? w + static_cast<int64_t>(r) * H : shared_gate) + 4 * s4 : nullptr;
    }
    // segment s's loads land in register set s & 1, two segments ahead of its computation
    float4 xn[2][kXq], wn[2][4];
    auto load_seg = [&](int sgi, float4 (&xr)[kXq], float4 (&wr)[4]) {
#pragma unroll
        for (int q = 0; q < kXq; q++) xr[q] = *reinterpret_cast<const float4*>(xrow[q] + sgi * kRouterSeg);
#pragma unroll
        for (int q = 0; q < 4; q++)
            wr[q] = wrow[q] ? *reinterpret_cast<const float4*>(wrow[q] + sgi * kRouterSeg)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    const int lt = lane & 15, lj = lane >> 4;
    const int tm0 = 16 * TM * (wv & 1), rn0 = 32 * (wv >> 1);
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
    floatx4 tot[TM][2], acc[TM][2];
    // staging of segment sgi (from registers) into LDS buffer sgi & 1, with x also stored as bf16 once per token
    auto stage = [&](int sgi, const float4 (&xr)[kXq], const float4 (&wr)[4]) {
        float* xsb = xs[sgi & 1];
        float* wsb = ws[sgi & 1];
#pragma unroll
        for (int q = 0; q < kXq; q++) {
            const int rr = (tid + 256 * q) >> 4;
            if (xb && blockIdx.y == 0 && t0 + rr < T)  // x as bf16 for the MFMA GEMMs, written once per token
                *reinterpret_cast<uint2*>(xb + static_cast<int64_t>(t0 + rr) * H + sgi * kRouterSeg + 4 * s4) =
                    make_uint2(pack2(xr[q].x, xr[q].y), pack2(xr[q].z, xr[q].w));
            xsb[(0 * kTok + rr) * kRmRow + s4] = xr[q].x;
            xsb[(1 * kTok + rr) * kRmRow + s4] = xr[q].y;
            xsb[(2 * kTok + rr) * kRmRow + s4] = xr[q].z;
            xsb[(3 * kTok + rr) * kRmRow + s4] = xr[q].w;
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int rr = (tid + 256 * q) >> 4;
            wsb[(0 * 64 + rr) * kRmRow + s4] = wr[q].x;
            wsb[(1 * 64 + rr) * kRmRow + s4] = wr[q].y;
            wsb[(2 * 64 + rr) * kRmRow + s4] = wr[q].z;
            wsb[(3 * 64 + rr) * kRmRow + s4] = wr[q].w;
        }
    };
    load_seg(0, xn[0], wn[0]);
    if (nseg > 1) load_seg(1, xn[1], wn[1]);
    stage(0, xn[0], wn[0]);
    if (nseg > 2) load_seg(2, xn[0], wn[0]);
    __syncthreads();
    // segment sgi, then segment sgi + 1 staged from its register set (xr, wr) and segment sgi + 3 loaded into it
    auto segment = [&](int sgi, float4 (&xr)[kXq], float4 (&wr)[4]) {
        const float* xsb = xs[sgi & 1];
        const float* wsb = ws[sgi & 1];
#pragma unroll
        for (int q = 0; q < 4; q++) {  // steps s = 4 q .. 4 q + 3
            float4 av[TM], bv[2];
#pragma unroll
            for (int m = 0; m < TM; m++)
                av[m] = *reinterpret_cast<const float4*>(&xsb[(lj * kTok + tm0 + 16 * m + lt) * kRmRow + 4 * q]);
#pragma unroll
            for (int n = 0; n < 2; n++)
                bv[n] = *reinterpret_cast<const float4*>(&wsb[(lj * 64 + rn0 + 16 * n + lt) * kRmRow + 4 * q]);
#pragma unroll
            for (int u = 0; u < 4; u++) {
#pragma unroll
                for (int m = 0; m < TM; m++) {
                    const float a = u == 0 ? av[m].x : u == 1 ? av[m].y : u == 2 ? av[m].z : av[m].w;
#pragma unroll
                    for (int n = 0; n < 2; n++) {
                        const float b = u == 0 ? bv[n].x : u == 1 ? bv[n].y : u == 2 ? bv[n].z : bv[n].w;
                        acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, (q == 0 && u == 0) ? zero : acc[m][n],
                                                                         0, 0, 0);
                    }
                }
            }
        }
        // the next segment goes into the other buffer, whose last reads (segment sgi - 1) ended before the barrier
        // that closed the previous iteration; its loads were issued two segments ago
        if (sgi + 1 < nseg) {
            stage(sgi + 1, xr, wr);
            if (sgi + 3 < nseg) load_seg(sgi + 3, xr, wr);
        }
#pragma unroll
        for (int m = 0; m < TM; m++)
#pragma unroll
            for (int n = 0; n < 2; n++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    tot[m][n][i] = sgi == 0 ? acc[m][n][i] : __fadd_rn(tot[m][n][i], acc[m][n][i]);
        __syncthreads();  // segment sgi + 1 is staged for everyone; buffer sgi & 1 is free again
    };
    for (int sgi = 0; sgi < nseg; sgi += 2) {
        segment(sgi, xn[1], wn[1]);
        if (sgi + 1 < nseg) segment(sgi + 1, xn[0], wn[0]);
    }
    // lane holds D[4 lj + i][lt]: token tm0 + 16 m + 4 lj + i, row rn0 + 16 n + lt
#pragma unroll
    for (int m = 0; m < TM; m++)
#pragma unroll
        for (int n = 0; n < 2; n++) {
            const int r = r0 + rn0 + 16 * n + lt;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = t0 + tm0 + 16 * m + 4 * lj + i;
                if (t < T && r < rows) {
                    const float v = tot[m][n][i];
                    if (r < E)
                        logits[static_cast<int64_t>(t) * E + r] = bias ? __fadd_rn(v, bias[r]) : v;
                    else
                        sg[t] = sigmoid(v);
                }
            }
        }
    // gate_row: the shared gate when it has no row in the tiles. The workgroups of one token tile share its tokens,
    // two per wavefront (one per half), in router_row's order, after their matrix-core work. This replaces a kernel
    // of its own (10.8 us per 4096-token layer): 22.25 -> 21.95 ms per 40-layer chunk.
    if (gate_row) {
        for (int tt = static_cast<int>(blockIdx.y) * 8; tt < kTok; tt += static_cast<int>(gridDim.y) * 8) {
            const int t = t0 + tt + 2 * wv + (lane >> 5);
            const bool valid = t < T;
            const float total = router_row(x + static_cast<int64_t>(valid ? t : 0) * H, gate_row, valid, H, lane);
            if ((lane & 31) == 0 && valid) sg[t] = sigmoid(total);
        }
    }
}



// ---------------------------------------------------------------------------------------------------------------
// A-operand decoders. At 32-value step KK of a 256-value block, lane group q (lanes 16 q .. 16 q + 15, one row
// each) supplies 8 of the step's 32 k-values; which 8 is the type's K order (k_slot below), and the B-operand is
// read from LDS in the same order, so the product is the block's dot product with the matrix core's additions in
// another order. The per-block state is fetched once (fetch), prepared once the loads have landed (prepare), then
// each step is unpacked (frag).
//
// Q4_K order: step KK, group q holds values 32 (2 q + (KK & 1)) + 8 (KK >> 1) + i of the block, the (KK >> 1)-th 8
// values of sub-block 2 q + (KK & 1). A group so only needs the scales of sub-blocks 2 q and 2 q + 1, whose 64 values
// are the low and high nibbles of qs bytes 32 q .. 32 q + 31.
struct Q4KRowState {
    uint4 hd;       // d, dmin, 12 scale bytes
    uint4 qs[2];    // qs bytes 32 q .. 32 q + 31
    float a[2], b[2];  // value = a[e] * nibble + b[e] for sub-block 2 q + e, a[e] scaled for fragment_q4k
};

__device__ __forceinline__ void fetch_q4k(const uint8_t* __restrict__ blk, int q, Q4KRowState& s) {
    s.hd = *reinterpret_cast<const uint4*>(blk);
    s.qs[0] = *reinterpret_cast<const uint4*>(blk + 16 + 32 * q);
    s.qs[1] = *reinterpret_cast<const uint4*>(blk + 32 + 32 * q);
}

// The scales of sub-blocks j = 2 q + e (q4k_scale_min with a per-lane j): j < 4 for q < 2, j >= 4 otherwise, and
// the byte holding j's fields sits 8 ((2 q + e) & 3) bits into its word either way. Both cases as one expression
// with per-lane shift and masks (j < 4: s0 & 63, s1 & 63; j >= 4: the low 4 bits from s2 and bits 4, 5 from the top
// of s0 / s1), so the wavefront does not branch on its lane groups.
__device__ __forceinline__ void prepare_q4k(Q4KRowState& s, int q) {
    const float d = half_to_float(s.hd.x), dmin = half_to_float(s.hd.x >> 16);
    const bool hi = q >= 2;
    const uint32_t sh_hi = hi ? 2u : 0u, mask_top = hi ? 0x30u : 0x3Fu, mask_low = hi ? 0xFu : 0u;
    const uint32_t sh0 = 16u * static_cast<uint32_t>(q & 1);
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const uint32_t sh = sh0 + 8u * e;
        const uint32_t s0 = s.hd.y >> sh, s1 = s.hd.z >> sh, s2 = s.hd.w >> sh;
        const uint32_t sc = ((s0 >> sh_hi) & mask_top) | (s2 & mask_low);
        const uint32_t m = ((s1 >> sh_hi) & mask_top) | ((s2 >> 4) & mask_low);
        // times 2^24 for the low nibbles, 2^20 for the high ones: the f16-subnormal scale of fragment_q4k (exact)
        s.a[e] = (d * (e ? 1048576.0f : 16777216.0f)) * static_cast<float>(sc);
        s.b[e] = -(dmin * static_cast<float>(m));
    }
}

// 4 values as f16 subnormals (values 0 and 2 in the halves of e, 1 and 3 in those of o; a half with zero exponent
// bits and mantissa q is q 2^-k) as bf16 of a * q + b, packed two per dword: each a v_fma_mix_f32 that reads the half
// directly (no conversion instruction per value), with a scaled by 2^k (exact), so a * q is the same exact product
__device__ __forceinline__ void affine4_h(uint32_t e, uint32_t o, float a, float b, uint32_t& p0, uint32_t& p1) {
    const wl_f16x2 he = __builtin_bit_cast(wl_f16x2, e), ho = __builtin_bit_cast(wl_f16x2, o);
    p0 = pack2(__builtin_fmaf(a, static_cast<float>(he.x), b), __builtin_fmaf(a, static_cast<float>(ho.x), b));
    p1 = pack2(__builtin_fmaf(a, static_cast<float>(he.y), b), __builtin_fmaf(a, static_cast<float>(ho.y), b));
}

template <int KK>
__device__ __forceinline__ bf16x8 fragment_q4k(const Q4KRowState& s) {
    constexpr int e = KK & 1, j = KK >> 1;  // sub-block 2 q + e, its bytes 8 j .. 8 j + 7
    const uint4 w = s.qs[j >> 1];
    const uint32_t w0 = (j & 1) ? w.z : w.x, w1 = (j & 1) ? w.w : w.y;
    // the nibbles in place as f16 subnormals: low ones (bits 0..3 of a half) q 2^-24, high ones (bits 4..7) q 2^-20
    constexpr uint32_t m = e ? 0x00F000F0u : 0x000F000Fu;
    uint4 p;
    affine4_h(w0 & m, (w0 >> 8) & m, s.a[e], s.b[e], p.x, p.y);
    affine4_h(w1 & m, (w1 >> 8) & m, s.a[e], s.b[e], p.z, p.w);
    return __builtin_bit_cast(bf16x8, p);
}

// Q6_K order: step KK = 2 t + s, group q (h = q >> 1, p = q & 1) holds values 128 h + 32 t + 16 p + 8 s + i. Over a
// block a group covers 4 scale groups of 16 (scales 8 h + 2 t + p), both nibbles of ql bytes 64 h + 16 p + [0, 16)
// and 64 h + 32 + 16 p + [0, 16), and qh bytes 32 h + 16 p + [0, 16).
struct Q6KRowState {
    uint4 ql[2];   // ql bytes 64 h + 32 u + 16 p .. + 15, u = 0, 1
    uint4 qh;      // qh bytes 32 h + 16 p .. + 15
    uint2 sc;      // scale bytes 8 h .. 8 h + 7
    float d;
    float a[4];    // value = a[t] * (q6 - 32), a[t] = d * scale 8 h + 2 t + p
};

__device__ __forceinline__ void fetch_q6k(const uint8_t* __restrict__ blk, int q, Q6KRowState& s) {
    const int h = q >> 1, p = q & 1;
    s.ql[0] = load16_a2(blk + 64 * h + 16 * p);
    s.ql[1] = load16_a2(blk + 64 * h + 32 + 16 * p);
    s.qh = load16_a2(blk + 128 + 32 * h + 16 * p);
    // scale bytes 192 + 8 h .. + 7: the dwords of their aligned start and, for a start 2 bytes into a dword, the last
    // two bytes as a 16-bit load (the realignment takes only its low half; nothing past the block is read)
    uint32_t sh;
    const uint8_t* sp = blk + 192 + 8 * h;
    const uint32_t* w = align_down4(sp, sh);
    const uint32_t w0 = w[0], w1 = w[1];
    const uint32_t w2 = *reinterpret_cast<const uint16_t*>(sp + 6);
    s.sc = make_uint2(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh));
    s.d = half_to_float(*reinterpret_cast<const uint16_t*>(blk + 208));
}

__device__ __forceinline__ void prepare_q6k(Q6KRowState& s, int q) {
    // scale 8 h + 2 t + p is byte 2 t + p of sc: word t >> 1, byte 2 (t & 1) + p
    const uint32_t sh = 8u * static_cast<uint32_t>(q & 1);
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const uint32_t w = (t >> 1) ? s.sc.y : s.sc.x;
        const int32_t sc = static_cast<int8_t>((w >> (16 * (t & 1) + sh)) & 0xFFu);
        s.a[t] = s.d * static_cast<float>(sc);
    }
}

template <int KK>
__device__ __forceinline__ bf16x8 fragment_q6k(const Q6KRowState& s) {
    constexpr int t = KK >> 1, sidx = KK & 1;
    const uint4 l = s.ql[t & 1];
    const uint32_t l0 = sidx ? l.z : l.x, l1 = sidx ? l.w : l.y;
    const uint32_t h0 = sidx ? s.qh.z : s.qh.x, h1 = sidx ? s.qh.w : s.qh.y;
    // 6-bit values: the nibble (low for t < 2) and qh bits 2 t, 2 t + 1 moved to bits 4, 5 of each byte
    constexpr uint32_t lsh = 4 * (t >> 1);
    auto six = [&](uint32_t lw, uint32_t hw) {
        const uint32_t hi = (t == 3 ? (hw >> 2) : (hw << (4 - 2 * t))) & 0x30303030u;
        return ((lw >> lsh) & 0x0F0F0F0Fu) | hi;
    };
    const uint32_t v0 = six(l0, h0), v1 = six(l1, h1);
    const float a = s.a[t];
    const float b = -32.0f * a;  // exact: a has at most 19 significant bits
    // a * (q - 32) == fma(a, q, -32 a): the product a * q is exact, so both round the same sum once
    uint4 p;
    const float a24 = a * 16777216.0f;  // the bytes as f16 subnormals (q 2^-24), exact
    affine4_h(v0 & 0x00FF00FFu, (v0 >> 8) & 0x00FF00FFu, a24, b, p.x, p.y);
    affine4_h(v1 & 0x00FF00FFu, (v1 >> 8) & 0x00FF00FFu, a24, b, p.z, p.w);
    return __builtin_bit_cast(bf16x8, p);
}

template <int TYPE>
struct RowState;
template <>
struct RowState<WL_TYPE_Q4_K> {
    Q4KRowState s;
    __device__ __forceinline__ void fetch(const uint8_t* blk, int q) { fetch_q4k(blk, q, s); }
    __device__ __forceinline__ void prepare(int q) { prepare_q4k(s, q); }
    template <int KK>
    __device__ __forceinline__ bf16x8 frag(int) const { return fragment_q4k<KK>(s); }
};
template <>
struct RowState<WL_TYPE_Q6_K> {
    Q6KRowState s;
    __device__ __forceinline__ void fetch(const uint8_t* blk, int q) { fetch_q6k(blk, q, s); }
    __device__ __forceinline__ void prepare(int q) { prepare_q6k(s, q); }
    template <int KK>
    __device__ __forceinline__ bf16x8 frag(int) const { return fragment_q6k<KK>(s); }
};

// ---------------------------------------------------------------------------------------------------------------
// LDS tile of one K chunk: [TILE tokens][256 values] bf16, 512 bytes per token, no padding; the 16-byte slot holding
// values 8c .. 8c + 7 of token t is slot c ^ (t & m) of the token's row, m = swizzle<TYPE>() (7 or 15), so the
// tokens a B-fragment read serves at once sit in different bank groups.
//
// B-fragment of token t = 16 n + lr and the 8 values of slot c (values 8 c .. 8 c + 7): byte address
// 512 t + 16 (c ^ (lr & m)) = 512 lr + 16 (c ^ (lr & m)) + 8192 n.
// Q4_K order, c = 8 q + 4 (KK & 1) + (KK >> 1); Q6_K order, c = 16 h + 4 t + 2 p + s (KK = 2 t + s, q = 2 h + p).
// In both, the XOR changes only the low 4 bits: a per-lane base for each KK.
template <int KK>
constexpr int q4k_slot_low() { return 4 * (KK & 1) + (KK >> 1); }

// The 16-byte slot c of token t sits at c ^ (t & swizzle): 8 tokens for Q4_K's B-fragment reads, 16 for Q6_K's
// (their lane groups read different slot patterns; each mask is the one the LDS bank-conflict counter reads zero
// for, measured on the MI355X).
template <int TYPE>
constexpr int swizzle() { return TYPE == WL_TYPE_Q4_K ? 7 : 15; }
struct BAddr {
    uint32_t step[8];
};
template <int TYPE>
__device__ __forceinline__ BAddr b_addr(int lr, int q) {
    BAddr ba{};
    const int y = lr & 7, y8 = (lr & swizzle<TYPE>()) >> 3;  // the swizzle's low 3 bits and its bit 3
    if constexpr (TYPE == WL_TYPE_Q4_K) {
        const uint32_t base = 512u * lr + 128u * (q ^ y8);
        ba.step[0] = base + 16u * (q4k_slot_low<0>() ^ y);
        ba.step[1] = base + 16u * (q4k_slot_low<1>() ^ y);
        ba.step[2] = base + 16u * (q4k_slot_low<2>() ^ y);
        ba.step[3] = base + 16u * (q4k_slot_low<3>() ^ y);
        ba.step[4] = base + 16u * (q4k_slot_low<4>() ^ y);
        ba.step[5] = base + 16u * (q4k_slot_low<5>() ^ y);
        ba.step[6] = base + 16u * (q4k_slot_low<6>() ^ y);
        ba.step[7] = base + 16u * (q4k_slot_low<7>() ^ y);
    } else {
        const int h = q >> 1, p = q & 1;
        const uint32_t base = 512u * lr + 256u * h;
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            const int t = kk >> 1, sidx = kk & 1;
            ba.step[kk] = base + 128u * ((t >> 1) ^ y8) + 16u * ((4 * (t & 1) + 2 * p + sidx) ^ y);
        }
    }
    return ba;
}
template <int TYPE, int KK>
__device__ __forceinline__ bf16x8 read_b1(const uint8_t* buf, const BAddr& ba, int n) {
    return *reinterpret_cast<const bf16x8*>(buf + ba.step[KK] + 8192 * n);
}
template <int TYPE, int NT, int KK>
__device__ __forceinline__ void read_b(const uint8_t* buf, const BAddr& ba, bf16x8 (&b)[NT]) {
#pragma unroll
    for (int n = 0; n < NT; n++) b[n] = read_b1<TYPE, KK>(buf, ba, n);
}

// Explicit MFMA / VALU interleave through scheduling barriers (the compiler's default order otherwise). Off: it
// multiplies this file's compile time by ~100.
constexpr bool kSchedGroups = false;

// One 32-value step, software-pipelined: the MFMAs of step KK (A-fragments `a`, B-fragments `b`) are interleaved
// with decoding step KK + 1's A-fragments into `an` (the chunk's last step decodes nothing: the next block's first
// fragments are decoded at the top of the next iteration) and, as each b[n] has been consumed, reading step
// KK + 1's b[n] in its place (the last step's successor reads from the other LDS buffer after the barrier), so the
// decode runs while the matrix core is busy.
template <int TYPE, int NT, int KK, int NTA>
__device__ __forceinline__ void gemm_step(const uint8_t* buf, const BAddr& ba, const RowState<TYPE> (&rs)[kRT],
                                          floatx4 (&acc)[kRT][NTA], const bf16x8 (&a)[kRT], bf16x8 (&b)[NT],
                                          bf16x8 (&an)[kRT], int q) {
#pragma unroll
    for (int r = 0; r < kRT; r++) {
        if constexpr (KK < 7) an[r] = rs[r].template frag<KK + 1>(q);
    }
#pragma unroll
    for (int n = 0; n < NT; n++) {
#pragma unroll
        for (int r = 0; r < kRT; r++)
            acc[r][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[r], b[n], acc[r][n], 0, 0, 0);
        if constexpr (KK < 7) b[n] = read_b1<TYPE, KK + 1>(buf, ba, n);
    }
    if constexpr (kSchedGroups) {
        // kRT NT MFMAs per step against ~34 kRT VALU instructions of decode
        constexpr int kValuPer = NT == 8 ? 4 : 8;
#pragma unroll
        for (int i = 0; i < kRT * NT; i++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (KK < 7 && (i & 3) == 3) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, kValuPer, 0);
        }
    }
}

// Direct global -> LDS staging of a K chunk with gfx950's global_load_lds_dwordx4: one wavefront instruction writes
// 64 consecutive 16-byte LDS slots (M0 + 16 lane), two token rows. With W = kGemmWaves, instruction `it` of
// wavefront w fills rows 2 W it + 2 w + (lane >> 5); lane slot s = lane & 31 of row t takes the 16 bytes of values
// 8 (s ^ (t & m)) .. + 7, and t & m = (2 w + (lane >> 5)) & m does not depend on it (2 W is a multiple of 16),
// so the lane's byte column `col` is fixed. The rows' byte offsets come from `rowtab`, laid out so that a lane's
// stage_iters (TILE / 16) are contiguous: rowtab[stage_iters (t % 2 W) + t / 2 W].
//
// The loads are issued from inline assembly so that the compiler, which cannot tell the two LDS buffers apart,
// does not wait for them before the next LDS read of the other buffer; the K loop waits for them itself
// (s_waitcnt vmcnt(0) and a barrier) before the buffer is read.
template <int TILE>
constexpr int stage_iters() { return tile_bytes<TILE>() / (kGemmWaves * 1024); }  // 9 for 144 tokens
static_assert(kGemmWaves % 8 == 0 && kTileTokens % (2 * kGemmWaves) == 0 && kDownTileTokens % (2 * kGemmWaves) == 0,
              "");
template <int TILE>
__host__ __device__ constexpr int rowtab_index(int t) {
    return stage_iters<TILE>() * (t % (2 * kGemmWaves)) + t / (2 * kGemmWaves);
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)(p)));
}

template <int TILE, int NT>
__device__ __forceinline__ void stage_async(uint32_t buf, const uint8_t* src, const uint32_t* rowtab, uint32_t col,
                                            int wv, int half) {
    constexpr int kIters = stage_iters<TILE>();
    static_assert(NT <= kIters, "");
    const uint32_t* tab = rowtab + kIters * (2 * wv + half);
    uint32_t off[NT];
#pragma unroll
    for (int i = 0; i < NT; i++) off[i] = tab[i];
#pragma unroll
    for (int it = 0; it < NT; it++) {  // iteration it: tokens 16 it .. 16 it + 15, token tile it
        // M0 (the LDS destination) is a register the compiler reserves: saved and restored around the load
        uint32_t saved;
        asm volatile(
            "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, %3\n\ts_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(buf + (kGemmWaves * it + wv) * 1024), "v"(off[it] + col), "s"(src)
            : "memory");
    }
}

// silu for a value rounded to bf16 right after (the gate_up epilogue): the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32, about 1 ulp each) instead of expf and an IEEE division, whose relative error of ~3e-7
// vanishes in the bf16 rounding but whose code, inlined for every accumulator, made k_gemm_gate_up 66 KB, more than
// the 64 KB instruction cache (49 KB with this; 4096-token prefill 22.3 -> 21.9 ms per chunk). Same limits as
// silu: g -> -inf gives -0, +inf gives +inf, NaN stays NaN.
__device__ __forceinline__ float silu_bf16(float g) {
    return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * g));
}

// Two bf16 values of the SwiGLU product from fp32 gate and up sums, rounded where the reference's bf16 tensors
// round them (engines/base.py:568-570 on bf16 F.linear outputs): the gate_up matmul returns gate and up as bf16,
// F.silu(gate) returns bf16, and so does silu(gate) * up (the product of two bf16 values is exact in fp32, so
// only its final rounding matters). Returns the packed pair (value 0 in the low half).
__device__ __forceinline__ uint32_t swiglu_bf16(float g0, float u0, float g1, float u1) {
    const uint32_t gp = pack2(g0, g1), up = pack2(u0, u1);
    const float gb0 = __builtin_bit_cast(float, gp << 16), gb1 = __builtin_bit_cast(float, gp & 0xFFFF0000u);
    const float ub0 = __builtin_bit_cast(float, up << 16), ub1 = __builtin_bit_cast(float, up & 0xFFFF0000u);
    const uint32_t sp = pack2(silu_bf16(gb0), silu_bf16(gb1));
    const float sb0 = __builtin_bit_cast(float, sp << 16), sb1 = __builtin_bit_cast(float, sp & 0xFFFF0000u);
    return pack2(sb0 * ub0, sb1 * ub1);
}

// A wavefront-uniform pointer in scalar registers (the value of lane 0).
__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<const uint8_t*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Waits for every outstanding load, the inline-assembly ones included; the compiler sees this wait, so it does not
// add waits of its own for loads issued before it.
__device__ __forceinline__ void wait_stage() { __builtin_amdgcn_s_waitcnt(0); }

// The K loop for NT token tiles, over `nitems` row sets (items) one after another: step st is block kc = st % nblocks
// of item st / nblocks, and the pipeline runs across items. Step st + 1's row states and LDS tile are requested at
// the top of step st; the last step requests the row states of its own block again (keeping the loop free of
// branches around the register loads) and no tile. With at most two blocks, both chunks stay in LDS (chunk kc in
// buffer kc) and are staged once for all items. After an item's last block, epi(item, acc) stores it and the
// accumulators restart from zero.
template <int TYPE, int TILE, int NT, int NTA, typename RowPtr, typename Epilogue>
__device__ __forceinline__ void gemm_loop(uint8_t (&bufs)[2][tile_bytes<TILE>()], floatx4 (&acc)[kRT][NTA], int nblocks,
                                          int nitems, const uint8_t* src, const uint32_t* rowtab, RowPtr row_ptr,
                                          Epilogue epi, int lr, int q) {
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)), half = lane >> 5;
    const uint32_t col = 16u * static_cast<uint32_t>((lane & 31) ^ ((2 * wv + half) & swizzle<TYPE>()));
    const uint32_t lds0 = lds_address(bufs[0]), lds1 = lds_address(bufs[1]);
    const BAddr ba = b_addr<TYPE>(lr, q);
    RowState<TYPE> rs[kRT], nx[kRT];
#pragma unroll
    for (int r = 0; r < kRT; r++) rs[r].fetch(row_ptr(0, r, lr), q);
    stage_async<TILE, NT>(lds0, src, rowtab, col, wv, half);
    bf16x8 a0[kRT], a1[kRT], b[NT];
    const int nsteps = nitems * nblocks;
    for (int st = 0; st < nsteps; st++) {
        if (!(nblocks <= 2 && st >= nblocks)) {  // resident chunks: staged and waited for by step nblocks - 1
            wait_stage();     // this chunk's LDS tile has landed
            __syncthreads();  // ... for every wavefront, and the other buffer is free
        }
        const int sn = st + 1 < nsteps ? st + 1 : st;
        const int in = sn / nblocks, kn = sn - in * nblocks;
#pragma unroll
        for (int r = 0; r < kRT; r++)
            nx[r].fetch(row_ptr(in, r, lr) + static_cast<int64_t>(kn) * BlockInfo<TYPE>::bytes, q);
        const bool resident = nblocks <= 2;
        if (st + 1 < nsteps && (!resident || sn < nblocks))
            stage_async<TILE, NT>((resident ? kn : ((st + 1) & 1)) ? lds1 : lds0,
                              src + static_cast<int64_t>(kn) * kTileRowBytes, rowtab, col, wv, half);
        const uint8_t* buf = bufs[resident ? st - (st / nblocks) * nblocks : (st & 1)];
        read_b<TYPE, NT, 0>(buf, ba, b);
        // the block's first fragments are decoded here, after the wait for every outstanding load, rather than in
        // the previous iteration's last step: the row-state loads get a whole iteration to land
#pragma unroll
        for (int r = 0; r < kRT; r++) {
            rs[r].prepare(q);
            a0[r] = rs[r].template frag<0>(q);
        }
        gemm_step<TYPE, NT, 0, NTA>(buf, ba, rs, acc, a0, b, a1, q);
        gemm_step<TYPE, NT, 1, NTA>(buf, ba, rs, acc, a1, b, a0, q);
        gemm_step<TYPE, NT, 2, NTA>(buf, ba, rs, acc, a0, b, a1, q);
        gemm_step<TYPE, NT, 3, NTA>(buf, ba, rs, acc, a1, b, a0, q);
        gemm_step<TYPE, NT, 4, NTA>(buf, ba, rs, acc, a0, b, a1, q);
        gemm_step<TYPE, NT, 5, NTA>(buf, ba, rs, acc, a1, b, a0, q);
        gemm_step<TYPE, NT, 6, NTA>(buf, ba, rs, acc, a0, b, a1, q);
        gemm_step<TYPE, NT, 7, NTA>(buf, ba, rs, acc, a1, b, a0, q);
#pragma unroll
        for (int r = 0; r < kRT; r++) rs[r] = nx[r];
        const int item = st / nblocks;
        if (st - item * nblocks == nblocks - 1) {
            epi(item, acc);
#pragma unroll
            for (int r = 0; r < kRT; r++)
#pragma unroll
                for (int n = 0; n < NTA; n++) acc[r][n] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
    }
    wait_stage();
}

// The K loop for tiles of at most 64 tokens (NT <= 4), whose steps have little arithmetic, so that each step's
// weight round trip would otherwise be exposed: the row states run kRing - 1 steps ahead in a ring of registers
// (the step loop is unrolled by kRing so every ring index is a constant), and the activation chunks are staged a
// phase at a time: every chunk of the row set at once when they fit in the LDS buffers (then once for all items),
// else kSlots chunks per phase, each phase staged, waited for and then computed. Only the row-state loads are in
// flight while a phase computes, and they are ordinary loads, so the compiler's own waits before each ring entry's
// first use are exact. Same results as gemm_loop: the same fragments and MFMAs in the same order.
constexpr int kRing = 3;
template <int TYPE, int TILE, int NT, int NTA, typename RowPtr, typename Epilogue>
__device__ __forceinline__ void gemm_loop_small(uint8_t (&bufs)[2][tile_bytes<TILE>()], floatx4 (&acc)[kRT][NTA],
                                                int nblocks, int nitems, const uint8_t* src, const uint32_t* rowtab,
                                                RowPtr row_ptr, Epilogue epi, int lr, int q) {
    constexpr int kChunk = NT * kGemmWaves * 1024;               // one staged chunk: NT token tiles
    constexpr int kSlots = 2 * tile_bytes<TILE>() / kChunk;      // chunks the two buffers hold
    static_assert(NT <= 4 && kSlots >= 2, "");
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)), half = lane >> 5;
    const uint32_t col = 16u * static_cast<uint32_t>((lane & 31) ^ ((2 * wv + half) & swizzle<TYPE>()));
    const uint32_t lds0 = lds_address(bufs[0]);
    const uint8_t* base = bufs[0];
    const BAddr ba = b_addr<TYPE>(lr, q);
    const bool resident = nblocks <= kSlots;
    const int nsteps = nitems * nblocks;
    RowState<TYPE> ring[kRing][kRT];
    auto fetch = [&](RowState<TYPE> (&rs)[kRT], int st) {
        const int item = st / nblocks, kc = st - item * nblocks;
#pragma unroll
        for (int r = 0; r < kRT; r++)
            rs[r].fetch(row_ptr(item, r, lr) + static_cast<int64_t>(kc) * BlockInfo<TYPE>::bytes, q);
    };
#pragma unroll
    for (int u = 0; u + 1 < kRing; u++)
        if (u < nsteps) fetch(ring[u], u);
    bf16x8 a0[kRT], a1[kRT], b[NT];
    for (int st0 = 0; st0 < nsteps; st0 += kRing) {
#pragma unroll
        for (int u = 0; u < kRing; u++) {
            const int st = st0 + u;
            if (st >= nsteps) break;
            const int item = st / nblocks, kc = st - item * nblocks;
            const int slot = resident ? kc : kc % kSlots;
            if (resident ? st == 0 : slot == 0) {
                // a new phase: every wavefront is done with the previous phase's chunks before they are replaced
                __syncthreads();
                const int n = resident ? nblocks : min(kSlots, nblocks - kc);
                for (int c = 0; c < n; c++)
                    stage_async<TILE, NT>(lds0 + c * kChunk, src + static_cast<int64_t>(kc + c) * kTileRowBytes,
                                          rowtab, col, wv, half);
                wait_stage();
                __syncthreads();
            }
            if (st + kRing - 1 < nsteps) fetch(ring[(u + kRing - 1) % kRing], st + kRing - 1);
            const uint8_t* buf = base + slot * kChunk;
            RowState<TYPE> (&rs)[kRT] = ring[u];
            read_b<TYPE, NT, 0>(buf, ba, b);
#pragma unroll
            for (int r = 0; r < kRT; r++) {
                rs[r].prepare(q);
                a0[r] = rs[r].template frag<0>(q);
            }
            gemm_step<TYPE, NT, 0, NTA>(buf, ba, rs, acc, a0, b, a1, q);
            gemm_step<TYPE, NT, 1, NTA>(buf, ba, rs, acc, a1, b, a0, q);
            gemm_step<TYPE, NT, 2, NTA>(buf, ba, rs, acc, a0, b, a1, q);
            gemm_step<TYPE, NT, 3, NTA>(buf, ba, rs, acc, a1, b, a0, q);
            gemm_step<TYPE, NT, 4, NTA>(buf, ba, rs, acc, a0, b, a1, q);
            gemm_step<TYPE, NT, 5, NTA>(buf, ba, rs, acc, a1, b, a0, q);
            gemm_step<TYPE, NT, 6, NTA>(buf, ba, rs, acc, a0, b, a1, q);
            gemm_step<TYPE, NT, 7, NTA>(buf, ba, rs, acc, a1, b, a0, q);
            if (kc == nblocks - 1) {
                epi(item, acc);
#pragma unroll
                for (int r = 0; r < kRT; r++)
#pragma unroll
                    for (int n = 0; n < NTA; n++) acc[r][n] = floatx4{0.f, 0.f, 0.f, 0.f};
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// The GEMM core: a workgroup of kGemmWaves wavefronts, each owning kRT row tiles of 16 (rows given by
// row_ptr(item, r, lr), for nitems row sets one after another) and the tile's up to TILE tokens as NT token tiles of
// 16 (NT = TILE / 16, 8, 4 or 1, the fewest that cover `count`; only those are staged). Per K chunk of 256 values
// (one block per row) the activations sit in LDS (double-buffered in gemm_loop; staged a phase at a time in
// gemm_loop_small, which takes NT = 4 and 1), and each of the 8 32-value steps decodes kRT A-fragments and runs
// kRT x NT MFMAs; epi(item, acc) stores each row set's results. src_row(t) is token t's row in src ([*, ld] bf16);
// rows past count load token 0's (their results are never stored).
template <int TYPE, int TILE, typename RowPtr, typename SrcRow, typename Epilogue>
__device__ __forceinline__ void gemm_tile(uint8_t (&bufs)[2][tile_bytes<TILE>()], floatx4 (&acc)[kRT][TILE / 16],
                                          int nblocks, int nitems, int count, const uint16_t* __restrict__ src,
                                          int64_t ld, SrcRow src_row, RowPtr row_ptr, Epilogue epi) {
    constexpr int NTA = TILE / 16;
    __shared__ __attribute__((aligned(16))) uint32_t rowtab[TILE];
    const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
    for (int t = threadIdx.x; t < TILE; t += blockDim.x)
        rowtab[rowtab_index<TILE>(t)] = static_cast<uint32_t>(src_row(t < count ? t : 0) * ld * 2);
#pragma unroll
    for (int r = 0; r < kRT; r++)
#pragma unroll
        for (int n = 0; n < NTA; n++) acc[r][n] = floatx4{0.f, 0.f, 0.f, 0.f};
    __syncthreads();
    const uint8_t* s8 = uniform_ptr(reinterpret_cast<const uint8_t*>(src));
    if (NTA > 8 && count > 128)
        gemm_loop<TYPE, TILE, NTA, NTA>(bufs, acc, nblocks, nitems, s8, rowtab, row_ptr, epi, lr, q);
    else if (count > 64)
        gemm_loop<TYPE, TILE, 8, NTA>(bufs, acc, nblocks, nitems, s8, rowtab, row_ptr, epi, lr, q);
    else if (count > 16)
        gemm_loop_small<TYPE, TILE, 4, NTA>(bufs, acc, nblocks, nitems, s8, rowtab, row_ptr, epi, lr, q);
    else
        gemm_loop_small<TYPE, TILE, 1, NTA>(bufs, acc, nblocks, nitems, s8, rowtab, row_ptr, epi, lr, q);
}

// Workgroups are dealt to the 8 XCDs round-robin by linear id, each XCD with its own L2. slab_tile maps the linear
// id to (row slab, tile) so that the nslab workgroups of one tile run back to back on one XCD and share its L2 copy of
// the tile's activations: XCD x takes tiles x, x + 8, ..., each as nslab consecutive workgroups. The grid is
// nslab * tiles8 workgroups, tiles8 = the tile bound rounded up to a multiple of 8.
constexpr int kXcds = 8;
__device__ __forceinline__ void slab_tile(int nslab, int& slab, int& tile) {
    const int b = static_cast<int>(blockIdx.x), x = b % kXcds, i = b / kXcds;
    slab = i % nslab;
    tile = (i / nslab) * kXcds + x;
}

// gate_up: slab = 128-row slab of the intermediate dim; wavefront w: gate rows j0 + 16r + lr (r < kRT / 2)
// and the matching up rows inter + j0 + ... (r >= kRT / 2), j0 = 128 slab + 8 kRT w. Epilogue h = silu(g) * u -> bf16.
// TILE is kTileTokens, or kDownTileTokens (and the down tile list) for Q6_K rows, whose larger row state leaves no
// registers for a ninth token tile.
template <int TYPE, int TILE>
__global__ __launch_bounds__(kGemmThreads) void k_gemm_gate_up(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t bufs[2][tile_bytes<TILE>()];
    if (a.skip && *a.skip) return;
    int slab, ti;
    slab_tile(a.nslab_gate_up, slab, ti);
    const int4* tiles = TILE == kTileTokens ? a.tiles : a.tiles_down;
    if (ti >= (TILE == kTileTokens ? a.n_tiles[0] : a.n_tiles_down[0])) return;
    const int4 tile = tiles[ti];
    const bool sh = tile.x == a.E;
    const int inter = sh ? a.sh_inter : a.inter;
    constexpr int kHalf = kRT / 2;
    const int j0 = slab * 128 + 16 * kHalf * (threadIdx.x >> 6);
    if (slab * 128 >= inter) return;
    const uint8_t* W = sh ? a.sh_gate_up : a.gate_up + static_cast<int64_t>(tile.x) * a.gate_up_stride;
    const int nb = a.H / kQK;
    const int64_t rs = static_cast<int64_t>(nb) * BlockInfo<TYPE>::bytes;
    const int pos0 = tile.y, count = tile.z;
    floatx4 acc[kRT][TILE / 16];
    auto row_ptr = [&](int, int r, int lr) {
        const int j = j0 + 16 * (r % kHalf) + lr;
        return W + static_cast<int64_t>((r < kHalf ? 0 : inter) + j) * rs;
    };
    auto src_row = [&](int t) -> int64_t { return sh ? pos0 + t : a.sorted[pos0 + t] / a.k; };
    uint16_t* out = sh ? a.h_sh16 : a.h16;
    auto epi = [&](int, floatx4 (&acc)[kRT][TILE / 16]) {
        const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
#pragma unroll
        for (int r = 0; r < kHalf; r++) {
#pragma unroll
            for (int n = 0; n < TILE / 16; n++) {
                const int t = 16 * n + lr;
                if (t < count) {
                    const int j = j0 + 16 * r + 4 * q;
                    const floatx4 g = acc[r][n], u = acc[r + kHalf][n];
                    *reinterpret_cast<uint2*>(out + static_cast<int64_t>(pos0 + t) * inter + j) =
                        make_uint2(swiglu_bf16(g[0], u[0], g[1], u[1]), swiglu_bf16(g[2], u[2], g[3], u[3]));
                }
            }
        }
    };
    gemm_tile<TYPE, TILE>(bufs, acc, nb, 1, count, a.xb, a.H, src_row, row_ptr, epi);
}

// down: a workgroup takes a.down_slabs consecutive 256-row slabs of the hidden dim (one pipeline across them); for
// slab item, wavefront w has rows 256 (slab0 + item) + 16 kRT w + 16 r + lr. o by position (row stride a.ldo;
// the shared expert's by token, stride H), rounded to bf16 as the reference's bf16 F.linear output is
// (gguf/metal.py:407). Its tiles hold at most 128 tokens (8 token tiles of accumulators keep Q6_K's wavefronts
// within 256 registers).
template <int TYPE>
__global__ __launch_bounds__(kGemmThreads) void k_gemm_down(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t bufs[2][tile_bytes<kDownTileTokens>()];
    if (a.skip && *a.skip) return;
    int group, ti;
    slab_tile(a.H / 256 / a.down_slabs, group, ti);
    int4 tile;
    if (a.dense_tokens > 0) {  // wl_linear: token tile ti of one matrix
        const int p = ti * kDownTileTokens;
        if (p >= a.dense_tokens) return;
        tile = make_int4(0, p, min(kDownTileTokens, a.dense_tokens - p), 0);
    } else {
        if (ti >= a.n_tiles_down[0]) return;
        tile = a.tiles_down[ti];
    }
    const bool sh = tile.x == a.E;
    const int inter = sh ? a.sh_inter : a.inter;
    const int row0 = group * a.down_slabs * 256 + 16 * kRT * (threadIdx.x >> 6);
    const uint8_t* W = sh ? a.sh_down : a.down + static_cast<int64_t>(tile.x) * a.down_stride;
    const int nb = inter / kQK;
    const int64_t rs = static_cast<int64_t>(nb) * BlockInfo<TYPE>::bytes;
    const int pos0 = tile.y, count = tile.z;
    floatx4 acc[kRT][kDownTileTokens / 16];
    auto row_ptr = [&](int item, int r, int lr) {
        return W + static_cast<int64_t>(row0 + 256 * item + 16 * r + lr) * rs;
    };
    auto src_row = [&](int t) -> int64_t { return pos0 + t; };
    uint16_t* out = sh ? a.o_sh16 : a.o16;
    const int64_t ldo = sh ? a.H : a.ldo;
    auto epi = [&](int item, floatx4 (&acc)[kRT][kDownTileTokens / 16]) {
        const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
#pragma unroll
        for (int r = 0; r < kRT; r++) {
#pragma unroll
            for (int n = 0; n < kDownTileTokens / 16; n++) {
                const int t = 16 * n + lr;
                if (t < count) {
                    const floatx4 v = acc[r][n];
                    *reinterpret_cast<uint2*>(out + static_cast<int64_t>(pos0 + t) * ldo + row0 + 256 * item +
                                              16 * r + 4 * q) = make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3]));
                }
            }
        }
    };
    gemm_tile<TYPE, kDownTileTokens>(bufs, acc, nb, a.down_slabs, count, sh ? a.h_sh16 : a.h16, inter, src_row,
                                     row_ptr, epi);
}

// ---------------------------------------------------------------------------------------------------------------
// Calls of at most kKsTile tokens (batched decode). Every tile then holds at most 64 tokens, and the kernels above
// give a tile's rows to few workgroups (one per 128 gate_up rows, per 512 down rows), each running the whole K
// loop while most CUs idle. Here a workgroup takes fewer rows and splits their K loop over its wavefronts:
// wavefront w = KQ rg + kq holds row group rg (kRT row tiles of 16) and computes the 256-value blocks kc with
// kc % KQ == kq. Phase p stages the KQ chunks p KQ .. p KQ + KQ - 1 of the tile's activations at once, one LDS slot
// each, and wavefront kq computes chunk p KQ + kq; the row states of its next chunk are requested as a phase
// starts computing. After the last phase the KQ partial sums of a row group are added in kq order (a fixed order,
// so results do not depend on timing) through LDS, and wavefront kq = 0 stores them.
constexpr int kKsTile = 64;

template <int TYPE, int NT, int KQ, typename RowPtr>
__device__ __forceinline__ void gemm_ksplit(uint8_t* lds, floatx4 (&acc)[kRT][kKsTile / 16], int nblocks,
                                            const uint8_t* src, const uint32_t* rowtab, RowPtr row_ptr, int lr,
                                            int q) {
    constexpr int NTA = kKsTile / 16;
    constexpr int kChunk = NT * kGemmWaves * 1024;  // one chunk: NT token tiles of 16 tokens x 256 values
    static_assert(NT <= NTA && kGemmWaves % KQ == 0, "");
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)), half = lane >> 5;
    const int kq = wv % KQ;
    const uint32_t col = 16u * static_cast<uint32_t>((lane & 31) ^ ((2 * wv + half) & swizzle<TYPE>()));
    const uint32_t lds0 = lds_address(lds);
    const BAddr ba = b_addr<TYPE>(lr, q);
    const int nphase = nblocks / KQ;
    RowState<TYPE> rs[kRT], nx[kRT];
#pragma unroll
    for (int r = 0; r < kRT; r++) rs[r].fetch(row_ptr(r, lr) + static_cast<int64_t>(kq) * BlockInfo<TYPE>::bytes, q);
    bf16x8 a0[kRT], a1[kRT], b[NT];
    for (int p = 0; p < nphase; p++) {
        if (p > 0) __syncthreads();  // every wavefront is done with the previous phase's chunks
        for (int c = 0; c < KQ; c++)
            stage_async<kKsTile, NT>(lds0 + c * kChunk, src + static_cast<int64_t>(p * KQ + c) * kTileRowBytes, rowtab,
                                     col, wv, half);
        wait_stage();  // the phase's chunks and this wavefront's row states have landed
        __syncthreads();
        if (p + 1 < nphase) {
#pragma unroll
            for (int r = 0; r < kRT; r++)
                nx[r].fetch(row_ptr(r, lr) + static_cast<int64_t>((p + 1) * KQ + kq) * BlockInfo<TYPE>::bytes, q);
        }
        const uint8_t* buf = lds + kq * kChunk;
        read_b<TYPE, NT, 0>(buf, ba, b);
#pragma unroll
        for (int r = 0; r < kRT; r++) {
            rs[r].prepare(q);
            a0[r] = rs[r].template frag<0>(q);
        }
        gemm_step<TYPE, NT, 0, NTA>(buf, ba, rs, acc, a0, b, a1, q);
        gemm_step<TYPE, NT, 1, NTA>(buf, ba, rs, acc, a1, b, a0, q);
        gemm_step<TYPE, NT, 2, NTA>(buf, ba, rs, acc, a0, b, a1, q);
        gemm_step<TYPE, NT, 3, NTA>(buf, ba, rs, acc, a1, b, a0, q);
        gemm_step<TYPE, NT, 4, NTA>(buf, ba, rs, acc, a0, b, a1, q);
        gemm_step<TYPE, NT, 5, NTA>(buf, ba, rs, acc, a1, b, a0, q);
        gemm_step<TYPE, NT, 6, NTA>(buf, ba, rs, acc, a0, b, a1, q);
        gemm_step<TYPE, NT, 7, NTA>(buf, ba, rs, acc, a1, b, a0, q);
        if (p + 1 < nphase) {
#pragma unroll
            for (int r = 0; r < kRT; r++) rs[r] = nx[r];
        }
    }
    // the partial sums of wavefronts kq > 0 cross through the (now free) staging slots
    __syncthreads();
    floatx4* red = reinterpret_cast<floatx4*>(lds);
    const int rg = wv / KQ;
    auto slot = [&](int j, int r, int n) { return (((rg * (KQ - 1) + j - 1) * kRT + r) * NT + n) * 64 + lane; };
    if (kq > 0) {
#pragma unroll
        for (int r = 0; r < kRT; r++)
#pragma unroll
            for (int n = 0; n < NT; n++) red[slot(kq, r, n)] = acc[r][n];
    }
    __syncthreads();
    if (kq == 0) {
        for (int j = 1; j < KQ; j++) {
#pragma unroll
            for (int r = 0; r < kRT; r++)
#pragma unroll
                for (int n = 0; n < NT; n++) {
                    const floatx4 v = red[slot(j, r, n)];
                    acc[r][n] = floatx4{acc[r][n][0] + v[0], acc[r][n][1] + v[1], acc[r][n][2] + v[2],
                                        acc[r][n][3] + v[3]};
                }
        }
    }
}

// The tile's activation rows (src_row(t), t < count, for rows of ld values) into rowtab; then the K-split loop for
// the fewest token tiles covering count (1 or 4).
template <int TYPE, int KQ, typename RowPtr, typename SrcRow>
__device__ __forceinline__ void gemm_tile_ks(uint8_t* lds, floatx4 (&acc)[kRT][kKsTile / 16], int nblocks,
                                             int count, const uint16_t* __restrict__ src, int64_t ld, SrcRow src_row,
                                             RowPtr row_ptr) {
    __shared__ __attribute__((aligned(16))) uint32_t rowtab[kKsTile];
    const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
    for (int t = threadIdx.x; t < kKsTile; t += blockDim.x)
        rowtab[rowtab_index<kKsTile>(t)] = static_cast<uint32_t>(src_row(t < count ? t : 0) * ld * 2);
#pragma unroll
    for (int r = 0; r < kRT; r++)
#pragma unroll
        for (int n = 0; n < kKsTile / 16; n++) acc[r][n] = floatx4{0.f, 0.f, 0.f, 0.f};
    __syncthreads();
    const uint8_t* s8 = uniform_ptr(reinterpret_cast<const uint8_t*>(src));
    if (count > 16)
        gemm_ksplit<TYPE, 4, KQ>(lds, acc, nblocks, s8, rowtab, row_ptr, lr, q);
    else
        gemm_ksplit<TYPE, 1, KQ>(lds, acc, nblocks, s8, rowtab, row_ptr, lr, q);
}

// gate_up, K split KQ ways: a workgroup takes kGemmWaves / KQ row groups, group rg the 16 gate rows
// j0 = slab * kSlab + 16 rg .. + 15 and the matching up rows (kSlab = 16 kGemmWaves / KQ; the host passes the
// number of such slabs of the widest intermediate dim in nslab_gate_up). Epilogue as k_gemm_gate_up's.
template <int TYPE, int KQ>
__global__ __launch_bounds__(kGemmThreads) void k_gemm_gate_up_ks(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[KQ * kKsTile * kTileRowBytes];
    static_assert(kRT == 2, "one gate and one up row tile per wavefront");
    constexpr int kSlab = 16 * kGemmWaves / KQ;
    if (a.skip && *a.skip) return;
    int slab, ti;
    slab_tile(a.nslab_gate_up, slab, ti);
    if (ti >= a.n_tiles[0]) return;
    const int4 tile = a.tiles[ti];
    const bool sh = tile.x == a.E;
    const int inter = sh ? a.sh_inter : a.inter;
    if (slab * kSlab >= inter) return;
    const int wv = static_cast<int>(threadIdx.x >> 6), rg = wv / KQ, kq = wv % KQ;
    const int j0 = slab * kSlab + 16 * rg;
    const uint8_t* W = sh ? a.sh_gate_up : a.gate_up + static_cast<int64_t>(tile.x) * a.gate_up_stride;
    const int nb = a.H / kQK;
    const int64_t rs = static_cast<int64_t>(nb) * BlockInfo<TYPE>::bytes;
    const int pos0 = tile.y, count = tile.z;
    floatx4 acc[kRT][kKsTile / 16];
    auto row_ptr = [&](int r, int lr) { return W + static_cast<int64_t>((r == 0 ? 0 : inter) + j0 + lr) * rs; };
    auto src_row = [&](int t) -> int64_t { return sh ? pos0 + t : a.sorted[pos0 + t] / a.k; };
    gemm_tile_ks<TYPE, KQ>(lds, acc, nb, count, a.xb, a.H, src_row, row_ptr);
    if (kq != 0) return;
    uint16_t* out = sh ? a.h_sh16 : a.h16;
    const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
#pragma unroll
    for (int n = 0; n < kKsTile / 16; n++) {
        const int t = 16 * n + lr;
        if (t < count) {
            const floatx4 g = acc[0][n], u = acc[1][n];
            *reinterpret_cast<uint2*>(out + static_cast<int64_t>(pos0 + t) * inter + j0 + 4 * q) =
                make_uint2(swiglu_bf16(g[0], u[0], g[1], u[1]), swiglu_bf16(g[2], u[2], g[3], u[3]));
        }
    }
}

// down, K split KQ ways: a workgroup takes the kRows = 16 kRT kGemmWaves / KQ output rows group * kRows .. + kRows
// - 1, row group rg the 16 kRT rows from group * kRows + 16 kRT rg. Epilogue as k_gemm_down's.
template <int TYPE, int KQ>
__global__ __launch_bounds__(kGemmThreads) void k_gemm_down_ks(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[KQ * kKsTile * kTileRowBytes];
    constexpr int kRows = 16 * kRT * kGemmWaves / KQ;
    if (a.skip && *a.skip) return;
    int group, ti;
    slab_tile(a.H / kRows, group, ti);
    if (ti >= a.n_tiles_down[0]) return;
    const int4 tile = a.tiles_down[ti];
    const bool sh = tile.x == a.E;
    const int inter = sh ? a.sh_inter : a.inter;
    const int wv = static_cast<int>(threadIdx.x >> 6), rg = wv / KQ, kq = wv % KQ;
    const int row0 = group * kRows + 16 * kRT * rg;
    const uint8_t* W = sh ? a.sh_down : a.down + static_cast<int64_t>(tile.x) * a.down_stride;
    const int nb = inter / kQK;
    const int64_t rs = static_cast<int64_t>(nb) * BlockInfo<TYPE>::bytes;
    const int pos0 = tile.y, count = tile.z;
    floatx4 acc[kRT][kKsTile / 16];
    auto row_ptr = [&](int r, int lr) { return W + static_cast<int64_t>(row0 + 16 * r + lr) * rs; };
    auto src_row = [&](int t) -> int64_t { return pos0 + t; };
    gemm_tile_ks<TYPE, KQ>(lds, acc, nb, count, sh ? a.h_sh16 : a.h16, inter, src_row, row_ptr);
    if (kq != 0) return;
    uint16_t* out = sh ? a.o_sh16 : a.o16;
    const int64_t ldo = sh ? a.H : a.ldo;
    const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
#pragma unroll
    for (int r = 0; r < kRT; r++) {
#pragma unroll
        for (int n = 0; n < kKsTile / 16; n++) {
            const int t = 16 * n + lr;
            if (t < count) {
                const floatx4 v = acc[r][n];
                *reinterpret_cast<uint2*>(out + static_cast<int64_t>(pos0 + t) * ldo + row0 + 16 * r + 4 * q) =
                    make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3]));
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------

int launch_router_tiled(const WlMoeLayer& L, const float* x, int64_t T, float* logits, float* sg, uint16_t* xb,
                        hipStream_t s) {
    const float* shared_gate = (L.shared_gate_up && L.shared_gate) ? L.shared_gate : nullptr;
    // with whole 64-row tiles of experts the shared gate is computed by the workgroups' VALU (gate_row) instead of
    // as a 1-row tile
    const bool separate = shared_gate && L.n_experts % 64 == 0;
    const float* tiled_gate = separate ? nullptr : shared_gate;
    const int rows = L.n_experts + (tiled_gate ? 1 : 0);
    const unsigned rtiles = static_cast<unsigned>((rows + 63) / 64);
    k_router_mfma<kRouterMfmaTM><<<dim3(static_cast<unsigned>((T + 32 * kRouterMfmaTM - 1) / (32 * kRouterMfmaTM)),
                                        rtiles),
                                   256, 0, s>>>(x, L.router, L.router_bias, tiled_gate, static_cast<int>(T), L.hidden,
                                                L.n_experts, logits, sg, xb, separate ? shared_gate : nullptr);
    return launch_status();
}

// The most GEMM tiles a call can need: an MFMA expert holds c > gemv_max pairs and ceil(c / cap) tiles, at most
// c / cap + 1, so the routed tiles number at most P / cap + (experts that can hold more than gemv_max pairs).
int max_tiles(const WlMoeLayer& L, int64_t T, int cap, int gemv_max) {
    const int64_t P = T * L.top_k;
    const int64_t big = P / (static_cast<int64_t>(gemv_max) + 1);
    const int64_t routed = (P + cap - 1) / cap + (big < L.n_experts ? big : L.n_experts);
    const int64_t shared = L.shared_gate_up ? (T + cap - 1) / cap : 0;
    return static_cast<int>(routed + shared);
}

// 256-row slabs per down workgroup: several when there are enough tiles to fill the GPU with fewer workgroups, so
// that each pays its pipeline start (and, with inter <= 512, its activation staging) once for several slabs.
// Up to kDownFewTokens tokens (batched decode) always two: the grid is sized by the tile bound, most of its
// workgroups find no tile, and with one workgroup per CU those are dispatched only as the working ones finish
// (64 tokens, Zipf routing: 85.3 us per layer against 87.4 with one slab, 100.2 with four).
constexpr int64_t kDownMinGroups = 1024;
constexpr int64_t kDownFewTokens = 256;
static int down_slabs(const WlMoeLayer& L, int64_t T) {
    const int nslab = L.hidden / 256;
    const int64_t tiles = (T * L.top_k + kDownTileTokens - 1) / kDownTileTokens;  // about the full tiles
    if (T <= kDownFewTokens && nslab % 2 == 0) return 2;
    int p = 1;
    while (p < kDownSlabsMax && nslab % (2 * p) == 0 && tiles * nslab / (2 * p) >= kDownMinGroups) p *= 2;
    return p;
}

static PrefillArgs prefill_args(const WlMoeLayer& L, int64_t T, const Workspace& w) {
    const bool shared = L.shared_gate_up != nullptr;
    PrefillArgs a{};
    a.gate_up = static_cast<const uint8_t*>(L.gate_up);
    a.gate_up_stride = L.gate_up_stride;
    a.down = static_cast<const uint8_t*>(L.down);
    a.down_stride = L.down_stride;
    a.sh_gate_up = static_cast<const uint8_t*>(L.shared_gate_up);
    a.sh_down = static_cast<const uint8_t*>(L.shared_down);
    a.xb = w.xb;
    a.sorted = w.sorted;
    a.tiles = w.tiles;
    a.n_tiles = w.n_tiles;
    a.tiles_down = w.tiles_down;
    a.n_tiles_down = w.n_tiles + 1;
    a.h16 = w.h16;
    a.h_sh16 = w.h_sh16;
    // the routed outputs share the fp32 buffer with the GEMV experts' outputs: position pos's bf16 row fills the
    // first half of its fp32 row (stride 2 H values)
    a.o16 = reinterpret_cast<uint16_t*>(w.o);
    a.ldo = 2 * static_cast<int64_t>(L.hidden);
    a.o_sh16 = reinterpret_cast<uint16_t*>(w.o_sh);
    a.H = L.hidden;
    a.inter = L.inter;
    a.sh_inter = shared ? L.shared_inter : 0;
    a.E = L.n_experts;
    a.k = L.top_k;
    const int inter_max = shared && L.shared_inter > L.inter ? L.shared_inter : L.inter;
    a.nslab_gate_up = (inter_max + 127) / 128;
    a.down_slabs = down_slabs(L, T);
    return a;
}

static int tiles8(const WlMoeLayer& L, int64_t T, int cap, int gemv_max) {
    return (max_tiles(L, T, cap, gemv_max) + kXcds - 1) / kXcds * kXcds;
}

// The K-split kernels' ways: gate_up (K = hidden) 4, or 2 when GEMV experts run beside it (half the LDS per
// workgroup, 64 KiB, so the GEMV workgroups still find room on its CUs), down (K = the expert width) 2.
constexpr int kKsGateUp = 4, kKsGateUpBeside = 2, kKsDown = 2;
template <int KQ>
constexpr int ks_slab() { return 16 * kGemmWaves / KQ; }  // gate rows per k_gemm_gate_up_ks<., KQ> workgroup
constexpr int kKsRows = 16 * kRT * kGemmWaves / kKsDown;  // output rows per k_gemm_down_ks workgroup

// Whether a call runs the K-split kernels: at most kKsTile tokens (so every tile holds at most that many), and
// shapes whose block counts divide into the ways and whose rows divide into the workgroups' row sets (the larger
// gate_up slab, of the 2-way kernel, is a multiple of the other).
static bool ks_eligible(const WlMoeLayer& L, int64_t T) {
    static_assert(ks_slab<kKsGateUpBeside>() % ks_slab<kKsGateUp>() == 0 && kKsGateUp % kKsGateUpBeside == 0, "");
    if (T > kKsTile) return false;
    auto inter_ok = [](int inter) {
        return inter % ks_slab<kKsGateUpBeside>() == 0 && (inter / kQK) % kKsDown == 0;
    };
    return (L.hidden / kQK) % kKsGateUp == 0 && L.hidden % kKsRows == 0 && inter_ok(L.inter) &&
           (!L.shared_gate_up || inter_ok(L.shared_inter));
}

template <int KQ>
static int launch_gate_up_ks(const WlMoeLayer& L, int64_t T, PrefillArgs a, int gemv_max, hipStream_t s) {
    const int inter_max = a.sh_inter > a.inter ? a.sh_inter : a.inter;
    a.nslab_gate_up = (inter_max + ks_slab<KQ>() - 1) / ks_slab<KQ>();
    const dim3 grid(static_cast<unsigned>(a.nslab_gate_up * tiles8(L, T, kTileTokens, gemv_max)));
    if (L.gate_up_type == WL_TYPE_Q4_K)
        k_gemm_gate_up_ks<WL_TYPE_Q4_K, KQ><<<grid, kGemmThreads, 0, s>>>(a);
    else
        k_gemm_gate_up_ks<WL_TYPE_Q6_K, KQ><<<grid, kGemmThreads, 0, s>>>(a);
    return launch_status();
}

// The MFMA experts' gate_up + SwiGLU (the routed experts with more than gemv_max pairs and the shared expert).
// The routed and shared experts share one launch, so their types must agree (checked by prefill_eligible).
int launch_mfma_gate_up(const WlMoeLayer& L, int64_t T, const Workspace& w, int gemv_max, bool with_gemv,
                        const uint32_t* skip, hipStream_t s) {
    PrefillArgs a = prefill_args(L, T, w);
    a.skip = skip;
    if (ks_eligible(L, T))
        return with_gemv ? launch_gate_up_ks<kKsGateUpBeside>(L, T, a, gemv_max, s)
                         : launch_gate_up_ks<kKsGateUp>(L, T, a, gemv_max, s);
    if (L.gate_up_type == WL_TYPE_Q4_K)
        k_gemm_gate_up<WL_TYPE_Q4_K, kTileTokens>
            <<<dim3(static_cast<unsigned>(a.nslab_gate_up * tiles8(L, T, kTileTokens, gemv_max))), kGemmThreads, 0,
               s>>>(a);
    else
        k_gemm_gate_up<WL_TYPE_Q6_K, kDownTileTokens>
            <<<dim3(static_cast<unsigned>(a.nslab_gate_up * tiles8(L, T, kDownTileTokens, gemv_max))), kGemmThreads,
               0, s>>>(a);
    return launch_status();
}

// The MFMA experts' down products.
int launch_mfma_down(const WlMoeLayer& L, int64_t T, const Workspace& w, int gemv_max, const uint32_t* skip,
                     hipStream_t s) {
    PrefillArgs a = prefill_args(L, T, w);
    a.skip = skip;
    if (ks_eligible(L, T)) {
        const dim3 grid(static_cast<unsigned>(L.hidden / kKsRows * tiles8(L, T, kDownTileTokens, gemv_max)));
        if (L.down_type == WL_TYPE_Q4_K)
            k_gemm_down_ks<WL_TYPE_Q4_K, kKsDown><<<grid, kGemmThreads, 0, s>>>(a);
        else
            k_gemm_down_ks<WL_TYPE_Q6_K, kKsDown><<<grid, kGemmThreads, 0, s>>>(a);
        return launch_status();
    }
    const dim3 g2(static_cast<unsigned>(L.hidden / 256 / a.down_slabs * tiles8(L, T, kDownTileTokens, gemv_max)));
    if (L.down_type == WL_TYPE_Q4_K)
        k_gemm_down<WL_TYPE_Q4_K><<<g2, kGemmThreads, 0, s>>>(a);
    else
        k_gemm_down<WL_TYPE_Q6_K><<<g2, kGemmThreads, 0, s>>>(a);
    return launch_status();
}

// y[t, :] = W x[t, :] for a single quantized matrix on the down GEMM: bf16 operands (x as given, W's exact values
// rounded to bf16 in registers), fp32 accumulation, bf16 output. rows and k are multiples of 256.
int launch_linear(int type, const uint8_t* w, int rows, int k, const uint16_t* x, int64_t T, uint16_t* y,
                  hipStream_t s) {
    PrefillArgs a{};
    a.down = w;
    a.down_stride = 0;
    a.h16 = const_cast<uint16_t*>(x);
    a.o16 = y;
    a.ldo = rows;
    a.H = rows;
    a.inter = k;
    a.E = 1;  // the one matrix is expert 0, never the shared slot
    a.down_slabs = 1;
    a.dense_tokens = static_cast<int>(T);
    const int tiles = static_cast<int>((T + kDownTileTokens - 1) / kDownTileTokens);
    const dim3 grid(static_cast<unsigned>(rows / 256 * ((tiles + kXcds - 1) / kXcds * kXcds)));
    if (type == WL_TYPE_Q4_K)
        k_gemm_down<WL_TYPE_Q4_K><<<grid, kGemmThreads, 0, s>>>(a);
    else
        k_gemm_down<WL_TYPE_Q6_K><<<grid, kGemmThreads, 0, s>>>(a);
    return launch_status();
}

// Whether the layer's shapes and types let the MFMA GEMMs run (expert_plan decides when they do).
bool prefill_eligible(const WlMoeLayer& L, int64_t T) {
    if (L.hidden % 256 != 0 || L.inter % 128 != 0) return false;
    if (L.shared_gate_up && (L.shared_gate_up_type != L.gate_up_type || L.shared_down_type != L.down_type ||
                             L.shared_inter % 128 != 0))
        return false;
    // the LDS staging addresses activation rows by 32-bit byte offsets
    const int64_t inter_max = L.shared_gate_up && L.shared_inter > L.inter ? L.shared_inter : L.inter;
    if (T * L.hidden * 2 >= (int64_t{1} << 31) || T * L.top_k * inter_max * 2 >= (int64_t{1} << 31)) return false;
    return true;
}

}  // namespace wl

extern "C" {

int wl_linear(int type, const void* w, int64_t rows, int64_t k, const uint16_t* x, int64_t tokens, uint16_t* y,
              void* stream) {
    using namespace wl;
    int rc = check_matrix(type, w, rows, k, wl_row_bytes(type, k));
    if (rc) return rc;
    if (!x || !y) return WL_EINVAL_NULL;
    if (tokens <= 0 || rows % 256 != 0) return WL_EINVAL_SHAPE;
    // the LDS staging addresses activation rows by 32-bit byte offsets
    if (tokens * k * 2 >= (int64_t{1} << 31) || tokens > kMaxTokens) return WL_EINVAL_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(y) % 16) return WL_EINVAL_ALIGN;
    if (type == WL_TYPE_Q4_K && reinterpret_cast<uintptr_t>(w) % 16) return WL_EINVAL_ALIGN;
    return launch_linear(type, static_cast<const uint8_t*>(w), static_cast<int>(rows), static_cast<int>(k), x,
                         tokens, y, static_cast<hipStream_t>(stream));
}

}  // extern "C"
