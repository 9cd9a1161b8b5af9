// Prefill (many tokens per expert): the expert products as grouped bf16 MFMA GEMMs.
//
// Replaces the reference's prefill branch: GGMLWeight.linear dequantizes the whole weight to bf16 and multiplies
// with torch (gguf/metal.py:401-408), once per expert (engines/base.py:534-591). Here no dequantized weight is
// ever written: each wavefront decodes its Q4_K / Q6_K rows straight into v_mfma_f32_16x16x32_bf16 A-operands in
// registers (fp32 value, rounded to bf16 like Tensor.to(torch.bfloat16)), while the tokens' activations (bf16) are
// staged in LDS as the B-operand. Accumulation is fp32.
//
//   k_router_tiled   logits for many tokens in the router's fixed order (64-value FMA segments, added left to right)
//   k_to_bf16        x -> bf16
//   k_tiles          per-expert tiles of up to 128 tokens (sorted positions), then the shared expert's
//   k_gemm_gate_up   per (tile, 128 intermediate rows): gate and up rows together, epilogue h = silu(g) * u -> bf16
//   k_gemm_down      per (tile, 256 output rows): o = down h, fp32, by sorted position (combined by k_combine)
//
// MFMA 16x16x32 bf16 operand layout (wave64): lane l holds A[l % 16][8 (l / 16) + i], B[8 (l / 16) + i][l % 16],
// and C[4 (l / 16) + i][l % 16], i < 8 (A, B) or < 4 (C). A wavefront covers 4 row tiles x 8 token tiles.
#include <hip/hip_runtime.h>

#include "wl_common.h"
#include "wl_host.h"
#include "wl_moe.h"
#include "wl_moe_dev.h"

namespace wl {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 256;              // k per staged chunk: one K-quant block per row
constexpr int kLdsRow = kBK + 8;      // bf16 per LDS row (16-byte pad: conflict-free B reads)

__device__ __forceinline__ uint32_t bf16_bits(float f) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f)));
}
__device__ __forceinline__ uint32_t pack2(float a, float b) { return bf16_bits(a) | (bf16_bits(b) << 16); }

// 8 bytes from a 2-byte-aligned address (3 aligned dwords, realigned); stays within [p - 2, p + 10).
__device__ __forceinline__ uint2 load8_a2(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t* q = reinterpret_cast<const uint32_t*>(a & ~static_cast<uintptr_t>(3));
    const uint32_t sh = static_cast<uint32_t>(a & 3u);
    const uint32_t w0 = q[0], w1 = q[1];
    const uint32_t w2 = sh ? q[2] : 0u;
    return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh));
}

// ---------------------------------------------------------------------------------------------------------------
// Router for many tokens. A workgroup computes a 64-token x 64-row tile (rows: experts, then the shared gate as row
// E); each thread 4 x 4 outputs. Per 64-value segment the operands are staged in LDS (transposed, so a thread's 4
// tokens / 4 rows are one 16-byte read) and every output chains 64 fused multiply-adds in ascending k; the
// segment partial is then added to the running total: the order of router_row and of the CPU replay.
__global__ __launch_bounds__(256) void k_router_tiled(const float* __restrict__ x, const float* __restrict__ w,
                                                      const float* __restrict__ bias,
                                                      const float* __restrict__ shared_gate, int T, int H, int E,
                                                      float* __restrict__ logits, float* __restrict__ sg) {
    __shared__ float xs[kRouterSeg][64];
    __shared__ float ws[kRouterSeg][64];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int t0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
    const int rows = E + (shared_gate ? 1 : 0);
    float seg[4][4], tot[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) tot[i][j] = 0.0f;
    const int nseg = H / kRouterSeg;
    for (int s = 0; s < nseg; s++) {
        __syncthreads();
        // stage: 64 tokens x 64 values and 64 rows x 64 values, transposed into [k][token] / [k][row]
        for (int i = tid; i < 64 * 16; i += 256) {
            const int rr = i >> 4, c4 = (i & 15) * 4;
            const int t = t0 + rr, r = r0 + rr;
            float4 xv = make_float4(0.f, 0.f, 0.f, 0.f), wv = make_float4(0.f, 0.f, 0.f, 0.f);
            if (t < T) xv = *reinterpret_cast<const float4*>(x + static_cast<int64_t>(t) * H + s * kRouterSeg + c4);
            if (r < rows) {
                const float* wr = r < E ? w + static_cast<int64_t>(r) * H : shared_gate;
                wv = *reinterpret_cast<const float4*>(wr + s * kRouterSeg + c4);
            }
            xs[c4 + 0][rr] = xv.x;
            xs[c4 + 1][rr] = xv.y;
            xs[c4 + 2][rr] = xv.z;
            xs[c4 + 3][rr] = xv.w;
            ws[c4 + 0][rr] = wv.x;
            ws[c4 + 1][rr] = wv.y;
            ws[c4 + 2][rr] = wv.z;
            ws[c4 + 3][rr] = wv.w;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) seg[i][j] = 0.0f;
#pragma unroll 8
        for (int kk = 0; kk < kRouterSeg; kk++) {
            const float4 xv = *reinterpret_cast<const float4*>(&xs[kk][4 * ty]);
            const float4 wv = *reinterpret_cast<const float4*>(&ws[kk][4 * tx]);
            const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
            const float wa[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) seg[i][j] = __builtin_fmaf(xa[i], wa[j], seg[i][j]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) tot[i][j] = s == 0 ? seg[i][j] : __fadd_rn(tot[i][j], seg[i][j]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int t = t0 + 4 * ty + i;
        if (t >= T) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = r0 + 4 * tx + j;
            if (r < E)
                logits[static_cast<int64_t>(t) * E + r] = bias ? __fadd_rn(tot[i][j], bias[r]) : tot[i][j];
            else if (r == E && shared_gate)
                sg[t] = sigmoid(tot[i][j]);
        }
    }
}

// x fp32 -> bf16, 8 values per thread.
__global__ __launch_bounds__(256) void k_to_bf16(const float* __restrict__ x, uint16_t* __restrict__ xb, int64_t n8) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n8) return;
    const float4 a = reinterpret_cast<const float4*>(x)[2 * i];
    const float4 b = reinterpret_cast<const float4*>(x)[2 * i + 1];
    reinterpret_cast<uint4*>(xb)[i] = make_uint4(pack2(a.x, a.y), pack2(a.z, a.w), pack2(b.x, b.y), pack2(b.z, b.w));
}

// Tiles of up to kTileTokens tokens: each routed expert's sorted positions, then the shared expert's tokens
// (expert id E). tiles[i] = (expert, first position or token, count); n_tiles[0] = how many.
// One workgroup of 256 threads, thread i owning experts 4i .. 4i + 3 (E <= 1024): tile counts, an exclusive scan
// of them across the workgroup, then each thread writes its experts' tiles in expert order.
__global__ __launch_bounds__(256) void k_tiles(const int32_t* __restrict__ offsets, int E, int T, int with_shared,
                                               int4* __restrict__ tiles, int32_t* __restrict__ n_tiles) {
    __shared__ int scan[2][256];
    const int tid = threadIdx.x;
    int cnt[4], mine = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = 4 * tid + i;
        cnt[i] = e < E ? (offsets[e + 1] - offsets[e] + kTileTokens - 1) / kTileTokens : 0;
        mine += cnt[i];
    }
    int cur = 0;
    scan[0][tid] = mine;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        const int v = scan[cur][tid] + (tid >= off ? scan[cur][tid - off] : 0);
        scan[cur ^ 1][tid] = v;
        cur ^= 1;
        __syncthreads();
    }
    int n = scan[cur][tid] - mine;  // tiles before this thread's experts
    const int total = scan[cur][255];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = 4 * tid + i;
        if (e >= E) break;
        const int b = offsets[e], c = offsets[e + 1] - b;
        for (int p = 0; p < c; p += kTileTokens) tiles[n++] = make_int4(e, b + p, min(kTileTokens, c - p), 0);
    }
    int m = total;
    if (with_shared)
        for (int p = tid * kTileTokens; p < T; p += 256 * kTileTokens)
            tiles[total + p / kTileTokens] = make_int4(E, p, min(kTileTokens, T - p), 0);
    if (with_shared) m += (T + kTileTokens - 1) / kTileTokens;
    if (tid == 0) n_tiles[0] = m;
}

// Stages a tile's activations [count tokens][kBK values from k0] (bf16) into LDS; rows past count are zero.
// rows[t] is the row of token t of the tile in `src` ([*, ld] bf16). All of a thread's loads are issued before
// any is stored (a blockDim of 256 gives 16 each).
__device__ __forceinline__ void stage_tile(uint16_t* lds, const uint16_t* __restrict__ src, int64_t ld, int k0,
                                           int count, const int* rows) {
    constexpr int kPer = kTileTokens * (kBK / 8) / 256;
    uint4 v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; u++) {
        const int i = threadIdx.x + 256 * u;
        const int t = i / (kBK / 8), c8 = (i % (kBK / 8)) * 8;
        v[u] = make_uint4(0u, 0u, 0u, 0u);
        if (t < count) v[u] = *reinterpret_cast<const uint4*>(src + static_cast<int64_t>(rows[t]) * ld + k0 + c8);
    }
#pragma unroll
    for (int u = 0; u < kPer; u++) {
        const int i = threadIdx.x + 256 * u;
        const int t = i / (kBK / 8), c8 = (i % (kBK / 8)) * 8;
        *reinterpret_cast<uint4*>(lds + t * kLdsRow + c8) = v[u];
    }
}

// ---------------------------------------------------------------------------------------------------------------
// A-operand decoders: the 8 values k = 32*kk + 8*q + i (i < 8) of one row's K-quant block as bf16, for every kk of
// the block. The per-block state is fetched once (fetch), then each kk is unpacked (fragment).
struct Q4KRowState {
    uint4 hd;      // d, dmin, 12 scale bytes
    uint2 qs[4];   // qs bytes 32m + 8q .. +7, m < 4
};

__device__ __forceinline__ void fetch_q4k(const uint8_t* __restrict__ blk, int q, Q4KRowState& s) {
    s.hd = *reinterpret_cast<const uint4*>(blk);
#pragma unroll
    for (int m = 0; m < 4; m++) s.qs[m] = *reinterpret_cast<const uint2*>(blk + 16 + 32 * m + 8 * q);
}

// v & 0x0F0F0F0F as an opaque value, so the byte conversions below stay single v_cvt_f32_ubyteN instructions
__device__ __forceinline__ uint32_t nibbles(uint32_t v) {
    uint32_t r;
    asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(v));
    return r;
}

// 4 bytes of w (values 0..255) as bf16 of a * q + b, packed two per dword
__device__ __forceinline__ void affine4(uint32_t w, float a, float b, uint32_t& p0, uint32_t& p1) {
    p0 = pack2(__builtin_fmaf(a, ubyte(w, 0), b), __builtin_fmaf(a, ubyte(w, 1), b));
    p1 = pack2(__builtin_fmaf(a, ubyte(w, 2), b), __builtin_fmaf(a, ubyte(w, 3), b));
}

template <int KK>
__device__ __forceinline__ bf16x8 fragment_q4k(const Q4KRowState& s) {
    const float d = half_to_float(s.hd.x), dmin = half_to_float(s.hd.x >> 16);
    uint32_t sc, m;
    q4k_scale_min(KK, s.hd.y, s.hd.z, s.hd.w, sc, m);
    const float a = d * static_cast<float>(sc), b = -(dmin * static_cast<float>(m));
    const uint2 raw = s.qs[KK >> 1];
    constexpr uint32_t sh = 4 * (KK & 1);
    const uint32_t lo = nibbles(raw.x >> sh), hi = nibbles(raw.y >> sh);
    uint4 p;
    affine4(lo, a, b, p.x, p.y);
    affine4(hi, a, b, p.z, p.w);
    return __builtin_bit_cast(bf16x8, p);
}

struct Q6KRowState {
    uint2 ql[4];   // ql bytes 64h + 32t2 + 8q .. +7, index 2h + t2
    uint2 qh[2];   // qh bytes 32h + 8q .. +7
    uint4 sc;      // the 16 int8 scales
    float d;
};

__device__ __forceinline__ void fetch_q6k(const uint8_t* __restrict__ blk, int q, Q6KRowState& s) {
#pragma unroll
    for (int m = 0; m < 4; m++) s.ql[m] = load8_a2(blk + 64 * (m >> 1) + 32 * (m & 1) + 8 * q);
#pragma unroll
    for (int h = 0; h < 2; h++) s.qh[h] = load8_a2(blk + 128 + 32 * h + 8 * q);
    // scales: bytes 192..207 from dwords of their aligned start; the fifth dword (needed only when the block starts
    // 2 bytes into a dword) ends at byte 210, the block's end
    const uintptr_t a = reinterpret_cast<uintptr_t>(blk + 192);
    const uint32_t* p = reinterpret_cast<const uint32_t*>(a & ~static_cast<uintptr_t>(3));
    const uint32_t sh = static_cast<uint32_t>(a & 3u);
    const uint32_t w0 = p[0], w1 = p[1], w2 = p[2], w3 = p[3];
    const uint32_t w4 = sh ? p[4] : 0u;
    s.sc = make_uint4(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh),
                      __builtin_amdgcn_alignbyte(w3, w2, sh), __builtin_amdgcn_alignbyte(w4, w3, sh));
    s.d = half_to_float(*reinterpret_cast<const uint16_t*>(blk + 208));
}

template <int KK>
__device__ __forceinline__ bf16x8 fragment_q6k(const Q6KRowState& s, int q) {
    // values e = 32 kk + 8 q + i: half h = kk / 4, quarter t = kk % 4, scale index e / 16 = 2 kk + q / 2; the
    // scale word holds indices 4w .. 4w + 3 with w = kk / 2, and q / 2 picks one of the two in this kk's half
    constexpr int h = KK >> 2, t = KK & 3;
    const uint2 l4 = s.ql[2 * h + (t & 1)];
    const uint2 h2 = s.qh[h];
    constexpr uint32_t lsh = 4 * (t >> 1), hsh = 2 * t;
    const uint32_t scw = (KK >> 1) == 0 ? s.sc.x : (KK >> 1) == 1 ? s.sc.y : (KK >> 1) == 2 ? s.sc.z : s.sc.w;
    const uint32_t sbyte = (scw >> (8 * (2 * (KK & 1) + (q >> 1)))) & 0xFFu;
    const float a = s.d * static_cast<float>(static_cast<int8_t>(sbyte));
    const float b = -32.0f * a;  // exact: a has at most 18 significant bits
    const uint32_t v0 = nibbles(l4.x >> lsh) | ((nibbles(h2.x >> hsh) & 0x03030303u) << 4);
    const uint32_t v1 = nibbles(l4.y >> lsh) | ((nibbles(h2.y >> hsh) & 0x03030303u) << 4);
    // a * (q - 32) == fma(a, q, -32 a): the product a * q is exact, so both round the same sum once
    uint4 p;
    affine4(v0, a, b, p.x, p.y);
    affine4(v1, a, b, p.z, p.w);
    return __builtin_bit_cast(bf16x8, p);
}

template <int TYPE>
struct RowState;
template <>
struct RowState<WL_TYPE_Q4_K> {
    Q4KRowState s;
    __device__ __forceinline__ void fetch(const uint8_t* blk, int q) { fetch_q4k(blk, q, s); }
    template <int KK>
    __device__ __forceinline__ bf16x8 frag(int) const { return fragment_q4k<KK>(s); }
};
template <>
struct RowState<WL_TYPE_Q6_K> {
    Q6KRowState s;
    __device__ __forceinline__ void fetch(const uint8_t* blk, int q) { fetch_q6k(blk, q, s); }
    template <int KK>
    __device__ __forceinline__ bf16x8 frag(int q) const { return fragment_q6k<KK>(s, q); }
};

// One 32-value step of the K chunk: 4 A-fragments decoded from the row states, then the token tiles in groups of 4
// (all 4 B-fragments read from LDS before their 16 MFMAs); groups past the tile's tokens are skipped.
template <int TYPE, int KK>
__device__ __forceinline__ void gemm_step(const uint16_t* lds, const RowState<TYPE> (&rs)[4], floatx4 (&acc)[4][8],
                                          int ngroups, int lr, int q) {
    bf16x8 af[4];
#pragma unroll
    for (int r = 0; r < 4; r++) af[r] = rs[r].template frag<KK>(q);
#pragma unroll
    for (int g = 0; g < 2; g++) {
        if (g < ngroups) {
            bf16x8 bf[4];
#pragma unroll
            for (int n = 0; n < 4; n++)
                bf[n] = *reinterpret_cast<const bf16x8*>(lds + (16 * (4 * g + n) + lr) * kLdsRow + 32 * KK + 8 * q);
#pragma unroll
            for (int n = 0; n < 4; n++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc[r][4 * g + n] =
                        __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[r], bf[n], acc[r][4 * g + n], 0, 0, 0);
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------
// The GEMM core: a workgroup of 4 wavefronts, each owning 4 row tiles of 16 (rows given by row_ptr(r, lr)) and
// the tile's (up to) 128 tokens as 8 token tiles. For each K chunk of 256 (one block per row) the activations are
// staged in LDS, every wavefront fetches its rows' blocks, and each of the 8 32-value steps decodes 4 A-fragments
// and runs up to 32 MFMAs.
template <int TYPE, typename RowPtr, typename SrcRow>
__device__ __forceinline__ void gemm_tile(uint16_t* lds, floatx4 (&acc)[4][8], int nblocks, int count,
                                          const uint16_t* __restrict__ src, int64_t ld, SrcRow src_row,
                                          RowPtr row_ptr) {
    __shared__ int rows[kTileTokens];
    const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
    const int ngroups = (count + 63) >> 6;
    for (int t = threadIdx.x; t < count; t += blockDim.x) rows[t] = static_cast<int>(src_row(t));
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int n = 0; n < 8; n++) acc[r][n] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int kc = 0; kc < nblocks; kc++) {
        __syncthreads();
        stage_tile(lds, src, ld, kc * kBK, count, rows);
        RowState<TYPE> rs[4];
#pragma unroll
        for (int r = 0; r < 4; r++) rs[r].fetch(row_ptr(r, lr) + static_cast<int64_t>(kc) * BlockInfo<TYPE>::bytes, q);
        __syncthreads();
        gemm_step<TYPE, 0>(lds, rs, acc, ngroups, lr, q);
        gemm_step<TYPE, 1>(lds, rs, acc, ngroups, lr, q);
        gemm_step<TYPE, 2>(lds, rs, acc, ngroups, lr, q);
        gemm_step<TYPE, 3>(lds, rs, acc, ngroups, lr, q);
        gemm_step<TYPE, 4>(lds, rs, acc, ngroups, lr, q);
        gemm_step<TYPE, 5>(lds, rs, acc, ngroups, lr, q);
        gemm_step<TYPE, 6>(lds, rs, acc, ngroups, lr, q);
        gemm_step<TYPE, 7>(lds, rs, acc, ngroups, lr, q);
    }
}

// gate_up: blockIdx.x = 128-row slab of the intermediate dim; wavefront w: gate rows j0 + 16r + lr (r = 0, 1)
// and the matching up rows inter + j0 + ... (r = 2, 3), j0 = 128 bx + 32 w. Epilogue h = silu(g) * u -> bf16.
template <int TYPE>
__global__ __launch_bounds__(256) void k_gemm_gate_up(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[kTileTokens * kLdsRow];
    if (static_cast<int>(blockIdx.y) >= a.n_tiles[0]) return;
    const int4 tile = a.tiles[blockIdx.y];
    const bool sh = tile.x == a.E;
    const int inter = sh ? a.sh_inter : a.inter;
    const int j0 = blockIdx.x * 128 + 32 * (threadIdx.x >> 6);
    if (static_cast<int>(blockIdx.x) * 128 >= inter) return;
    const uint8_t* W = sh ? a.sh_gate_up : a.gate_up + static_cast<int64_t>(tile.x) * a.gate_up_stride;
    const int nb = a.H / kQK;
    const int64_t rs = static_cast<int64_t>(nb) * BlockInfo<TYPE>::bytes;
    const int pos0 = tile.y, count = tile.z;
    floatx4 acc[4][8];
    auto row_ptr = [&](int r, int lr) {
        const int j = j0 + 16 * (r & 1) + lr;
        return W + static_cast<int64_t>((r < 2 ? 0 : inter) + j) * rs;
    };
    auto src_row = [&](int t) -> int64_t { return sh ? pos0 + t : a.sorted[pos0 + t] / a.k; };
    gemm_tile<TYPE>(lds, acc, nb, count, a.xb, a.H, src_row, row_ptr);
    const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
    uint16_t* out = sh ? a.h_sh16 : a.h16;
#pragma unroll
    for (int r = 0; r < 2; r++) {
#pragma unroll
        for (int n = 0; n < 8; n++) {
            const int t = 16 * n + lr;
            if (t < count) {
                const int j = j0 + 16 * r + 4 * q;
                const floatx4 g = acc[r][n], u = acc[r + 2][n];
                const uint2 v = make_uint2(pack2(silu(g[0]) * u[0], silu(g[1]) * u[1]),
                                           pack2(silu(g[2]) * u[2], silu(g[3]) * u[3]));
                *reinterpret_cast<uint2*>(out + static_cast<int64_t>(pos0 + t) * inter + j) = v;
            }
        }
    }
}

// down: blockIdx.x = 256-row slab of the hidden dim; wavefront w: rows r0 + 64 w + 16 r + lr. o fp32 by position.
template <int TYPE>
__global__ __launch_bounds__(256) void k_gemm_down(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[kTileTokens * kLdsRow];
    if (static_cast<int>(blockIdx.y) >= a.n_tiles[0]) return;
    const int4 tile = a.tiles[blockIdx.y];
    const bool sh = tile.x == a.E;
    const int inter = sh ? a.sh_inter : a.inter;
    const int row0 = blockIdx.x * 256 + 64 * (threadIdx.x >> 6);
    const uint8_t* W = sh ? a.sh_down : a.down + static_cast<int64_t>(tile.x) * a.down_stride;
    const int nb = inter / kQK;
    const int64_t rs = static_cast<int64_t>(nb) * BlockInfo<TYPE>::bytes;
    const int pos0 = tile.y, count = tile.z;
    floatx4 acc[4][8];
    auto row_ptr = [&](int r, int lr) { return W + static_cast<int64_t>(row0 + 16 * r + lr) * rs; };
    auto src_row = [&](int t) -> int64_t { return pos0 + t; };
    gemm_tile<TYPE>(lds, acc, nb, count, sh ? a.h_sh16 : a.h16, inter, src_row, row_ptr);
    const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
    float* out = sh ? a.o_sh : a.o;
#pragma unroll
    for (int r = 0; r < 4; r++) {
#pragma unroll
        for (int n = 0; n < 8; n++) {
            const int t = 16 * n + lr;
            if (t < count) {
                const floatx4 v = acc[r][n];
                *reinterpret_cast<float4*>(out + static_cast<int64_t>(pos0 + t) * a.H + row0 + 16 * r + 4 * q) =
                    make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------------------------

int launch_router_tiled(const WlMoeLayer& L, const float* x, int64_t T, float* logits, float* sg, hipStream_t s) {
    const float* shared_gate = (L.shared_gate_up && L.shared_gate) ? L.shared_gate : nullptr;
    const int rows = L.n_experts + (shared_gate ? 1 : 0);
    const dim3 grid(static_cast<unsigned>((T + 63) / 64), static_cast<unsigned>((rows + 63) / 64));
    k_router_tiled<<<grid, 256, 0, s>>>(x, L.router, L.router_bias, shared_gate, static_cast<int>(T), L.hidden,
                                        L.n_experts, logits, sg);
    return launch_status();
}

int max_tiles(const WlMoeLayer& L, int64_t T) {
    const int64_t P = T * L.top_k;
    const int64_t routed = (P + kTileTokens - 1) / kTileTokens + L.n_experts;
    const int64_t shared = L.shared_gate_up ? (T + kTileTokens - 1) / kTileTokens : 0;
    return static_cast<int>(routed + shared);
}

int launch_prefill_experts(const WlMoeLayer& L, const float* x, int64_t T, const Workspace& w, hipStream_t s) {
    const int64_t n8 = T * L.hidden / 8;
    k_to_bf16<<<static_cast<unsigned>((n8 + 255) / 256), 256, 0, s>>>(x, w.xb, n8);
    const bool shared = L.shared_gate_up != nullptr;
    k_tiles<<<1, 256, 0, s>>>(w.offsets, L.n_experts, static_cast<int>(T), shared ? 1 : 0, w.tiles, w.n_tiles);
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
    a.h16 = w.h16;
    a.h_sh16 = w.h_sh16;
    a.o = w.o;
    a.o_sh = w.o_sh;
    a.H = L.hidden;
    a.inter = L.inter;
    a.sh_inter = shared ? L.shared_inter : 0;
    a.E = L.n_experts;
    a.k = L.top_k;
    const int tiles = max_tiles(L, T);
    const int inter_max = shared && L.shared_inter > L.inter ? L.shared_inter : L.inter;
    const dim3 g1(static_cast<unsigned>((inter_max + 127) / 128), static_cast<unsigned>(tiles));
    // the routed and shared experts share one launch, so their types must agree (checked by prefill_eligible)
    if (L.gate_up_type == WL_TYPE_Q4_K)
        k_gemm_gate_up<WL_TYPE_Q4_K><<<g1, 256, 0, s>>>(a);
    else
        k_gemm_gate_up<WL_TYPE_Q6_K><<<g1, 256, 0, s>>>(a);
    const dim3 g2(static_cast<unsigned>(L.hidden / 256), static_cast<unsigned>(tiles));
    if (L.down_type == WL_TYPE_Q4_K)
        k_gemm_down<WL_TYPE_Q4_K><<<g2, 256, 0, s>>>(a);
    else
        k_gemm_down<WL_TYPE_Q6_K><<<g2, 256, 0, s>>>(a);
    return launch_status();
}

bool prefill_eligible(const WlMoeLayer& L, int64_t T) {
    if (L.flags & WL_MOE_NO_MFMA) return false;
    if (!(L.flags & WL_MOE_FORCE_MFMA) && T * L.top_k < static_cast<int64_t>(kMfmaMinTokensPerExpert) * L.n_experts)
        return false;
    if (L.hidden % 256 != 0 || L.inter % 128 != 0) return false;
    if (L.shared_gate_up && (L.shared_gate_up_type != L.gate_up_type || L.shared_down_type != L.down_type ||
                             L.shared_inter % 128 != 0))
        return false;
    return true;
}

}  // namespace wl
