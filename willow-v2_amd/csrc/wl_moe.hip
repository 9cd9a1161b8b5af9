// The MoE layer on the device: router, top-k, token->expert grouping, SwiGLU experts, weighted combine.
// Replaces engines/base.py:445-591 (Engine.moe, batched_decode_experts, each_expert, combine_decode_experts) and
// the Metal gemv_batch / gemv_combine launches it makes; routing never leaves the GPU (no host sync per layer).
#include <hip/hip_runtime.h>

#include <mutex>
#include <type_traits>

#include "wl_common.h"
#include "wl_host.h"
#include "wl_moe.h"
#include "wl_moe_dev.h"

namespace wl {

// ---------------------------------------------------------------------------------------------------------------
// Router. logits[t, e] = x[t] . W[e] (+ bias[e]) in a fixed order the CPU oracle replays exactly:
//   k is cut into segments of kRouterSeg consecutive values; each segment's partial is a chain of fused
//   multiply-adds in ascending k starting from 0; the partials are added left to right; then the bias.
// The shared-expert gate is row E (weight vector shared_gate, no bias); its output is sigmoid(logit).
// Small batches (2 tokens up to the tiled kernel's minimum) on the fp32 matrix core, the hidden dim split over the
// workgroup's wavefronts. A workgroup of 8 wavefronts computes one 16-token x 16-row tile (rows: experts, then the
// shared gate as row E). The 64-value segments are taken in rounds of 8 kRsDepth: wavefront w first loads segments
// 8 d + w (d < kRsDepth) of the round into registers, all at once, then for each d stages the 16 tokens' and 16 rows'
// values of its segment in its own LDS area as [j][token or row][s] (20-float rows) and runs 16 v_mfma_f32_16x16x4_f32
// from a zero accumulator: the segment's partial for all 256 outputs, each a fused multiply-add chain in ascending k
// (the instruction's four products are fused multiply-adds in k order, as k_router_mfma relies on). After the round,
// thread (token, row) adds the round's partials to its running total in segment order. With xb, the first row tile's
// workgroups also store the tokens' values as bf16.
constexpr int kRsWaves = 8;
constexpr int kRsDepth = 4;                // segments per wavefront held in registers
constexpr int kRsRow = 20;                 // floats per staged (j, token) row: 16 values + 4 of padding
constexpr int kRsTile = 4 * 16 * kRsRow;   // one staged operand

__global__ __launch_bounds__(64 * kRsWaves) void k_router_split(const float* __restrict__ x,
                                                                const float* __restrict__ w,
                                                                const float* __restrict__ bias,
                                                                const float* __restrict__ shared_gate, int T, int H,
                                                                int E, float* __restrict__ logits,
                                                                float* __restrict__ sg, uint16_t* __restrict__ xb) {
    __shared__ __attribute__((aligned(16))) float stage[kRsWaves][2][kRsTile];
    __shared__ float part[kRsDepth * kRsWaves][16][17];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int t0 = blockIdx.x * 16, r0 = blockIdx.y * 16;
    const int rows = E + (shared_gate ? 1 : 0);
    const int nseg = H / kRouterSeg;
    // staging: float4 f = lane + 64 i (i < 4) holds values 4 (f % 16) .. + 3 of token / row f / 16
    const float* xrow[4];
    const float* wrow[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int f = lane + 64 * i, rr = f >> 4, c4 = 4 * (f & 15);
        const int t = t0 + rr, r = r0 + rr;
        xrow[i] = x + static_cast<int64_t>(t < T ? t : T - 1) * H + c4;
        wrow[i] = r < rows ? (r < E ? w + static_cast<int64_t>(r) * H : shared_gate) + c4 : nullptr;
    }
    float* sa = stage[wv][0];
    float* sb = stage[wv][1];
    const int lt = lane & 15, lj = lane >> 4;
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
    const int st = tid >> 4, sr = tid & 15;  // summing thread (tid < 256): token st, row sr
    float total = 0.0f;
    for (int q0 = 0; q0 < nseg; q0 += kRsWaves * kRsDepth) {
        float4 xn[kRsDepth][4], wn[kRsDepth][4];
#pragma unroll
        for (int d = 0; d < kRsDepth; d++) {
            const int seg = q0 + kRsWaves * d + wv;
            if (seg < nseg) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    xn[d][i] = *reinterpret_cast<const float4*>(xrow[i] + seg * kRouterSeg);
                    wn[d][i] = wrow[i] ? *reinterpret_cast<const float4*>(wrow[i] + seg * kRouterSeg)
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
        }
#pragma unroll
        for (int d = 0; d < kRsDepth; d++) {
            const int seg = q0 + kRsWaves * d + wv;
            if (seg < nseg) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int f = lane + 64 * i, rr = f >> 4, s4 = f & 15;
                    const float4 xv = xn[d][i], wv4 = wn[d][i];
                    if (xb && blockIdx.y == 0 && t0 + rr < T)
                        *reinterpret_cast<uint2*>(xb + static_cast<int64_t>(t0 + rr) * H + seg * kRouterSeg +
                                                  4 * s4) = make_uint2(pack2(xv.x, xv.y), pack2(xv.z, xv.w));
                    sa[(0 * 16 + rr) * kRsRow + s4] = xv.x;
                    sa[(1 * 16 + rr) * kRsRow + s4] = xv.y;
                    sa[(2 * 16 + rr) * kRsRow + s4] = xv.z;
                    sa[(3 * 16 + rr) * kRsRow + s4] = xv.w;
                    sb[(0 * 16 + rr) * kRsRow + s4] = wv4.x;
                    sb[(1 * 16 + rr) * kRsRow + s4] = wv4.y;
                    sb[(2 * 16 + rr) * kRsRow + s4] = wv4.z;
                    sb[(3 * 16 + rr) * kRsRow + s4] = wv4.w;
                }
                lane_sync();
                floatx4 acc;
#pragma unroll
                for (int q = 0; q < 4; q++) {  // steps s = 4 q .. 4 q + 3
                    const float4 av = *reinterpret_cast<const float4*>(&sa[(lj * 16 + lt) * kRsRow + 4 * q]);
                    const float4 bv = *reinterpret_cast<const float4*>(&sb[(lj * 16 + lt) * kRsRow + 4 * q]);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, bv.x, q == 0 ? zero : acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, bv.y, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.z, bv.z, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.w, bv.w, acc, 0, 0, 0);
                }
                // lane holds D[4 lj + i][lt]: token 4 lj + i, row lt
#pragma unroll
                for (int i = 0; i < 4; i++) part[kRsWaves * d + wv][4 * lj + i][lt] = acc[i];
                lane_sync();  // the staging area is rewritten for the next d
            }
        }
        __syncthreads();
        if (tid < 256) {
            const int n = min(kRsWaves * kRsDepth, nseg - q0);
            for (int u = 0; u < n; u++) {
                const float v = part[u][st][sr];
                total = (q0 == 0 && u == 0) ? v : __fadd_rn(total, v);
            }
        }
        __syncthreads();
    }
    if (tid < 256) {
        const int t = t0 + st, r = r0 + sr;
        if (t < T && r < rows) {
            if (r < E)
                logits[static_cast<int64_t>(t) * E + r] = bias ? __fadd_rn(total, bias[r]) : total;
            else
                sg[t] = sigmoid(total);
        }
    }
}

// One token: the shared router_row (the fused decode kernel computes the same rows with it).
__global__ __launch_bounds__(64) void k_router1(const float* __restrict__ x, const float* __restrict__ w,
                                                const float* __restrict__ bias,
                                                const float* __restrict__ shared_gate, int H, int E,
                                                float* __restrict__ logits, float* __restrict__ sg) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 2 + (lane >> 5);
    const int rows_total = E + (shared_gate ? 1 : 0);
    const bool valid = row < rows_total;
    const float* wr = row < E ? w + static_cast<int64_t>(row) * H : shared_gate;
    const float total = router_row(x, wr, valid, H, lane);
    if ((lane & 31) == 0 && valid) {
        if (row < E)
            logits[row] = bias ? __fadd_rn(total, bias[row]) : total;
        else
            sg[0] = sigmoid(total);
    }
}

// ---------------------------------------------------------------------------------------------------------------
// The layer's input as RMSNorm of x (WL_MOE_PRE_NORM), one wavefront per token, in the fixed order the layer
// documents (the fused decode kernel applies the same NormX as it loads x): xn[t] = x[t] * inv * (1 + w).
__global__ __launch_bounds__(256) void k_rms_norm(const float* __restrict__ x, const float* __restrict__ w, float eps,
                                                 int T, int H, float* __restrict__ xn) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    const float* xt = x + static_cast<int64_t>(t) * H;
    const NormX nx{xt, w, norm_inv(router_row(xt, xt, true, H, lane), H, eps)};
    float4* out = reinterpret_cast<float4*>(xn + static_cast<int64_t>(t) * H);
    for (int i = lane; i < H / 4; i += 64) out[i] = nx(i);
}

// ---------------------------------------------------------------------------------------------------------------
// Top-k: one wavefront per token (wave_topk). crank[t, slot] = the rank of the slot's expert id among the token's
// k ids (ascending): the order the combine adds experts in, and the pick's entry in the grouping's table.
// min_w > 0: the layer's skip_small_experts (skip_small; dropped picks id -1).
template <int EJ>
__global__ __launch_bounds__(256) void k_topk(const float* __restrict__ logits, int T, int E, int k, int renorm,
                                              int32_t* __restrict__ ids, float* __restrict__ wts,
                                              int32_t* __restrict__ crank, float min_w) {
    __shared__ uint32_t scratch[4][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wv;
    if (t >= T) return;
    int id, id_rank;
    float w;
    wave_topk<EJ>(logits + static_cast<int64_t>(t) * E, E, k, renorm != 0, scratch[wv], lane, id, w, id_rank);
    if (min_w > 0.0f) skip_small(w, id, k, min_w, lane);
    if (lane < k) {
        ids[static_cast<int64_t>(t) * k + lane] = id;
        wts[static_cast<int64_t>(t) * k + lane] = w;
        if (crank) crank[static_cast<int64_t>(t) * k + lane] = id_rank;
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Router for a few tokens (2 .. kRouterPartsMaxT, inside wl_moe_layer), the K loop spread over 4x the workgroups of
// k_router_split: a workgroup takes 16 tokens x 16 rows and kRsWaves consecutive segments, its wavefront w the
// segment kRsWaves blockIdx.z + w, whose partial (the 64-value fused multiply-add chain from zero, on the fp32
// matrix core, staged as in k_router_split) it stores to parts[seg][t][r], rows r < E + (shared gate); no barrier
// and no partial sum inside the workgroup. k_topk_parts then adds each row's partials in segment order and the
// bias: the order of router_row, so the logits are the same bits. With xb, the first row tile's workgroups also
// store the tokens' values as bf16.
__global__ __launch_bounds__(64 * kRsWaves) void k_router_parts(const float* __restrict__ x,
                                                                const float* __restrict__ w,
                                                                const float* __restrict__ shared_gate, int T,
                                                                int H, int E, float* __restrict__ parts,
                                                                uint16_t* __restrict__ xb,
                                                                uint32_t* __restrict__ topk_done) {
    __shared__ __attribute__((aligned(16))) float stage[kRsWaves][2][kRsTile];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // the count k_topk_group (next on this stream) starts from: zeroed here by every call, so a workspace whose
    // words were never initialised still groups (its last-workgroup test only needs the count to start at 0)
    if (topk_done && tid == 0 && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0)
        __hip_atomic_store(topk_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int t0 = blockIdx.x * 16, r0 = blockIdx.y * 16;
    const int rows = E + (shared_gate ? 1 : 0);
    const int seg = static_cast<int>(blockIdx.z) * kRsWaves + wv;
    if (seg >= H / kRouterSeg) return;  // the wavefront alone: nothing below synchronizes the workgroup
    // float4 f = lane + 64 i (i < 4) holds values 4 (f % 16) .. + 3 of the segment for token / row f / 16
    float4 xn[4], wn[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int f = lane + 64 * i, rr = f >> 4, c4 = 4 * (f & 15);
        const int t = t0 + rr, r = r0 + rr;
        xn[i] = *reinterpret_cast<const float4*>(x + static_cast<int64_t>(t < T ? t : T - 1) * H + seg * kRouterSeg +
                                                 c4);
        const float* wr = r < rows ? (r < E ? w + static_cast<int64_t>(r) * H : shared_gate) : nullptr;
        wn[i] = wr ? *reinterpret_cast<const float4*>(wr + seg * kRouterSeg + c4) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float* sa = stage[wv][0];
    float* sb = stage[wv][1];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int f = lane + 64 * i, rr = f >> 4, s4 = f & 15;
        const float4 xv = xn[i], wv4 = wn[i];
        if (xb && blockIdx.y == 0 && t0 + rr < T)
            *reinterpret_cast<uint2*>(xb + static_cast<int64_t>(t0 + rr) * H + seg * kRouterSeg + 4 * s4) =
                make_uint2(pack2(xv.x, xv.y), pack2(xv.z, xv.w));
        sa[(0 * 16 + rr) * kRsRow + s4] = xv.x;
        sa[(1 * 16 + rr) * kRsRow + s4] = xv.y;
        sa[(2 * 16 + rr) * kRsRow + s4] = xv.z;
        sa[(3 * 16 + rr) * kRsRow + s4] = xv.w;
        sb[(0 * 16 + rr) * kRsRow + s4] = wv4.x;
        sb[(1 * 16 + rr) * kRsRow + s4] = wv4.y;
        sb[(2 * 16 + rr) * kRsRow + s4] = wv4.z;
        sb[(3 * 16 + rr) * kRsRow + s4] = wv4.w;
    }
    lane_sync();
    const int lt = lane & 15, lj = lane >> 4;
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
    floatx4 acc;
#pragma unroll
    for (int q = 0; q < 4; q++) {  // steps s = 4 q .. 4 q + 3
        const float4 av = *reinterpret_cast<const float4*>(&sa[(lj * 16 + lt) * kRsRow + 4 * q]);
        const float4 bv = *reinterpret_cast<const float4*>(&sb[(lj * 16 + lt) * kRsRow + 4 * q]);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, bv.x, q == 0 ? zero : acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, bv.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.z, bv.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.w, bv.w, acc, 0, 0, 0);
    }
    // lane holds D[4 lj + i][lt]: token t0 + 4 lj + i, row r0 + lt
    const int r = r0 + lt;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int t = t0 + 4 * lj + i;
        if (t < T && r < rows) parts[(static_cast<int64_t>(seg) * T + t) * rows + r] = acc[i];
    }
}

// Top-k over k_router_parts' partials: one workgroup per token. Thread r adds row r's nseg partials in segment
// order (then the bias; the shared gate's row E gives sg[t] = sigmoid of its sum) into LDS, with every load of the
// row issued before the adds when the segment count NSEG is a compile-time one; then wavefront 0 runs wave_topk as
// k_topk. blockDim.x: rows rounded up to a wavefront, at most 1024 (beyond, threads take several rows).
template <int EJ, int NSEG>
__device__ __forceinline__ void topk_parts(const float* __restrict__ parts, int nseg, const float* __restrict__ bias,
                                           int T, int E, int rows, int k, int renorm, int32_t* __restrict__ ids,
                                           float* __restrict__ wts, int32_t* __restrict__ crank,
                                           float* __restrict__ sg, float min_w) {
    __shared__ float lg[64 * EJ];
    __shared__ uint32_t scratch[64];
    const int t = blockIdx.x;
    const int64_t stride = static_cast<int64_t>(T) * rows;
    for (int r = threadIdx.x; r < rows; r += blockDim.x) {
        const float* p = parts + static_cast<int64_t>(t) * rows + r;
        float tot;
        if constexpr (NSEG > 0) {
            float v[NSEG];
#pragma unroll
            for (int i = 0; i < NSEG; i++) v[i] = p[i * stride];
            tot = v[0];
#pragma unroll
            for (int i = 1; i < NSEG; i++) tot = __fadd_rn(tot, v[i]);
        } else {
            tot = p[0];
            for (int i = 1; i < nseg; i++) tot = __fadd_rn(tot, p[i * stride]);
        }
        if (r < E)
            lg[r] = bias ? __fadd_rn(tot, bias[r]) : tot;
        else
            sg[t] = sigmoid(tot);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        int id, id_rank;
        float wsel;
        wave_topk<EJ>(lg, E, k, renorm != 0, scratch, lane, id, wsel, id_rank);
        if (min_w > 0.0f) skip_small(wsel, id, k, min_w, lane);
        if (lane < k) {
            ids[static_cast<int64_t>(t) * k + lane] = id;
            wts[static_cast<int64_t>(t) * k + lane] = wsel;
            if (crank) crank[static_cast<int64_t>(t) * k + lane] = id_rank;
        }
    }
}

template <int EJ, int NSEG>
__global__ __launch_bounds__(1024) void k_topk_parts(const float* __restrict__ parts, int nseg,
                                                     const float* __restrict__ bias, int T, int E, int rows, int k,
                                                     int renorm, int32_t* __restrict__ ids, float* __restrict__ wts,
                                                     int32_t* __restrict__ crank, float* __restrict__ sg,
                                                     float min_w) {
    topk_parts<EJ, NSEG>(parts, nseg, bias, T, E, rows, k, renorm, ids, wts, crank, sg, min_w);
}

// ---------------------------------------------------------------------------------------------------------------
// Token->expert grouping (a stable counting sort of the T*k (token, slot) pairs by expert id).
// Within a chunk of kSortChunk tokens, bit t of row e of an LDS bitmap says token t picked expert e; a pair's rank
// among its expert's pairs is the popcount of the bits before it, so the result is deterministic and stable
// (pairs of one expert stay in token order). Outputs:
//   offsets[E+1]    first sorted position of each expert's pairs; offsets[E] = the pairs grouped (T*k less
//                   the picks skip_small dropped, which have no position)
//   active[0]       number of experts with at least one pair; active[1..] those experts, ascending
//   sorted[P]       pair id (t*k + slot) at each sorted position
//   picks[P]        the combine's table: entry t*k + crank[q] of pair q = (its position | kPosBf16 for an MFMA
//                   expert, or 0xFFFFFFFF for a dropped pick; the bits of its weight wts[q])
// One chunk: k_sort_small. Many chunks: k_sort_hist (per-chunk bitmaps, counts and ranks) -> k_sort_scan (chunk
// bases, offsets, active experts, tile lists) -> k_sort_scatter.

// Bitmaps of one chunk; returns with counts[e] filled (LDS) and `bits` holding the chunk's bitmap.
__device__ void chunk_bitmap(const int32_t* __restrict__ ids, int t_begin, int t_end, int k, int E, uint32_t* bits,
                             int32_t* counts) {
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int i = tid; i < E * kSortWords; i += nt) bits[i] = 0;
    __syncthreads();
    const int pairs = (t_end - t_begin) * k;
    for (int q = tid; q < pairs; q += nt) {
        const int t = q / k;
        const int e = ids[static_cast<int64_t>(t_begin) * k + q];
        if (e >= 0 && e < E) atomicOr(&bits[e * kSortWords + (t >> 5)], 1u << (t & 31));
    }
    __syncthreads();
    for (int e = tid; e < E; e += nt) {
        int c = 0;
#pragma unroll
        for (int wd = 0; wd < kSortWords; wd++) c += __popc(bits[e * kSortWords + wd]);
        counts[e] = c;
    }
    __syncthreads();
}

__device__ __forceinline__ int chunk_rank(const uint32_t* bits, int e, int t) {
    int r = 0;
    const int wd = t >> 5;
    for (int i = 0; i < wd; i++) r += __popc(bits[e * kSortWords + i]);
    r += __popc(bits[e * kSortWords + wd] & ((1u << (t & 31)) - 1u));
    return r;
}

// With tiles non-null (an MFMA plan), the sort's single-workgroup stage also writes the GEMMs' tile lists, for the
// experts with more than gemv_max pairs (and the shared expert); `active` then lists only the others (the GEMV
// experts), and the table entries of MFMA experts' pairs carry kPosBf16.
struct TileOut {
    int4* tiles;
    int4* tiles_down;
    int32_t* n_tiles;
    int with_shared;
    int gemv_max;
};

__global__ __launch_bounds__(1024) void k_sort_hist(const int32_t* __restrict__ ids, int T, int k, int E,
                                                   int32_t* __restrict__ rank, int32_t* __restrict__ hist) {
    extern __shared__ uint32_t smem[];
    uint32_t* bits = smem;
    int32_t* counts = reinterpret_cast<int32_t*>(bits + E * kSortWords);
    const int c = blockIdx.x;
    const int t_begin = c * kSortChunk;
    const int t_end = min(T, t_begin + kSortChunk);
    chunk_bitmap(ids, t_begin, t_end, k, E, bits, counts);
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int e = tid; e < E; e += nt) hist[static_cast<int64_t>(c) * E + e] = counts[e];
    const int pairs = (t_end - t_begin) * k;
    for (int q = tid; q < pairs; q += nt) {
        const int64_t p = static_cast<int64_t>(t_begin) * k + q;
        const int e = ids[p];
        rank[p] = (e >= 0 && e < E) ? chunk_rank(bits, e, q / k) : 0;
    }
}

// The combine's table (picks): each token's entries in ascending expert id, so k_combine reads them in one pass
// with no dependent load (the pair's position and weight come together).
struct PickOut {
    const int32_t* crank;  // [T, k] from the top-k
    const float* wts;      // [T, k]
    uint2* picks;          // [T, k]
    __device__ __forceinline__ void put(int64_t q, int k, uint32_t entry, int rank, float w) const {
        picks[q - q % k + rank] = make_uint2(entry, __builtin_bit_cast(uint32_t, w));
    }
};

// flag_above: pairs of experts with more than this many pairs get kPosBf16 in their table entries (MFMA experts)
__global__ __launch_bounds__(256) void k_sort_scatter(const int32_t* __restrict__ ids, int T, int k, int E,
                                                      const int32_t* __restrict__ rank,
                                                      const int32_t* __restrict__ hist,
                                                      const int32_t* __restrict__ offsets, int flag_above,
                                                      int32_t* __restrict__ sorted, PickOut po) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= static_cast<int64_t>(T) * k) return;
    const int e = ids[p];
    uint32_t entry = 0xFFFFFFFFu;  // a pick skip_small dropped (id -1): no position, the combine leaves it out
    if (e >= 0 && e < E) {
        const int c = static_cast<int>(p / k) / kSortChunk;
        const int pos = hist[static_cast<int64_t>(c) * E + e] + rank[p];
        const bool bf16 = offsets[e + 1] - offsets[e] > flag_above;
        sorted[pos] = static_cast<int32_t>(p);
        entry = static_cast<uint32_t>(pos) | (bf16 ? kPosBf16 : 0u);
    }
    po.put(p, k, entry, po.crank[p], po.wts[p]);
}

// One chunk (T <= kSortChunk), a workgroup of 1024 threads: one thread per expert builds the stable counting sort
// (the same outputs as the multi-chunk path) and the GEMM tile lists from the LDS bitmaps, with workgroup scans
// made of wavefront scans (three barriers each).
constexpr int kSortSmallThreads = 1024;

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(v, o);
        if (lane >= o) v += u;
    }
    return v;
}

// Exclusive prefix sum of one value per thread over the workgroup (thread order); *total = the sum. wsum holds one
// int per wavefront. Ends with a barrier, so wsum can be used again at once.
__device__ int block_scan_excl(int v, int* wsum, int* total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int inc = wave_incl_scan(v, lane);
    if (lane == 63) wsum[wv] = inc;
    __syncthreads();
    if (wv == 0) {
        int w = lane < nw ? wsum[lane] : 0;
        w = wave_incl_scan(w, lane);
        if (lane < nw) wsum[lane] = w;
    }
    __syncthreads();
    const int r = (wv > 0 ? wsum[wv - 1] : 0) + inc - v;
    *total = wsum[nw - 1];
    __syncthreads();
    return r;
}

// GEMM tiles: each MFMA expert's sorted positions, then the shared expert's tokens (expert id E), cut into tiles
// of at most `cap` tokens; tiles[i] = (expert, first position or token, count, 0), n_tiles[0] = how many. Thread e
// holds expert e's count c (0 for an expert left to the GEMV kernels) and first position off; every thread of the
// workgroup takes part (E <= blockDim.x).
__device__ void tile_list(int4* __restrict__ tiles, int32_t* __restrict__ n_tiles, int cap, int e, int E,
                                int c, int off, int T, int with_shared, int* wsum) {
    int total;
    int n = block_scan_excl(e < E ? (c + cap - 1) / cap : 0, wsum, &total);
    if (e < E)
        for (int p = 0; p < c; p += cap) tiles[n++] = make_int4(e, off + p, min(cap, c - p), 0);
    if (with_shared)
        for (int p = static_cast<int>(threadIdx.x) * cap; p < T; p += static_cast<int>(blockDim.x) * cap)
            tiles[total + p / cap] = make_int4(E, p, min(cap, T - p), 0);
    if (threadIdx.x == 0) n_tiles[0] = total + (with_shared ? (T + cap - 1) / cap : 0);
}

// Fork scope (wl_moe_fork_begin): the split plan's MFMA experts run on the device's second stream and meet the
// caller's stream through words of the call's workspace instead of a fork and a join event per call. The grouping
// publishes its results (kForkSorted = 1, after clearing kForkDone); the second stream's k_fork_wait waits for that
// and clears it, then the MFMA kernels run and k_fork_store sets kForkDone = 1; the combine waits for kForkDone.
// A word is only set after the one that clears it has been waited for, so the words need no epochs: the grouping's
// clearing of kForkDone comes after the previous call's combine (the caller's stream), and the next kForkSorted
// after the previous call's k_fork_wait cleared it (which the previous kForkDone, and so this grouping, waited
// for). Every wait is bounded; one that gives up sets kStatusFork in the status word, after which every k_fork_wait
// sets the skip word, so the MFMA kernels never read a grouping that is not there (wl_moe_workspace_status reports
// WL_ESYNC and clears the words).

// The grouping's results in memory for every agent, then the flags: every wavefront waits for its own stores to
// land in the L2, and one thread's release store writes the L2 back once.
__device__ __forceinline__ void publish_grouping(uint32_t* sync, int withhold) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_store(sync + kForkDone, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (!withhold) __hip_atomic_store(sync + kForkSorted, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// *a = va (when a), then *b = vb with release (when b); one thread, after the kernels before it on the stream.
__global__ __launch_bounds__(64) void k_fork_store(uint32_t* a, uint32_t va, uint32_t* b, uint32_t vb) {
    if (threadIdx.x != 0) return;
    if (a) __hip_atomic_store(a, va, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (b) __hip_atomic_store(b, vb, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// The second stream's wait for the grouping (one thread; at most spin_limit polls). Relaxed polls: an acquire
// would invalidate this XCD's L2 on every poll under the kernels of the caller's stream; the MFMA kernels that
// read the grouping are dispatched after this kernel ends and acquire at their start.
__global__ __launch_bounds__(64) void k_fork_wait(uint32_t* sync, uint32_t spin_limit) {
    if (threadIdx.x != 0) return;
    uint32_t* sorted = sync + kForkSorted;
    bool ok = (__hip_atomic_load(sync + kStatusWord, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kStatusFork) == 0;
    for (uint32_t spins = 0; ok && __hip_atomic_load(sorted, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 1u;
         spins++) {
        if (spins >= spin_limit)
            ok = false;
        else
            __builtin_amdgcn_s_sleep(1);
    }
    if (ok)
        __hip_atomic_store(sorted, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        __hip_atomic_fetch_or(sync + kStatusWord, kStatusFork, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(sync + kForkSkip, ok ? 0u : 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The caller's stream's wait for the second stream's MFMA experts (one thread; at most spin_limit polls): the
// combine is launched after this kernel, so no workgroup of a wide grid holds a CU while the MFMA kernels may still
// need it. Relaxed polls; the combine acquires at its start. A wait that gives up sets kStatusFork.
__global__ __launch_bounds__(64) void k_fork_gate(uint32_t* sync, uint32_t spin_limit) {
    if (threadIdx.x != 0) return;
    bool ok = false;
    for (uint32_t spins = 0; spins < spin_limit && !ok; spins++) {
        ok = __hip_atomic_load(sync + kForkDone, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1u;
        if (!ok) __builtin_amdgcn_s_sleep(1);
    }
    if (!ok) __hip_atomic_fetch_or(sync + kStatusWord, kStatusFork, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ void sort_small(const int32_t* __restrict__ ids, int T, int k, int E,
                                           int32_t* __restrict__ offsets, int32_t* __restrict__ active,
                                           int32_t* __restrict__ sorted, PickOut po, TileOut to,
                                           uint32_t* fork_sync, int withhold) {
    __shared__ int32_t lds_ids[kSortChunk * WL_MAX_TOPK];
    __shared__ uint32_t bits[kSortWords * 64 * kMaxEJ];  // expert e: words kSortWords e .. + kSortWords - 1
    __shared__ uint32_t lds_off[64 * kMaxEJ];  // first sorted position | kPosBf16 for an MFMA expert
    __shared__ int wsum[kSortSmallThreads / 64];
    const int tid = threadIdx.x;
    const int P = T * k;
    // the table's inputs for pair q = tid, loaded with the ids (the only pair of a thread when P <= blockDim.x)
    const int my_rank = tid < P ? po.crank[tid] : 0;
    const float my_w = tid < P ? po.wts[tid] : 0.0f;
    for (int q = tid; q < P; q += blockDim.x) lds_ids[q] = ids[q];
    for (int i = tid; i < kSortWords * E; i += blockDim.x) bits[i] = 0u;
    __syncthreads();
    for (int q = tid; q < P; q += blockDim.x) {
        const int e = lds_ids[q], t = q / k;
        if (e >= 0 && e < E) atomicOr(&bits[kSortWords * e + (t >> 5)], 1u << (t & 31));
    }
    __syncthreads();
    const int e = tid;
    int c = 0;
    if (e < E)
#pragma unroll
        for (int wd = 0; wd < kSortWords; wd++) c += __popc(bits[kSortWords * e + wd]);
    if (P <= 1024 && E <= 256 && T <= kDownTileTokens) {
        // Few pairs (batched decode): every MFMA expert and the shared expert fit one tile of either list, so
        // the four scans below (positions, GEMV experts, the two tile lists) are one scan of three packed counts:
        // pairs in bits 0..10 (<= 1024), GEMV experts in 11..19 and MFMA experts in 20..28 (<= 256 each), whose
        // prefix sums stay inside their fields. The same outputs, with 4 barriers instead of 13.
        const bool big = to.tiles && c > to.gemv_max;  // an MFMA expert
        const bool act = c > 0 && !big;                 // a GEMV expert
        int total;
        const int pre = block_scan_excl(c | (act ? 1 << 11 : 0) | (big ? 1 << 20 : 0), wsum, &total);
        const int off = pre & 0x7FF, apos = (pre >> 11) & 0x1FF, tpos = pre >> 20;
        const int n_big = total >> 20;
        if (e < E) {
            offsets[e] = off;
            lds_off[e] = static_cast<uint32_t>(off) | (big ? kPosBf16 : 0u);
            if (act) active[1 + apos] = e;
            if (big) {
                to.tiles[tpos] = make_int4(e, off, c, 0);
                to.tiles_down[tpos] = make_int4(e, off, c, 0);
            }
        }
        if (tid == 0) {
            offsets[E] = total & 0x7FF;  // the pairs grouped: T k less any skip_small dropped
            active[0] = (total >> 11) & 0x1FF;
            if (to.tiles) {
                if (to.with_shared) {
                    to.tiles[n_big] = make_int4(E, 0, T, 0);
                    to.tiles_down[n_big] = make_int4(E, 0, T, 0);
                }
                to.n_tiles[0] = to.n_tiles[1] = n_big + (to.with_shared ? 1 : 0);
            }
        }
        __syncthreads();  // lds_off for every thread
        for (int q = tid; q < P; q += blockDim.x) {
            const int ex = lds_ids[q];
            uint32_t entry = 0xFFFFFFFFu;  // a pick skip_small dropped (id -1): the combine leaves it out
            if (ex >= 0 && ex < E) {
                const uint32_t o = lds_off[ex];
                const int pos = static_cast<int>(o & ~kPosBf16) + chunk_rank(bits, ex, q / k);
                sorted[pos] = q;
                entry = static_cast<uint32_t>(pos) | (o & kPosBf16);
            }
            if (q == tid)
                po.put(q, k, entry, my_rank, my_w);
            else
                po.put(q, k, entry, po.crank[q], po.wts[q]);
        }
        if (fork_sync) publish_grouping(fork_sync, withhold);
        return;
    }
    int total;
    const int off = block_scan_excl(c, wsum, &total);
    const bool big = to.tiles && c > to.gemv_max;  // an MFMA expert
    if (e < E) {
        offsets[e] = off;
        lds_off[e] = static_cast<uint32_t>(off) | (big ? kPosBf16 : 0u);
    }
    if (tid == 0) offsets[E] = total;  // the pairs grouped: T k less any skip_small dropped
    const int apos = block_scan_excl((c > 0 && !big) ? 1 : 0, wsum, &total);  // its barriers also publish lds_off
    if (e < E && c > 0 && !big) active[1 + apos] = e;
    if (tid == 0) active[0] = total;
    for (int q = tid; q < P; q += blockDim.x) {
        const int ex = lds_ids[q];
        uint32_t entry = 0xFFFFFFFFu;  // a pick skip_small dropped (id -1): the combine leaves it out
        if (ex >= 0 && ex < E) {
            const uint32_t o = lds_off[ex];
            const int pos = static_cast<int>(o & ~kPosBf16) + chunk_rank(bits, ex, q / k);
            sorted[pos] = q;
            entry = static_cast<uint32_t>(pos) | (o & kPosBf16);
        }
        if (q == tid)
            po.put(q, k, entry, my_rank, my_w);
        else
            po.put(q, k, entry, po.crank[q], po.wts[q]);
    }
    if (to.tiles) {
        tile_list(to.tiles, to.n_tiles, kTileTokens, e, E, big ? c : 0, off, T, to.with_shared, wsum);
        tile_list(to.tiles_down, to.n_tiles + 1, kDownTileTokens, e, E, big ? c : 0, off, T, to.with_shared, wsum);
    }
    if (fork_sync) publish_grouping(fork_sync, withhold);
}

__global__ __launch_bounds__(kSortSmallThreads) void k_sort_small(const int32_t* __restrict__ ids, int T, int k,
                                                                  int E, int32_t* __restrict__ offsets,
                                                                  int32_t* __restrict__ active,
                                                                  int32_t* __restrict__ sorted, PickOut po,
                                                                  TileOut to, uint32_t* fork_sync, int withhold) {
    sort_small(ids, T, k, E, offsets, active, sorted, po, to, fork_sync, withhold);
}

static_assert(kRouterPartsMaxT <= kSortChunk, "k_topk_group groups its tokens as one chunk");

// The grouping's outputs for k_topk_group (as k_sort_small's arguments) and the workspace's sync words.
struct GroupOut {
    int32_t* offsets;
    int32_t* active;
    int32_t* sorted;
    PickOut po;
    TileOut to;
    uint32_t* sync;  // kTopkDone; the fork-scope words when fork
    int fork;
    int withhold;
};

// Top-k over the router's partials (k_topk_parts, one workgroup per token) followed by the grouping (k_sort_small)
// in the same launch, for calls of at most kSortChunk tokens: each workgroup, once its token's picks are stored,
// counts itself done in kTopkDone (a release at agent scope first); the last of the T then acquires and groups all
// tokens' picks, and resets the count. One launch boundary fewer on the path before any expert work starts.
template <int EJ, int NSEG>
__global__ __launch_bounds__(1024) void k_topk_group(const float* __restrict__ parts, int nseg,
                                                     const float* __restrict__ bias, int T, int E, int rows, int k,
                                                     int renorm, int32_t* __restrict__ ids, float* __restrict__ wts,
                                                     int32_t* __restrict__ crank, float* __restrict__ sg,
                                                     GroupOut g, float min_w) {
    __shared__ int last;
    topk_parts<EJ, NSEG>(parts, nseg, bias, T, E, rows, k, renorm, ids, wts, crank, sg, min_w);
    __syncthreads();  // the picks are stored by wavefront 0, whose thread 0 counts the workgroup done
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const uint32_t prev = __hip_atomic_fetch_add(g.sync + kTopkDone, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        last = prev == static_cast<uint32_t>(T - 1) ? 1 : 0;
        if (last) {
            __hip_atomic_store(g.sync + kTopkDone, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
    }
    __syncthreads();
    if (last)
        sort_small(ids, T, k, E, g.offsets, g.active, g.sorted, g.po, g.to, g.fork ? g.sync : nullptr, g.withhold);
}

// Many chunks: one thread per expert turns its per-chunk counts (hist[c][e]) into the chunk's first sorted
// position, chunks read kScanBatch at a time with their loads issued together; offsets, active experts and tile
// lists as in k_sort_small.
constexpr int kScanBatch = 16;
__global__ __launch_bounds__(kSortSmallThreads) void k_sort_scan(int T, int k, int E, int nchunks,
                                                                 int32_t* __restrict__ hist,
                                                                 int32_t* __restrict__ offsets,
                                                                 int32_t* __restrict__ active, TileOut to) {
    __shared__ int wsum[kSortSmallThreads / 64];
    const int e = threadIdx.x;
    const bool mine = e < E;
    int pre[kScanBatch];  // with nchunks <= kScanBatch: the expert's per-chunk prefixes, kept for the second pass
    int run = 0;
    for (int c0 = 0; c0 < nchunks; c0 += kScanBatch) {
        int v[kScanBatch];
#pragma unroll
        for (int u = 0; u < kScanBatch; u++)
            v[u] = (mine && c0 + u < nchunks) ? hist[static_cast<int64_t>(c0 + u) * E + e] : 0;
#pragma unroll
        for (int u = 0; u < kScanBatch; u++) {
            pre[u] = run;
            if (mine && c0 + u < nchunks && nchunks > kScanBatch) hist[static_cast<int64_t>(c0 + u) * E + e] = run;
            run += v[u];
        }
    }
    const int c = mine ? run : 0;
    int total;
    const int off = block_scan_excl(c, wsum, &total);
    if (mine) offsets[e] = off;
    if (threadIdx.x == 0) offsets[E] = total;  // the pairs grouped: T k less any skip_small dropped
    if (mine) {
        if (nchunks <= kScanBatch) {
#pragma unroll
            for (int u = 0; u < kScanBatch; u++)
                if (u < nchunks) hist[static_cast<int64_t>(u) * E + e] = pre[u] + off;
        } else {
            for (int c0 = 0; c0 < nchunks; c0 += kScanBatch) {
                int v[kScanBatch];
#pragma unroll
                for (int u = 0; u < kScanBatch; u++)
                    v[u] = c0 + u < nchunks ? hist[static_cast<int64_t>(c0 + u) * E + e] : 0;
#pragma unroll
                for (int u = 0; u < kScanBatch; u++)
                    if (c0 + u < nchunks) hist[static_cast<int64_t>(c0 + u) * E + e] = v[u] + off;
            }
        }
    }
    const bool big = to.tiles && c > to.gemv_max;  // an MFMA expert
    const int apos = block_scan_excl((c > 0 && !big) ? 1 : 0, wsum, &total);
    if (mine && c > 0 && !big) active[1 + apos] = e;
    if (threadIdx.x == 0) active[0] = total;
    if (to.tiles) {
        tile_list(to.tiles, to.n_tiles, kTileTokens, e, E, big ? c : 0, off, T, to.with_shared, wsum);
        tile_list(to.tiles_down, to.n_tiles + 1, kDownTileTokens, e, E, big ? c : 0, off, T, to.with_shared, wsum);
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Experts on the fp32 GEMV kernels. A launch's work slots are the routed experts listed in active[1 ..
// active[0]] (when a.routed) and then the shared expert over all T tokens (when a.shared_slot); each slot's rows
// are cut into row groups of one workgroup each, and the workgroups loop over the (slot, row group) items, so the
// grid can be sized for the most experts a call may have while only the listed ones cost anything. Outputs are
// indexed by sorted position (routed) or token (shared).
struct ExpertView {
    const uint8_t* w;
    int64_t stride_rows;  // offset of the up half (gate_up) in rows
    int begin, end;       // token positions
    bool routed;
};

__device__ __forceinline__ int expert_slots(const ExpertArgs& a) {
    return (a.routed ? a.active[0] : 0) + a.shared_slot;
}

__device__ __forceinline__ ExpertView expert_view(const ExpertArgs& a, int slot, bool up_proj) {
    ExpertView v;
    const int n_routed = a.routed ? a.active[0] : 0;
    if (slot < n_routed) {
        const int e = a.active[1 + slot];
        v.w = (up_proj ? a.gate_up : a.down) + static_cast<int64_t>(e) * (up_proj ? a.gate_up_stride : a.down_stride);
        v.stride_rows = a.inter;
        v.begin = a.offsets[e];
        v.end = a.offsets[e + 1];
        v.routed = true;
    } else {
        v.w = up_proj ? a.sh_gate_up : a.sh_down;
        v.stride_rows = a.sh_inter;
        v.begin = 0;
        v.end = a.T;
        v.routed = false;
    }
    return v;
}

// The GEMV expert kernels run the few tokens of an expert (at most 8 when it shares a call with MFMA experts)
// against exact fp32 weights. Layout: each 256-value block of a weight row belongs to one lane, and a row to L
// consecutive lanes (L = the power of two <= min(blocks per row, 8); lane c takes blocks c, c + L, ...). A lane
// loads its whole block at once, converts each of its values to fp32 once, and runs every token of the current
// chunk through it: value = a q + b per sub-block (Q4_K: 32 values; Q6_K: 16), so a token adds
// a * sum(q x) + b * sum(x) per sub-block, with sum(x) read from LDS. The chunk's activation rows (x for gate_up,
// h for down) sit in LDS, staged once per chunk by the whole workgroup with all loads in flight at once: block kb of
// a row starts at float 260 kb (4 floats of skew, so the 8 lanes reading 8 different blocks hit different banks;
// the rows' other lanes read the same addresses, a broadcast), and the sums of every 16 values follow the rows.
constexpr int kGemvTok = 8;         // most tokens per LDS chunk
constexpr int kBlkFloats = 260;     // LDS floats per 256-value block of an activation row
constexpr int kGemvLdsMax = 40 << 10;

__host__ __device__ inline int lds_row_floats(int width) { return width / 256 * kBlkFloats; }
__host__ __device__ inline int lds_chunk_floats(int width) { return lds_row_floats(width) + width / 16; }

// Tokens per chunk for activation rows of `width` values: at most kGemvTok, within kGemvLdsMax of LDS.
__host__ inline int gemv_chunk(int width) {
    const int per = kGemvLdsMax / (4 * lds_chunk_floats(width));
    return per < 1 ? 1 : (per < kGemvTok ? per : kGemvTok);
}

// Lanes per row: the largest power of two <= min(blocks per row, 8).
__host__ inline int gemv_lanes(int nb) { return nb >= 8 ? 8 : nb >= 4 ? 4 : nb >= 2 ? 2 : 1; }

// rows u < n of the chunk: src_row(u)[0, width) -> LDS (rows of lds_row_floats(width), then the n rows' 16-value
// sums, width / 16 each). Ends with a barrier.
template <typename SrcRow>
__device__ __forceinline__ void stage_chunk(float* lds, int n, int width, SrcRow src_row) {
    const int per_row = width / 4, ld = lds_row_floats(width), ng = width / 16;
    for (int f = threadIdx.x; f < n * per_row; f += blockDim.x) {
        const int u = f / per_row, i = 4 * (f - u * per_row);
        *reinterpret_cast<float4*>(lds + u * ld + (i >> 8) * kBlkFloats + (i & 255)) =
            *reinterpret_cast<const float4*>(src_row(u) + i);
    }
    __syncthreads();
    float* sums = lds + n * ld;
    for (int f = threadIdx.x; f < n * ng; f += blockDim.x) {
        const int u = f / ng, gg = f - u * ng;
        float4 x[4];
        const float4* q = reinterpret_cast<const float4*>(lds + u * ld + (gg >> 4) * kBlkFloats + 16 * (gg & 15));
#pragma unroll
        for (int j = 0; j < 4; j++) x[j] = q[j];
        sums[f] = sum16(x);
    }
    __syncthreads();
}

// sum of f[i] * x[i] for 16 values, x 16-byte aligned in LDS
__device__ __forceinline__ float dot16_lds(const float* f, const float* x) {
    const float4* q = reinterpret_cast<const float4*>(x);
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 v = q[i];
        s0 = __builtin_fmaf(f[4 * i], v.x, s0);
        s1 = __builtin_fmaf(f[4 * i + 1], v.y, s1);
        s0 = __builtin_fmaf(f[4 * i + 2], v.z, s0);
        s1 = __builtin_fmaf(f[4 * i + 3], v.w, s1);
    }
    return s0 + s1;
}

// the four bytes of w (fields of at most 8 bits) as floats into f[0..3]
__device__ __forceinline__ void bytes_to_f32(uint32_t w, float* f) {
    f[0] = ubyte(w, 0);
    f[1] = ubyte(w, 1);
    f[2] = ubyte(w, 2);
    f[3] = ubyte(w, 3);
}

// acc[u] += (block . x_u) for the chunk's tokens u < n: xs = the block's 256 values of token 0 in LDS (token u at
// xs + u ldx), ss = its 16 sums of token 0 (token u at ss + u lds_).
template <int TYPE>
struct BlockDot;

template <>
struct BlockDot<WL_TYPE_Q4_K> {
    // blk: 16-byte aligned. Sub-block j = 2 q + e: values 64 q + 32 e + i are the low (e = 0) or high (e = 1)
    // nibbles of qs bytes 32 q + i; value = (d sc_j) q - dmin m_j. fetch() issues the block's loads; run() uses
    // them, so whatever runs in between (the activation staging) overlaps the loads.
    uint4 hd, qv[8];
    __device__ void fetch(const uint8_t* __restrict__ blk) {
        const uint4* p = reinterpret_cast<const uint4*>(blk);
        hd = p[0];
#pragma unroll
        for (int i = 0; i < 8; i++) qv[i] = p[1 + i];
    }
    __device__ void run(const float* xs, int ldx, const float* ss, int lds_, int n, float (&acc)[kGemvTok]) const {
        const float d = half_to_float(hd.x), dmin = half_to_float(hd.x >> 16);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t w[8] = {qv[2 * q].x, qv[2 * q].y, qv[2 * q].z, qv[2 * q].w,
                                   qv[2 * q + 1].x, qv[2 * q + 1].y, qv[2 * q + 1].z, qv[2 * q + 1].w};
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int j = 2 * q + e;
                uint32_t sc, m;
                q4k_scale_min(j, hd.y, hd.z, hd.w, sc, m);
                const float a = (d * (e ? 1048576.0f : 16777216.0f)) * static_cast<float>(sc),
                            b = -(dmin * static_cast<float>(m));
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    // the nibbles in place as f16 subnormals (q 2^-24 low, q 2^-20 high), a scaled to match: the
                    // products and every rounding after them are the same as with the nibbles converted to floats
                    const uint32_t msk = e ? 0x00F000F0u : 0x000F000Fu;
                    uint32_t ev[4], od[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        ev[i] = opaque(w[4 * hh + i] & msk);
                        od[i] = opaque((w[4 * hh + i] >> 8) & msk);
                    }
#pragma unroll
                    for (int u = 0; u < kGemvTok; u++) {
                        if (u < n) {
                            const float4* x4 = reinterpret_cast<const float4*>(xs + u * ldx + 32 * j + 16 * hh);
                            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                            for (int i = 0; i < 4; i++) {
                                const float4 v = x4[i];
                                const wl_f16x2 he = __builtin_bit_cast(wl_f16x2, ev[i]);
                                const wl_f16x2 ho = __builtin_bit_cast(wl_f16x2, od[i]);
                                s0 = __builtin_fmaf(static_cast<float>(he.x), v.x, s0);
                                s1 = __builtin_fmaf(static_cast<float>(ho.x), v.y, s1);
                                s0 = __builtin_fmaf(static_cast<float>(he.y), v.z, s0);
                                s1 = __builtin_fmaf(static_cast<float>(ho.y), v.w, s1);
                            }
                            acc[u] += a * (s0 + s1) + b * ss[u * lds_ + 2 * j + hh];
                        }
                    }
                }
            }
        }
    }
};

// n consecutive bytes' dwords from a 2-byte-aligned address, realigned: reads the n + 1 aligned dwords around them
// (from at most 2 bytes before p to at most 4 after p + 4 n).
template <int N>
__device__ __forceinline__ void load_words_a2(const uint8_t* p, uint32_t (&out)[N]) {
    uint32_t sh;
    const uint32_t* q = align_down4(p, sh);
    uint32_t w[N + 1];
#pragma unroll
    for (int i = 0; i <= N; i++) w[i] = q[i];
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
}

template <>
struct BlockDot<WL_TYPE_Q6_K> {
    // blk: 2-byte aligned. Value 128 h + 32 t + c: low 4 bits in ql[64 h + 32 (t & 1) + c] (high nibble for t >= 2),
    // high 2 bits at bit 2 t of qh[32 h + c]; value = (d sc_g) (q6 - 32), g = its 16-value group.
    // Every read stays within [blk - 2, blk + 210): ql up to byte 132, qh up to 196, scales as 4 dwords from
    // byte 192 - (blk & 3) and a 16-bit load of bytes 206..207. fetch() issues the loads, run() uses them.
    uint32_t ql[2][16], qh[2][8], sw[4], d16;
    __device__ void fetch(const uint8_t* __restrict__ blk) {
        load_words_a2<16>(blk, ql[0]);
        load_words_a2<16>(blk + 64, ql[1]);
        load_words_a2<8>(blk + 128, qh[0]);
        load_words_a2<8>(blk + 160, qh[1]);
        uint32_t sh;
        const uint32_t* q = align_down4(blk + 192, sh);
        const uint32_t w0 = q[0], w1 = q[1], w2 = q[2], w3 = q[3];
        const uint32_t tail = *reinterpret_cast<const uint16_t*>(blk + 206);
        sw[0] = __builtin_amdgcn_alignbyte(w1, w0, sh);
        sw[1] = __builtin_amdgcn_alignbyte(w2, w1, sh);
        sw[2] = __builtin_amdgcn_alignbyte(w3, w2, sh);
        sw[3] = __builtin_amdgcn_alignbyte(tail, w3, sh);
        d16 = *reinterpret_cast<const uint16_t*>(blk + 208);
    }
    __device__ void run(const float* xs, int ldx, const float* ss, int lds_, int n, float (&acc)[kGemvTok]) const {
        const float d = half_to_float(d16);
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int g = 8 * h + 2 * t;  // the two 16-value groups of these 32 values
                const float a0 = d * static_cast<float>(static_cast<int8_t>((sw[g >> 2] >> (8 * (g & 3))) & 0xFFu));
                const float a1 =
                    d * static_cast<float>(static_cast<int8_t>((sw[(g + 1) >> 2] >> (8 * ((g + 1) & 3))) & 0xFFu));
                const float b0 = -32.0f * a0, b1 = -32.0f * a1;
                float f[32];
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const uint32_t lo = (ql[h][8 * (t & 1) + i] >> (4 * (t >> 1))) & 0x0F0F0F0Fu;
                    const uint32_t hi = ((qh[h][i] >> (2 * t)) & 0x03030303u) << 4;
                    bytes_to_f32(opaque(lo | hi), f + 4 * i);
                }
#pragma unroll
                for (int u = 0; u < kGemvTok; u++) {
                    if (u < n) {
                        const float* x = xs + u * ldx + 128 * h + 32 * t;
                        const float s0 = dot16_lds(f, x), s1 = dot16_lds(f + 16, x + 16);
                        acc[u] += a0 * s0 + b0 * ss[u * lds_ + g] + a1 * s1 + b1 * ss[u * lds_ + g + 1];
                    }
                }
            }
        }
    }
};

// sum over the L lanes of a row (L a power of two, 1..8)
template <int L>
__device__ __forceinline__ float row_sum(float v) {
    if constexpr (L == 1)
        return v;
    else
        return group_sum<L>(v);
}

// gate_up + SwiGLU. A wavefront takes JW = 32 / L intermediate rows j: lanes [0, 32) the gate rows j, lanes
// [32, 64) the up rows inter + j (L lanes per row); a workgroup 4 JW rows. h[pos, j] = silu(gate . x_t) *
// (up . x_t) for each of the slot's tokens. rows: the intermediate width of every slot of the launch.
template <int TYPE, int L>
__global__ __launch_bounds__(256) void k_gate_up(ExpertArgs a, int rows, int chunk) {
    extern __shared__ __attribute__((aligned(16))) float lds_x[];
    constexpr int JW = 32 / L, JG = 4 * JW;
    const int groups = (rows + JG - 1) / JG;
    // an item is (token chunk index tc, slot, row group), tc outermost: a slot's chunks go to different
    // workgroups, so one with 8 tokens is not a single item taking twice as long as the rest (chunks tc,
    // tc + nc, ... when a slot holds more than kGemvTok tokens)
    const int nc = (kGemvTok + chunk - 1) / chunk;
    const int per_c = expert_slots(a) * groups;
    const int items = per_c * nc;
    const int lane = threadIdx.x & 63, c = lane % L, rw = (lane & 31) / L;
    const bool up_half = lane >= 32;
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int nb = a.H / kQK;
    const int64_t rs = static_cast<int64_t>(nb) * BlockInfo<TYPE>::bytes;
    const int ldx = lds_row_floats(a.H), ldsum = a.H / 16;
    for (int item = blockIdx.x; item < items; item += gridDim.x) {
        const int tc = item / per_c, it = item - tc * per_c;
        const int slot = it / groups;
        const ExpertView v = expert_view(a, slot, true);
        const int first = v.begin + tc * chunk;
        if (first >= v.end) continue;  // whole workgroup: the slot has fewer chunks
        const int inter = static_cast<int>(v.stride_rows);
        const int j = (it - slot * groups) * JG + wv * JW + rw;
        const uint8_t* wrow = v.w + static_cast<int64_t>((up_half ? inter : 0) + min(j, inter - 1)) * rs;
        float* hout = v.routed ? a.h : a.h_sh;
        BlockDot<TYPE> blk;
        blk.fetch(wrow + c * BlockInfo<TYPE>::bytes);  // the first block's loads overlap the staging below
        for (int p0 = first; p0 < v.end; p0 += nc * chunk) {
            const int n = min(chunk, v.end - p0);
            __syncthreads();  // the previous chunk's LDS rows are no longer read
            stage_chunk(lds_x, n, a.H, [&](int u) {
                const int pos = p0 + u;
                return a.x + static_cast<int64_t>(v.routed ? a.sorted[pos] / a.k : pos) * a.H;
            });
            if ((it - slot * groups) * JG + wv * JW >= inter) continue;  // whole wavefront
            float acc[kGemvTok];
#pragma unroll
            for (int u = 0; u < kGemvTok; u++) acc[u] = 0.0f;
            for (int kb = c; kb < nb; kb += L) {
                if (kb != c || p0 != first) blk.fetch(wrow + kb * BlockInfo<TYPE>::bytes);
                blk.run(lds_x + kb * kBlkFloats, ldx, lds_x + n * ldx + 16 * kb, ldsum, n, acc);
            }
#pragma unroll
            for (int u = 0; u < kGemvTok; u++) {
                if (u < n) {
                    const float sum = row_sum<L>(acc[u]);
                    const float us = __shfl_xor(sum, 32);  // the up row's sum, from the other half
                    if (!up_half && c == 0 && j < inter)
                        hout[static_cast<int64_t>(p0 + u) * inter + j] = silu(sum) * us;
                }
            }
        }
    }
}

// The down kernel spreads each block of a row over 8 lanes (one 16-byte slice per lane, so a wavefront's weight
// loads are contiguous) and reads a lane's h runs from LDS once per token for kDnPasses rows. (Lane-per-block
// loads as in k_gate_up read a 210-byte Q6_K block per lane with strided dword loads: slower for down, measured.)
// Its LDS rows are padded by 4 floats after every 64 values (lds_padded_index).
constexpr int kDnPasses = 4;       // down: row passes per wavefront (R rows each)
__host__ __device__ inline int lds_padded_floats(int width) { return width + 4 * (width / 64); }
__device__ __forceinline__ int lds_padded_index(int i) { return i + 4 * (i >> 6); }

// Tokens per chunk for rows of `width` values: kGemvTok, or fewer when their LDS copy would pass kGemvLdsMax.
__host__ inline int gemv_chunk_padded(int width) {
    const int per = kGemvLdsMax / (4 * lds_padded_floats(width));
    return per < 1 ? 1 : (per < kGemvTok ? per : kGemvTok);
}

// rows u < n of the chunk: src_row(u) -> LDS row u (width values, a multiple of 64), 16 bytes per load
template <typename SrcRow>
__device__ __forceinline__ void stage_padded_rows(float* lds, int n, int width, SrcRow src_row) {
    const int per_row = width / 4;
    const int ld = lds_padded_floats(width);
    for (int f = threadIdx.x; f < n * per_row; f += blockDim.x) {
        const int u = f / per_row, i = 4 * (f - u * per_row);
        *reinterpret_cast<float4*>(lds + u * ld + lds_padded_index(i)) =
            *reinterpret_cast<const float4*>(src_row(u) + i);
    }
}

// the lane's 16 values from LDS row u at value offset i (16-aligned: never straddles a padding gap)
__device__ __forceinline__ void lds_padded_run(const float* lds, int ld, int u, int i, float4 x[4]) {
    const float4* q = reinterpret_cast<const float4*>(lds + u * ld + lds_padded_index(i));
#pragma unroll
    for (int j = 0; j < 4; j++) x[j] = q[j];
}

// down: a row group is 4 wavefronts x kDnPasses passes x R output rows (R = 64 / WIDTH, WIDTH = 8 nb lanes per
// row when nb = inter / 256 is 1, 2 or 4: the lane then holds one block of each of its rows, decoded once; otherwise
// one row per pass over all 64 lanes, blocks g, g + 8, ..., decoded again per token). o[pos, r] = down[r] . h[pos];
// a lane's h runs are the same for every row it covers, so each token's are read from LDS once per block.
template <int TYPE, int WIDTH>
__global__ __launch_bounds__(256) void k_down(ExpertArgs a, int chunk) {
    extern __shared__ __attribute__((aligned(16))) float lds_h[];
    constexpr int R = WIDTH == 64 ? 1 : 64 / WIDTH;
    constexpr int kRowsPerWave = R * kDnPasses;
    const int groups = (a.H + 4 * kRowsPerWave - 1) / (4 * kRowsPerWave);
    const int items = expert_slots(a) * groups;
    const int lane = threadIdx.x & 63, g = lane >> 3, c = lane & 7;
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lo_start = BlockInfo<TYPE>::lo_start(c), hi_off = BlockInfo<TYPE>::hi_offset;
    for (int it = blockIdx.x; it < items; it += gridDim.x) {
        const int slot = it / groups;
        const ExpertView v = expert_view(a, slot, false);
        const int inter = static_cast<int>(v.stride_rows);
        const int nb = inter / kQK;
        const int ld = lds_padded_floats(inter);
        const int64_t rs = static_cast<int64_t>(nb) * BlockInfo<TYPE>::bytes;
        const int row_off = R > 1 ? g / nb : 0;
        const int kb0 = R > 1 ? g % nb : g;
        const int kb_step = R > 1 ? nb : 8;
        const bool slot_used = R > 1 ? (g < R * nb) : true;
        const int wave_row0 = (it - slot * groups) * 4 * kRowsPerWave + wv * kRowsPerWave;
        const float* hin = v.routed ? a.h : a.h_sh;
        float* oout = v.routed ? a.o : a.o_sh;
        Lane32 w[kDnPasses];
        auto decode_rows = [&](int kb) {
            RawLane<TYPE> raw[kDnPasses];
#pragma unroll
            for (int q = 0; q < kDnPasses; q++) {
                const int row = min(wave_row0 + q * R + row_off, a.H - 1);  // past H: never stored
                raw[q].fetch(v.w + static_cast<int64_t>(row) * rs + kb * BlockInfo<TYPE>::bytes, c);
            }
#pragma unroll
            for (int q = 0; q < kDnPasses; q++) raw[q].unpack(c, w[q]);
        };
        const bool one_block = R > 1;  // the lane's only block is kb0
        if (one_block && slot_used && wave_row0 < a.H) decode_rows(kb0);
        for (int p0 = v.begin; p0 < v.end; p0 += chunk) {
            const int n = min(chunk, v.end - p0);
            __syncthreads();
            stage_padded_rows(lds_h, n, inter, [&](int u) { return hin + static_cast<int64_t>(p0 + u) * inter; });
            __syncthreads();
            if (wave_row0 >= a.H) continue;  // whole wavefront
#pragma unroll 1
            for (int u = 0; u < n; u++) {
                float acc[kDnPasses];
#pragma unroll
                for (int q = 0; q < kDnPasses; q++) acc[q] = 0.0f;
                if (slot_used) {
                    for (int kb = kb0; kb < nb; kb += kb_step) {
                        if (!one_block) decode_rows(kb);
                        float4 xl[4], xh[4];
                        lds_padded_run(lds_h, ld, u, kb * kQK + lo_start, xl);
                        lds_padded_run(lds_h, ld, u, kb * kQK + lo_start + hi_off, xh);
                        const float sxl = sum16(xl), sxh = sum16(xh);
#pragma unroll
                        for (int q = 0; q < kDnPasses; q++) acc[q] += lane_dot_s(w[q], xl, xh, sxl, sxh);
                    }
                }
#pragma unroll
                for (int q = 0; q < kDnPasses; q++) {
                    const float sum = group_sum<WIDTH>(acc[q]);
                    const int row = wave_row0 + q * R + row_off;
                    if ((lane & (WIDTH - 1)) == 0 && slot_used && row < a.H)
                        oout[static_cast<int64_t>(p0 + u) * a.H + row] = sum;
                }
            }
        }
    }
}

// y[t, r] = sum over the token's experts in ascending id of w * o[pos, r], then + sg[t] * o_sh[t, r]. A workgroup
// takes kCombineSpan values of one token, 8 per thread, so the token's table entries (picks: position and weight,
// already in ascending expert id, the same for the whole workgroup) are read with scalar loads once per workgroup.
// For k <= 8 every entry is loaded first and then every o row, so the loads overlap instead of forming k dependent
// chains; the sum is the same in both forms. Position pos's output row starts at byte 4 H pos of o: fp32 from a
// GEMV expert, or bf16 (its first 2 H bytes) from an MFMA expert, which its entry marks with kPosBf16. SH: the
// shared expert's output type (float or uint16_t for bf16, rows of H). H is a multiple of 8.
constexpr int kCombineUnroll = 8;
constexpr int kCombineSpan = 8 * 256;

struct Float8 {
    float4 a, b;
};
__device__ __forceinline__ Float8 load8(const float* p) {
    return {*reinterpret_cast<const float4*>(p), *reinterpret_cast<const float4*>(p + 4)};
}
__device__ __forceinline__ float4 bf16x4_to_float4(uint32_t lo, uint32_t hi) {
    return make_float4(__builtin_bit_cast(float, lo << 16), __builtin_bit_cast(float, lo & 0xFFFF0000u),
                       __builtin_bit_cast(float, hi << 16), __builtin_bit_cast(float, hi & 0xFFFF0000u));
}
__device__ __forceinline__ Float8 load8(const uint16_t* p) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    return {bf16x4_to_float4(v.x, v.y), bf16x4_to_float4(v.z, v.w)};
}
// 8 values of position pos's output row, from column r (flag: the row is bf16)
__device__ __forceinline__ Float8 load_o8(const float* o, int64_t pos, int H, int r, bool bf16) {
    return bf16 ? load8(reinterpret_cast<const uint16_t*>(o) + pos * 2 * H + r) : load8(o + pos * H + r);
}

template <typename SH>
__global__ __launch_bounds__(256) void k_combine(int T, int H, int k, const uint2* __restrict__ picks,
                                                 const float* __restrict__ o,
                                                 const SH* __restrict__ o_sh, const float* __restrict__ sg,
                                                 const float* __restrict__ resid, float* __restrict__ y,
                                                 const uint32_t* status) {
    // fork scope (status: the workspace's status word). k_fork_gate, just before on this stream, has seen the MFMA
    // experts done; one acquire drops any line of their outputs this XCD's caches still hold from an earlier call.
    // Once a hand-off has given up, those outputs are stale, so every output is NaN until wl_moe_workspace_status
    // has reported it.
    if (status) {
        if (threadIdx.x == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        __syncthreads();
    }
    const bool stale =
        status && (__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kStatusFork) != 0;
    const int spans = (H + kCombineSpan - 1) / kCombineSpan;
    const int t = static_cast<int>(blockIdx.x) / spans;
    const int r = (static_cast<int>(blockIdx.x) - t * spans) * kCombineSpan + 8 * static_cast<int>(threadIdx.x);
    if (t >= T || r >= H) return;
    const int P = T * k;
    const int64_t base = static_cast<int64_t>(t) * k;
    float4 a0 = make_float4(0.f, 0.f, 0.f, 0.f), a1 = a0;
    auto add = [&](int n, float wv, const Float8& ov) {
        if (n == 0) {
            a0 = make_float4(wv * ov.a.x, wv * ov.a.y, wv * ov.a.z, wv * ov.a.w);
            a1 = make_float4(wv * ov.b.x, wv * ov.b.y, wv * ov.b.z, wv * ov.b.w);
        } else {
            a0.x += wv * ov.a.x;
            a0.y += wv * ov.a.y;
            a0.z += wv * ov.a.z;
            a0.w += wv * ov.a.w;
            a1.x += wv * ov.b.x;
            a1.y += wv * ov.b.y;
            a1.z += wv * ov.b.z;
            a1.w += wv * ov.b.w;
        }
    };
    // an entry's position (-1 for a dropped pick, whose entry is 0xFFFFFFFF, or out of range) and flag
    auto position = [&](uint32_t pp, bool& bf16) {
        bf16 = (pp & kPosBf16) != 0;
        const int pos = static_cast<int>(pp & ~kPosBf16);
        return pos < P ? pos : -1;
    };
    if (k <= kCombineUnroll) {
        int pos[kCombineUnroll];
        bool bf[kCombineUnroll];
        float wv[kCombineUnroll];
#pragma unroll
        for (int n = 0; n < kCombineUnroll; n++) {
            pos[n] = -1;
            bf[n] = false;
            wv[n] = 0.0f;
            if (n < k) {
                const uint2 e = picks[base + n];
                pos[n] = position(e.x, bf[n]);
                wv[n] = __builtin_bit_cast(float, e.y);
            }
        }
        Float8 ov[kCombineUnroll];
#pragma unroll
        for (int n = 0; n < kCombineUnroll; n++)
            if (n < k && pos[n] >= 0) ov[n] = load_o8(o, pos[n], H, r, bf[n]);
#pragma unroll
        for (int n = 0; n < kCombineUnroll; n++)
            if (n < k && pos[n] >= 0) add(n, wv[n], ov[n]);
    } else {
        for (int n = 0; n < k; n++) {
            const uint2 e = picks[base + n];
            bool bf16;
            const int pos = position(e.x, bf16);
            if (pos < 0) continue;
            add(n, __builtin_bit_cast(float, e.y), load_o8(o, pos, H, r, bf16));
        }
    }
    if (o_sh) {
        const float gv = sg ? sg[t] : 1.0f;
        const Float8 sv = load8(o_sh + static_cast<int64_t>(t) * H + r);
        a0.x += gv * sv.a.x;
        a0.y += gv * sv.a.y;
        a0.z += gv * sv.a.z;
        a0.w += gv * sv.a.w;
        a1.x += gv * sv.b.x;
        a1.y += gv * sv.b.y;
        a1.z += gv * sv.b.z;
        a1.w += gv * sv.b.w;
    }
    if (resid) {  // y = x + MoE (WL_MOE_RESIDUAL)
        const Float8 xv = load8(resid + static_cast<int64_t>(t) * H + r);
        a0 = make_float4(__fadd_rn(xv.a.x, a0.x), __fadd_rn(xv.a.y, a0.y), __fadd_rn(xv.a.z, a0.z),
                         __fadd_rn(xv.a.w, a0.w));
        a1 = make_float4(__fadd_rn(xv.b.x, a1.x), __fadd_rn(xv.b.y, a1.y), __fadd_rn(xv.b.z, a1.z),
                         __fadd_rn(xv.b.w, a1.w));
    }
    if (stale) {
        const float q = __builtin_nanf("");
        a0 = make_float4(q, q, q, q);
        a1 = a0;
    }
    float* out = y + static_cast<int64_t>(t) * H + r;
    *reinterpret_cast<float4*>(out) = a0;
    *reinterpret_cast<float4*>(out + 4) = a1;
}

// ---------------------------------------------------------------------------------------------------------------
// Host side

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Carves the workspace; with base == nullptr only computes the size.
// Whether wl_moe_layer's router runs as k_router_parts + k_topk_parts (a single token runs the fused kernel).
static bool router_parts(int64_t T) { return T >= 2 && T <= kRouterPartsMaxT; }

Workspace carve(const WlMoeLayer& L, int64_t T, void* base) {
    Workspace w{};
    const int64_t P = T * L.top_k;
    const int64_t nchunks = (T + kSortChunk - 1) / kSortChunk;
    const bool shared = L.shared_gate_up != nullptr;
    size_t off = 0;
    auto take = [&](size_t bytes) -> void* {
        void* p = base ? static_cast<char*>(base) + off : nullptr;
        off = align_up(off + bytes, 256);
        return p;
    };
    w.sync = static_cast<uint32_t*>(take(sizeof(uint32_t) * kSyncWords));
    w.logits = static_cast<float*>(take(sizeof(float) * T * (L.n_experts + 1)));
    w.sg = static_cast<float*>(take(sizeof(float) * T));
    w.ids = static_cast<int32_t*>(take(sizeof(int32_t) * P));
    w.wts = static_cast<float*>(take(sizeof(float) * P));
    w.crank = static_cast<int32_t*>(take(sizeof(int32_t) * P));
    w.rank = static_cast<int32_t*>(take(sizeof(int32_t) * P));
    w.hist = static_cast<int32_t*>(take(sizeof(int32_t) * nchunks * L.n_experts));
    w.offsets = static_cast<int32_t*>(take(sizeof(int32_t) * (L.n_experts + 1)));
    w.active = static_cast<int32_t*>(take(sizeof(int32_t) * (L.n_experts + 1)));
    w.sorted = static_cast<int32_t*>(take(sizeof(int32_t) * P));
    w.picks = static_cast<uint2*>(take(sizeof(uint2) * P));
    w.h = static_cast<float*>(take(sizeof(float) * P * L.inter));
    w.o = static_cast<float*>(take(sizeof(float) * P * L.hidden));
    w.h_sh = static_cast<float*>(take(shared ? sizeof(float) * T * L.shared_inter : 0));
    w.o_sh = static_cast<float*>(take(shared ? sizeof(float) * T * L.hidden : 0));
    const ExpertPlan plan = expert_plan(L, T);
    const bool mfma = plan != kPlanGemv;
    const int gmax = plan_gemv_max(plan);
    w.xb = static_cast<uint16_t*>(take(mfma ? sizeof(uint16_t) * T * L.hidden : 0));
    w.tiles = static_cast<int4*>(take(mfma ? sizeof(int4) * max_tiles(L, T, kTileTokens, gmax) : 0));
    w.tiles_down = static_cast<int4*>(take(mfma ? sizeof(int4) * max_tiles(L, T, kDownTileTokens, gmax) : 0));
    w.n_tiles = static_cast<int32_t*>(take(mfma ? 2 * sizeof(int32_t) : 0));
    w.h16 = static_cast<uint16_t*>(take(mfma ? sizeof(uint16_t) * P * L.inter : 0));
    w.h_sh16 = static_cast<uint16_t*>(take(mfma && shared ? sizeof(uint16_t) * T * L.shared_inter : 0));
    w.xn = static_cast<float*>(take((L.flags & WL_MOE_PRE_NORM) ? sizeof(float) * T * L.hidden : 0));
    w.parts = static_cast<float*>(take(router_parts(T) ? sizeof(float) * (L.hidden / kRouterSeg) * T *
                                                             (L.n_experts + 1) : 0));
    w.bytes = off;
    return w;
}

static int check_one_layer(const WlMoeLayer* L);

int check_layer(const WlMoeLayer* L) {
    const int rc = check_one_layer(L);
    if (rc || !L->next) return rc;
    return check_one_layer(L->next);  // only its own fields; its next is not followed
}

static int check_one_layer(const WlMoeLayer* L) {
    if (!L) return WL_EINVAL_NULL;
    if ((L->flags & WL_MOE_PRE_NORM) && (!(L->norm_eps >= 0.0f) || reinterpret_cast<uintptr_t>(L->norm_weight) % 16))
        return WL_EINVAL_SHAPE;
    if (!(L->min_expert_weight >= 0.0f && L->min_expert_weight <= 1.0f)) return WL_EINVAL_SHAPE;  // NaN too
    if (!L->gate_up || !L->down || !L->router) return WL_EINVAL_NULL;
    if (block_bytes(L->gate_up_type) < 0 || block_bytes(L->down_type) < 0) return WL_EINVAL_TYPE;
    if (L->hidden <= 0 || L->hidden % kQK != 0 || L->hidden > kRouterSeg * 32 * kRouterMaxJ) return WL_EINVAL_SHAPE;
    if (L->inter <= 0 || L->inter % kQK != 0 || L->inter > kMaxK) return WL_EINVAL_SHAPE;
    if (L->n_experts < 1 || L->n_experts > 64 * kMaxEJ) return WL_EINVAL_SHAPE;
    if (L->top_k < 1 || L->top_k > L->n_experts || L->top_k > WL_MAX_TOPK) return WL_EINVAL_TOPK;
    if (L->gate_up_stride < 2LL * L->inter * (L->hidden / kQK) * block_bytes(L->gate_up_type)) return WL_EINVAL_SHAPE;
    if (L->down_stride < static_cast<int64_t>(L->hidden) * (L->inter / kQK) * block_bytes(L->down_type))
        return WL_EINVAL_SHAPE;
    if (reinterpret_cast<uintptr_t>(L->gate_up) % base_alignment(L->gate_up_type) ||
        L->gate_up_stride % base_alignment(L->gate_up_type))
        return WL_EINVAL_ALIGN;
    if (reinterpret_cast<uintptr_t>(L->down) % base_alignment(L->down_type) ||
        L->down_stride % base_alignment(L->down_type))
        return WL_EINVAL_ALIGN;
    if (reinterpret_cast<uintptr_t>(L->router) % 16) return WL_EINVAL_ALIGN;
    if (L->shared_gate_up) {
        if (!L->shared_down) return WL_EINVAL_NULL;
        if (block_bytes(L->shared_gate_up_type) < 0 || block_bytes(L->shared_down_type) < 0) return WL_EINVAL_TYPE;
        if (L->shared_inter <= 0 || L->shared_inter % kQK != 0 || L->shared_inter > kMaxK) return WL_EINVAL_SHAPE;
        if (reinterpret_cast<uintptr_t>(L->shared_gate_up) % base_alignment(L->shared_gate_up_type) ||
            reinterpret_cast<uintptr_t>(L->shared_down) % base_alignment(L->shared_down_type))
            return WL_EINVAL_ALIGN;
        if (L->shared_gate && reinterpret_cast<uintptr_t>(L->shared_gate) % 16) return WL_EINVAL_ALIGN;
    }
    return WL_OK;
}

static int launch_router(const WlMoeLayer& L, const float* x, int64_t T, float* logits, float* sg, uint16_t* xb,
                         hipStream_t s) {
    const float* shared_gate = (L.shared_gate_up && L.shared_gate) ? L.shared_gate : nullptr;
    const int rows = L.n_experts + (shared_gate ? 1 : 0);
    const int grid = (rows + 1) / 2;
    if (T == 1)
        k_router1<<<grid, 64, 0, s>>>(x, L.router, L.router_bias, shared_gate, L.hidden, L.n_experts, logits, sg);
    else
        k_router_split<<<dim3(static_cast<unsigned>((T + 15) / 16), static_cast<unsigned>((rows + 15) / 16)),
                          64 * kRsWaves, 0, s>>>(x, L.router, L.router_bias, shared_gate, static_cast<int>(T),
                                                 L.hidden, L.n_experts, logits, sg, xb);
    return launch_status();
}

static int launch_topk(const WlMoeLayer& L, const float* logits, int64_t T, int32_t* ids, float* wts,
                       int32_t* crank, float min_w, hipStream_t s) {
    const int grid = static_cast<int>((T + 3) / 4);
    const int E = L.n_experts, k = L.top_k, rn = L.norm_topk_prob ? 1 : 0, Ti = static_cast<int>(T);
    if (E <= 64)
        k_topk<1><<<grid, 256, 0, s>>>(logits, Ti, E, k, rn, ids, wts, crank, min_w);
    else if (E <= 128)
        k_topk<2><<<grid, 256, 0, s>>>(logits, Ti, E, k, rn, ids, wts, crank, min_w);
    else if (E <= 256)
        k_topk<4><<<grid, 256, 0, s>>>(logits, Ti, E, k, rn, ids, wts, crank, min_w);
    else if (E <= 512)
        k_topk<8><<<grid, 256, 0, s>>>(logits, Ti, E, k, rn, ids, wts, crank, min_w);
    else
        k_topk<16><<<grid, 256, 0, s>>>(logits, Ti, E, k, rn, ids, wts, crank, min_w);
    return launch_status();
}

// Router and top-k of a call of 2 .. kRouterPartsMaxT tokens: k_router_parts, then k_topk_parts.
static int launch_router_parts(const WlMoeLayer& L, const float* x, int64_t T, const Workspace& w, uint16_t* xb,
                               hipStream_t s) {
    const float* shared_gate = (L.shared_gate_up && L.shared_gate) ? L.shared_gate : nullptr;
    const int rows = L.n_experts + (shared_gate ? 1 : 0);
    const int nseg = L.hidden / kRouterSeg;
    k_router_parts<<<dim3(static_cast<unsigned>((T + 15) / 16), static_cast<unsigned>((rows + 15) / 16),
                          static_cast<unsigned>((nseg + kRsWaves - 1) / kRsWaves)),
                     64 * kRsWaves, 0, s>>>(x, L.router, shared_gate, static_cast<int>(T), L.hidden, L.n_experts,
                                            w.parts, xb, w.sync + kTopkDone);
    return launch_status();
}

// With g, the grouping follows in the same launch (k_topk_group, 1024 threads: one per expert for the grouping).
static int launch_topk_parts(const WlMoeLayer& L, int64_t T, const Workspace& w, float* sg, const GroupOut* g,
                             hipStream_t s) {
    const int rows = L.n_experts + ((L.shared_gate_up && L.shared_gate) ? 1 : 0);
    const int nseg = L.hidden / kRouterSeg;
    const int Ti = static_cast<int>(T);
    const unsigned grid = static_cast<unsigned>(T);
    const int E = L.n_experts, k = L.top_k, rn = L.norm_topk_prob ? 1 : 0;
    const unsigned threads = static_cast<unsigned>(rows + 63) / 64 * 64 < 1024u ? (rows + 63) / 64 * 64 : 1024u;
    // every instance has the same parameters; 32 segments: hidden 2048
    if (g) {
        auto pick = [&](auto seg32) {
            constexpr int S = decltype(seg32)::value;
            return E <= 64 ? k_topk_group<1, S> : E <= 128 ? k_topk_group<2, S> : E <= 256 ? k_topk_group<4, S>
                   : E <= 512 ? k_topk_group<8, S> : k_topk_group<16, S>;
        };
        auto kernel = nseg == 32 ? pick(std::integral_constant<int, 32>{}) : pick(std::integral_constant<int, 0>{});
        kernel<<<grid, kSortSmallThreads, 0, s>>>(w.parts, nseg, L.router_bias, Ti, E, rows, k, rn, w.ids, w.wts,
                                                  w.crank, sg, *g, L.min_expert_weight);
        return launch_status();
    }
    auto pick = [&](auto seg32) {
        constexpr int S = decltype(seg32)::value;
        return E <= 64 ? k_topk_parts<1, S> : E <= 128 ? k_topk_parts<2, S> : E <= 256 ? k_topk_parts<4, S>
               : E <= 512 ? k_topk_parts<8, S> : k_topk_parts<16, S>;
    };
    auto kernel = nseg == 32 ? pick(std::integral_constant<int, 32>{}) : pick(std::integral_constant<int, 0>{});
    kernel<<<grid, threads, 0, s>>>(w.parts, nseg, L.router_bias, Ti, E, rows, k, rn, w.ids, w.wts, w.crank, sg,
                                    L.min_expert_weight);
    return launch_status();
}

// The grouping; with an MFMA plan (tiles) also the tile lists of the experts with more than gemv_max pairs; in a
// fork scope (fork) it then publishes itself to the second stream (withhold: WL_MOE_TEST_STARVE, it does not).
static int launch_sort(const WlMoeLayer& L, const Workspace& w, const int32_t* ids, int64_t T, bool tiles,
                       int gemv_max, bool fork, bool withhold, hipStream_t s) {
    const int E = L.n_experts, k = L.top_k;
    const TileOut to{tiles ? w.tiles : nullptr, w.tiles_down, w.n_tiles, L.shared_gate_up ? 1 : 0, gemv_max};
    const int nchunks = static_cast<int>((T + kSortChunk - 1) / kSortChunk);
    if (nchunks == 1) {
        k_sort_small<<<1, kSortSmallThreads, 0, s>>>(ids, static_cast<int>(T), k, E, w.offsets, w.active, w.sorted,
                                                     PickOut{w.crank, w.wts, w.picks}, to, fork ? w.sync : nullptr,
                                                     withhold ? 1 : 0);
    } else {
        const size_t lds = sizeof(uint32_t) * E * kSortWords + sizeof(int32_t) * E;
        k_sort_hist<<<nchunks, 1024, lds, s>>>(ids, static_cast<int>(T), k, E, w.rank, w.hist);
        k_sort_scan<<<1, kSortSmallThreads, 0, s>>>(static_cast<int>(T), k, E, nchunks, w.hist, w.offsets,
                                                    w.active, to);
        const int64_t P = T * k;
        k_sort_scatter<<<static_cast<int>((P + 255) / 256), 256, 0, s>>>(
            ids, static_cast<int>(T), k, E, w.rank, w.hist, w.offsets, tiles ? gemv_max : 0x7FFFFFFF, w.sorted,
            PickOut{w.crank, w.wts, w.picks});
        if (fork)
            k_fork_store<<<1, 64, 0, s>>>(w.sync + kForkDone, 0u, withhold ? nullptr : w.sync + kForkSorted, 1u);
    }
    return launch_status();
}

// Workgroups of a GEMV expert launch: enough to fill the GPU several times over, never more than the items
static unsigned gemv_grid(int64_t items) {
    constexpr int64_t kMaxGroups = 2048;
    return static_cast<unsigned>(items < kMaxGroups ? (items > 0 ? items : 1) : kMaxGroups);
}

template <int TYPE, int L>
static void launch_gate_up_l(const ExpertArgs& a, int rows, int max_slots, hipStream_t s) {
    constexpr int JG = 4 * (32 / L);
    const int chunk = gemv_chunk(a.H);
    const unsigned grid =
        gemv_grid(static_cast<int64_t>(max_slots) * ((rows + JG - 1) / JG) * ((kGemvTok + chunk - 1) / chunk));
    k_gate_up<TYPE, L><<<grid, 256, sizeof(float) * chunk * lds_chunk_floats(a.H), s>>>(a, rows, chunk);
}

template <int TYPE>
static void launch_gate_up_t(const ExpertArgs& a, int rows, int max_slots, hipStream_t s) {
    switch (gemv_lanes(a.H / kQK)) {
        case 1: launch_gate_up_l<TYPE, 1>(a, rows, max_slots, s); break;
        case 2: launch_gate_up_l<TYPE, 2>(a, rows, max_slots, s); break;
        case 4: launch_gate_up_l<TYPE, 4>(a, rows, max_slots, s); break;
        default: launch_gate_up_l<TYPE, 8>(a, rows, max_slots, s); break;
    }
}

static void launch_gate_up(int type, const ExpertArgs& a, int rows, int max_slots, hipStream_t s) {
    if (type == WL_TYPE_Q4_K)
        launch_gate_up_t<WL_TYPE_Q4_K>(a, rows, max_slots, s);
    else
        launch_gate_up_t<WL_TYPE_Q6_K>(a, rows, max_slots, s);
}

template <int TYPE, int WIDTH>
static void launch_down_w(const ExpertArgs& a, int inter, int max_slots, hipStream_t s) {
    constexpr int R = WIDTH == 64 ? 1 : 64 / WIDTH;
    const unsigned grid =
        gemv_grid(static_cast<int64_t>(max_slots) * ((a.H + 4 * R * kDnPasses - 1) / (4 * R * kDnPasses)));
    const int chunk = gemv_chunk_padded(inter);
    k_down<TYPE, WIDTH><<<grid, 256, sizeof(float) * chunk * lds_padded_floats(inter), s>>>(a, chunk);
}

template <int TYPE>
static void launch_down_t(const ExpertArgs& a, int inter, int max_slots, hipStream_t s) {
    switch (row_geom_width(inter / kQK)) {
        case 8: launch_down_w<TYPE, 8>(a, inter, max_slots, s); break;
        case 16: launch_down_w<TYPE, 16>(a, inter, max_slots, s); break;
        case 32: launch_down_w<TYPE, 32>(a, inter, max_slots, s); break;
        default: launch_down_w<TYPE, 64>(a, inter, max_slots, s); break;
    }
}

static void launch_down(int type, const ExpertArgs& a, int inter, int max_slots, hipStream_t s) {
    if (type == WL_TYPE_Q4_K)
        launch_down_t<WL_TYPE_Q4_K>(a, inter, max_slots, s);
    else
        launch_down_t<WL_TYPE_Q6_K>(a, inter, max_slots, s);
}

// The fp32 GEMV expert stages (gate_up + SwiGLU, then down) of the experts listed in `active`, and of the shared
// expert when with_shared. max_routed bounds how many experts the list can hold (it sizes the grids; the kernels
// read the actual count).
static ExpertArgs gemv_args(const WlMoeLayer& L, const float* x, int64_t tokens, const Workspace& w, int max_routed,
                            bool with_shared) {
    ExpertArgs a{};
    a.gate_up = static_cast<const uint8_t*>(L.gate_up);
    a.gate_up_stride = L.gate_up_stride;
    a.down = static_cast<const uint8_t*>(L.down);
    a.down_stride = L.down_stride;
    a.sh_gate_up = static_cast<const uint8_t*>(L.shared_gate_up);
    a.sh_down = static_cast<const uint8_t*>(L.shared_down);
    a.x = x;
    a.T = static_cast<int>(tokens);
    a.H = L.hidden;
    a.inter = L.inter;
    a.sh_inter = with_shared ? L.shared_inter : 0;
    a.k = L.top_k;
    a.offsets = w.offsets;
    a.active = w.active;
    a.sorted = w.sorted;
    a.h = w.h;
    a.h_sh = w.h_sh;
    a.o = w.o;
    a.o_sh = w.o_sh;
    a.routed = max_routed > 0 ? 1 : 0;
    return a;
}

static void launch_gemv_gate_up(const WlMoeLayer& L, ExpertArgs a, int max_routed, bool with_shared,
                                hipStream_t s) {
    // the routed experts and the shared expert share a launch when their types and widths agree
    const bool fuse = with_shared && L.shared_gate_up_type == L.gate_up_type && L.shared_inter == L.inter;
    a.shared_slot = fuse ? 1 : 0;
    if (max_routed > 0 || fuse) launch_gate_up(L.gate_up_type, a, L.inter, max_routed + a.shared_slot, s);
    if (with_shared && !fuse) {
        a.routed = 0;
        a.shared_slot = 1;
        launch_gate_up(L.shared_gate_up_type, a, L.shared_inter, 1, s);
    }
}

static void launch_gemv_down(const WlMoeLayer& L, ExpertArgs a, int max_routed, bool with_shared, hipStream_t s) {
    const bool fuse = with_shared && L.shared_down_type == L.down_type && L.shared_inter == L.inter;
    a.shared_slot = fuse ? 1 : 0;
    if (max_routed > 0 || fuse) launch_down(L.down_type, a, L.inter, max_routed + a.shared_slot, s);
    if (with_shared && !fuse) {
        a.routed = 0;
        a.shared_slot = 1;
        launch_down(L.shared_down_type, a, L.shared_inter, 1, s);
    }
}

ExpertPlan expert_plan(const WlMoeLayer& L, int64_t T) {
    if (L.flags & WL_MOE_NO_MFMA) return kPlanGemv;
    if (!(L.flags & WL_MOE_FORCE_MFMA) && T <= kGemvMaxTokens) return kPlanGemv;  // no expert can exceed 8 pairs
    if (!prefill_eligible(L, T)) return kPlanGemv;
    return (L.flags & WL_MOE_FORCE_MFMA) ? kPlanMfma : kPlanSplit;
}

}  // namespace wl

using namespace wl;

extern "C" {

const char* wl_error_string(int code) {
    switch (code) {
        case WL_OK: return "ok";
        case WL_EINVAL_TYPE: return "unsupported ggml type (only Q4_K = 12 and Q6_K = 14 run here)";
        case WL_EINVAL_SHAPE: return "invalid shape: sizes must be positive, k a multiple of 256, within limits";
        case WL_EINVAL_NULL: return "a required pointer is NULL";
        case WL_EINVAL_ALIGN: return "misaligned pointer or stride (Q4_K: 16 bytes; Q6_K: 4; activations: 16)";
        case WL_EINVAL_TOPK: return "top_k must be in 1..min(n_experts, 16)";
        case WL_EINVAL_WORKSPACE: return "workspace is NULL or smaller than wl_moe_workspace_bytes()";
        case WL_EINVAL_DTYPE: return "output dtype must be WL_DTYPE_F32 or WL_DTYPE_BF16";
        case WL_EINVAL_COUNT: return "expert count must be in 1..64";
        case WL_EINVAL_OVERLAP: return "y overlaps x: the layer writes y while x is still being read";
        case WL_ESYNC:
            return "a bounded wait gave up: a fused-kernel workgroup waiting for another (not every workgroup was "
                   "resident; those outputs hold NaN) or a fork-scope hand-off (the scope's MFMA experts were "
                   "skipped since; those outputs are stale)";
        case WL_EINVAL_SCOPE:
            return "fork scope: wl_moe_fork_begin with a scope already open on this device, or wl_moe_fork_end "
                   "without one open on this stream";
        case WL_EINVAL_SCRATCH:
            return "the call needs more workspace than wl_moe_layer_noalloc's scratch holds "
                   "(WL_NOALLOC_SCRATCH_BYTES): use wl_moe_layer with a workspace";
        default: break;
    }
    if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
    return "unknown error";
}

int wl_abi_version(void) { return (1 << 16) | 3; }  // 1.3: min_expert_weight (was reserved2, 0); 1.2: next, noalloc

int wl_moe_check(const WlMoeLayer* layer) { return check_layer(layer); }

size_t wl_moe_workspace_bytes(const WlMoeLayer* layer, int64_t tokens) {
    if (check_layer(layer) != WL_OK || tokens <= 0) return 0;
    return carve(*layer, tokens, nullptr).bytes;
}

int wl_moe_route(const WlMoeLayer* layer, const float* x, int64_t tokens, float* logits, int32_t* ids,
                 float* weights, float* shared_gate_out, void* stream) {
    int rc = check_layer(layer);
    if (rc) return rc;
    if (!x || !logits || !ids || !weights) return WL_EINVAL_NULL;
    if (layer->shared_gate_up && layer->shared_gate && !shared_gate_out) return WL_EINVAL_NULL;
    if (tokens <= 0 || tokens > kMaxTokens) return WL_EINVAL_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16) return WL_EINVAL_ALIGN;
    hipStream_t s = static_cast<hipStream_t>(stream);
    rc = tokens >= kTiledRouterMinTokens ? launch_router_tiled(*layer, x, tokens, logits, shared_gate_out, nullptr, s)
                                         : launch_router(*layer, x, tokens, logits, shared_gate_out, nullptr, s);
    if (rc) return rc;
    return launch_topk(*layer, logits, tokens, ids, weights, nullptr, 0.0f, s);  // route(): no skipping
}


// The split plan's two expert sets are disjoint until the combine, so wl_moe_layer runs the MFMA experts on a
// second stream of the device beside the GEMV experts (64 tokens with Zipf(1.1) routing: 131 -> 100 us per layer):
// fork (an event on the caller's stream that the second stream waits for), the MFMA kernels on the second stream,
// join (an event there that the caller's stream waits for). Both chains are latency-bound and leave most of the
// GPU idle. The branch that waits for the fork and is waited for at the join starts and ends later than the
// caller's, so it gets the shorter chain: the MFMA experts with the K-split gate_up (at 64 tokens 96.0 -> 95.0 us
// per layer against the GEMV experts there). The stream and events are created on a device's first split call and
// kept; the whole fork-to-join sequence runs under one lock, so concurrent calls from several host threads stay
// correct (their MFMA work queues on the one second stream). Under graph capture the fork and join become graph
// edges. A fork scope (wl_moe_fork_begin / wl_moe_fork_end) forks and joins once for many calls on one stream, and
// the calls inside it hand their MFMA work over through workspace words (k_fork_wait, k_fork_store): two graph
// edges for a 40-layer step instead of two per layer, each pair costing ~10 us of the layer.
struct ForkStreams {
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    bool scope_open = false;
    hipStream_t scope = nullptr;  // the open scope's stream
};
constexpr int kForkDevices = 64;
static ForkStreams g_fork[kForkDevices];
static std::mutex g_fork_lock;
// fork-scope waits: polls (each after a short sleep) before giving up; WL_MOE_TEST_STARVE: the grouping does not
// publish itself and the second stream's wait gives up after kForkStarveSpin
constexpr uint32_t kForkSpin = 1u << 22, kForkStarveSpin = 1u << 11;

// This device's fork resources (created on first use), or nullptr with *rc set.
static ForkStreams* fork_streams(int* rc) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kForkDevices) {
        *rc = e != hipSuccess ? static_cast<int>(e) : WL_EINVAL_SHAPE;
        return nullptr;
    }
    ForkStreams& f = g_fork[dev];
    if (!f.side) {
        ForkStreams n;
        e = hipStreamCreateWithFlags(&n.side, hipStreamNonBlocking);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&n.fork, hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&n.join, hipEventDisableTiming);
        if (e != hipSuccess) {
            if (n.join) (void)hipEventDestroy(n.join);
            if (n.fork) (void)hipEventDestroy(n.fork);
            if (n.side) (void)hipStreamDestroy(n.side);
            *rc = static_cast<int>(e);
            return nullptr;
        }
        f = n;
    }
    *rc = WL_OK;
    return &f;
}

static int run_layer(const WlMoeLayer* layer, const float* x, int64_t tokens, float* y, int32_t* ids,
                     float* weights, void* workspace, size_t workspace_bytes, void* stream, void* const* events,
                     bool may_fork) {
    int rc = check_layer(layer);
    if (rc) return rc;
    if (!x || !y) return WL_EINVAL_NULL;
    if (tokens <= 0 || tokens > kMaxTokens) return WL_EINVAL_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(y) % 16) return WL_EINVAL_ALIGN;
    {  // y and x must not overlap: the fused kernel reads x in every workgroup while the owners write y
        const uintptr_t xb = reinterpret_cast<uintptr_t>(x), yb = reinterpret_cast<uintptr_t>(y);
        const uintptr_t n = static_cast<uintptr_t>(tokens) * static_cast<uintptr_t>(layer->hidden) * sizeof(float);
        if (xb < yb + n && yb < xb + n) return WL_EINVAL_OVERLAP;
    }
    const WlMoeLayer& L = *layer;
    const Workspace need = carve(L, tokens, nullptr);
    if (!workspace || workspace_bytes < need.bytes) return WL_EINVAL_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(workspace) % 256) return WL_EINVAL_ALIGN;
    Workspace w = carve(L, tokens, workspace);
    if (ids) w.ids = ids;
    if (weights) w.wts = weights;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool shared = L.shared_gate_up != nullptr;
    float* sg = (shared && L.shared_gate) ? w.sg : nullptr;
    auto record = [&](int i) {
        if (events) (void)hipEventRecord(static_cast<hipEvent_t>(events[i]), s);
    };
    if (fused_eligible(L, tokens)) {  // one launch: the whole layer (stage 0 of a profile holds it)
        record(0);
        rc = launch_fused(L, x, y, ids, weights, w, s);
        for (int i = 1; i <= kMoeStages; i++) record(i);
        return rc;
    }

    // stage boundaries for wl_moe_layer_profile: event i is recorded before stage i, event kMoeStages after the last
    auto mark = record;
    mark(0);
    const float* resid = (L.flags & WL_MOE_RESIDUAL) ? x : nullptr;
    if (L.flags & WL_MOE_PRE_NORM) {  // every stage below runs on the normalized input
        k_rms_norm<<<static_cast<unsigned>((tokens + 3) / 4), 256, 0, s>>>(x, L.norm_weight, L.norm_eps,
                                                                           static_cast<int>(tokens), L.hidden, w.xn);
        x = w.xn;
    }
    // an MFMA plan: the router also writes x as bf16 and the sort also writes the GEMM tile lists
    const ExpertPlan plan = expert_plan(L, tokens);
    const bool mfma = plan != kPlanGemv;
    const int gemv_max = plan_gemv_max(plan);
    // routed experts that may run on the GEMV kernels: each holds between 1 and gemv_max pairs
    const int64_t P = tokens * L.top_k;
    // the second stream is worth it while the experts average fewer than kForkMaxAvg tokens (at prefill sizes nearly
    // every expert is an MFMA expert, and the second stream's empty GEMV launches cost more than they overlap: 22.4
    // -> 22.7 ms per 4096-token chunk)
    constexpr int64_t kForkMaxAvg = 32;
    const bool few_gemv = plan == kPlanSplit && P >= kForkMaxAvg * L.n_experts;
    // with a split plan (and no stage events) the MFMA experts run on the device's second stream, in an open fork
    // scope on this stream handed over through the workspace's fork words, else forked and joined by events
    ForkStreams* fk = nullptr;
    bool in_scope = false;
    std::unique_lock<std::mutex> fork_guard;
    if (plan == kPlanSplit && may_fork && !events && !few_gemv) {
        fork_guard = std::unique_lock<std::mutex>(g_fork_lock);
        fk = fork_streams(&rc);
        if (!fk) return rc;
        in_scope = fk->scope_open && fk->scope == s;
    }
    const bool starve = (L.flags & WL_MOE_TEST_STARVE) != 0;
    if (router_parts(tokens)) {
        rc = launch_router_parts(L, x, tokens, w, mfma ? w.xb : nullptr, s);
        if (rc) return rc;
        mark(1);
        // the grouping in the same launch (mark 3 follows mark 2 at once)
        const GroupOut g{w.offsets, w.active, w.sorted, PickOut{w.crank, w.wts, w.picks},
                         TileOut{mfma ? w.tiles : nullptr, w.tiles_down, w.n_tiles, L.shared_gate_up ? 1 : 0, gemv_max},
                         w.sync, in_scope ? 1 : 0, starve ? 1 : 0};
        rc = launch_topk_parts(L, tokens, w, sg, &g, s);
        if (rc) return rc;
        mark(2);
    } else {
        rc = tokens >= kTiledRouterMinTokens
                 ? launch_router_tiled(L, x, tokens, w.logits, sg, mfma ? w.xb : nullptr, s)
                 : launch_router(L, x, tokens, w.logits, sg, mfma ? w.xb : nullptr, s);
        if (rc) return rc;
        mark(1);
        rc = launch_topk(L, w.logits, tokens, w.ids, w.wts, w.crank, L.min_expert_weight, s);
        if (rc) return rc;
        mark(2);
    }
    if (!router_parts(tokens)) {
        rc = launch_sort(L, w, w.ids, tokens, mfma, gemv_max, in_scope, starve, s);
        if (rc) return rc;
    }
    mark(3);
    const int max_gemv = plan == kPlanMfma ? 0 : static_cast<int>(P < L.n_experts ? P : L.n_experts);
    // the shared expert runs on the MFMA GEMMs in an MFMA plan (it sees every token), else on the GEMV kernels
    const ExpertArgs ga = gemv_args(L, x, tokens, w, max_gemv, shared && !mfma);
    // the GEMV launches' grid bound: at prefill sizes a GEMV expert is rare, and a grid sized for one per possible
    // expert costs ~4.5 us per launch to dispatch and retire empty; one workgroup per CU loops over whatever items
    // there are
    const int gemv_slots = few_gemv && max_gemv > 8 ? 8 : max_gemv;
    hipStream_t s_mfma = s;  // the MFMA experts' stream
    const uint32_t* skip = in_scope ? w.sync + kForkSkip : nullptr;
    if (fk) {
        s_mfma = fk->side;
        if (in_scope) {
            k_fork_wait<<<1, 64, 0, s_mfma>>>(w.sync, starve ? kForkStarveSpin : kForkSpin);
        } else {
            hipError_t e = hipEventRecord(fk->fork, s);
            if (e == hipSuccess) e = hipStreamWaitEvent(s_mfma, fk->fork, 0);
            if (e != hipSuccess) return static_cast<int>(e);
        }
    }
    if (mfma) {
        rc = launch_mfma_gate_up(L, tokens, w, gemv_max, plan == kPlanSplit, skip, s_mfma);
        if (rc) return rc;
    }
    launch_gemv_gate_up(L, ga, gemv_slots, shared && !mfma, s);
    rc = launch_status();
    if (rc) return rc;
    mark(4);
    if (mfma) {
        rc = launch_mfma_down(L, tokens, w, gemv_max, skip, s_mfma);
        if (rc) return rc;
    }
    launch_gemv_down(L, ga, gemv_slots, shared && !mfma, s);
    rc = launch_status();
    if (rc) return rc;
    if (in_scope) {  // the combine waits for kForkDone
        k_fork_store<<<1, 64, 0, s_mfma>>>(nullptr, 0u, w.sync + kForkDone, 1u);
        rc = launch_status();
        if (rc) return rc;
    } else if (fk) {  // join: the combine waits for the MFMA experts
        hipError_t e = hipEventRecord(fk->join, s_mfma);
        if (e == hipSuccess) e = hipStreamWaitEvent(s, fk->join, 0);
        if (e != hipSuccess) return static_cast<int>(e);
    }
    if (fork_guard.owns_lock()) fork_guard.unlock();
    if (in_scope) {  // the combine follows the MFMA experts' kForkDone (a one-thread gate on this stream)
        k_fork_gate<<<1, 64, 0, s>>>(w.sync, kForkSpin);
        rc = launch_status();
        if (rc) return rc;
    }
    const uint32_t* combine_status = in_scope ? w.sync + kStatusWord : nullptr;
    mark(5);
    const unsigned cgrid = static_cast<unsigned>(tokens * ((L.hidden + kCombineSpan - 1) / kCombineSpan));
    if (mfma)
        k_combine<uint16_t><<<cgrid, 256, 0, s>>>(static_cast<int>(tokens), L.hidden, L.top_k, w.picks, w.o,
                                                  shared ? reinterpret_cast<const uint16_t*>(w.o_sh) : nullptr, sg,
                                                  resid, y, combine_status);
    else
        k_combine<float><<<cgrid, 256, 0, s>>>(static_cast<int>(tokens), L.hidden, L.top_k, w.picks, w.o,
                                               shared ? w.o_sh : nullptr, sg, resid, y, combine_status);
    rc = launch_status();
    mark(6);
    return rc;
}


int wl_moe_layer(const WlMoeLayer* layer, const float* x, int64_t tokens, float* y, int32_t* ids, float* weights,
                 void* workspace, size_t workspace_bytes, void* stream) {
    return run_layer(layer, x, tokens, y, ids, weights, workspace, workspace_bytes, stream, nullptr, true);
}

int wl_moe_fork_begin(void* stream) {
    std::lock_guard<std::mutex> guard(g_fork_lock);
    int rc = WL_OK;
    ForkStreams* fk = fork_streams(&rc);
    if (!fk) return rc;
    if (fk->scope_open) return WL_EINVAL_SCOPE;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = hipEventRecord(fk->fork, s);
    if (e == hipSuccess) e = hipStreamWaitEvent(fk->side, fk->fork, 0);
    if (e != hipSuccess) return static_cast<int>(e);
    fk->scope_open = true;
    fk->scope = s;
    return WL_OK;
}

int wl_moe_fork_end(void* stream) {
    std::lock_guard<std::mutex> guard(g_fork_lock);
    int rc = WL_OK;
    ForkStreams* fk = fork_streams(&rc);
    if (!fk) return rc;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (!fk->scope_open || fk->scope != s) return WL_EINVAL_SCOPE;
    hipError_t e = hipEventRecord(fk->join, fk->side);
    if (e == hipSuccess) e = hipStreamWaitEvent(s, fk->join, 0);
    if (e != hipSuccess) return static_cast<int>(e);
    fk->scope_open = false;
    fk->scope = nullptr;
    return WL_OK;
}

int wl_moe_layer_profile(const WlMoeLayer* layer, const float* x, int64_t tokens, float* y, int32_t* ids,
                         float* weights, void* workspace, size_t workspace_bytes, void* stream,
                         void* const* events_host) {
    if (!events_host) return WL_EINVAL_NULL;
    for (int i = 0; i <= kMoeStages; i++)
        if (!events_host[i]) return WL_EINVAL_NULL;
    return run_layer(layer, x, tokens, y, ids, weights, workspace, workspace_bytes, stream, events_host, false);
}

int wl_moe_stage_count(void) { return kMoeStages; }

int wl_moe_plan(const WlMoeLayer* layer, int64_t tokens) {
    if (check_layer(layer) != WL_OK || tokens <= 0) return -1;
    if (fused_eligible(*layer, tokens)) return 1;
    return static_cast<int>(expert_plan(*layer, tokens));
}

int wl_moe_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
    if (!workspace) return WL_EINVAL_NULL;
    if (workspace_bytes < sizeof(uint32_t) * kSyncWords) return WL_EINVAL_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(workspace) % 256) return WL_EINVAL_ALIGN;
    return zero_sync(workspace, static_cast<hipStream_t>(stream));
}

const char* wl_moe_stage_name(int stage) {
    static const char* names[kMoeStages] = {"router", "topk", "sort", "gate_up", "down", "combine"};
    return stage >= 0 && stage < kMoeStages ? names[stage] : "";
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------------------------
// The no-allocation entry point: wl_moe_layer on a workspace that is a file-scope device array. Each GPU the
// library runs on holds its own copy of `scratch` (WL_NOALLOC_SCRATCH_BYTES) until the process ends. Host code never
// uses the array's name as a device address: on a call's first use of a device, with that device current,
// hipGetSymbolAddress gives this device's copy, which is kept per device and used for everything after, and the
// fused kernel's synchronization words at its start are zeroed there (a fill kernel on the caller's stream; the
// array is zero at load too). Calls keep those words consistent afterwards.
namespace wl {

static __device__ __attribute__((aligned(256))) uint8_t scratch[WL_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static void* g_scratch[kMaxDevices];  // this device's copy of `scratch`, once set up
static std::mutex g_scratch_lock;

// The current device's scratch address, set up on first use (hipGetSymbolAddress, then the sync words zeroed on
// `s`); nullptr with *rc set when that fails.
static void* scratch_address(hipStream_t s, int* rc) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        *rc = static_cast<int>(e);
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        *rc = WL_EINVAL_SHAPE;
        return nullptr;
    }
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            *rc = e != hipSuccess ? static_cast<int>(e) : WL_EINVAL_NULL;
            return nullptr;
        }
        const int z = zero_sync(ptr, s);
        if (z != WL_OK) {
            *rc = z;
            return nullptr;
        }
        g_scratch[dev] = ptr;
    }
    *rc = WL_OK;
    return g_scratch[dev];
}

}  // namespace wl

extern "C" int wl_moe_workspace_status(void* workspace, size_t workspace_bytes, void* stream) {
    using namespace wl;
    hipStream_t s = static_cast<hipStream_t>(stream);
    void* ws = workspace;
    if (!ws) {
        int rc = WL_OK;
        ws = scratch_address(s, &rc);
        if (!ws) return rc;
    } else {
        if (workspace_bytes < sizeof(uint32_t) * kSyncWords) return WL_EINVAL_WORKSPACE;
        if (reinterpret_cast<uintptr_t>(workspace) % 256) return WL_EINVAL_ALIGN;
    }
    uint32_t* word = static_cast<uint32_t*>(ws) + kStatusWord;
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return static_cast<int>(e);
    uint32_t v = 0;
    e = hipMemcpy(&v, word, sizeof(v), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return static_cast<int>(e);
    if (!v) return WL_OK;
    if (v & kStatusFork) {  // a fork-scope wait gave up: once the second stream has drained, its words start over
        e = hipDeviceSynchronize();
        if (e != hipSuccess) return static_cast<int>(e);
        uint32_t* base = static_cast<uint32_t*>(ws);
        for (const int i : {kForkSorted, kForkDone, kForkSkip}) {
            const int rz = zero_words(base + i, 1, s);
            if (rz) return rz;
        }
    }
    int rc = zero_words(word, 1, s);
    if (rc) return rc;
    e = hipStreamSynchronize(s);
    return e != hipSuccess ? static_cast<int>(e) : WL_ESYNC;
}

extern "C" int wl_moe_layer_noalloc(const WlMoeLayer* layer, const float* x, int64_t tokens, float* y,
                                    int32_t* ids, float* weights, void* stream) {
    using namespace wl;
    const int rc0 = check_layer(layer);
    if (rc0) return rc0;
    if (tokens <= 0 || tokens > kMaxTokens) return WL_EINVAL_SHAPE;
    if (carve(*layer, tokens, nullptr).bytes > WL_NOALLOC_SCRATCH_BYTES) return WL_EINVAL_SCRATCH;
    if (!x || !y) return WL_EINVAL_NULL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = WL_OK;
    void* ws = scratch_address(s, &rc);
    if (!ws) return rc;
    return run_layer(layer, x, tokens, y, ids, weights, ws, WL_NOALLOC_SCRATCH_BYTES, stream, nullptr, false);
}
