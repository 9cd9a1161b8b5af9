// Device functions shared by the multi-kernel MoE path (wl_moe.hip) and the fused decode kernel
// (wl_moe_fused.hip), so both compute bit-identical logits, routing, SwiGLU rows and down rows.
#pragma once

#include "wl_common.h"
#include "wl_moe.h"

namespace wl {

// One token's router logits for two rows at once: lanes [0, 32) work on row `row` of their half, lanes [32, 64)
// on the other half's row; each lane owns the 64-value segments s = slot, slot + 32, ... and chains fused
// multiply-adds over them in ascending k; the segment partials are then added left to right. Every lane of a
// half returns its row's sum (no bias). Call with the whole wavefront; `valid` may differ between the halves.
// x as stored, or scaled on load (RMSNorm): x4(i) returns the float4 of values 4 i .. 4 i + 3.
struct PlainX {
    const float* x;
    __device__ __forceinline__ float4 operator()(int i) const { return reinterpret_cast<const float4*>(x)[i]; }
};

// The RMSNorm of engines/base.py:27-31 (zero-centered: x * inv * (1 + w)) applied as x is loaded, in the fixed
// order the layer documents: inv from norm_inv, then each value rounded after each product. w may be NULL (0).
__device__ __forceinline__ float4 norm_apply(float4 v, bool has_w, float4 u, float inv) {
    float4 g = make_float4(1.f, 1.f, 1.f, 1.f);
    if (has_w) g = make_float4(__fadd_rn(1.f, u.x), __fadd_rn(1.f, u.y), __fadd_rn(1.f, u.z), __fadd_rn(1.f, u.w));
    return make_float4(__fmul_rn(__fmul_rn(v.x, inv), g.x), __fmul_rn(__fmul_rn(v.y, inv), g.y),
                       __fmul_rn(__fmul_rn(v.z, inv), g.z), __fmul_rn(__fmul_rn(v.w, inv), g.w));
}

struct NormX {
    const float* x;
    const float* w;
    float inv;
    __device__ __forceinline__ float4 operator()(int i) const {
        const float4 v = reinterpret_cast<const float4*>(x)[i];
        const float4 u = w ? reinterpret_cast<const float4*>(w)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        return norm_apply(v, w != nullptr, u, inv);
    }
};

// A router row's weights for router_row_xw: float4 i of 64-value segment s.
struct GlobalRow {
    const float* w;
    __device__ __forceinline__ float4 operator()(int s, int i) const {
        return reinterpret_cast<const float4*>(w + s * kRouterSeg)[i];
    }
};

template <typename XF, typename WF>
__device__ __forceinline__ float router_row_xw(XF x4, WF w4, bool valid, int H, int lane);

template <typename XF>
__device__ __forceinline__ float router_row_x(XF x4, const float* __restrict__ wr, bool valid, int H, int lane) {
    return router_row_xw(x4, GlobalRow{wr}, valid, H, lane);
}

__device__ __forceinline__ float router_row(const float* __restrict__ x, const float* __restrict__ wr, bool valid,
                                            int H, int lane) {
    return router_row_x(PlainX{x}, wr, valid, H, lane);
}

// 1 / sqrt(s / H + eps), each step correctly rounded once (the norm's scale from the sum of squares s). The square
// root is __builtin_sqrtf (llvm.sqrt.f32, expanded to a correctly rounded sequence since HIP builds keep fp32
// division and square root correctly rounded by default); HIP's __fsqrt_rn maps to the native v_sqrt_f32, which is
// not, and differs from a correctly rounded root in the last bit for about a third of inputs.
__device__ __forceinline__ float norm_inv(float s, int H, float eps) {
    return __fdiv_rn(1.0f, __builtin_sqrtf(__fadd_rn(__fdiv_rn(s, static_cast<float>(H)), eps)));
}

template <typename XF, typename WF>
__device__ __forceinline__ float router_row_xw(XF x4, WF w4, bool valid, int H, int lane) {
    const int slot = lane & 31, src_base = lane & 32;
    const int nseg = H / kRouterSeg;
    float total = 0.0f;
    // one round per 32 segments (a single round up to H = 2048), kept as a loop so the body is emitted once
#pragma unroll 1
    for (int j = 0; 32 * j < nseg; j++) {
        float p = 0.0f;
        const int s = slot + 32 * j;
        if (valid && s < nseg) {
            // the segment's x requested before the chain starts (all 16 loads in flight; interleaved with the
            // chain by the scheduler, two were, and each group of four FMAs waited out a load)
            float4 xs[kRouterSeg / 4];
#pragma unroll
            for (int i = 0; i < kRouterSeg / 4; i++) xs[i] = x4(s * (kRouterSeg / 4) + i);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < kRouterSeg / 4; i++) {
                const float4 wv = w4(s, i), xv = xs[i];
                p = __builtin_fmaf(xv.x, wv.x, p);
                p = __builtin_fmaf(xv.y, wv.y, p);
                p = __builtin_fmaf(xv.z, wv.z, p);
                p = __builtin_fmaf(xv.w, wv.w, p);
            }
        }
        // gather the half's 32 partials first (independent shuffles), then add them in segment order
        float parts[32];
#pragma unroll
        for (int sl = 0; sl < 32; sl++) parts[sl] = __shfl(p, src_base + sl);
        // every shuffle issued before the first add (left to the scheduler, each add waited for its shuffle with
        // two more in flight: 32 LDS round trips a third at a time)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int sl = 0; sl < 32; sl++) {
            const int sg = sl + 32 * j;
            if (sg < nseg) total = sg == 0 ? parts[sl] : __fadd_rn(total, parts[sl]);
        }
    }
    return total;
}

// the number of lanes below this one whose bit is set in the wavefront mask m (v_mbcnt_lo / v_mbcnt_hi)
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                      __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u)));
}

// float -> uint32 with the same order (larger float, larger key)
__device__ __forceinline__ uint32_t order_key(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Top-k of one token's logits (lt[0..E), E <= 64*EJ), one wavefront. Softmax over all E in fp32; the selection is
// on the logits (softmax is monotone): largest first, ties to the lower expert id, NaN ranked as -inf. Lane r < k
// returns the r-th pick: its expert id, its weight exp(l - max) / sum (divided by the sum of the k picks' weights,
// added in pick order, when renorm), and id_rank = its position among the k ids in ascending order.
// The k-th largest key is found by a bitwise radix select over ballots (32 steps, no cross-lane latency chain);
// the k picks are then compacted and ranked through `scratch` (64 words of LDS owned by this wavefront).
// scratch must point to LDS. It is not volatile (volatile accesses keep the generic address space and become flat
// instructions, each waiting on two counters); lane_sync orders the writes of one lane before the reads of another:
// a wavefront's LDS instructions complete in issue order, so only the compiler has to be kept from moving them.
__device__ __forceinline__ void lane_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The softmax statistics of one token's logits lt[0..E) (one wavefront, EJ logits per lane: lane + 64 j): the
// logits with NaN as -inf, their max m and the sum s of exp(l - m) (per lane in j order, then across the wave).
template <int EJ>
__device__ __forceinline__ void softmax_stats(const float* __restrict__ lt, int E, int lane, float (&v)[EJ],
                                              bool (&valid)[EJ], float& m, float& s) {
    m = -INFINITY;
#pragma unroll
    for (int j = 0; j < EJ; j++) {
        const int idx = lane + 64 * j;
        valid[j] = idx < E;
        const float lv = valid[j] ? lt[idx] : -INFINITY;
        v[j] = lv == lv ? lv : -INFINITY;
        m = fmaxf(m, v[j]);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    s = 0.0f;
#pragma unroll
    for (int j = 0; j < EJ; j++)
        if (valid[j]) s += expf(v[j] - m);
    s = group_sum<64>(s);
}

// softmax_stats' sum s for a known max m (bitwise the same: per lane in j order, then across the wave).
template <int EJ>
__device__ __forceinline__ float softmax_sum(const float* __restrict__ lt, int E, int lane, float m) {
    float lv[EJ];  // every read issued before the first use (read under the branch, each waited out its own)
#pragma unroll
    for (int j = 0; j < EJ; j++) lv[j] = lt[lane + 64 * j < E ? lane + 64 * j : 0];
    __builtin_amdgcn_sched_barrier(0);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < EJ; j++)
        if (lane + 64 * j < E) s += expf((lv[j] == lv[j] ? lv[j] : -INFINITY) - m);
    return group_sum<64>(s);
}

// The routing weight of pick r = lane (< k; my_v its logit): exp(l - m) / s, divided by the sum of the k picks'
// weights added in pick order when renorm. Call with the whole wavefront.
__device__ __forceinline__ float pick_weight(float my_v, float m, float s, int k, bool renorm, int lane) {
    const float p = lane < k ? expf(my_v - m) / s : 0.0f;
    float wsum = 0.0f;
    // 8 picks' readlanes at a time (independent), added in pick order
    for (int r0 = 0; r0 < k; r0 += 8) {
        float pr[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            pr[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), (r0 + i) & 63));
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (r0 + i < k) wsum = r0 + i == 0 ? pr[i] : wsum + pr[i];
    }
    return renorm ? p / wsum : p;
}

// Engine.skip_small_experts (engines/base.py:413-430) on one token's picks, lane r < k holding pick r (largest
// weight first) with weight w and expert id: a pick is kept when its weight is at least min_w, and pick 0 always;
// the kept weights are scaled by S / K, S the sum of the k weights and K of the kept ones (each added in pick
// order); a dropped pick gets id -1 and weight 0. Returns whether lane's pick is kept. Call with the whole
// wavefront; min_w > 0.
__device__ __forceinline__ bool skip_small(float& w, int& id, int k, float min_w, int lane) {
    const bool keep = lane < k && (lane == 0 || w >= min_w);
    const float kw = keep ? w : 0.0f;
    float S = 0.0f, K = 0.0f;
    for (int r0 = 0; r0 < k; r0 += 8) {
        float pr[8], kr[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            pr[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), (r0 + i) & 63));
            kr[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, kw), (r0 + i) & 63));
        }
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (r0 + i < k) {
                S = r0 + i == 0 ? pr[i] : S + pr[i];
                K = r0 + i == 0 ? kr[i] : K + kr[i];
            }
    }
    const float scale = S / K;
    if (lane < k) {
        if (keep) {
            w = w * scale;
        } else {
            w = 0.0f;
            id = -1;
        }
    }
    return keep;
}

// max(v, the value of the lane DPP control CTRL selects) on unsigned 32-bit values, every lane sourcing
__device__ __forceinline__ int umax_dpp_impl(int v, int o) {
    return static_cast<int>(max(static_cast<uint32_t>(v), static_cast<uint32_t>(o)));
}
template <int CTRL>
__device__ __forceinline__ int umax_dpp(int v) {
    return umax_dpp_impl(v, __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false));
}

template <int EJ>
__device__ __forceinline__ void wave_topk(const float* __restrict__ lt, int E, int k, bool renorm,
                                          uint32_t* scratch, int lane, int& out_id, float& out_w,
                                          int& out_id_rank) {
    float v[EJ];
    bool valid[EJ];
    float m, s;
    softmax_stats<EJ>(lt, E, lane, v, valid, m, s);
    uint32_t key[EJ];
#pragma unroll
    for (int j = 0; j < EJ; j++) key[j] = order_key(v[j]);

    // K = the largest key with at least k keys >= K. The EJ ballots of a step are independent (counted after all
    // are taken); once exactly k keys are >= a candidate the selected set is decided and the search stops.
    uint32_t K = 0;
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = K | (1u << bit);
        uint64_t bal[EJ];
#pragma unroll
        for (int j = 0; j < EJ; j++) bal[j] = __ballot(valid[j] && key[j] >= cand);
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < EJ; j++) cnt += __popcll(bal[j]);
        if (cnt >= k) {
            K = cand;
            if (cnt == k) break;
        }
    }
    int n_gt = 0;
#pragma unroll
    for (int j = 0; j < EJ; j++) n_gt += __popcll(__ballot(valid[j] && key[j] > K));
    const int need = k - n_gt;
    const uint64_t below = __lanemask_lt();
    int ties_before = 0, picked_before = 0;
#pragma unroll
    for (int j = 0; j < EJ; j++) {
        const uint64_t eq = __ballot(valid[j] && key[j] == K);
        const bool tie = valid[j] && key[j] == K;
        const int my_tie = ties_before + __popcll(eq & below);
        const bool sel = valid[j] && (key[j] > K || (tie && my_tie < need));
        const uint64_t sm = __ballot(sel);
        if (sel) {
            const int c = picked_before + __popcll(sm & below);
            scratch[2 * c] = __builtin_bit_cast(uint32_t, v[j]);
            scratch[2 * c + 1] = static_cast<uint32_t>(lane + 64 * j);
        }
        ties_before += __popcll(eq);
        picked_before += __popcll(sm);
    }
    lane_sync();
    // lane r < k ranks compacted pick r among the k (descending value, ties to the lower id) and by id, and puts
    // it at its descending position in the second half of scratch (id in bits 0..15, id rank in 16..31)
    if (lane < k) {
        const uint2 mine = make_uint2(scratch[2 * lane], scratch[2 * lane + 1]);
        const uint32_t mk = order_key(__builtin_bit_cast(float, mine.x));
        int desc = 0, id_rank = 0;
        for (int q = 0; q < k; q++) {
            const uint2 o = make_uint2(scratch[2 * q], scratch[2 * q + 1]);
            const uint32_t ok = order_key(__builtin_bit_cast(float, o.x));
            desc += (ok > mk || (ok == mk && o.y < mine.y)) ? 1 : 0;
            id_rank += o.y < mine.y ? 1 : 0;
        }
        scratch[32 + 2 * desc] = mine.x;
        scratch[32 + 2 * desc + 1] = mine.y | (static_cast<uint32_t>(id_rank) << 16);
    }
    lane_sync();
    int my_id = 0;
    float my_v = -INFINITY;
    out_id_rank = 0;
    if (lane < k) {
        const uint2 r = make_uint2(scratch[32 + 2 * lane], scratch[32 + 2 * lane + 1]);
        my_v = __builtin_bit_cast(float, r.x);
        my_id = static_cast<int>(r.y & 0xFFFFu);
        out_id_rank = static_cast<int>(r.y >> 16);
    }
    out_id = my_id;
    out_w = pick_weight(my_v, m, s, k, renorm, lane);
}

// The ids of k of the largest values in v (lane l holds values l + 64 j, j < EJ, as order keys; 0 = no value),
// written to out[r] for r < k in descending order of value (one wavefront, 1 <= k <= the number of values).
// k rounds of a wave maximum (DPP within rows, then the row maxima); in each, the lowest lane holding the maximum
// gives up one value holding it. Equal values are taken in an unspecified order: for a guess, not a routing.
template <int EJ>
__device__ __forceinline__ void select_top_keys(uint32_t (&key)[EJ], int k, int lane, int* out) {
    for (int r = 0; r < k; r++) {
        uint32_t m = key[0];
#pragma unroll
        for (int j = 1; j < EJ; j++) m = max(m, key[j]);
        int u = static_cast<int>(m);
        u = umax_dpp<0xB1>(u);   // quad_perm [1,0,3,2]
        u = umax_dpp<0x4E>(u);   // quad_perm [2,3,0,1]
        u = umax_dpp<0x141>(u);  // row_half_mirror
        u = umax_dpp<0x140>(u);  // row_mirror: every lane holds its row's maximum
        const uint32_t M = max(max(static_cast<uint32_t>(__builtin_amdgcn_readlane(u, 0)),
                                   static_cast<uint32_t>(__builtin_amdgcn_readlane(u, 16))),
                               max(static_cast<uint32_t>(__builtin_amdgcn_readlane(u, 32)),
                                   static_cast<uint32_t>(__builtin_amdgcn_readlane(u, 48))));
        const int owner = __builtin_ctzll(__ballot(m == M));
        if (lane == owner) {
            int jj = 0;
#pragma unroll
            for (int j = EJ - 1; j >= 0; j--)
                if (key[j] == M) jj = j;
            out[r] = lane + 64 * jj;
#pragma unroll
            for (int j = 0; j < EJ; j++)
                if (j == jj) key[j] = 0;
        }
    }
}

// One intermediate row j of a fused [gate | up] matrix (gate row j, up row inter + j) times one token x, one
// wavefront; every lane returns the two sums.
template <int TYPE>
__device__ __forceinline__ void gate_up_row(const uint8_t* __restrict__ w, int j, int inter, int H,
                                            const float* __restrict__ x, int lane, float& g, float& u) {
    const int gi = lane >> 3, c = lane & 7;
    const int nb = H / kQK;
    const int64_t rs = static_cast<int64_t>(nb) * BlockInfo<TYPE>::bytes;
    const uint8_t* wg = w + static_cast<int64_t>(j) * rs;
    const uint8_t* wu = w + static_cast<int64_t>(inter + j) * rs;
    const int lo_start = BlockInfo<TYPE>::lo_start(c), hi_off = BlockInfo<TYPE>::hi_offset;
    float ag = 0.0f, au = 0.0f;
    for (int kb = gi; kb < nb; kb += 8) {
        Lane32 lg, lu;
        decode<TYPE>(wg + static_cast<int64_t>(kb) * BlockInfo<TYPE>::bytes, c, lg);
        decode<TYPE>(wu + static_cast<int64_t>(kb) * BlockInfo<TYPE>::bytes, c, lu);
        const float* xt = x + kb * kQK + lo_start;
        float4 xl[4], xh[4];
        load_run(xt, xl);
        load_run(xt + hi_off, xh);
        const float sxl = sum16(xl), sxh = sum16(xh);
        ag += lane_dot_s(lg, xl, xh, sxl, sxh);
        au += lane_dot_s(lu, xl, xh, sxl, sxh);
    }
    g = group_sum<64>(ag);
    u = group_sum<64>(au);
}

typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats -> two bf16 (round to nearest even, like Tensor.to(torch.bfloat16)) in one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(floatx2{a, b}, bf16x2));
}

}  // namespace wl
