// Fused decode: the whole MoE layer for one token in ONE kernel launch (vs. router / top-k / grouping / gate_up /
// down / combine as six launches), which is what bounds batch-1 decode: every launch costs microseconds while a
// layer moves only ~20 MB.
//
// A persistent grid of G workgroups (one per CU, 8 wavefronts each) in two roles:
//   gate_up workgroups  A: the router's logits (2 rows per wavefront task) and the shared expert's gate_up rows,
//                          neither of which depends on the routing;
//                       then: the routing (wave_topk over the logits, once all have arrived), then the picked
//                          experts' gate_up rows into h, several rows per wavefront, all fetched before any is
//                          computed. Then they exit.
//   down workgroups     fetch the shared expert's down rows, wait for the logits, route, fetch the picked
//                          experts' down rows into registers, wait for h_shared (shared expert's SwiGLU output)
//                          and dot it, wait for h, then write y = sum_e w_e (down_e h_e) + sg * shared_down h_sh,
//                          experts in ascending id. R output rows per wavefront.
// The arithmetic (router_row, wave_topk, the gate_up and down dot products, the combine order) is the multi-kernel
// path's.
//
// No barriers: every value that crosses workgroups (logits, h_shared, h) is a 64-bit word (tag << 32 | bits)
// written and read with relaxed device-scope atomics (single-copy atomic, bypassing the per-XCD L2s). The tag is
// this call's epoch, so a consumer polls the data itself until every word it needs carries the current tag.
// Each workgroup keeps its own epoch counter (one 128-byte line each, incremented as it exits), so all agree on
// the epoch without communicating and nothing is ever reset. Every wait is bounded (kSpinLimit polls): a
// workgroup that gives up writes NaN instead of hanging.
#include <hip/hip_runtime.h>

#include "wl_common.h"
#include "wl_host.h"
#include "wl_moe.h"
#include "wl_moe_dev.h"

namespace wl {

constexpr int kFusedThreads = 512;
constexpr int kFusedWaves = kFusedThreads / 64;
constexpr int kGateUpTasks = 4;  // gate_up rows a wavefront fetches before computing
constexpr uint32_t kSpinLimit = 1u << 20;

struct FusedArgs {
    const uint8_t* gate_up;
    int64_t gate_up_stride;
    const uint8_t* down;
    int64_t down_stride;
    const float* router;
    const float* router_bias;
    const uint8_t* sh_gate_up;
    const uint8_t* sh_down;
    const float* sh_gate;
    const float* x;
    float* y;
    int32_t* ids_out;
    float* wts_out;
    uint32_t* sync;  // kSyncWords: epochs, then tagged logits [E+1], h_shared [I], h [k, I]
    int H, I, E, k, renorm, G;
};

__device__ __forceinline__ void put_tagged(uint32_t* sync_base, int word, uint32_t tag, float v) {
    const uint64_t w = (static_cast<uint64_t>(tag) << 32) | __builtin_bit_cast(uint32_t, v);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(sync_base + word), w, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Copies the n tagged words at src into lds once every one carries `tag` (workgroup-cooperative); false if
// kSpinLimit polls pass first. n <= 32 * blockDim.x.
__device__ __forceinline__ bool gather_tagged(const uint32_t* src, int n, uint32_t tag, float* lds) {
    const uint64_t* p = reinterpret_cast<const uint64_t*>(src);
    uint32_t pending = 0;
    for (int q = 0; q < 32 && static_cast<int>(threadIdx.x) + q * static_cast<int>(blockDim.x) < n; q++)
        pending |= 1u << q;
    for (uint32_t spins = 0;; spins++) {
        uint32_t m = pending;
        while (m) {
            const int q = __builtin_ctz(m);
            m &= m - 1;
            const int i = threadIdx.x + q * blockDim.x;
            const uint64_t w = __hip_atomic_load(const_cast<uint64_t*>(p + i), __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
            if (static_cast<uint32_t>(w >> 32) == tag) {
                lds[i] = __builtin_bit_cast(float, static_cast<uint32_t>(w));
                pending &= ~(1u << q);
            }
        }
        if (__syncthreads_and(pending == 0)) return true;
        if (spins >= kSpinLimit) return false;
        __builtin_amdgcn_s_sleep(1);
    }
}

template <int GU, int DN, int EJ, int NBD>
__global__ __launch_bounds__(kFusedThreads) void k_moe_decode(FusedArgs a) {
    constexpr int R = 8 / NBD, WIDTH = 8 * NBD;
    __shared__ float lds_h[kFusedMaxK * kFusedMaxInter];
    __shared__ float lds_hsh[kFusedMaxInter];
    __shared__ float lds_logits[kFusedMaxE + 1];
    __shared__ int lds_sel[kFusedMaxK];
    __shared__ float lds_wsel[kFusedMaxK];
    __shared__ uint32_t tk_scratch[64];
    __shared__ uint32_t lds_epoch;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int G = a.G;
    const int H = a.H, I = a.I, E = a.E, k = a.k;
    const bool shared = a.sh_gate_up != nullptr;
    const bool sh_gate = shared && a.sh_gate != nullptr;
    const int n_logits = E + (sh_gate ? 1 : 0);
    const int gi = lane >> 3, c = lane & 7;
    const int ND = H / R;                                    // down wavefronts
    const int NDW = (ND + kFusedWaves - 1) / kFusedWaves;    // down workgroups: blocks [0, NDW)
    const bool down_wg = static_cast<int>(blockIdx.x) < NDW;
    uint32_t* epoch_word = a.sync + kFlagStride * blockIdx.x;

    if (threadIdx.x == 0) lds_epoch = __hip_atomic_load(epoch_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const uint32_t tag = lds_epoch + 1u;
    bool ok = true;

    // The routing from the logits, by wavefront 0; every wavefront reads it from LDS afterwards.
    auto route = [&]() {
        ok = gather_tagged(a.sync + kTagLogits, n_logits, tag, lds_logits) && ok;
        if (wv == 0) {
            int my_id, my_rank;
            float my_w;
            wave_topk<EJ>(lds_logits, E, k, a.renorm != 0, tk_scratch, lane, my_id, my_w, my_rank);
            if (lane < k) {
                lds_sel[my_rank] = my_id;
                lds_wsel[my_rank] = my_w;
                if (blockIdx.x == 0) {
                    if (a.ids_out) a.ids_out[lane] = my_id;
                    if (a.wts_out) a.wts_out[lane] = my_w;
                }
            }
        }
        __syncthreads();
    };

    if (down_wg) {
        const int d = blockIdx.x * kFusedWaves + wv;
        const bool dwave = d < ND;
        const int row = d * R + gi / NBD, kb = gi % NBD;
        constexpr int64_t dn_rs = static_cast<int64_t>(NBD) * BlockInfo<DN>::bytes;
        const int lo = kb * kQK + BlockInfo<DN>::lo_start(c), hi = lo + BlockInfo<DN>::hi_offset;
        Lane32 shl;
        if (shared && dwave) decode<DN>(a.sh_down + row * dn_rs + kb * BlockInfo<DN>::bytes, c, shl);
        route();
        Lane32 pre[kFusedMaxK];
        float wsel[kFusedMaxK];
#pragma unroll
        for (int s = 0; s < kFusedMaxK; s++) {
            wsel[s] = lds_wsel[s];
            if (s < k && dwave)
                decode<DN>(a.down + static_cast<int64_t>(lds_sel[s]) * a.down_stride + row * dn_rs +
                               kb * BlockInfo<DN>::bytes, c, pre[s]);
        }
        float sh_dot = 0.0f, sgv = 1.0f;
        if (shared) {
            ok = gather_tagged(a.sync + kTagHsh, I, tag, lds_hsh) && ok;
            if (sh_gate) sgv = sigmoid(lds_logits[E]);
            if (dwave) {
                float4 hl[4], hh[4];
                load_run(lds_hsh + lo, hl);
                load_run(lds_hsh + hi, hh);
                sh_dot = group_sum<WIDTH>(lane_dot(shl, hl, hh));
            }
        }
        ok = gather_tagged(a.sync + kTagH, k * I, tag, lds_h) && ok;
        if (dwave) {
            float acc = 0.0f;
#pragma unroll
            for (int s = 0; s < kFusedMaxK; s++) {
                if (s < k) {
                    float4 hl[4], hh[4];
                    load_run(lds_h + s * I + lo, hl);
                    load_run(lds_h + s * I + hi, hh);
                    const float dv = group_sum<WIDTH>(lane_dot(pre[s], hl, hh));
                    acc = s == 0 ? wsel[s] * dv : acc + wsel[s] * dv;
                }
            }
            if (shared) acc = acc + sgv * sh_dot;
            if ((lane & (WIDTH - 1)) == 0) a.y[row] = ok ? acc : __builtin_nanf("");
        }
    } else {
        const int NG = G - NDW;
        const int gslot = wv * NG + (static_cast<int>(blockIdx.x) - NDW);  // consecutive slots on different CUs
        const int NWg = NG * kFusedWaves;
        const int nb = H / kQK;  // <= 8: one gate/up block per lane group
        const bool gu_lane = gi < nb;
        const int lo_gu = gi * kQK + BlockInfo<GU>::lo_start(c), hi_gu = lo_gu + BlockInfo<GU>::hi_offset;
        const int64_t gu_rs = static_cast<int64_t>(nb) * BlockInfo<GU>::bytes;
        float4 xl[4], xh[4];
        float sxl = 0.0f, sxh = 0.0f;
        if (gu_lane) {
            load_run(a.x + lo_gu, xl);
            load_run(a.x + hi_gu, xh);
            sxl = sum16(xl);
            sxh = sum16(xh);
        }
        auto gate_up_dots = [&](const Lane32& lg, const Lane32& lu, float& g, float& u) {
            float ag = 0.0f, au = 0.0f;
            if (gu_lane) {
                ag = lane_dot_s(lg, xl, xh, sxl, sxh);
                au = lane_dot_s(lu, xl, xh, sxl, sxh);
            }
            g = group_sum<64>(ag);
            u = group_sum<64>(au);
        };
        // phase A: router rows, shared gate_up rows
        const int n_router = (n_logits + 1) / 2;
        const int n_a = n_router + (shared ? I : 0);
        for (int t = gslot; t < n_a; t += NWg) {
            if (t < n_router) {
                const int row = 2 * t + (lane >> 5);
                const bool valid = row < n_logits;
                const float* wr = row < E ? a.router + static_cast<int64_t>(row) * H : a.sh_gate;
                const float total = router_row(a.x, wr, valid, H, lane);
                if ((lane & 31) == 0 && valid)
                    put_tagged(a.sync + kTagLogits, 2 * row, tag,
                               (row < E && a.router_bias) ? __fadd_rn(total, a.router_bias[row]) : total);
            } else {
                const int j = t - n_router;
                Lane32 lg, lu;
                if (gu_lane) {
                    decode<GU>(a.sh_gate_up + j * gu_rs + gi * BlockInfo<GU>::bytes, c, lg);
                    decode<GU>(a.sh_gate_up + (I + j) * gu_rs + gi * BlockInfo<GU>::bytes, c, lu);
                }
                float g, u;
                gate_up_dots(lg, lu, g, u);
                if (lane == 0) put_tagged(a.sync + kTagHsh, 2 * j, tag, silu(g) * u);
            }
        }
        route();
        int sel[kFusedMaxK];
#pragma unroll
        for (int s = 0; s < kFusedMaxK; s++) sel[s] = lds_sel[s];
        for (int u0 = gslot; u0 < k * I; u0 += NWg * kGateUpTasks) {
            Lane32 lg[kGateUpTasks], lu[kGateUpTasks];
#pragma unroll
            for (int q = 0; q < kGateUpTasks; q++) {
                const int u = u0 + q * NWg;
                if (u < k * I && gu_lane) {
                    const int s = u / I, j = u - s * I;
                    int e = 0;
#pragma unroll
                    for (int r = 0; r < kFusedMaxK; r++)
                        if (r == s) e = sel[r];
                    const uint8_t* w = a.gate_up + static_cast<int64_t>(e) * a.gate_up_stride;
                    decode<GU>(w + j * gu_rs + gi * BlockInfo<GU>::bytes, c, lg[q]);
                    decode<GU>(w + (I + j) * gu_rs + gi * BlockInfo<GU>::bytes, c, lu[q]);
                }
            }
#pragma unroll
            for (int q = 0; q < kGateUpTasks; q++) {
                const int u = u0 + q * NWg;
                if (u < k * I) {
                    float g, up;
                    gate_up_dots(lg[q], lu[q], g, up);
                    if (lane == 0) put_tagged(a.sync + kTagH, 2 * u, tag, silu(g) * up);  // u = s * I + j
                }
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(epoch_word, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void k_zero_words(uint32_t* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// ---------------------------------------------------------------------------------------------------------------

template <int GU, int DN, int EJ, int NBD>
static hipError_t launch_fused_t(const FusedArgs& a, hipStream_t s) {
    k_moe_decode<GU, DN, EJ, NBD><<<a.G, kFusedThreads, 0, s>>>(a);
    return hipGetLastError();
}

template <int GU, int DN, int EJ>
static hipError_t launch_fused_nbd(const FusedArgs& a, hipStream_t s) {
    switch (a.I / kQK) {
        case 1: return launch_fused_t<GU, DN, EJ, 1>(a, s);
        case 2: return launch_fused_t<GU, DN, EJ, 2>(a, s);
        default: return launch_fused_t<GU, DN, EJ, 4>(a, s);
    }
}

template <int GU, int DN>
static hipError_t launch_fused_ej(const FusedArgs& a, hipStream_t s) {
    if (a.E <= 64) return launch_fused_nbd<GU, DN, 1>(a, s);
    if (a.E <= 128) return launch_fused_nbd<GU, DN, 2>(a, s);
    return launch_fused_nbd<GU, DN, 4>(a, s);
}

// Workgroups of the persistent grid: one per CU of the current device (cached per device); 0 when the kernel
// cannot keep one workgroup per CU resident.
static int fused_grid() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (!cached[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_cu, reinterpret_cast<const void*>(&k_moe_decode<WL_TYPE_Q4_K, WL_TYPE_Q6_K, 4, 2>),
                kFusedThreads, 0) != hipSuccess || per_cu < 1)
            return 0;
        cached[dev] = cus < kFusedMaxG ? cus : kFusedMaxG;
    }
    return cached[dev];
}

bool fused_eligible(const WlMoeLayer& L, int64_t T) {
    if ((L.flags & WL_MOE_NO_FUSED) || T != 1 || L.n_experts > kFusedMaxE || L.top_k > kFusedMaxK) return false;
    if (L.gate_up_type != WL_TYPE_Q4_K || L.hidden > 8 * kQK) return false;
    const int nbd = L.inter / kQK;
    if (nbd != 1 && nbd != 2 && nbd != 4) return false;
    if (L.shared_gate_up && (L.shared_inter != L.inter || L.shared_gate_up_type != L.gate_up_type ||
                             L.shared_down_type != L.down_type))
        return false;
    const int G = fused_grid();
    if (G < 2) return false;
    const int down_waves = L.hidden / (8 / nbd);
    const int down_wgs = (down_waves + kFusedWaves - 1) / kFusedWaves;
    return down_wgs <= G / 2;  // leaves at least half the workgroups for the router and gate_up work
}

int launch_fused(const WlMoeLayer& L, const float* x, float* y, int32_t* ids, float* wts, const Workspace& w,
                 hipStream_t s) {
    FusedArgs a{};
    a.gate_up = static_cast<const uint8_t*>(L.gate_up);
    a.gate_up_stride = L.gate_up_stride;
    a.down = static_cast<const uint8_t*>(L.down);
    a.down_stride = L.down_stride;
    a.router = L.router;
    a.router_bias = L.router_bias;
    a.sh_gate_up = static_cast<const uint8_t*>(L.shared_gate_up);
    a.sh_down = static_cast<const uint8_t*>(L.shared_down);
    a.sh_gate = L.shared_gate_up ? L.shared_gate : nullptr;
    a.x = x;
    a.y = y;
    a.ids_out = ids;
    a.wts_out = wts;
    a.sync = w.sync;
    a.H = L.hidden;
    a.I = L.inter;
    a.E = L.n_experts;
    a.k = L.top_k;
    a.renorm = L.norm_topk_prob ? 1 : 0;
    a.G = fused_grid();
    hipError_t e = L.down_type == WL_TYPE_Q4_K ? launch_fused_ej<WL_TYPE_Q4_K, WL_TYPE_Q4_K>(a, s)
                                               : launch_fused_ej<WL_TYPE_Q4_K, WL_TYPE_Q6_K>(a, s);
    return e == hipSuccess ? WL_OK : static_cast<int>(e);
}

int zero_sync(void* workspace, hipStream_t s) {
    k_zero_words<<<32, 256, 0, s>>>(static_cast<uint32_t*>(workspace), kSyncWords);
    return launch_status();
}

}  // namespace wl
