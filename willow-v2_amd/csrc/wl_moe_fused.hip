// Fused decode: the whole MoE layer for one token in ONE kernel launch (vs. router / top-k / grouping / gate_up /
// down / combine as six launches), which is what bounds batch-1 decode: every launch costs microseconds while a
// layer moves only ~20 MB.
//
// A persistent grid of G workgroups (one per CU, 8 wavefronts each) runs three phases separated by two grid
// barriers:
//   A  router logits (2 rows per task) and the shared expert's gate_up rows (independent of the routing)
//   -- barrier 1: the master workgroup (block 0) waits for everyone, computes the top-k once (wave_topk) and
//      publishes the routing with the release --
//   B  the first H/R wavefront slots ("down waves", R output rows each) fetch the down rows of the k picked experts
//      into registers and compute the shared expert's down rows; the other wavefronts compute the picked experts'
//      gate_up rows into h (several rows per wavefront, all fetched before any is computed)
//   -- barrier 2 --
//   C  every workgroup copies h into LDS; down waves dot their prefetched rows with it and write
//      y = sum_e w_e (down_e h_e) + sg * shared, experts in ascending id
// The arithmetic (router_row, wave_topk, the gate_up and down dot products, the combine order) is the multi-kernel
// path's.
//
// Synchronization without cache maintenance: the values that cross workgroups (logits, routing, h) are written and
// read with relaxed device-scope atomics, which bypass the per-XCD L2s; a thread drains its outstanding memory
// operations (s_waitcnt 0) before it raises a flag. The barrier is a flag per workgroup, each in its own 128-byte
// line, holding the count of barriers it has passed (monotonic across calls, so nothing is ever reset): a workgroup
// raises its flag to the target, the master polls all flags, then writes the target into the release word the
// others poll. Every wait is bounded (kSpinLimit polls): a workgroup that gives up writes NaN instead of hanging.
#include <hip/hip_runtime.h>

#include "wl_common.h"
#include "wl_host.h"
#include "wl_moe.h"
#include "wl_moe_dev.h"

namespace wl {

constexpr int kFusedThreads = 512;
constexpr int kFusedWaves = kFusedThreads / 64;
constexpr int kFusedMaxInter = 1024;
constexpr int kGateUpTasks = 4;  // gate_up rows a wavefront fetches before computing
constexpr uint32_t kSpinLimit = 1u << 20;
// sync area (uint32 words): [0] release; [kFlagStride * (1 + b)] flag of workgroup b; then the routing:
// [kRouteBase + 2s] expert id of slot s (ascending id), [kRouteBase + 2s + 1] its weight; [kRouteBase + 2*kMaxK]
// the shared-expert gate
constexpr int kRouteBase = kFlagStride * (1 + kFusedMaxG);

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
    uint32_t* sync;
    float* logits;  // [E + 1]: router logits, then the shared gate's
    float* h_sh;    // [I]
    float* h;       // [k, I]  by slot in ascending expert id
    int H, I, E, k, renorm, G;
};

__device__ __forceinline__ void st_co(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_co(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_co_u32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_co_u32(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_co_u64(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every memory operation this thread issued before has completed (stores acknowledged by the coherent level).
__device__ __forceinline__ void drain() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ bool reached(uint32_t v, uint32_t target) {
    return static_cast<int32_t>(v - target) >= 0;
}

// Raise this workgroup's flag to `target` once all its threads' coherent stores have landed.
__device__ __forceinline__ void arrive(uint32_t* sync, uint32_t target) {
    drain();
    __syncthreads();
    if (threadIdx.x == 0) st_co_u32(sync + kFlagStride * (1 + blockIdx.x), target);
}

// Master: wait until every workgroup's flag reached `target`.
__device__ __forceinline__ bool master_wait(const uint32_t* sync, int G, uint32_t target) {
    for (uint32_t spins = 0;; spins++) {
        int done = 1;
        for (int b = threadIdx.x; b < G; b += blockDim.x)
            if (!reached(ld_co_u32(sync + kFlagStride * (1 + b)), target)) done = 0;
        if (__syncthreads_and(done)) return true;
        if (spins >= kSpinLimit) return false;
        __builtin_amdgcn_s_sleep(1);
    }
}

__device__ __forceinline__ void release(uint32_t* sync, uint32_t target) {
    drain();
    __syncthreads();
    if (threadIdx.x == 0) st_co_u32(sync, target);
}

// Others: wait for the master's release.
__device__ __forceinline__ bool wait_release(const uint32_t* sync, uint32_t target, int* flag) {
    if (threadIdx.x == 0) {
        int ok = 1;
        uint32_t spins = 0;
        while (!reached(ld_co_u32(sync), target)) {
            __builtin_amdgcn_s_sleep(2);
            if (++spins >= kSpinLimit) {
                ok = 0;
                break;
            }
        }
        *flag = ok;
    }
    __syncthreads();
    return *flag != 0;
}

template <int GU, int DN, int EJ, int NBD>
__global__ __launch_bounds__(kFusedThreads) void k_moe_decode(FusedArgs a) {
    constexpr int R = 8 / NBD, WIDTH = 8 * NBD;
    __shared__ float lds_h[kFusedMaxK * kFusedMaxInter];
    __shared__ float lds_hsh[kFusedMaxInter];
    __shared__ float lds_logits[256 + 1];
    __shared__ uint32_t lds_route[2 * kFusedMaxK + 1];
    __shared__ uint32_t tk_scratch[64];
    __shared__ int lds_flag;
    __shared__ uint32_t lds_epoch;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int G = a.G, W = G * kFusedWaves;
    const int slot = wv * G + static_cast<int>(blockIdx.x);  // consecutive slots land on different CUs
    const int H = a.H, I = a.I, E = a.E, k = a.k;
    const bool master = blockIdx.x == 0;
    const bool shared = a.sh_gate_up != nullptr;
    const bool sh_gate = shared && a.sh_gate != nullptr;
    const int gi = lane >> 3, c = lane & 7;
    const int nb = H / kQK;  // <= 8: one gate/up block per lane group
    const bool gu_lane = gi < nb;

    if (threadIdx.x == 0) lds_epoch = ld_co_u32(a.sync + kFlagStride * (1 + blockIdx.x));
    // this lane's x operands for every gate_up row (block gi), fetched once
    const int lo_gu = gi * kQK + BlockInfo<GU>::lo_start(c), hi_gu = lo_gu + BlockInfo<GU>::hi_offset;
    float4 xl[4], xh[4];
    float sxl = 0.0f, sxh = 0.0f;
    if (gu_lane) {
        load_run(a.x + lo_gu, xl);
        load_run(a.x + hi_gu, xh);
        sxl = sum16(xl);
        sxh = sum16(xh);
    }
    const int64_t gu_rs = static_cast<int64_t>(nb) * BlockInfo<GU>::bytes;
    auto gate_up_dots = [&](const Lane32& lg, const Lane32& lu, float& g, float& u) {
        float ag = 0.0f, au = 0.0f;
        if (gu_lane) {
            ag = lane_dot_s(lg, xl, xh, sxl, sxh);
            au = lane_dot_s(lu, xl, xh, sxl, sxh);
        }
        g = group_sum<64>(ag);
        u = group_sum<64>(au);
    };
    __syncthreads();
    const uint32_t epoch = lds_epoch;

    // ---- phase A: router rows, shared gate_up rows
    const int rows_total = E + (sh_gate ? 1 : 0);
    const int n_router = (rows_total + 1) / 2;
    const int n_a = n_router + (shared ? I : 0);
    for (int t = slot; t < n_a; t += W) {
        if (t < n_router) {
            const int row = 2 * t + (lane >> 5);
            const bool valid = row < rows_total;
            const float* wr = row < E ? a.router + static_cast<int64_t>(row) * H : a.sh_gate;
            const float total = router_row(a.x, wr, valid, H, lane);
            if ((lane & 31) == 0 && valid)
                st_co(a.logits + row, (row < E && a.router_bias) ? __fadd_rn(total, a.router_bias[row]) : total);
        } else {
            const int j = t - n_router;
            Lane32 lg, lu;
            if (gu_lane) {
                decode<GU>(a.sh_gate_up + j * gu_rs + gi * BlockInfo<GU>::bytes, c, lg);
                decode<GU>(a.sh_gate_up + (I + j) * gu_rs + gi * BlockInfo<GU>::bytes, c, lu);
            }
            float g, u;
            gate_up_dots(lg, lu, g, u);
            if (lane == 0) st_co(a.h_sh + j, silu(g) * u);
        }
    }

    // ---- barrier 1; the master routes
    bool ok = true;
    arrive(a.sync, epoch + 1);
    if (master) {
        ok = master_wait(a.sync, G, epoch + 1);
        for (int i = threadIdx.x; i < E + (sh_gate ? 1 : 0); i += blockDim.x) lds_logits[i] = ld_co(a.logits + i);
        __syncthreads();
        if (wv == 0) {
            int my_id, my_rank;
            float my_w;
            wave_topk<EJ>(lds_logits, E, k, a.renorm != 0, tk_scratch, lane, my_id, my_w, my_rank);
            if (lane < k) {
                st_co_u32(a.sync + kRouteBase + 2 * my_rank, static_cast<uint32_t>(my_id));
                st_co_u32(a.sync + kRouteBase + 2 * my_rank + 1, __builtin_bit_cast(uint32_t, my_w));
                if (a.ids_out) a.ids_out[lane] = my_id;
                if (a.wts_out) a.wts_out[lane] = my_w;
            }
            if (lane == 0)
                st_co_u32(a.sync + kRouteBase + 2 * kFusedMaxK,
                          __builtin_bit_cast(uint32_t, sh_gate ? sigmoid(lds_logits[E]) : 1.0f));
        }
        release(a.sync, epoch + 1);
    } else {
        ok = wait_release(a.sync, epoch + 1, &lds_flag);
    }
    if (threadIdx.x < 2 * kFusedMaxK + 1) lds_route[threadIdx.x] = ld_co_u32(a.sync + kRouteBase + threadIdx.x);
    if (shared)
        for (int i = threadIdx.x; i < I; i += blockDim.x) lds_hsh[i] = ld_co(a.h_sh + i);
    __syncthreads();
    int sel[kFusedMaxK];
    float wsel[kFusedMaxK];
#pragma unroll
    for (int s = 0; s < kFusedMaxK; s++) {
        sel[s] = static_cast<int>(lds_route[2 * s]);
        wsel[s] = __builtin_bit_cast(float, lds_route[2 * s + 1]);
    }
    const float sgv = __builtin_bit_cast(float, lds_route[2 * kFusedMaxK]);

    // ---- phase B
    const int ND = H / R;  // down waves
    const int row = slot * R + gi / NBD, kb = gi % NBD;
    constexpr int64_t dn_rs = static_cast<int64_t>(NBD) * BlockInfo<DN>::bytes;
    const int lo = kb * kQK + BlockInfo<DN>::lo_start(c), hi = lo + BlockInfo<DN>::hi_offset;
    Lane32 pre[kFusedMaxK];
    float sh_dot = 0.0f;
    if (slot < ND) {
#pragma unroll
        for (int s = 0; s < kFusedMaxK; s++)
            if (s < k)
                decode<DN>(a.down + static_cast<int64_t>(sel[s]) * a.down_stride + row * dn_rs +
                               kb * BlockInfo<DN>::bytes, c, pre[s]);
        if (shared) {
            Lane32 l;
            decode<DN>(a.sh_down + row * dn_rs + kb * BlockInfo<DN>::bytes, c, l);
            float4 hl[4], hh[4];
            load_run(lds_hsh + lo, hl);
            load_run(lds_hsh + hi, hh);
            sh_dot = group_sum<WIDTH>(lane_dot(l, hl, hh));
        }
    } else {
        const int NW = W - ND;
        for (int u0 = slot - ND; u0 < k * I; u0 += NW * kGateUpTasks) {
            Lane32 lg[kGateUpTasks], lu[kGateUpTasks];
#pragma unroll
            for (int q = 0; q < kGateUpTasks; q++) {
                const int u = u0 + q * NW;
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
                const int u = u0 + q * NW;
                if (u < k * I) {
                    float g, up;
                    gate_up_dots(lg[q], lu[q], g, up);
                    if (lane == 0) st_co(a.h + u, silu(g) * up);  // u = s * I + j
                }
            }
        }
    }

    // ---- barrier 2
    arrive(a.sync, epoch + 2);
    if (master) {
        ok = master_wait(a.sync, G, epoch + 2) && ok;
        release(a.sync, epoch + 2);
    } else {
        ok = wait_release(a.sync, epoch + 2, &lds_flag) && ok;
    }

    // ---- phase C
    {
        const int n2 = k * I / 2;
        const uint64_t* src = reinterpret_cast<const uint64_t*>(a.h);
        uint64_t* dst = reinterpret_cast<uint64_t*>(lds_h);
        for (int i = threadIdx.x; i < n2; i += blockDim.x) dst[i] = ld_co_u64(src + i);
    }
    __syncthreads();
    if (slot < ND) {
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < kFusedMaxK; s++) {
            if (s < k) {
                float4 hl[4], hh[4];
                load_run(lds_h + s * I + lo, hl);
                load_run(lds_h + s * I + hi, hh);
                const float d = group_sum<WIDTH>(lane_dot(pre[s], hl, hh));
                acc = s == 0 ? wsel[s] * d : acc + wsel[s] * d;
            }
        }
        if (shared) acc = acc + sgv * sh_dot;
        if ((lane & (WIDTH - 1)) == 0) a.y[row] = ok ? acc : __builtin_nanf("");
    }
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
    if ((L.flags & WL_MOE_NO_FUSED) || T != 1 || L.n_experts > 256 || L.top_k > kFusedMaxK) return false;
    if (L.gate_up_type != WL_TYPE_Q4_K || L.hidden > 8 * kQK) return false;
    const int nbd = L.inter / kQK;
    if (nbd != 1 && nbd != 2 && nbd != 4) return false;
    if (L.shared_gate_up && (L.shared_inter != L.inter || L.shared_gate_up_type != L.gate_up_type ||
                             L.shared_down_type != L.down_type))
        return false;
    const int G = fused_grid();
    if (G < 1) return false;
    const int R = 8 / nbd;
    return L.hidden / R < G * kFusedWaves;  // leaves wavefronts for the gate_up work
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
    a.logits = w.logits;
    a.h_sh = w.h_sh;
    a.h = w.h;
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
    k_zero_words<<<16, 256, 0, s>>>(static_cast<uint32_t*>(workspace), kSyncWords);
    return launch_status();
}

}  // namespace wl
