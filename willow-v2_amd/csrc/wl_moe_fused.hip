// Fused decode: the whole MoE layer for one token in ONE kernel launch (vs. router / top-k / grouping / gate_up /
// down / combine as six launches), which is what bounds batch-1 decode: every launch costs microseconds while a
// layer moves only ~20 MB.
//
// A persistent grid of G workgroups (one per CU, 8 wavefronts each), all in the same role:
//   phase A   the router's logits (a row per wavefront task) and the shared expert's gate_up rows (h_shared),
//             neither of which depends on the routing; each workgroup also loads the shared expert's down rows of
//             the output rows it owns (8 per workgroup);
//   routing   every workgroup gathers the logits and h_shared and runs the top-k itself (candidate ranks
//             counted by the workgroup, the weights by wavefront 3);
//   phase B   every wavefront issues the loads of its gate_up tasks (a gate row and its up row of one picked
//             expert) at once, kept as raw words; while they are in flight the owners dot their shared down rows
//             with h_shared; then the gate_up rows are decoded and dotted, and h (silu(g) * u) published;
//   down      workgroup b owns output rows 8b .. 8b + 7; its wavefront s < k requests those 8 rows of the s-th
//             picked expert's down matrix, which arrive while h crosses workgroups, gathers that expert's h
//             (I values, polled by the wavefront alone) and dots its rows into LDS;
//   combine   in the same workgroup: y = sum_e w_e P_e + sg * shared_down h_sh for its 8 rows, experts in
//             ascending id. Only the logits, h_shared and h cross workgroups.
// fused_eligible requires a grid large enough for one pass: one owner group per workgroup and kGateUpTasks
// gate_up tasks per wavefront (Qwen3.6's shapes on 256 CUs use every workgroup).
// Every CU streams its share of the routed experts' bytes: gate_up rows as soon as the routing is known, down rows
// as soon as its gate_up work is done (requested earlier, they would wait in the CU's load queues ahead of the
// gate_up arithmetic).
// The arithmetic (router_row, the top-k's picks and weights, the gate_up and down dot products, the combine
// order) is the multi-kernel path's.
//
// No barriers: every value that crosses workgroups (logits, h_shared, h) is a 64-bit word (tag << 32 | bits)
// written and read with relaxed device-scope atomics (single-copy atomic, bypassing the per-XCD L2s). The tag is
// this call's epoch, so a consumer polls the data itself until every word it needs carries the current tag.
// Each workgroup keeps its own epoch counter (one 128-byte line each, incremented as it exits), so all agree on
// the epoch without communicating and nothing is ever reset. Every wait is bounded (kSpinLimit polls): a
// workgroup that gives up writes NaN for its outputs and sets the workspace's status word, which
// wl_moe_workspace_status reports (and clears) on the host. Co-residency of the whole grid is what the hand-offs
// need; launch_fused checks it for the exact kernel instance it launches.
#include <hip/hip_runtime.h>

#include "wl_common.h"
#include "wl_host.h"
#include "wl_moe.h"
#include "wl_moe_dev.h"

#include <mutex>

namespace wl {

constexpr int kFusedThreads = 512;
constexpr int kFusedWaves = kFusedThreads / 64;
constexpr int kGateUpTasks = 2;  // gate_up tasks a wavefront has in flight at once (G = 256: all of them)
constexpr int kOwnRows = 8;      // output rows per owner group: the shared and routed down rows and the final sum
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr uint32_t kStarveSpinLimit = 1u << 11;  // WL_MOE_TEST_STARVE: waits known to fail give up after this
static_assert(kFusedThreads >= kFusedMaxE && kFusedMaxE % 32 == 0 && kFusedMaxE / 32 >= kFusedMaxK,
              "the top-k gives every logit a thread and needs at least k groups of 32");

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
    uint32_t* sync;  // kSyncWords: epochs, then tagged logits [E+1], h_shared [I], h [k, I], the status word
    int H, I, E, k, renorm, G;
    uint32_t spin_limit;  // polls before a wait gives up
    int silent_wg;        // WL_MOE_TEST_STARVE: this workgroup publishes nothing (-1: none)
    // the next layer's rows read before its routing is known (NULL next_router: no prefetch); same shapes
    const float* next_router;
    const float* next_sh_gate;
    const float* next_norm_w;  // the next layer's RMSNorm weight, when it has one
    const uint8_t* next_sh_gate_up;
    const uint8_t* next_sh_down;
    const float* norm_w;  // NORM: the RMSNorm weight (zero-centered) or NULL
    float norm_eps;
    int residual;         // y = x + MoE
    float min_w;          // > 0: skip_small_experts with this threshold (the picks kept are the experts run)
    // the next-layer guess (NORM only). Producer (guess_router non-NULL): the next layer's router (and bias) on this
    // layer's x normalized with the next layer's RMSNorm (weight or NULL, eps), one row per workgroup while it waits
    // for h, left in the workspace. Consumer (consume_guess): the previous call's guess on this workspace, read
    // as this call starts; its top-k names the experts whose gate_up rows this call pulls into the caches
    const float* guess_router;
    const float* guess_bias;
    const float* guess_norm_w;
    float guess_eps;
    int consume_guess;
};

// The 128-byte lines of what wavefront slot t reads in phase A (router row t, or the shared expert's gate row j and
// up row I + j for t = n_router + j), and of an owner workgroup's shared down rows: lane l touches line l of the
// wavefront's share (one dword each), so the lines come into this XCD's L2 (and the memory-side cache) ahead of
// the next layer's phase A, which runs the same task on the same workgroup and wavefront.
__device__ __forceinline__ uint32_t touch_lines(const uint8_t* base, int bytes, int lane) {
    const int lines = (bytes + 127) / 128 + 1;  // +1: the rows need not start on a line
    uint32_t v = 0;
    if (lane < lines && base) {
        const uint8_t* p = base + 128 * lane;
        if (lane == lines - 1) p = base + bytes - 4;  // the last line, without reading past the rows
        v = *reinterpret_cast<const uint32_t*>(reinterpret_cast<uintptr_t>(p) & ~uintptr_t{3});
    }
    return v;
}

__device__ __forceinline__ void put_tagged(uint32_t* sync_base, int word, uint32_t tag, float v) {
    const uint64_t w = (static_cast<uint64_t>(tag) << 32) | __builtin_bit_cast(uint32_t, v);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(sync_base + word), w, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Gathers n tagged values (value i: the 64-bit word at sync + src(i), a 32-bit word offset), handing each to
// put(i, value) once it carries `tag` (workgroup-cooperative: thread t polls values t + q blockDim.x, q < Q;
// n <= Q blockDim.x); false if spin_limit polls pass first. lds_bad: an LDS word that is 0 on entry; a thread that
// gave up sets it, and after one barrier every thread reads the verdict (__syncthreads_and takes three barriers).
// Two polling rounds are in flight: a round's loads are issued before the previous round's are checked, so a value
// is seen about half a load's round trip after it lands instead of a whole one (the logits exchange of the b=1
// decode: 15.88 -> 15.62 us per layer; three or four rounds in flight measured slower, their extra loads queueing
// at the few lines every workgroup polls). Every slot is loaded in every round (a value already in, or an index
// past n, reloads a word whose result is dropped), so a round's loads are unconditional and the compiler keeps the
// older round outstanding while it checks.
template <int Q, typename Src, typename Put>
__device__ __forceinline__ bool gather_tagged(const uint32_t* sync, int n, uint32_t tag, uint32_t spin_limit, Src src,
                                              Put put, uint32_t* lds_bad) {
    const uint64_t* w[Q];
    bool pend[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int i = threadIdx.x + q * blockDim.x;
        pend[q] = i < n;
        w[q] = reinterpret_cast<const uint64_t*>(sync + src(pend[q] ? i : 0));
    }
    auto ld = [](const uint64_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto waiting = [&] {
        bool r = false;
#pragma unroll
        for (int q = 0; q < Q; q++) r = r || pend[q];
        return r;
    };
    auto check = [&](const uint64_t (&v)[Q]) {
#pragma unroll
        for (int q = 0; q < Q; q++)
            if (pend[q] && static_cast<uint32_t>(v[q] >> 32) == tag) {
                put(threadIdx.x + q * blockDim.x, __builtin_bit_cast(float, static_cast<uint32_t>(v[q])));
                pend[q] = false;
            }
    };
    uint64_t ra[Q], rb[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) ra[q] = ld(w[q]);
    for (uint32_t spins = 0; spins <= spin_limit; spins += 2) {
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int q = 0; q < Q; q++) rb[q] = ld(w[q]);
        check(ra);
        if (!waiting()) break;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int q = 0; q < Q; q++) ra[q] = ld(w[q]);
        check(rb);
        if (!waiting()) break;
    }
    if (waiting()) *lds_bad = 1u;
    __syncthreads();
    return *lds_bad == 0u;
}

// The same over a share of the workgroup, thread t of nt (values t + q nt), with no barrier at the end: returns
// whether every value of this thread arrived.
template <int Q, typename Src, typename Put>
__device__ __forceinline__ bool gather_tagged_part(const uint32_t* sync, int n, uint32_t tag, uint32_t spin_limit,
                                                   Src src, Put put, int t, int nt) {
    const uint64_t* w[Q];
    bool pend[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int i = t + q * nt;
        pend[q] = i < n;
        w[q] = reinterpret_cast<const uint64_t*>(sync + src(pend[q] ? i : 0));
    }
    auto ld = [](const uint64_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto waiting = [&] {
        bool r = false;
#pragma unroll
        for (int q = 0; q < Q; q++) r = r || pend[q];
        return r;
    };
    auto check = [&](const uint64_t (&v)[Q]) {
#pragma unroll
        for (int q = 0; q < Q; q++)
            if (pend[q] && static_cast<uint32_t>(v[q] >> 32) == tag) {
                put(t + q * nt, __builtin_bit_cast(float, static_cast<uint32_t>(v[q])));
                pend[q] = false;
            }
    };
    uint64_t ra[Q], rb[Q];
#pragma unroll
    for (int q = 0; q < Q; q++) ra[q] = ld(w[q]);
    for (uint32_t spins = 0; spins <= spin_limit; spins += 2) {
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int q = 0; q < Q; q++) rb[q] = ld(w[q]);
        check(ra);
        if (!waiting()) break;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int q = 0; q < Q; q++) ra[q] = ld(w[q]);
        check(rb);
        if (!waiting()) break;
    }
    return !waiting();
}

// The expert logits for the top-k, gathered by its wavefront alone: lane l polls logits l + 64 j (j < EJ, those
// below E), writes each to lds_logits as it lands and keeps its order key (NaN as -inf; 0 for an index past E, or
// for a logit that never arrived) in key[j]. Returns whether every one of the lane's logits arrived.
template <int EJ>
__device__ __forceinline__ bool gather_logits_wave(const uint32_t* sync, int E, uint32_t tag, uint32_t spin_limit,
                                                   float* lds_logits, uint32_t (&key)[EJ]) {
    const int lane = threadIdx.x & 63;
    auto put = [&](int i, float v) {
        lds_logits[i] = v;
        const int j = (i - lane) >> 6;
#pragma unroll
        for (int jj = 0; jj < EJ; jj++)
            if (jj == j) key[jj] = order_key(v == v ? v : -INFINITY);
    };
#pragma unroll
    for (int j = 0; j < EJ; j++) key[j] = 0u;
    return gather_tagged_part<EJ>(sync, E, tag, spin_limit, [&](int i) { return kTagLogits + 2 * i; }, put, lane, 64);
}

// The same for one wavefront alone: n = 64 Q values, lane l polling values l + 64 q. It first waits on the last
// value of each lane only (64 words instead of 64 Q per round), then gathers them all: an expert's last h values
// come from the highest-numbered workgroups, which start last, so by the time those are in, nearly all of them
// are, and the bulk polls no longer load the memory system while the producers finish (17.90 -> 17.60 us per
// layer). All Q loads of a polling round are issued before any is checked.
template <int Q, typename Src, typename Dst>
__device__ __forceinline__ bool gather_tagged_wave(const uint32_t* sync, uint32_t tag, uint32_t spin_limit, Src src,
                                                   Dst dst) {
    static_assert(Q <= 32, "");
    const int lane = threadIdx.x & 63;
    for (uint32_t spins = 0; spins < spin_limit; spins++) {
        const uint64_t w = __hip_atomic_load(reinterpret_cast<const uint64_t*>(sync + src(lane + 64 * (Q - 1))),
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__all(static_cast<uint32_t>(w >> 32) == tag)) break;
        __builtin_amdgcn_s_sleep(1);
    }
    uint32_t pending = Q == 32 ? 0xFFFFFFFFu : (1u << Q) - 1u;
    for (uint32_t spins = 0;; spins++) {
        uint64_t w[Q];
#pragma unroll
        for (int q = 0; q < Q; q++)
            w[q] = (pending >> q) & 1u ? __hip_atomic_load(reinterpret_cast<const uint64_t*>(sync + src(lane + 64 * q)),
                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                       : 0;
#pragma unroll
        for (int q = 0; q < Q; q++)
            if (((pending >> q) & 1u) && static_cast<uint32_t>(w[q] >> 32) == tag) {
                *dst(lane + 64 * q) = __builtin_bit_cast(float, static_cast<uint32_t>(w[q]));
                pending &= ~(1u << q);
            }
        if (__all(pending == 0)) return true;
        if (spins >= spin_limit) return false;
        __builtin_amdgcn_s_sleep(1);
    }
}

template <int GU, int DN, int EJ, int NBD, bool NORM, bool GUESS>
__global__ __launch_bounds__(kFusedThreads) void k_moe_decode(FusedArgs a) {
    constexpr int WIDTH = 8 * NBD;  // lanes per down row (8 per block)
    constexpr int R = 64 / WIDTH;   // down rows per wavefront pass
    __shared__ float lds_h[kFusedMaxK][kFusedMaxInter];  // the h of each picked expert (wavefront s: slot s)
    __shared__ float lds_hsh[kFusedMaxInter];
    __shared__ float lds_logits[kFusedMaxE + 1];
    __shared__ int lds_sel[kFusedMaxK];
    __shared__ float lds_wsel[kFusedMaxK];
    __shared__ float lds_sh[kOwnRows];
    __shared__ float lds_p[kFusedMaxK * kOwnRows];
    __shared__ __attribute__((aligned(16))) float lds_res[kOwnRows];  // with NORM: the owner rows' x, for the residual
    __shared__ __attribute__((aligned(16))) uint64_t lds_cand[kFusedMaxE];
    __shared__ int lds_pick[kFusedMaxK];
    __shared__ uint32_t lds_bad[3];  // a wait gave up: the routing gather's, the call's; wavefronts done
    __shared__ int lds_kk;  // experts run: k, or with min_w those skip_small keeps
    // x (NORM: normalized) for every read, 4 floats of padding after every 64 values (x_slot)
    __shared__ __attribute__((aligned(16))) float lds_xn[kFusedMaxHidden + kFusedMaxHidden / 16];
    // GUESS (the next-layer guess): x normalized with the next layer's RMSNorm; the previous call's guess (ids)
    __shared__ __attribute__((aligned(16))) float lds_xg[GUESS ? kFusedMaxHidden : 4];
    __shared__ int lds_gsel[GUESS ? kFusedMaxK : 1];
    __shared__ int lds_gvalid;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int b = blockIdx.x, G = a.G;
    const int H = a.H, I = a.I, E = a.E, k = a.k;
    const bool shared = a.sh_gate_up != nullptr;
    const bool sh_gate = shared && a.sh_gate != nullptr;
    const int n_logits = E + (sh_gate ? 1 : 0);
    const int gi = lane >> 3, c = lane & 7;
    const int NW = G * kFusedWaves;
    const int slot = wv * G + b;  // wavefront slot: consecutive slots on different CUs
    constexpr int64_t dn_rs = static_cast<int64_t>(NBD) * BlockInfo<DN>::bytes;
    // a lane's place in a down row: block kb, and its two 16-value runs of h
    const int drow = lane / WIDTH, kb = (lane % WIDTH) >> 3;
    const int lo = kb * kQK + BlockInfo<DN>::lo_start(c), hi = lo + BlockInfo<DN>::hi_offset;
    uint32_t* epoch_word = a.sync + kFlagStride * b;

    // every thread reads the epoch itself: no barrier, and the load overlaps the first weight loads
    const uint32_t tag = __hip_atomic_load(epoch_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    bool ok = true;
    const bool publish = b != a.silent_wg;

    // The layer's input: x, or with NORM its RMSNorm, written once to LDS by the workgroup. Thread i loads x's
    // values 4i..4i+3 (and the norm weight's), so x crosses from L2 once per workgroup, in coalesced loads; with
    // NORM wavefront 0 then takes the sum of squares from LDS in the router's order (router_row of x with itself)
    // and every thread normalizes its four values in place. Every later read of x (router rows, gate_up runs) comes
    // from LDS: a router lane's own 64-value segment read from global memory takes 16 loads that each touch 32
    // lines, in every wavefront. (Every wavefront reading all of x from global memory for its own sum of squares
    // took ~8 us at this grid: 2048 wavefronts on the same 64 lines.)
    static_assert(kFusedMaxHidden / 4 <= kFusedThreads, "one float4 of x per thread");
    static_assert(kFusedMaxHidden <= 32 * kRouterSeg, "a router row: one 64-value segment per lane of a half-wave");
    // A wavefront whose first phase-A task is a router row requests that row (lane s < 32: segment s) before the
    // prologue, so its latency overlaps the wait for x instead of following the prologue.
    float4 wpre[kRouterSeg / 4];
    {
        if (slot < n_logits && lane < H / kRouterSeg) {
            const float* wr0 = slot < E ? a.router + static_cast<int64_t>(slot) * H : a.sh_gate;
#pragma unroll
            for (int i = 0; i < kRouterSeg / 4; i++)
                wpre[i] = reinterpret_cast<const float4*>(wr0 + lane * kRouterSeg)[i];
        }
    }
    const bool guess = GUESS && a.guess_router != nullptr;
    // float4 i of x sits at float4 x_slot(i) of lds_xn: a router lane's 64-value segment then starts 4 banks past
    // its neighbour's instead of on the same ones (a 4-way instead of a 32-way conflict)
    auto x_slot = [](int i) { return i + (i >> 4); };
    auto xload = [&](int i) -> float4 { return reinterpret_cast<const float4*>(lds_xn)[x_slot(i)]; };
    if constexpr (NORM) {
        __shared__ float lds_inv, lds_inv_g;
        const bool mine = static_cast<int>(threadIdx.x) < H / 4;
        float4 xv = make_float4(0.f, 0.f, 0.f, 0.f), nw = xv, gw = xv;
        if (mine) {
            xv = reinterpret_cast<const float4*>(a.x)[threadIdx.x];
            // the owner rows' x for the residual (LDS holds the normalized x), so the final sum reads it from LDS
            if (b < H / kOwnRows && (static_cast<int>(threadIdx.x) >> 1) == b)
                reinterpret_cast<float4*>(lds_res)[threadIdx.x & 1] = xv;
            if (a.norm_w) nw = reinterpret_cast<const float4*>(a.norm_w)[threadIdx.x];
            if (guess && a.guess_norm_w) gw = reinterpret_cast<const float4*>(a.guess_norm_w)[threadIdx.x];
            reinterpret_cast<float4*>(lds_xn)[x_slot(threadIdx.x)] = xv;
        }
        __syncthreads();
        if (wv == 0) {
            const float ss = router_row_xw(xload, [&](int sg, int i) { return xload(sg * (kRouterSeg / 4) + i); },
                                           true, H, lane);
            if (lane == 0) {
                lds_inv = norm_inv(ss, H, a.norm_eps);
                lds_inv_g = norm_inv(ss, H, a.guess_eps);  // the same x: only the weight and eps differ
            }
        }
        __syncthreads();
        if (mine) {
            reinterpret_cast<float4*>(lds_xn)[x_slot(threadIdx.x)] =
                norm_apply(xv, a.norm_w != nullptr, nw, lds_inv);
            if (guess)
                reinterpret_cast<float4*>(lds_xg)[threadIdx.x] = norm_apply(xv, a.guess_norm_w != nullptr, gw,
                                                                            lds_inv_g);
        }
        __syncthreads();
    } else {
        if (static_cast<int>(threadIdx.x) < H / 4)
            reinterpret_cast<float4*>(lds_xn)[x_slot(threadIdx.x)] =
                reinterpret_cast<const float4*>(a.x)[threadIdx.x];
        __syncthreads();
    }


    // x, for the gate_up dot products: a lane's two 16-value runs of its block gi
    const int nb = H / kQK;  // <= 8: one gate/up block per lane group
    const bool gu_lane = gi < nb;
    const int lo_gu = gi * kQK + BlockInfo<GU>::lo_start(c), hi_gu = lo_gu + BlockInfo<GU>::hi_offset;
    const int64_t gu_rs = static_cast<int64_t>(nb) * BlockInfo<GU>::bytes;
    // loaded now; their run sums are taken where they are first used (phase A's shared gate_up task, and once
    // before phase B for both of its tasks), so nothing waits for x here
    float4 xl[4], xh[4];
    if (gu_lane) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            xl[i] = xload(lo_gu / 4 + i);
            xh[i] = xload(hi_gu / 4 + i);
        }
    }
    auto gate_up_dots_s = [&](const Lane32& lg, const Lane32& lu, float sxl, float sxh, float& g, float& u) {
        float ag = 0.0f, au = 0.0f;
        if (gu_lane) {
            ag = lane_dot_s(lg, xl, xh, sxl, sxh);
            au = lane_dot_s(lu, xl, xh, sxl, sxh);
        }
        g = group_sum<64>(ag);
        u = group_sum<64>(au);
    };
    auto gate_up_dots = [&](const Lane32& lg, const Lane32& lu, float& g, float& u) {
        gate_up_dots_s(lg, lu, gu_lane ? sum16(xl) : 0.0f, gu_lane ? sum16(xh) : 0.0f, g, u);
    };

    // workgroup b < H / kOwnRows owns output rows kOwnRows b .. + kOwnRows - 1; wavefront w < 8 / R takes rows
    // kOwnRows b + R w + drow of the shared down matrix (fetched after phase A's loads, used once h_shared is known)
    const bool owner = b < H / kOwnRows;
    const bool sh_wave = wv < kOwnRows / R;
    RawLane<DN> shraw;
    uint32_t touched = 0;  // prefetch loads: consumed (never used) at the very end, so they are kept

    // phase A: router rows, shared gate_up rows
    const int n_router = n_logits;  // one router row per wavefront task (lanes 0..31), more tasks in parallel
    const int n_a = n_router + (shared ? I : 0);
    for (int t = slot; t < n_a; t += NW) {
        if (t < n_router) {
            const int row = t;
            const bool valid = lane < 32;
            const float* wr = row < E ? a.router + static_cast<int64_t>(row) * H : a.sh_gate;
            float total;
            if (t == slot)  // the row requested before the prologue
                total = router_row_xw(xload, [&](int, int i) { return wpre[i]; }, valid, H, lane);
            else
                total = router_row_x(xload, wr, valid, H, lane);
            if ((lane & 31) == 0 && valid && publish)
                put_tagged(a.sync, kTagLogits + 2 * row, tag,
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
            if (lane == 0 && publish) put_tagged(a.sync, kTagHsh + 2 * j, tag, silu(g) * u);
        }
    }
    // the shared down rows: requested only now, after phase A, whose router rows would otherwise queue behind them
    if (shared && sh_wave && owner)
        shraw.fetch(a.sh_down + static_cast<int64_t>(kOwnRows * b + R * wv + drow) * dn_rs +
                        kb * BlockInfo<DN>::bytes, c);

    // the previous call's next-layer guess (a decoder loop's previous layer, WL_MOE_GUESS_NEXT), read in the last
    // wavefront, which has no phase A task: when every guess logit the previous call left in the workspace carries
    // that call's tag, their top-k (the guessed experts) goes to LDS for the prefetch below.
    const int lpr = static_cast<int>((gu_rs + 127) / 128);  // 128-byte lines per gate_up row
    const int nrj = (I - b + G - 1) / G;                     // this workgroup's gate_up rows j = b + G m < I
    if constexpr (GUESS) {
        if (a.consume_guess && wv == kFusedWaves - 1) {
            const uint32_t prev = tag - 1u;
            const int set = static_cast<int>(prev & 1u);
            bool fresh = true;
            uint32_t key[EJ];
#pragma unroll
            for (int j = 0; j < EJ; j++) {
                const int idx = lane + 64 * j;
                key[j] = 0u;
                if (idx < E) {
                    const uint64_t w = __hip_atomic_load(
                        reinterpret_cast<const uint64_t*>(a.sync + kTagGuess + 2 * (set * kFusedMaxE + idx)),
                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    fresh = fresh && static_cast<uint32_t>(w >> 32) == prev;
                    const float v = __builtin_bit_cast(float, static_cast<uint32_t>(w));
                    key[j] = order_key(v == v ? v : -INFINITY);
                }
            }
            const bool valid = __all(fresh);
            if (valid) select_top_keys<EJ>(key, k, lane, lds_gsel);
            if (lane == 0) lds_gvalid = valid ? 1 : 0;
        }
    }

    // routing: the logits and h_shared (both from phase A) gathered, then the top-k. The barrier keeps the
    // workgroup's idle wavefronts from polling while its phase A work (and everyone else's) is still loading; the
    // barrier after the top-k is the one that makes the gathered values visible to every wavefront.
    if (threadIdx.x < 3) lds_bad[threadIdx.x] = 0u;
    __syncthreads();
    // wavefront 0 gathers the expert logits into registers for the top-k (the keys need no LDS round trip and no
    // barrier before it); the other wavefronts gather the rest: the shared gate's logit and h_shared
    uint32_t k32[EJ];
    if (wv == 0) {
        ok = gather_logits_wave<EJ>(a.sync, E, tag, a.spin_limit, lds_logits, k32) && ok;
        lane_sync();  // its lds_logits writes before any lane's reads below
    } else {
        const int n_gate = n_logits - E;  // 1 with a shared gate, else 0
        const int n_rest = n_gate + (shared ? I : 0);
        auto src = [&](int i) { return i < n_gate ? kTagLogits + 2 * (E + i) : kTagHsh + 2 * (i - n_gate); };
        auto put = [&](int i, float v) {
            if (i < n_gate)
                lds_logits[E + i] = v;
            else
                lds_hsh[i - n_gate] = v;
        };
        constexpr int nt = kFusedThreads - 64;
        static_assert(3 * nt >= 1 + kFusedMaxInter, "three values per thread at most");
        const int t = static_cast<int>(threadIdx.x) - 64;
        ok = (n_rest <= 2 * nt ? gather_tagged_part<2>(a.sync, n_rest, tag, a.spin_limit, src, put, t, nt)
                               : gather_tagged_part<3>(a.sync, n_rest, tag, a.spin_limit, src, put, t, nt)) &&
             ok;
    }
    // the guessed experts' gate_up rows this workgroup reads below (its gate_up task u = s I + j sits on wavefront
    // slot u mod (8 G), so on workgroup u mod G: rows j = b, b + G, ... and their up rows), one 4-byte load per
    // 128-byte line, spread over wavefronts 1 .. 7 while wavefront 0 runs the top-k: HBM carries nothing else then,
    // and the lines reach this XCD's L2 before the loads below ask for them.
    if constexpr (GUESS) {
        if (a.consume_guess && wv > 0 && lds_gvalid) {
            const int per_e = 2 * nrj * lpr, lines = k * per_e;
            for (int L = lane + 64 * (wv - 1); L < lines; L += 64 * (kFusedWaves - 1)) {
                const int s = L / per_e, rl = L - s * per_e, r = rl / lpr, ln = rl - r * lpr;
                const int j = b + G * (r < nrj ? r : r - nrj);
                const int row = r < nrj ? j : I + j;
                const int64_t off = static_cast<int64_t>(row) * gu_rs +
                                    (ln + 1 < lpr ? 128 * ln : static_cast<int>(gu_rs) - 4);
                touched ^= *reinterpret_cast<const uint32_t*>(
                    a.gate_up + static_cast<int64_t>(lds_gsel[s]) * a.gate_up_stride + off);
            }
        }
    }
    // top-k, in wavefront 0. Lane l holds the order keys of logits l + 64 j (k32, from its gather). The groups of 32
    // logits (i / 32) have their largest order key formed in registers (a half-wavefront maximum); with T0 the
    // smallest maximum of the groups that hold a logit, at least that many keys are >= T0, so when those are at
    // least k the top k are among the candidates key >= T0 (typically 8 to 25), otherwise every logit is one. The
    // candidates (key: order key, then inverted id; 64 bits, all distinct: larger first, ties to the lower id) are
    // compacted in LDS and each counts the candidates above it: up to 32 of them in one fixed pass over a
    // zero-padded list, split between the two halves of the wavefront. The k of rank < k place themselves; their
    // weights (wave_topk's arithmetic) are computed after the gate_up loads have been issued.
    static_assert(kFusedMaxK <= 8, "");
    if (wv == 0) {
        bool valid[EJ];
#pragma unroll
        for (int j = 0; j < EJ; j++) valid[j] = lane + 64 * j < E;  // k32[j] is 0 where not: below every logit's
        if (lane < 32) lds_cand[lane] = 0;  // below every candidate's key
        // each 32-logit group's largest key: group 2 j + (l >> 5) is held by half l >> 5 of the wavefront at j
        const int ng = (E + 31) / 32;
        uint32_t t0 = 0xFFFFFFFFu;
#pragma unroll
        for (int j = 0; j < EJ; j++) {
            uint32_t g = k32[j];
            g = max(g, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(g), 0xB1, 0xF, 0xF, false)));
            g = max(g, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(g), 0x4E, 0xF, 0xF, false)));
            g = max(g, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(g), 0x141, 0xF, 0xF, false)));
            g = max(g, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(g), 0x140, 0xF, 0xF, false)));
            const auto sw = __builtin_amdgcn_permlane16_swap(g, g, false, false);
            g = max(static_cast<uint32_t>(sw[0]), static_cast<uint32_t>(sw[1]));
            if (2 * j < ng) t0 = min(t0, static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(g), 0)));
            if (2 * j + 1 < ng) t0 = min(t0, static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(g), 32)));
        }
        if (ng < k) t0 = 0;
        lane_sync();
        int n_cand = 0;
#pragma unroll
        for (int j = 0; j < EJ; j++) {
            const int idx = lane + 64 * j;
            const bool cand = valid[j] && k32[j] >= t0;
            const uint64_t m = __ballot(cand);
            if (cand)
                lds_cand[n_cand + lanes_below(m)] =
                    (static_cast<uint64_t>(k32[j]) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(idx));
            n_cand += __popcll(m);
        }
        lane_sync();
        uint64_t ck[EJ];
        int above[EJ];
#pragma unroll
        for (int q = 0; q < EJ; q++) {
            const int u = lane + 64 * q;
            ck[q] = u < n_cand ? lds_cand[u] : 0;
            above[q] = 0;
        }
        if (n_cand <= 32) {
            // lane l and lane l + 32 both rank candidate l (l < 32), against list entries 0..15 and 16..31; the
            // two counts meet in one v_permlane32_swap (each lane gets its partner's, and adds its own)
            const int half = lane >> 5;
            const uint64_t mine = lds_cand[lane & 31];
            int c0 = 0, c1 = 0;  // two counts, so the compares do not form one dependent chain
            uint4 rr[8];  // the 8 list reads in flight at once, then the compares
#pragma unroll
            for (int u = 0; u < 16; u += 2) rr[u / 2] = *reinterpret_cast<const uint4*>(&lds_cand[16 * half + u]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < 16; u += 2) {
                const uint4 r = rr[u / 2];
                const uint64_t o0 = (static_cast<uint64_t>(r.y) << 32) | r.x;
                const uint64_t o1 = (static_cast<uint64_t>(r.w) << 32) | r.z;
                c0 += o0 > mine ? 1 : 0;
                c1 += o1 > mine ? 1 : 0;
            }
            const auto sw = __builtin_amdgcn_permlane32_swap(c0 + c1, c0 + c1, false, false);
            above[0] = static_cast<int>(sw[0]) + static_cast<int>(sw[1]);
        } else {
            for (int u0 = 0; u0 < n_cand; u0 += 2) {  // entries past n_cand (< kFusedMaxE) are never counted
                const uint4 r = *reinterpret_cast<const uint4*>(&lds_cand[u0]);
                const uint64_t o0 = (static_cast<uint64_t>(r.y) << 32) | r.x;
                const uint64_t o1 = (static_cast<uint64_t>(r.w) << 32) | r.z;
#pragma unroll
                for (int q = 0; q < EJ; q++)
                    above[q] += (o0 > ck[q] ? 1 : 0) + ((u0 + 1 < n_cand && o1 > ck[q]) ? 1 : 0);
            }
        }
#pragma unroll
        for (int q = 0; q < EJ; q++)
            if (lane + 64 * q < n_cand && above[q] < k)
                lds_pick[above[q]] = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(ck[q]));
        lane_sync();
        // the picks in ascending id order for the tasks; the weights (needed only by the final sum) come later
        if (a.min_w > 0.0f) {
            const int my_id = lane < k ? lds_pick[lane] : 0;
            // skip_small_experts: which picks run depends on the weights, so they are computed here, before any
            // gate_up load (the same arithmetic as below); only the kept picks become tasks
            const float lv0 = lds_logits[__builtin_amdgcn_readfirstlane(my_id)];
            const float m = lv0 == lv0 ? lv0 : -INFINITY;
            const float ssum = softmax_sum<EJ>(lds_logits, E, lane, m);
            const float lv = lds_logits[my_id];
            float my_w = pick_weight(lane < k ? (lv == lv ? lv : -INFINITY) : -INFINITY, m, ssum, k, a.renorm != 0,
                                     lane);
            int out_id = my_id;
            const bool keep = skip_small(my_w, out_id, k, a.min_w, lane);
            const uint64_t kept = __ballot(keep);
            int my_rank = 0;  // position among the kept ids in ascending order
#pragma unroll
            for (int q = 0; q < kFusedMaxK; q++)
                my_rank += (((kept >> q) & 1u) && __builtin_amdgcn_readlane(my_id, q) < my_id) ? 1 : 0;
            if (keep) {
                lds_sel[my_rank] = my_id;
                lds_wsel[my_rank] = my_w;
            }
            if (lane < k && b == 0) {
                if (a.ids_out) a.ids_out[lane] = out_id;
                if (a.wts_out) a.wts_out[lane] = my_w;
            }
            if (lane == 0) lds_kk = __popcll(kept);
        } else {
            // the candidates were compacted in ascending id order, so a pick's place among the k ids is the number
            // of picks before it in the list
            int before = 0;
#pragma unroll
            for (int q = 0; q < EJ; q++) {
                const bool picked = lane + 64 * q < n_cand && above[q] < k;
                const uint64_t pm = __ballot(picked);
                if (picked)
                    lds_sel[before + lanes_below(pm)] = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(ck[q]));
                before += __popcll(pm);
            }
            if (lane == 0) lds_kk = k;
        }
    }
    __syncthreads();
    const int kk = lds_kk;  // the experts run (k unless skip_small dropped some)
    int sel[kFusedMaxK];
#pragma unroll
    for (int s = 0; s < kFusedMaxK; s++) sel[s] = lds_sel[s];
    auto expert_of = [&](int s) {
        int e = 0;
#pragma unroll
        for (int r = 0; r < kFusedMaxK; r++)
            if (r == s) e = sel[r];
        return e;
    };

    // phase B: every load of this wavefront's gate_up tasks (at most kGateUpTasks), before any arithmetic
    const int n_tasks = kk * I;
    RawLane<GU> graw[kGateUpTasks][2];
#pragma unroll
    for (int q = 0; q < kGateUpTasks; q++) {
        const int u = slot + q * NW;
        if (u < n_tasks && gu_lane) {
            const int s = u / I, j = u - s * I;
            const uint8_t* w = a.gate_up + static_cast<int64_t>(expert_of(s)) * a.gate_up_stride;
            graw[q][0].fetch(w + j * gu_rs + gi * BlockInfo<GU>::bytes, c);
            graw[q][1].fetch(w + (I + j) * gu_rs + gi * BlockInfo<GU>::bytes, c);
        }
    }
    // the routing weights, needed only by the final sum: wavefront 3 computes them while the loads above are in flight
    // (softmax over all logits with the max from pick 0, as softmax_stats takes it; renormalised in pick order). Not
    // wavefront 0: its SIMD has just run the top-k and runs the shared down rows next.
    if (wv == 3 && !(a.min_w > 0.0f)) {
        const int my_id = lane < k ? lds_pick[lane] : 0;
        const float lv0 = lds_logits[__builtin_amdgcn_readfirstlane(my_id)];
        const float m = lv0 == lv0 ? lv0 : -INFINITY;
        const float ssum = softmax_sum<EJ>(lds_logits, E, lane, m);
        const float lv = lds_logits[my_id];
        const float my_w = pick_weight(lane < k ? (lv == lv ? lv : -INFINITY) : -INFINITY, m, ssum, k,
                                       a.renorm != 0, lane);
        int my_rank = 0;
#pragma unroll
        for (int q = 0; q < kFusedMaxK; q++) my_rank += (q < k && __builtin_amdgcn_readlane(my_id, q) < my_id) ? 1 : 0;
        if (lane < k) {
            lds_wsel[my_rank] = my_w;
            if (b == 0) {
                if (a.ids_out) a.ids_out[lane] = my_id;
                if (a.wts_out) a.wts_out[lane] = my_w;
            }
        }
    }

    // the shared expert's down rows of this workgroup's owner group, while the loads above are in flight
    float sgv = 1.0f;
    if (sh_gate) sgv = sigmoid(lds_logits[E]);
    if (shared && sh_wave && owner) {
        Lane32 w;
        shraw.unpack(c, w);
        float4 hl[4], hh[4];
        load_run(lds_hsh + lo, hl);
        load_run(lds_hsh + hi, hh);
        const float v = group_sum<WIDTH>(lane_dot(w, hl, hh));
        if ((lane % WIDTH) == 0) lds_sh[R * wv + drow] = v;
    }

    // gate_up: decode, dot, publish h[s][j] (x's run sums once for the wavefront's tasks; the nibbles go into
    // v_fma_mix_f32 products as f16 subnormals, lane_dot_q4mix)
    const float sxl = gu_lane ? sum16(xl) : 0.0f, sxh = gu_lane ? sum16(xh) : 0.0f;
#pragma unroll
    for (int q = 0; q < kGateUpTasks; q++) {
        const int u = slot + q * NW;
        if (u < n_tasks) {
            Lane32 lg, lu;
            if (gu_lane) {
                graw[q][0].unpack_mix(c, lg);
                graw[q][1].unpack_mix(c, lu);
            }
            float g = 0.0f, up = 0.0f;
            if (gu_lane) {
                g = lane_dot_q4mix(lg, xl, xh, sxl, sxh);
                up = lane_dot_q4mix(lu, xl, xh, sxl, sxh);
            }
            g = group_sum<64>(g);
            up = group_sum<64>(up);
            if (lane == 0 && publish) put_tagged(a.sync, kTagH + 2 * u, tag, silu(g) * up);  // u = s * I + j
        }
    }

    // down: wavefront s < k takes the owner's rows of the s-th picked expert. They are requested only now (so far
    // the gate_up rows had the bandwidth and the load queues to themselves) and arrive while h crosses workgroups;
    // then the wavefront gathers that expert's h, dots its 8 rows and leaves the sums in LDS
    // next-layer overlap: the lines this wavefront's phase A task reads in the next layer (and, in the last
    // wavefront, the next layer's shared down rows of this owner), requested now: this wavefront's first h poll
    // below would not succeed before they arrive anyway. Consumed (never used) at the very end.
    if (a.next_router) {
        const int t = slot;
        if (guess && t < E) {
            // guess_rows computes this row of the next layer's router on this workgroup
        } else if (t < n_router) {
            const float* wr = t < E ? a.next_router + static_cast<int64_t>(t) * H : a.next_sh_gate;
            touched = touch_lines(reinterpret_cast<const uint8_t*>(wr), 4 * H, lane);
        } else if (t < n_a) {
            const int j = t - n_router;
            const int part = lane >> 5;  // lanes 0..31 the gate row, 32..63 the up row
            touched = touch_lines(a.next_sh_gate_up + static_cast<int64_t>(part ? I + j : j) * gu_rs,
                                  static_cast<int>(gu_rs), lane & 31);
        }
        if (wv == kFusedWaves - 1 && owner && a.next_sh_down)
            touched ^= touch_lines(a.next_sh_down + static_cast<int64_t>(kOwnRows * b) * dn_rs,
                                   static_cast<int>(kOwnRows * dn_rs), lane);
        if (wv == kFusedWaves - 2 && a.next_norm_w)  // every workgroup reads all of it first thing
            touched ^= touch_lines(reinterpret_cast<const uint8_t*>(a.next_norm_w), 4 * H, lane);
    }
    // the next-layer guess (producer): the next layer's router rows e = b, b + G, ... on x normalized with that
    // layer's RMSNorm (router_row's order, then the bias), computed while this wavefront waits for h (after its
    // down rows are requested) and left in the workspace's guess set tag & 1 for the next call. The wavefront is
    // one of the first picked experts', whose h comes from the first gate_up tasks and so is gathered earlier. Row e
    // is computed on the workgroup whose wavefront slot e reads it in the next layer's phase A (workgroup e mod G,
    // the same XCD), so this also stands for that row's prefetch.
    const int guess_wave = k > 1 ? 1 : 0;
    auto guess_rows = [&]() {
        for (int e = b; e < E; e += G) {
            const float total = router_row_x([&](int i) { return reinterpret_cast<const float4*>(lds_xg)[i]; },
                                             a.guess_router + static_cast<int64_t>(e) * H, lane < 32, H, lane);
            if (lane == 0 && publish)
                put_tagged(a.sync, kTagGuess + 2 * (static_cast<int>(tag & 1u) * kFusedMaxE + e), tag,
                           a.guess_bias ? __fadd_rn(total, a.guess_bias[e]) : total);
        }
    };
    if (guess && wv == guess_wave && !(owner && wv < kk)) guess_rows();
    if (owner && wv < kk) {
        auto own_row = [&](int pass) { return kOwnRows * b + R * pass + drow; };
        RawLane<DN> draw[NBD];
        const uint8_t* w = a.down + static_cast<int64_t>(expert_of(wv)) * a.down_stride;
#pragma unroll
        for (int p = 0; p < NBD; p++)
            draw[p].fetch(w + static_cast<int64_t>(own_row(p)) * dn_rs + kb * BlockInfo<DN>::bytes, c);
        if (guess && wv == guess_wave) guess_rows();
        // the down rows unpacked while h crosses workgroups (the first h poll waits for their loads anyway)
        Lane32 wr[NBD];
#pragma unroll
        for (int p = 0; p < NBD; p++) draw[p].unpack(c, wr[p]);
        float* hs = lds_h[wv];
        ok = gather_tagged_wave<4 * NBD>(
                 a.sync, tag, a.spin_limit, [&](int i) { return kTagH + 2 * (wv * I + i); },
                 [&](int i) { return &hs[i]; }) &&
             ok;
        lane_sync();
        float4 hl[4], hh[4];  // the lane's two runs of h: the same in every pass
        load_run(hs + lo, hl);
        load_run(hs + hi, hh);
        const float shl = sum16(hl), shh = sum16(hh);
#pragma unroll
        for (int p = 0; p < NBD; p++) {
            const float v = group_sum<WIDTH>(lane_dot_s(wr[p], hl, hh, shl, shh));
            if ((lane % WIDTH) == 0) lds_p[wv * kOwnRows + R * p + drow] = v;
        }
    }

    // combine: the owner's rows y[j] = sum_s w_s P[s][j] (+ sg * shared), s in ascending expert id, by the last
    // wavefront of the workgroup to get here; the others exit. A wavefront's LDS operations are performed in order
    // and the count is an acquire-release LDS atomic, so the last one reads every other's partial sums, shared rows,
    // weights and verdict (a flag word: whether every wait of the call ended).
    if (!ok) lds_bad[1] = 1u;
    __asm__ volatile("" ::"v"(touched));  // the prefetch loads count as used, so they are kept
    uint32_t prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(&lds_bad[2], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (__builtin_amdgcn_readfirstlane(prev) != kFusedWaves - 1) return;
    const bool all_ok = lds_bad[1] == 0u;
    if (owner && lane < kOwnRows) {
        const int r = lane;
        // every weight and partial read before the chain (a loop over kk waited out one LDS read per term)
        float wv[kFusedMaxK], pv[kFusedMaxK];
#pragma unroll
        for (int s = 0; s < kFusedMaxK; s++) {
            wv[s] = lds_wsel[s];
            pv[s] = lds_p[s * kOwnRows + r];
        }
        __builtin_amdgcn_sched_barrier(0);
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < kFusedMaxK; s++)
            if (s < kk) acc = s == 0 ? wv[s] * pv[s] : acc + wv[s] * pv[s];
        if (shared) acc = acc + sgv * lds_sh[r];
        if (a.residual) acc = __fadd_rn(NORM ? lds_res[r] : a.x[kOwnRows * b + r], acc);
        a.y[kOwnRows * b + r] = all_ok ? acc : __builtin_nanf("");
    }
    if (!all_ok && lane == 0)  // a vector atomic, visible to the host's status query
        __hip_atomic_fetch_or(a.sync + kStatusWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (lane == 0) __hip_atomic_store(epoch_word, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void k_zero_words(uint32_t* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// ---------------------------------------------------------------------------------------------------------------

// The fused kernel instance a layer runs: gate_up Q4_K; down Q4_K or Q6_K; EJ logits per lane of the top-k; NBD
// down blocks per row (inter / 256). The next-layer guess (WL_MOE_GUESS_NEXT with the pre-norm) has instances of
// its own, at Qwen3.6's shapes only (elsewhere the flag is ignored), so the code of the other instances is the same
// as without it.
static bool guess_instance(const WlMoeLayer& L) {
    return (L.flags & WL_MOE_GUESS_NEXT) && (L.flags & WL_MOE_PRE_NORM) && L.n_experts > 128 &&
           L.n_experts <= 256 && L.inter == 2 * kQK;
}

static const void* fused_instance(const WlMoeLayer& L) {
    const int ej = L.n_experts <= 64 ? 1 : L.n_experts <= 128 ? 2 : 4;
    const int nbd = L.inter / kQK;
    const bool norm = (L.flags & WL_MOE_PRE_NORM) != 0;
    if (guess_instance(L))
        return L.down_type == WL_TYPE_Q4_K
                   ? reinterpret_cast<const void*>(&k_moe_decode<WL_TYPE_Q4_K, WL_TYPE_Q4_K, 4, 2, true, true>)
                   : reinterpret_cast<const void*>(&k_moe_decode<WL_TYPE_Q4_K, WL_TYPE_Q6_K, 4, 2, true, true>);
#define WL_FUSED_PICK(DN, NORM)                                                                                    \
    switch (ej * 8 + (nbd == 1 ? 1 : nbd == 2 ? 2 : 4)) {                                                           \
        case 9: return reinterpret_cast<const void*>(&k_moe_decode<WL_TYPE_Q4_K, DN, 1, 1, NORM, false>);          \
        case 10: return reinterpret_cast<const void*>(&k_moe_decode<WL_TYPE_Q4_K, DN, 1, 2, NORM, false>);         \
        case 12: return reinterpret_cast<const void*>(&k_moe_decode<WL_TYPE_Q4_K, DN, 1, 4, NORM, false>);         \
        case 17: return reinterpret_cast<const void*>(&k_moe_decode<WL_TYPE_Q4_K, DN, 2, 1, NORM, false>);         \
        case 18: return reinterpret_cast<const void*>(&k_moe_decode<WL_TYPE_Q4_K, DN, 2, 2, NORM, false>);         \
        case 20: return reinterpret_cast<const void*>(&k_moe_decode<WL_TYPE_Q4_K, DN, 2, 4, NORM, false>);         \
        case 33: return reinterpret_cast<const void*>(&k_moe_decode<WL_TYPE_Q4_K, DN, 4, 1, NORM, false>);         \
        case 34: return reinterpret_cast<const void*>(&k_moe_decode<WL_TYPE_Q4_K, DN, 4, 2, NORM, false>);         \
        default: return reinterpret_cast<const void*>(&k_moe_decode<WL_TYPE_Q4_K, DN, 4, 4, NORM, false>);        \
    }
    if (L.down_type == WL_TYPE_Q4_K) {
        if (norm) {
            WL_FUSED_PICK(WL_TYPE_Q4_K, true)
        }
        WL_FUSED_PICK(WL_TYPE_Q4_K, false)
    }
    if (norm) {
        WL_FUSED_PICK(WL_TYPE_Q6_K, true)
    }
    WL_FUSED_PICK(WL_TYPE_Q6_K, false)
#undef WL_FUSED_PICK
}

// Workgroups of the persistent grid for `kernel`: one per CU of the current device, or 0 when this kernel instance
// cannot keep one workgroup per CU resident (its hand-offs need the whole grid resident at once). Cached per device
// and instance.
static int fused_grid(const void* kernel) {
    constexpr int kSlots = 32;
    struct Entry {
        const void* kernel;
        int grid;
    };
    static Entry cache[64][kSlots] = {};
    static std::mutex lock;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    std::lock_guard<std::mutex> guard(lock);
    for (int i = 0; i < kSlots; i++) {
        if (cache[dev][i].kernel == kernel) return cache[dev][i].grid;
        if (!cache[dev][i].kernel) {
            int cus = 0, per_cu = 0;
            if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kFusedThreads, 0) != hipSuccess)
                return 0;
            const int grid = per_cu >= 1 ? (cus < kFusedMaxG ? cus : kFusedMaxG) : 0;
            cache[dev][i] = Entry{kernel, grid};
            return grid;
        }
    }
    return 0;
}

bool fused_eligible(const WlMoeLayer& L, int64_t T) {
    if ((L.flags & WL_MOE_NO_FUSED) || T != 1 || L.n_experts > kFusedMaxE || L.top_k > kFusedMaxK) return false;
    if (L.gate_up_type != WL_TYPE_Q4_K || L.hidden > 8 * kQK) return false;
    const int nbd = L.inter / kQK;
    if (nbd != 1 && nbd != 2 && nbd != 4) return false;
    if (L.shared_gate_up && (L.shared_inter != L.inter || L.shared_gate_up_type != L.gate_up_type ||
                             L.shared_down_type != L.down_type))
        return false;
    if (L.hidden % kOwnRows != 0 || L.hidden > kFusedMaxHidden) return false;
    // one pass per workgroup: an owner group at most, kGateUpTasks per wavefront at most
    const int G = fused_grid(fused_instance(L));
    const int64_t tasks = static_cast<int64_t>(L.top_k) * L.inter;
    return G >= 1 && L.hidden / kOwnRows <= G && tasks <= static_cast<int64_t>(kGateUpTasks) * kFusedWaves * G;
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
    const void* kernel = fused_instance(L);
    a.G = fused_grid(kernel);
    if (a.G < 1) return WL_EINVAL_SHAPE;  // fused_eligible said otherwise: the device changed in between
    const bool starve = (L.flags & WL_MOE_TEST_STARVE) != 0;
    a.spin_limit = starve ? kStarveSpinLimit : kSpinLimit;
    a.silent_wg = starve ? a.G - 1 : -1;
    a.norm_w = L.norm_weight;
    a.norm_eps = L.norm_eps;
    a.residual = (L.flags & WL_MOE_RESIDUAL) ? 1 : 0;
    a.min_w = L.min_expert_weight;
    const WlMoeLayer* nx = L.next;
    // the next layer's phase A maps tasks to workgroups and wavefronts the same way only with the same shapes
    if (nx && nx->hidden == L.hidden && nx->n_experts == L.n_experts && nx->inter == L.inter &&
        nx->top_k == L.top_k && nx->gate_up_type == L.gate_up_type && nx->down_type == L.down_type &&
        (nx->shared_gate_up != nullptr) == (L.shared_gate_up != nullptr) &&
        (!L.shared_gate_up || (nx->shared_inter == L.shared_inter && nx->shared_gate_up_type == L.shared_gate_up_type &&
                               nx->shared_down_type == L.shared_down_type &&
                               (nx->shared_gate != nullptr) == (L.shared_gate != nullptr)))) {
        a.next_router = nx->router;
        a.next_sh_gate = nx->shared_gate_up ? nx->shared_gate : nullptr;
        a.next_sh_gate_up = static_cast<const uint8_t*>(nx->shared_gate_up);
        a.next_sh_down = static_cast<const uint8_t*>(nx->shared_down);
        a.next_norm_w = (nx->flags & WL_MOE_PRE_NORM) ? nx->norm_weight : nullptr;
        if (guess_instance(L) && (nx->flags & WL_MOE_PRE_NORM)) {
            a.guess_router = nx->router;
            a.guess_bias = nx->router_bias;
            a.guess_norm_w = nx->norm_weight;
            a.guess_eps = nx->norm_eps;
        }
    }
    // a guessing call also reads the guess the previous call may have left for it, in its last wavefront when
    // that one has no phase A task
    const int n_a =
        L.n_experts + ((L.shared_gate_up && L.shared_gate) ? 1 : 0) + (L.shared_gate_up ? L.shared_inter : 0);
    a.consume_guess = guess_instance(L) && n_a <= (kFusedWaves - 1) * a.G ? 1 : 0;
    void* args[] = {&a};
    const hipError_t e = hipLaunchKernel(kernel, dim3(static_cast<unsigned>(a.G)), dim3(kFusedThreads), args, 0, s);
    return e == hipSuccess ? WL_OK : static_cast<int>(e);
}

int zero_sync(void* workspace, hipStream_t s) { return zero_words(static_cast<uint32_t*>(workspace), kSyncWords, s); }

int zero_words(uint32_t* p, int n, hipStream_t s) {
    k_zero_words<<<(n + 255) / 256 < 32 ? (n + 255) / 256 : 32, 256, 0, s>>>(p, n);
    return launch_status();
}

}  // namespace wl
