// Shared definitions of the MoE-layer kernels: limits, kernel argument block, workspace layout.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

#include "../../include/willow_hip.h"

namespace wl {

constexpr int kRouterSeg = 64;     // router: values per fused-multiply-add segment
constexpr int kRouterMaxJ = 8;     // router: segments per lane (hidden <= 64 * 32 * 8)
constexpr int kMaxEJ = 16;         // top-k: logits per lane (n_experts <= 1024)
constexpr int kSortChunk = 256;    // grouping: tokens per bitmap chunk
constexpr int kSortWords = kSortChunk / 32;
constexpr int64_t kMaxTokens = 1 << 20;
constexpr int kMoeStages = 6;  // router, topk, sort, gate_up, down, combine
// fused decode kernel limits
constexpr int kFusedMaxK = 8;         // experts per token
constexpr int kFusedMaxE = 256;       // experts
constexpr int kFusedMaxInter = 1024;  // expert width
constexpr int kFusedMaxG = 512;       // workgroups (one per CU)
constexpr int kFusedMaxHidden = 2048; // model width
constexpr int kFlagStride = 32;       // words between workgroups' epoch counters (one 128-byte line each)
// fused decode kernel: its words at the start of the workspace: epoch counters, then the tagged 64-bit values
// that cross workgroups (logits [E+1], shared-expert SwiGLU output [I], routed SwiGLU outputs [k, I])
constexpr int kTagLogits = kFlagStride * kFusedMaxG;
constexpr int kTagHsh = kTagLogits + 2 * (kFusedMaxE + 16);
constexpr int kTagH = kTagHsh + 2 * kFusedMaxInter;
// then the status word: nonzero once a bounded wait gave up (wl_moe_workspace_status); bit 0 a fused-kernel
// workgroup's, bit 1 a fork-scope hand-off's (sticky: while it is set the scope's MFMA kernels do nothing)
constexpr int kStatusWord = kTagH + 2 * kFusedMaxK * kFusedMaxInter;
constexpr uint32_t kStatusFused = 1u, kStatusFork = 2u;
// then, each on a line of its own, the fork-scope hand-off words of a split-plan call (wl_moe_fork_begin): the
// grouping is done (1, set by the grouping, cleared by the second stream's wait), the MFMA experts are done (1, set
// on the second stream, cleared by the grouping), and the MFMA kernels' skip word (1 after a wait gave up)
constexpr int kForkSorted = kStatusWord + kFlagStride;
constexpr int kForkDone = kForkSorted + kFlagStride;
constexpr int kForkSkip = kForkDone + kFlagStride;
// and the count of top-k workgroups done in a call of 2 .. kRouterPartsMaxT tokens (the last one runs the grouping
// and resets it to 0)
constexpr int kTopkDone = kForkSkip + kFlagStride;
// the fused kernel's next-layer guess (WL_MOE_GUESS_NEXT): the next layer's router logits on this layer's input,
// tagged 64-bit values [2][E]: a call with tag t writes set t & 1 and reads the previous call's guess from the
// other set, so no call overwrites a set that a call still running reads
constexpr int kTagGuess = kTopkDone + kFlagStride;
constexpr int kSyncWords = kTagGuess + 2 * 2 * kFusedMaxE;

struct ExpertArgs {
    const uint8_t* gate_up;
    int64_t gate_up_stride;
    const uint8_t* down;
    int64_t down_stride;
    const uint8_t* sh_gate_up;
    const uint8_t* sh_down;
    const float* x;
    int T, H, inter, sh_inter, k;
    // work slots: the routed experts listed in active[1 .. active[0]] (when routed), then the shared expert over
    // all T tokens (when shared_slot); a launch's workgroups loop over (slot, row group) items
    int routed, shared_slot;
    const int32_t* offsets;
    const int32_t* active;
    const int32_t* sorted;
    float* h;
    float* h_sh;
    float* o;
    float* o_sh;
};

constexpr int kTileTokens = 144;             // prefill: tokens per gate_up GEMM tile (9 MFMA token tiles)
constexpr int kDownTileTokens = 128;         // prefill: tokens per down GEMM tile (8 MFMA token tiles)
constexpr int kDownSlabsMax = 4;            // prefill: most 256-row slabs per down workgroup
// An expert given at most this many tokens runs on the fp32 GEMV kernels with exact weights, one given more on the
// bf16 MFMA GEMMs: the reference applies the rule of gguf/metal.py:20,404-407 to each expert's own tokens
// (engines/base.py:566-571).
constexpr int kGemvMaxTokens = 8;
constexpr uint32_t kPosBf16 = 0x80000000u;  // position flag: the pair's expert output is bf16 (an MFMA expert)
constexpr int kTiledRouterMinTokens = 2048;  // router as a tiled kernel from this many tokens
constexpr int kRouterPartsMaxT = 64;         // wl_moe_layer's router for 2 .. this many tokens: per-segment partials

struct PrefillArgs {
    const uint8_t* gate_up;
    int64_t gate_up_stride;
    const uint8_t* down;
    int64_t down_stride;
    const uint8_t* sh_gate_up;
    const uint8_t* sh_down;
    const uint16_t* xb;      // [T, H] bf16
    const int32_t* sorted;   // [T*k] pair id by sorted position
    const int4* tiles;       // gate_up tiles: (expert or E for the shared expert, first position / token, count)
    const int32_t* n_tiles;
    const int4* tiles_down;  // down tiles, the same of at most kDownTileTokens tokens
    const int32_t* n_tiles_down;
    uint16_t* h16;           // [T*k, inter] bf16 by sorted position
    uint16_t* h_sh16;        // [T, shared_inter] bf16
    uint16_t* o16;           // bf16 by sorted position, row pos at o16 + pos * ldo (the reference's bf16 F.linear output)
    int64_t ldo;             // o16's row stride in values
    uint16_t* o_sh16;        // [T, H] bf16
    int H, inter, sh_inter, E, k;
    int nslab_gate_up;       // 128-row slabs of the widest intermediate dim
    int down_slabs;          // 256-row slabs per down workgroup
    int dense_tokens;        // > 0: k_gemm_down runs one matrix (down) over this many tokens, tiles implied
    const uint32_t* skip;    // in a fork scope: nonzero when the wait for the grouping gave up (the kernel returns)
};

struct Workspace {
    uint32_t* sync;     // [kSyncWords] the fused kernel's epoch counters and tagged exchange slots (zeroed once)
    float* logits;      // [T, E + 1]
    float* sg;          // [T]      sigmoid(shared gate)
    int32_t* ids;       // [T, k]
    float* wts;         // [T, k]
    int32_t* crank;     // [T, k]   each slot's rank among the token's expert ids (ascending)
    int32_t* rank;      // [T*k]    rank of a pair within its chunk and expert
    int32_t* hist;      // [chunks, E]
    int32_t* offsets;   // [E+1]
    int32_t* active;    // [1+E]
    int32_t* sorted;    // [T*k]
    uint2* picks;       // [T, k]   the combine's table: (position | kPosBf16, weight bits) in ascending expert id
    float* h;           // [T*k, inter]   by sorted position
    float* o;           // [T*k, hidden]  by sorted position
    float* h_sh;        // [T, shared_inter]
    float* o_sh;        // [T, hidden]
    // prefill (MFMA) path only
    uint16_t* xb;       // [T, hidden] bf16
    int4* tiles;        // [max_tiles(kTileTokens)]
    int4* tiles_down;   // [max_tiles(kDownTileTokens)]
    int32_t* n_tiles;   // [2]: gate_up tiles, down tiles
    uint16_t* h16;      // [T*k, inter] bf16
    uint16_t* h_sh16;   // [T, shared_inter] bf16
    float* xn;          // [T, hidden] the normalized input (WL_MOE_PRE_NORM)
    float* parts;       // [hidden / kRouterSeg, T, E + 1] the router's segment partials (2 .. kRouterPartsMaxT tokens)
    size_t bytes;
};

Workspace carve(const WlMoeLayer& L, int64_t T, void* base);
int check_layer(const WlMoeLayer* L);
bool fused_eligible(const WlMoeLayer& L, int64_t T);
int launch_fused(const WlMoeLayer& L, const float* x, float* y, int32_t* ids, float* wts, const Workspace& w,
                 hipStream_t s);
int zero_sync(void* workspace, hipStream_t s);
int zero_words(uint32_t* p, int n, hipStream_t s);  // a fill kernel (no hipMemsetAsync: graph-capture safe)
// How the routed experts of a T-token call are run: kPlanGemv (every expert on the fp32 GEMV kernels), kPlanSplit
// (experts with more than kGemvMaxTokens tokens on the MFMA GEMMs, the rest on GEMV), kPlanMfma (every expert on
// the MFMA GEMMs; WL_MOE_FORCE_MFMA). The fused single-kernel decode is chosen before this (fused_eligible).
enum ExpertPlan { kPlanGemv = 0, kPlanSplit = 2, kPlanMfma = 3 };
ExpertPlan expert_plan(const WlMoeLayer& L, int64_t T);
// Whether the layer's shapes and types let the MFMA GEMMs run at T tokens.
bool prefill_eligible(const WlMoeLayer& L, int64_t T);
// The most pairs an expert may have and still run on the GEMV kernels under `plan`.
inline int plan_gemv_max(ExpertPlan plan) {
    return plan == kPlanMfma ? 0 : plan == kPlanSplit ? kGemvMaxTokens : 0x7FFFFFFF;
}
int max_tiles(const WlMoeLayer& L, int64_t T, int cap, int gemv_max);
int launch_router_tiled(const WlMoeLayer& L, const float* x, int64_t T, float* logits, float* sg, uint16_t* xb,
                        hipStream_t s);
// with_gemv: the call also has GEMV experts (a split plan), which may run beside this launch on a second stream;
// the K-split gate_up kernel then splits K 2 ways instead of 4 (64 KiB of LDS per workgroup instead of 128, which
// kept the GEMV workgroups off its CUs). The choice depends on the plan alone, so every entry point runs the same
// kernels on the same call.
int launch_mfma_gate_up(const WlMoeLayer& L, int64_t T, const Workspace& w, int gemv_max, bool with_gemv,
                        const uint32_t* skip, hipStream_t s);
// skip (nullable): the fork-scope skip word, which the kernels read first (a nonzero value: they do nothing)
int launch_mfma_down(const WlMoeLayer& L, int64_t T, const Workspace& w, int gemv_max, const uint32_t* skip,
                     hipStream_t s);
int launch_linear(int type, const uint8_t* w, int rows, int k, const uint16_t* x, int64_t T, uint16_t* y,
                  hipStream_t s);

}  // namespace wl
