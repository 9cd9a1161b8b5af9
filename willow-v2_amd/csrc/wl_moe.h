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
constexpr int kSyncWords = kTagH + 2 * kFusedMaxK * kFusedMaxInter;

struct ExpertArgs {
    const uint8_t* gate_up;
    int64_t gate_up_stride;
    const uint8_t* down;
    int64_t down_stride;
    const uint8_t* sh_gate_up;
    const uint8_t* sh_down;
    const float* x;
    int T, H, inter, sh_inter, k;
    int n_routed;  // grid slots [0, n_routed) are routed experts; slot n_routed (if launched) the shared expert
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
constexpr int kGemvMaxTokens = 8;  // fp32 GEMV experts up to this many tokens, bf16 MFMA GEMMs above (gguf/metal.py:20)
constexpr int kTiledRouterMinTokens = 2048;  // router as a tiled kernel from this many tokens

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
    uint16_t* o16;           // [T*k, H] bf16 by sorted position (the reference's bf16 F.linear output)
    uint16_t* o_sh16;        // [T, H] bf16
    int H, inter, sh_inter, E, k;
    int nslab_gate_up;       // 128-row slabs of the widest intermediate dim
    int down_slabs;          // 256-row slabs per down workgroup
    int dense_tokens;        // > 0: k_gemm_down runs one matrix (down) over this many tokens, tiles implied
};

struct Workspace {
    uint32_t* sync;     // [kSyncWords] the fused kernel's epoch counters and tagged exchange slots (zeroed once)
    float* logits;      // [T, E + 1]
    float* sg;          // [T]      sigmoid(shared gate)
    int32_t* ids;       // [T, k]
    float* wts;         // [T, k]
    int32_t* corder;    // [T, k]   slots in ascending expert id
    int32_t* rank;      // [T*k]    rank of a pair within its chunk and expert
    int32_t* hist;      // [chunks, E]
    int32_t* offsets;   // [E+1]
    int32_t* active;    // [1+E]
    int32_t* sorted;    // [T*k]
    int32_t* pair_pos;  // [T*k]
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
    size_t bytes;
};

Workspace carve(const WlMoeLayer& L, int64_t T, void* base);
int check_layer(const WlMoeLayer* L);
bool fused_eligible(const WlMoeLayer& L, int64_t T);
int launch_fused(const WlMoeLayer& L, const float* x, float* y, int32_t* ids, float* wts, const Workspace& w,
                 hipStream_t s);
int zero_sync(void* workspace, hipStream_t s);
bool prefill_eligible(const WlMoeLayer& L, int64_t T);
int max_tiles(const WlMoeLayer& L, int64_t T, int cap);
int launch_router_tiled(const WlMoeLayer& L, const float* x, int64_t T, float* logits, float* sg, uint16_t* xb,
                        hipStream_t s);
int launch_prefill_experts(const WlMoeLayer& L, const float* x, int64_t T, const Workspace& w, hipStream_t s);
int launch_linear(int type, const uint8_t* w, int rows, int k, const uint16_t* x, int64_t T, uint16_t* y,
                  hipStream_t s);

}  // namespace wl
