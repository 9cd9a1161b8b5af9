/*
 * willow_hip.h — C ABI of the MI355X (gfx950) MoE-layer library libwillow_hip.so.
 *
 * The library computes willow's Qwen3.6-35B-A3B mixture-of-experts layer straight from GGUF Q4_K / Q6_K blocks
 * held in device memory: router, top-k selection, token->expert grouping, SwiGLU experts, and the weighted
 * combine with the sigmoid-gated shared expert.
 *
 * Conventions (every entry point):
 *   - All pointers are DEVICE pointers (hipMalloc'd, e.g. owned by torch tensors) unless the name ends in _host.
 *   - `stream` is a hipStream_t passed as void*; NULL means the default stream. Work is only enqueued:
 *     no entry point synchronizes, allocates device memory, or keeps mutable global state.
 *   - Return value: 0 = ok; negative = WL_E* argument error detected on the host before anything was enqueued;
 *     positive = the hipError_t reported by the launch. wl_error_string() describes either.
 *   - Quantized weights are GGML blocks in the exact byte layout GGUF stores (type ids as in ggml):
 *       Q4_K (12): 256 values / 144 B = d f16 | dmin f16 | 12 B packed 6-bit scales+mins | 128 B nibbles
 *       Q6_K (14): 256 values / 210 B = ql[128] | qh[64] | int8 scales[16] | d f16
 *     A [rows x k] matrix is rows of k/256 consecutive blocks; `row_stride` is the byte distance between rows.
 *   - Activations are fp32, row-major [tokens x features]; accumulation is fp32.
 */
#ifndef WILLOW_HIP_H
#define WILLOW_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WL_TYPE_Q4_K 12
#define WL_TYPE_Q6_K 14

#define WL_DTYPE_F32 0
#define WL_DTYPE_BF16 1

#define WL_OK 0
#define WL_EINVAL_TYPE -1      /* ggml type is not Q4_K or Q6_K */
#define WL_EINVAL_SHAPE -2     /* k not a multiple of 256, a size <= 0, or a size past the library's limits */
#define WL_EINVAL_NULL -3      /* a required pointer is NULL */
#define WL_EINVAL_ALIGN -4     /* a base pointer or stride is not aligned as the kernels need */
#define WL_EINVAL_TOPK -5      /* top_k < 1, top_k > n_experts, or top_k > WL_MAX_TOPK */
#define WL_EINVAL_WORKSPACE -6 /* workspace NULL or smaller than wl_moe_workspace_bytes() */
#define WL_EINVAL_DTYPE -7     /* output dtype is not WL_DTYPE_F32 / WL_DTYPE_BF16 */
#define WL_EINVAL_COUNT -8     /* too many experts for one batched call */
#define WL_EINVAL_SCRATCH -9   /* wl_moe_layer_noalloc: the call needs more than WL_NOALLOC_SCRATCH_BYTES */
#define WL_ESYNC -10           /* wl_moe_workspace_status: a bounded wait gave up since the last query */
#define WL_EINVAL_OVERLAP -11  /* wl_moe_layer: y overlaps x */
#define WL_EINVAL_SCOPE -12    /* wl_moe_fork_begin with a scope open on the device; wl_moe_fork_end without one on
                                  this stream */

#define WL_MAX_TOPK 16
#define WL_MAX_BATCH_EXPERTS 64 /* experts per wl_gemv_batch / wl_gemv_combine call */

/* Human-readable text for a return code (static storage; never NULL). */
const char* wl_error_string(int code);

/* ABI version of this header: (major << 16) | minor. */
int wl_abi_version(void);

/* Bytes of one row of `k` values stored as `type`, or a negative WL_E* code.
 * Replaces gguf/metal.py:323-325 (row_bytes). */
int64_t wl_row_bytes(int type, int64_t k);

/* out[rows x k] = dequantized w, as fp32 or bf16 (round to nearest even). Bit-exact with the CPU dequantizers.
 * Replaces gguf/metal.py:357-363 (dequantize_gpu) and gguf/quants.py:207-227 (dequantize) for Q4_K / Q6_K. */
int wl_dequant(int type, const void* w, int64_t rows, int64_t k, int64_t row_stride, int out_dtype, void* out,
               void* stream);

/* y[t, r] = sum_k W[r, k] * x[t, k] for t < tokens: x fp32 [tokens x k], y fp32 [tokens x rows].
 * Replaces gguf/metal.py:327-334 (gemv) and the decode branch of GGMLWeight.linear (:401-408). */
int wl_gemv(int type, const void* w, int64_t rows, int64_t k, int64_t row_stride, const float* x, int64_t tokens,
            float* y, void* stream);

/* y[t, r] = sum_k W[r, k] * x[t, k] for t < tokens on the bf16 matrix core: x bf16 [tokens x k] (row stride k),
 * W's exact values rounded to bf16 in registers (never written out), fp32 accumulation, y bf16 [tokens x rows].
 * rows and k multiples of 256; W dense rows (row stride = wl_row_bytes(type, k)), 16-byte aligned for Q4_K.
 * Replaces the prefill branch of GGMLWeight.linear, gguf/metal.py:401-408 (dequantize_gpu to bf16, then a bf16
 * F.linear), without the dequantized copy. */
int wl_linear(int type, const void* w, int64_t rows, int64_t k, const uint16_t* x, int64_t tokens, uint16_t* y,
              void* stream);

/* For each i < n: out[positions_host[i], :] = W_i x, with W_i the [rows x k] matrix at byte offset
 * offsets_host[i] from `base`; x fp32 [k], out fp32 [*, rows]. offsets/positions are HOST arrays (n <=
 * WL_MAX_BATCH_EXPERTS) passed by value to the kernel. Replaces gguf/metal.py:336-343 (gemv_batch). */
int wl_gemv_batch(int type, const void* base, int64_t rows, int64_t k, const int64_t* offsets_host,
                  const int64_t* positions_host, int n, const float* x, float* out, void* stream);

/* y[r] = sum over i < n, in order of i, of weights[perm_host[i]] * (W_i x_i)[r]; x fp32 [n x k], weights fp32 on
 * the device, y fp32 [rows]. fp32 throughout (the Metal kernel rounds to bf16 at every step).
 * Replaces gguf/metal.py:345-355 (gemv_combine). */
int wl_gemv_combine(int type, const void* base, int64_t rows, int64_t k, const int64_t* offsets_host,
                    const int64_t* perm_host, int n, const float* x, const float* weights, float* y, void* stream);

/* One MoE layer's weights, all device pointers (a view into the HBM-resident expert store).
 * Expert e's fused gate_up matrix [2*inter x hidden] (gate rows first, then up rows, as gguf/compiler.py:69-88
 * fuses them) starts at gate_up + e * gate_up_stride; its down matrix [hidden x inter] at down + e * down_stride. */
typedef struct WlMoeLayer {
    const void* gate_up;         /* [n_experts] x [2*inter x hidden] of gate_up_type */
    const void* down;            /* [n_experts] x [hidden x inter] of down_type */
    const float* router;         /* fp32 [n_experts x hidden]  (mlp.gate.weight) */
    const float* router_bias;    /* fp32 [n_experts] or NULL */
    const void* shared_gate_up;  /* [2*shared_inter x hidden] of shared_gate_up_type, or NULL: no shared expert */
    const void* shared_down;     /* [hidden x shared_inter] of shared_down_type */
    const float* shared_gate;    /* fp32 [hidden] (mlp.shared_expert_gate.weight), or NULL: gate of 1 */
    int64_t gate_up_stride;      /* bytes between experts' gate_up matrices */
    int64_t down_stride;         /* bytes between experts' down matrices */
    int32_t gate_up_type, down_type, shared_gate_up_type, shared_down_type;
    int32_t hidden, inter, shared_inter;
    int32_t n_experts, top_k, norm_topk_prob;
    int32_t flags;               /* WL_MOE_* bits; 0 = defaults */
    int32_t reserved;            /* 0 */
    /* The layer the caller runs next, or NULL. When it has the same shapes and types, the batch-1 fused kernel
     * pulls the rows that the next layer's first phase reads whatever the routing (its router rows and shared
     * expert rows) into the GPU's caches while this layer waits on its own exchanges: the next-layer overlap that
     * the reference's guess_next_layer provides for its SSD reads (engines/base.py:392-406). Only read, never
     * written; it must stay valid until the call's work has run. */
    const struct WlMoeLayer* next;
    /* With WL_MOE_PRE_NORM in flags: the layer runs on rms_norm(x) instead of x, as the reference's zero-centered
     * RMSNorm computes it (engines/base.py:27-31: x * rsqrt(mean(x^2) + eps) * (1 + w)), in this fixed fp32 order:
     * s = sum of x_i^2 in the router's order (64-value segments, each a chain of fused multiply-adds from 0 in
     * ascending i, the segments added left to right), inv = 1 / sqrt(s / hidden + eps) (each step rounded once),
     * x_i * inv * (1 + w_i) (rounded after each product; w = 0 when norm_weight is NULL). */
    const float* norm_weight;    /* fp32 [hidden] (post_attention_layernorm.weight) or NULL */
    float norm_eps;
    /* Routed experts whose routing weight is below this are skipped (0 = off): each token keeps its top expert,
     * the others below the threshold are dropped (their ids read -1, their weights 0) and the kept weights are
     * scaled by sum(all k weights) / sum(kept weights), both sums in pick order, so they add up to what the k did:
     * Engine.skip_small_experts (engines/base.py:413-430), applied in the layer as Engine.moe applies it
     * (:463-464), so dropped experts' weights are never read. wl_moe_route returns the routing without it. */
    float min_expert_weight;
} WlMoeLayer;

#define WL_MOE_NO_FUSED 1        /* flags: never take the fused single-kernel decode path */
#define WL_MOE_NO_MFMA 2         /* flags: every expert on the fp32 GEMV kernels at any token count */
#define WL_MOE_FORCE_MFMA 4      /* flags: every expert on the bf16 MFMA GEMMs at any token count (testing) */
#define WL_MOE_PRE_NORM 16       /* flags: run on rms_norm(x) (norm_weight, norm_eps; see WlMoeLayer) */
#define WL_MOE_RESIDUAL 32       /* flags: y = x + MoE(input), the residual add of engines/qwen36/model.py:22; y and
                                    x must not overlap */
#define WL_MOE_GUESS_NEXT 64     /* flags, batch-1 decode with WL_MOE_PRE_NORM: the next call on this workspace is
                                    `next`, on an input derived from this call's x (the model's decoder loop). The
                                    fused kernel then also computes the next layer's router on rms_norm_next(x) (its
                                    norm weight and eps) and leaves it in the workspace; the next call (with this
                                    flag too) takes its top-k as a guess of its experts and pulls their gate_up rows
                                    into the GPU's caches before its routing is known: the early read of
                                    guess_next_layer (engines/base.py:392-406,472-474). Results are unchanged; on
                                    the MI355X it measured slower (1.5 us per layer), so it is off unless asked for.
                                    Ignored unless `next` has the same shapes and WL_MOE_PRE_NORM too, and outside
                                    256 experts of width 512. */
#define WL_MOE_TEST_STARVE 8     /* flags, testing only: in the fused kernel one workgroup withholds its results and
                                    the others' bounded waits give up early, so the call ends with NaN outputs and
                                    the workspace's status word set (the failure wl_moe_workspace_status reports) */

/* Checks a layer description without touching device memory; 0 or a WL_E* code. */
int wl_moe_check(const WlMoeLayer* layer);

/* Bytes of device workspace wl_moe_layer needs for `tokens` tokens (0 on an invalid layer). */
size_t wl_moe_workspace_bytes(const WlMoeLayer* layer, int64_t tokens);

/* The workspace's health since the previous query (NULL: the current device's wl_moe_layer_noalloc scratch).
 * The fused kernel's hand-offs between workgroups need the whole grid resident at once; the library checks that
 * before it launches, and every wait is bounded, so a workgroup that still waits too long gives up, writes NaN for
 * its outputs and sets a status word. The waits of a fork scope (wl_moe_fork_begin) are bounded too; one that
 * gives up sets the word, and until it is cleared the scope's MFMA experts are skipped and every split-plan call
 * in a scope writes NaN for its outputs (those experts' results would be stale).
 * This synchronizes `stream` (and, after a fork-scope wait gave up, the device), reads and clears the word, and
 * returns WL_OK, WL_ESYNC when it was set, or a hipError_t. Not for use under stream capture. */
int wl_moe_workspace_status(void* workspace, size_t workspace_bytes, void* stream);

/* Zeroes the synchronization words at the start of a workspace (the fused decode kernel's per-workgroup epoch
 * counters and epoch-tagged exchange slots, the fork-scope words, the count of top-k workgroups done) with a fill
 * kernel on `stream`. Call once after allocating a workspace, before its first
 * wl_moe_layer; calls keep these words consistent afterwards. Calls that share one workspace must be ordered (one
 * stream): concurrent ones race. */
int wl_moe_workspace_init(void* workspace, size_t workspace_bytes, void* stream);

/* Which path wl_moe_layer takes for `tokens` tokens; -1 on an invalid layer.
 *   1 = one fused persistent kernel (batch-1 decode at Qwen3.6-like shapes);
 *   0 = the multi-kernel path with every expert on the fp32 GEMV kernels (exact weights; up to 8 tokens no expert
 *       can be given more than 8);
 *   2 = the multi-kernel path with each expert placed by its own token count, as the reference's each_expert
 *       hands F.linear only that expert's tokens (engines/base.py:566-571) and GGMLWeight.linear switches at
 *       MAX_TOKENS = 8 (gguf/metal.py:20,404-407): an expert given more than 8 tokens (and the shared expert, which
 *       sees every token) on the bf16 MFMA grouped GEMMs (weights rounded to bf16, bf16 gate/up/SwiGLU/output as
 *       bf16 tensors round them, fp32 accumulation), the others on the fp32 GEMV kernels;
 *   3 = every expert on the MFMA GEMMs (WL_MOE_FORCE_MFMA). */
int wl_moe_plan(const WlMoeLayer* layer, int64_t tokens);

/* Router: logits = x W_r^T (+ bias) in a fixed floating-point order: hidden is cut into segments of 64
 * consecutive values; each segment's partial is a chain of fused multiply-adds in ascending index starting from 0;
 * the partials are added left to right; then the bias is added. Then softmax in fp32, top-k on the logits
 * (largest first, ties -> lower expert id), renormalized when norm_topk_prob. ids int32 [tokens x top_k],
 * weights fp32 [tokens x top_k],
 * logits fp32 [tokens x n_experts] (workspace-sized, required). shared_gate_out fp32 [tokens] =
 * sigmoid(x . shared_gate) when layer->shared_gate != NULL (else may be NULL).
 * Replaces engines/base.py:448 (router linear) + :91-97 (route). */
int wl_moe_route(const WlMoeLayer* layer, const float* x, int64_t tokens, float* logits, int32_t* ids,
                 float* weights, float* shared_gate_out, void* stream);

/* The whole layer: y fp32 [tokens x hidden] = sum over the token's top_k experts, in ascending expert id, of
 * weight * down(silu(gate x) * (up x)), plus sigmoid(x . shared_gate) * shared_down(silu(...) * (...)).
 * ids/weights (optional, may be NULL) receive the routing. Replaces engines/base.py:445-490 (Engine.moe) with its
 * dispatch (:456-467, :492-591) kept on the device: no host synchronization. In the split plan (wl_moe_plan() ==
 * 2), while the experts average fewer than 32 tokens, the experts on the MFMA GEMMs run on a second stream of the
 * device (created on the first such call and kept) beside the GEMV experts on `stream`, forked from and joined back
 * to `stream` by two events; under stream capture both become graph edges. */
int wl_moe_layer(const WlMoeLayer* layer, const float* x, int64_t tokens, float* y, int32_t* ids, float* weights,
                 void* workspace, size_t workspace_bytes, void* stream);

/* A fork scope on `stream` (the current device): wl_moe_fork_begin forks the device's second stream from `stream`
 * once, wl_moe_fork_end joins it back once, and the split-plan wl_moe_layer calls on `stream` in between hand their
 * MFMA experts to the second stream and back through words of their workspaces (set and polled by the kernels)
 * instead of a fork and a join event each. Under stream capture that is two graph edges for a whole decode step of
 * layers instead of two per layer (64 tokens with Zipf(1.1) routing, 40 layers: ~10 us per layer). One scope per
 * device at a time, begun and ended on the same stream, with every call in it issued from one host thread in
 * order; the workspaces must have been prepared by wl_moe_workspace_init. Between the calls the caller may run
 * other work on `stream` (a model's attention), as long as each call's grouping follows the previous call's within
 * the bounded wait (on the order of 100 ms); a wait that gives up is reported by wl_moe_workspace_status. Calls on
 * other streams fork and join per call as outside a scope. No counterpart in the reference, which launches its
 * experts from the host per layer (engines/base.py:515); the callers it is for are step-level graphs of layers
 * (engines/base.py:392-406 overlaps the next layer's expert reads for the same purpose). */
int wl_moe_fork_begin(void* stream);
int wl_moe_fork_end(void* stream);

/* wl_moe_layer with a hipEvent_t recorded on `stream` at every stage boundary: events_host[i] just before stage i,
 * events_host[wl_moe_stage_count()] after the last (so wl_moe_stage_count() + 1 events, none NULL). On the fused
 * path (wl_moe_plan() == 1) stage 0 holds the single fused kernel and the other stages are empty. For per-stage
 * timing with hipEventElapsedTime; do not use under stream capture. No counterpart in the reference, whose only
 * timers are host-side (engines/base.py:384-390). */
int wl_moe_layer_profile(const WlMoeLayer* layer, const float* x, int64_t tokens, float* y, int32_t* ids,
                         float* weights, void* workspace, size_t workspace_bytes, void* stream,
                         void* const* events_host);

/* Number of stages wl_moe_layer runs, and their names ("router", "topk", "sort", "gate_up", "down", "combine"). */
int wl_moe_stage_count(void);
const char* wl_moe_stage_name(int stage);

/* Bytes of the device scratch array wl_moe_layer_noalloc runs on (one copy per GPU, held until the process ends).
 * It covers calls whose wl_moe_workspace_bytes() is up to this size: at Qwen3.6-35B-A3B's shapes (hidden 2048, 256 experts
 * of width 512, top-8, shared expert) up to 128 tokens. */
#define WL_NOALLOC_SCRATCH_BYTES (16u << 20)

/* wl_moe_layer without a workspace and without allocating anything: the workspace is a file-scope device array of
 * WL_NOALLOC_SCRATCH_BYTES on the current device (its address is looked up, and its synchronization words zeroed
 * by a fill kernel on `stream`, on the first call on each device). For callers that cannot allocate: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. Calls that need more than the scratch
 * holds return WL_EINVAL_SCRATCH before enqueuing anything. Every call on a device shares that device's scratch, so
 * calls that overlap on one GPU (different streams, or host threads) race: order them on one stream. The caller
 * still passes x, y and (optionally) ids / weights, as for wl_moe_layer, with the same results.
 * No counterpart in the reference (whose MoE layer allocates per call); it is for callers that cannot allocate. */
int wl_moe_layer_noalloc(const WlMoeLayer* layer, const float* x, int64_t tokens, float* y, int32_t* ids,
                         float* weights, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WILLOW_HIP_H */
