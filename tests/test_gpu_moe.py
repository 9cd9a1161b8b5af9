"""GPU parity of the fused MoE layer (wl_moe_route, wl_moe_layer) against the CPU oracle: expert ids exact, routing
weights to fp32 rounding, outputs within max|y - y_ref| / max|y_ref| <= 2e-3 (fp32 accumulation)."""
import numpy as np
import pytest
import torch

from gguf import synth
from oracle import cref, moe_ref

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.fixture(scope="module")
def c2(hip, layer_c2):
    return hip.MoELayer.from_host(layer_c2)


def run_layer(hip, layer, x):
    T = x.shape[0]
    ids = torch.empty(T, layer.top_k, dtype=torch.int32, device="cuda")
    wts = torch.empty(T, layer.top_k, dtype=torch.float32, device="cuda")
    y = layer(torch.from_numpy(x).cuda(), ids=ids, weights=wts)
    torch.cuda.synchronize()
    return y.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()


def check_layer(hip, layer, lw, x, label):
    if layer.plan(x.shape[0]) in ("split", "mfma"):  # experts on the bf16 MFMA GEMMs: the bf16 chain
        return check_prefill(hip, layer, lw, x, label)
    print(f"[moe] {label}: T={x.shape[0]}", flush=True)
    y, ids, wts = run_layer(hip, layer, x)
    y_ref, ids_ref, wts_ref, _ = moe_ref.layer(x, lw, return_routing=True)
    np.testing.assert_array_equal(ids, ids_ref)
    np.testing.assert_allclose(wts, wts_ref, rtol=2e-6, atol=1e-7)
    err = moe_ref.rel_err(y, y_ref)
    print(f"[moe] {label}: rel err {err:.2e}", flush=True)
    assert err < TOL
    return err


@pytest.mark.parametrize("T", [1, 2, 9, 64, 300, 1000, 2100])
def test_route_c2(hip, c2, layer_c2, T):
    """Routing bits at token counts that take each router kernel (one token, the small-batch kernel, the
    matrix-core kernel from 2048 tokens): logits bit-exact with the CPU replay of the fixed FMA order."""
    x = synth.tokens(2, T)
    wts, ids, sg, lg = c2.route(torch.from_numpy(x).cuda(), return_logits=True)
    logits = cref.router_logits(x, layer_c2["router"])
    np.testing.assert_array_equal(lg.cpu().numpy().view(np.uint32), logits.view(np.uint32))
    w_ref, ids_ref = moe_ref.route(logits, 8, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(wts.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-7)
    z = cref.router_logits(x, layer_c2["shared_gate"][None])[:, 0]
    np.testing.assert_allclose(sg.cpu().numpy(), moe_ref.sigmoid(z), rtol=1e-6)


@pytest.mark.parametrize("experts,shared_gate,T", [(40, True, 2085), (64, False, 2050), (72, True, 2049)])
def test_route_variants(hip, experts, shared_gate, T):
    """The matrix-core router on ragged shapes: expert counts that are not a multiple of its 64-row tiles (the
    shared gate then rides in the last tile), token counts that are not a multiple of its token tiles, a bias."""
    lw = synth.moe_layer(80, hidden=1024, inter=256, shared_inter=256, experts=experts, top_k=4, zipf_alpha=1.1)
    if not shared_gate:
        lw["shared_gate"] = None
    layer = hip.MoELayer.from_host(lw)
    x = synth.tokens(81, T, 1024)
    wts, ids, sg, lg = layer.route(torch.from_numpy(x).cuda(), return_logits=True)
    logits = cref.router_logits(x, lw["router"], lw["router_bias"])
    np.testing.assert_array_equal(lg.cpu().numpy().view(np.uint32), logits.view(np.uint32))
    w_ref, ids_ref = moe_ref.route(logits, 4, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(wts.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-7)
    if shared_gate:
        z = cref.router_logits(x, lw["shared_gate"][None])[:, 0]
        np.testing.assert_allclose(sg.cpu().numpy(), moe_ref.sigmoid(z), rtol=1e-6)
    else:
        assert sg is None


def test_layer_c2_decode_b1(hip, c2, layer_c2):
    """The full Qwen3.6-35B-A3B-shaped layer at batch 1 (seed 1 weights, x seed 2)."""
    check_layer(hip, c2, layer_c2, synth.tokens(2, 1), "c2 b=1")


def test_fused_matches_multi_kernel(hip, c2, layer_c2):
    """Batch-1 decode runs as one fused persistent kernel; it must give the multi-kernel path's routing bits and
    its outputs up to the compiler's multiply-add contraction in the combine (~1e-6)."""
    multi = hip.MoELayer.from_host(layer_c2, fused=False)
    assert c2.plan(1) == "fused" and multi.plan(1) == "gemv" and c2.plan(2) == "gemv" and c2.plan(8) == "gemv"
    assert c2.plan(9) == "split" and c2.plan(600) == "split"
    for seed in range(5):
        x = synth.tokens(200 + seed, 1)
        y_f, ids_f, w_f = run_layer(hip, c2, x)
        y_m, ids_m, w_m = run_layer(hip, multi, x)
        np.testing.assert_array_equal(ids_f, ids_m)
        np.testing.assert_array_equal(w_f, w_m)
        assert moe_ref.rel_err(y_f, y_m) < 1e-5


@pytest.mark.parametrize("case", ["tie16", "tie_boundary", "nan_row"])
def test_topk_ties_and_nan(hip, case):
    """Selection on exactly tied and NaN logits, for the fused kernel's top-k (one token) and the multi-kernel path's
    (wave_topk): ties go to the lower expert id, NaN ranks as -inf, as the oracle's route does (engines/base.py:91-97
    with a fixed tie rule). tie16: 16 experts share the largest logit, 8 are picked; tie_boundary: 3 experts tie
    across the 8th/9th place; nan_row: one router row is NaN."""
    lw = dict(synth.moe_layer(31, experts=64, top_k=8))
    router = lw["router"].copy()
    x = synth.tokens(32, 1)
    base = cref.router_logits(x, router)[0]
    order = np.argsort(-base, kind="stable")
    if case == "tie16":
        router[order[:16]] = router[order[0]]  # 16 identical rows: identical logits, the largest
    elif case == "tie_boundary":
        router[order[7:10]] = router[order[7]]  # the 8th, 9th and 10th tie
    else:
        router[order[0]] = np.nan  # the would-be top expert
    lw["router"] = router
    logits = cref.router_logits(x, router)
    _, ids_ref = moe_ref.route(logits, 8, True)
    for fused in (True, False):
        layer = hip.MoELayer.from_host(lw, fused=fused)
        assert layer.plan(1) == ("fused" if fused else "gemv")
        print(f"[moe] topk {case} fused={fused}", flush=True)
        y, ids, wts = run_layer(hip, layer, x)
        np.testing.assert_array_equal(ids, ids_ref)
        assert np.isfinite(y).all()  # a NaN logit ranks and weighs as -inf: no NaN reaches the output


@pytest.mark.parametrize("T,fused", [(1, True), (1, False), (9, True), (64, True), (300, True)])
def test_skip_small_experts(hip, layer_c2, T, fused):
    """min_expert_weight (Engine.skip_small_experts, engines/base.py:413-430, applied in Engine.moe at :463-464):
    the layer's ids and weights equal the oracle's skip_small of its routing (a dropped pick has id -1 and weight 0,
    the kept weights are scaled back to the sum of the k) and its output the oracle's layer on the kept experts
    only, each expert placed by its kept tokens. One token in the fused kernel and on the multi-kernel path, 9 and
    64 tokens (top-k over the router's partials, split plan), 300 tokens (two grouping chunks)."""
    thr = 0.12
    layer = hip.MoELayer.from_host(layer_c2, fused=fused, min_expert_weight=thr)
    x = synth.tokens(400 + T, T)
    plan = layer.plan(T)
    chain = "split" if plan in ("split", "mfma") else "fp32"
    print(f"[moe] skip_small T={T} plan={plan}", flush=True)
    y, ids, wts = run_layer(hip, layer, x)
    y_ref, ids_ref, wts_ref, _ = moe_ref.layer(x, layer_c2, chain=chain, return_routing=True,
                                               dtype=np.float64 if chain == "split" else np.float32,
                                               min_expert_weight=thr)
    np.testing.assert_array_equal(ids, ids_ref)
    np.testing.assert_allclose(wts, wts_ref, rtol=4e-6, atol=1e-7)
    assert (ids == -1).any() and (ids[:, 0] >= 0).all()  # some picks dropped, never a token's top one
    err = moe_ref.rel_err(y, y_ref)
    print(f"[moe] skip_small T={T}: rel err {err:.2e}", flush=True)
    assert err < TOL
    # the routing call (route(), engines/base.py:91-97) is unaffected by the threshold
    w_r, ids_r, _, _ = layer.route(torch.from_numpy(x).cuda(), return_logits=True)
    assert (ids_r.cpu().numpy() >= 0).all()


def test_fused_back_to_back(hip, c2, layer_c2):
    """Many fused calls in a row on one workspace (the grid barrier's words must reset each time), checked
    against the oracle at the end."""
    x = synth.tokens(300, 16)
    xs = torch.from_numpy(x).cuda()
    ys = torch.empty(16, 2048, device="cuda")
    ws = c2.workspace(1)
    for i in range(16):
        c2(xs[i:i + 1], out=ys[i:i + 1], workspace=ws)
    torch.cuda.synchronize()
    y_ref = moe_ref.layer(x, layer_c2)
    assert np.isfinite(ys.cpu().numpy()).all()
    assert moe_ref.rel_err(ys.cpu().numpy(), y_ref) < TOL


def test_layer_c2_repeatable(hip, c2, layer_c2):
    x = synth.tokens(3, 4)
    a = run_layer(hip, c2, x)[0]
    b = run_layer(hip, c2, x)[0]
    np.testing.assert_array_equal(a, b)  # no atomics in the sums: bit-identical reruns


@pytest.fixture(scope="module")
def c2_fp32(hip, layer_c2):
    """The same layer pinned to the fp32 expert kernels at every token count."""
    return hip.MoELayer.from_host(layer_c2, mfma="never")


@pytest.mark.parametrize("T", [2, 7, 8, 9, 64, 256, 257])
def test_layer_c2_batches(hip, c2, layer_c2, T):
    """Up to 8 tokens every expert on the fp32 GEMV kernels; from 9 each expert by its own token count (the shared
    expert and experts with more than 8 tokens on the bf16 MFMA GEMMs, checked against the oracle's split chain).
    At 9 and 64 tokens nearly every routed expert stays on GEMV; at 256 and 257 (8 pairs per expert on average)
    both classes are large. 256 and 257 also sit either side of the down GEMM's switch from two 256-row slabs per
    workgroup to the tile-count rule."""
    check_layer(hip, c2, layer_c2, synth.tokens(100 + T, T), f"c2 b={T}")


@pytest.mark.parametrize("T", [64, 300])
def test_layer_c2_fp32_experts(hip, c2_fp32, layer_c2, T):
    """The fp32 expert kernels at batch sizes the default plan gives to the MFMA path."""
    assert c2_fp32.plan(T) == "gemv"
    check_layer(hip, c2_fp32, layer_c2, synth.tokens(100 + T, T), f"c2 fp32 b={T}")


def test_layer_multi_chunk_sort(hip, c2, layer_c2):
    """300 tokens: the token->expert grouping runs as per-chunk histograms + scan + scatter."""
    check_layer(hip, c2, layer_c2, synth.tokens(300, 300), "c2 T=300")


@pytest.mark.parametrize("case", ["c2", "zipf_bias", "no_shared_gate", "experts_40"])
def test_layer_routing_equals_route(hip, layer_c2, case):
    """wl_moe_layer routes 2 to 64 tokens with the K-split router (k_router_parts: per-segment partials from 4x the
    workgroups, added in segment order by k_topk_parts); its ids and routing weights equal wl_moe_route's (the
    one-kernel router, then k_topk) bit for bit, so the logits are the same bits: at 1 and 65 tokens, either side of
    its range, too."""
    if case == "c2":
        lw = layer_c2
    elif case == "zipf_bias":  # a router bias (log-Zipf)
        lw = synth.moe_layer(3, zipf_alpha=1.1)
    elif case == "no_shared_gate":
        lw = dict(synth.moe_layer(7, experts=64, top_k=8))
        lw["shared_gate"] = None
    else:  # rows not a multiple of 16
        lw = synth.moe_layer(8, experts=40, top_k=4)
    layer = hip.MoELayer.from_host(lw)
    for T in (1, 2, 9, 33, 64, 65):
        x = synth.tokens(60 + T, T)
        _, ids, wts = run_layer(hip, layer, x)
        w_ref, ids_ref, _ = layer.route(torch.from_numpy(x).cuda())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ids, ids_ref.cpu().numpy(), err_msg=f"{case} T={T}")
        np.testing.assert_array_equal(wts.view(np.uint32), w_ref.cpu().numpy().view(np.uint32),
                                      err_msg=f"{case} T={T}")


def test_layer_zipf_b64(hip):
    """The batched-decode case: 64 tokens, expert popularity Zipf(1.1)-shaped through a router bias."""
    lw = synth.moe_layer(3, zipf_alpha=1.1)
    layer = hip.MoELayer.from_host(lw)
    x = synth.tokens(33, 64)
    assert layer.plan(64) == "split"
    check_layer(hip, layer, lw, x, "zipf b=64")
    check_layer(hip, hip.MoELayer.from_host(lw, mfma="never"), lw, x, "zipf b=64 fp32")
    _, ids, _ = run_layer(hip, layer, x)
    counts = np.bincount(ids.reshape(-1), minlength=256)
    assert counts.max() >= 32  # a hot expert sees at least half the tokens
    assert (counts > 0).sum() < 256
    # both classes present: experts above 8 tokens on the MFMA GEMMs, the rest on GEMV
    assert (counts > 8).sum() >= 4 and ((counts > 0) & (counts <= 8)).sum() >= 4


@pytest.mark.parametrize("variant", ["no_shared", "no_shared_gate", "q4k_down", "q6k_gate_up", "topk1",
                                     "few_experts", "hidden_1024", "inter_256_no_norm", "inter_1024",
                                     "inter_1024_no_shared"])
def test_layer_variants(hip, variant):
    kw = dict(hidden=1024, inter=512, shared_inter=512, experts=32, top_k=4)
    if variant == "q4k_down":
        kw["down_type"] = "Q4_K"
    if variant == "q6k_gate_up":  # Q6_K gate_up: the fused decode kernel takes only Q4_K, so 1 token is multi-kernel
        kw["gate_up_type"] = "Q6_K"
    if variant == "topk1":
        kw["top_k"] = 1
    if variant == "few_experts":
        kw.update(experts=4, top_k=4)
    if variant == "hidden_1024":
        kw.update(hidden=1024, experts=64, top_k=8)
    if variant == "inter_256_no_norm":
        kw.update(inter=256, shared_inter=768)
    if variant.startswith("inter_1024"):
        # 1024-wide experts: the fused kernel's four-block down rows; with the shared expert the routing gather
        # takes 65 logits + 1024 shared values, more than two per thread (its three-slot form)
        kw.update(inter=1024, shared_inter=1024, experts=64, top_k=4)
    lw = synth.moe_layer(50, **kw)
    if variant in ("no_shared", "inter_1024_no_shared"):
        lw["shared_gate_up"] = lw["shared_down"] = lw["shared_gate"] = None
    if variant == "no_shared_gate":
        lw["shared_gate"] = None
    if variant == "inter_256_no_norm":
        lw["norm_topk_prob"] = False
    layer = hip.MoELayer.from_host(lw)
    if variant == "q6k_gate_up":
        assert layer.plan(1) == "gemv"
    if variant.startswith("inter_1024"):
        assert layer.plan(1) == "fused"
    for T in (1, 5):
        check_layer(hip, layer, lw, synth.tokens(51 + T, T, kw["hidden"]), f"{variant}")


def check_prefill(hip, layer, lw, x, label, tol=TOL):
    """A plan with MFMA experts against the oracle's chain for that plan ("split": the reference's per-expert
    rule; "mfma": every expert on the bf16 chain of engines/base.py:568-570 with bf16 tensors), and against the
    all-fp32 oracle within bf16 accuracy. The chain oracle accumulates in float64, so each bf16 rounding applies to
    the exactly rounded fp32 sum: with numpy's own fp32 summation order the oracle's output can sit one bf16 ulp
    (3.9e-3 relative) away from the exact chain at a token whose value lies on a rounding boundary, a flip no
    accumulation order is entitled to more than another."""
    chain = {"split": "split", "mfma": "bf16"}[layer.plan(x.shape[0])]
    print(f"[prefill] {label}: T={x.shape[0]} chain={chain}", flush=True)
    y, ids, wts = run_layer(hip, layer, x)
    y_b, ids_ref, wts_ref, _ = moe_ref.layer(x, lw, chain=chain, return_routing=True, dtype=np.float64)
    np.testing.assert_array_equal(ids, ids_ref)
    np.testing.assert_allclose(wts, wts_ref, rtol=2e-6, atol=1e-7)
    err = moe_ref.rel_err(y, y_b)
    err32 = moe_ref.rel_err(y, moe_ref.layer(x, lw))
    print(f"[prefill] {label}: rel err {err:.2e} vs the {chain} oracle, {err32:.2e} vs the fp32 oracle", flush=True)
    assert err < tol
    assert err32 < 2e-2
    return err


def test_prefill_mfma_c2(hip, c2, layer_c2):
    """600 tokens through the full layer: tiled router, grouped bf16 MFMA GEMMs for ~19 tokens per expert."""
    assert c2.plan(600) == "split"
    check_prefill(hip, c2, layer_c2, synth.tokens(600, 600), "c2 T=600")


def test_prefill_full_chunk_sampled(hip, c2, layer_c2):
    """The headline prefill chunk itself, 4096 tokens through the full-shape layer (tiled router, 16-chunk
    grouping, full 144-token tiles): every token's expert ids and weights against the oracle, and the outputs of 24
    sampled tokens, since a token's output depends on that token alone."""
    from oracle import cref
    T = 4096
    x = synth.tokens(4096, T)
    y, ids, wts = run_layer(hip, c2, x)
    logits = cref.router_logits(x, layer_c2["router"], layer_c2.get("router_bias"))
    wts_ref, ids_ref = moe_ref.route(logits, layer_c2["top_k"], layer_c2["norm_topk_prob"])
    np.testing.assert_array_equal(ids, ids_ref)
    np.testing.assert_allclose(wts, wts_ref, rtol=2e-6, atol=1e-7)
    pick = np.sort(np.random.default_rng(5).choice(T, 24, replace=False))
    counts = np.bincount(ids_ref.reshape(-1), minlength=layer_c2["experts"])
    y_ref = moe_ref.layer(x[pick], layer_c2, chain="split", counts=counts, layer_tokens=T, dtype=np.float64)
    err = moe_ref.rel_err(y[pick], y_ref)
    print(f"[prefill] full chunk T=4096, 24 sampled tokens: rel err {err:.2e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("variant", ["base", "q4k_down", "q6k_gate_up", "no_shared", "inter_256", "partial_tiles"])
def test_prefill_mfma_variants(hip, variant):
    kw = dict(hidden=1024, inter=512, shared_inter=512, experts=16, top_k=4)
    if variant == "q4k_down":
        kw["down_type"] = "Q4_K"
    if variant == "q6k_gate_up":
        kw["gate_up_type"] = "Q6_K"
    if variant == "inter_256":
        kw.update(inter=256, shared_inter=256)
    lw = synth.moe_layer(70, **kw)
    if variant in ("no_shared", "inter_1024_no_shared"):
        lw["shared_gate_up"] = lw["shared_down"] = lw["shared_gate"] = None
    layer = hip.MoELayer.from_host(lw, mfma="always")
    T = 37 if variant == "partial_tiles" else 300  # 300 * 4 / 16 = 75 tokens per expert on average
    check_prefill(hip, layer, lw, synth.tokens(71, T, kw["hidden"]), variant)


@pytest.mark.parametrize("T", [12, 64])
def test_mfma_small_batches_k_split(hip, layer_c2, T):
    """At most 64 tokens with every expert on the MFMA GEMMs (the full-shape layer): the K-split kernels, gate_up's
    K over 4 wavefronts of a workgroup and down's over 2, whose partial sums are added in a fixed order through LDS.
    12 tokens: every tile holds at most 16 tokens (one token tile); 64: tiles of up to 64 tokens, the shared
    expert's among them. A second run gives the same bits."""
    layer = hip.MoELayer.from_host(layer_c2, mfma="always")
    assert layer.plan(T) == "mfma"
    x = synth.tokens(900 + T, T)
    check_prefill(hip, layer, layer_c2, x, f"c2 mfma b={T}")
    y1, _, _ = run_layer(hip, layer, x)
    y2, _, _ = run_layer(hip, layer, x)
    np.testing.assert_array_equal(y1.view(np.uint32), y2.view(np.uint32))


def test_fused_give_up_is_reported(hip, layer_c2):
    """The fused kernel's hand-offs need every workgroup resident; a wait that runs out gives up rather than hang.
    Forced from the host (WL_MOE_TEST_STARVE: one workgroup withholds its results, the other waits give up after
    a short bounded spin, so every workgroup still exits): the outputs hold NaN, wl_moe_workspace_status reports
    ESYNC once and clears it, and the next ordinary call on the same workspace is correct."""
    layer = hip.MoELayer.from_host(layer_c2)
    starved = hip.MoELayer.from_host(layer_c2)
    starved.struct.flags |= hip.MOE_TEST_STARVE
    assert layer.plan(1) == "fused" and starved.plan(1) == "fused"
    ws = layer.workspace(1)
    x = synth.tokens(40, 1)
    xt = torch.from_numpy(x).cuda()
    assert layer.status(ws) == 0
    y_bad = starved(xt, workspace=ws).cpu().numpy()
    assert np.isnan(y_bad).any()
    assert layer.status(ws) == hip.ESYNC
    assert layer.status(ws) == 0  # reported once, then cleared
    y = layer(xt, workspace=ws).cpu().numpy()
    assert layer.status(ws) == 0
    assert np.isfinite(y).all()
    assert moe_ref.rel_err(y, moe_ref.layer(x, layer_c2)) < TOL


# The fused kernel's guess logits in a workspace: two sets of 256 64-bit words (call tag << 32 | float bits) at this
# 32-bit word offset, after the per-workgroup epoch lines (32 words x 512), the tagged logits (2 x 272), h_shared
# (2 x 1024), h (2 x 8 x 1024), the status line and the four fork / top-k lines (32 words each).
GUESS_WORD = 32 * 512 + 2 * 272 + 2 * 1024 + 2 * 8 * 1024 + 5 * 32


def latest_guess(ws):
    """The guess logits of the most recent call that left one: the set whose 256 tags are that call's."""
    words = ws[4 * GUESS_WORD:4 * (GUESS_WORD + 2 * 2 * 256)].cpu().numpy().view(np.uint32).reshape(2, 256, 2)
    tags = words[:, :, 1]
    s = int(np.argmax(tags[:, 0]))
    assert (tags[s] == tags[s, 0]).all() and tags[s, 0] > 0
    return words[s, :, 0].view(np.float32).copy()


def test_next_layer_guess(hip, c2, layer_c2):
    """WL_MOE_GUESS_NEXT, the early read of guess_next_layer (engines/base.py:392-406,472-474): three chained
    decoder steps x_{l+1} = x_l + MoE_l(rms_norm_l(x_l)) of the full-shape layer (a different norm weight per
    layer, so each routes differently). The guess only pulls rows into the caches, so every output and routing
    equals the chain without it bit for bit. The guess itself: the next layer's logits the kernel leaves in its
    workspace equal the oracle's fixed-order router on rms_norm_{l+1}(x_l) (the reference's router_guess_input,
    engines/qwen36/model.py:30-31) bit for bit."""
    rng = np.random.default_rng(17)
    norm_w = [(rng.standard_normal(2048) * 0.1).astype(np.float32) for _ in range(3)]
    x0 = synth.tokens(77, 1) * np.float32(2.0)
    runs = {}
    for guess in (False, True):
        chain = [c2.with_norm(torch.from_numpy(w).cuda()) for w in norm_w]
        for l in range(2):
            chain[l].set_next(chain[l + 1], guess=guess)
        ws = chain[0].workspace(1)
        x = torch.from_numpy(x0).cuda()
        xs, ys, idss, guess_logits = [], [], [], []
        for l, layer in enumerate(chain):
            print(f"[moe] next-layer guess={guess}: layer {l}", flush=True)
            ids = torch.empty(1, 8, dtype=torch.int32, device="cuda")
            y = layer(x, ids=ids, workspace=ws)
            torch.cuda.synchronize()
            if guess and l < 2:
                guess_logits.append(latest_guess(ws))
            xs.append(x.cpu().numpy())
            ys.append(y.cpu().numpy())
            idss.append(ids.cpu().numpy())
            x = y
        assert layer.status(ws) == 0
        runs[guess] = (xs, ys, idss, guess_logits)
    for l in range(3):
        np.testing.assert_array_equal(runs[True][2][l], runs[False][2][l])
        np.testing.assert_array_equal(runs[True][1][l].view(np.uint32), runs[False][1][l].view(np.uint32))
    xs, ys, _, guess_logits = runs[True]
    for l in range(2):
        want = cref.router_logits(moe_ref.rms_norm(xs[l], norm_w[l + 1], 1e-6), layer_c2["router"])[0]
        np.testing.assert_array_equal(guess_logits[l].view(np.uint32), want.view(np.uint32))
    # the chain itself against the oracle, layer by layer
    for l in range(3):
        y_ref = xs[l] + moe_ref.layer(moe_ref.rms_norm(xs[l], norm_w[l], 1e-6), layer_c2)
        assert moe_ref.rel_err(ys[l], y_ref) < TOL


@pytest.fixture(scope="module")
def c2_norm_weight():
    return (np.random.default_rng(5).standard_normal(2048) * 0.1).astype(np.float32)


@pytest.mark.parametrize("T,weighted,residual", [(1, True, True), (1, False, False), (1, True, False),
                                                   (9, True, True), (64, True, True), (64, False, False)])
def test_pre_norm_residual(hip, c2, layer_c2, c2_norm_weight, T, weighted, residual):
    """WL_MOE_PRE_NORM / WL_MOE_RESIDUAL (one decoder step's x + MoE(rms_norm(x)), engines/qwen36/model.py:22) at
    batch 1 (fused kernel) and 9, 64 (multi-kernel GEMV / split plans). The normalization is bit-exact with the
    oracle's fixed-order rms_norm, so the flagged layer on x equals, bit for bit, x + the plain layer on the oracle's
    rms_norm(x); the plain layer on that input is checked against the oracle."""
    w = c2_norm_weight if weighted else None
    layer = hip.MoELayer.from_host(layer_c2, pre_norm=True, norm_weight=w, norm_eps=1e-6, residual=residual)
    x = synth.tokens(6, T) * np.float32(3.0)  # off unit scale, so a dropped normalization cannot pass
    xn = moe_ref.rms_norm(x, w, 1e-6)
    print(f"[moe] pre_norm T={T} weighted={weighted} residual={residual} plan={layer.plan(T)}", flush=True)
    y, ids, wts = run_layer(hip, layer, x)
    y_plain, ids_plain, wts_plain = run_layer(hip, c2, xn)
    np.testing.assert_array_equal(ids, ids_plain)
    np.testing.assert_array_equal(wts.view(np.uint32), wts_plain.view(np.uint32))
    want = (x + y_plain) if residual else y_plain
    np.testing.assert_array_equal(y.view(np.uint32), want.view(np.uint32))
    check_layer(hip, c2, layer_c2, xn, f"pre_norm T={T}")
