"""The CPU oracle, pinned: the dequantizers against the format's known answers and against each other, the router
replay against exact arithmetic, route() against brute force, and the layer against float64 and against
transformers' Qwen3.5-MoE block. No GPU."""
import fractions
import os

import numpy as np
import pytest
import torch

from gguf import synth
from oracle import cref, moe_ref
from oracle import quants_ref as q

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "known_blocks.npz")


@pytest.fixture(scope="module")
def known():
    return np.load(GOLDEN)


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K"])
def test_known_blocks(known, name):
    key = name.lower()
    blocks, values = known[key + "_blocks"], known[key + "_values"]
    for fn in (q.DEQUANTIZERS[name], q.CHUNK_DEQUANTIZERS[name], lambda b: cref.dequant_scalar(b, name)):
        np.testing.assert_array_equal(fn(blocks), values)


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K"])
def test_formulations_agree_bitwise(name):
    rng = np.random.default_rng(7)
    blocks = synth.BLOCKS[name](rng, 3000)
    # also fully random bytes, with the fp16 scale fields kept finite (any sign, subnormals included)
    raw = rng.integers(0, 256, (1000, q.BLOCK_SIZES[name][1]), dtype=np.uint8)
    for off in ((0, 2) if name == "Q4_K" else (208,)):
        raw[:, off + 1] &= 0xBF  # clear the top exponent bit: no inf / NaN
    for b in (blocks, raw):
        a = q.DEQUANTIZERS[name](b)
        for other in (q.CHUNK_DEQUANTIZERS[name](b), cref.dequant_scalar(b, name)):
            np.testing.assert_array_equal(a.view(np.uint32), other.view(np.uint32))


def test_q4_k_exact_in_float32():
    """Every product is exact in fp32, so the float64 value rounded once equals the fp32 result: evaluation order
    and fused multiply-add cannot change a dequantized weight."""
    rng = np.random.default_rng(3)
    b = synth.q4_k_blocks(rng, 2000)
    scale, mn, qv = q.q4_k_parts(b)
    exact = scale.astype(np.float64)[..., None] * qv.astype(np.float64) - mn.astype(np.float64)[..., None]
    np.testing.assert_array_equal(exact.astype(np.float32).reshape(len(b), 256), q.dequant_q4_k(b))
    b6 = synth.q6_k_blocks(rng, 2000)
    s6, q6 = q.q6_k_parts(b6)
    exact6 = s6.astype(np.float64)[..., None] * q6.astype(np.float64)
    assert np.array_equal(exact6.astype(np.float32).astype(np.float64), exact6)  # no rounding at all


def test_k_scale_min_roundtrip():
    """Packing 8 arbitrary 6-bit (scale, min) pairs ggml-style and unpacking gives them back."""
    rng = np.random.default_rng(5)
    for _ in range(200):
        sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        s = np.zeros(12, dtype=np.uint8)
        for j in range(4):
            s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
            s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
            s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
        got_sc, got_mn = q.k_scale_min(s[None])
        np.testing.assert_array_equal(got_sc[0], sc)
        np.testing.assert_array_equal(got_mn[0], mn)


def test_bf16_matches_torch():
    rng = np.random.default_rng(11)
    a = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, 3.4e38], dtype=np.float32)]).astype(np.float32)
    # ties: values exactly halfway between two bf16 numbers
    ties = (np.arange(1000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    a = np.concatenate([a, ties])
    ours = q.f32_to_bf16_bits(a)
    theirs = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)


def test_dequantize_dispatch():
    rng = np.random.default_rng(0)
    w = synth.matrix(rng, "Q4_K", 4, 512)
    assert q.dequantize(w, "Q4_K", (4, 512), "f32").shape == (4, 512)
    assert q.dequantize(w, "Q4_K", (4, 512)).dtype == np.uint16  # bf16 bits by default, as gguf/quants.py
    with pytest.raises(NotImplementedError):
        q.dequantize(w, "Q5_K", (4, 512))


def _fma_exact(a, b, c):
    """fp32 fused multiply-add computed exactly with rationals, rounded once to float32."""
    exact = fractions.Fraction(float(a)) * fractions.Fraction(float(b)) + fractions.Fraction(float(c))
    # round to nearest even float32 via float64 candidates
    f = np.float32(float(exact))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    best = min(cands, key=lambda v: (abs(fractions.Fraction(float(v)) - exact),
                                     int(np.array([v], dtype=np.float32).view(np.uint32)[0]) & 1))
    return np.float32(best)


def test_router_replay_exact():
    """The C replay equals the documented order computed with exact rational fused multiply-adds."""
    rng = np.random.default_rng(9)
    T, H, E = 2, 128, 3
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    bias = rng.standard_normal(E).astype(np.float32)
    got = cref.router_logits(x, w, bias)
    for t in range(T):
        for e in range(E):
            total = None
            for s in range(H // 64):
                p = np.float32(0)
                for k in range(64 * s, 64 * s + 64):
                    p = _fma_exact(x[t, k], w[e, k], p)
                total = p if total is None else np.float32(total + p)
            assert got[t, e] == np.float32(total + bias[e])


def test_router_replay_accuracy():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((16, 2048)).astype(np.float32)
    w = (rng.standard_normal((256, 2048)) * 0.02).astype(np.float32)
    got = cref.router_logits(x, w)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    bound = 2048 * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    assert np.all(np.abs(got - ref) <= bound)


def test_route_brute_force():
    rng = np.random.default_rng(2)
    logits = rng.standard_normal((50, 64)).astype(np.float32)
    logits[3, [5, 9]] = logits[3, 1]  # ties: the lower id first
    weights, ids = moe_ref.route(logits, 8, True)
    for t in range(50):
        order = sorted(range(64), key=lambda e: (-float(logits[t, e]), e))[:8]
        assert list(ids[t]) == order
    assert list(ids[3][:3]) == [1, 5, 9] or logits[3].max() > logits[3, 1]
    np.testing.assert_allclose(weights.sum(-1), 1.0, rtol=1e-6)
    assert np.all(np.diff(weights, axis=-1) <= 0)
    w_raw, _ = moe_ref.route(logits, 8, False)
    p = np.exp(logits.astype(np.float64) - logits.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(w_raw, np.take_along_axis(p, ids.astype(np.int64), -1), rtol=1e-5)


def _small_layer(seed=4, experts=8, top_k=2, hidden=256, inter=256, down_type="Q6_K"):
    return synth.moe_layer(seed, hidden=hidden, inter=inter, shared_inter=inter, experts=experts, top_k=top_k,
                           down_type=down_type)


def test_layer_float64_loop():
    """The fp32 oracle layer against a float64 per-token loop over its own routing."""
    lw = _small_layer()
    x = synth.tokens(8, 5, 256)
    y, ids, wts, sg = moe_ref.layer(x, lw, return_routing=True)
    inter = lw["inter"]
    expect = np.zeros((5, 256))
    for t in range(5):
        for s in range(lw["top_k"]):
            e = ids[t, s]
            gu = q.dequantize_matrix(lw["gate_up"][e], "Q4_K", 2 * inter, 256).astype(np.float64) @ x[t]
            h = gu[:inter] / (1 + np.exp(-gu[:inter])) * gu[inter:]
            expect[t] += wts[t, s] * (q.dequantize_matrix(lw["down"][e], "Q6_K", 256, inter).astype(np.float64) @ h)
        gu = q.dequantize_matrix(lw["shared_gate_up"], "Q4_K", 2 * inter, 256).astype(np.float64) @ x[t]
        h = gu[:inter] / (1 + np.exp(-gu[:inter])) * gu[inter:]
        g = 1 / (1 + np.exp(-(x[t].astype(np.float64) @ lw["shared_gate"])))
        expect[t] += g * (q.dequantize_matrix(lw["shared_down"], "Q6_K", 256, inter).astype(np.float64) @ h)
    assert moe_ref.rel_err(y, expect) < 1e-5


def test_layer_matches_transformers_block():
    """Third-party pin: transformers' Qwen3_5MoeSparseMoeBlock on the same dequantized fp32 weights gives the
    same output (it routes on F.linear logits; inputs are chosen with clear top-k margins)."""
    mod = pytest.importorskip("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe")
    cfg_mod = pytest.importorskip("transformers.models.qwen3_5_moe.configuration_qwen3_5_moe")
    lw = _small_layer(experts=8, top_k=2)
    H, I, E = 256, 256, 8
    cfg = cfg_mod.Qwen3_5MoeTextConfig(hidden_size=H, moe_intermediate_size=I, shared_expert_intermediate_size=I,
                                       num_experts=E, num_experts_per_tok=2, hidden_act="silu")
    block = mod.Qwen3_5MoeSparseMoeBlock(cfg).float()
    with torch.no_grad():
        block.gate.weight.copy_(torch.from_numpy(lw["router"]))
        for e in range(E):
            block.experts.gate_up_proj[e].copy_(torch.from_numpy(q.dequantize_matrix(lw["gate_up"][e], "Q4_K", 2 * I, H)))
            block.experts.down_proj[e].copy_(torch.from_numpy(q.dequantize_matrix(lw["down"][e], "Q6_K", H, I)))
        sgu = q.dequantize_matrix(lw["shared_gate_up"], "Q4_K", 2 * I, H)
        block.shared_expert.gate_proj.weight.copy_(torch.from_numpy(sgu[:I]))
        block.shared_expert.up_proj.weight.copy_(torch.from_numpy(sgu[I:]))
        block.shared_expert.down_proj.weight.copy_(torch.from_numpy(q.dequantize_matrix(lw["shared_down"], "Q6_K", H, I)))
        block.shared_expert_gate.weight.copy_(torch.from_numpy(lw["shared_gate"][None]))
    x = synth.tokens(12, 6, H)
    logits = cref.router_logits(x, lw["router"])
    srt = np.sort(logits, -1)
    assert np.all(srt[:, -2] - srt[:, -3] > 1e-4)  # no near-ties at the top-k boundary
    with torch.no_grad():
        theirs = block(torch.from_numpy(x)[None])[0].numpy()
    ours = moe_ref.layer(x, lw)
    assert moe_ref.rel_err(ours, theirs) < 1e-5


def test_rms_norm_oracle():
    """The oracle's RMSNorm against the reference's formula in torch (engines/base.py:27-31, zero-centered) within
    a few ulps (torch's rsqrt is not correctly rounded), against float64, and its sum of squares in the router's
    order against exact rational arithmetic on a short row."""
    import torch
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((6, 512)) * np.array([1, 10, 1e-3, 1e3, 1, 1])[:, None]).astype(np.float32)
    w = (rng.standard_normal(512) * 0.1).astype(np.float32)
    ours = moe_ref.rms_norm(x, w, 1e-6)
    xt = torch.from_numpy(x)
    theirs = (xt * torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + 1e-6) * (1.0 + torch.from_numpy(w))).numpy()
    np.testing.assert_allclose(ours, theirs, rtol=4e-7, atol=0)
    x64 = x.astype(np.float64)
    exact = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * (1 + w.astype(np.float64))
    np.testing.assert_allclose(ours, exact, rtol=1e-6)
    assert np.array_equal(moe_ref.rms_norm(x, None, 1e-6), moe_ref.rms_norm(x, np.zeros(512, np.float32), 1e-6))
    from fractions import Fraction
    short = x[:1, :128]
    ss = cref.router_logits(short, short)[0, 0]
    # the replayed order: two 64-value fused multiply-add chains (each step rounded once), then their sum
    def fma_chain(v):
        acc = np.float32(0)
        for e in v:
            acc = np.float32(Fraction(float(acc)) + Fraction(float(e)) * Fraction(float(e)))
        return acc
    assert ss == np.float32(fma_chain(short[0, :64]) + fma_chain(short[0, 64:]))


def test_topk_margins():
    logits = np.array([[5, 4, 3, 2, 1, 0], [1, 1, 1, 1, 1, 1], [0, 3, 9, 3, 2, 8]], dtype=np.float32)
    np.testing.assert_array_equal(moe_ref.topk_margins(logits, 2), [1, 0, 5])
    np.testing.assert_array_equal(moe_ref.topk_margins(logits, 3), [1, 0, 0])


def test_skip_small_closed_forms():
    """moe_ref.skip_small (engines/base.py:413-430) on cases whose answer is fixed by the definition: the kept
    weights keep their ratios and add up to the sum of all k (a scale of K / S or an S without the dropped ones
    fails); a weight equal to the threshold is kept (>=); the top pick is kept when everything is below; nothing
    dropped leaves the routing bit for bit unchanged."""
    ids = np.array([[7, 3, 9, 1]], dtype=np.int32)
    w = np.array([[0.5, 0.25, 0.125, 0.125]], dtype=np.float32)
    out, oid = moe_ref.skip_small(w, ids, 0.2)
    np.testing.assert_array_equal(oid, [[7, 3, -1, -1]])
    assert out[0, 2] == 0.0 and out[0, 3] == 0.0
    assert out[0, 0] == 2 * out[0, 1]  # one scale for both: the ratio of two powers of 2 stays exact
    assert abs(float(out[0, 0]) + float(out[0, 1]) - 1.0) <= 2 ** -23  # S = 1, not K = 0.75
    assert out[0, 0] > 0.5  # scaled up, by S / K = 4 / 3
    # equal to the threshold: kept
    w2 = np.array([[0.5, 0.25, 0.25]], dtype=np.float32)
    out2, oid2 = moe_ref.skip_small(w2, ids[:, :3], 0.25)
    np.testing.assert_array_equal(oid2, ids[:, :3])
    np.testing.assert_array_equal(out2, w2)
    # all below: the top pick alone, carrying the whole sum
    w3 = np.array([[0.3, 0.3, 0.2, 0.2]], dtype=np.float32)
    out3, oid3 = moe_ref.skip_small(w3, ids, 0.9)
    np.testing.assert_array_equal(oid3, [[7, -1, -1, -1]])
    assert abs(float(out3[0, 0]) - 1.0) <= 2 ** -23 and (out3[0, 1:] == 0).all()
    # nothing dropped: unchanged bit for bit (K == S, scale exactly 1)
    logits = np.random.default_rng(3).standard_normal((50, 64)).astype(np.float32)
    wr, ir = moe_ref.route(logits, 8, True)
    out4, oid4 = moe_ref.skip_small(wr, ir, 1e-12)
    np.testing.assert_array_equal(out4.view(np.uint32), wr.view(np.uint32))
    np.testing.assert_array_equal(oid4, ir)


def test_layer_skip_small_experts():
    """layer(min_expert_weight): a threshold no weight reaches equals the layer with each token's top expert alone at
    the weight sum of its k (here 1, renormalized), built from the oracle's own expert_ffn; a threshold every weight
    passes equals the plain layer bit for bit."""
    lw = synth.moe_layer(21, experts=16, top_k=4)
    x = synth.tokens(22, 5)
    plain = moe_ref.layer(x, lw)
    np.testing.assert_array_equal(moe_ref.layer(x, lw, min_expert_weight=1e-12), plain)
    y, ids, wts, sg = moe_ref.layer(x, lw, min_expert_weight=1.0, return_routing=True)
    assert (ids[:, 1:] == -1).all() and (wts[:, 1:] == 0).all()
    _, ids_full = moe_ref.route(cref.router_logits(x, lw["router"], lw.get("router_bias")), 4, True)
    np.testing.assert_array_equal(ids[:, 0], ids_full[:, 0])
    inter, hidden = lw["inter"], lw["hidden"]
    want = np.zeros_like(plain)
    for t in range(x.shape[0]):
        e = ids[t, 0]
        gu = q.dequantize_matrix(lw["gate_up"][e], lw["gate_up_type"], 2 * inter, hidden)
        dn = q.dequantize_matrix(lw["down"][e], lw["down_type"], hidden, inter)
        want[t] = moe_ref.expert_ffn(x[t:t + 1], gu, dn, inter)[0] * wts[t, 0]
    # the shared expert's part alone: the same layer with every routed expert's blocks zero (they dequantize to 0)
    sh = moe_ref.layer(x, dict(lw, gate_up=np.zeros_like(lw["gate_up"]), down=np.zeros_like(lw["down"])))
    np.testing.assert_allclose(y - sh, want, rtol=1e-5, atol=1e-5 * float(np.abs(want).max()))
