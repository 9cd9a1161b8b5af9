"""GPU parity of the quantized kernels (wl_dequant, wl_gemv, wl_linear, wl_gemv_batch, wl_gemv_combine) against the
CPU oracle. Dequantized weights must be bit-exact; products within the normwise bound 2e-3 (fp32 accumulation), or
4e-3 for wl_linear, whose output is rounded to bf16 (2^-9 relative) as the reference's bf16 F.linear is."""
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gguf import synth
from oracle import moe_ref
from oracle import quants_ref as q

pytestmark = pytest.mark.gpu
TOL = 2e-3
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "known_blocks.npz")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K"])
def test_dequant_known_blocks(hip, name):
    g = np.load(GOLDEN)
    blocks, values = g[name.lower() + "_blocks"], g[name.lower() + "_values"]
    out = hip.dequantize_gpu(dev(blocks), name, (len(blocks), 256), torch.float32).cpu().numpy()
    np.testing.assert_array_equal(out, values)


@pytest.mark.parametrize("name,rows,k", [("Q4_K", 512, 2048), ("Q6_K", 2048, 512), ("Q4_K", 3, 256),
                                         ("Q6_K", 5, 768), ("Q4_K", 7, 2560)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_dequant_bit_exact(hip, name, rows, k, dtype):
    print(f"[dequant] {name} {rows}x{k} {dtype}", flush=True)
    rng = np.random.default_rng(rows * 7 + k)
    w = synth.matrix(rng, name, rows, k)
    expect = q.dequantize(w, name, (rows, k), dtype)
    got = hip.dequantize_gpu(dev(w), name, (rows, k), torch.bfloat16 if dtype == "bf16" else torch.float32)
    got = got.cpu()
    got = got.view(torch.int16).numpy().view(np.uint16) if dtype == "bf16" else got.numpy()
    np.testing.assert_array_equal(got.view(np.uint16 if dtype == "bf16" else np.uint32),
                                  expect.view(np.uint16 if dtype == "bf16" else np.uint32))


def test_gemv_config0(hip):
    """The 512x2048 Q4_K GEMV (seed 0)."""
    case = synth.gemv_case(0)
    expect = case["x"] @ q.dequantize_matrix(case["w"], "Q4_K", 512, 2048).T
    got = hip.gemv(dev(case["w"]), "Q4_K", (512, 2048), dev(case["x"])).cpu().numpy()
    err = moe_ref.rel_err(got, expect)
    print(f"[gemv c0] rel err {err:.2e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("name,rows,k,tokens", [
    ("Q4_K", 1024, 2048, 1), ("Q4_K", 512, 2048, 3), ("Q4_K", 512, 2048, 8), ("Q4_K", 100, 2048, 11),
    ("Q6_K", 2048, 512, 1), ("Q6_K", 2048, 512, 5), ("Q6_K", 33, 256, 2), ("Q6_K", 17, 768, 1),
    ("Q4_K", 64, 512, 4), ("Q4_K", 9, 1024, 1), ("Q6_K", 40, 2560, 3), ("Q4_K", 5, 4096, 2)])
def test_gemv_shapes(hip, name, rows, k, tokens):
    print(f"[gemv] {name} {rows}x{k} T={tokens}", flush=True)
    case = synth.gemv_case(rows + k + tokens, rows, k, name, tokens)
    w32 = q.dequantize_matrix(case["w"], name, rows, k).astype(np.float64)
    expect = case["x"].astype(np.float64) @ w32.T
    got = hip.gemv(dev(case["w"]), name, (rows, k), dev(case["x"])).cpu().numpy()
    assert moe_ref.rel_err(got, expect) < TOL


def test_gemv_batch_and_combine(hip):
    """gate_up of 4 experts in one launch (gemv_batch), then down + weighted sum (gemv_combine), as
    Engine.batched_decode_experts drives them (engines/base.py:492-532)."""
    rng = np.random.default_rng(21)
    E, H, I = 6, 2048, 512
    gu = synth.matrix(rng, "Q4_K", 2 * I, H, count=E).reshape(E, -1)
    dn = synth.matrix(rng, "Q6_K", H, I, count=E).reshape(E, -1)
    x = rng.standard_normal(H).astype(np.float32)
    picks = [4, 1, 5, 2]
    gu_d, dn_d = dev(gu), dev(dn)
    out = torch.zeros(len(picks), 2 * I, dtype=torch.float32, device="cuda")
    hip.gemv_batch(gu_d, "Q4_K", (2 * I, H), dev(x), [e * gu.shape[1] for e in picks], [3, 0, 1, 2], out)
    out = out.cpu().numpy()
    for pos, e in zip([3, 0, 1, 2], picks):
        expect = q.dequantize_matrix(gu[e], "Q4_K", 2 * I, H) @ x
        assert moe_ref.rel_err(out[pos], expect) < TOL
    h = rng.standard_normal((len(picks), I)).astype(np.float32)
    weights = rng.random(8).astype(np.float32)
    perm = [6, 0, 3, 1]
    y = hip.gemv_combine(dn_d, "Q6_K", (H, I), dev(h), [e * dn.shape[1] for e in picks], dev(weights), perm)
    expect = sum(weights[perm[i]] * (q.dequantize_matrix(dn[e], "Q6_K", H, I).astype(np.float64) @ h[i])
                 for i, e in enumerate(picks))
    assert moe_ref.rel_err(y.cpu().numpy()[0], expect) < TOL


def test_ggml_weight_linear(hip):
    rng = np.random.default_rng(4)
    w = synth.matrix(rng, "Q4_K", 256, 1024)
    weight = hip.GGMLWeight(dev(w).reshape(-1), "Q4_K", (256, 1024))
    dense = torch.from_numpy(q.dequantize_matrix(w, "Q4_K", 256, 1024)).double()
    for tokens in (1, 8, 20):  # 20 > MAX_TOKENS: dequantize to bf16 + torch matmul, as gguf/metal.py:407
        x = torch.randn(tokens, 1024, generator=torch.Generator().manual_seed(tokens))
        y = F.linear(x.cuda(), weight)
        assert y.dtype == x.dtype and y.shape == (tokens, 256)
        expect = (x.double() @ dense.T).numpy()
        assert moe_ref.rel_err(y.cpu().numpy(), expect) < (TOL if tokens <= 8 else 2e-2)
    base, offset = weight.location()
    assert offset == 0 and base.numel() == w.size


def test_ggml_weight_linear_routes(hip):
    """Above MAX_TOKENS: with keep_dense (the default) the bf16 values are dequantized once and kept, and each call is
    the reference's bf16 F.linear on them (gguf/metal.py:407), bit for bit; with keep_dense False each call
    dequantizes to a temporary and runs the same F.linear, nothing kept, also bit for bit."""
    rng = np.random.default_rng(14)
    w = synth.matrix(rng, "Q6_K", 512, 2048)
    weight = hip.GGMLWeight(dev(w).reshape(-1), "Q6_K", (512, 2048))
    x = torch.randn(70, 2048, generator=torch.Generator().manual_seed(15)).cuda()
    want = F.linear(x.to(torch.bfloat16), hip.dequantize_gpu(weight.raw, "Q6_K", (512, 2048))).float()
    y = F.linear(x, weight)
    kept = weight.dense()
    assert torch.equal(y, want)
    assert torch.equal(F.linear(x, weight), want) and weight.dense() is kept  # dequantized once
    dense = torch.from_numpy(q.dequantize_matrix(w, "Q6_K", 512, 2048))
    assert torch.equal(kept.float().cpu(), dense.to(torch.bfloat16).float())  # the blocks' values, rounded to bf16
    weight.drop_dense()
    weight.keep_dense = False
    y2 = F.linear(x, weight)
    assert weight._dense is None
    assert torch.equal(y2, want)


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K"])
@pytest.mark.parametrize("rows,k", [(256, 256), (512, 2048), (2048, 512)])
@pytest.mark.parametrize("tokens", [9, 20, 64, 65, 130, 300])
def test_linear_mfma(hip, name, rows, k, tokens):
    """wl_linear against bf16(x) . bf16(dequantized W)^T in fp64: token counts on each K-loop form (one, four and
    eight token tiles of 16, and several 128-token tiles, the last one partial)."""
    rng = np.random.default_rng(rows + k + tokens)
    w = synth.matrix(rng, name, rows, k)
    x = rng.standard_normal((tokens, k)).astype(np.float32)
    y = hip.linear_mfma(dev(w).reshape(-1), name, (rows, k), torch.from_numpy(x).cuda())
    assert y.dtype == torch.bfloat16 and y.shape == (tokens, rows)
    wb = q.round_bf16(q.dequantize_matrix(w, name, rows, k)).astype(np.float64)
    ref = q.round_bf16(x).astype(np.float64) @ wb.T
    err = moe_ref.rel_err(y.float().cpu().numpy(), ref)
    assert err < 4e-3, err


def test_linear_mfma_rejects(hip):
    w = torch.zeros(255 * 144, dtype=torch.uint8, device="cuda")
    x = torch.zeros(16, 256, device="cuda")
    with pytest.raises(ValueError):  # rows not a multiple of 256
        hip.linear_mfma(w, "Q4_K", (255, 256), x)


def test_errors_raise(hip):
    w = torch.zeros(144, dtype=torch.uint8, device="cuda")
    with pytest.raises(NotImplementedError):
        hip.dequantize_gpu(w, "Q5_K", (1, 256))
    with pytest.raises(ValueError):
        hip.gemv(w, "Q4_K", (1, 100), torch.zeros(1, 100, device="cuda"))
