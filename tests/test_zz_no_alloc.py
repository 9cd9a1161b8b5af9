"""wl_moe_layer_noalloc (the entry point that allocates nothing: its workspace is a device array inside the
library) against wl_moe_layer on the same inputs, through the C ABI: outputs and routing bit-identical, on calls
in a row with shrinking inputs (the scratch keeps the previous call's contents), each plan covered (split MFMA +
GEMV at 64 tokens, all-GEMV at 5, the fused kernel at 1); a call too large for the scratch is refused; split calls
made inside an open fork scope equal the calls outside one (they take no part in the scope: every call of this
entry point runs its MFMA and GEMV experts on the caller's stream)."""
import ctypes

import numpy as np
import pytest
import torch

from gguf import synth

pytestmark = pytest.mark.gpu


def test_noalloc_matches_workspace_entry_point(hip, layer_c2):
    layer = hip.MoELayer.from_host(layer_c2)
    for T, plan in ((64, "split"), (5, "gemv"), (1, "fused")):
        print(f"[noalloc] T={T} plan={plan}", flush=True)
        assert layer.plan(T) == plan
        x = torch.from_numpy(synth.tokens(500 + T, T)).cuda()
        ids_a = torch.empty(T, 8, dtype=torch.int32, device="cuda")
        w_a = torch.empty(T, 8, dtype=torch.float32, device="cuda")
        y_a = layer(x, ids=ids_a, weights=w_a)
        y_b = torch.empty(T, 2048, dtype=torch.float32, device="cuda")
        ids_b = torch.empty_like(ids_a)
        w_b = torch.empty_like(w_a)
        layer.call_noalloc(x, y_b, ids=ids_b, weights=w_b)
        torch.cuda.synchronize()
        assert torch.isfinite(y_b).all()
        np.testing.assert_array_equal(ids_b.cpu().numpy(), ids_a.cpu().numpy())
        np.testing.assert_array_equal(w_b.cpu().numpy().view(np.uint32), w_a.cpu().numpy().view(np.uint32))
        np.testing.assert_array_equal(y_b.cpu().numpy().view(np.uint32), y_a.cpu().numpy().view(np.uint32))


def test_noalloc_refuses_oversize(hip, layer_c2):
    layer = hip.MoELayer.from_host(layer_c2)
    T = 4096
    assert layer.workspace_bytes(T) > hip.NOALLOC_SCRATCH_BYTES
    x = torch.zeros(T, 2048, dtype=torch.float32, device="cuda")
    y = torch.full((T, 2048), 7.0, dtype=torch.float32, device="cuda")
    rc = hip.library().wl_moe_layer_noalloc(ctypes.byref(layer.struct), x.data_ptr(), T, y.data_ptr(), None, None,
                                            torch.cuda.current_stream().cuda_stream)
    assert rc == -9  # WL_EINVAL_SCRATCH, before anything was enqueued
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
    with pytest.raises(ValueError):
        layer.call_noalloc(x, y)


def test_noalloc_in_fork_scope(hip):
    """Split-plan calls of the no-allocation entry point made while a fork scope is open on the stream, three
    layers in a row: they run unforked (the entry point never takes the second stream, so an open scope does not
    change what it launches), and the results equal the same calls outside a scope bit for bit."""
    layers = [hip.MoELayer.from_host(synth.moe_layer(190 + i, experts=64, top_k=8)) for i in range(3)]
    T = 40  # 64 experts, top-8: both expert classes (wl_moe_layer would use the second stream here)
    assert all(layer.plan(T) == "split" for layer in layers)
    xs = [torch.from_numpy(synth.tokens(1500 + i, T)).cuda() for i in range(3)]
    want = [layer(x) for layer, x in zip(layers, xs)]
    got = [torch.empty(T, 2048, dtype=torch.float32, device="cuda") for _ in layers]
    print("[noalloc] fork scope, 3 layers, T=40", flush=True)
    with hip.fork_scope():
        for layer, x, y in zip(layers, xs, got):
            layer.call_noalloc(x, y)
    torch.cuda.synchronize()
    assert layers[0].status_noalloc() == 0
    for i in range(3):
        assert torch.isfinite(want[i]).all()
        assert torch.equal(got[i], want[i]), f"layer {i}: max diff {(got[i] - want[i]).abs().max().item()}"
