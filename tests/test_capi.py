"""The C ABI without a GPU: the library loads, exports every entry point include/willow_hip.h declares, and rejects
bad arguments on the host (with the documented codes) before anything is launched."""
import ctypes
import os
import re

import pytest

from gguf import hip

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "willow_hip.h")
FAKE = 0x10000  # a non-NULL, aligned address that is never dereferenced: every call below fails validation first


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\S[^()\n]*?\b(wl_\w+)\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = hip.library()
    names = declared_functions()
    assert len(names) >= 11
    for name in names:
        assert hasattr(lib, name), name


def test_abi_version_and_struct_layout():
    assert hip.library().wl_abi_version() >> 16 == 1
    # 7 weight pointers, 2 shared-expert pointers, 12 int32 fields, next, norm_weight, norm_eps + min_expert_weight
    assert ctypes.sizeof(hip.WlMoeLayer) == 7 * 8 + 2 * 8 + 12 * 4 + 8 + 8 + 8 == 144


def test_error_strings():
    lib = hip.library()
    for code in range(-11, 1):
        assert lib.wl_error_string(code)
    assert b"unsupported" in lib.wl_error_string(-1)


def test_row_bytes():
    lib = hip.library()
    assert lib.wl_row_bytes(12, 2048) == 8 * 144 == hip.row_bytes("Q4_K", 2048)
    assert lib.wl_row_bytes(14, 512) == 2 * 210 == hip.row_bytes("Q6_K", 512)
    assert lib.wl_row_bytes(13, 256) == -1
    assert lib.wl_row_bytes(12, 100) == -2


@pytest.mark.parametrize("args,code", [
    ((13, FAKE, 4, 256, 144), -1),      # Q5_K: unsupported type
    ((12, None, 4, 256, 144), -3),      # NULL weights
    ((12, FAKE, 4, 300, 144), -2),      # k not a multiple of 256
    ((12, FAKE, 0, 256, 144), -2),      # no rows
    ((12, FAKE + 8, 4, 256, 144), -4),  # Q4_K base not 16-byte aligned
    ((14, FAKE + 2, 4, 256, 210), -4),  # Q6_K base not dword aligned
    ((12, FAKE, 4, 512, 144), -2),      # row stride shorter than a row
])
def test_gemv_validation(args, code):
    lib = hip.library()
    type_id, w, rows, k, stride = args
    assert lib.wl_gemv(type_id, w, rows, k, stride, FAKE, 1, FAKE, None) == code
    assert lib.wl_dequant(type_id, w, rows, k, stride, 0, FAKE, None) == code


def test_gemv_null_and_dtype():
    lib = hip.library()
    assert lib.wl_gemv(12, FAKE, 4, 256, 144, None, 1, FAKE, None) == -3
    assert lib.wl_gemv(12, FAKE, 4, 256, 144, FAKE, 0, FAKE, None) == -2
    assert lib.wl_gemv(12, FAKE, 4, 256, 144, FAKE + 4, 1, FAKE, None) == -4  # x misaligned
    assert lib.wl_dequant(12, FAKE, 4, 256, 144, 7, FAKE, None) == -7


def test_batch_validation():
    lib = hip.library()
    offs = hip._int64_array([0, 144 * 4])
    pos = hip._int64_array([0, 1])
    assert lib.wl_gemv_batch(12, FAKE, 4, 256, offs, pos, 0, FAKE, FAKE, None) == -8
    assert lib.wl_gemv_batch(12, FAKE, 4, 256, offs, pos, 65, FAKE, FAKE, None) == -8
    bad = hip._int64_array([0, 8])
    assert lib.wl_gemv_batch(12, FAKE, 4, 256, bad, pos, 2, FAKE, FAKE, None) == -4
    assert lib.wl_gemv_combine(12, FAKE, 4, 256, offs, pos, 2, FAKE, None, FAKE, None) == -3


def layer_struct(**over):
    s = hip.WlMoeLayer()
    s.gate_up, s.down, s.router = FAKE, FAKE, FAKE
    s.gate_up_stride = 2 * 512 * 8 * 144
    s.down_stride = 2048 * 2 * 210
    s.gate_up_type, s.down_type = 12, 14
    s.shared_gate_up_type, s.shared_down_type = 12, 14
    s.hidden, s.inter, s.shared_inter = 2048, 512, 512
    s.n_experts, s.top_k, s.norm_topk_prob = 256, 8, 1
    for k, v in over.items():
        setattr(s, k, v)
    return s


@pytest.mark.parametrize("over,code", [
    ({}, 0),
    ({"top_k": 0}, -5),
    ({"top_k": 17}, -5),
    ({"n_experts": 4, "top_k": 8}, -5),
    ({"down_type": 13}, -1),
    ({"hidden": 2000}, -2),
    ({"inter": 0}, -2),
    ({"gate_up_stride": 100}, -2),
    ({"router": None}, -3),
    ({"gate_up": FAKE + 4}, -4),
    ({"shared_gate_up": FAKE}, -3),  # shared gate_up without shared down
    ({"shared_gate_up": FAKE, "shared_down": FAKE, "shared_inter": 100}, -2),
    ({"min_expert_weight": 0.05}, 0),
    ({"min_expert_weight": 1.0}, 0),
    ({"min_expert_weight": -0.1}, -2),
    ({"min_expert_weight": 1.5}, -2),
    ({"min_expert_weight": float("nan")}, -2),
])
def test_layer_validation(over, code):
    lib = hip.library()
    s = layer_struct(**over)
    assert lib.wl_moe_check(ctypes.byref(s)) == code
    if code == 0:
        assert lib.wl_moe_workspace_bytes(ctypes.byref(s), 1) > 0
        assert lib.wl_moe_workspace_bytes(ctypes.byref(s), 64) > lib.wl_moe_workspace_bytes(ctypes.byref(s), 1)
        assert lib.wl_moe_layer(ctypes.byref(s), FAKE, 1, FAKE + (1 << 24), None, None, None, 0, None) == -6
        assert lib.wl_moe_layer(ctypes.byref(s), FAKE, 0, FAKE, None, None, FAKE, 1 << 30, None) == -2
    else:
        assert lib.wl_moe_workspace_bytes(ctypes.byref(s), 1) == 0
        assert lib.wl_moe_layer(ctypes.byref(s), FAKE, 1, FAKE, None, None, FAKE, 1 << 30, None) == code


def test_python_errors():
    with pytest.raises(NotImplementedError):
        hip.check(-1)
    with pytest.raises(ValueError):
        hip.check(-2)
    with pytest.raises(hip.HipError):
        hip.check(1)
    with pytest.raises(NotImplementedError):
        hip._type_id("IQ4_XS")


def test_noalloc_validation_without_a_gpu():
    """wl_moe_layer_noalloc checks the layer and the size it would need before touching the device."""
    lib = hip.library()
    s = hip.WlMoeLayer()
    s.gate_up = s.down = s.router = s.shared_gate_up = s.shared_down = s.shared_gate = FAKE
    s.gate_up_stride, s.down_stride = 1179648, 860160
    s.gate_up_type = s.shared_gate_up_type = 12
    s.down_type = s.shared_down_type = 14
    s.hidden, s.inter, s.shared_inter, s.n_experts, s.top_k, s.norm_topk_prob = 2048, 512, 512, 256, 8, 1
    assert lib.wl_moe_workspace_bytes(ctypes.byref(s), 128) <= hip.NOALLOC_SCRATCH_BYTES
    assert lib.wl_moe_workspace_bytes(ctypes.byref(s), 4096) > hip.NOALLOC_SCRATCH_BYTES
    assert lib.wl_moe_layer_noalloc(ctypes.byref(s), FAKE, 4096, FAKE, None, None, None) == -9
    assert lib.wl_moe_layer_noalloc(ctypes.byref(s), FAKE, 0, FAKE, None, None, None) == -2
    assert lib.wl_moe_layer_noalloc(ctypes.byref(s), None, 1, FAKE, None, None, None) == -3
    s.top_k = 0
    assert lib.wl_moe_layer_noalloc(ctypes.byref(s), FAKE, 1, FAKE, None, None, None) == -5


def test_norm_residual_validation_without_a_gpu():
    """wl_moe_layer rejects y overlapping x, and a pre-norm layer with a negative eps or a misaligned weight, before
    it touches the device."""
    lib = hip.library()
    s = hip.WlMoeLayer()
    s.gate_up = s.down = s.router = s.shared_gate_up = s.shared_down = s.shared_gate = FAKE
    s.gate_up_stride, s.down_stride = 1179648, 860160
    s.gate_up_type = s.shared_gate_up_type = 12
    s.down_type = s.shared_down_type = 14
    s.hidden, s.inter, s.shared_inter, s.n_experts, s.top_k, s.norm_topk_prob = 2048, 512, 512, 256, 8, 1
    s.flags = hip.MOE_RESIDUAL
    ws = ctypes.c_void_p(FAKE)
    assert lib.wl_moe_layer(ctypes.byref(s), FAKE, 2, FAKE, None, None, ws, 0, None) == -11
    assert lib.wl_moe_layer(ctypes.byref(s), FAKE, 2, FAKE + 2048 * 4, None, None, ws, 0, None) == -11
    assert lib.wl_moe_layer(ctypes.byref(s), FAKE, 2, FAKE + 2 * 2048 * 4, None, None, ws, 0, None) == -6
    s.flags = hip.MOE_PRE_NORM
    s.norm_eps = -1.0
    assert lib.wl_moe_layer(ctypes.byref(s), FAKE, 1, FAKE + 2048 * 4, None, None, ws, 0, None) == -2
    s.norm_eps = float("nan")
    assert lib.wl_moe_layer(ctypes.byref(s), FAKE, 1, FAKE + 2048 * 4, None, None, ws, 0, None) == -2
    s.norm_eps, s.norm_weight = 1e-6, FAKE + 4
    assert lib.wl_moe_layer(ctypes.byref(s), FAKE, 1, FAKE + 2048 * 4, None, None, ws, 0, None) == -2
    s.norm_weight = FAKE
    with_norm = lib.wl_moe_workspace_bytes(ctypes.byref(s), 4)
    s.flags = 0
    assert with_norm - lib.wl_moe_workspace_bytes(ctypes.byref(s), 4) >= 4 * 2048 * 4  # the normalized input
