"""HIP kernels that compute straight from GGUF's quantized Q4_K / Q6_K blocks on an MI355X (gfx950), through a
thin ctypes shim over libwillow_hip.so (C ABI: include/willow_hip.h).

A drop-in for gguf/metal.py on this path: the same module surface (TYPES, MAX_TOKENS, available, row_bytes, gemv,
gemv_batch, gemv_combine, dequantize_gpu, GGMLWeight; gguf/metal.py:20,295,320-408), computing in fp32 where the
Metal kernels round to bf16. It adds the fused MoE layer (moe_layer / MoELayer), which replaces Engine.moe's
router -> host sync -> per-expert launches (engines/base.py:445-591) with device-side routing.

There is no CPU fallback: without the built library (or without a GPU) every compute call raises.
"""
import ctypes
import os

import torch
import torch.nn.functional as F

TYPES = ("Q4_K", "Q6_K")
TYPE_IDS = {"Q4_K": 12, "Q6_K": 14}
BLOCK_SIZES = {"Q4_K": (256, 144), "Q6_K": (256, 210)}  # gguf/reader.py:25,27
MAX_TOKENS = 8  # F.linear on a GGMLWeight runs the GEMV kernel up to this many tokens (gguf/metal.py:20)
MAX_BATCH_EXPERTS = 64
DTYPE_F32, DTYPE_BF16 = 0, 1
MOE_NO_FUSED, MOE_NO_MFMA, MOE_FORCE_MFMA, MOE_TEST_STARVE, MOE_PRE_NORM, MOE_RESIDUAL = 1, 2, 4, 8, 16, 32
MOE_GUESS_NEXT = 64
ESYNC = -10  # wl_moe_workspace_status: a bounded wait gave up
EINVAL_SCOPE = -12  # wl_moe_fork_begin / wl_moe_fork_end used outside their pairing
NOALLOC_SCRATCH_BYTES = 16 << 20  # WL_NOALLOC_SCRATCH_BYTES

LIBRARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libwillow_hip.so")


class HipError(RuntimeError):
    """A launch failed on the device (code = hipError_t)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"libwillow_hip: {message} (hipError {code})")
        self.code = code


class WlMoeLayer(ctypes.Structure):
    """Mirror of the C struct WlMoeLayer (include/willow_hip.h)."""
    _fields_ = [
        ("gate_up", ctypes.c_void_p), ("down", ctypes.c_void_p), ("router", ctypes.c_void_p),
        ("router_bias", ctypes.c_void_p), ("shared_gate_up", ctypes.c_void_p), ("shared_down", ctypes.c_void_p),
        ("shared_gate", ctypes.c_void_p), ("gate_up_stride", ctypes.c_int64), ("down_stride", ctypes.c_int64),
        ("gate_up_type", ctypes.c_int32), ("down_type", ctypes.c_int32), ("shared_gate_up_type", ctypes.c_int32),
        ("shared_down_type", ctypes.c_int32), ("hidden", ctypes.c_int32), ("inter", ctypes.c_int32),
        ("shared_inter", ctypes.c_int32), ("n_experts", ctypes.c_int32), ("top_k", ctypes.c_int32),
        ("norm_topk_prob", ctypes.c_int32), ("flags", ctypes.c_int32), ("reserved", ctypes.c_int32),
        ("next", ctypes.c_void_p), ("norm_weight", ctypes.c_void_p), ("norm_eps", ctypes.c_float),
        ("min_expert_weight", ctypes.c_float),
    ]


_lib = None


def library() -> ctypes.CDLL:
    """libwillow_hip.so, loaded once. torch is imported first so the library binds to torch's HIP runtime."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY):
        raise RuntimeError(f"{LIBRARY} is missing: build it with `python willow-v2_amd/build.py` "
                           "(or __graft_entry__.build())")
    lib = ctypes.CDLL(LIBRARY)
    vp, i64, i32, c_int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int
    i64p = ctypes.POINTER(ctypes.c_int64)
    lib.wl_error_string.argtypes, lib.wl_error_string.restype = [c_int], ctypes.c_char_p
    lib.wl_abi_version.argtypes, lib.wl_abi_version.restype = [], c_int
    lib.wl_row_bytes.argtypes, lib.wl_row_bytes.restype = [c_int, i64], i64
    lib.wl_dequant.argtypes = [c_int, vp, i64, i64, i64, c_int, vp, vp]
    lib.wl_gemv.argtypes = [c_int, vp, i64, i64, i64, vp, i64, vp, vp]
    lib.wl_linear.argtypes = [c_int, vp, i64, i64, vp, i64, vp, vp]
    lib.wl_gemv_batch.argtypes = [c_int, vp, i64, i64, i64p, i64p, c_int, vp, vp, vp]
    lib.wl_gemv_combine.argtypes = [c_int, vp, i64, i64, i64p, i64p, c_int, vp, vp, vp, vp]
    layer_p = ctypes.POINTER(WlMoeLayer)
    lib.wl_moe_check.argtypes = [layer_p]
    lib.wl_moe_workspace_bytes.argtypes, lib.wl_moe_workspace_bytes.restype = [layer_p, i64], ctypes.c_size_t
    lib.wl_moe_route.argtypes = [layer_p, vp, i64, vp, vp, vp, vp, vp]
    lib.wl_moe_layer.argtypes = [layer_p, vp, i64, vp, vp, vp, vp, ctypes.c_size_t, vp]
    lib.wl_moe_layer_profile.argtypes = [layer_p, vp, i64, vp, vp, vp, vp, ctypes.c_size_t, vp,
                                         ctypes.POINTER(ctypes.c_void_p)]
    lib.wl_moe_stage_count.argtypes, lib.wl_moe_stage_count.restype = [], c_int
    lib.wl_moe_plan.argtypes, lib.wl_moe_plan.restype = [layer_p, i64], c_int
    lib.wl_moe_workspace_init.argtypes, lib.wl_moe_workspace_init.restype = [vp, ctypes.c_size_t, vp], c_int
    lib.wl_moe_stage_name.argtypes, lib.wl_moe_stage_name.restype = [c_int], ctypes.c_char_p
    lib.wl_moe_layer_noalloc.argtypes, lib.wl_moe_layer_noalloc.restype = [layer_p, vp, i64, vp, vp, vp, vp], c_int
    lib.wl_moe_workspace_status.argtypes, lib.wl_moe_workspace_status.restype = [vp, ctypes.c_size_t, vp], c_int
    lib.wl_moe_fork_begin.argtypes, lib.wl_moe_fork_begin.restype = [vp], c_int
    lib.wl_moe_fork_end.argtypes, lib.wl_moe_fork_end.restype = [vp], c_int
    for name in ("wl_dequant", "wl_gemv", "wl_linear", "wl_gemv_batch", "wl_gemv_combine", "wl_moe_check", "wl_moe_route",
                 "wl_moe_layer", "wl_moe_layer_profile"):
        getattr(lib, name).restype = c_int
    _lib = lib
    return lib


def check(rc: int):
    """Turns a return code into the reference's exception types: NotImplementedError for an unsupported type
    (gguf/quants.py:214-216), ValueError for other argument errors, HipError for device errors."""
    if rc == 0:
        return
    message = library().wl_error_string(rc).decode()
    if rc == -1:
        raise NotImplementedError(f"libwillow_hip: {message}")
    if rc == ESYNC:
        raise HipError(rc, message)
    if rc < 0:
        raise ValueError(f"libwillow_hip: {message} (code {rc})")
    raise HipError(rc, message)


def available() -> bool:
    """Whether the kernels can run here: a ROCm GPU and the built library (gguf/metal.py:320-321)."""
    return torch.cuda.is_available() and torch.version.hip is not None and os.path.exists(LIBRARY)


def row_bytes(type_name: str, k: int) -> int:
    """gguf/metal.py:323-325."""
    elements, block_bytes = BLOCK_SIZES[type_name]
    return k // elements * block_bytes


def _type_id(type_name: str) -> int:
    if type_name not in TYPE_IDS:
        raise NotImplementedError(f"ggml type {type_name} is not supported by the HIP kernels (supported: "
                                  f"{', '.join(TYPES)})")
    return TYPE_IDS[type_name]


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class fork_scope:
    """A fork scope on the current stream of `device` (wl_moe_fork_begin / wl_moe_fork_end): the split-plan layer
    calls inside it hand their MFMA experts to the device's second stream through their workspaces instead of a
    fork and a join event each (under graph capture, two graph edges for the whole block instead of two per call).
    Use it around a block of layer calls issued in order from one thread, e.g. the layers of one decode step."""

    def __init__(self, device=None):
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.stream = None

    def __enter__(self):
        self.stream = _stream(self.device)
        check(library().wl_moe_fork_begin(self.stream))
        return self

    def __exit__(self, *exc):
        check(library().wl_moe_fork_end(self.stream))
        return False


def _on_gpu(t: torch.Tensor, what: str):
    if not t.is_cuda:
        raise ValueError(f"{what} must be on the GPU (got {t.device})")


def gemv(raw: torch.Tensor, type_name: str, shape: tuple, x: torch.Tensor) -> torch.Tensor:
    """raw: the weight's bytes (uint8, on the GPU); x [tokens, k] (any float dtype) -> fp32 [tokens, rows]
    (gguf/metal.py:327-334, which returns bf16)."""
    rows, k = shape
    _on_gpu(raw, "raw")
    xf = x.reshape(-1, k).to(device=raw.device, dtype=torch.float32).contiguous()
    y = torch.empty(xf.shape[0], rows, dtype=torch.float32, device=raw.device)
    check(library().wl_gemv(_type_id(type_name), raw.data_ptr(), rows, k, row_bytes(type_name, k), xf.data_ptr(),
                            xf.shape[0], y.data_ptr(), _stream(raw.device)))
    return y


def linear_mfma(raw: torch.Tensor, type_name: str, shape: tuple, x: torch.Tensor) -> torch.Tensor:
    """x [T, k] -> bf16 [T, rows] on the bf16 matrix core with the weights dequantized in registers: the numbers
    of gguf/metal.py:407 (bf16 F.linear of the weight dequantized to bf16) without writing the bf16 weight out.
    rows and k must be multiples of 256."""
    rows, k = shape
    _on_gpu(raw, "raw")
    xb = x.reshape(-1, k).to(device=raw.device, dtype=torch.bfloat16).contiguous()
    y = torch.empty(xb.shape[0], rows, dtype=torch.bfloat16, device=raw.device)
    check(library().wl_linear(_type_id(type_name), raw.data_ptr(), rows, k, xb.data_ptr(), xb.shape[0], y.data_ptr(),
                              _stream(raw.device)))
    return y


def _int64_array(values):
    arr = (ctypes.c_int64 * len(values))(*[int(v) for v in values])
    return arr


def gemv_batch(base: torch.Tensor, type_name: str, shape: tuple, x: torch.Tensor, offsets: list, positions: list,
               out: torch.Tensor):
    """Several experts' [rows, k] weights at byte offsets in base (uint8, on the GPU), times one token x [k]:
    writes expert i's result to row positions[i] of out [n, rows] (gguf/metal.py:336-343)."""
    rows, k = shape
    _on_gpu(base, "base")
    if len(offsets) != len(positions):
        raise ValueError("offsets and positions differ in length")
    xf = x.reshape(-1)[:k].to(device=base.device, dtype=torch.float32).contiguous()
    target = out if (out.dtype == torch.float32 and out.is_contiguous()) else torch.empty(
        out.shape, dtype=torch.float32, device=out.device)
    if target is not out:
        target.copy_(out)
    check(library().wl_gemv_batch(_type_id(type_name), base.data_ptr(), rows, k, _int64_array(offsets),
                                  _int64_array(positions), len(offsets), xf.data_ptr(), target.data_ptr(),
                                  _stream(base.device)))
    if target is not out:
        out.copy_(target)


def gemv_combine(base: torch.Tensor, type_name: str, shape: tuple, x: torch.Tensor, offsets: list,
                 weights: torch.Tensor, perm: list) -> torch.Tensor:
    """sum over i of weights[perm[i]] * (W_i x[i]), in order of i, in fp32 (gguf/metal.py:345-355 rounds each
    step to bf16). W_i: [rows, k] at byte offsets[i] in base; x [n, k]; weights [top_k] on the GPU -> fp32
    [1, rows]."""
    rows, k = shape
    _on_gpu(base, "base")
    xf = x.reshape(-1, k).to(device=base.device, dtype=torch.float32).contiguous()
    wf = weights.reshape(-1).to(device=base.device, dtype=torch.float32).contiguous()
    if len(offsets) != xf.shape[0] or len(perm) != len(offsets):
        raise ValueError("offsets, perm and x's rows must agree")
    y = torch.empty(1, rows, dtype=torch.float32, device=base.device)
    check(library().wl_gemv_combine(_type_id(type_name), base.data_ptr(), rows, k, _int64_array(offsets),
                                    _int64_array(perm), len(offsets), xf.data_ptr(), wf.data_ptr(), y.data_ptr(),
                                    _stream(base.device)))
    return y


def dequantize_gpu(raw: torch.Tensor, type_name: str, shape: tuple, dtype: torch.dtype = torch.bfloat16):
    """raw (uint8, on the GPU) -> [rows, k] of dtype (bf16 by default, as gguf/metal.py:357-363; fp32 too),
    bit-exact with gguf/quants.py's dequantizers."""
    rows, k = shape
    _on_gpu(raw, "raw")
    if dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("dequantize_gpu: dtype must be torch.bfloat16 or torch.float32")
    out = torch.empty(rows, k, dtype=dtype, device=raw.device)
    check(library().wl_dequant(_type_id(type_name), raw.data_ptr(), rows, k, row_bytes(type_name, k),
                               DTYPE_BF16 if dtype == torch.bfloat16 else DTYPE_F32, out.data_ptr(),
                               _stream(raw.device)))
    return out


class GGMLWeight:
    """A [rows, k] weight kept as its ggml blocks on the GPU, used in place of a dense tensor: F.linear(x, weight)
    runs the HIP kernels (through __torch_function__), as gguf/metal.py:365-408. raw is a uint8 tensor on the GPU
    (a view into the HBM-resident expert store) or on the CPU, in which case it is copied over on first use.

    Above MAX_TOKENS tokens the reference dequantizes the weight to bf16 on every call and runs a bf16 F.linear
    (gguf/metal.py:407). With keep_dense (the default) the bf16 values are dequantized once, on the first such call,
    and kept in HBM beside the blocks (2 bytes per value; the non-expert weights are a few GB at most against 288 GB),
    so each call is the same bf16 F.linear on the same values, the library GEMM alone. With keep_dense False nothing
    is kept between calls: each call is the reference's own form, the weight dequantized to a bf16 temporary and
    the library GEMM on it (bit for bit the reference's arithmetic). linear_mfma (wl_linear, the weights dequantized
    in registers, no temporary) is the form for a caller that cannot hold the temporary; on dense shapes it is the
    slower one at every token count measured from 16 to 8192."""

    keep_dense = True

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        bias = (kwargs or {}).get("bias", args[2] if len(args) > 2 else None)
        if func is F.linear and len(args) > 1 and isinstance(args[1], GGMLWeight) and bias is None:
            return args[1].linear(args[0])
        return NotImplemented

    def __init__(self, raw: torch.Tensor, type_name: str, shape: tuple):
        _type_id(type_name)
        self.raw, self.type_name, self.shape = raw, type_name, tuple(shape)
        if raw.numel() != self.shape[0] * row_bytes(type_name, self.shape[1]):
            raise ValueError(f"{raw.numel()} bytes do not hold a {type_name} {self.shape} matrix")
        self.nbytes = raw.numel()
        self.device = raw.device if raw.is_cuda else torch.device("cuda")
        self._dense = None

    def to_gpu(self):
        if not self.raw.is_cuda:
            self.raw = self.raw.to(self.device, non_blocking=True)

    def location(self):
        """(the GPU buffer holding this weight's bytes as a uint8 tensor, their byte offset in it)
        (gguf/metal.py:393-399)."""
        self.to_gpu()
        base = self.raw if self.raw._base is None else self.raw._base
        return base, self.raw.storage_offset() - base.storage_offset()

    def dense(self) -> torch.Tensor:
        """The weight's values as bf16 [rows, k] on the GPU: dequantized once (bit-exact with gguf/quants.py, rounded
        to bf16 as gguf/metal.py:357-363 does), then kept until drop_dense()."""
        if self._dense is None:
            self.to_gpu()
            self._dense = dequantize_gpu(self.raw, self.type_name, self.shape)
        return self._dense

    def drop_dense(self):
        """Frees the kept bf16 values (the next call above MAX_TOKENS with keep_dense dequantizes again)."""
        self._dense = None

    def linear(self, x: torch.Tensor) -> torch.Tensor:
        self.to_gpu()
        flat = x.reshape(-1, x.shape[-1]).to(self.device)
        if flat.shape[0] <= MAX_TOKENS:
            y = gemv(self.raw, self.type_name, self.shape, flat).to(x.dtype)
        elif self.keep_dense:  # the reference's arithmetic (gguf/metal.py:407) on bf16 values kept in HBM
            y = F.linear(flat.to(torch.bfloat16), self.dense()).to(x.dtype)
        else:  # the reference's own form (gguf/metal.py:407): dequantized on every call, nothing kept
            y = F.linear(flat.to(torch.bfloat16), dequantize_gpu(self.raw, self.type_name, self.shape)).to(x.dtype)
        return y.view(*x.shape[:-1], y.shape[-1]).to(x.device)


from .moe import MoELayer, moe_layer  # noqa: E402  (needs the names above)
