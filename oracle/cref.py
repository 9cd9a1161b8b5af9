"""Oracle (test infrastructure): ctypes loader for oracle_ref.c, compiled with gcc into oracle/build/."""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCE = os.path.join(HERE, "oracle_ref.c")
LIBRARY = os.path.join(HERE, "build", "liboracle_ref.so")


def build(force: bool = False) -> str:
    """Compiles oracle_ref.c (a second or so). -ffp-contract=off keeps every multiply and add as written."""
    if force or not os.path.exists(LIBRARY) or os.path.getmtime(LIBRARY) < os.path.getmtime(SOURCE):
        os.makedirs(os.path.dirname(LIBRARY), exist_ok=True)
        tmp = LIBRARY + f".tmp{os.getpid()}"
        subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", SOURCE, "-o", tmp, "-lm"],
                       check=True)
        os.replace(tmp, LIBRARY)
    return LIBRARY


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = ctypes.CDLL(build())
        f32p, u8p = ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_uint8)
        i64 = ctypes.c_int64
        _lib.oracle_router_logits.argtypes = [f32p, f32p, f32p, i64, i64, i64, f32p]
        _lib.oracle_dequant_q4_k_scalar.argtypes = [u8p, i64, f32p]
        _lib.oracle_dequant_q6_k_scalar.argtypes = [u8p, i64, f32p]
    return _lib


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def router_logits(x: np.ndarray, w: np.ndarray, bias=None) -> np.ndarray:
    """fp32 x [T, H] . W [E, H]^T (+ bias [E]) in the GPU router's fixed FMA order (see oracle_ref.c)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    tokens, hidden = x.shape
    experts = w.shape[0]
    assert w.shape[1] == hidden and hidden % 64 == 0
    out = np.empty((tokens, experts), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().oracle_router_logits(_ptr(x, ctypes.c_float), _ptr(w, ctypes.c_float),
                               None if b is None else _ptr(b, ctypes.c_float), tokens, hidden, experts,
                               _ptr(out, ctypes.c_float))
    return out


def dequant_scalar(blocks: np.ndarray, type_name: str) -> np.ndarray:
    """[n, block_bytes] uint8 -> [n, 256] float32, one value at a time in C."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = blocks.shape[0]
    out = np.empty((n, 256), dtype=np.float32)
    fn = {"Q4_K": lib().oracle_dequant_q4_k_scalar, "Q6_K": lib().oracle_dequant_q6_k_scalar}[type_name]
    fn(_ptr(blocks, ctypes.c_uint8), n, _ptr(out, ctypes.c_float))
    return out
