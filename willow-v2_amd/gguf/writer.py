"""A minimal GGUF v3 writer, the inverse of gguf/reader.py: for synthetic model files (tests, the loader
benchmark), since no real checkpoint is available offline.

    write_gguf(path, metadata, tensors, alignment=32)
metadata: {key: value}; a value is a str, bool, int (u32 if it fits, else i64), float (f32), a list of one of
those, or an explicit (value_type, value) pair with the GGUF value type ids of gguf/reader.py (VALUE_DTYPES,
VALUE_STRING, VALUE_ARRAY: then value = (item_type, list)). tensors: [(name, ggml type name, shape in PyTorch order, data)], data a
bytes-like or numpy array holding exactly tensor_nbytes(shape, type) bytes. Each tensor's data starts at a multiple
of `alignment` from the data section, which itself starts at a multiple of `alignment`; an alignment other than
32 is recorded as general.alignment.
"""
import struct

import numpy as np

from .reader import ALIGNMENT_DEFAULT, MAGIC, TYPE_IDS, VALUE_ARRAY, VALUE_DTYPES, VALUE_STRING, tensor_nbytes

STRING, ARRAY = VALUE_STRING, VALUE_ARRAY
U32, I64, F32, BOOL = 4, 11, 6, 7


def _infer(value):
    if isinstance(value, tuple) and len(value) == 2 and isinstance(value[0], int):
        return value
    if isinstance(value, bool):
        return BOOL, value
    if isinstance(value, str):
        return STRING, value
    if isinstance(value, (int, np.integer)):
        return (U32 if 0 <= value < 1 << 32 else I64), int(value)
    if isinstance(value, (float, np.floating)):
        return F32, float(value)
    if isinstance(value, (list, np.ndarray)):
        items = list(value)
        kind = _infer(items[0])[0] if items else U32
        if kind == U32 and any(not 0 <= v < 1 << 32 for v in items):
            kind = I64
        return ARRAY, (kind, items)
    raise TypeError(f"no GGUF metadata type for {type(value).__name__}")


def _string(s: str) -> bytes:
    raw = s.encode("utf-8")
    return struct.pack("<Q", len(raw)) + raw


def _value(kind: int, value) -> bytes:
    if kind == STRING:
        return _string(value)
    if kind == ARRAY:
        item, items = value
        body = struct.pack("<IQ", item, len(items))
        if item in VALUE_DTYPES:
            return body + np.asarray(items, dtype=VALUE_DTYPES[item]).tobytes()
        return body + b"".join(_value(item, v) for v in items)
    return np.asarray(value, dtype=VALUE_DTYPES[kind]).tobytes()


def write_gguf(path: str, metadata: dict, tensors: list, alignment: int = 32, version: int = 3):
    alignment = int(metadata.get("general.alignment", alignment))
    if alignment != ALIGNMENT_DEFAULT and "general.alignment" not in metadata:
        metadata = {**metadata, "general.alignment": (U32, alignment)}  # readers assume 32 without it
    head = [MAGIC, struct.pack("<IQQ", version, len(tensors), len(metadata))]
    for key, value in metadata.items():
        kind, v = _infer(value)
        head += [_string(key), struct.pack("<I", kind), _value(kind, v)]
    offset, placed = 0, []
    for name, type_name, shape, data in tensors:
        nbytes = tensor_nbytes(tuple(shape), type_name)
        buf = memoryview(np.ascontiguousarray(data) if isinstance(data, np.ndarray) else data).cast("B")
        if buf.nbytes != nbytes:
            raise ValueError(f"{name}: {buf.nbytes} bytes of data for {nbytes} bytes of {type_name} {tuple(shape)}")
        offset = -(-offset // alignment) * alignment
        ne = tuple(reversed(shape))
        head += [_string(name), struct.pack(f"<I{len(ne)}Q", len(ne), *ne),
                 struct.pack("<IQ", TYPE_IDS[type_name], offset)]
        placed.append((offset, buf))
        offset += nbytes
    header = b"".join(head)
    data_start = -(-len(header) // alignment) * alignment
    with open(path, "wb") as f:
        f.write(header + bytes(data_start - len(header)))
        pos = 0
        for off, buf in placed:
            f.write(bytes(off - pos))
            f.write(buf)
            pos = off + buf.nbytes
