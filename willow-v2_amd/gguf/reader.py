"""GGUF header reader: the tensor directory and metadata of a (possibly split) .gguf model, with no tensor data
read. The same surface as gguf/reader.py of the reference (GGML_TYPES, BLOCK_SIZES, GGUFTensor, tensor_nbytes,
read_gguf_file, split_paths, model_stem, read_gguf; gguf/reader.py:8-171), so the expert scan and the HBM loader
take its output unchanged.

File layout (GGUF v2/v3, little endian):
    "GGUF"  u32 version  u64 n_tensors  u64 n_kv
    n_kv x   (string key, u32 value type, value)
    n_tensors x (string name, u32 n_dims, u64 ne[n_dims], u32 ggml type, u64 offset)
    padding to general.alignment (default 32); tensor data, each tensor at data_start + offset.
A string is a u64 byte count followed by UTF-8 bytes. ne lists the innermost (row) dimension first; shapes here are
in PyTorch order, outermost first. Malformed files end the program with a message (SystemExit), as the reference's
reader does.
"""
import mmap
import os
import re
import struct
from dataclasses import dataclass

import numpy as np

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32
QK_K = 256

# ggml type id -> (name, values per block, bytes per block). The ids and block sizes are ggml's on-disk format,
# so this table necessarily lists the same entries as the reference's (gguf/reader.py:14-45).
GGML_TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4),
    27: ("I64", 1, 8), 28: ("F64", 1, 8), 30: ("BF16", 1, 2),
    # 32-value blocks: fp16 scale (and min), 4/5/8-bit values
    2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22), 7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34),
    9: ("Q8_1", 32, 36), 20: ("IQ4_NL", 32, 18), 39: ("MXFP4", 32, 17), 42: ("Q2_0", 64, 18),
    # 256-value super-blocks
    10: ("Q2_K", QK_K, 84), 11: ("Q3_K", QK_K, 110), 12: ("Q4_K", QK_K, 144), 13: ("Q5_K", QK_K, 176),
    14: ("Q6_K", QK_K, 210), 15: ("Q8_K", QK_K, 292), 16: ("IQ2_XXS", QK_K, 66), 17: ("IQ2_XS", QK_K, 74),
    18: ("IQ3_XXS", QK_K, 98), 19: ("IQ1_S", QK_K, 50), 21: ("IQ3_S", QK_K, 110), 22: ("IQ2_S", QK_K, 82),
    23: ("IQ4_XS", QK_K, 136), 29: ("IQ1_M", QK_K, 56), 34: ("TQ1_0", QK_K, 54), 35: ("TQ2_0", QK_K, 66),
}
BLOCK_SIZES = {name: (values, nbytes) for name, values, nbytes in GGML_TYPES.values()}

# metadata value types: scalars by struct code; 8 = string, 9 = array
SCALAR_FORMATS = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}
STRING, ARRAY = 8, 9
_NUMPY_FORMATS = {0: "<u1", 1: "<i1", 2: "<u2", 3: "<i2", 4: "<u4", 5: "<i4", 6: "<f4", 10: "<u8", 11: "<i8",
                  12: "<f8"}

SPLIT_RE = re.compile(r"^(.*)-(\d{5})-of-(\d{5})\.gguf$")


@dataclass
class GGUFTensor:
    name: str
    path: str    # the file holding the tensor's data (one of a split model's files)
    offset: int  # absolute byte offset of the data in that file
    type: str    # ggml type name, e.g. "Q4_K"
    shape: tuple  # PyTorch order, outermost first
    nbytes: int


def tensor_nbytes(shape: tuple, type_name: str) -> int:
    """Bytes of a tensor of `shape` (rows of shape[-1] values) in ggml type `type_name`."""
    values, nbytes = BLOCK_SIZES[type_name]
    if shape[-1] % values:
        raise ValueError(f"row length {shape[-1]} is not a multiple of the {type_name} block size {values}")
    return int(np.prod(shape, dtype=np.int64)) // values * nbytes


class _Header:
    """Sequential little-endian decoding of a GGUF header held in a buffer."""

    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, fmt: str):
        out = struct.unpack_from("<" + fmt, self.buf, self.pos)
        self.pos += struct.calcsize("<" + fmt)
        return out

    def u32(self) -> int:
        return self.take("I")[0]

    def u64(self) -> int:
        return self.take("Q")[0]

    def string(self) -> str:
        n = self.u64()
        raw = bytes(self.buf[self.pos:self.pos + n])
        self.pos += n
        return raw.decode("utf-8", errors="replace")

    def value(self, kind: int):
        if kind == STRING:
            return self.string()
        if kind == ARRAY:
            item, count = self.take("IQ")
            if item in _NUMPY_FORMATS:  # vocabularies: ~250k scores or token types in one read
                arr = np.frombuffer(self.buf, dtype=_NUMPY_FORMATS[item], count=count, offset=self.pos)
                self.pos += arr.nbytes
                return arr.tolist()
            return [self.value(item) for _ in range(count)]
        if kind not in SCALAR_FORMATS:
            raise SystemExit(f"unknown GGUF metadata value type {kind}")
        return self.take(SCALAR_FORMATS[kind])[0]


def read_gguf_file(path: str):
    """One .gguf file's header: (metadata dict, {name: GGUFTensor}) (gguf/reader.py:104-137)."""
    with open(path, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
        view = memoryview(mm)
        try:
            if bytes(view[:4]) != GGUF_MAGIC:
                raise SystemExit(f"{path} is not a GGUF file")
            h = _Header(view)
            h.pos = 4
            version, n_tensors, n_kv = h.take("IQQ")
            if version < 2:
                raise SystemExit(f"{path} is GGUF version {version}; only versions 2 and 3 are supported")
            metadata = {}
            for _ in range(n_kv):
                key = h.string()
                metadata[key] = h.value(h.u32())
            entries = []
            for _ in range(n_tensors):
                name = h.string()
                ne = h.take(f"{h.u32()}Q")
                type_id, offset = h.take("IQ")
                if type_id not in GGML_TYPES:
                    raise SystemExit(f"{path}: tensor {name} has unknown ggml type {type_id}")
                entries.append((name, tuple(reversed(ne)), GGML_TYPES[type_id][0], offset))
            alignment = metadata.get("general.alignment", DEFAULT_ALIGNMENT)
            data_start = -(-h.pos // alignment) * alignment
        finally:
            view.release()
    tensors = {name: GGUFTensor(name, path, data_start + offset, type_name, shape, tensor_nbytes(shape, type_name))
               for name, shape, type_name, offset in entries}
    return metadata, tensors


def split_paths(path: str) -> list:
    """Every file of a split model (<name>-0000i-of-0000n.gguf) given any one of them; [path] for a single file
    (gguf/reader.py:139-150)."""
    m = SPLIT_RE.match(os.path.basename(path))
    if not m:
        return [path]
    stem, count = m.group(1), m.group(3)
    folder = os.path.dirname(path)
    paths = [os.path.join(folder, f"{stem}-{i:05d}-of-{count}.gguf") for i in range(1, int(count) + 1)]
    missing = [p for p in paths if not os.path.exists(p)]
    if missing:
        raise SystemExit(f"Split GGUF is missing {len(missing)} of {count} files, e.g. {missing[0]}")
    return paths


def model_stem(path: str) -> str:
    """The model path without .gguf and without a split suffix (gguf/reader.py:152-156)."""
    m = SPLIT_RE.match(os.path.basename(path))
    name = m.group(1) if m else os.path.basename(path).removesuffix(".gguf")
    return os.path.join(os.path.dirname(path), name)


def read_gguf(path: str):
    """A whole (possibly split) model: (metadata of the first file, {name: GGUFTensor} over all files)
    (gguf/reader.py:158-171)."""
    metadata, tensors = None, {}
    for p in split_paths(path):
        meta, found = read_gguf_file(p)
        if metadata is None:
            metadata = meta
        tensors.update(found)
    return metadata, tensors
