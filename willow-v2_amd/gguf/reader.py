"""GGUF header parsing for the HBM loader: which tensors a model file holds, where their bytes are, and the
model's metadata. No tensor data is read here.

The GGUF container (versions 2 and 3, little endian), as llama.cpp's ggml writes it:

    magic "GGUF" | u32 version | u64 tensor count | u64 metadata count
    metadata:     key (string) | u32 value type | value            -- repeated
    tensor infos: name (string) | u32 dims | u64 extent per dim (innermost first) | u32 ggml type | u64 offset
    zero padding up to `general.alignment` (32 when absent), then the data section;
    a tensor's bytes start at data section + its offset.

A string is a u64 length and that many UTF-8 bytes; an array value is a u32 item type, a u64 count and the items.
Shapes here are PyTorch order (outermost first), the reverse of the extents on disk. Large models are split over
files named <stem>-00001-of-0000N.gguf; read_gguf takes any one of them and returns the union of their tensors.

Errors in a file raise GGUFFormatError (a ValueError) naming the file and the byte position.
"""
import os
import re
import struct
from dataclasses import dataclass, field

import numpy as np


class GGUFFormatError(ValueError):
    """The file is not a GGUF container this reader understands."""


MAGIC = b"GGUF"
ALIGNMENT_KEY = "general.alignment"
ALIGNMENT_DEFAULT = 32

# The ggml block formats: type id -> (name, values per block, bytes per block). These numbers are ggml's on-disk
# definition of each format; the two the kernels run are Q4_K (d, dmin fp16 + 12 packed scale bytes + 128 nibble
# bytes) and Q6_K (128 low-nibble bytes + 64 high-bit bytes + 16 int8 scales + d fp16).
_SUPER = 256
GGML_TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22),
    7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36), 10: ("Q2_K", _SUPER, 84),
    11: ("Q3_K", _SUPER, 110), 12: ("Q4_K", _SUPER, 144), 13: ("Q5_K", _SUPER, 176), 14: ("Q6_K", _SUPER, 210),
    15: ("Q8_K", _SUPER, 292), 16: ("IQ2_XXS", _SUPER, 66), 17: ("IQ2_XS", _SUPER, 74), 18: ("IQ3_XXS", _SUPER, 98),
    19: ("IQ1_S", _SUPER, 50), 20: ("IQ4_NL", 32, 18), 21: ("IQ3_S", _SUPER, 110), 22: ("IQ2_S", _SUPER, 82),
    23: ("IQ4_XS", _SUPER, 136), 24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4), 27: ("I64", 1, 8),
    28: ("F64", 1, 8), 29: ("IQ1_M", _SUPER, 56), 30: ("BF16", 1, 2), 34: ("TQ1_0", _SUPER, 54),
    35: ("TQ2_0", _SUPER, 66), 39: ("MXFP4", 32, 17), 42: ("Q2_0", 64, 18),
}
BLOCK_SIZES = {name: (values, nbytes) for name, values, nbytes in GGML_TYPES.values()}
TYPE_IDS = {name: tid for tid, (name, _, _) in GGML_TYPES.items()}

# Metadata value types. Fixed-size ones: id -> numpy little-endian dtype; 8 is a string, 9 an array.
VALUE_DTYPES = {0: np.dtype("<u1"), 1: np.dtype("<i1"), 2: np.dtype("<u2"), 3: np.dtype("<i2"),
                4: np.dtype("<u4"), 5: np.dtype("<i4"), 6: np.dtype("<f4"), 7: np.dtype("?"),
                10: np.dtype("<u8"), 11: np.dtype("<i8"), 12: np.dtype("<f8")}
VALUE_STRING, VALUE_ARRAY = 8, 9

_SHARD_NAME = re.compile(r"(?P<stem>.+)-(?P<index>\d{5})-of-(?P<total>\d{5})\.gguf$")


@dataclass(frozen=True)
class GGUFTensor:
    """Where one tensor's bytes are: `file`, from byte `offset` (absolute), `nbytes` long."""
    name: str
    type: str       # ggml type name ("Q4_K", "F32", ...)
    shape: tuple    # PyTorch order, outermost first
    file: str
    offset: int
    nbytes: int

    def slice(self, index: int, count: int):
        """(file, offset, size) of the index-th of `count` equal slices along the outermost dimension (one expert
        of a stacked expert tensor: quantized blocks never straddle rows, so the slices are byte ranges)."""
        size = self.nbytes // count
        return self.file, self.offset + index * size, size


@dataclass
class GGUFHeader:
    """A model's metadata (from its first file) and every tensor of all its files, by name."""
    metadata: dict
    tensors: dict
    files: list = field(default_factory=list)

    def __iter__(self):  # (metadata, tensors) = header
        return iter((self.metadata, self.tensors))


def tensor_nbytes(shape, type_name: str) -> int:
    """Size in bytes of a tensor of `shape` (PyTorch order) stored as `type_name`; the innermost extent must be
    a whole number of blocks."""
    values, block = BLOCK_SIZES[type_name]
    rows = int(np.prod(shape[:-1], dtype=np.int64)) if len(shape) > 1 else 1
    if shape[-1] % values != 0:
        raise ValueError(f"a {type_name} row holds a multiple of {values} values, not {shape[-1]}")
    return rows * (shape[-1] // values) * block


class _Parser:
    """Decodes the header fields of one file from a bytes buffer, tracking the position for error messages."""

    def __init__(self, data: bytes, path: str):
        self.data, self.path, self.at = data, path, 0

    def fail(self, why: str):
        raise GGUFFormatError(f"{self.path}, byte {self.at}: {why}")

    def need(self, n: int):
        if self.at + n > len(self.data):
            raise _Short(self.at + n)

    def fixed(self, dtype: np.dtype, count: int = 1):
        n = dtype.itemsize * count
        self.need(n)
        out = np.frombuffer(self.data, dtype=dtype, count=count, offset=self.at)
        self.at += n
        return out

    def u32(self) -> int:
        return int(self.fixed(VALUE_DTYPES[4])[0])

    def u64(self) -> int:
        return int(self.fixed(VALUE_DTYPES[10])[0])

    def text(self) -> str:
        n = self.u64()
        self.need(n)
        raw = self.data[self.at:self.at + n]
        self.at += n
        return raw.decode("utf-8", errors="replace")

    def value(self, kind: int):
        if kind in VALUE_DTYPES:
            return self.fixed(VALUE_DTYPES[kind])[0].item()
        if kind == VALUE_STRING:
            return self.text()
        if kind == VALUE_ARRAY:
            item_kind, count = self.u32(), self.u64()
            if item_kind in VALUE_DTYPES:  # vocabularies: one numpy read for ~250k items
                return self.fixed(VALUE_DTYPES[item_kind], count).tolist()
            return [self.value(item_kind) for _ in range(count)]
        self.fail(f"metadata value type {kind} is not defined by GGUF")


class _Short(Exception):
    """The buffer ended before the header did; `size` bytes are needed at least."""

    def __init__(self, size: int):
        self.size = size


def _parse(data: bytes, path: str):
    p = _Parser(data, path)
    p.need(24)
    if data[:4] != MAGIC:
        p.fail(f"starts with {data[:4]!r}, not the GGUF magic {MAGIC!r}")
    p.at = 4
    version = p.u32()
    if version not in (2, 3):
        p.fail(f"container version {version} (this reader knows versions 2 and 3)")
    n_tensors, n_meta = p.u64(), p.u64()
    metadata = {}
    for _ in range(n_meta):
        key = p.text()
        metadata[key] = p.value(p.u32())
    infos = []
    for _ in range(n_tensors):
        name = p.text()
        dims = p.u32()
        extents = p.fixed(VALUE_DTYPES[10], dims).tolist()
        type_id, offset = p.u32(), p.u64()
        if type_id not in GGML_TYPES:
            p.fail(f"tensor {name!r} uses ggml type id {type_id}, which has no block layout here")
        infos.append((name, GGML_TYPES[type_id][0], tuple(int(e) for e in reversed(extents)), int(offset)))
    alignment = int(metadata.get(ALIGNMENT_KEY, ALIGNMENT_DEFAULT))
    if alignment <= 0:
        p.fail(f"{ALIGNMENT_KEY} is {alignment}")
    data_start = (p.at + alignment - 1) // alignment * alignment
    tensors = {name: GGUFTensor(name, type_name, shape, path, data_start + offset, tensor_nbytes(shape, type_name))
               for name, type_name, shape, offset in infos}
    return metadata, tensors


def read_gguf_file(path: str):
    """(metadata, {name: GGUFTensor}) of one file. The header is read in growing pieces from the file's start, so
    a model of many GB costs a few MB of reads (more for a large vocabulary)."""
    size = os.path.getsize(path)
    want = min(size, 1 << 20)
    with open(path, "rb") as f:
        while True:
            f.seek(0)
            data = f.read(want)
            try:
                return _parse(data, path)
            except _Short as short:
                if want >= size:
                    raise GGUFFormatError(f"{path}: the header runs past the end of the file "
                                          f"({size} bytes)") from None
                want = min(size, max(2 * want, short.size))


def shard_files(path: str) -> list:
    """The files of the model `path` belongs to, in order: every <stem>-0000i-of-0000N.gguf when `path` is named
    as a shard, else [path]. Raises FileNotFoundError when a shard is missing."""
    m = _SHARD_NAME.fullmatch(os.path.basename(path))
    if m is None:
        return [path]
    total = int(m["total"])
    folder = os.path.dirname(path)
    files = [os.path.join(folder, f"{m['stem']}-{i:05d}-of-{m['total']}.gguf") for i in range(1, total + 1)]
    absent = [f for f in files if not os.path.isfile(f)]
    if absent:
        raise FileNotFoundError(f"model {m['stem']} is split over {total} files; {len(absent)} are missing "
                                f"({', '.join(os.path.basename(f) for f in absent[:3])})")
    return files


def read_gguf(path: str) -> GGUFHeader:
    """The header of a model: the first file's metadata and the tensors of all its files."""
    files = shard_files(path)
    metadata, tensors = read_gguf_file(files[0])
    for extra in files[1:]:
        tensors.update(read_gguf_file(extra)[1])
    return GGUFHeader(metadata, tensors, files)
