"""The GGUF header reader and the expert index (gguf/reader.py, gguf/experts.py; the reference's counterparts are
gguf/reader.py and the expert scan of gguf/compiler.py:24-88), on the CPU. The reader is pinned on a header
assembled byte by byte here from the published GGUF layout (not by this package's writer); the writer, the
split-file handling and the index are then checked on files the writer makes."""
import os
import struct

import numpy as np
import pytest

from gguf import synth
from gguf.experts import ExpertLayoutError, decoder_layer_count, index_experts
from gguf.reader import (BLOCK_SIZES, GGML_TYPES, GGUFFormatError, read_gguf, read_gguf_file, shard_files,
                         tensor_nbytes)
from gguf.writer import write_gguf


def s(text: str) -> bytes:
    raw = text.encode()
    return struct.pack("<Q", len(raw)) + raw


def handmade_header(version=3, type_b=12, magic=b"GGUF"):
    """GGUF v3: 6 metadata pairs, 2 tensors; alignment 64."""
    kv = [
        s("general.architecture") + struct.pack("<I", 8) + s("qwen35moe"),
        s("general.alignment") + struct.pack("<I", 4) + struct.pack("<I", 64),
        s("a.i32s") + struct.pack("<I", 9) + struct.pack("<IQ", 5, 3) + struct.pack("<3i", 1, -2, 3),
        s("a.strs") + struct.pack("<I", 9) + struct.pack("<IQ", 8, 2) + s("x") + s("yz"),
        s("a.flag") + struct.pack("<I", 7) + struct.pack("<?", True),
        s("a.f64") + struct.pack("<I", 12) + struct.pack("<d", 0.25),
    ]
    tensors = [
        s("t.f32") + struct.pack("<I", 2) + struct.pack("<2Q", 4, 3) + struct.pack("<IQ", 0, 0),   # ne (4, 3)
        s("t.q") + struct.pack("<I", 2) + struct.pack("<2Q", 512, 2) + struct.pack("<IQ", type_b, 64),
    ]
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kv)) + b"".join(kv) + b"".join(tensors)
    return head


def test_reader_on_handmade_header(tmp_path):
    head = handmade_header()
    p = tmp_path / "h.gguf"
    p.write_bytes(head + bytes(4096))
    md, ts = read_gguf_file(str(p))
    assert md == {"general.architecture": "qwen35moe", "general.alignment": 64, "a.i32s": [1, -2, 3],
                  "a.strs": ["x", "yz"], "a.flag": True, "a.f64": 0.25}
    data_start = (len(head) + 63) // 64 * 64
    a, b = ts["t.f32"], ts["t.q"]
    assert (a.shape, a.type, a.offset, a.nbytes) == ((3, 4), "F32", data_start, 48)
    # two rows of 512 Q4_K values: 2 x 2 blocks of 144 bytes
    assert (b.shape, b.type, b.offset, b.nbytes) == ((2, 512), "Q4_K", data_start + 64, 576)
    assert a.file == b.file == str(p)


def test_reader_needs_more_than_the_first_read(tmp_path):
    """A header longer than the reader's first piece (a large vocabulary array) is read in further pieces."""
    big = s("tok.scores") + struct.pack("<I", 9) + struct.pack("<IQ", 6, 400_000) + bytes(4 * 400_000)
    head = handmade_header()
    n_kv = struct.unpack_from("<Q", head, 16)[0]
    head = head[:16] + struct.pack("<Q", n_kv + 1) + head[24:]
    kv_end = head.index(s("t.f32"))
    head = head[:kv_end] + big + head[kv_end:]
    p = tmp_path / "big.gguf"
    p.write_bytes(head + bytes(4096))
    md, ts = read_gguf_file(str(p))
    assert len(md["tok.scores"]) == 400_000 and md["a.f64"] == 0.25
    assert ts["t.q"].offset == (len(head) + 63) // 64 * 64 + 64


@pytest.mark.parametrize("bad", ["magic", "version", "type", "truncated"])
def test_reader_rejects(tmp_path, bad):
    head = {"magic": handmade_header(magic=b"GGUX"), "version": handmade_header(version=1),
            "type": handmade_header(type_b=99), "truncated": handmade_header()[:-9]}[bad]
    p = tmp_path / "bad.gguf"
    p.write_bytes(head + (b"" if bad == "truncated" else bytes(128)))
    with pytest.raises(GGUFFormatError):
        read_gguf_file(str(p))


def test_block_sizes_follow_the_block_layouts():
    """Bytes per block from the field layout of each format (fp16 = 2 bytes)."""
    fp16 = 2
    assert BLOCK_SIZES["Q4_K"] == (256, 2 * fp16 + 12 + 256 // 2)      # d, dmin, 12 scale bytes, nibbles
    assert BLOCK_SIZES["Q6_K"] == (256, 256 // 2 + 256 // 4 + 16 + fp16)  # ql, qh, int8 scales, d
    assert BLOCK_SIZES["Q5_K"] == (256, 2 * fp16 + 12 + 256 // 2 + 256 // 8)
    assert BLOCK_SIZES["Q8_0"] == (32, fp16 + 32)
    assert BLOCK_SIZES["Q4_0"] == (32, fp16 + 16)
    assert BLOCK_SIZES["F32"] == (1, 4) and BLOCK_SIZES["BF16"] == (1, 2)
    assert GGML_TYPES[12][0] == "Q4_K" and GGML_TYPES[14][0] == "Q6_K" and GGML_TYPES[0][0] == "F32"
    assert tensor_nbytes((256, 2048, 512), "Q6_K") == 256 * 2048 * 2 * 210
    with pytest.raises(ValueError):
        tensor_nbytes((4, 100), "Q4_K")


def test_writer_round_trip(tmp_path):
    rng = np.random.default_rng(5)
    a = rng.standard_normal((3, 5)).astype(np.float32)
    q = synth.matrix(rng, "Q6_K", 4, 512)
    md = {"general.architecture": "qwen35moe", "k.big": 1 << 40, "k.neg": -3, "k.list": [1.5, 2.5], "k.s": "é"}
    p = str(tmp_path / "w.gguf")
    write_gguf(p, md, [("a", "F32", (3, 5), a), ("q", "Q6_K", (4, 512), q), ("one", "F32", (7,), a.ravel()[:7])],
               alignment=128)
    meta, ts = read_gguf(p)
    assert meta == {**md, "general.alignment": 128}
    raw = np.fromfile(p, dtype=np.uint8)
    for name, want in (("a", a), ("q", q), ("one", a.ravel()[:7])):
        t = ts[name]
        assert t.offset % 128 == 0
        assert raw[t.offset:t.offset + t.nbytes].tobytes() == np.ascontiguousarray(want).tobytes()
    assert ts["one"].shape == (7,)


def test_split_files(tmp_path):
    lw = synth.moe_layer(3, hidden=256, inter=256, shared_inter=256, experts=4, top_k=2)
    a = str(tmp_path / "M-Q4_K_M-00001-of-00002.gguf")
    b = str(tmp_path / "M-Q4_K_M-00002-of-00002.gguf")
    synth.write_moe_gguf(a, [lw])
    write_gguf(b, {"split.count": 2}, [("blk.0.extra.weight", "F32", (4,), np.ones(4, np.float32))])
    assert shard_files(b) == [a, b] and shard_files(a) == [a, b]
    assert shard_files(str(tmp_path / "x.gguf")) == [str(tmp_path / "x.gguf")]
    header = read_gguf(b)
    md, ts = header
    assert header.files == [a, b]
    assert md["general.architecture"] == "qwen35moe"          # the first file's metadata
    assert ts["blk.0.extra.weight"].file == b and ts["blk.0.ffn_down_exps.weight"].file == a
    os.remove(b)
    with pytest.raises(FileNotFoundError):
        shard_files(a)


def small_layers(down_types=("Q6_K", "Q4_K"), experts=4):
    return [synth.moe_layer(10 + i, hidden=256, inter=256, shared_inter=256, experts=experts, top_k=2,
                            down_type=dt) for i, dt in enumerate(down_types)]


def test_index_experts(tmp_path):
    layers = small_layers()
    p = str(tmp_path / "m.gguf")
    synth.write_moe_gguf(p, layers + [layers[0]], extra_metadata={"qwen35moe.nextn_predict_layers": 1})
    md, ts = read_gguf(p)
    assert decoder_layer_count(md) == 2  # the appended multi-token-prediction layer is skipped
    index = index_experts(md, ts)
    gate_bytes = 256 * 144  # 256 rows of one Q4_K block
    assert [lay.layer for lay in index] == [0, 1]
    assert [(lay.n_experts, lay.hidden, lay.inter) for lay in index] == [(4, 256, 256)] * 2
    assert [(lay.gate_up_type, lay.down_type) for lay in index] == [("Q4_K", "Q6_K"), ("Q4_K", "Q4_K")]
    assert index[0].gate_up_bytes == 2 * gate_bytes and index[0].down_bytes == 256 * 210
    raw = np.fromfile(p, dtype=np.uint8)
    for lay in index:
        for e in range(4):
            ranges = lay.gate_up_ranges(e)
            assert [size for _, _, size in ranges] == [gate_bytes, gate_bytes]
            fused = b"".join(raw[o:o + n].tobytes() for _, o, n in ranges)
            assert fused == layers[lay.layer]["gate_up"][e].tobytes()  # gate rows, then up rows
            _, o, n = lay.down_range(e)
            assert raw[o:o + n].tobytes() == layers[lay.layer]["down"][e].tobytes()


@pytest.mark.parametrize("bad", ["dense_layer", "gate_up_mismatch", "down_shape"])
def test_index_rejects(tmp_path, bad):
    layers = small_layers()
    if bad == "gate_up_mismatch":  # up stored in another type than gate
        layers[1] = synth.moe_layer(11, hidden=256, inter=256, shared_inter=256, experts=4, top_k=2)
    p = str(tmp_path / "m.gguf")
    extra = {"qwen35moe.block_count": 3} if bad == "dense_layer" else None
    synth.write_moe_gguf(p, layers, extra_metadata=extra)
    md, ts = read_gguf(p)
    if bad == "gate_up_mismatch":
        t = ts["blk.1.ffn_up_exps.weight"]
        ts["blk.1.ffn_up_exps.weight"] = type(t)(t.name, "Q6_K", t.shape, t.file, t.offset, t.nbytes)
    if bad == "down_shape":
        t = ts["blk.0.ffn_down_exps.weight"]
        ts["blk.0.ffn_down_exps.weight"] = type(t)(t.name, t.type, (4, 512, 128), t.file, t.offset, t.nbytes)
    with pytest.raises(ExpertLayoutError):
        index_experts(md, ts)
