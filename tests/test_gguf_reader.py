"""The GGUF header reader and the expert scan (gguf/reader.py, gguf/compiler.py:24-88 of the reference), on the
CPU. The reader is pinned on a header assembled byte by byte here from the published GGUF layout (not by this
package's writer); the writer, the split-file handling and the scan are then checked on files the writer makes."""
import os
import struct

import numpy as np
import pytest

from gguf import synth
from gguf.compiler import fuse_gate_up, num_decoder_layers, scan_experts
from gguf.reader import (BLOCK_SIZES, GGML_TYPES, model_stem, read_gguf, read_gguf_file, split_paths,
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
    assert a.path == b.path == str(p)


@pytest.mark.parametrize("bad", ["magic", "version", "type"])
def test_reader_rejects(tmp_path, bad):
    head = {"magic": handmade_header(magic=b"GGUX"), "version": handmade_header(version=1),
            "type": handmade_header(type_b=99)}[bad]
    p = tmp_path / "bad.gguf"
    p.write_bytes(head + bytes(128))
    with pytest.raises(SystemExit):
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
    assert split_paths(b) == [a, b]
    assert model_stem(b) == str(tmp_path / "M-Q4_K_M")
    assert model_stem(str(tmp_path / "x.gguf")) == str(tmp_path / "x")
    md, ts = read_gguf(b)
    assert md["general.architecture"] == "qwen35moe"          # the first file's metadata
    assert ts["blk.0.extra.weight"].path == b and ts["blk.0.ffn_down_exps.weight"].path == a
    os.remove(b)
    with pytest.raises(SystemExit):
        split_paths(a)


def small_layers(down_types=("Q6_K", "Q4_K"), experts=4):
    return [synth.moe_layer(10 + i, hidden=256, inter=256, shared_inter=256, experts=experts, top_k=2,
                            down_type=dt) for i, dt in enumerate(down_types)]


def test_scan_experts_and_fuse(tmp_path):
    layers = small_layers()
    p = str(tmp_path / "m.gguf")
    synth.write_moe_gguf(p, layers + [layers[0]], extra_metadata={"qwen35moe.nextn_predict_layers": 1})
    md, ts = read_gguf(p)
    assert num_decoder_layers(md) == 2  # the appended multi-token-prediction layer is skipped
    n_layers, n_exp, max_payload, plan, info = scan_experts(md, ts)
    gate_bytes = 256 * 144  # 256 rows of one Q4_K block
    assert (n_layers, n_exp) == (2, 4)
    assert info["0.down"] == {"shape": [256, 256], "dtype": "Q6_K"} and info["1.down"]["dtype"] == "Q4_K"
    assert max_payload == 2 * gate_bytes + 256 * 210
    raw = np.fromfile(p, dtype=np.uint8)
    for (layer, e), parts in plan.items():
        assert [q[0] for q in parts] == ["gate", "up", "down"]
        t = ts[f"blk.{layer}.ffn_gate_exps.weight"]
        assert parts[0][2] == t.offset + e * gate_bytes and parts[0][3] == gate_bytes
        got = raw[parts[0][2]:parts[0][2] + gate_bytes]
        assert got.tobytes() == layers[layer]["gate_up"][e, :256].tobytes()
    fplan, finfo = fuse_gate_up(plan, info)
    assert finfo["0.gate_up"] == {"shape": [512, 256], "dtype": "Q4_K"} and "0.gate" not in finfo
    (part, srcs), (dpart, dsrc) = fplan[(1, 2)]
    assert part == "gate_up" and dpart == "down" and len(srcs) == 2
    fused = b"".join(raw[o:o + n].tobytes() for _, o, n in srcs)
    assert fused == layers[1]["gate_up"][2].tobytes()


def test_scan_rejects_dense_layers(tmp_path):
    layers = small_layers()
    p = str(tmp_path / "m.gguf")
    synth.write_moe_gguf(p, layers, extra_metadata={"qwen35moe.block_count": 3})
    md, ts = read_gguf(p)
    with pytest.raises(SystemExit):
        scan_experts(md, ts)
