"""The GGUF reader (trit_hip_gguf_open) against the reference's Gguf::open
(src/models/gguf/mod.rs:130-226) and its type table
(src/cpu/ggml_quants.rs:51-75): the tensors' byte ranges, the metadata, and
each check's error in the reference's words. Host code only: CPU tests."""

import struct

import numpy as np
import pytest

from trit_amd import gguf_writer as G
from trit_amd import hip

TYPES = "F32, F16, BF16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q5_K, and Q6_K"


def sample(path, **kw):
    meta = [
        ("general.architecture", G.STR, "qwen3_asr"),
        ("a.u8", G.U8, 200), ("a.i8", G.I8, -5), ("a.u16", G.U16, 60000), ("a.i16", G.I16, -30000),
        ("a.u32", G.U32, 4000000000), ("a.i32", G.I32, -7), ("a.f32", G.F32, 0.5), ("a.bool", G.BOOL, 1),
        ("a.u64", G.U64, 1 << 40), ("a.i64", G.I64, 12), ("a.f64", G.F64, 1e-6),
        ("a.nested", G.ARR, (G.ARR, [(G.U32, [1, 2]), (G.U32, [3])])),
        ("tokenizer.ggml.tokens", G.ARR, (G.STR, ["a", "é", "<|x|>"])),
    ]
    tensors = [
        ("w.q8", G.GGML["Q8_0"], [64, 3], bytes(range(34)) * 6),
        ("w.f16", G.GGML["F16"], [5], b"\x01\x02" * 5),
        ("w.q4k", G.GGML["Q4_K"], [256, 2], b"\x07" * 288),
        ("n.f32", G.GGML["F32"], [3], np.arange(3, dtype=np.float32).tobytes()),
    ]
    data = G.write(path, meta, tensors, **kw)
    return data, tensors


def test_tensors_and_metadata(tmp_path):
    path = tmp_path / "ok.gguf"
    data, tensors = sample(path)
    g = hip.Gguf(path)
    got = g.tensors()
    sizes = [6 * 34, 10, 288, 12]
    want, off = [], 0
    for (name, kind, dims, raw), size in zip(tensors, sizes):
        assert len(raw) == size
        want.append((name, {8: "Q8_0", 1: "F16", 12: "Q4_K", 0: "F32"}[kind], dims, data + off, data + off + size))
        off = (off + size + 31) // 32 * 32
    assert got == want
    assert g.u64("a.u8") == 200 and g.u64("a.u16") == 60000 and g.u64("a.u32") == 4000000000
    assert g.u64("a.u64") == 1 << 40 and g.u64("a.i64") == 12
    assert g.f64("a.f32") == 0.5 and g.f64("a.f64") == 1e-6 and g.f64("a.i8") == -5.0
    assert g.str("general.architecture") == "qwen3_asr"
    with pytest.raises(hip.TritError, match="no integer a.i8"):
        g.u64("a.i8")  # negative
    with pytest.raises(hip.TritError, match="no string a.u8"):
        g.str("a.u8")
    with pytest.raises(hip.TritError, match="no integer missing"):
        g.u64("missing")
    g.free()


def test_version_2_and_alignment(tmp_path):
    path = tmp_path / "v2.gguf"
    data, _ = sample(path, version=2, alignment=64)
    # general.alignment is absent from this file's metadata: the data
    # starts at the next multiple of 32, and the writer's 64-byte spacing
    # of the tensors is what the offsets say.
    got = hip.Gguf(path).tensors()
    assert got[0][3] % 32 == 0 and got[1][3] - got[0][3] == 256


def test_alignment_from_metadata(tmp_path):
    path = tmp_path / "a64.gguf"
    meta = [("general.alignment", G.U32, 64)]
    G.write(path, meta, [("t", G.GGML["F32"], [1], b"\0" * 4), ("u", G.GGML["F32"], [1], b"\0" * 4)], alignment=64)
    t = hip.Gguf(path).tensors()
    assert t[0][3] % 64 == 0 and t[1][3] == t[0][3] + 64


def expect(path, text):
    with pytest.raises(hip.TritError) as e:
        hip.Gguf(path)
    assert text in str(e.value) and str(path) in str(e.value), str(e.value)


def test_errors(tmp_path):
    p = tmp_path / "x.gguf"
    sample(p, magic=b"GGUG")
    expect(p, "not a GGUF file")
    for v in (1, 4):
        sample(p, version=v)
        expect(p, f"GGUF version {v}; Trit reads 2 and 3")
    sample(p)
    with open(p, "rb") as f:
        head = f.read(60)
    with open(p, "wb") as f:
        f.write(head)
    expect(p, "the header ends early")
    # A metadata type past 12.
    with open(p, "wb") as f:
        f.write(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13))
    expect(p, "metadata type 13 is not GGUF")
    # Arrays: four levels read, a fifth is too deep.
    deep = (G.U8, [1])
    for _ in range(3):
        deep = (G.ARR, [deep])
    G.write(p, [("d", G.ARR, deep)], [])
    hip.Gguf(p)
    G.write(p, [("d", G.ARR, (G.ARR, [deep]))], [])
    expect(p, "the header arrays are nested too deep")
    with open(p, "wb") as f:
        f.write(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", (1 << 24) + 1))
    expect(p, "a header string is too long")
    with open(p, "wb") as f:
        f.write(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" +
                struct.pack("<IIQ", G.ARR, G.U8, (1 << 24) + 1))
    expect(p, "a header array is too long")
    with open(p, "wb") as f:
        f.write(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 2) + b"\xc3\x28")
    expect(p, "a header string is not UTF-8")
    with open(p, "wb") as f:
        f.write(b"GGUF" + struct.pack("<IQQ", 3, 1000, 0) + b"\0" * 64)
    expect(p, "the tensor list runs past the end of the file")
    G.write(p, [("general.alignment", G.U32, 0)], [("t", 0, [1], b"\0" * 4)])
    expect(p, "general.alignment is 0")
    G.write(p, [], [("t", 99, [4], b"\0" * 16)])
    expect(p, "tensor t has ggml type 99; Trit reads " + TYPES)
    G.write(p, [], [("t", G.GGML["Q8_0"], [33], b"\0" * 68)])
    expect(p, "tensor t has ggml type 8; Trit reads " + TYPES)
    G.write(p, [], [("t", G.GGML["F32"], [4], b"\0" * 16)])
    with open(p, "r+b") as f:
        f.truncate(f.seek(0, 2) - 8)
    expect(p, "tensor t runs past the end of the file")
    G.write(p, [], [("t", G.GGML["F32"], [1 << 62, 8], b"\0" * 4)])
    expect(p, "tensor t runs past the end of the file")
    with pytest.raises(hip.TritError, match="Could not read"):
        hip.Gguf(tmp_path / "missing.gguf")
