"""The weight-cache reader's checks of a file's structure (trit_hip_decoder_load),
on the CPU: each malformed file below is refused before any device memory is
touched, with the message that names its fault. The files are written here
in the reader's format (magic, format, key, config, norms, layers)."""

import ctypes as C
import struct

import pytest

from trit_amd import hip

MAGIC = b"TRITHIPW"
FORMAT = 2
Q8_0, INT8, TERNARY, F16 = 1, 2, 3, 5


def key():
    lib = hip.lib()
    lib.trit_hip_version.restype = C.c_char_p
    return lib.trit_hip_version().decode() + " layout 2"


def header(cfg, k=None, fmt=FORMAT):
    c = hip.LmConfig.of(cfg)
    k = key() if k is None else k
    return (MAGIC + struct.pack("<II", fmt, len(k)) + k.encode() + struct.pack("<I", C.sizeof(c)) +
            bytes(c))


CFG = dict(d=64, ffn=128, layers=1, heads=2, kv_heads=1, head_dim=32, vocab=100, eps=1e-6, rope_base=1e6,
           qk_norm=1)


def norms(cfg, count=None):
    n = cfg["layers"] * (2 * cfg["d"] + 2 * cfg["head_dim"] * cfg["qk_norm"]) + cfg["d"]
    n = n if count is None else count
    return struct.pack("<Q", n) + b"\0" * (4 * n)


def layer(kind, n, k, group, codes, scales, bias=0):
    out = struct.pack("<iiii", kind, n, k, group)
    for size in (codes, scales, bias):
        out += struct.pack("<Q", size) + b"\0" * size
    return out


def load(tmp_path, data):
    p = tmp_path / "w.bin"
    p.write_bytes(data)
    with pytest.raises(hip.TritError) as e:
        hip.CausalLm.load(p)
    return str(e.value)


def test_key_and_format(tmp_path):
    assert "another cache format" in load(tmp_path, header(CFG, fmt=1) + norms(CFG))
    assert "build it again" in load(tmp_path, header(CFG, k="trit_hip 0.1.0 (gfx950)") + norms(CFG))
    assert "not a trit_hip weight cache" in load(tmp_path, b"NOTACACHE" * 4)


def test_norm_count_exact(tmp_path):
    """A norm block shorter than the config implies (it would be read past
    its end by the decoder) and a longer one are both refused."""
    want = 2 * 64 + 2 * 32 + 64
    for count in (want - 1, 1, want + 1):
        assert "bad norm count" in load(tmp_path, header(CFG) + norms(CFG, count))
    no_qk = dict(CFG, qk_norm=0)
    assert "bad norm count" in load(tmp_path, header(no_qk) + norms(no_qk, want))


def test_layer_sizes_exact(tmp_path):
    """Each buffer must have exactly the bytes its kind, n and k imply: a
    Q8_0 layer's codes one byte short, its scales as f32 instead of f16, an
    int8 layer with a 32-group, a ternary layer's codes as bytes, a bias of
    the wrong length; each is refused."""
    n, k = 64, 128
    good_q8 = (Q8_0, n, k, 32, n * k, n * k // 32 * 2)
    cases = [
        layer(Q8_0, n, k, 32, n * k - 1, n * k // 32 * 2),
        layer(Q8_0, n, k, 32, n * k, n * k // 32 * 4),
        layer(Q8_0, n, k, 32, n * k, n * k // 32 * 2, bias=4 * n - 4),
        layer(INT8, n, k, 32, n * k, n * k // 32 * 4),
        layer(TERNARY, n, k, 128, n * k, n * k // 128 * 4),
        layer(F16, n, k, 0, n * k, 0),
    ]
    for bad in cases:
        msg = load(tmp_path, header(CFG) + norms(CFG) + bad)
        assert "its layer's size" in msg or "not valid" in msg, msg
    # A well-formed first layer passes the checks (the file then ends).
    ok = layer(*good_q8)
    with pytest.raises(hip.TritError):
        hip.CausalLm.load(_write(tmp_path, header(CFG) + norms(CFG) + ok[:16]))


def _write(tmp_path, data):
    p = tmp_path / "w2.bin"
    p.write_bytes(data)
    return p
