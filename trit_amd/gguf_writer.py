"""A GGUF v3 writer (tests and the load-time measurement): metadata of every GGUF type, tensors at
aligned offsets (the format the reference reads, src/models/gguf/mod.rs:
130-226), and a decoder laid out as transcribe.cpp writes a Qwen3-ASR
language model (`stt.qwen3_asr.decoder.*` keys, `dec.*` tensors,
src/models/gguf/blocks.rs:25-45, src/models/gguf/qwen3_asr.rs:103-136).
"""

from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
GGML = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14,
        "BF16": 30}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(kind: int, v) -> bytes:
    if kind == ARR:
        item, items = v
        return struct.pack("<IQ", item, len(items)) + b"".join(_value(item, x) for x in items)
    fmt = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
           I64: "<q", F64: "<d"}
    if kind == STR:
        return _str(v)
    return struct.pack(fmt[kind], v)


def write(path, meta, tensors, version=3, alignment=32, magic=b"GGUF", pad_end=0):
    """meta: [(key, kind, value)]; tensors: [(name, ggml type id, dims (ne0 first), bytes)]."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(meta))
    for key, kind, v in meta:
        head += _str(key) + struct.pack("<I", kind) + _value(kind, v)
    offsets, off = [], 0
    for name, kind, dims, data in tensors:
        offsets.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, kind, dims, data), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", kind, o)
    data_start = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (data_start - len(head)))
        for (name, kind, dims, data), o in zip(tensors, offsets):
            f.seek(data_start + o)
            f.write(bytes(data))
        f.write(b"\0" * pad_end)
    return data_start


def write_decoder(path, w, prefix="stt.qwen3_asr.decoder", arch="qwen3_asr", untied_head=None, replace=None):
    """The language model of synthetic weights `w` (trit_amd.synth.LmWeights)
    as a transcribe.cpp Qwen3-ASR file: q, k, v and gate, up as tensors of
    their own (their Q8_0 rows split from the stacked layers). `replace`:
    {tensor name: (ggml type id, dims, bytes)} written in place of those."""
    c = w.cfg
    d, ffn, hd = c["d"], c["ffn"], c["head_dim"]
    qd, kd = c["heads"] * hd, c["kv_heads"] * hd
    meta = [("general.architecture", STR, arch), ("general.alignment", U32, 32)]
    for key, val in [("hidden_size", d), ("intermediate_size", ffn), ("n_layers", c["layers"]),
                     ("n_heads", c["heads"]), ("n_kv_heads", c["kv_heads"]), ("head_dim", hd),
                     ("vocab_size", c["vocab"])]:
        meta.append((f"{prefix}.{key}", U32, val))
    meta += [(f"{prefix}.rms_norm_eps", F32, c["eps"]), (f"{prefix}.rope_theta", F32, c["rope_base"]),
             (f"{prefix}.tie_word_embeddings", BOOL, untied_head is None)]
    row = lambda k: k // 32 * 34  # Q8_0 bytes a row
    tensors = [("dec.token_embd.weight", GGML["F16"], [d, c["vocab"]], np.ascontiguousarray(w.embed).tobytes())]
    for i, L in enumerate(w.layers):
        b = f"dec.blocks.{i}."
        qkv = np.frombuffer(bytes(L.qkv), np.uint8)
        gu = np.frombuffer(bytes(L.gate_up), np.uint8)
        r = row(d)
        tensors += [
            (b + "attn.q.weight", GGML["Q8_0"], [d, qd], qkv[: qd * r].tobytes()),
            (b + "attn.k.weight", GGML["Q8_0"], [d, kd], qkv[qd * r: (qd + kd) * r].tobytes()),
            (b + "attn.v.weight", GGML["Q8_0"], [d, kd], qkv[(qd + kd) * r:].tobytes()),
            (b + "attn.o.weight", GGML["Q8_0"], [qd, d], bytes(L.o)),
            (b + "ffn.gate.weight", GGML["Q8_0"], [d, ffn], gu[: ffn * r].tobytes()),
            (b + "ffn.up.weight", GGML["Q8_0"], [d, ffn], gu[ffn * r:].tobytes()),
            (b + "ffn.down.weight", GGML["Q8_0"], [ffn, d], bytes(L.down)),
            (b + "norm_attn.weight", GGML["F32"], [d], L.norm_attn.astype(np.float32).tobytes()),
            (b + "norm_ffn.weight", GGML["F32"], [d], L.norm_mlp.astype(np.float32).tobytes()),
        ]
        if c.get("qk_norm", 1):
            tensors += [(b + "attn.q_norm.weight", GGML["F32"], [hd], L.q_norm.astype(np.float32).tobytes()),
                        (b + "attn.k_norm.weight", GGML["F32"], [hd], L.k_norm.astype(np.float32).tobytes())]
    tensors.append(("dec.output_norm.weight", GGML["F32"], [d], w.final_norm.astype(np.float32).tobytes()))
    if untied_head is not None:
        tensors.append(("dec.output.weight", GGML["F16"], [d, c["vocab"]], np.ascontiguousarray(untied_head).tobytes()))
    if replace:
        tensors = [(n, *replace[n]) if n in replace else (n, k, dm, b) for n, k, dm, b in tensors]
    write(path, meta, tensors)
